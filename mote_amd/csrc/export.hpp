// Marks a function as part of the exported C ABI (include/mote_hip.h); the
// library is built with -fvisibility=hidden, so nothing else is exported.
#pragma once

#define MOTE_EXPORT extern "C" __attribute__((visibility("default")))
