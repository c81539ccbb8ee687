// Fatal-signal report for the benchmark process (libmote_probe.so, loaded only
// by bench.py): on SIGSEGV, SIGBUS, SIGILL, SIGFPE or SIGABRT it writes the
// signal, the faulting address, the program counter and the whole of
// /proc/self/maps to a file descriptor, so that a host fault inside a runtime
// or profiler library names that library, and then hands the signal to the
// handler that was installed before it (Python's faulthandler, which prints
// the Python stack, or a profiler's), or to the default action.
//
// Everything the handler calls is async-signal-safe (open, read, write,
// close, sigaction, raise); the text is formatted into a stack buffer.
#include <csignal>
#include <cstdint>
#include <cstring>

#include <fcntl.h>
#include <ucontext.h>
#include <unistd.h>

#include "export.hpp"

namespace {

constexpr int kSignals[] = {SIGSEGV, SIGBUS, SIGILL, SIGFPE, SIGABRT};
constexpr int kCount = sizeof(kSignals) / sizeof(kSignals[0]);
struct sigaction g_previous[kCount];
int g_fd = 2;

void put(const char* s, size_t n) {
    while (n > 0) {
        const ssize_t w = write(g_fd, s, n);
        if (w <= 0) return;
        s += w;
        n -= static_cast<size_t>(w);
    }
}

void put_str(const char* s) { put(s, strlen(s)); }

void put_hex(uint64_t v) {
    char b[19];
    b[0] = '0';
    b[1] = 'x';
    for (int i = 0; i < 16; ++i) b[2 + i] = "0123456789abcdef"[(v >> (60 - 4 * i)) & 15];
    put(b, 18);
}

void handler(int sig, siginfo_t* info, void* context) {
    int slot = 0;
    while (slot < kCount && kSignals[slot] != sig) ++slot;
    put_str("\n*** mote_probe fault report: signal ");
    char num[4] = {static_cast<char>('0' + sig / 10 % 10), static_cast<char>('0' + sig % 10), ' ', 0};
    put(num, 3);
    put_str("address ");
    put_hex(reinterpret_cast<uint64_t>(info ? info->si_addr : nullptr));
    put_str(" pc ");
    uint64_t pc = 0;
    if (context != nullptr) pc = static_cast<uint64_t>(static_cast<ucontext_t*>(context)->uc_mcontext.gregs[REG_RIP]);
    put_hex(pc);
    put_str("\n*** /proc/self/maps:\n");
    const int maps = open("/proc/self/maps", O_RDONLY);
    if (maps >= 0) {
        char buf[4096];
        for (;;) {
            const ssize_t n = read(maps, buf, sizeof buf);
            if (n <= 0) break;
            put(buf, static_cast<size_t>(n));
        }
        close(maps);
    }
    put_str("*** end of maps\n");
    // Hand the signal on: the previous handler if there was one, else the
    // default action (restored, then raised again).
    if (slot < kCount) {
        const struct sigaction& prev = g_previous[slot];
        if ((prev.sa_flags & SA_SIGINFO) != 0 && prev.sa_sigaction != nullptr) {
            sigaction(sig, &prev, nullptr);
            prev.sa_sigaction(sig, info, context);
            return;
        }
        if (prev.sa_handler != SIG_DFL && prev.sa_handler != SIG_IGN && prev.sa_handler != nullptr) {
            sigaction(sig, &prev, nullptr);
            prev.sa_handler(sig);
            return;
        }
    }
    struct sigaction dfl;
    memset(&dfl, 0, sizeof dfl);
    dfl.sa_handler = SIG_DFL;
    sigemptyset(&dfl.sa_mask);
    sigaction(sig, &dfl, nullptr);
    raise(sig);
}

}  // namespace

// Installs the fatal-signal report, written to `fd` (2: stderr), in front of
// the handlers installed so far.  Returns 0, or -1 if a sigaction call failed.
MOTE_EXPORT int mote_probe_install_fault_report(int fd) noexcept {
    g_fd = fd;
    for (int i = 0; i < kCount; ++i) {
        struct sigaction act;
        memset(&act, 0, sizeof act);
        act.sa_sigaction = handler;
        act.sa_flags = SA_SIGINFO | SA_NODEFER;
        sigemptyset(&act.sa_mask);
        if (sigaction(kSignals[i], &act, &g_previous[i]) != 0) return -1;
    }
    return 0;
}
