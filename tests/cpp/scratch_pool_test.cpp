// CPU test of the split-K scratch pool's locking (mote_amd/csrc/
// scratch_pool.hpp), built with the host compiler by tests/test_scratch_pool.py.
//
// Two threads play two callers of a split-K entry point on one stream: each
// takes a lease, "queues" its tiles kernel, sleeps, "queues" its epilogue and
// drops the lease.  The queue they append to stands for the stream; the test
// fails if any caller's two entries are not adjacent (the interleaving where
// one call's epilogue would add the other call's partial sums).  Calls on two
// streams must not wait for each other; growth retires and release frees
// every buffer exactly once.
#include "scratch_pool.hpp"

#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <set>
#include <string>
#include <thread>
#include <vector>

using mote::q4_0::ScratchPool;

namespace {

std::mutex g_mu;
std::set<void*> g_live;
int g_allocs = 0, g_frees = 0;

int fake_alloc(void** p, std::size_t bytes) {
    std::lock_guard<std::mutex> lock(g_mu);
    *p = std::malloc(bytes ? 1 : 1);
    g_live.insert(*p);
    ++g_allocs;
    return 0;
}

int fake_free(void* p) {
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_live.erase(p) != 1) return 99;  // double or foreign free
    std::free(p);
    ++g_frees;
    return 0;
}

int failures = 0;
#define CHECK(c)                                                        \
    do {                                                                \
        if (!(c)) {                                                     \
            std::fprintf(stderr, "FAILED line %d: %s\n", __LINE__, #c); \
            ++failures;                                                 \
        }                                                               \
    } while (0)

void test_calls_on_one_stream_stay_adjacent() {
    ScratchPool pool(fake_alloc, fake_free);
    const void* stream = reinterpret_cast<const void*>(0x1000);
    std::mutex queue_mu;
    std::vector<std::string> queue;
    auto push = [&](const std::string& s) {
        std::lock_guard<std::mutex> lock(queue_mu);
        queue.push_back(s);
    };
    auto caller = [&](char name, int calls) {
        for (int i = 0; i < calls; ++i) {
            ScratchPool::Lease lease;
            CHECK(pool.acquire(0, stream, 4096u * (i % 5 + 1), &lease) == 0);
            CHECK(lease.held());
            CHECK(lease.ptr() != nullptr);
            push(std::string(1, name) + "-tiles");
            std::this_thread::sleep_for(std::chrono::microseconds(200));
            push(std::string(1, name) + "-epilogue");
        }
    };
    std::thread a(caller, 'A', 50), b(caller, 'B', 50);
    a.join();
    b.join();
    CHECK(queue.size() == 200);
    for (size_t i = 0; i + 1 < queue.size(); i += 2) {
        CHECK(queue[i].substr(1) == "-tiles");
        CHECK(queue[i + 1].substr(1) == "-epilogue");
        CHECK(queue[i][0] == queue[i + 1][0]);
    }
    CHECK(pool.release(0, stream) == 0);
    CHECK(pool.streams() == 0);
}

void test_streams_do_not_wait_for_each_other() {
    ScratchPool pool(fake_alloc, fake_free);
    const void* s1 = reinterpret_cast<const void*>(0x1000);
    const void* s2 = reinterpret_cast<const void*>(0x2000);
    {
        ScratchPool::Lease held;
        CHECK(pool.acquire(0, s1, 64, &held) == 0);
        std::atomic<bool> done{false};
        std::thread other([&] {
            ScratchPool::Lease lease;
            CHECK(pool.acquire(0, s2, 64, &lease) == 0);  // a different stream: no wait
            CHECK(lease.ptr() != held.ptr());
            done = true;
        });
        for (int i = 0; i < 2000 && !done; ++i) std::this_thread::sleep_for(std::chrono::milliseconds(1));
        CHECK(done.load());
        other.join();
        // same stream on another device: its own buffer
        ScratchPool::Lease dev1;
        CHECK(pool.acquire(1, s1, 64, &dev1) == 0);
        CHECK(dev1.ptr() != held.ptr());
    }
    CHECK(pool.release(0, s1) == 0);
    CHECK(pool.release(0, s2) == 0);
    CHECK(pool.release(1, s1) == 0);
    CHECK(pool.streams() == 0);
}

void test_growth_retires_and_release_frees_everything() {
    const int allocs0 = g_allocs, frees0 = g_frees;
    {
        ScratchPool pool(fake_alloc, fake_free);
        const void* s = reinterpret_cast<const void*>(0x3000);
        void* first = nullptr;
        {
            ScratchPool::Lease l;
            CHECK(pool.acquire(0, s, 1, &l) == 0);
            CHECK(l.fresh());  // allocated by this acquire
            first = l.ptr();
        }
        {
            ScratchPool::Lease l;  // fits the 1 MiB minimum: same buffer
            CHECK(pool.acquire(0, s, 1u << 20, &l) == 0);
            CHECK(l.ptr() == first);
            CHECK(!l.fresh());
        }
        {
            ScratchPool::Lease l;  // grows: a new buffer, the old one retired
            CHECK(pool.acquire(0, s, (1u << 20) + 1, &l) == 0);
            CHECK(l.ptr() != first);
            CHECK(l.fresh());
        }
        CHECK(g_allocs - allocs0 == 2);
        CHECK(g_frees - frees0 == 0);
        CHECK(pool.release(0, s) == 0);
        CHECK(g_frees - frees0 == 2);
        CHECK(pool.release(0, s) == 0);  // nothing left: no second free
        CHECK(g_frees - frees0 == 2);
        {
            ScratchPool::Lease l;  // a stream used again after release starts afresh
            CHECK(pool.acquire(0, s, 16, &l) == 0);
            CHECK(g_allocs - allocs0 == 3);
        }
        CHECK(pool.release(0, s) == 0);
        CHECK(g_frees - frees0 == 3);
    }
}

void test_release_waits_for_a_held_lease() {
    ScratchPool pool(fake_alloc, fake_free);
    const void* s = reinterpret_cast<const void*>(0x4000);
    auto lease = new ScratchPool::Lease;
    CHECK(pool.acquire(0, s, 64, lease) == 0);
    std::atomic<bool> released{false};
    std::thread t([&] {
        CHECK(pool.release(0, s) == 0);
        released = true;
    });
    std::this_thread::sleep_for(std::chrono::milliseconds(50));
    CHECK(!released.load());  // the buffer is still in use by the lease
    delete lease;
    t.join();
    CHECK(released.load());
    CHECK(pool.streams() == 0);
}

}  // namespace


void test_detach_hands_back_every_buffer_once() {
    ScratchPool pool(fake_alloc, fake_free);
    const void* stream = reinterpret_cast<const void*>(0x3000);
    const int frees0 = g_frees;
    {
        ScratchPool::Lease a;
        CHECK(pool.acquire(0, stream, 1 << 20, &a) == 0);
    }
    {
        ScratchPool::Lease b;  // grows: the first buffer is retired
        CHECK(pool.acquire(0, stream, 3 << 20, &b) == 0);
        CHECK(b.fresh());
    }
    std::vector<void*> parked = pool.detach(0, stream);
    CHECK(parked.size() == 2);
    CHECK(g_frees == frees0);          // nothing freed yet: the caller owns them
    CHECK(pool.streams() == 0);        // the stream is forgotten
    CHECK(pool.detach(0, stream).empty());
    {
        ScratchPool::Lease c;  // a stream created later at the same address starts afresh
        CHECK(pool.acquire(0, stream, 1 << 20, &c) == 0);
        CHECK(c.fresh());
        for (void* p : parked) CHECK(c.ptr() != p);
    }
    CHECK(pool.free_all(parked) == 0);
    CHECK(g_frees == frees0 + 2);
    CHECK(pool.release(0, stream) == 0);
    CHECK(g_frees == frees0 + 3);
}

void test_acquire_that_may_not_allocate() {
    ScratchPool pool(fake_alloc, fake_free);
    const void* stream = reinterpret_cast<const void*>(0x5000);
    const int allocs0 = g_allocs;
    {
        ScratchPool::Lease a;  // no buffer yet: refused, nothing allocated, no lease held
        CHECK(pool.acquire(0, stream, 64, &a, false) == ScratchPool::kWouldAllocate);
        CHECK(!a.held());
        CHECK(g_allocs == allocs0);
    }
    void* first = nullptr;
    {
        ScratchPool::Lease b;  // an allocating acquire sizes the buffer (1 MiB)
        CHECK(pool.acquire(0, stream, 64, &b) == 0);
        first = b.ptr();
    }
    {
        ScratchPool::Lease c;  // fits: the same buffer, no allocation
        CHECK(pool.acquire(0, stream, 1 << 20, &c, false) == 0);
        CHECK(c.held() && c.ptr() == first && !c.fresh());
    }
    {
        ScratchPool::Lease d;  // would grow: refused, the buffer kept
        CHECK(pool.acquire(0, stream, (1 << 20) + 1, &d, false) == ScratchPool::kWouldAllocate);
        CHECK(!d.held());
    }
    CHECK(g_allocs == allocs0 + 1);
    {
        ScratchPool::Lease e;  // the refusal left the stream usable
        CHECK(pool.acquire(0, stream, 1 << 20, &e) == 0);
        CHECK(e.ptr() == first);
    }
    CHECK(pool.release(0, stream) == 0);
}

int main() {
    test_detach_hands_back_every_buffer_once();
    test_acquire_that_may_not_allocate();
    test_calls_on_one_stream_stay_adjacent();
    test_streams_do_not_wait_for_each_other();
    test_growth_retires_and_release_frees_everything();
    test_release_waits_for_a_held_lease();
    CHECK(g_live.empty());  // every buffer the pools allocated was freed once
    CHECK(g_allocs == g_frees);
    if (failures == 0) std::printf("scratch pool: all checks passed\n");
    return failures == 0 ? 0 : 1;
}
