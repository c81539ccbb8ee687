// Per-(device, stream) scratch buffers of the split-K tiles (host code only;
// no HIP types, so the locking can be tested with a plain C++ compiler).
//
// A split-K call queues two kernels that share one buffer: the tiles write
// their partial sums to it and the epilogue adds them.  acquire() hands out
// the stream's buffer together with the stream's scratch lock, and the lock is
// held until the Lease is destroyed, so a caller that queues both kernels
// while it holds the lease keeps them adjacent on the stream: two host threads
// calling on one stream are ordered A-tiles, A-epilogue, B-tiles, B-epilogue,
// never A-tiles, B-tiles, A-epilogue (where A's epilogue would add B's
// partial sums).  Calls on different streams use different buffers and never
// wait for each other.
//
// A buffer grows to the next power of two (at least 1 MiB) when a call needs
// more.  The outgrown buffer is retired, not freed, because kernels queued
// earlier on the stream may still read it.  A caller that must not allocate
// (a stream under graph capture) acquires with may_allocate false and gets
// kWouldAllocate instead of a growth.  detach() forgets a stream and
// hands back all of its buffers (current and retired) without freeing them:
// the library's mote_hip_stream_destroy parks them with an event recorded on
// the stream and frees them once that event has completed, so destroying a
// stream never waits for its queued work.  release() frees them at once, for
// a caller that knows the stream's work has completed.
#pragma once

#include <cstddef>
#include <map>
#include <memory>
#include <mutex>
#include <utility>
#include <vector>

namespace mote::q4_0 {

class ScratchPool {
   public:
    using AllocFn = int (*)(void** ptr, std::size_t bytes);  // 0 on success
    using FreeFn = int (*)(void* ptr);

    ScratchPool(AllocFn alloc, FreeFn free) : alloc_(alloc), free_(free) {}
    ScratchPool(const ScratchPool&) = delete;
    ScratchPool& operator=(const ScratchPool&) = delete;

   private:
    struct Entry {
        std::mutex mu;
        void* ptr = nullptr;
        std::size_t size = 0;
        std::vector<void*> retired;
    };

   public:
    // The buffer of one call and the stream's scratch lock.  Members are
    // destroyed in reverse order: the lock is released before the entry's
    // last reference can go.
    class Lease {
       public:
        void* ptr() const { return ptr_; }
        bool held() const { return lock_.owns_lock(); }
        // Whether this acquire allocated the buffer (its contents are then
        // undefined; the caller clears what must start at zero).
        bool fresh() const { return fresh_; }

       private:
        friend class ScratchPool;
        std::shared_ptr<Entry> entry_;
        std::unique_lock<std::mutex> lock_;
        void* ptr_ = nullptr;
        bool fresh_ = false;
    };

    // Status of an acquire that would have to allocate but may not.
    static constexpr int kWouldAllocate = -2;

    // Blocks while another lease of the same (device, stream) is held.
    // Returns 0, kWouldAllocate, or the allocator's status (the lease is then
    // not held).
    int acquire(int device, const void* stream, std::size_t bytes, Lease* lease, bool may_allocate = true) {
        std::shared_ptr<Entry> entry;
        {
            std::lock_guard<std::mutex> guard(map_mu_);
            auto& slot = entries_[{device, stream}];
            if (!slot) slot = std::make_shared<Entry>();
            entry = slot;
        }
        std::unique_lock<std::mutex> lock(entry->mu);
        lease->fresh_ = false;
        if (entry->size < bytes) {
            if (!may_allocate) return kWouldAllocate;
            std::size_t want = std::size_t{1} << 20;
            while (want < bytes) want <<= 1;
            void* fresh = nullptr;
            const int status = alloc_(&fresh, want);
            if (status != 0) return status;
            if (entry->ptr != nullptr) entry->retired.push_back(entry->ptr);
            entry->ptr = fresh;
            entry->size = want;
            lease->fresh_ = true;
        }
        lease->ptr_ = entry->ptr;
        lease->entry_ = std::move(entry);
        lease->lock_ = std::move(lock);
        return 0;
    }

    // Forgets (device, stream) and returns every buffer it held (the current
    // one and the retired ones), which the caller now owns and frees once the
    // stream's queued work has completed; a stream created later at the same
    // address starts without a buffer.  Waits for a lease still held.
    std::vector<void*> detach(int device, const void* stream) {
        std::shared_ptr<Entry> entry;
        {
            std::lock_guard<std::mutex> guard(map_mu_);
            auto found = entries_.find({device, stream});
            if (found == entries_.end()) return {};
            entry = std::move(found->second);
            entries_.erase(found);
        }
        std::lock_guard<std::mutex> lock(entry->mu);  // waits for a lease still held
        std::vector<void*> out;
        for (void* p : entry->retired)
            if (p != nullptr) out.push_back(p);
        if (entry->ptr != nullptr) out.push_back(entry->ptr);
        entry->retired.clear();
        entry->ptr = nullptr;
        entry->size = 0;
        return out;
    }

    // Frees every buffer of (device, stream) and forgets the stream.  The
    // caller guarantees the stream has no queued work left.  Returns the
    // first failing free's status, else 0.
    int release(int device, const void* stream) { return free_all(detach(device, stream)); }

    // Frees buffers handed out by detach(); returns the first failing free's
    // status, else 0.
    int free_all(const std::vector<void*>& buffers) {
        int status = 0;
        for (void* p : buffers) {
            const int s = free_(p);
            if (status == 0) status = s;
        }
        return status;
    }

    // Streams with a buffer (for tests).
    std::size_t streams() {
        std::lock_guard<std::mutex> guard(map_mu_);
        return entries_.size();
    }

   private:
    AllocFn alloc_;
    FreeFn free_;
    std::mutex map_mu_;
    std::map<std::pair<int, const void*>, std::shared_ptr<Entry>> entries_;
};

}  // namespace mote::q4_0
