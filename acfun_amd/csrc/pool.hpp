// pool.hpp -- the caching policy of the library's device memory pool,
// independent of HIP so that it can be exercised on the host.
//
// Free blocks are kept per (device, rounded size), each with the stream it
// was freed on, or marked idle.  An allocation on stream s takes, in order:
//   1. a block freed on s itself: reuse is ordered after every earlier use by
//      the stream's own order, no wait needed;
//   2. an idle block: no work that used it can still be running;
//   3. when blocks of the size sit cached on other streams and those streams
//      hold at least kReclaimBytes of cache: the device is synchronized once,
//      which finishes every use of the blocks freed before the sync began
//      whatever stream (live or since destroyed) queued it; those blocks
//      become idle, and the allocation takes one of them.  A block that
//      another host thread frees while the sync runs keeps its stream: the
//      work it was freed after may have been queued after the sync began;
//   4. a new block from the backend; if that fails, every cached block of the
//      device is released (after a device sync) and the allocation retried.
// A caller that keeps to one stream never pays for 3.  A caller that creates
// a stream per call and drops it leaves its blocks behind on dead streams;
// step 3 brings them back once they add up to kReclaimBytes, so the pool
// stays within that much of the working set instead of growing without bound.
//
// Backend (B) interface:
//   void* alloc(size_t bytes)            nullptr on failure
//   void  release(void* p)
//   void  sync_device()                  waits for all work on the device
#pragma once
#include <cstddef>
#include <map>
#include <mutex>
#include <utility>
#include <vector>

namespace acfun {

template <class B, class Stream>
class PoolCore {
  public:
    static constexpr size_t kReclaimBytes = size_t(64) << 20;

    explicit PoolCore(B& backend) : b_(backend) {}

    // Blocks are rounded up so that similar sizes share a free list.
    static size_t round_size(size_t b) {
        if (b <= 4096) return 4096;
        if (b <= (1u << 20)) return (b + 65535) & ~size_t(65535);
        return (b + (1u << 20) - 1) & ~size_t((1u << 20) - 1);
    }

    void* alloc(int dev, size_t bytes, Stream s) {
        const size_t rb = round_size(bytes);
        bool reclaim = false;
        {
            std::lock_guard<std::mutex> lk(mu_);
            auto it = free_.find({dev, rb});
            if (it != free_.end()) {
                auto& v = it->second;
                for (size_t i = v.size(); i-- > 0;)            // 1. same stream, newest first
                    if (!v[i].idle && v[i].s == s) return take(dev, rb, v, i);
                bool foreign = false;
                for (size_t i = 0; i < v.size(); ++i) {        // 2. idle
                    if (v[i].idle) return take(dev, rb, v, i);
                    foreign = true;
                }
                reclaim = foreign && foreign_bytes(dev, s) >= kReclaimBytes;
            }
        }
        if (reclaim) {                                         // 3. reclaim other streams' blocks
            unsigned long long seq0;
            {
                std::lock_guard<std::mutex> lk(mu_);
                seq0 = seq_;                                   // frees up to here precede the sync
            }
            b_.sync_device();
            std::lock_guard<std::mutex> lk(mu_);
            ++reclaims_;
            for (auto& kv : free_) {
                if (kv.first.first != dev) continue;
                for (auto& bl : kv.second) {
                    if (bl.idle || bl.seq > seq0) continue;
                    bl.idle = true;
                    auto sb = stream_bytes_.find({dev, bl.s});
                    if (sb != stream_bytes_.end() && (sb->second -= kv.first.second) == 0) stream_bytes_.erase(sb);
                }
            }
            auto it = free_.find({dev, rb});
            if (it != free_.end()) {
                auto& v = it->second;
                for (size_t i = 0; i < v.size(); ++i)
                    if (v[i].idle || v[i].s == s) return take(dev, rb, v, i);
            }
        }
        void* p = b_.alloc(rb);                                // 4. new
        if (!p) {
            std::vector<void*> drop;
            {
                std::lock_guard<std::mutex> lk(mu_);
                for (auto it = free_.begin(); it != free_.end();) {
                    if (it->first.first == dev) {
                        for (auto& bl : it->second) drop.push_back(bl.p);
                        cached_[dev] -= it->first.second * it->second.size();
                        it = free_.erase(it);
                    } else {
                        ++it;
                    }
                }
                for (auto it = stream_bytes_.begin(); it != stream_bytes_.end();)
                    it = it->first.first == dev ? stream_bytes_.erase(it) : std::next(it);
                for (void* q : drop) size_.erase(q);
            }
            b_.sync_device();
            for (void* q : drop) b_.release(q);
            p = b_.alloc(rb);
            if (!p) return nullptr;
        }
        std::lock_guard<std::mutex> lk(mu_);
        size_[p] = rb;
        return p;
    }

    void free(int dev, void* p, Stream s) {
        if (!p) return;
        std::lock_guard<std::mutex> lk(mu_);
        auto it = size_.find(p);
        if (it == size_.end()) return;
        const size_t rb = it->second;
        free_[{dev, rb}].push_back(Block{p, s, false, ++seq_});
        cached_[dev] += rb;
        stream_bytes_[{dev, s}] += rb;
    }

    size_t cached_bytes(int dev) const {
        std::lock_guard<std::mutex> lk(mu_);
        auto it = cached_.find(dev);
        return it == cached_.end() ? 0 : it->second;
    }
    // blocks the backend has handed out and not taken back (in use or cached)
    size_t live_blocks() const {
        std::lock_guard<std::mutex> lk(mu_);
        return size_.size();
    }
    size_t reclaims() const {
        std::lock_guard<std::mutex> lk(mu_);
        return reclaims_;
    }

  private:
    struct Block {
        void* p;
        Stream s;
        bool idle;
        unsigned long long seq;                        // order of the free
    };

    // cached bytes of dev that belong to streams other than s (not idle)
    size_t foreign_bytes(int dev, Stream s) const {
        size_t total = 0;
        for (auto& kv : stream_bytes_)
            if (kv.first.first == dev && !(kv.first.second == s)) total += kv.second;
        return total;
    }

    void* take(int dev, size_t rb, std::vector<Block>& v, size_t i) {
        const Block bl = v[i];
        v.erase(v.begin() + (std::ptrdiff_t)i);
        cached_[dev] -= rb;
        if (!bl.idle) {
            auto it = stream_bytes_.find({dev, bl.s});
            if (it != stream_bytes_.end() && (it->second -= rb) == 0) stream_bytes_.erase(it);
        }
        return bl.p;
    }

    B& b_;
    mutable std::mutex mu_;
    std::map<std::pair<int, size_t>, std::vector<Block>> free_;
    std::map<std::pair<int, Stream>, size_t> stream_bytes_;   // non-idle cached bytes per stream
    std::map<int, size_t> cached_;                             // cached bytes per device
    std::map<void*, size_t> size_;
    size_t reclaims_ = 0;
    unsigned long long seq_ = 0;                       // frees so far
};

}  // namespace acfun
