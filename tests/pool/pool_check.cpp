// Host-only checks of the device pool's caching policy (acfun_amd/csrc/pool.hpp)
// with a mock backend whose "device" counts synchronizations.  Prints "ok"
// and exits 0 when every check holds.
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <map>
#include <vector>

#include "../../acfun_amd/csrc/pool.hpp"

namespace {
struct Mock {
    int allocs = 0, releases = 0, syncs = 0;
    long long budget = 1ll << 40;           // bytes the "device" may hand out
    long long used = 0;
    std::map<void*, size_t> live;
    ~Mock() {
        for (auto& kv : live) std::free(kv.first);
    }
    void* alloc(size_t b) {
        if (used + (long long)b > budget) return nullptr;
        used += (long long)b;
        ++allocs;
        void* p = std::malloc(b);
        live[p] = b;
        return p;
    }
    void release(void* p) {
        ++releases;
        used -= (long long)live[p];
        live.erase(p);
        std::free(p);
    }
    std::function<void()> on_sync;          // runs during a sync (another host thread)
    void sync_device() {
        ++syncs;
        if (on_sync) on_sync();
    }
};

using Pool = acfun::PoolCore<Mock, int>;
int fails = 0;
void expect(bool c, const char* what) {
    if (!c) { std::printf("FAIL: %s\n", what); ++fails; }
}
}  // namespace

int main() {
    {   // one stream, steady state: every block reused, never a sync
        Mock m;
        Pool pool(m);
        for (int it = 0; it < 1000; ++it) {
            void* a = pool.alloc(0, 3 << 20, 7);
            void* b = pool.alloc(0, 100, 7);
            pool.free(0, b, 7);
            pool.free(0, a, 7);
        }
        expect(m.allocs == 2, "single stream allocates its two blocks once");
        expect(m.syncs == 0, "single stream never synchronizes");
    }
    {   // a stream per call, dropped after: bounded growth through reclaims
        Mock m;
        Pool pool(m);
        for (int stream = 1; stream <= 2000; ++stream) {
            void* a = pool.alloc(0, 3 << 20, stream);
            void* b = pool.alloc(0, 100, stream);
            pool.free(0, b, stream);
            pool.free(0, a, stream);
        }
        const size_t bound = Pool::kReclaimBytes / (3 << 20) + 2;   // blocks of the large size
        expect(m.allocs <= (int)(2 * bound), "stream-per-call growth bounded by the reclaim threshold");
        expect(m.syncs > 0 && m.syncs <= 2000 / (int)(bound - 2) + 1, "few reclaims");
        expect(pool.reclaims() == (size_t)m.syncs, "each sync is a reclaim");
    }
    {   // a block another thread frees while the reclaim's sync runs keeps its stream:
        // the work it was freed after may have been queued after the sync began
        Mock m;
        Pool pool(m);
        const size_t S = 8 << 20;
        std::vector<void*> v;
        for (int i = 0; i < 9; ++i) v.push_back(pool.alloc(0, S, 100 + i));   // 72 MiB on other streams
        void* late = pool.alloc(0, S, 50);
        for (int i = 0; i < 9; ++i) pool.free(0, v[i], 100 + i);
        m.on_sync = [&]() { pool.free(0, late, 50); };
        std::vector<void*> got{pool.alloc(0, S, 7)};                          // reclaims
        m.on_sync = nullptr;
        expect(m.syncs == 1, "one reclaim");
        for (int i = 0; i < 9; ++i) got.push_back(pool.alloc(0, S, 7));       // the reclaimed blocks, one more
        bool clean = m.syncs == 1;
        for (void* g : got) clean = clean && g != late;
        expect(clean, "a block freed during the sync is not handed to another stream");
        expect(pool.alloc(0, S, 50) == late, "its own stream reuses it");
    }
    {   // a block of another live stream is never handed out without a sync
        Mock m;
        Pool pool(m);
        void* a = pool.alloc(0, 4096, 1);
        pool.free(0, a, 1);
        void* b = pool.alloc(0, 4096, 2);
        expect(b != a && m.syncs == 0, "other stream's block not reused below the threshold");
        void* c = pool.alloc(0, 4096, 1);
        expect(c == a, "same stream reuses at once (stream order)");
    }
    {   // reclaimed (idle) blocks serve any stream; devices and sizes do not mix
        Mock m;
        Pool pool(m);
        void* big[24];
        for (int i = 0; i < 24; ++i) big[i] = pool.alloc(0, 3 << 20, 1);
        for (int i = 0; i < 24; ++i) pool.free(0, big[i], 1);    // 72 MiB cached on stream 1
        void* x = pool.alloc(0, 3 << 20, 2);                      // triggers the reclaim
        expect(m.syncs == 1 && m.allocs == 24, "reclaim reuses instead of allocating");
        void* y = pool.alloc(0, 3 << 20, 3);
        expect(m.syncs == 1 && m.allocs == 24 && y != x, "idle blocks serve a third stream, no sync");
        void* z = pool.alloc(1, 3 << 20, 3);
        expect(m.allocs == 25, "other device gets its own block");
        void* w = pool.alloc(0, 2 << 20, 3);
        expect(m.allocs == 26 && w != z, "other size class gets its own block");
    }
    {   // out of memory: cached blocks are released after a device sync, then the allocation retried
        Mock m;
        m.budget = 6 << 20;
        Pool pool(m);
        void* a = pool.alloc(0, 4 << 20, 1);
        pool.free(0, a, 1);
        void* b = pool.alloc(0, 5 << 20, 2);         // does not fit beside the cached 4 MiB
        expect(b != nullptr, "allocation succeeds after the cache is dropped");
        expect(m.syncs == 1 && m.releases == 1, "cache dropped once, after a device sync");
        expect(pool.cached_bytes(0) == 0, "nothing cached after the drop");
        expect(pool.alloc(0, 2 << 20, 2) == nullptr, "a request beyond the budget fails");
    }
    {   // cached bytes account both ways; foreign pointers are ignored
        Mock m;
        Pool pool(m);
        void* a = pool.alloc(0, 1 << 20, 1);
        void* b = pool.alloc(0, 1 << 20, 1);
        pool.free(0, a, 1);
        pool.free(0, b, 1);
        expect(pool.cached_bytes(0) == (size_t)(2 << 20), "two MiB cached");
        (void)pool.alloc(0, 1 << 20, 1);
        expect(pool.cached_bytes(0) == (size_t)(1 << 20), "one MiB cached after a reuse");
        pool.free(0, nullptr, 1);
        pool.free(0, (void*)&m, 1);
        expect(pool.cached_bytes(0) == (size_t)(1 << 20), "foreign pointers ignored");
    }
    if (fails) return 1;
    std::printf("ok\n");
    return 0;
}
