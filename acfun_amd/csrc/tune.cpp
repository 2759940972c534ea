// tune.cpp -- the tile search, replacing the reference's cache-blocking
// autotune (src/autotune.cpp:29-30,89-142,148-302,336-388).
//
// The reference times (KC, NC) cache blocks for its CPU micro-kernel per
// GEMM shape and caches the winners per machine.  Here the free parameters
// are the launch shapes of the kernels that run:
//   "g32"   k_gemm32 (fp32 GEMM, 1x1 and implicit-GEMM convs): tile, stages and
//           K groups;
//   "i8mm"  k_i8mm (int8 convs): tile and stages;
//   "w23"   the F(2,3) unit kernels: unit width and persistent or one unit per
//           workgroup;
//   "f32"   k_gemm_f32 (the unaligned fallback): tile and split-K.
// A kernel family asks tune_lookup() for its shape's choice and, the first
// time a shape is seen in a process, registers it with tune_record() together
// with a maker that can replay the launch on scratch operands of that shape.
// acfun_autotune() times, for every registered shape (plus the GEMM shapes
// named in ACFUN_TUNE_SHAPES="MxNxK,..."), the built-in choice (candidate -1 of
// the runner) and every candidate in three interleaved rounds, adopts a
// candidate only when it beats the built-in choice by more than 3%
// (tune_rule.hpp; choice -1 keeps the built-in one) and writes the table to
// the cache file ($ACFUN_TUNE_CACHE, else $HOME/.cache/acfun_amd/tune.txt), one
// line per (arch, kind, shape):
//   <arch> <kind> <ncand> <k0>,<k1>,... <choice>
// so one file serves several GPU types.  Later processes read it at first
// use; ACFUN_AUTOTUNE=1 runs the search at the first GEMM of a process.
#include <sys/stat.h>

#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

#include "rt.hpp"
#include "tune_rule.hpp"

namespace acfun {
namespace {

using TKey = std::tuple<std::string, std::string, std::vector<int>>;   // arch, kind, shape
struct Pending { std::string arch, kind; std::vector<int> key; int ncand; TuneMaker maker; };

std::mutex g_mu;
std::map<TKey, std::pair<int, int>> g_table;    // (choice, candidates) per point, all arches
std::map<TKey, size_t> g_index;                 // points registered in this process -> g_pending
std::vector<Pending> g_pending;
bool g_loaded = false;
bool g_busy = false;
std::string g_status = "default heuristics (no tile search run)";
long long g_hits = 0;                           // launches that used a searched choice
int g_adopted = 0;                              // shapes whose search replaced the built-in choice
std::string g_status_out;

std::string cache_path() {
    if (const char* p = std::getenv("ACFUN_TUNE_CACHE"); p && *p) return p;
    const char* h = std::getenv("HOME");
    return std::string(h ? h : "/tmp") + "/.cache/acfun_amd/tune.txt";
}

void load_cache_locked() {
    if (g_loaded) return;
    g_loaded = true;
    FILE* f = fopen(cache_path().c_str(), "r");
    if (!f) return;
    char arch[64], kind[16], keys[512];
    int ncand, choice, n = 0;
    while (fscanf(f, "%63s %15s %d %511s %d", arch, kind, &ncand, keys, &choice) == 5) {
        std::vector<int> key;
        for (char* t = strtok(keys, ","); t; t = strtok(nullptr, ",")) key.push_back(atoi(t));
        if (choice < -1 || choice >= ncand || key.empty()) continue;
        g_table[TKey{arch, kind, key}] = {choice, ncand};
        ++n;
    }
    fclose(f);
    if (n) g_status = "tile table from cache " + cache_path() + " (" + std::to_string(n) + " shapes)";
}

// mkdir -p with mkdir(2) on each path component (no shell, no child process).
bool make_dirs(const std::string& dir) {
    for (size_t i = 1; i <= dir.size(); ++i) {
        if (i < dir.size() && dir[i] != '/') continue;
        const std::string part = dir.substr(0, i);
        if (mkdir(part.c_str(), 0755) != 0 && errno != EEXIST) return false;
    }
    struct stat st;
    return stat(dir.c_str(), &st) == 0 && S_ISDIR(st.st_mode);
}

bool save_cache_locked() {
    const std::string p = cache_path();
    const size_t slash = p.rfind('/');
    if (slash != std::string::npos && slash > 0 && !make_dirs(p.substr(0, slash))) return false;
    FILE* f = fopen(p.c_str(), "w");
    if (!f) return false;
    for (auto& kv : g_table) {
        const auto& [arch, kind, key] = kv.first;
        std::string ks;
        for (size_t i = 0; i < key.size(); ++i) ks += (i ? "," : "") + std::to_string(key[i]);
        fprintf(f, "%s %s %d %s %d\n", arch.c_str(), kind.c_str(), kv.second.second, ks.c_str(),
                kv.second.first);
    }
    return fclose(f) == 0;
}

// Mean time of one run of candidate c (-1: the built-in choice) over one
// timed batch of five; a candidate the shape does not admit returns +inf.
float time_batch(const TuneRunner& run, int c, hipStream_t s, hipEvent_t e0, hipEvent_t e1) {
    if (hipEventRecord(e0, s) != hipSuccess) return 1e30f;
    for (int i = 0; i < 5; ++i)
        if (!run(c, s)) return 1e30f;
    if (hipEventRecord(e1, s) != hipSuccess || hipEventSynchronize(e1) != hipSuccess) return 1e30f;
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, e0, e1) != hipSuccess) return 1e30f;
    return ms / 5.f;
}

}  // namespace

const char* device_arch() {
    static std::mutex mu;
    static std::string names[16];
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= 16) return "unknown";
    std::lock_guard<std::mutex> lk(mu);
    if (names[d].empty()) {
        hipDeviceProp_t pr;
        if (hipGetDeviceProperties(&pr, d) != hipSuccess) return "unknown";
        std::string a = pr.gcnArchName;
        names[d] = a.substr(0, a.find(':'));
    }
    return names[d].c_str();
}

int tune_lookup(const char* kind, const std::vector<int>& key, int ncand, bool* record) {
    *record = false;
    const TKey k{device_arch(), kind, key};
    std::lock_guard<std::mutex> lk(g_mu);
    load_cache_locked();
    auto it = g_table.find(k);
    // a choice searched over another candidate list (an older build) is ignored
    if (it != g_table.end() && it->second.second == ncand) {
        ++g_hits;
        return it->second.first;
    }
    *record = !g_busy && g_index.find(k) == g_index.end();
    return -1;
}

void tune_record(const char* kind, const std::vector<int>& key, int ncand, TuneMaker maker) {
    TKey k{device_arch(), kind, key};
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_busy || g_index.count(k)) return;
    g_index[k] = g_pending.size();
    g_pending.push_back(Pending{std::get<0>(k), kind, key, ncand, std::move(maker)});
}

bool autotune_wanted() {
    static int want = -1;
    std::lock_guard<std::mutex> lk(g_mu);
    if (want < 0) {
        const char* e = std::getenv("ACFUN_AUTOTUNE");
        want = e && std::atoi(e) > 0 ? 1 : 0;
        return want == 1;
    }
    return false;
}

void autotune_run() {
    // GEMM shapes named in the environment join the shapes this process ran
    if (const char* e = std::getenv("ACFUN_TUNE_SHAPES")) {
        std::string s(e);
        size_t pos = 0;
        while (pos < s.size()) {
            size_t nx = s.find(',', pos);
            std::string t = s.substr(pos, nx == std::string::npos ? std::string::npos : nx - pos);
            int M, N, K;
            if (sscanf(t.c_str(), "%dx%dx%d", &M, &N, &K) == 3 && M > 0 && N > 0 && K > 0)
                gemm32_register(M, N, K);
            if (nx == std::string::npos) break;
            pos = nx + 1;
        }
    }
    std::vector<Pending> todo;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        load_cache_locked();
        if (g_busy) return;
        g_busy = true;
        todo.swap(g_pending);
        g_index.clear();
    }
    hipStream_t s = lib_stream();
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int tuned = 0;
    if (hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess) {
        for (Pending& p : todo) {
            const TKey k{p.arch, p.kind, p.key};
            {
                std::lock_guard<std::mutex> lk(g_mu);
                auto it = g_table.find(k);
                if (it != g_table.end() && it->second.second == p.ncand) continue;
            }
            TuneRunner run = p.maker ? p.maker() : TuneRunner();
            if (!run) continue;
            // index 0: the built-in choice (runner candidate -1), then the candidates;
            // one untimed run each, then three rounds that time every one in turn
            std::vector<float> ms(p.ncand + 1, 1e30f);
            std::vector<bool> ok(p.ncand + 1, false);
            for (int c = -1; c < p.ncand; ++c) ok[c + 1] = run(c, s);
            for (int r = 0; r < 3; ++r)
                for (int c = -1; c < p.ncand; ++c)
                    if (ok[c + 1]) ms[c + 1] = std::min(ms[c + 1], time_batch(run, c, s, e0, e1));
            (void)hipStreamSynchronize(s);
            const int choice = tune_pick(ms[0], ms.data() + 1, p.ncand);
            if (choice < 0 && !(ms[0] < 1e29f)) continue;   // nothing could be timed
            std::lock_guard<std::mutex> lk(g_mu);
            g_table[k] = {choice, p.ncand};
            if (choice >= 0) ++g_adopted;
            ++tuned;
        }
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipStreamSynchronize(s);
    (void)hipGetLastError();     // a candidate refused by the runtime leaves no error behind
    std::lock_guard<std::mutex> lk(g_mu);
    const bool saved = save_cache_locked();
    g_busy = false;
    g_status = "tile search (" + std::string(device_arch()) + "): " + std::to_string(tuned) +
               " shapes searched, " + std::to_string(g_adopted) +
               " beat their built-in choice by more than 3%, " +
               (saved ? "cached at " : "NOT cached (cannot write) ") + cache_path();
}

const char* tune_status() {
    std::lock_guard<std::mutex> lk(g_mu);
    load_cache_locked();
    g_status_out = g_status + "; " + std::to_string(g_hits) + " launches used a searched choice";
    return g_status_out.c_str();
}

}  // namespace acfun
