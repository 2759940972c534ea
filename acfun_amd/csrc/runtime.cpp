// runtime.cpp -- device bring-up, library stream, caching pool, staging of
// host buffers for the synchronous API, and the error string.
#include "rt.hpp"
#include "pool.hpp"

#include <cstdarg>
#include <cstdio>
#include <algorithm>
#include <cstring>
#include <map>
#include <mutex>
#include <string>

namespace acfun {

// ------------------------------------------------------------------ errors
static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

const char* last_error() { return g_err; }

bool check(hipError_t e, const char* what) {
    if (e == hipSuccess) return true;
    set_error("%s: %s", what, hipGetErrorString(e));
    return false;
}

bool check_launch(const char* kernel) { return check(hipGetLastError(), kernel); }

// ------------------------------------------------------------------ timing
namespace {
struct ProfLaunch {
    hipEvent_t start, stop;
    hipEvent_t prev;     // stop event of the previous timed launch on the stream (or null)
    int tag;             // prof_tag() at the launch (a model's layer index; -1 outside models)
};
struct ProfKernel {
    std::vector<ProfLaunch> ev;                           // events created on demand, reused
    size_t used = 0;
};
std::map<hipStream_t, hipEvent_t> g_prof_last;            // last timed stop event per stream
bool g_prof_on = false;
int g_prof_tag = -1;
std::map<std::string, ProfKernel> g_prof;
std::mutex g_prof_mu;
std::string g_prof_layers;                                // model layer records (prof_layer)

// Duration of one recorded launch in ms (see acfun_prof_kernel_ms), -1 on error.
double launch_ms(const ProfLaunch& e) {
    if (hipEventSynchronize(e.stop) != hipSuccess) return -1.0;
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, e.start, e.stop) != hipSuccess) return -1.0;
    // A dispatch's start event can be signalled while it still waits for the
    // previous kernel on its stream: count from that kernel's end then.
    float since_prev = 0.f;
    if (e.prev && hipEventElapsedTime(&since_prev, e.prev, e.stop) == hipSuccess &&
        since_prev > 0.f && since_prev < ms)
        ms = since_prev;
    return ms;
}
}  // namespace

void prof_tag(int tag) { g_prof_tag = tag; }

bool prof_on() { return g_prof_on; }

void prof_layer(const char* record) {
    if (!g_prof_on) return;
    std::lock_guard<std::mutex> lk(g_prof_mu);
    g_prof_layers += record;
    g_prof_layers += '\n';
}

bool prof_events(const char* kernel, hipStream_t s, hipEvent_t* start, hipEvent_t* stop) {
    if (!g_prof_on) return false;
    std::lock_guard<std::mutex> lk(g_prof_mu);
    ProfKernel& k = g_prof[kernel];
    if (k.used == k.ev.size()) {
        hipEvent_t a, b;
        if (hipEventCreate(&a) != hipSuccess) return false;
        if (hipEventCreate(&b) != hipSuccess) { (void)hipEventDestroy(a); return false; }
        k.ev.push_back(ProfLaunch{a, b, nullptr, -1});
    }
    ProfLaunch& L = k.ev[k.used++];
    L.tag = g_prof_tag;
    auto it = g_prof_last.find(s);
    L.prev = it == g_prof_last.end() ? nullptr : it->second;
    g_prof_last[s] = L.stop;
    *start = L.start;
    *stop = L.stop;
    return true;
}

// ------------------------------------------------------------------ device
namespace {
constexpr int kMaxDev = 16;
struct DevState {
    bool init = false;
    bool usable = false;
    hipStream_t stream = nullptr;
    int cus = 0;
};
DevState g_dev[kMaxDev];
std::mutex g_dev_mu;

int current_device() {
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess) return -1;
    return d;
}
}  // namespace

bool ensure_device() {
    int d = current_device();
    if (d < 0 || d >= kMaxDev) {
        int n = 0;
        hipError_t e = hipGetDeviceCount(&n);
        set_error("no usable HIP device (hipGetDeviceCount: %s, count %d)",
                  hipGetErrorString(e), n);
        return false;
    }
    DevState& st = g_dev[d];
    if (st.init) {
        if (!st.usable) set_error("device %d is not a gfx950 GPU", d);
        return st.usable;
    }
    std::lock_guard<std::mutex> lk(g_dev_mu);
    if (!st.init) {
        hipDeviceProp_t prop;
        if (!check(hipGetDeviceProperties(&prop, d), "hipGetDeviceProperties")) return false;
        st.usable = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0;
        st.cus = prop.multiProcessorCount;
        if (st.usable) {
            // Default priority, non-blocking with respect to the null stream.
            if (!check(hipStreamCreateWithFlags(&st.stream, hipStreamNonBlocking),
                       "hipStreamCreate")) {
                st.usable = false;
            }
        } else {
            set_error("device %d is %s, this library is built for gfx950 only", d,
                      prop.gcnArchName);
        }
        st.init = true;
    }
    return st.usable;
}

hipStream_t lib_stream() {
    int d = current_device();
    return (d >= 0 && d < kMaxDev) ? g_dev[d].stream : nullptr;
}

int num_cus() {
    int d = current_device();
    return (d >= 0 && d < kMaxDev && g_dev[d].cus > 0) ? g_dev[d].cus : 256;
}

// ------------------------------------------------------------------ memory
namespace {
// HIP side of the pool (pool.hpp).
struct HipPoolBackend {
    void* alloc(size_t bytes) {
        void* p = nullptr;
        if (hipMalloc(&p, bytes) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
        return p;
    }
    void release(void* p) { (void)hipFree(p); }
    void sync_device() { (void)hipDeviceSynchronize(); }
};
HipPoolBackend g_pool_backend;
PoolCore<HipPoolBackend, hipStream_t> g_pool(g_pool_backend);
}  // namespace

void* pool_alloc(size_t bytes, hipStream_t s) {
    void* p = g_pool.alloc(current_device(), bytes, s);
    if (!p) set_error("hipMalloc: out of device memory (%zu bytes)", bytes);
    return p;
}

void pool_free(void* p, hipStream_t s) { g_pool.free(current_device(), p, s); }

size_t pool_cached_bytes() { return g_pool.cached_bytes(current_device()); }

void* Arena::get(size_t bytes) {
    if (!base_) {
        owned_.emplace_back(bytes ? bytes : 1, s_);
        if (!owned_.back().p) return nullptr;
        return owned_.back().p;
    }
    const size_t need = aligned(bytes ? bytes : 1);
    if (need > cap_ - used_) {
        set_error("scratch region exhausted (%zu of %zu bytes used, %zu more needed)", used_, cap_,
                  need);
        return nullptr;
    }
    void* p = base_ + used_;
    used_ += need;
    return p;
}

bool is_device_ptr(const void* p) {
    if (!p) return false;
    hipPointerAttribute_t a;
    hipError_t e = hipPointerGetAttributes(&a, p);
    if (e != hipSuccess) {
        (void)hipGetLastError();  // unregistered host memory: clear the sticky status
        return false;
    }
    return a.type == hipMemoryTypeDevice || a.type == hipMemoryTypeManaged;
}

// ------------------------------------------------------------------ staging
HostCall::~HostCall() {
    for (void* p : owned_) pool_free(p, s_);
}

const void* HostCall::in(const void* host, size_t bytes) {
    if (!host || bytes == 0 || failed_) return host;
    if (is_device_ptr(host)) return host;
    void* d = pool_alloc(bytes, s_);
    if (!d) { failed_ = true; return nullptr; }
    owned_.push_back(d);
    if (!check(hipMemcpyAsync(d, host, bytes, hipMemcpyHostToDevice, s_), "H2D copy")) {
        failed_ = true;
        return nullptr;
    }
    return d;
}

void* HostCall::out(void* host, size_t bytes) {
    if (!host || bytes == 0 || failed_) return host;
    if (is_device_ptr(host)) return host;
    void* d = pool_alloc(bytes, s_);
    if (!d) { failed_ = true; return nullptr; }
    owned_.push_back(d);
    back_.push_back({host, d, bytes});
    return d;
}

void* HostCall::inout(void* host, size_t bytes) {
    if (!host || bytes == 0 || failed_) return host;
    if (is_device_ptr(host)) return host;
    void* d = const_cast<void*>(in(host, bytes));
    if (d) back_.push_back({host, d, bytes});
    return d;
}

bool HostCall::finish() {
    bool ok = !failed_;
    if (ok) {
        for (auto& b : back_) {
            if (!check(hipMemcpyAsync(b.host, b.dev, b.bytes, hipMemcpyDeviceToHost, s_),
                       "D2H copy")) { ok = false; break; }
        }
    }
    if (!check(hipStreamSynchronize(s_), "hipStreamSynchronize")) ok = false;
    return ok;
}

}  // namespace acfun

// ------------------------------------------------------------------ C ABI: timing
extern "C" void acfun_prof_enable(int on) {
    std::lock_guard<std::mutex> lk(acfun::g_prof_mu);
    if (on) {                            // a new measurement starts empty; off keeps the records
        for (auto& kv : acfun::g_prof) kv.second.used = 0;
        acfun::g_prof_last.clear();
        acfun::g_prof_layers.clear();
    }
    acfun::g_prof_on = on != 0;
}

extern "C" double acfun_prof_kernel_ms(const char* kernel, int* launches) {
    if (launches) *launches = 0;
    if (!kernel) return 0.0;
    std::lock_guard<std::mutex> lk(acfun::g_prof_mu);
    auto it = acfun::g_prof.find(kernel);
    if (it == acfun::g_prof.end() || it->second.used == 0) return 0.0;
    double total = 0.0;
    for (size_t i = 0; i < it->second.used; ++i) {
        const double ms = acfun::launch_ms(it->second.ev[i]);
        if (ms < 0) {
            acfun::set_error("acfun_prof_kernel_ms: HIP event query failed");
            return -1.0;
        }
        total += ms;
    }
    if (launches) *launches = (int)it->second.used;
    return total / (double)it->second.used;
}

extern "C" int acfun_prof_report(char* buf, int len) {
    std::string r;
    {
        std::lock_guard<std::mutex> lk(acfun::g_prof_mu);
        // per (tag, kernel): launch count and summed duration
        std::map<std::pair<int, std::string>, std::pair<int, double>> agg;
        for (auto& kv : acfun::g_prof)
            for (size_t i = 0; i < kv.second.used; ++i) {
                const double ms = acfun::launch_ms(kv.second.ev[i]);
                if (ms < 0) {
                    acfun::set_error("acfun_prof_report: HIP event query failed");
                    return -1;
                }
                auto& a = agg[{kv.second.ev[i].tag, kv.first}];
                a.first += 1;
                a.second += ms;
            }
        char line[256];
        for (auto& kv : agg) {
            snprintf(line, sizeof(line), "K\t%d\t%s\t%d\t%.6f\n", kv.first.first,
                     kv.first.second.c_str(), kv.second.first, kv.second.second);
            r += line;
        }
        size_t p = 0;
        while (p < acfun::g_prof_layers.size()) {
            size_t e = acfun::g_prof_layers.find('\n', p);
            if (e == std::string::npos) e = acfun::g_prof_layers.size();
            r += "L\t";
            r += acfun::g_prof_layers.substr(p, e - p);
            r += '\n';
            p = e + 1;
        }
    }
    if (buf && len > 0) {
        const size_t n = std::min(r.size(), (size_t)len - 1);
        memcpy(buf, r.data(), n);
        buf[n] = 0;
    }
    return (int)r.size() + 1;
}
