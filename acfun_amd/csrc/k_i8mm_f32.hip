// k_i8mm_f32.hip -- the fp32-output instantiations of k_i8mm (i8mm.hpp): the
// reference's float-I/O int8 convolution routes, with the optional fused
// residual and the per-workgroup output maxima a model's next int8 layer uses.
#include "i8mm.hpp"

#include <algorithm>

namespace acfun {
namespace {
using namespace i8k;

template <int BM, int BN, int NST, int AM, int EPI>
bool launch_t(I8M& p, const I8Tile& t, hipStream_t s) {
    constexpr size_t lds = i8mm_lds(BM, BN, NST);
    static_assert(lds <= 160 * 1024, "k_i8mm LDS");
    // set once per process, thread-safely, before any launch below
    static const bool attr = [&] {
        (void)hipFuncSetAttribute((const void*)k_i8mm<BM, BN, NST, AM, EPI, OUT_F32>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        return true;
    }();
    (void)attr;
    i8mm_prepare(p, BM, BN);
    dim3 grid((unsigned)i8mm_grid(p, t));
    p.grid = (int)grid.x;
    ACFUN_LAUNCH("k_i8mm", (k_i8mm<BM, BN, NST, AM, EPI, OUT_F32>), grid, dim3(256), lds, s, p);
    return check_launch("k_i8mm");
}

template <int AM, int EPI>
bool launch_tile(I8M& p, const I8Tile& t, hipStream_t s) {
#define ACFUN_I8MM(BM, BN, NST) \
    if (t.bm == BM && t.bn == BN && t.nst == NST) return launch_t<BM, BN, NST, AM, EPI>(p, t, s);
    ACFUN_I8MM(64, 64, 2) ACFUN_I8MM(64, 64, 3) ACFUN_I8MM(128, 64, 3) ACFUN_I8MM(64, 128, 3)
    ACFUN_I8MM(128, 128, 2)
#undef ACFUN_I8MM
    set_error("k_i8mm: no fp32 tile %dx%dx%d", t.bm, t.bn, t.nst);
    return false;
}

template <int EPI>
bool launch_epi(I8M& p, const I8Tile& t, int am, hipStream_t s) {
    if (am == AM_C128) return launch_tile<AM_C128, EPI>(p, t, s);
    if (am == AM_C64) return launch_tile<AM_C64, EPI>(p, t, s);
    return launch_tile<AM_GEN, EPI>(p, t, s);
}
}  // namespace

int i8mm_grid(const I8M& p, const I8Tile& t) {
    const long long total = (long long)((p.M + t.bm - 1) / t.bm) * ((p.N + t.bn - 1) / t.bn);
    long long g = total;
    if (t.per_cu > 0) {
        // at most per_cu persistent workgroups per CU, a multiple of 8 (the per-XCD runs)
        g = std::min(total, (long long)t.per_cu * num_cus());
        if (g >= 8) g &= ~7ll;
    }
    // one output-maximum partial per workgroup where a pass reports them
    if (g > kAmaxParts) g = kAmaxParts;
    return (int)g;
}

bool launch_i8mm_f32(I8M& p, const I8Tile& t, int am, hipStream_t s) {
    if (p.epi == EPI_WINO) return launch_epi<EPI_WINO>(p, t, am, s);
    return launch_epi<EPI_GEMM>(p, t, am, s);
}

}  // namespace acfun
