// k_i8mm_q8.hip -- the requantized-output instantiations of k_i8mm (i8mm.hpp):
// OUT_AMAX (first pass: per-workgroup max|v| of the float output, nothing
// stored) and OUT_Q8 (second pass: the same tiles recomputed, requantized to
// s8 with the maximum of the first pass), 64 x 64 tiles.
#include "i8mm.hpp"

namespace acfun {
namespace {
using namespace i8k;

template <int NST, int AM, int EPI, int OUT>
bool launch_t(I8M& p, const I8Tile& t, hipStream_t s) {
    constexpr size_t lds = i8mm_lds(64, 64, NST);
    // set once per process, thread-safely, before any launch below
    static const bool attr = [&] {
        (void)hipFuncSetAttribute((const void*)k_i8mm<64, 64, NST, AM, EPI, OUT>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        return true;
    }();
    (void)attr;
    i8mm_prepare(p, 64, 64);
    dim3 grid((unsigned)i8mm_grid(p, t));
    p.grid = (int)grid.x;
    if (OUT == OUT_AMAX)
        ACFUN_LAUNCH("k_i8mm_amax", (k_i8mm<64, 64, NST, AM, EPI, OUT>), grid, dim3(256), lds, s, p);
    else
        ACFUN_LAUNCH("k_i8mm_q8", (k_i8mm<64, 64, NST, AM, EPI, OUT>), grid, dim3(256), lds, s, p);
    return check_launch("k_i8mm (s8 output)");
}

template <int AM, int EPI, int OUT>
bool launch_nst(I8M& p, const I8Tile& t, hipStream_t s) {
    if (t.nst == 2) return launch_t<2, AM, EPI, OUT>(p, t, s);
    return launch_t<3, AM, EPI, OUT>(p, t, s);
}

template <int EPI, int OUT>
bool launch_am(I8M& p, const I8Tile& t, int am, hipStream_t s) {
    if (am == AM_C128) return launch_nst<AM_C128, EPI, OUT>(p, t, s);
    if (am == AM_C64) return launch_nst<AM_C64, EPI, OUT>(p, t, s);
    return launch_nst<AM_GEN, EPI, OUT>(p, t, s);
}
}  // namespace

bool launch_i8mm_q8(I8M& p, const I8Tile& t, int am, int out, hipStream_t s) {
    if (t.bm != 64 || t.bn != 64) {
        set_error("k_i8mm: the s8 output needs 64x64 tiles (asked %dx%d)", t.bm, t.bn);
        return false;
    }
    if (p.epi == EPI_WINO)
        return out == OUT_AMAX ? launch_am<EPI_WINO, OUT_AMAX>(p, t, am, s)
                               : launch_am<EPI_WINO, OUT_Q8>(p, t, am, s);
    return out == OUT_AMAX ? launch_am<EPI_GEMM, OUT_AMAX>(p, t, am, s)
                           : launch_am<EPI_GEMM, OUT_Q8>(p, t, am, s);
}

}  // namespace acfun
