// k_stem.hip -- convolutions with few input channels (a network's stem, such as
// ResNet-50's 7x7 / stride-2 conv on RGB input), the reference's im2col + GEMM
// route (src/layers.cpp:178-194) for Cin <= 4.
//
// With Cin = 3 the implicit GEMM's K = KH*KW*Cin is small and does not split
// into whole-tap chunks, which leaves the general kernels gathering A element
// by element.  Here a workgroup (256 threads, 2 x 2 waves, one 32 x 32
// v_mfma_f32_32x32x2f32 block per wave) owns 64 consecutive output pixels of
// one image and 64 output channels:
//   - its weights stay in registers for the workgroup's life (k-step s of lane
//     l holds w[2s + l/32][column l%32]), so B costs no memory traffic per tile;
//   - the input rows the 64 pixels read (a window of whole padded rows, each a
//     contiguous run of W*Cin floats in NHWC) come to LDS by DMA
//     (buffer_load_dwordx4 ... lds: a wave instruction fills 256 consecutive
//     window floats; padding reads zeros through an out-of-range offset), two
//     windows deep: the next tile's window loads during this tile's MFMAs.
//     A window row starts lead = pad*Cin rounded up to 4 floats left of the
//     image row, so 4-float groups are 16-byte aligned in both (W*Cin % 4 == 0);
//   - each lane reads its A value of a k-step from the window at its pixel's
//     offset plus the tap's offset (compile-time per k-step);
//   - the epilogue adds the bias, applies the activation and stores from the
//     MFMA layout: a store instruction writes 32 consecutive channels of two
//     pixels, two 128-byte runs.
// Summation is in k order per output (fp32 MFMA), within the fp32 tolerance of
// the reference's GEMM.
#include "rt.hpp"

#include <algorithm>

namespace acfun {
namespace {

typedef float f16s __attribute__((ext_vector_type(16)));

// Launch-derived fields of k_conv_smallc.
struct SmallC {
    int N, H, W, OH, OW, Cout, stride, pad, act;
    int tpi;        // 64-pixel tiles per image
    int tiles;      // N * tpi
    int gct;        // 64-channel tiles of Cout (one per workgroup: blockIdx % gct)
    int rows;       // input rows of a window
    int lead;       // floats of a window row left of the image row: pad*Cin rounded up to 4
    int pitch;      // floats of a window row: lead + ((OW-1)*stride + KW - pad)*Cin, rounded up to 4
    int wsize;      // rows * pitch
    int nchunk;     // 256-float DMA chunks of a window
    int wstride;    // floats of a window region: 256 * nchunk
};

constexpr int kWinMax = 6400;           // floats of one window region (25 KB; two per workgroup)
constexpr int kDump = 256;              // floats after the two regions: target of a wave's spare DMA

constexpr int vm_enc(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0F70; }

template <int KH, int KW, int CIN>
__global__ __launch_bounds__(256, 3) void k_conv_smallc(const float* __restrict__ in, const float* __restrict__ w,
                                                        const float* __restrict__ bias, float* __restrict__ out,
                                                        SmallC c) {
    constexpr int K = KH * KW * CIN, NKS = (K + 1) / 2;
    typedef __attribute__((address_space(3))) void lds_void;
    extern __shared__ float win[];       // two window regions of c.wstride floats, then kDump
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1, r32 = lane & 31, h = lane >> 5;

    // ---- this workgroup: channel tile ct, pixel tiles t0, t0 + tstr, ... (cnt);
    // with one channel tile the pixel tiles go in 8 contiguous runs, one per
    // XCD (workgroup id mod 8), so neighbouring windows share an L2
    const int G = (int)gridDim.x / c.gct, b = (int)blockIdx.x / c.gct, ct = (int)blockIdx.x % c.gct;
    int t0, tstr, cnt;
    if (c.gct == 1 && (G & 7) == 0) {
        const int x = b & 7, i = b >> 3, gx = G >> 3;
        const int sx = (int)(((long long)x * c.tiles) >> 3);
        const int ex = (int)(((long long)(x + 1) * c.tiles) >> 3);
        t0 = sx + i;
        tstr = gx;
        cnt = ex > t0 ? (ex - t0 + gx - 1) / gx : 0;
    } else {
        t0 = b;
        tstr = G;
        cnt = b < c.tiles ? (c.tiles - b + G - 1) / G : 0;
    }
    if (cnt == 0) return;                                       // uniform per workgroup

    // ---- the weights of this lane's column, one per k-step
    const int col = ct * 64 + wn * 32 + r32;
    float bw[NKS];
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
        const int k = 2 * s + h;
        bw[s] = (k < K && col < c.Cout) ? w[(long long)k * c.Cout + col] : 0.0f;
    }
    const float bcol = (bias && col < c.Cout) ? bias[col] : 0.0f;

    // ---- a tile's window: input rows row0 .. row0 + rows - 1 of image n, each
    // the padded columns -pad .. Wp - pad - 1 times Cin (zeros outside the image)
    const int ohw = c.OH * c.OW;
    auto tile_geo = [&](int t, int& n, int& p0, int& oh0) {
        n = t / c.tpi;
        p0 = (t - n * c.tpi) * 64;
        oh0 = p0 / c.OW;
    };
    // Window DMA: chunk k (256 floats) is wave k % 4's instruction k / 4; lane
    // l's 4 floats start at e = 256 k + 4 l, (row r, offset j) = divmod(e,
    // pitch), the same for every tile, stepped by (1024 / pitch, 1024 % pitch)
    // with one carry.  Every wave issues nwi instructions per window (a fixed
    // count keeps every wait fixed); one past the chunks reads zeros into the
    // dump area.
    const __amdgpu_buffer_rsrc_t irs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)in, (short)0, (int)((long long)c.N * c.H * c.W * CIN * 4), 0x00020000);
    const int eb = 256 * wave + 4 * lane;
    const int r0 = eb / c.pitch, j0 = eb - r0 * c.pitch;
    const int dq = 1024 / c.pitch, dr = 1024 - dq * c.pitch;
    const int nwi = (c.nchunk + 3) >> 2;  // DMA instructions per wave and window
    float* const dump = win + 2 * c.wstride;
    auto stage_window = [&](int t, float* dst) {
        int n, p0, oh0;
        tile_geo(t, n, p0, oh0);
        const int row0 = oh0 * c.stride - c.pad;
        const int rowlen = c.W * CIN;
        const int ibase = n * c.H * rowlen;
        int r = r0, j = j0;
        for (int i = 0; i < nwi; ++i) {
            const int k = 4 * i + wave;
            const int ih = row0 + r, jg = j - c.lead;
            const bool ok = k < c.nchunk && 256 * k + 4 * lane < c.wsize && (unsigned)ih < (unsigned)c.H &&
                            (unsigned)jg < (unsigned)rowlen;
            const unsigned v = ok ? (unsigned)(ibase + ih * rowlen + jg) * 4u : 0x80000000u;
            float* const d = k < c.nchunk ? dst + 256 * k : dump;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(irs, (lds_void*)d, 16, v, 0, 0, 0);
            r += dq;
            j += dr;
            if (j >= c.pitch) {
                j -= c.pitch;
                ++r;
            }
        }
    };
    // the window DMA (nwin loads) of tile t was issued before the 16 stores of
    // the previous full tile, or before nothing: leaving those stores
    // outstanding proves the window landed (loads and stores complete in order)
    stage_window(t0, win);
    bool prev_full = false;

    for (int it = 0; it < cnt; ++it) {
        const int t = t0 + it * tstr;
        const float* const cur = win + (it & 1) * c.wstride;
        if (prev_full) __builtin_amdgcn_s_waitcnt(vm_enc(16));
        else __builtin_amdgcn_s_waitcnt(vm_enc(0));
        // the window of tile t is in cur; every wave is past its reads of the other one
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (it + 1 < cnt) stage_window(t + tstr, win + ((it + 1) & 1) * c.wstride);

        int n, p0, oh0;
        tile_geo(t, n, p0, oh0);
        const int npx = ohw - p0 < 64 ? ohw - p0 : 64;
        // this lane's A row: pixel p0 + wm*32 + r32 (rows past the tile read pixel p0)
        const int pr = wm * 32 + r32;
        const int pp = p0 + (pr < npx ? pr : 0);
        const int oh = pp / c.OW, ow = pp - oh * c.OW;
        // Within window row kh, tap k = (kh*KW + kw)*Cin + ch sits at float
        // kw*Cin + ch = k - kh*KW*Cin past the row's start, a compile-time
        // offset.  rb[kh]: this lane's pixel in row kh, plus 1 for half 1
        // (which reads k + 1 in the same row).
        constexpr int KWC = KW * CIN;
        const int lb = (oh - oh0) * c.stride * c.pitch + c.lead - c.pad * CIN + ow * c.stride * CIN + h;
        int rb[KH];
#pragma unroll
        for (int kh = 0; kh < KH; ++kh) rb[kh] = lb + kh * c.pitch;

        f16s acc;
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
#pragma unroll
        for (int s = 0; s < NKS; ++s) {
            const int k0 = 2 * s, kh0 = k0 / KWC, o0 = k0 - kh0 * KWC;
            const int k1 = k0 + 1, kh1 = k1 / KWC;
            float a;
            if (k1 >= K) {
                // the padding k-step of an odd K: half 1 multiplies 0 (not an
                // input value, which could be infinite; it reads half 0's
                // element, the last of the row, to stay inside the window)
                a = cur[rb[kh0] + o0 - h];
                a = h ? 0.0f : a;
            } else if (kh1 == kh0) {
                a = cur[rb[kh0] + o0];
            } else {
                // k0 ends row kh0, k1 starts row kh1
                a = cur[h ? rb[kh1] - 1 : rb[kh0] + o0];
            }
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, bw[s], acc, 0, 0, 0);
        }

        // ---- epilogue: lane l, register e <-> pixel p0 + wm*32 + 8(e/4) + 4(l/32) + e%4, channel col
        const long long obase = (long long)n * ohw + p0;
        const bool full = npx == 64 && (ct + 1) * 64 <= c.Cout;
        if (full) {
            float* const ol = out + (obase + wm * 32 + 4 * h) * c.Cout + col;
#pragma unroll
            for (int e = 0; e < 16; ++e)
                ol[(long long)(8 * (e >> 2) + (e & 3)) * c.Cout] = act_apply(acc[e] + bcol, c.act);
        } else if (col < c.Cout) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int p = wm * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
                if (p < npx) out[(obase + p) * c.Cout + col] = act_apply(acc[e] + bcol, c.act);
            }
        }
        prev_full = full;
    }
    __builtin_amdgcn_s_waitcnt(vm_enc(0));
}

template <int KH, int KW, int CIN>
bool launch_smallc(const float* in, const float* w, const float* bias, float* out, SmallC c, hipStream_t s) {
    const size_t lds = (size_t)(2 * c.wstride + kDump) * sizeof(float);
    // set once per process, thread-safely, before any launch below
    static const bool attr = [] {
        (void)hipFuncSetAttribute((const void*)k_conv_smallc<KH, KW, CIN>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (2 * kWinMax + kDump) * (int)sizeof(float));
        return true;
    }();
    (void)attr;
    // at most three workgroups per CU (the register budget), as LDS allows, a
    // multiple of 8 per channel tile (the per-XCD runs)
    const int fit = std::max(1, (int)((160 * 1024) / (lds + 256)));
    long long gp = std::min<long long>(c.tiles, (long long)std::min(3, fit) * num_cus() / c.gct);
    if (gp < 1) gp = 1;
    if (gp >= 8) gp &= ~7ll;
    ACFUN_LAUNCH("k_conv_smallc", (k_conv_smallc<KH, KW, CIN>), dim3((unsigned)(gp * c.gct)), dim3(256), lds, s, in,
                 w, bias, out, c);
    return check_launch("k_conv_smallc");
}

// the instantiated shapes: (KH, KW, Cin)
bool shape_known(int KH, int KW, int Cin) {
    return (KH == 7 && KW == 7 && Cin == 3) || (KH == 3 && KW == 3 && Cin == 3);
}

// The window geometry of a shape (SmallC's rows .. wstride).
void smallc_geo(const ConvShape& g, SmallC& c) {
    const long long rowsmax = (g.OW + 62) / g.OW + 1;             // output rows of 64 consecutive pixels
    const long long rows = (rowsmax - 1) * g.stride + g.KH;
    const long long lead = (g.pad * g.Cin + 3) & ~3;
    const long long pitch = (lead + ((long long)(g.OW - 1) * g.stride + g.KW - g.pad) * g.Cin + 3) & ~3ll;
    const long long wsize = rows * pitch;
    const bool fits = wsize <= kWinMax;
    c.rows = (int)rows;
    c.lead = (int)lead;
    c.pitch = fits ? (int)pitch : 0;
    c.wsize = fits ? (int)wsize : 0;
    c.nchunk = (c.wsize + 255) / 256;
    c.wstride = 256 * c.nchunk;
}

}  // namespace

bool conv_smallc_ok(const ConvShape& g, int Cout, const float* in) {
    if (!shape_known(g.KH, g.KW, g.Cin) || Cout <= 0 || g.OH <= 0 || g.OW <= 0 || g.stride <= 0 || g.pad < 0)
        return false;
    if ((g.W * g.Cin) % 4 != 0 || (((uintptr_t)in) & 15u) != 0) return false;   // 16-byte DMA groups
    SmallC c{};
    smallc_geo(g, c);
    return c.wsize > 0 && c.wstride <= kWinMax && (long long)g.N * g.H * g.W * g.Cin * 4 < 0x7fffffffll &&
           (long long)g.N * g.OH * g.OW * Cout < (1ll << 40);
}

bool conv_smallc_f32(const ConvShape& g, const float* in, const float* w, const float* bias, int Cout, float* out,
                     int act, hipStream_t s) {
    if (!conv_smallc_ok(g, Cout, in)) {
        set_error("conv_smallc: unsupported shape");
        return false;
    }
    SmallC c{};
    c.N = g.N; c.H = g.H; c.W = g.W; c.OH = g.OH; c.OW = g.OW; c.Cout = Cout;
    c.stride = g.stride; c.pad = g.pad; c.act = act;
    const int ohw = g.OH * g.OW;
    c.tpi = (ohw + 63) / 64;
    c.tiles = g.N * c.tpi;
    c.gct = (Cout + 63) / 64;
    smallc_geo(g, c);
    if (g.KH == 7) return launch_smallc<7, 7, 3>(in, w, bias, out, c, s);
    return launch_smallc<3, 3, 3>(in, w, bias, out, c, s);
}

}  // namespace acfun
