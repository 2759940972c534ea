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

typedef __attribute__((address_space(3))) void stem_lds;

// The tiles of this workgroup: channel tile ct (blockIdx % gct) and pixel
// tiles t0, t0 + tstr, ... (cnt of them); with one channel tile the pixel
// tiles go in 8 contiguous runs, one per XCD (workgroup id mod 8), so
// neighbouring windows share an L2.
struct StemWork { int ct, t0, tstr, cnt; };
__device__ __forceinline__ StemWork stem_work(const SmallC& c) {
    StemWork w;
    const int G = (int)gridDim.x / c.gct, b = (int)blockIdx.x / c.gct;
    w.ct = (int)blockIdx.x % c.gct;
    if (c.gct == 1 && (G & 7) == 0) {
        const int x = b & 7, i = b >> 3, gx = G >> 3;
        const int sx = (int)(((long long)x * c.tiles) >> 3);
        const int ex = (int)(((long long)(x + 1) * c.tiles) >> 3);
        w.t0 = sx + i;
        w.tstr = gx;
        w.cnt = ex > w.t0 ? (ex - w.t0 + gx - 1) / gx : 0;
    } else {
        w.t0 = b;
        w.tstr = G;
        w.cnt = b < c.tiles ? (c.tiles - b + G - 1) / G : 0;
    }
    return w;
}

// Pixel tile t: image n, first pixel p0 (of OH*OW), its output row oh0.
__device__ __forceinline__ void stem_tile(const SmallC& c, int t, int& n, int& p0, int& oh0) {
    n = t / c.tpi;
    p0 = (t - n * c.tpi) * 64;
    oh0 = p0 / c.OW;
}

// Window DMA of elements of US bytes (4: fp32, 1: s8): chunk k (256 elements)
// is wave k % 4's instruction k / 4; lane l's 4 elements (4 * US bytes) start
// at e = 256 k + 4 l, (row r, offset j) = divmod(e, pitch), the same for every
// tile, stepped by (1024 / pitch, 1024 % pitch) with one carry.  Every wave
// issues nwi instructions per window (a fixed count keeps every wait fixed);
// one past the chunks reads zeros into the dump area.
template <int CIN, int US>
struct StemDma {
    static_assert(US == 4 || US == 1, "StemDma: fp32 or s8 elements");
    __amdgpu_buffer_rsrc_t irs;
    int r0, j0, dq, dr, nwi, wave, lane;
    // nwi_fixed > 0: that many instructions per window (at least the chunks need)
    __device__ __forceinline__ void init(const void* in, const SmallC& c, int wave_, int lane_, int nwi_fixed = 0) {
        wave = wave_;
        lane = lane_;
        irs = __builtin_amdgcn_make_buffer_rsrc((void*)in, (short)0, (int)((long long)c.N * c.H * c.W * CIN * US),
                                                0x00020000);
        const int eb = 256 * wave + 4 * lane;
        r0 = eb / c.pitch;
        j0 = eb - r0 * c.pitch;
        dq = 1024 / c.pitch;
        dr = 1024 - dq * c.pitch;
        nwi = nwi_fixed > 0 ? nwi_fixed : (c.nchunk + 3) >> 2;
    }
    // the window of pixel tile t into dst (a region of c.wstride elements); with
    // live false the same number of instructions, all reading zeros into dump
    __device__ __forceinline__ void issue(const SmallC& c, int t, void* dst, void* dump, bool live = true) const {
        int n, p0, oh0;
        stem_tile(c, t, n, p0, oh0);
        const int row0 = oh0 * c.stride - c.pad;
        const int rowlen = c.W * CIN;
        const int ibase = n * c.H * rowlen;
        int r = r0, j = j0;
        for (int i = 0; i < nwi; ++i) {
            const int k = 4 * i + wave;
            const int ih = row0 + r, jg = j - c.lead;
            const bool ok = live && k < c.nchunk && 256 * k + 4 * lane < c.wsize && (unsigned)ih < (unsigned)c.H &&
                            (unsigned)jg < (unsigned)rowlen;
            const unsigned v = ok ? (unsigned)(ibase + ih * rowlen + jg) * (unsigned)US : 0x80000000u;
            char* const d = live && k < c.nchunk ? (char*)dst + 256 * US * k : (char*)dump;
            if constexpr (US == 4) __builtin_amdgcn_raw_ptr_buffer_load_lds(irs, (stem_lds*)d, 16, v, 0, 0, 0);
            else __builtin_amdgcn_raw_ptr_buffer_load_lds(irs, (stem_lds*)d, 4, v, 0, 0, 0);
            r += dq;
            j += dr;
            if (j >= c.pitch) {
                j -= c.pitch;
                ++r;
            }
        }
    }
};

// Columns c0 .. c0 + 63 of the row-major [K][ld] array src (zero past ld)
// into LDS dst as [K][64], by the workgroup: coalesced loads, 8 in flight per
// thread (loads of clamped, valid indices, then 0 where out of range).
template <typename T>
__device__ __forceinline__ void stem_stage_cols(const T* __restrict__ src, int K, int ld, int c0, T* dst) {
    const int n = K * 64;
    for (int i0 = 0; i0 < n; i0 += 256 * 8) {
        T v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int e = i0 + 256 * u + (int)threadIdx.x;
            const int k = e >> 6, cc = c0 + (e & 63);
            const bool ok = e < n && cc < ld;
            const T x = src[(long long)(ok ? k : 0) * ld + (ok ? cc : 0)];
            v[u] = ok ? x : T(0);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int e = i0 + 256 * u + (int)threadIdx.x;
            if (e < n) dst[e] = v[u];
        }
    }
}

template <int KH, int KW, int CIN>
__global__ __launch_bounds__(256, 3) void k_conv_smallc(const float* __restrict__ in, const float* __restrict__ w,
                                                        const float* __restrict__ bias, float* __restrict__ out,
                                                        SmallC c) {
    constexpr int K = KH * KW * CIN, NKS = (K + 1) / 2;
    extern __shared__ float win[];       // two window regions of c.wstride floats, then kDump
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1, r32 = lane & 31, h = lane >> 5;
    const StemWork wk = stem_work(c);
    const int ct = wk.ct, t0 = wk.t0, tstr = wk.tstr, cnt = wk.cnt;
    if (cnt == 0) return;                                       // uniform per workgroup

    // ---- the weights of this lane's column, one per k-step
    // (through LDS: the workgroup's 64 columns, coalesced, into the window
    // area before any window arrives)
    const int col = ct * 64 + wn * 32 + r32;
    stem_stage_cols<float>(w, K, c.Cout, ct * 64, win);
    __syncthreads();
    float bw[NKS];
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
        const int k = 2 * s + h;
        bw[s] = k < K ? win[k * 64 + wn * 32 + r32] : 0.0f;
    }
    __syncthreads();
    const float bcol = (bias && col < c.Cout) ? bias[col] : 0.0f;

    // ---- a tile's window: input rows row0 .. row0 + rows - 1 of image n (zeros
    // outside the image), by StemDma
    const int ohw = c.OH * c.OW;
    StemDma<CIN, 4> dma;
    dma.init(in, c, wave, lane);
    float* const dump = win + 2 * c.wstride;
    // the window DMA (nwi loads) of tile t was issued before the 16 stores of
    // the previous full tile, or before nothing: leaving those stores
    // outstanding proves the window landed (loads and stores complete in order)
    dma.issue(c, t0, win, dump);
    bool prev_full = false;

    for (int it = 0; it < cnt; ++it) {
        const int t = t0 + it * tstr;
        const float* const cur = win + (it & 1) * c.wstride;
        if (prev_full) __builtin_amdgcn_s_waitcnt(vm_enc(16));
        else __builtin_amdgcn_s_waitcnt(vm_enc(0));
        // the window of tile t is in cur; every wave is past its reads of the other one
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (it + 1 < cnt) dma.issue(c, t + tstr, win + ((it + 1) & 1) * c.wstride, dump);

        int n, p0, oh0;
        stem_tile(c, t, n, p0, oh0);
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
            // all 16 values first, then the 16 stores in one run (the next
            // tile's wait counts exactly these 16)
            float vs[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) vs[e] = act_apply(acc[e] + bcol, c.act);
            float* const ol = out + (obase + wm * 32 + 4 * h) * c.Cout + col;
#pragma unroll
            for (int e = 0; e < 16; ++e) __builtin_nontemporal_store(vs[e], &ol[(long long)(8 * (e >> 2) + (e & 3)) * c.Cout]);
        } else if (col < c.Cout) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int p = wm * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
                if (p < npx) __builtin_nontemporal_store(act_apply(acc[e] + bcol, c.act), &out[(obase + p) * c.Cout + col]);
            }
        }
        prev_full = full;
    }
    __builtin_amdgcn_s_waitcnt(vm_enc(0));
}


// ---------------------------------------------------------------- k_i8stem
constexpr int kI8Win = 3;               // s8 windows in flight per workgroup
constexpr int kI8Nwi = 7;               // DMA instructions per wave and window (28 chunks, 7 KB)
// The int8 form (acfun_conv2d_int8's GEMM route, src/conv_int8.cpp:63-148, for
// the same shapes), in two launches after the absmax partials:
//   - k_quant_s8d writes the input once as dense s8 NHWC (3 bytes a pixel):
//     s8 = u8 - 128 as the reference's conversions give it, with the tensor's
//     scale (every block reduces the partials, as k_quant16 does);
//   - k_i8stem multiplies on v_mfma_i32_32x32x32_i8.  K is laid out as one
//     32-byte row per kernel row kh (bytes kw*Cin + ch, 21 used for 7x7x3; the
//     weights beyond are zero).  The s8 windows come by the same DMA (4 bytes
//     a lane), three deep, padding 0 (the reference's u8 128); lane l's A bytes
//     for row kh are the 16 bytes at its pixel's window offset + 16 (l/32):
//     five aligned dwords joined by alignbyte (bytes past the 21 meet zero
//     weights).  The weights (s8, with their column sums) are built into
//     registers once from the [K][Cout] layout.  The epilogue is k_i8mm's GEMM
//     route: fl(fl(acc_u * alpha) + beta), acc_u = acc_s + 128 * Sw, the
//     activation, and the per-workgroup output maximum.

// The tensor's max|x| from the absmax partials, as k_quant16 reduces them
// (every thread of the block gets it).
__device__ __forceinline__ float stem_maxa(const float* part, int nparts) {
    __shared__ float red[4];
    const int tid = threadIdx.x, lane = tid & 63;
    float m = 0.0f;
    for (int i = tid; i < nparts; i += 256) {
        const float a = part[i];
        m = a > m ? a : m;
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float o = __shfl_xor(m, off, 64);
        m = o > m ? o : m;
    }
    if (lane == 0) red[tid >> 6] = m;
    __syncthreads();
    float maxa = red[0];
    for (int k = 1; k < 4; ++k) maxa = red[k] > maxa ? red[k] : maxa;
    return maxa;
}

// x * 127/max has |.| <= 127 up to rounding (|x| <= max), where the
// reference's clamp(cvt(rint(t)) + 128, 0, 255) - 128 equals a float clamp of
// rint(t) but for NaN, which both send to -128 (fmaxf(NaN, -128) = -128).
__device__ __forceinline__ unsigned stem_q(float x, float inv_s) {
    return (unsigned)(int)fminf(fmaxf(rintf(__fmul_rn(x, inv_s)), -128.0f), 127.0f) & 0xffu;
}

// 16 elements a thread (16-byte loads and store), grid-stride; a ragged end
// element by element.
__global__ __launch_bounds__(256) void k_quant_s8d(const float* __restrict__ x, long long n,
                                                  int8_t* __restrict__ q, const float* __restrict__ part,
                                                  int nparts) {
    const float maxa = stem_maxa(part, nparts);
    const bool zero = maxa < 1e-12f;             // an all-zero input: s8 0 (output 0)
    const float inv_s = 127.0f / maxa;
    typedef int i4s __attribute__((ext_vector_type(4)));
    const long long stride = (long long)gridDim.x * 256;
    for (long long g = (long long)blockIdx.x * 256 + threadIdx.x; g * 16 < n; g += stride) {
        const long long i0 = g * 16;
        if (i0 + 16 <= n) {
            unsigned w[4] = {0u, 0u, 0u, 0u};
            if (!zero) {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float4 v = *(const float4*)(x + i0 + 4 * k);
                    w[k] = stem_q(v.x, inv_s) | (stem_q(v.y, inv_s) << 8) | (stem_q(v.z, inv_s) << 16) |
                           (stem_q(v.w, inv_s) << 24);
                }
            }
            *(i4s*)(q + i0) = i4s{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
        } else {
            for (long long e = i0; e < n; ++e) q[e] = zero ? (int8_t)0 : (int8_t)stem_q(x[e], inv_s);
        }
    }
}

template <int KH, int KW, int CIN>
__global__ __launch_bounds__(256, 3) void k_i8stem(const int8_t* __restrict__ q8, const int8_t* __restrict__ wq,
                                                   const float* __restrict__ ws, const float* __restrict__ bias,
                                                   const float* __restrict__ part, int nparts,
                                                   float* __restrict__ out, float* __restrict__ amax, SmallC c) {
    constexpr int KWC = KW * CIN;
    static_assert(KWC <= 32, "k_i8stem: one 32-byte K row per kernel row");
    typedef int i4s __attribute__((ext_vector_type(4)));
    typedef int i16s __attribute__((ext_vector_type(16)));
    // kI8Win s8 window regions of c.wstride + 64 bytes (the A reads run up to
    // 20 bytes past a row), then the 256-byte dump area
    extern __shared__ float win[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1, r32 = lane & 31, h = lane >> 5;
    const int rs = c.wstride + 64;
    unsigned char* const reg0 = (unsigned char*)win;
    unsigned char* const dump = reg0 + kI8Win * rs;

    const StemWork wk = stem_work(c);
    const int ct = wk.ct, t0 = wk.t0, tstr = wk.tstr, cnt = wk.cnt;
    if (cnt == 0) {                                            // uniform per workgroup
        if (amax && tid == 0) amax[blockIdx.x] = 0.0f;
        return;
    }
    // windows of tiles it and it + 1 in flight ahead of tile it: every window is
    // kI8Nwi DMA instructions per wave (a dead one when there is no tile)
    // ---- this lane's column: B bytes of each kernel row (16 (l/32) ..), the
    // column sum Sw over both halves, and the epilogue factors.  The
    // workgroup's 64 columns come through LDS (coalesced, into the window
    // area before any window arrives).
    const int col = ct * 64 + wn * 32 + r32;
    stem_stage_cols<int8_t>(wq, KH * KWC, c.Cout, ct * 64, (int8_t*)reg0);
    __syncthreads();
    i4s bq[KH];
    int swh = 0;
#pragma unroll
    for (int kh = 0; kh < KH; ++kh) {
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
            unsigned wd = 0;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int j = 16 * h + 4 * qd + b;
                const int v = j < KWC ? (int)((const int8_t*)reg0)[(kh * KWC + j) * 64 + wn * 32 + r32] : 0;
                swh += v;
                wd |= ((unsigned)v & 0xffu) << (8 * b);
            }
            bq[kh][qd] = (int)wd;
        }
    }
    __syncthreads();

    StemDma<CIN, 1> dma;
    dma.init(q8, c, wave, lane, kI8Nwi);
    dma.issue(c, t0, reg0, dump);
    dma.issue(c, t0 + tstr, reg0 + rs, dump, cnt > 1);

    const float maxa = stem_maxa(part, nparts);
    const bool zero = maxa < 1e-12f;             // an all-zero input: output 0 (src/conv_int8.cpp:78)
    const float sa = maxa / 127.0f;

    const int sw = swh + __shfl_xor(swh, 32, 64);
    const int corr = 128 * sw;
    float al = 0.0f, be = 0.0f;
    if (col < c.Cout) {   // src/conv_int8.cpp:100-107: alpha = sa*ws; beta = b - (alpha*128)*Sw
        al = __fmul_rn(sa, ws[col]);
        be = __fsub_rn(bias ? bias[col] : 0.0f, __fmul_rn(__fmul_rn(al, 128.0f), (float)sw));
        if (zero) {
            al = 0.0f;
            be = 0.0f;
        }
    }

    const int ohw = c.OH * c.OW;
    bool full1 = false, full2 = false;          // tiles it - 1 and it - 2 stored 16 values a lane
    float amx = 0.0f;
    int bufi = 0;                               // it % kI8Win
    for (int it = 0; it < cnt; ++it) {
        const int t = t0 + it * tstr;
        const unsigned char* const s8w = reg0 + bufi * rs;
        // After the window DMA of tile it came the window DMA of tile it + 1
        // (kI8Nwi loads) and the stores of tiles it - 2 and it - 1 (16 for a
        // full tile, else counted as none); loads and stores complete in order.
        const int nst = (full1 ? 1 : 0) + (full2 ? 1 : 0);
        if (nst == 2) __builtin_amdgcn_s_waitcnt(vm_enc(kI8Nwi + 32));
        else if (nst == 1) __builtin_amdgcn_s_waitcnt(vm_enc(kI8Nwi + 16));
        else __builtin_amdgcn_s_waitcnt(vm_enc(kI8Nwi));
        // the window of tile it is in place; every wave is past its reads of
        // tile it - 1's window, whose region takes tile it + 2's
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        const int nb2 = bufi == 0 ? 2 : bufi - 1;  // (it + 2) % kI8Win
        dma.issue(c, t + 2 * tstr, reg0 + nb2 * rs, dump, it + 2 < cnt);
        bufi = bufi == kI8Win - 1 ? 0 : bufi + 1;

        int n, p0, oh0;
        stem_tile(c, t, n, p0, oh0);
        const int npx = ohw - p0 < 64 ? ohw - p0 : 64;
        const int pr = wm * 32 + r32;
        const int pp = p0 + (pr < npx ? pr : 0);
        const int oh = pp / c.OW, ow = pp - oh * c.OW;
        // byte of tap (kh, 0, 0) of this lane's pixel in window row kh, plus 16 for half 1
        const int lb = (oh - oh0) * c.stride * c.pitch + c.lead - c.pad * CIN + ow * c.stride * CIN + 16 * h;

        i16s acc;
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] = 0;
#pragma unroll
        for (int kh = 0; kh < KH; ++kh) {
            const int bo = lb + kh * c.pitch;
            const unsigned* const dw = (const unsigned*)(s8w + (bo & ~3));
            const unsigned sh = (unsigned)(bo & 3);
            const unsigned d0 = dw[0], d1 = dw[1], d2 = dw[2], d3 = dw[3], d4 = dw[4];
            i4s a;
            a[0] = (int)__builtin_amdgcn_alignbyte(d1, d0, sh);
            a[1] = (int)__builtin_amdgcn_alignbyte(d2, d1, sh);
            a[2] = (int)__builtin_amdgcn_alignbyte(d3, d2, sh);
            a[3] = (int)__builtin_amdgcn_alignbyte(d4, d3, sh);
            acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bq[kh], acc, 0, 0, 0);
        }

        // ---- epilogue: lane l, register e <-> pixel p0 + wm*32 + 8(e/4) + 4(l/32) + e%4, channel col
        const long long obase = (long long)n * ohw + p0;
        const bool full = npx == 64 && (ct + 1) * 64 <= c.Cout;
        auto value = [&](int e) {
            float v = __fadd_rn(__fmul_rn((float)(int)((unsigned)acc[e] + (unsigned)corr), al), be);
            v = act_apply(v, c.act);
            if (amax) {
                const float av = fabsf(v);
                amx = av > amx ? av : amx;           // NaN never wins
            }
            return v;
        };
        if (full) {
            // all 16 values first, then the 16 stores in one run (the next
            // tile's wait counts exactly these 16)
            float vs[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) vs[e] = value(e);
            float* const ol = out + (obase + wm * 32 + 4 * h) * c.Cout + col;
#pragma unroll
            for (int e = 0; e < 16; ++e) __builtin_nontemporal_store(vs[e], &ol[(long long)(8 * (e >> 2) + (e & 3)) * c.Cout]);
        } else if (col < c.Cout) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int p = wm * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
                if (p < npx) __builtin_nontemporal_store(value(e), &out[(obase + p) * c.Cout + col]);
            }
        }
        full2 = full1;
        full1 = full;
    }
    // this workgroup's max|v| of the output, a partial of the next layer's absmax
    if (amax) {
        __shared__ float wmax[4];
        for (int off = 32; off > 0; off >>= 1) {
            const float o = __shfl_xor(amx, off, 64);
            amx = o > amx ? o : amx;
        }
        if (lane == 0) wmax[wave] = amx;
        __syncthreads();
        if (tid == 0) {
            float mm = wmax[0];
            for (int w = 1; w < 4; ++w) mm = wmax[w] > mm ? wmax[w] : mm;
            amax[blockIdx.x] = mm;
        }
    }
    __builtin_amdgcn_s_waitcnt(vm_enc(0));
}

template <int KH, int KW, int CIN>
bool launch_smallc(const float* in, const float* w, const float* bias, float* out, SmallC c, hipStream_t s) {
    // the windows, or the weight columns staged at the start if larger
    const size_t lds = std::max((size_t)(2 * c.wstride + kDump), (size_t)KH * KW * CIN * 64) * sizeof(float);
    // set once per process, thread-safely, before any launch below
    static const bool attr = [] {
        (void)hipFuncSetAttribute((const void*)k_conv_smallc<KH, KW, CIN>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize,
                                  std::max(2 * kWinMax + kDump, KH * KW * CIN * 64) * (int)sizeof(float));
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

bool conv_i8stem(const ConvShape& g, const float* in, const int8_t* wq, const float* ws, const float* bias,
                 int Cout, float* out, int act, const float* part, int nparts, float* amax, int* grid,
                 int8_t* q8, hipStream_t s) {
    // (one output-maximum partial per workgroup: at most kI8AmaxParts, and at
    // least one workgroup per 64-channel tile)
    if (!conv_smallc_ok(g, Cout, in) || nparts < 0 || nparts > kI8AmaxParts || (Cout + 63) / 64 > kI8AmaxParts ||
        (((uintptr_t)q8) & 15u) != 0) {
        set_error("conv_i8stem: unsupported shape");
        return false;
    }
    SmallC c{};
    c.N = g.N; c.H = g.H; c.W = g.W; c.OH = g.OH; c.OW = g.OW; c.Cout = Cout;
    c.stride = g.stride; c.pad = g.pad; c.act = act;
    c.tpi = (g.OH * g.OW + 63) / 64;
    c.tiles = g.N * c.tpi;
    c.gct = (Cout + 63) / 64;
    smallc_geo(g, c);
    if (c.nchunk > 4 * kI8Nwi) {
        set_error("conv_i8stem: window of %d chunks", c.nchunk);
        return false;
    }
    // the dense s8 input
    const long long n = (long long)g.N * g.H * g.W * g.Cin;
    const long long qb = std::min((n / 16 + 255) / 256 + 1, 8ll * num_cus());
    ACFUN_LAUNCH("k_quant_s8d", k_quant_s8d, dim3((unsigned)qb), dim3(256), 0, s, in, n, q8, part, nparts);
    if (!check_launch("k_quant_s8d")) return false;
    // the windows, or the weight columns staged at the start if larger
    const size_t lds = std::max((size_t)kI8Win * (c.wstride + 64) + 256, (size_t)g.KH * g.KW * g.Cin * 64);
    auto go = [&](auto kern) {
        // at most three workgroups per CU (the register budget), a multiple of
        // 8 per channel tile (the per-XCD runs), at most kI8AmaxParts
        long long gp = std::min<long long>(c.tiles, 3ll * num_cus() / c.gct);
        gp = std::min<long long>(gp, kI8AmaxParts / c.gct);
        if (gp < 1) gp = 1;
        if (gp >= 8) gp &= ~7ll;
        if (grid) *grid = (int)(gp * c.gct);
        ACFUN_LAUNCH("k_i8stem", kern, dim3((unsigned)(gp * c.gct)), dim3(256), lds, s, q8, wq, ws, bias, part,
                     nparts, out, amax, c);
        return check_launch("k_i8stem");
    };
    if (g.KH == 7) return go(k_i8stem<7, 7, 3>);
    return go(k_i8stem<3, 3, 3>);
}

}  // namespace acfun
