// i8mm.hpp -- k_i8mm, the int8 implicit GEMM of the convolution routes, as a
// kernel template shared by the files that instantiate it: k_i8mm_f32.hip
// (fp32 output, the reference's float I/O) and k_i8mm_q8.hip (the two passes
// of a requantized s8 output), compiled in parallel.
#pragma once
#include "rt.hpp"

#include <type_traits>

namespace acfun {

enum { EPI_I32 = 0, EPI_GEMM = 1, EPI_WINO = 2 };

namespace i8k {

typedef int i4 __attribute__((ext_vector_type(4)));
typedef float f4v __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- k_i8mm
// int8 implicit GEMM for the convolution routes: LDS-DMA staging and int8
// MFMA, persistent workgroups.
//
// Workgroup = 256 threads; its waves own a BM x BN output tile as 2 x 2 waves
// of FM x FN v_mfma_i32_32x32x32_i8 blocks (FM = BM/64, FN = BN/64).  K (k' =
// tap*Cinp + ic) is consumed in chunks of 128 bytes; a stage holds A: BM rows
// x 8 quads of 16 bytes and B: BN rows x 8 quads, quad q of row r at slot
// r*8 + (q ^ swz(r)), swz(r) = (r ^ (r >> 3)) & 7, so 8 and 16 consecutive
// rows read at one quad fall on distinct banks.  Both are filled by
// buffer_load_dwordx4 ... lds: a wave instruction fills 64 consecutive slots
// (8 rows); lane l the 16 bytes of row 8I + l/8, slot l%8.  A's 16 bytes are
// 16 channels of one input pixel at one tap (NHWC s8, channels padded to
// Cinp, a multiple of 16); a tap outside the image, a row past M or a k past
// K reads zeros through an out-of-range offset -- s8 0 is the reference's
// padding value u8 128.  NST stages: chunk c+NST-1 is issued while chunk c is
// multiplied, across tile boundaries (a workgroup runs its tiles back to
// back).  In k-step s (32 k) lane half h reads quad 2s+h of its A and B rows
// with one ds_read_b128 each.  At a tile's last chunk each lane forms the
// reference's epilogue for its 16 x FM x FN accumulators, adds the fused
// residual, applies the activation and stores dwords (inline asm, so the
// compiler's wait insertion keeps exact counts for the loads; the waits stay
// correct with stores queued, since loads complete in issue order).
//
// The workgroups' tiles are cut into 8 contiguous runs, one per XCD
// (workgroup id mod 8), so the BN-blocks of one pixel block share an L2.
// A-operand addressing: AM_C128 when Cinp is a multiple of 128 (a chunk lies
// in one tap: tap, offset and bounds test are per chunk and wave-uniform),
// AM_C64 when Cinp = 64 (two taps per chunk), AM_GEN otherwise.
struct I8M {
    const int8_t* A;     // s8 NHWC [N*H*W][Cinp]
    const int8_t* Bt;    // [N][ldb], ldb a multiple of 128, zero beyond taps*Cinp
    int M, N, K, ldb;    // K = taps * Cinp
    int H, W, Cinp, KW, stride, pad, OH, OW;
    unsigned a_bytes, b_bytes;
    int epi, act;
    const int* Sw;       // EPI_GEMM: column sums of the weights
    const float* ws;     // per-channel weight scales (with scal: factors made here)
    const float* bias;   // nullable
    const float* scal;   // device scalars [0] inv_s [1] sa [2] zero flag (nullable)
    const float* s_in;   // or: the activation scale itself (an s8 input; 0 = all-zero input)
    const float* alpha;  // explicit per-channel factors (nullable: made from scal, ws)
    const float* beta;
    const float* res;    // residual added before the activation (nullable)
    float* Cf;
    int ldc, ldr;
    int vec;             // Cf (and res) rows allow 16-byte stores/loads
    int gm, gn;          // grid in tiles
    float* amax;         // per-workgroup max|stored value| at [blockIdx.x] (nullable)
    // OUT_Q8: s8 output [M][ldq] (columns N..ldq-1 written 0), requantized with
    // inv = 127/max over the nqparts partial maxima of the OUT_AMAX pass
    int8_t* Cq;
    int ldq;
    int rule;            // 0: RNE; 1: the Winograd route's input rule (cvec = N & ~15)
    const float* qparts;
    int nqparts;
    float* s_out;        // max/127 (0: all-zero output), written by workgroup 0
    // set by i8mm_prepare: the grid in tiles (gm, gn above) and the float
    // reciprocals of the divisors of the pixel and tap decode
    float r_ohw, r_ow, r_cinp, r_kw;
    int grid;            // set by the launcher: the launch's workgroups (= partials of amax)
};

// Fills the launch-derived fields of p for BM x BN tiles.  The reciprocals are
// correctly rounded (host division), which udiv_small's one-step correction
// relies on.
inline void i8mm_prepare(I8M& p, int BM, int BN) {
    p.gm = (p.M + BM - 1) / BM;
    p.gn = (p.N + BN - 1) / BN;
    p.r_ohw = 1.0f / (float)(p.OH * p.OW > 0 ? p.OH * p.OW : 1);
    p.r_ow = 1.0f / (float)(p.OW > 0 ? p.OW : 1);
    p.r_cinp = 1.0f / (float)(p.Cinp > 0 ? p.Cinp : 1);
    p.r_kw = 1.0f / (float)(p.KW > 0 ? p.KW : 1);
}

// Output modes of k_i8mm: fp32 (the reference's float output), the maximum
// |value| only (first pass of a requantized output), s8 requantized (second pass).
enum { OUT_F32 = 0, OUT_AMAX = 1, OUT_Q8 = 2 };

// Workgroups of k_i8mm when it reports the output's absmax: its consumer's
// quantizer reduces this many per-workgroup partials (unused ones zero).
constexpr int kAmaxParts = kI8AmaxParts;

enum { AM_GEN = 0, AM_C128 = 1, AM_C64 = 2 };

__device__ __forceinline__ int i8swz(int r) { return (r ^ (r >> 3)) & 7; }

// floor(a / b) for 0 <= a < 2^24, 1 <= b < 2^24 via a float reciprocal, corrected
// by one step either way; q*b <= a + b < 2^25, so a 24-bit multiply forms it.
__device__ __forceinline__ int udiv_small(int a, int b, float rb) {
    const int q = (int)((float)a * rb);
    const int qb = (int)__umul24((unsigned)q, (unsigned)b);
    return q - (qb > a) + (qb + b <= a);
}

// Calls f(std::integral_constant<int, act>) for the wave-uniform activation
// code (0, 1 or 2), so each epilogue loop is compiled for one fixed form.
template <class F>
__device__ __forceinline__ void with_act(int act, F&& f) {
    if (act == 1) f(std::integral_constant<int, 1>{});
    else if (act == 2) f(std::integral_constant<int, 2>{});
    else f(std::integral_constant<int, 0>{});
}

constexpr int vmcnt_enc(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0F70; }

// LDS of k_i8mm: NST operand stages, then NST + 1 slots of the per-channel
// epilogue parameters of a tile (three arrays of BN words each).
constexpr size_t i8mm_lds(int BM, int BN, int NST) {
    return (size_t)NST * (BM + BN) * 128 + (size_t)(NST + 1) * 3 * BN * 4;
}

template <int BM, int BN, int NST, int AM, int EPI, int OUT>
__global__ __launch_bounds__(256) void k_i8mm(I8M p) {
    static_assert(OUT == OUT_F32 || (BM == 64 && BN == 64), "k_i8mm: s8 and max outputs use 64x64 tiles");
    constexpr int FM = BM / 64, FN = BN / 64;
    // 64 x 64 tiles stage their epilogue through the LDS stage of the tile's last
    // chunk (16 KB = 64 x 64 floats), then store whole rows with 16-byte stores
    constexpr bool STAGED = BM == 64 && BN == 64 && OUT != OUT_AMAX;
    constexpr int SA = BM * 128, STG = (BM + BN) * 128;
    constexpr int AIT = BM / 32, BIT = BN / 32;      // DMA instructions per wave per chunk
    constexpr int ITEMS = AIT + BIT;
    constexpr int AHEAD = NST - 1;
    constexpr unsigned kOOB = 0x80000000u;
    typedef __attribute__((address_space(3))) void lds_void;
    typedef int i16v __attribute__((ext_vector_type(16)));
    extern __shared__ __attribute__((aligned(16))) int8_t sm8[];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nch = (p.K + 127) >> 7;

    // ---- tiles of this workgroup: t0, t0 + tstr, ... (cnt of them)
    const int total = p.gm * p.gn, G = gridDim.x, b = blockIdx.x;
    int t0, tstr, cnt;
    if ((G & 7) == 0) {
        const int x = b & 7, i = b >> 3, gx = G >> 3;
        const int sx = (int)(((long long)x * total) >> 3);
        const int ex = (int)(((long long)(x + 1) * total) >> 3);
        t0 = sx + i;
        tstr = gx;
        cnt = ex > t0 ? (ex - t0 + gx - 1) / gx : 0;
    } else {
        t0 = b;
        tstr = G;
        cnt = b < total ? (total - b + G - 1) / G : 0;
    }
    const int nit = cnt * nch;

    // =============================== compute waves
    const int wm = wave >> 1, wn = wave & 1;
    const __amdgpu_buffer_rsrc_t ares =
        __builtin_amdgcn_make_buffer_rsrc((void*)p.A, (short)0, (int)p.a_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t bres =
        __builtin_amdgcn_make_buffer_rsrc((void*)p.Bt, (short)0, (int)p.b_bytes, 0x00020000);
    // The tile's per-channel epilogue parameters travel by the same LDS DMA as
    // the operands (issued just before the items of the tile's first chunk, so
    // the wait for any chunk of the tile covers them), into slot (tile index
    // mod NST + 1): array 0 alpha (or the weight scales), 1 beta (or the
    // bias), 2 the weight column sums.  A missing array is a zero-length
    // buffer and reads as 0.  The issue cursor runs at most NST chunks, so at
    // most NST tiles, ahead of the tile whose epilogue reads its slot: NST + 1
    // slots keep them apart.  No vector load of the loop then has a register
    // result, which would make the compiler wait for every DMA in flight.
    constexpr int PSLOT = 3 * BN * 4, NPS = NST + 1;
    int8_t* const prm = sm8 + NST * STG;
    const float* pa0 = p.alpha ? p.alpha : p.ws;
    const float* pa1 = (EPI == EPI_GEMM && p.alpha) ? p.beta : p.bias;
    const int* pa2 = EPI == EPI_GEMM ? p.Sw : nullptr;
    // wave w (< 3) loads array w: one descriptor per wave from scalar selects
    const void* pbase = wave == 0 ? (const void*)pa0
                      : wave == 1 ? (pa1 ? (const void*)pa1 : (const void*)pa0)
                                  : (pa2 ? (const void*)pa2 : (const void*)pa0);
    const int psize = wave == 0 ? p.N * 4 : wave == 1 ? (pa1 ? p.N * 4 : 0) : (pa2 ? p.N * 4 : 0);
    const __amdgpu_buffer_rsrc_t prs =
        __builtin_amdgcn_make_buffer_rsrc((void*)pbase, (short)0, psize, 0x00020000);

    // ---- DMA rows of this lane: row 8*(wave + 4t) + lane/8 of the A and B
    // stages, quad slot lane%8 holding data quad aq/bq
    const int sl = lane & 7, rl = lane >> 3;
    int aq[AIT], bk[BIT];
#pragma unroll
    for (int t = 0; t < AIT; ++t) aq[t] = sl ^ i8swz(8 * (wave + 4 * t) + rl);
#pragma unroll
    for (int t = 0; t < BIT; ++t) bk[t] = 16 * (sl ^ i8swz(8 * (wave + 4 * t) + rl));
    // issue-side per-tile state
    int abase[AIT], amask[AIT];          // fast modes: byte offset at tap 0, in-bounds taps
    int apix[AIT], aih[AIT], aiw[AIT];   // AM_GEN
    unsigned bv[BIT];
    // Per-tile pixel decode.  A 1x1 / stride 1 / pad 0 convolution's row m is
    // input pixel m; otherwise m -> (image, oh, ow) by float-reciprocal
    // division while m < 2^24 (exact after udiv_small's correction).
    const bool gemm1 = p.K == p.Cinp && p.KW == 1 && p.stride == 1 && p.pad == 0 && p.OH == p.H &&
                       p.OW == p.W;
    const bool small_m = p.M < (1 << 24);
    const int ohw = p.OH * p.OW;
    const float rohw = p.r_ohw, row_ = p.r_ow;
    // bits [lo, hi) of 8
    auto span8 = [](int lo, int hi) -> unsigned {
        lo = lo > 0 ? lo : 0;
        hi = hi < 8 ? hi : 8;
        return hi > lo ? (1u << hi) - (1u << lo) : 0u;
    };
    int ik = 0;                                       // the issue cursor's tile (index in this workgroup)
    int ic = 0;                                       // and its chunk in that tile
    int itn = 0;                                      // column block of the issue cursor's tile
    auto setup = [&](int k) {
        const int L = t0 + k * tstr;
        const int tm = L / p.gn, tn = L - tm * p.gn;
        itn = tn;
#pragma unroll
        for (int t = 0; t < AIT; ++t) {
            const int m = tm * BM + 8 * (wave + 4 * t) + rl;
            if (AM != AM_GEN && gemm1) {
                // pixel m at its only tap (bit 0); past M no tap is in range
                abase[t] = m < p.M ? m * p.Cinp + (AM == AM_C64 ? 16 * (aq[t] & 3) : 16 * aq[t]) : 0;
                amask[t] = m < p.M ? 1 : 0;
                continue;
            }
            int pix = 0, ih0 = -(1 << 28), iw0 = 0;
            if (m < p.M) {
                if (gemm1) {
                    pix = m;
                    ih0 = iw0 = 0;
                } else {
                    int n, oh, ow;
                    if (small_m) {            // (products below m < 2^24: 24-bit multiplies)
                        n = udiv_small(m, ohw, rohw);
                        const int rem = m - __mul24(n, ohw);
                        oh = udiv_small(rem, p.OW, row_);
                        ow = rem - __mul24(oh, p.OW);
                    } else {
                        n = m / ohw;
                        oh = (m - n * ohw) / p.OW;
                        ow = m - n * ohw - oh * p.OW;
                    }
                    pix = n * p.H * p.W;
                    ih0 = oh * p.stride - p.pad;
                    iw0 = ow * p.stride - p.pad;
                }
            }
            if (AM == AM_GEN) {
                apix[t] = pix;
                aih[t] = ih0;
                aiw[t] = iw0;
            } else {
                const int q16 = AM == AM_C64 ? 16 * (aq[t] & 3) : 16 * aq[t];
                abase[t] = m < p.M ? (pix + ih0 * p.W + iw0) * p.Cinp + q16 : 0;
                // bit kh*8 + kw: tap (kh, kw) inside the image (KW <= 8, kh < 4:
                // the fast modes need KH <= 4).  Rows and columns in range form
                // bit spans; the kh-th byte of the mask is the column span when
                // row kh is in range.
                const unsigned rm = span8(-ih0, p.H - ih0), cm = span8(-iw0, p.W - iw0);
                const unsigned rs4 = (rm & 1u) | ((rm & 2u) << 7) | ((rm & 4u) << 14) | ((rm & 8u) << 21);
                amask[t] = (int)(rs4 * cm);
            }
        }
#pragma unroll
        for (int t = 0; t < BIT; ++t) {
            const int n = tn * BN + 8 * (wave + 4 * t) + rl;
            bv[t] = n < p.N ? (unsigned)(n * p.ldb + bk[t]) : kOOB;
        }
    };
    // issue-side per-chunk state (wave-uniform): fast modes track the tap of
    // the chunk's first quad (kh, kw) and its channel offset ic0; AM_C128 also
    // keeps the chunk's byte offset from the tap-(0, 0) pixel and its mask bit
    int ikh = 0, ikw = 0, iic = 0, aoff = 0, abit = 0;
    int islot = 0;                                    // parameter slot of the issue cursor's tile
    const float rcinp = p.r_cinp, rkw = p.r_kw;
    const int taps = p.K / p.Cinp;
    auto tap_off = [&](int kh, int kw) { return (kh * p.W + kw) * p.Cinp; };
    auto issue_params = [&]() {                       // the issue cursor's tile's epilogue parameters
        if (wave < 3 && lane < BN / 4) {
            const unsigned off = (unsigned)((itn * BN + 4 * lane) * 4);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                prs, (lds_void*)(prm + islot * PSLOT + wave * BN * 4), 16, off, 0, 0, 0);
        }
    };
    // DMA item t of chunk c into stage st.  A chunk past the end (live false)
    // is issued all out of range: it writes zeros to a stage no chunk reads
    // again and keeps the number of loads per iteration fixed, so every wait
    // of the loop is the same.
    auto issue = [&](int t, int c, int8_t* st, bool live) {
        if (t < AIT) {
            unsigned v = kOOB;
            if (AM == AM_GEN) {
                const int k = (c << 7) + 16 * aq[t];
                if (live && k < p.K) {
                    const int tap = udiv_small(k, p.Cinp, rcinp);
                    const int ic = k - tap * p.Cinp;
                    const int kh = udiv_small(tap, p.KW, rkw);
                    const int kw = tap - kh * p.KW;
                    const int ih = aih[t] + kh, iw = aiw[t] + kw;
                    if ((unsigned)ih < (unsigned)p.H && (unsigned)iw < (unsigned)p.W)
                        v = (unsigned)((apix[t] + ih * p.W + iw) * p.Cinp + ic);
                }
            } else if (AM == AM_C128) {
                const bool ok = live && ((amask[t] >> abit) & 1);
                v = ok ? (unsigned)(abase[t] + aoff) : kOOB;
            } else {
                // two taps per chunk: quads 0-3 at (ikh, ikw), quads 4-7 at the next tap
                int kh = ikh, kw = ikw + 1;
                if (kw == p.KW) { kw = 0; ++kh; }
                const bool second = aq[t] >= 4;
                const bool inK = !second || (2 * c + 1 < taps);
                const int th = second ? kh : ikh, tw = second ? kw : ikw;
                const bool ok = live && inK && ((amask[t] >> (th * 8 + tw)) & 1);
                v = ok ? (unsigned)(abase[t] + tap_off(th, tw)) : kOOB;
            }
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ares, (lds_void*)(st + (wave + 4 * t) * 1024), 16, v, 0, 0, 0);
        } else {
            const int tt = t - AIT;
            // (a local, not the captured array element, as the builtin's operand:
            // with the latter clang drops the kernel's host-side stub)
            const unsigned v = live ? bv[tt] + (unsigned)(c << 7) : kOOB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                bres, (lds_void*)(st + SA + (wave + 4 * tt) * 1024), 16, v, 0, 0, 0);
        }
    };
    // the issue cursor's next chunk; at the end of a tile, the next tile (its
    // rows, then its parameters)
    auto advance = [&]() {
        if (AM == AM_C128) {
            iic += 128;
            aoff += 128;
            if (iic == p.Cinp) {
                iic = 0;
                if (++ikw == p.KW) { ikw = 0; ++ikh; }
                aoff = tap_off(ikh, ikw);
                abit = ikh * 8 + ikw;
            }
        } else if (AM == AM_C64) {
            ikw += 2;
            while (ikw >= p.KW) { ikw -= p.KW; ++ikh; }
        }
        if (++ic == nch) {
            ic = 0;
            ikh = ikw = iic = aoff = abit = 0;
            if (++ik < cnt) {
                setup(ik);
                islot = islot == NPS - 1 ? 0 : islot + 1;
                issue_params();
            }
        }
    };

    // ---- LDS read offsets (bytes within a stage) of this lane, per k-step
    const int r32 = lane & 31, hq = lane >> 5;
    int rda[4][FM], rdb[4][FN];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const int r = wm * (BM / 2) + 32 * i + r32;
            rda[s][i] = r * 128 + 16 * ((2 * s + hq) ^ i8swz(r));
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int r = wn * (BN / 2) + 32 * j + r32;
            rdb[s][j] = SA + r * 128 + 16 * ((2 * s + hq) ^ i8swz(r));
        }
    }
    i16v acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;

    // OUT_Q8: the first pass's partial maxima (at most kAmaxParts = 768 floats)
    // come by DMA into the last stage, which the prologue leaves free; they are
    // reduced after the first chunk's wait, which covers them.
    static_assert(kAmaxParts <= 768, "k_i8mm: the partial maxima fill at most 3 DMA rows");
    if (OUT == OUT_Q8 && wave < 3) {
        const __amdgpu_buffer_rsrc_t qrs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)p.qparts, (short)0, p.nqparts * 4, 0x00020000);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            qrs, (lds_void*)(sm8 + (NST - 1) * STG + wave * 1024), 16,
            (unsigned)(wave * 1024 + 16 * lane), 0, 0, 0);
    }

    // ---- prologue: the first AHEAD chunks of the item stream (tile, chunk)
    if (nit > 0) {
        setup(0);
        issue_params();
    }
#pragma unroll
    for (int a = 0; a < AHEAD; ++a) {
        const bool live = a < nit;
#pragma unroll
        for (int t = 0; t < ITEMS; ++t) issue(t, ic, sm8 + a * STG, live);
        if (live) advance();
    }

    const float sa = p.s_in ? p.s_in[0] : (p.scal ? p.scal[1] : 0.0f);
    const bool zero = p.s_in ? sa == 0.0f : (p.scal && p.scal[2] != 0.0f);
    // OUT_Q8: the output's max|v| from the first pass's partials (the prologue's
    // DMA is already in flight; these loads sit behind it in the counter)
    float qinv = 0.0f;
    bool qzero = false;
    // the output's max|v| from the partials (slots past nqparts read 0)
    auto reduce_qparts = [&]() {
        __shared__ float qred[4];
        const float* qp = (const float*)(sm8 + (NST - 1) * STG);
        float m = qp[tid];
        m = qp[tid + 256] > m ? qp[tid + 256] : m;
        m = qp[tid + 512] > m ? qp[tid + 512] : m;
        for (int off = 32; off > 0; off >>= 1) {
            const float o = __shfl_xor(m, off, 64);
            m = o > m ? o : m;
        }
        if (lane == 0) qred[wave] = m;
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        m = qred[0];
        for (int w = 1; w < 4; ++w) m = qred[w] > m ? qred[w] : m;
        qzero = m < 1e-12f;                     // as src/conv_int8.cpp:78 for the consumer
        qinv = 127.0f / m;
        if (blockIdx.x == 0 && tid == 0) p.s_out[0] = qzero ? 0.0f : m / 127.0f;
    };
    if (OUT == OUT_Q8 && nit == 0) {            // (no tile: the partials have landed after this wait)
        __builtin_amdgcn_s_waitcnt(vmcnt_enc(0));
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        reduce_qparts();
    }
    int st = 0, ck = 0, cc = 0, cslot = 0;     // compute cursor
    float amx = 0.0f;                           // max|stored value| of this lane
    for (int g = 0; g < nit; ++g) {
        // Chunk g.  Every iteration issues ITEMS loads (chunk g + AHEAD, real or
        // out of range), so the AHEAD - 1 chunks issued after chunk g account
        // for (AHEAD - 1) * ITEMS loads, plus at most a parameter load or the
        // stores of an epilogue queued after them.  Loads complete in issue
        // order, so leaving that many outstanding proves chunk g (and all
        // parameters issued before it) landed; anything extra queued after
        // chunk g only makes the wait longer.  The stores are inline asm, so
        // the compiler's own waits see loads only.
        __builtin_amdgcn_s_waitcnt(vmcnt_enc((AHEAD - 1) * ITEMS));
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        // (before this iteration's DMA reuses the stage the partials came into)
        if (OUT == OUT_Q8 && g == 0) reduce_qparts();
        const int L = t0 + ck * tstr;
        const int tm = L / p.gn, tn = L - tm * p.gn;
        const int m0 = tm * BM, n0 = tn * BN;
        const int8_t* S = sm8 + st * STG;
        const int sta = st == 0 ? NST - 1 : st - 1;   // (g + AHEAD) % NST
        int8_t* NA = sm8 + sta * STG;
        const bool more = g + AHEAD < nit;
        // All of the chunk's operand reads go out first (one LDS round trip per
        // chunk instead of one per k-step), then the MFMAs with the DMA of
        // chunk g + AHEAD issued between them.
        i4 fa[4][FM], fb[4][FN];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
#pragma unroll
            for (int i = 0; i < FM; ++i) fa[s][i] = *(const i4*)(S + rda[s][i]);
#pragma unroll
            for (int j = 0; j < FN; ++j) fb[s][j] = *(const i4*)(S + rdb[s][j]);
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[s][i], fb[s][j], acc[i][j], 0, 0, 0);
#pragma unroll
            for (int t = s * ITEMS / 4; t < (s + 1) * ITEMS / 4; ++t) issue(t, ic, NA, more);
        }
        if (more) advance();
        st = st == NST - 1 ? 0 : st + 1;
        if (++cc < nch) continue;
        // ---- epilogue of tile ck: lane l, register e of block (i, j) <->
        //      row m0 + wm*BM/2 + 32i + 8(e/4) + 4(l/32) + e%4, column n0 + wn*BN/2 + 32j + l%32
        // the tile's parameters landed with its last chunk (waited for above)
        float pv0[FN], pv1[FN];
        int pv2[FN];
        {
            const int8_t* ps = prm + cslot * PSLOT;
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int col = wn * (BN / 2) + 32 * j + r32;
                pv0[j] = ((const float*)ps)[col];
                pv1[j] = ((const float*)(ps + BN * 4))[col];
                pv2[j] = ((const int*)(ps + 2 * BN * 4))[col];
            }
        }
        const bool full = m0 + BM <= p.M && n0 + BN <= p.N;
        const bool relu1 = p.act == 1, relu2 = p.act == 2;
        float al[FN], be[FN];
        int corr[FN];
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            corr[j] = 0;
            if (EPI == EPI_GEMM) {
                corr[j] = 128 * pv2[j];
                if (p.alpha) {
                    al[j] = pv0[j];
                    be[j] = pv1[j];
                } else {   // src/conv_int8.cpp:100-107: alpha = sa*ws; beta = b - (alpha*128)*Sw
                    al[j] = __fmul_rn(sa, pv0[j]);
                    be[j] = __fsub_rn(pv1[j], __fmul_rn(__fmul_rn(al[j], 128.0f), (float)pv2[j]));
                }
            } else {       // src/winograd_int8.cpp:155: (s_in*0.25)*ws, then fma with the bias
                al[j] = p.alpha ? pv0[j] : __fmul_rn(__fmul_rn(sa, 0.25f), pv0[j]);
                be[j] = pv1[j];
            }
            // An all-zero input gives 0 without the bias (src/conv_int8.cpp:78).
            // Zero factors give exactly +0 below: the product of a finite value
            // and 0 is a signed zero, and adding +0 to it gives +0.
            al[j] = zero ? 0.0f : al[j];
            be[j] = zero ? 0.0f : be[j];
        }
        // The route's formula on one accumulator.  GEMM routes: fl(fl(acc_u *
        // alpha) + beta); Winograd route: fmaf(4*acc_s, alpha_w, bias), with
        // (float)(4a) = 4*(float)a exactly.
        auto epi = [&](int a, int j) -> float {
            if (EPI == EPI_GEMM)
                return __fadd_rn(__fmul_rn((float)(int)((unsigned)a + (unsigned)corr[j]), al[j]), be[j]);
            return fmaf(4.0f * (float)a, al[j], be[j]);
        };
        // Lane l, register e of block (i, j) <-> row m0 + wm*BM/2 + 32i + 8(e/4) +
        // 4(l/32) + e%4, column n0 + wn*BN/2 + 32j + l%32.
        const int mb = m0 + wm * (BM / 2) + 4 * hq, nb = n0 + wn * (BN / 2) + r32;
        if (OUT == OUT_AMAX) {
            // first pass of a requantized output: the tile's max|v|, nothing stored;
            // one loop per activation form and per full or edge tile
            with_act(p.act, [&](auto actc) {
                constexpr int ACT = decltype(actc)::value;
                auto tile_max = [&](auto fullc) {
                    constexpr bool FULL = decltype(fullc)::value;
#pragma unroll
                    for (int j = 0; j < FN; ++j)
#pragma unroll
                        for (int i = 0; i < FM; ++i)
#pragma unroll
                            for (int e = 0; e < 16; ++e) {
                                const int m = mb + 32 * i + 8 * (e >> 2) + (e & 3), n = nb + 32 * j;
                                const float v = act_apply(epi(acc[i][j][e], j), ACT);
                                acc[i][j][e] = 0;
                                const float av = (FULL || (m < p.M && n < p.N)) ? fabsf(v) : 0.0f;
                                amx = av > amx ? av : amx;           // NaN never wins
                            }
                };
                if (full) tile_max(std::true_type{});
                else tile_max(std::false_type{});
            });
        } else if (STAGED) {
            // (1) every wave is done reading the last chunk's stage; (2) each wave
            // writes its 32 x 32 block of pre-activation values there, row-major,
            // quad q of row r at quad q ^ (8 * bit 2 of r), so a store's two row
            // halves fall on different banks; (3) whole rows are read back.
            float* const stg = (float*)(sm8 + (st == 0 ? NST - 1 : st - 1) * STG);
            auto sidx = [](int r, int c) { return r * 64 + ((((c >> 2) ^ (((r >> 2) & 1) << 3))) << 2) + (c & 3); };
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int r = wm * 32 + 8 * (e >> 2) + 4 * hq + (e & 3), c = wn * 32 + r32;
                stg[sidx(r, c)] = epi(acc[0][0][e], 0);
                acc[0][0][e] = 0;
            }
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            if (OUT == OUT_F32) {
                // thread t: quad t%16 of rows t/16 + 16i; one loop per activation
                // form, with or without the workgroup maximum (I8M::amax)
                const int q = tid & 15;
                const bool fast = full && p.vec;
                auto rows = [&](auto actc, auto trackc, auto fastc) {
                    constexpr int ACT = decltype(actc)::value;
                    constexpr bool TRACK = decltype(trackc)::value, FAST = decltype(fastc)::value;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int r = (tid >> 4) + 16 * i;
                        const int m = m0 + r, n = n0 + 4 * q;
                        f4v v = *(const f4v*)&stg[sidx(r, 4 * q)];
                        float* dst = p.Cf + (long long)m * p.ldc + n;
                        if (FAST || (p.vec && m < p.M && n + 4 <= p.N)) {
                            if (p.res) {
                                const f4v rv = *(const f4v*)(p.res + (long long)m * p.ldr + n);
                                v = v + rv;          // fl(v + res) per lane, as a separate Add
                            }
#pragma unroll
                            for (int k = 0; k < 4; ++k) {
                                v[k] = act_apply(v[k], ACT);
                                if (TRACK) {
                                    const float av = fabsf(v[k]);
                                    amx = av > amx ? av : amx;
                                }
                            }
                            // s_nop: a VALU write to the data registers of a store of
                            // more than 8 bytes needs a wait state after it
                            asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1" ::"v"(dst), "v"(v)
                                         : "memory");
                        } else if (!FAST && m < p.M) {
#pragma unroll
                            for (int k = 0; k < 4; ++k) {
                                if (n + k >= p.N) continue;
                                float w = v[k];
                                if (p.res) w = __fadd_rn(w, p.res[(long long)m * p.ldr + n + k]);
                                w = act_apply(w, ACT);
                                if (TRACK) {
                                    const float av = fabsf(w);
                                    amx = av > amx ? av : amx;
                                }
                                asm volatile("global_store_dword %0, %1, off sc1" ::"v"(dst + k), "v"(w)
                                             : "memory");
                            }
                        }
                    }
                };
                // (full tiles with 16-byte rows: no bounds test per quad)
                with_act(p.act, [&](auto actc) {
                    if (fast) {
                        if (p.amax) rows(actc, std::true_type{}, std::true_type{});
                        else rows(actc, std::false_type{}, std::true_type{});
                    } else {
                        if (p.amax) rows(actc, std::true_type{}, std::false_type{});
                        else rows(actc, std::false_type{}, std::false_type{});
                    }
                });
            } else {
                // OUT_Q8: thread t: 16 columns 16*(t%4).. of row t/4, one 16-byte store;
                // columns N..ldq-1 (the channel padding of the s8 layout) are 0
                const int r = tid >> 2, c0 = 16 * (tid & 3);
                const int m = m0 + r, n = n0 + c0;
                if (m < p.M && n < p.ldq) {
                    // Rounding form 0: RNE (rule 0).  Rule 1 (the Winograd route's
                    // input rule): add-then-truncate below N & ~15 (form 1), lroundf's
                    // half-away above (form 2); a thread's 16 columns start at a
                    // multiple of 16, so they share one form.  Then the clamp; padding
                    // columns and an all-zero output give 0.
                    const int form = p.rule == 0 ? 0 : (n < (p.N & ~15) ? 1 : 2);
                    unsigned w4[4] = {0u, 0u, 0u, 0u};
                    auto quant = [&](auto actc, auto formc) {
                        constexpr int ACT = decltype(actc)::value, FORM = decltype(formc)::value;
#pragma unroll
                        for (int k4 = 0; k4 < 4; ++k4) {
                            const f4v v = *(const f4v*)&stg[sidx(r, c0 + 4 * k4)];
#pragma unroll
                            for (int k = 0; k < 4; ++k) {
                                const int c = n + 4 * k4 + k;
                                const float t = __fmul_rn(act_apply(v[k], ACT), qinv);
                                // (|t| <= 127 up to rounding: the reference's conversions
                                // differ from a float clamp only at NaN, which the RNE and
                                // add-then-truncate forms send to -128, lroundf to 0)
                                float rq = FORM == 0 ? rintf(t)
                                         : FORM == 1 ? truncf(__fadd_rn(t, copysignf(0.5f, t)))
                                                     : (t != t ? 0.0f : roundf(t));
                                rq = fminf(fmaxf(rq, -128.0f), 127.0f);
                                const int qv = c < p.N ? (int)rq : 0;
                                w4[k4] |= ((unsigned)qv & 0xffu) << (8 * k);
                            }
                        }
                    };
                    if (!qzero) {
                        with_act(p.act, [&](auto actc) {
                            if (form == 0) quant(actc, std::integral_constant<int, 0>{});
                            else if (form == 1) quant(actc, std::integral_constant<int, 1>{});
                            else quant(actc, std::integral_constant<int, 2>{});
                        });
                    }
                    const i4 pk = {(int)w4[0], (int)w4[1], (int)w4[2], (int)w4[3]};
                    int8_t* dq = p.Cq + (long long)m * p.ldq + n;
                    asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1" ::"v"(dq), "v"(pk)
                                 : "memory");
                }
            }
        } else {
            // larger tiles: each lane stores its accumulators' elements directly
            float* const cl = p.Cf + (long long)mb * p.ldc + nb;      // this lane's first row
            auto tile_out = [&](auto fullc, auto resc) {
                constexpr bool FULL = decltype(fullc)::value, RES = decltype(resc)::value;
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    const int n = nb + 32 * j;
#pragma unroll
                    for (int i = 0; i < FM; ++i) {
                        float rv[16];
                        if (RES) {     // residual of the fused Add, all 16 loads in flight at once
#pragma unroll
                            for (int e = 0; e < 16; ++e) {
                                const int m = mb + 32 * i + 8 * (e >> 2) + (e & 3);
                                rv[e] = (FULL || (m < p.M && n < p.N)) ? p.res[(long long)m * p.ldr + n] : 0.0f;
                            }
                        }
#pragma unroll
                        for (int e = 0; e < 16; ++e) {
                            const int m = mb + 32 * i + 8 * (e >> 2) + (e & 3);
                            float v = epi(acc[i][j][e], j);
                            acc[i][j][e] = 0;
                            if (RES) v = __fadd_rn(v, rv[e]);
                            v = act_select(v, relu1, relu2);
                            if (FULL || (m < p.M && n < p.N)) {
                                float* dst = cl + (32 * i + 8 * (e >> 2) + (e & 3)) * (long long)p.ldc + 32 * j;
                                asm volatile("global_store_dword %0, %1, off sc1" ::"v"(dst), "v"(v) : "memory");
                                const float av = fabsf(v);
                                amx = av > amx ? av : amx;             // NaN never wins
                            }
                        }
                    }
                }
            };
            using T_ = std::true_type;
            using F_ = std::false_type;
            if (full) {
                if (p.res) tile_out(T_{}, T_{});
                else tile_out(T_{}, F_{});
            } else {
                if (p.res) tile_out(F_{}, T_{});
                else tile_out(F_{}, F_{});
            }
        }
        cc = 0;
        ++ck;
        cslot = cslot == NPS - 1 ? 0 : cslot + 1;
    }
    // this workgroup's max|v| of the output tensor, a partial of the next
    // layer's absmax (the reference's max|x| of its input, src/conv_int8.cpp:77)
    if (p.amax) {
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
            p.amax[blockIdx.x] = mm;
        }
    }
}


}  // namespace i8k

using i8k::I8M;
using i8k::kAmaxParts;
using i8k::AM_GEN;
using i8k::AM_C128;
using i8k::AM_C64;
using i8k::OUT_F32;
using i8k::OUT_AMAX;
using i8k::OUT_Q8;

// k_i8mm tile: BM x BN output tile, NST LDS stages, per_cu persistent
// workgroups per CU (0: one tile per workgroup).
struct I8Tile { int bm, bn, nst, per_cu; };

// Launches k_i8mm for p (p.epi: EPI_GEMM or EPI_WINO; am: AM_*).
// launch_i8mm_f32 (k_i8mm_f32.hip): fp32 output p.Cf.
// launch_i8mm_q8 (k_i8mm_q8.hip): out = OUT_AMAX writes per-workgroup maxima to
// p.amax; out = OUT_Q8 reads them (p.qparts, p.nqparts) and writes p.Cq, p.s_out.
// Both passes of one output must use the same tile and grid.
bool launch_i8mm_f32(I8M& p, const I8Tile& t, int am, hipStream_t s);
bool launch_i8mm_q8(I8M& p, const I8Tile& t, int am, int out, hipStream_t s);
// The grid launch_i8mm_* uses for p and t (workgroups).
int i8mm_grid(const I8M& p, const I8Tile& t);

// Arguments of k_i8q1 (k_i8q1.hip): a float-input 1x1 / stride-1 / pad-0 int8
// convolution (the GEMM route, RNE quantization) with the activation
// quantization done while the A operand is staged, instead of a quantize pass
// into an s8 tensor before k_i8mm.
struct I8Q1 {
    const float* x;       // fp32 NHWC activations [M][Cin]
    const int8_t* Bt;     // prepared weights [N][ldb] (s8, zero past Cinp), N * ldb < 2^31
    const int* Sw;        // their column sums
    const float* ws;      // per-channel weight scales
    const float* bias;    // nullable
    const float* part;    // absmax partials of x (nparts of them, at most kAmaxParts)
    int nparts;
    float* scal;          // nullable: {inv_s, sa, zero flag, max}, written by workgroup 0
    const float* res;     // nullable residual [M][ldr], added before the activation
    float* Cf;            // output [M][ldc]
    float* amax;          // nullable: per-workgroup max|stored value| at [workgroup]
    int M, N, Cin, Cinp, ldb, ldc, ldr, act;
    int grid;             // set by the launcher (workgroups = partials written to amax)
};
// Cinp (Cin rounded up to 16) up to this many channels: the block of 64
// quantized rows stays in LDS.
constexpr int kI8Q1MaxCinp = 512;
bool launch_i8q1(I8Q1& a, hipStream_t s);
// Whether a 1x1 conv with Cout output channels takes k_i8q1 (Cout <= 64
// unless ACFUN_I8Q1 forces it on or off; read once).
bool i8q1_route(int Cout);

}  // namespace acfun
