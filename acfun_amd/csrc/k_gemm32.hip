// k_gemm32.hip -- fp32 GEMM C[M,N] = A[M,K] * B[K,N] (+bias[n], ReLU) on
// v_mfma_f32_32x32x2f32 with LDS-DMA staging: the engine behind acfun_gemm,
// acfun_gemm_epi, acfun_fc and the 1x1 conv route (reference
// src/gemm_avx512.cpp:245-337, src/layers.cpp:19-36,66-101) whenever the
// operands are 16-byte aligned with K, N, lda, ldb multiples of 4.
//
// Workgroup = 64 x 64 tile of C, 4 waves in a 2 x 2 grid, each wave one
// 32 x 32 accumulator (16 registers per lane): a single dependent MFMA chain,
// which gfx950 issues back to back.  K is consumed in chunks of 64:
//   A stage [64 rows][16 quads], quad q of row r at slot q ^ (r & 15);
//   B stage [64 k][16 quads],    quad q of row k at slot q ^ ((k & 32) >> 2).
// Both are filled by buffer_load_dwordx4 ... lds (no data VGPRs; rows and
// columns past the matrix read zeros through the buffer range check or an
// out-of-range offset), three stages deep with chunk c+2 issued while chunk
// c is multiplied when the grid is one wave of workgroups, else two stages
// (two workgroups per CU) with chunk c+1 in flight.  MFMA k assignment: in k-step s of a chunk, lane half h = l/32
// carries k = 32h + s for both operands, so a lane reads its A row as eight
// ds_read_b128 and B as one ds_read_b32 per step at an immediate offset; the
// swizzles keep both conflict-free.  The epilogue adds bias, optionally a
// residual tensor (a model's Add fused into the conv before it: the same two
// roundings as a separate Add), applies ReLU (max_ps order) and stores 128
// contiguous bytes per half-wave row.
#include "rt.hpp"

namespace acfun {
namespace {

typedef float f16v __attribute__((ext_vector_type(16)));
typedef float f4g __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void32;

constexpr int G32_BM = 64, G32_BN = 64, G32_KC = 64;
constexpr int G32_STAGE = 2 * 1024 * 4;           // floats per stage: A + B, 1024 quads each

// Implicit-GEMM convolution geometry (CONV mode): A is the NHWC input
// [n][H][W][Cin], row m of the GEMM the output pixel (n, oh, ow), k = tap*Cin + ic.
struct G32Conv {
    int H, W, Cin, KW, stride, pad, OH, OW;
    unsigned bytes;    // N*H*W*Cin*4, below 2^31
};

template <int NST, bool CONV>
__global__ __launch_bounds__(256) void k_gemm32(const float* __restrict__ A,
                                                const float* __restrict__ B,
                                                float* __restrict__ C,
                                                const float* __restrict__ bias,
                                                const float* __restrict__ res, int M, int N,
                                                int K, int lda, int ldb, int ldc, int ldr,
                                                int act, G32Conv cv) {
    constexpr unsigned kOOB = 0x80000000u;
    extern __shared__ __attribute__((aligned(16))) float sm[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * G32_BM, n0 = blockIdx.x * G32_BN;
    const int nch = (K + G32_KC - 1) / G32_KC;

    // ---- DMA descriptors.  Wave w issues A blocks and B blocks w + 4t
    // (t = 0..3); lane l of block b covers slot 64b + l = row*16 + quad slot.
    const __amdgpu_buffer_rsrc_t ares = CONV
        ? __builtin_amdgcn_make_buffer_rsrc((void*)A, (short)0, (int)cv.bytes, 0x00020000)
        : __builtin_amdgcn_make_buffer_rsrc(
              (void*)(A + (long long)m0 * lda), (short)0,
              (int)((long long)(M - m0) * lda * 4 < 0x7fffffff ? (long long)(M - m0) * lda * 4 : 0x7fffffff),
              0x00020000);
    const __amdgpu_buffer_rsrc_t bres = __builtin_amdgcn_make_buffer_rsrc(
        (void*)B, (short)0, (int)((long long)K * ldb * 4), 0x00020000);
    const int arow = 4 * wave + (lane >> 4);               // + 16t
    const int aq = (lane & 15) ^ (arow & 15);              // same for every t
    const unsigned av = (unsigned)(arow * lda + 4 * aq) * 4u;
    const unsigned astep = 16u * lda * 4u;                 // 16 rows per t
    // CONV: per row t, the byte offset of channel quad aq of tap (0, 0) and the
    // in-image taps as bits kh*8 + kw (KH, KW <= 8)
    int cbase[4];
    unsigned long long cmask[4];
    if (CONV) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int m = m0 + arow + 16 * t;
            cbase[t] = 0;
            cmask[t] = 0;
            if (m < M) {
                const int hw = cv.OH * cv.OW;
                const int n = m / hw, rem = m - n * hw;
                const int oh = rem / cv.OW, ow = rem - oh * cv.OW;
                const int ih0 = oh * cv.stride - cv.pad, iw0 = ow * cv.stride - cv.pad;
                cbase[t] = ((n * cv.H + ih0) * cv.W + iw0) * cv.Cin * 4 + 16 * aq;
                unsigned rm = 0, cm = 0;
                for (int d = 0; d < 8; ++d) {
                    rm |= ((unsigned)(ih0 + d) < (unsigned)cv.H) ? (1u << d) : 0u;
                    cm |= ((unsigned)(iw0 + d) < (unsigned)cv.W) ? (1u << d) : 0u;
                }
                unsigned long long mk = 0;
                for (int d = 0; d < 8; ++d)
                    if ((rm >> d) & 1u) mk |= (unsigned long long)cm << (8 * d);
                cmask[t] = mk;
            }
        }
    }
    const int brow = 4 * wave + (lane >> 4);               // k row within the chunk, + 16t
    int bq[2];
    bool bok[2];
    unsigned bv[2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {                        // t < 2: k < 32; t >= 2: k >= 32
        bq[hh] = (lane & 15) ^ (hh << 3);
        bok[hh] = n0 + 4 * bq[hh] < N;
        bv[hh] = (unsigned)(brow * ldb + n0 + 4 * bq[hh]) * 4u;
    }
    const unsigned bstep = 16u * ldb * 4u;
    const bool kragged = (K & (G32_KC - 1)) != 0;

    // Every variable part of an address is in the per-lane offset (which the
    // buffer range check covers); the scalar offset stays 0.
    auto issue = [&](int t, int c, float* st) {            // item t of chunk c into stage st
        const int k0 = c * G32_KC;
        if (t < 4) {
            unsigned v;
            if (CONV) {
                // a 64-channel chunk lies in one tap (Cin % 64 == 0): wave-uniform
                const int tap = k0 / cv.Cin, ic0 = k0 - tap * cv.Cin;
                const int kh = tap / cv.KW, kw = tap - kh * cv.KW;
                const bool ok = (cmask[t] >> (kh * 8 + kw)) & 1ull;
                v = ok ? (unsigned)(cbase[t] + ((kh * cv.W + kw) * cv.Cin + ic0) * 4) : kOOB;
            } else {
                v = av + (unsigned)k0 * 4u + (unsigned)t * astep;
                if (kragged && k0 + 4 * aq >= K) v = kOOB;
            }
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ares, (lds_void32*)(st + (wave + 4 * t) * 256),
                                                     16, v, 0, 0, 0);
        } else {
            const int tt = t - 4, hh = tt >> 1;
            unsigned v = bok[hh] ? bv[hh] + (unsigned)k0 * ldb * 4u + (unsigned)tt * bstep : kOOB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                bres, (lds_void32*)(st + 4096 + (wave + 4 * tt) * 256), 16, v, 0, 0, 0);
        }
    };

    // ---- per-lane read offsets within a stage (floats)
    const int r = lane & 31, h = lane >> 5;
    const int rowA = 32 * wm + r;
    int aoff[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) aoff[j] = (rowA * 16 + ((8 * h + j) ^ (rowA & 15))) * 4;
    const int col = 32 * wn + r;
    const int boff = 4096 + ((32 * h) * 16 + ((col >> 2) ^ (h << 3))) * 4 + (col & 3);

    f16v acc;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.f;

    // Bias and residual of this lane's 16 outputs, loaded first (loads complete
    // in issue order) so their latency hides behind chunk 0's.
    const int n = n0 + col;
    float bn = 0.f, rv[16];
    if (n < N && bias) bn = bias[n];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int m = m0 + 32 * wm + 8 * (e >> 2) + 4 * h + (e & 3);
        rv[e] = (res && n < N && m < M) ? res[(long long)m * ldr + n] : 0.f;
    }

    // NST = 3: chunk c+2 is issued while chunk c is multiplied; NST = 2 (two
    // workgroups per CU): chunk c+1.  NST stages hold min(NST, nch) chunks.
    constexpr int AHEAD = NST - 1;
#pragma unroll
    for (int t = 0; t < 8; ++t) issue(t, 0, sm);
    if (AHEAD == 2 && nch > 1) {
#pragma unroll
        for (int t = 0; t < 8; ++t) issue(t, 1, sm + G32_STAGE);
    }

    int st = 0;
    for (int c = 0; c < nch; ++c) {
        // outstanding in issue order: ..., chunk c, [chunk c+1] (8 items each)
        if (AHEAD == 2 && c + 1 < nch) __builtin_amdgcn_s_waitcnt(0x0F78);   // vmcnt(8)
        else __builtin_amdgcn_s_waitcnt(0x0F70);                             // vmcnt(0)
        // LDS-only workgroup barrier: this wave's LDS reads are complete;
        // the loads of later chunks stay in flight.
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        const float* S = sm + st * G32_STAGE;
        const int sta = AHEAD == 2 ? (st == 0 ? 2 : st - 1) : (st ^ 1);     // (c + AHEAD) % NST
        float* NA = sm + sta * G32_STAGE;
        const bool more = c + AHEAD < nch;
        f4g a[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) a[j] = *(const f4g*)&S[aoff[j]];
#pragma unroll
        for (int s = 0; s < 32; ++s) {
            const float b = S[boff + s * 64];
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s >> 2][s & 3], b, acc, 0, 0, 0);
            if ((s & 3) == 3 && more) issue(s >> 2, c + AHEAD, NA);
        }
        st = AHEAD == 2 ? (st == 2 ? 0 : st + 1) : (st ^ 1);
    }

    // ---- epilogue: lane l, register e <-> row 8*(e/4) + 4*(l/32) + e%4, column l%32
    if (n < N) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int m = m0 + 32 * wm + 8 * (e >> 2) + 4 * h + (e & 3);
            if (m < M) {
                float v = acc[e];
                if (bias) v = v + bn;
                if (res) v = v + rv[e];                   // fused residual Add
                v = act_apply(v, act);
                C[(long long)m * ldc + n] = v;
            }
        }
    }
}

}  // namespace

namespace {
template <bool CONV>
bool launch_gemm32(int M, int N, int K, const float* A, int lda, const float* B, int ldb, float* C,
                   int ldc, const float* bias, int act, hipStream_t s, const float* res, int ldr,
                   const G32Conv& cv) {
    if (M <= 0 || N <= 0) return true;
    static bool attr = false;
    if (!attr) {
        attr = true;
        (void)hipFuncSetAttribute((const void*)k_gemm32<3, CONV>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 3 * G32_STAGE * 4);
        (void)hipFuncSetAttribute((const void*)k_gemm32<2, CONV>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 2 * G32_STAGE * 4);
    }
    dim3 grid((unsigned)((N + G32_BN - 1) / G32_BN), (unsigned)((M + G32_BM - 1) / G32_BM));
    const int nch = (K + G32_KC - 1) / G32_KC;
    const long long tiles = (long long)grid.x * grid.y;
    // Three stages (one workgroup per CU) only pay when the grid is a single
    // wave of workgroups; otherwise two stages let two workgroups share a CU.
    // LDS holds only the stages that can be in use.
    const bool deep = nch > 2 && tiles < 2ll * num_cus();
    const int stages = deep ? 3 : (nch < 2 ? 1 : 2);
    const size_t lds = (size_t)stages * G32_STAGE * 4;
    if (deep)
        ACFUN_LAUNCH("k_gemm_f32", (k_gemm32<3, CONV>), grid, dim3(256), lds, s, A, B, C, bias, res, M,
                     N, K, lda, ldb, ldc, ldr, act, cv);
    else
        ACFUN_LAUNCH("k_gemm_f32", (k_gemm32<2, CONV>), grid, dim3(256), lds, s, A, B, C, bias, res, M,
                     N, K, lda, ldb, ldc, ldr, act, cv);
    return check_launch("k_gemm32");
}
}  // namespace

bool gemm32_f32(int M, int N, int K, const float* A, int lda, const float* B, int ldb, float* C,
                int ldc, const float* bias, int act, hipStream_t s, const float* res, int ldr) {
    return launch_gemm32<false>(M, N, K, A, lda, B, ldb, C, ldc, bias, act, s, res, ldr, G32Conv{});
}

bool conv32_ok(const ConvShape& g, int Cout, const float* in, const float* w) {
    auto al = [](const void* q) { return ((uintptr_t)q & 15u) == 0; };
    const long long M = (long long)g.N * g.OH * g.OW;
    const long long K = (long long)g.KH * g.KW * g.Cin;
    return g.Cin % 64 == 0 && g.KH <= 8 && g.KW <= 8 && Cout % 4 == 0 && al(in) && al(w) &&
           (long long)g.N * g.H * g.W * g.Cin * 4 < 0x7fffffffll && K * Cout * 4 < 0x7fffffffll &&
           M < (1ll << 31) && (Cout + 63) / 64 < 65536 * 32 && (M + 63) / 64 < 65536;
}

bool conv32_f32(const ConvShape& g, const float* in, const float* w, const float* bias, int Cout,
                float* out, int act, hipStream_t s, const float* res, int ldr) {
    G32Conv cv{g.H, g.W, g.Cin, g.KW, g.stride, g.pad, g.OH, g.OW,
               (unsigned)((long long)g.N * g.H * g.W * g.Cin * 4)};
    const int M = g.N * g.OH * g.OW, K = g.KH * g.KW * g.Cin;
    return launch_gemm32<true>(M, Cout, K, in, g.Cin, w, Cout, out, Cout, bias, act, s, res, ldr, cv);
}

bool gemm32_ok(int M, int N, int K, const float* A, int lda, const float* B, int ldb) {
    auto al = [](const void* q) { return ((uintptr_t)q & 15u) == 0; };
    return K > 0 && K % 4 == 0 && N % 4 == 0 && lda % 4 == 0 && ldb % 4 == 0 && al(A) && al(B) &&
           (long long)K * ldb * 4 < 0x7fffffffll && (long long)(M + 64) * lda * 4 < (1ll << 40) &&
           (long long)lda * 16 * 4 < 0x7fffffffll && (N + 63) / 64 < 65536 * 32 &&
           (M + 63) / 64 < 65536;
}

}  // namespace acfun
