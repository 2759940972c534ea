// k_bf16.hip -- acfun_gemm_bf16 on bf16 MFMA.
//
// Replaces the reference's AVX-512 BF16 path (src/gemm_bf16_avx512.cpp): A and
// B are rounded to bf16 (round to nearest even on bit 16, :37-44) and the
// products accumulate in fp32.  Products of two bf16 values are exact in fp32,
// so the result differs from the reference only by the fp32 accumulation
// order.
//
// One packing launch writes the rounded operands k-contiguous -- A as
// [M][Kp], B transposed as [N][Kp], Kp = K rounded up to 128, zeros beyond K
// -- and k_bf16mm multiplies them on v_mfma_f32_32x32x16_bf16: 64 x 64 tiles,
// 2 x 2 waves, K in chunks of 256 bytes (128 bf16) DMA'd into LDS by
// buffer_load_dwordx4 ... lds, quad q of row r at slot r*16 + (q ^ (r % 16)),
// four stages (three chunks ahead).  In k-step s lane half h reads quad 2s+h
// of its A row and its B row: eight bf16 each, the MFMA's 16 k per step.  At
// 1024^3 the grid is one tile per CU and the K loop is bound by the DMA round
// trip, so the chunks are large and many are in flight.
#include "rt.hpp"

namespace acfun {
namespace {

typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef int i4v __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

// fp32 -> bf16 bits as the reference packs its operands
// (src/gemm_bf16_avx512.cpp:37-44): add 0x7fff plus bit 16, keep the upper
// half.  The 32-bit add wraps, so some NaNs become infinities or zero there
// too.
__device__ __forceinline__ unsigned bf16_bits(float f) {
    const unsigned u = __float_as_uint(f);
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// One lane: 8 consecutive k of one row of A -> one 16-byte store (two 16-byte
// loads when the row segment is whole and aligned).
__device__ __forceinline__ void pack_a_bf16(long long t, const float* __restrict__ A, int M, int K,
                                            int lda, unsigned short* __restrict__ Ab, int Kp, bool va) {
    const int kq = Kp >> 3;
    if (t >= (long long)M * kq) return;
    const int m = (int)(t / kq), k0 = (int)(t - (long long)m * kq) * 8;
    const float* src = A + (long long)m * lda + k0;
    float v[8];
    if (va && k0 + 8 <= K) {
        const float4 x0 = *(const float4*)src, x1 = *(const float4*)(src + 4);
        v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w;
        v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = k0 + e < K ? src[e] : 0.f;
    }
    unsigned w[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const unsigned lo = k0 + 2 * p < K ? bf16_bits(v[2 * p]) : 0u;
        const unsigned hi = k0 + 2 * p + 1 < K ? bf16_bits(v[2 * p + 1]) : 0u;
        w[p] = lo | (hi << 16);
    }
    *(i4v*)(Ab + (long long)m * Kp + k0) = i4v{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
}

// One block: a 64 k x 64 n tile of B -> Bt[n][k] through LDS.  Thread t loads
// quad t % 16 of rows t / 16 + 16 i (256 contiguous bytes per row), rounds
// each value (the same bf16_bits) and writes it transposed into LDS; then 8
// threads store the 128 bytes of one Bt row segment (16 bytes each).  k past K
// is zero (Kp padding); n past N is not stored.
__device__ __forceinline__ void pack_bt_bf16(int tile, const float* __restrict__ B, int K, int N, int ldb,
                                             unsigned short* __restrict__ Bt, int Kp, bool vb) {
    __shared__ unsigned short tr[64][64 + 8];          // [n][k], rows padded by 16 bytes
    const int t = (int)threadIdx.x;
    const int ntn = (N + 63) >> 6;
    const int kb = tile / ntn, nb = tile - kb * ntn;
    const int k0 = kb * 64, n0 = nb * 64;
    const int q = t & 15, n = n0 + 4 * q;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int kr = (t >> 4) + 16 * i, k = k0 + kr;
        float v[4] = {0.f, 0.f, 0.f, 0.f};
        if (k < K) {
            const float* src = B + (long long)k * ldb + n;
            if (vb && n + 4 <= N) {
                const float4 x = *(const float4*)src;
                v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = n + e < N ? src[e] : 0.f;
            }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) tr[4 * q + e][kr] = k < K ? (unsigned short)bf16_bits(v[e]) : (unsigned short)0;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int nr = (t >> 3) + 32 * i, kc = 8 * (t & 7);
        if (n0 + nr < N && k0 + kc < Kp)
            *(i4v*)(Bt + (long long)(n0 + nr) * Kp + k0 + kc) = *(const i4v*)&tr[nr][kc];
    }
}

// Both operands in one launch: blocks [0, nba) pack A (8 k per lane), the
// rest B (a 64 x 64 tile per block).
__global__ __launch_bounds__(256) void k_pack_bf16(const float* __restrict__ A, const float* __restrict__ B,
                                                   int M, int N, int K, int lda, int ldb, int Kp, int nba,
                                                   unsigned short* __restrict__ Ab,
                                                   unsigned short* __restrict__ Bt, int va, int vb) {
    const int b = (int)blockIdx.x;
    if (b < nba) pack_a_bf16((long long)b * 256 + threadIdx.x, A, M, K, lda, Ab, Kp, va != 0);
    else pack_bt_bf16(b - nba, B, K, N, ldb, Bt, Kp, vb != 0);
}

constexpr int BF_BM = 64, BF_BN = 64, BF_NST = 4, BF_KB = 256;   // K chunk: 256 bytes, 128 bf16
constexpr int BF_SA = BF_BM * BF_KB, BF_STG = (BF_BM + BF_BN) * BF_KB;
static_assert(BF_NST == 4, "the waits below leave at most two chunks in flight");
// s_waitcnt vmcnt(n), n < 64
constexpr int bf_vmcnt(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0F70; }

__global__ __launch_bounds__(256) void k_bf16mm(const unsigned short* __restrict__ Ab,
                                                const unsigned short* __restrict__ Bt,
                                                float* __restrict__ C, int M, int N, int Kp,
                                                int ldc, unsigned a_bytes, unsigned b_bytes) {
    constexpr int AIT = BF_BM / 16, BIT = BF_BN / 16, ITEMS = AIT + BIT;   // 1 KB (4 rows) per item
    constexpr int AHEAD = BF_NST - 1;
    constexpr unsigned kOOB = 0x80000000u;
    extern __shared__ __attribute__((aligned(16))) char smb[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    // XCD-contiguous tile order (workgroup id mod 8 = XCD)
    const int gn = (N + BF_BN - 1) / BF_BN, total = gn * ((M + BF_BM - 1) / BF_BM);
    int L = blockIdx.x;
    if ((total & 7) == 0) L = (L & 7) * (total >> 3) + (L >> 3);
    const int m0 = (L / gn) * BF_BM, n0 = (L % gn) * BF_BN;
    const int nch = Kp >> 7;
    const __amdgpu_buffer_rsrc_t ares =
        __builtin_amdgcn_make_buffer_rsrc((void*)Ab, (short)0, (int)a_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t bres =
        __builtin_amdgcn_make_buffer_rsrc((void*)Bt, (short)0, (int)b_bytes, 0x00020000);
    // DMA rows of this lane: row 4*(wave + 4t) + lane/16, slot lane%16 holding
    // quad (lane%16) ^ (row%16)
    const int sl = lane & 15, rl = lane >> 4;
    unsigned av[AIT], bv[BIT];
#pragma unroll
    for (int t = 0; t < AIT; ++t) {
        const int row = 4 * (wave + 4 * t) + rl, q = sl ^ (row & 15);
        av[t] = m0 + row < M ? (unsigned)((m0 + row) * Kp * 2 + 16 * q) : kOOB;
    }
#pragma unroll
    for (int t = 0; t < BIT; ++t) {
        const int row = 4 * (wave + 4 * t) + rl, q = sl ^ (row & 15);
        bv[t] = n0 + row < N ? (unsigned)((n0 + row) * Kp * 2 + 16 * q) : kOOB;
    }
    auto issue = [&](int t, int c, char* st) {
        if (t < AIT) {
            const unsigned v = av[t] + (unsigned)(c << 8);   // kOOB + k stays out of range
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ares, (lds_void*)(st + (wave + 4 * t) * 1024), 16,
                                                     v, 0, 0, 0);
        } else {
            const int tt = t - AIT;
            const unsigned v = bv[tt] + (unsigned)(c << 8);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(bres, (lds_void*)(st + BF_SA + (wave + 4 * tt) * 1024),
                                                     16, v, 0, 0, 0);
        }
    };
    // LDS read offsets (bytes within a stage) per k-step
    const int r32 = lane & 31, hq = lane >> 5;
    const int ra = wm * 32 + r32, rb = wn * 32 + r32;
    int rda[8], rdb[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        rda[s] = ra * BF_KB + 16 * ((2 * s + hq) ^ (ra & 15));
        rdb[s] = BF_SA + rb * BF_KB + 16 * ((2 * s + hq) ^ (rb & 15));
    }
    f16v acc;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.f;

#pragma unroll
    for (int a = 0; a < AHEAD; ++a)
        if (a < nch) {
#pragma unroll
            for (int t = 0; t < ITEMS; ++t) issue(t, a, smb + a * BF_STG);
        }
    int st = 0;
    for (int c = 0; c < nch; ++c) {
        // chunk c landed: the chunks after it (at most AHEAD - 1) stay in flight
        const int later = nch - 1 - c < AHEAD - 1 ? nch - 1 - c : AHEAD - 1;
        if (later >= 2) __builtin_amdgcn_s_waitcnt(bf_vmcnt(2 * ITEMS));
        else if (later == 1) __builtin_amdgcn_s_waitcnt(bf_vmcnt(ITEMS));
        else __builtin_amdgcn_s_waitcnt(bf_vmcnt(0));
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        const char* S = smb + st * BF_STG;
        char* NA = smb + (st == 0 ? BF_NST - 1 : st - 1) * BF_STG;   // (c + AHEAD) % NST: chunk c - 1's
        const bool more = c + AHEAD < nch;
        i4v fa[8], fb[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            fa[s] = *(const i4v*)(S + rda[s]);
            fb[s] = *(const i4v*)(S + rdb[s]);
        }
        if (more) {                                      // its stage was read before this chunk
#pragma unroll
            for (int t = 0; t < ITEMS; ++t) issue(t, c + AHEAD, NA);
        }
#pragma unroll
        for (int s = 0; s < 8; ++s)
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf8, fa[s]),
                                                          __builtin_bit_cast(bf8, fb[s]), acc, 0, 0, 0);
        st = st == BF_NST - 1 ? 0 : st + 1;
    }
    // epilogue: lane l, register e <-> row m0 + 32wm + 8(e/4) + 4(l/32) + e%4, column n0 + 32wn + l%32
    const int n = n0 + wn * 32 + r32;
    if (n >= N) return;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int m = m0 + wm * 32 + 8 * (e >> 2) + 4 * hq + (e & 3);
        if (m < M) C[(long long)m * ldc + n] = acc[e];
    }
}

// C[0:M, 0:N] (row stride ldb = ldc) = bf16(A[0:M, :]) x bf16(B[:, 0:N]) on bf16 MFMA
bool bf16_region(int M, int N, int ldb, int K, const float* A, const float* B, float* C,
                 hipStream_t s) {
    const int Kp = (K + 127) / 128 * 128;
    if ((long long)M * Kp * 2 >= 0x7fffffffll || (long long)N * Kp * 2 >= 0x7fffffffll) {
        set_error("acfun_gemm_bf16: operands beyond 2 GB");
        return false;
    }
    Scratch ab((size_t)M * Kp * 2, s), bt((size_t)N * Kp * 2, s);
    if (!ab.p || !bt.p) return false;
    const long long na = (long long)M * (Kp / 8);
    const long long nba = (na + 255) / 256, nbb = (long long)(Kp / 64) * ((N + 63) / 64);
    if (nba + nbb >= (1ll << 31)) {
        set_error("acfun_gemm_bf16: operands too large");
        return false;
    }
    auto al = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
    const int va = al(A) && K % 4 == 0, vb = al(B) && ldb % 4 == 0 && N % 4 == 0;
    ACFUN_LAUNCH("k_pack_bf16", k_pack_bf16, dim3((unsigned)(nba + nbb)), dim3(256), 0, s, A, B, M, N, K, K, ldb, Kp,
                       (int)nba, ab.as<unsigned short>(), bt.as<unsigned short>(), va, vb);
    if (!check_launch("k_pack_bf16")) return false;
    constexpr int lds = BF_NST * BF_STG;
    // set once per process, thread-safely, before any launch below
    static const bool attr = [&] {
        (void)hipFuncSetAttribute((const void*)k_bf16mm, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
        return true;
    }();
    (void)attr;
    const long long tiles = (long long)((M + BF_BM - 1) / BF_BM) * ((N + BF_BN - 1) / BF_BN);
    ACFUN_LAUNCH("k_bf16mm", k_bf16mm, dim3((unsigned)tiles), dim3(256), lds, s, ab.as<unsigned short>(),
                 bt.as<unsigned short>(), C, M, N, Kp, ldb, (unsigned)((long long)M * Kp * 2),
                 (unsigned)((long long)N * Kp * 2));
    return check_launch("k_bf16mm");
}

}  // namespace

// The reference's split (src/gemm_bf16_avx512.cpp:123-168): its 16 x 16
// micro-tiles multiply bf16-rounded operands; the rows past the last multiple
// of 16 of M and the columns past the last multiple of 16 of N (its 256 x 128
// tiles are multiples of 16) take the scalar fp32 path on the unrounded
// operands.  Here k_bf16mm covers the first region and the fp32 GEMM engine
// the two strips.  K <= 0 leaves C untouched, as there (:173).
bool gemm_bf16_dev(int M, int N, int K, const float* A, const float* B, float* C, hipStream_t s) {
    if (M <= 0 || N <= 0 || K <= 0) return true;
    const int M16 = M / 16 * 16, N16 = N / 16 * 16;
    if (M16 < M && !gemm_f32(M - M16, N, K, A + (long long)M16 * K, K, B, N, C + (long long)M16 * N, N,
                             nullptr, 0, s))
        return false;
    if (N16 < N && M16 > 0 && !gemm_f32(M16, N - N16, K, A, K, B + N16, N, C + N16, N, nullptr, 0, s))
        return false;
    if (M16 == 0 || N16 == 0) return true;
    return bf16_region(M16, N16, N, K, A, B, C, s);
}

}  // namespace acfun
