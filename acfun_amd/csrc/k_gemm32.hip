// k_gemm32.hip -- fp32 GEMM C[M,N] = A[M,K] * B[K,N] (+bias[n], ReLU) on
// v_mfma_f32_32x32x2f32 with LDS-DMA staging: the engine behind acfun_gemm,
// acfun_gemm_epi, acfun_fc and the 1x1 conv route (reference
// src/gemm_avx512.cpp:245-337, src/layers.cpp:19-36,66-101) whenever the
// operands are 16-byte aligned with K, N, lda, ldb multiples of 4.
//
// Workgroup = 64 x 64 tile of C, 4 waves in a 2 x 2 grid, each wave one
// 32 x 32 accumulator (16 registers per lane): a single dependent MFMA chain,
// which gfx950 issues back to back.  K is consumed in chunks of KC = 64:
//   A stage [64 rows][16 quads], quad q of row r at slot q ^ (r & 15);
//   B stage [64 k][16 quads],    quad q of row k at slot q ^ ((k & 32) >> 2);
// or KC = 32:
//   A stage [64 rows][8 quads],  quad q of row r at slot q ^ ((r >> 1) & 7);
//   B stage [32 k][16 quads],    quad q of row k at slot q ^ ((k & 16) >> 1).
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
//
// KS > 1: KS groups of four waves in one workgroup split K by chunk
// (group kg takes chunks kg, kg + KS, ...), each with its own stages; the
// groups' accumulators are summed through LDS at the end, group 1's first.
// With two groups each group finalizes and stores half of the tile, so all
// eight waves share the merge and the stores.
#include "rt.hpp"

#include <cstdlib>
#include <memory>

namespace acfun {
namespace {

typedef float f16v __attribute__((ext_vector_type(16)));
typedef float f4g __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void32;


// Implicit-GEMM convolution geometry (CONV mode): A is the NHWC input
// [n][H][W][Cin], row m of the GEMM the output pixel (n, oh, ow), k = tap*Cin + ic.
struct G32Conv {
    int H, W, Cin, KW, stride, pad, OH, OW;
    unsigned bytes;    // N*H*W*Cin*4, below 2^31
};

constexpr int g32_stage(int BM, int BN, int KC) { return BM * KC + KC * BN; }   // floats
constexpr int g32_vmcnt(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0F70; }

template <int BM, int BN, int NST, bool CONV, int KS, int KC>
__global__ __launch_bounds__(256 * KS) void k_gemm32(const float* __restrict__ A,
                                                const float* __restrict__ B,
                                                float* __restrict__ C,
                                                const float* __restrict__ bias,
                                                const float* __restrict__ res, int M, int N,
                                                int K, int lda, int ldb, int ldc, int ldr,
                                                int act, G32Conv cv) {
    constexpr unsigned kOOB = 0x80000000u;
    constexpr int FM = BM / 64, FN = BN / 64;          // 32 x 32 blocks per wave
    constexpr int STAGE = g32_stage(BM, BN, KC);
    constexpr int SB = BM * KC;                         // B's offset in a stage (floats)
    constexpr int QA = KC / 4;                          // quads per A row
    constexpr int RPI = 64 / QA;                        // A rows per DMA instruction
    constexpr int AIT = BM * QA / 256, BIT = KC * BN / 1024;   // DMA instructions per wave per chunk
    constexpr int ITEMS = AIT + BIT;
    constexpr int BQ = BN / 4;                          // quads per B row
    constexpr int KSTEP = KC / 2;                       // MFMA k-steps per chunk
    static_assert(KC == 64 || KC == 32, "chunk of 32 or 64");
    static_assert(AIT >= 1 && BIT >= 1, "whole DMA instructions");
    extern __shared__ __attribute__((aligned(16))) float sm[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // KS > 1: group kg = wave / 4 takes chunks kg, kg + KS, ... with its own
    // stages; the accumulators are summed through LDS at the end.
    const int kg = KS > 1 ? wave >> 2 : 0, wl = wave & 3;
    const int wm = wl >> 1, wn = wl & 1;
    // Tile order: the 1-D grid is cut into 8 contiguous runs, one per XCD
    // (workgroup id mod 8), and within a run tiles go in groups of 4 tile rows,
    // column-major inside a group -- so the workgroups one XCD runs at a time
    // cover a compact patch and their A rows and B columns share its L2.
    const int gn = (N + BN - 1) / BN, gm = (M + BM - 1) / BM, total = gm * gn;
    int L = blockIdx.x;
    if ((total & 7) == 0) L = (L & 7) * (total >> 3) + (L >> 3);
    constexpr int GRP = 4;
    const int grp = L / (GRP * gn), gbase = grp * GRP;
    const int rows = gm - gbase < GRP ? gm - gbase : GRP;
    const int r_in = L - grp * GRP * gn;
    const int tm = gbase + r_in % rows, tn = r_in / rows;
    const int m0 = tm * BM, n0 = tn * BN;
    const int nch0 = (K + KC - 1) / KC;
    const int nch = (nch0 + KS - 1) / KS;                 // chunks per group (local)

    // ---- DMA descriptors.  A: wave w issues instructions w + 4t (t < AIT),
    // each RPI rows x QA quads; lane l -> row RPI(w + 4t) + l/QA, quad slot
    // l%QA.  B: instructions w + 4t (t < BIT), each 64 slots of k rows of BQ
    // quads.
    const __amdgpu_buffer_rsrc_t ares = CONV
        ? __builtin_amdgcn_make_buffer_rsrc((void*)A, (short)0, (int)cv.bytes, 0x00020000)
        : __builtin_amdgcn_make_buffer_rsrc(
              (void*)(A + (long long)m0 * lda), (short)0,
              (int)((long long)(M - m0) * lda * 4 < 0x7fffffff ? (long long)(M - m0) * lda * 4 : 0x7fffffff),
              0x00020000);
    const __amdgpu_buffer_rsrc_t bres = __builtin_amdgcn_make_buffer_rsrc(
        (void*)B, (short)0, (int)((long long)K * ldb * 4), 0x00020000);
    const int arow = RPI * wl + lane / QA;                 // + 4 RPI t
    // the quad this lane's slot holds (the swizzle is the same for every t:
    // 4 RPI t is a multiple of 16)
    const int aq = KC == 64 ? (lane & 15) ^ (arow & 15) : (lane & 7) ^ ((arow >> 1) & 7);
    const unsigned av = (unsigned)(arow * lda + 4 * aq) * 4u;
    const unsigned astep = 4u * RPI * lda * 4u;            // 4 RPI rows per t
    // CONV: per row t, the byte offset of channel quad aq of tap (0, 0) and the
    // in-image taps as bits kh*8 + kw (KH, KW <= 8)
    int cbase[AIT];
    unsigned long long cmask[AIT];
    if (CONV) {
#pragma unroll
        for (int t = 0; t < AIT; ++t) {
            const int m = m0 + arow + 4 * RPI * t;
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
    bool bok[BIT];
    unsigned bv[BIT];
#pragma unroll
    for (int t = 0; t < BIT; ++t) {
        const int slot = 64 * (wl + 4 * t) + lane;
        const int krow = slot / BQ;
        const int q = (slot % BQ) ^ ((krow & (KC / 2)) ? 8 : 0);   // quad q of k row r: slot q ^ 8[r >= KC/2]
        bok[t] = n0 + 4 * q < N;
        bv[t] = (unsigned)(krow * ldb + n0 + 4 * q) * 4u;
    }
    const bool kragged = (K & (KC - 1)) != 0;

    // Every variable part of an address is in the per-lane offset (which the
    // buffer range check covers); the scalar offset stays 0.
    auto issue = [&](int t, int c, float* st) {            // item t of (local) chunk c into stage st
        const int k0 = (KS * c + kg) * KC;
        if (t < AIT) {
            unsigned v;
            if (KS > 1 && k0 >= K) {
                v = kOOB;                                   // a group's padding chunk: zeros
            } else if (CONV) {
                // a chunk lies in one tap (Cin % 64 == 0): wave-uniform
                const int tap = k0 / cv.Cin, ic0 = k0 - tap * cv.Cin;
                const int kh = tap / cv.KW, kw = tap - kh * cv.KW;
                const bool ok = (cmask[t] >> (kh * 8 + kw)) & 1ull;
                v = ok ? (unsigned)(cbase[t] + ((kh * cv.W + kw) * cv.Cin + ic0) * 4) : kOOB;
            } else {
                v = av + (unsigned)k0 * 4u + (unsigned)t * astep;
                if (kragged && k0 + 4 * aq >= K) v = kOOB;
            }
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ares, (lds_void32*)(st + (wl + 4 * t) * 256),
                                                     16, v, 0, 0, 0);
        } else {
            const int tt = t - AIT;
            const unsigned v = bok[tt] && k0 < K ? bv[tt] + (unsigned)k0 * ldb * 4u : kOOB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                bres, (lds_void32*)(st + SB + (wl + 4 * tt) * 256), 16, v, 0, 0, 0);
        }
    };

    // ---- per-lane read offsets within a stage (floats).  MFMA k assignment:
    // in k-step s of a chunk, lane half h carries k = (KC/2) h + s for both
    // operands.
    const int r = lane & 31, h = lane >> 5;
    constexpr int AQ = KC / 8;                          // A quads a lane reads per chunk
    int aoff[FM][AQ], boff[FN];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        const int rowA = (BM / 2) * wm + 32 * i + r;
#pragma unroll
        for (int j = 0; j < AQ; ++j)
            aoff[i][j] = KC == 64 ? (rowA * 16 + ((8 * h + j) ^ (rowA & 15))) * 4
                                  : (rowA * 8 + ((4 * h + j) ^ ((rowA >> 1) & 7))) * 4;
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int col = (BN / 2) * wn + 32 * j + r;
        boff[j] = SB + ((KSTEP * h) * BQ + ((col >> 2) ^ (h << 3))) * 4 + (col & 3);
    }

    f16v acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    // Bias of this lane's columns, loaded first (loads complete in issue order)
    // so its latency hides behind chunk 0's.
    float bn[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int n = n0 + (BN / 2) * wn + 32 * j + r;
        bn[j] = (bias && n < N) ? bias[n] : 0.f;
    }
    // With one 32 x 32 block per wave the residual is loaded up front as well.
    constexpr bool PRE = FM * FN == 1;
    float rv0[16];
    if (PRE) {
        const int n = n0 + (BN / 2) * wn + r;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int m = m0 + (BM / 2) * wm + 8 * (e >> 2) + 4 * h + (e & 3);
            rv0[e] = (res && n < N && m < M) ? res[(long long)m * ldr + n] : 0.f;
        }
    }

    // Chunk c goes to stage c % NST, and chunk c + NST - 1 is issued while
    // chunk c is multiplied.
    constexpr int AHEAD = NST - 1;
    static_assert(NST >= 2 && NST <= 4, "two to four stages");
    float* const smg = sm + kg * NST * STAGE;           // this group's stages
#pragma unroll
    for (int c0 = 0; c0 < AHEAD; ++c0) {
        if (c0 < nch) {
#pragma unroll
            for (int t = 0; t < ITEMS; ++t) issue(t, c0, smg + c0 * STAGE);
        }
    }

    // Software pipeline per chunk c (operands in registers):
    //   the DMA of chunk c+AHEAD, all of it up front (issued between the first
    //   k-steps' MFMAs it measured 4 % slower at 1024^3: the last loads had
    //   only the deferred k-steps to land in);
    //   MFMAs of k-steps 0..27;
    //   the last four k-steps' operands set aside;
    //   wait for chunk c+1's DMA, LDS-only barrier, LDS reads of all of chunk
    //   c+1's operands;
    //   MFMAs of k-steps 28..31 of chunk c, which cover the barrier and the
    //   LDS latency of the reads.
    // The barrier before chunk c+1's reads also orders every wave's reads of
    // chunk c-1's stage before the DMA of chunk c+AHEAD overwrites it.
    constexpr int DEFER = 4;
    f4g a[FM][AQ];
    float bb[FN][KSTEP];
    auto wait_chunk = [&](int c) {            // chunk c's DMA has landed (everyone's)
        // outstanding in issue order: ..., chunk c, then chunks c+1 ..
        // min(c + AHEAD - 1, nch - 1) (ITEMS loads each) that may stay in flight
        const int later = nch - 1 - c < AHEAD - 1 ? nch - 1 - c : AHEAD - 1;
        if (AHEAD >= 3 && later >= 2) __builtin_amdgcn_s_waitcnt(g32_vmcnt(2 * ITEMS));
        else if (AHEAD >= 2 && later >= 1) __builtin_amdgcn_s_waitcnt(g32_vmcnt(ITEMS));
        else __builtin_amdgcn_s_waitcnt(g32_vmcnt(0));
        // LDS-only workgroup barrier: this wave's LDS reads are complete; the
        // loads of later chunks stay in flight.
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    auto read_chunk = [&](const float* S) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < AQ; ++j) a[i][j] = *(const f4g*)&S[aoff[i][j]];
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int s = 0; s < KSTEP; ++s) bb[j][s] = S[boff[j] + s * BN];
    };
    if (nch > 0) {
        wait_chunk(0);
        read_chunk(smg);
    }
    int st = 0;                                         // c % NST
    for (int c = 0; c < nch; ++c) {
        const int sta = st == 0 ? AHEAD : st - 1;       // (c + AHEAD) % NST
        float* NA = smg + sta * STAGE;
        const bool more = c + AHEAD < nch;
#pragma unroll
        for (int s = 0; s < KSTEP - DEFER; ++s) {
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][s >> 2][s & 3], bb[j][s],
                                                                     acc[i][j], 0, 0, 0);
            if (more && s == 0) {                  // its stage was read before this chunk
#pragma unroll
                for (int t = 0; t < ITEMS; ++t) issue(t, c + AHEAD, NA);
            }
        }
        f4g al[FM];
        float bl[FN][DEFER];
#pragma unroll
        for (int i = 0; i < FM; ++i) al[i] = a[i][AQ - 1];
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int u = 0; u < DEFER; ++u) bl[j][u] = bb[j][KSTEP - DEFER + u];
        st = st == NST - 1 ? 0 : st + 1;
        if (c + 1 < nch) {
            wait_chunk(c + 1);
            read_chunk(smg + st * STAGE);
        }
#pragma unroll
        for (int u = 0; u < DEFER; ++u)
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(al[i][u], bl[j][u], acc[i][j], 0, 0, 0);
    }

    // Each output is group 0's sum plus the other groups' partials, in group
    // order.  Two groups: each finalizes half of every block's registers
    // (group 0 e < 8, group 1 e >= 8), adding the other group's partial read
    // back from LDS (g0 + g1 is the same float sum in either order), and
    // stores that half.  More groups: their partials through LDS into group 0.
    int e_lo = 0;                                       // this wave's first register to store
    if (KS == 2) {
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");   // stages no longer read
        float* const red = sm + wl * (FM * FN * 16 * 64) + lane;   // slot e of block b: (16 b + e) * 64
        auto hand = [&](auto kgc) {
            constexpr int G = decltype(kgc)::value;
            constexpr int GIVE = G == 0 ? 8 : 0, KEEP = 8 - GIVE;
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        red[((i * FN + j) * 16 + GIVE + e) * 64] = acc[i][j][GIVE + e];
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        acc[i][j][KEEP + e] += red[((i * FN + j) * 16 + KEEP + e) * 64];
        };
        if (kg == 0) hand(std::integral_constant<int, 0>{});
        else hand(std::integral_constant<int, 1>{});
        e_lo = kg == 0 ? 0 : 8;
    } else if (KS > 2) {
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");   // stages no longer read
        constexpr int PART = 4 * FM * FN * 16 * 64;     // floats of one group's partial tile
        float* const red = sm + wl * (FM * FN * 16 * 64) + lane;
        if (kg > 0) {
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int e = 0; e < 16; ++e) red[(kg - 1) * PART + ((i * FN + j) * 16 + e) * 64] = acc[i][j][e];
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (kg > 0) return;
#pragma unroll
        for (int g = 0; g < KS - 1; ++g)
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int e = 0; e < 16; ++e) acc[i][j][e] += red[g * PART + ((i * FN + j) * 16 + e) * 64];
    }

    // ---- epilogue: lane l, register e of block (i, j) <->
    //      row m0 + BM/2*wm + 32i + 8*(e/4) + 4*(l/32) + e%4, column n0 + BN/2*wn + 32j + l%32
    //      (registers E0 .. E1-1 of this wave)
    auto store = [&](auto e0c, auto e1c) {
        constexpr int E0 = decltype(e0c)::value, E1 = decltype(e1c)::value;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int n = n0 + (BN / 2) * wn + 32 * j + r;
            if (n >= N) continue;
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                float rv[16];
                if (res && !PRE) {                        // all the loads in flight at once
#pragma unroll
                    for (int e = E0; e < E1; ++e) {
                        const int m = m0 + (BM / 2) * wm + 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
                        rv[e] = m < M ? res[(long long)m * ldr + n] : 0.f;
                    }
                }
#pragma unroll
                for (int e = E0; e < E1; ++e) {
                    const int m = m0 + (BM / 2) * wm + 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
                    if (m < M) {
                        float v = acc[i][j][e];
                        if (bias) v = v + bn[j];
                        if (res) v = v + (PRE ? rv0[e] : rv[e]);   // fused residual Add
                        v = act_apply(v, act);
                        // non-temporal: C streams out instead of waiting dirty in
                        // L2 for the kernel's final write-back
                        __builtin_nontemporal_store(v, &C[(long long)m * ldc + n]);
                    }
                }
            }
        }
    };
    if (KS != 2) store(std::integral_constant<int, 0>{}, std::integral_constant<int, 16>{});
    else if (e_lo == 0) store(std::integral_constant<int, 0>{}, std::integral_constant<int, 8>{});
    else store(std::integral_constant<int, 8>{}, std::integral_constant<int, 16>{});
}

// ---------------------------------------------------------------- k_gemm32p
// Persistent form for short K and many tiles, where one tile per workgroup
// leaves a tile's load latency and epilogue exposed: each workgroup runs a
// list of 64 x 64 tiles back to back, and one DMA stream of (tile, chunk)
// items runs NST - 1 chunks ahead of the MFMAs across tile boundaries, so
// the next tile's operands load during the current tile's last chunks and
// its epilogue.  K in chunks of 32 (the KC = 32 stage layouts above), NST
// stages of 16 KB, three workgroups per CU.  Tiles: XCD x = blockIdx % 8 owns
// a contiguous run of k_gemm32's tile order, which its workgroups take round
// robin.  Every iteration issues the same number of DMA loads (items past
// the workgroup's last chunk are issued out of range and write zeros to a
// stage no chunk reads again), so every wait of the loop is the same.
// Epilogue: the waves write the tile's sums into the stage of its last chunk
// (every wave has read it), then thread t forms quad t % 16 of rows t/16 +
// 16i: + bias, + the fused residual, the activation, one 16-byte store (rows
// and quads past M and N element by element).  Per output the arithmetic is
// k_gemm32's: the chunk sums in k order, then fl(fl(sum + bias) + res).
template <int NST, bool CONV>
__global__ __launch_bounds__(256) void k_gemm32p(const float* __restrict__ A,
                                                 const float* __restrict__ B,
                                                 float* __restrict__ C,
                                                 const float* __restrict__ bias,
                                                 const float* __restrict__ res, int M, int N, int K,
                                                 int lda, int ldb, int ldc, int ldr, int act, int vec,
                                                 unsigned a_bytes, G32Conv cv) {
    constexpr int BM = 64, BN = 64, KC = 32;
    constexpr int STAGE = g32_stage(BM, BN, KC);        // 4096 floats
    constexpr int SB = BM * KC;
    constexpr int QA = KC / 4, RPI = 64 / QA;           // 8 quads per A row, 8 rows per instruction
    constexpr int AIT = BM * QA / 256, BIT = KC * BN / 1024;
    constexpr int ITEMS = AIT + BIT;
    constexpr int BQ = BN / 4, KSTEP = KC / 2, AQ = KC / 8;
    constexpr int AHEAD = NST - 1;
    static_assert(NST >= 2 && AIT == 2 && BIT == 2, "k_gemm32p layout");
    constexpr unsigned kOOB = 0x80000000u;
    extern __shared__ __attribute__((aligned(16))) float sm[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;

    const int gn = (N + BN - 1) / BN, gm = (M + BM - 1) / BM, total = gm * gn;
    const int G = (int)gridDim.x, b = (int)blockIdx.x;
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
    const int nch = (K + KC - 1) / KC;
    const int nit = cnt * nch;
    if (nit == 0) return;                               // uniform per workgroup
    constexpr int GRP = 4;
    auto tile_of = [&](int k, int& m0, int& n0) {      // k-th tile of this workgroup
        const int L = t0 + k * tstr;
        const int grp = L / (GRP * gn), gbase = grp * GRP;
        const int rows = gm - gbase < GRP ? gm - gbase : GRP;
        const int r_in = L - grp * GRP * gn;
        m0 = (gbase + r_in % rows) * BM;
        n0 = (r_in / rows) * BN;
    };

    const __amdgpu_buffer_rsrc_t ares =
        __builtin_amdgcn_make_buffer_rsrc((void*)A, (short)0, (int)a_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t bres = __builtin_amdgcn_make_buffer_rsrc(
        (void*)B, (short)0, (int)((long long)K * ldb * 4), 0x00020000);
    // DMA slots of this lane (the KC = 32 layouts): A row arow + 32t, quad aq;
    // B k row krow[t], quad bq[t]
    const int arow = RPI * wave + lane / QA;
    const int aq = (lane & 7) ^ ((arow >> 1) & 7);
    int bkr[BIT], bq4[BIT];
#pragma unroll
    for (int t = 0; t < BIT; ++t) {
        const int slot = 64 * (wave + 4 * t) + lane;
        bkr[t] = slot / BQ;
        bq4[t] = 4 * ((slot % BQ) ^ ((bkr[t] & (KC / 2)) ? 8 : 0));
    }
    const bool kragged = (K & (KC - 1)) != 0;
    // issue cursor: tile ik of this workgroup, chunk ic; its rows' descriptors
    int ik = 0, ic = 0, in0 = 0;
    unsigned arowoff[AIT];                              // plain: byte offset of the row (kOOB past M)
    int cbase[AIT];                                     // CONV: tap-(0,0) offset, in-image taps
    unsigned long long cmask[AIT];
    auto setup = [&](int k) {
        int m0, n0;
        tile_of(k, m0, n0);
        in0 = n0;
#pragma unroll
        for (int t = 0; t < AIT; ++t) {
            const int m = m0 + arow + 32 * t;
            if (!CONV) {
                arowoff[t] = m < M ? (unsigned)(m * lda + 4 * aq) * 4u : kOOB;
            } else {
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
    };
    // item t of the issue cursor's chunk into stage st (out of range when !live)
    auto issue = [&](int t, float* st, bool live) {
        const int k0 = ic * KC;
        if (t < AIT) {
            unsigned v = kOOB;
            if (live) {
                if (CONV) {
                    const int tap = k0 / cv.Cin, ic0 = k0 - tap * cv.Cin;
                    const int kh = tap / cv.KW, kw = tap - kh * cv.KW;
                    if ((cmask[t] >> (kh * 8 + kw)) & 1ull)
                        v = (unsigned)(cbase[t] + ((kh * cv.W + kw) * cv.Cin + ic0) * 4);
                } else if (arowoff[t] != kOOB && !(kragged && k0 + 4 * aq >= K)) {
                    v = arowoff[t] + (unsigned)k0 * 4u;
                }
            }
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ares, (lds_void32*)(st + (wave + 4 * t) * 256), 16, v, 0,
                                                     0, 0);
        } else {
            const int tt = t - AIT;
            const unsigned v = live && in0 + bq4[tt] < N && k0 + bkr[tt] < K
                                   ? (unsigned)((k0 + bkr[tt]) * ldb + in0 + bq4[tt]) * 4u
                                   : kOOB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(bres, (lds_void32*)(st + SB + (wave + 4 * tt) * 256), 16, v,
                                                     0, 0, 0);
        }
    };
    auto advance = [&]() {
        if (++ic == nch) {
            ic = 0;
            if (++ik < cnt) setup(ik);
        }
    };

    // per-lane read offsets within a stage (floats): in k-step s lane half h
    // carries k = 16h + s
    const int r = lane & 31, h = lane >> 5;
    int aoff[AQ];
    const int rowA = 32 * wm + r;
#pragma unroll
    for (int j = 0; j < AQ; ++j) aoff[j] = (rowA * 8 + ((4 * h + j) ^ ((rowA >> 1) & 7))) * 4;
    const int col = 32 * wn + r;
    const int boff = SB + ((KSTEP * h) * BQ + ((col >> 2) ^ (h << 3))) * 4 + (col & 3);

    f16v acc;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.f;

    setup(0);
#pragma unroll
    for (int a = 0; a < AHEAD; ++a) {
        const bool live = a < nit;
#pragma unroll
        for (int t = 0; t < ITEMS; ++t) issue(t, sm + a * STAGE, live);
        if (live) advance();
    }

    int st = 0, ck = 0, cc = 0;
    for (int g = 0; g < nit; ++g) {
        // Chunk g has landed once at most the (AHEAD - 1) * ITEMS loads issued
        // after it are outstanding: loads complete in issue order, and the
        // epilogue's inline-asm stores queued among them only lengthen the wait.
        __builtin_amdgcn_s_waitcnt(g32_vmcnt((AHEAD - 1) * ITEMS));
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        const float* S = sm + st * STAGE;
        float* NA = sm + (st == 0 ? NST - 1 : st - 1) * STAGE;   // (g + AHEAD) % NST
        const bool more = g + AHEAD < nit;
        f4g a[AQ];
        float bb[KSTEP];
#pragma unroll
        for (int j = 0; j < AQ; ++j) a[j] = *(const f4g*)&S[aoff[j]];
#pragma unroll
        for (int k = 0; k < KSTEP; ++k) bb[k] = S[boff + k * BN];
#pragma unroll
        for (int k = 0; k < KSTEP; ++k) {
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[k >> 2][k & 3], bb[k], acc, 0, 0, 0);
            if (k == 1) {
#pragma unroll
                for (int t = 0; t < ITEMS; ++t) issue(t, NA, more);
            }
        }
        if (more) advance();
        st = st == NST - 1 ? 0 : st + 1;
        if (++cc < nch) continue;
        cc = 0;
        // ---- epilogue of tile ck through the stage of its last chunk
        int m0, n0;
        tile_of(ck, m0, n0);
        ++ck;
        float* const stg = sm + (st == 0 ? NST - 1 : st - 1) * STAGE;
        auto sidx = [](int rr, int cq) { return rr * 64 + ((((cq >> 2) ^ (((rr >> 2) & 1) << 3))) << 2) + (cq & 3); };
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int rr = 32 * wm + 8 * (e >> 2) + 4 * h + (e & 3);
            stg[sidx(rr, col)] = acc[e];
            acc[e] = 0.f;
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        const int q = tid & 15, n = n0 + 4 * q;
        f4g bq = {0.f, 0.f, 0.f, 0.f};
        if (bias) {
            if (vec && n + 4 <= N) {
                bq = *(const f4g*)(bias + n);
            } else {
#pragma unroll
                for (int kq = 0; kq < 4; ++kq) bq[kq] = n + kq < N ? bias[n + kq] : 0.f;
            }
        }
        const bool full = m0 + BM <= M && n0 + BN <= N;
        f4g rv[4];
        if (res && vec && full) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                rv[i] = *(const f4g*)(res + (long long)(m0 + (tid >> 4) + 16 * i) * ldr + n);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int rr = (tid >> 4) + 16 * i, m = m0 + rr;
            if (m >= M) continue;
            f4g v = *(const f4g*)&stg[sidx(rr, 4 * q)];
            float* dst = C + (long long)m * ldc + n;
            if (vec && n + 4 <= N) {
                if (bias) v = v + bq;
                if (res) v = v + (full ? rv[i] : *(const f4g*)(res + (long long)m * ldr + n));
#pragma unroll
                for (int kq = 0; kq < 4; ++kq) v[kq] = act_apply(v[kq], act);
                // s_nop: a VALU write to the data registers of a store of more
                // than 8 bytes needs a wait state after it
                asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1" ::"v"(dst), "v"(v) : "memory");
            } else {
#pragma unroll
                for (int kq = 0; kq < 4; ++kq) {
                    if (n + kq >= N) continue;
                    float w = v[kq];
                    if (bias) w = w + bq[kq];
                    if (res) w = w + res[(long long)m * ldr + n + kq];
                    w = act_apply(w, act);
                    asm volatile("global_store_dword %0, %1, off sc1" ::"v"(dst + kq), "v"(w) : "memory");
                }
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(g32_vmcnt(0));          // the out-of-range loads and the stores
}

}  // namespace

namespace {
struct G32Tile { int bm, bn, nst, ks = 1, kc = 64, pers = 0; };

// Tile choice.  Measured on MI355X (config 1 and the ResNet-50 batch-64
// layers): 64 x 64 tiles, two or three workgroups per CU, beat the 128-row
// tiles at every K, since one workgroup per CU leaves the DMA latency and the
// epilogue exposed.  ACFUN_G32_KMIN=<K> enables the larger tiles from that K
// (sweeps).  Three stages when the 64 x 64 grid is a single wave of workgroups.
G32Tile pick_g32(int M, int N, int K) {
    const long long cus = num_cus();
    const int nch = (K + 63) / 64;
    auto tiles = [&](int bm, int bn) {
        return (long long)((M + bm - 1) / bm) * ((N + bn - 1) / bn);
    };
    // ACFUN_G32_KMIN: the K from which the larger tiles are used (sweeps)
    static const int kmin = [] {
        const char* e = getenv("ACFUN_G32_KMIN");
        return e ? atoi(e) : 0x7fffffff;
    }();
    if (K >= kmin && N > 64 && tiles(128, 128) >= cus) return G32Tile{128, 128, 2};
    if (K >= kmin && tiles(128, 64) >= cus) return G32Tile{128, 64, nch > 2 ? 3 : 2};
    // At most one 64 x 64 tile per CU and a long K: two four-wave groups per
    // workgroup split K (two waves per SIMD instead of one).
    static const bool ks_off = getenv("ACFUN_G32_NOKS") != nullptr;
    if (!ks_off && nch >= 8 && tiles(64, 64) <= cus) return G32Tile{64, 64, 2, 2};
    // Two or more 64 x 64 tiles per CU: the persistent kernel, two stages,
    // four workgroups per CU (config 5, fp32: 5.71 -> 5.09 ms per batch of 64;
    // three stages at three per CU: 5.33 ms).  ACFUN_G32P=0 turns it off.
    static const bool pers = [] {
        const char* e = getenv("ACFUN_G32P");
        return !(e && atoi(e) == 0);
    }();
    if (pers && tiles(64, 64) >= 2 * cus) return G32Tile{64, 64, 2, 1, 32, 1};
    // Three stages (one workgroup per CU) only when the tiles fit in one wave;
    // between one and two tiles per CU two stages at two workgroups per CU
    // (config 5's 392-tile layers: GEMM 3136 x 512 x 2048 94.9 -> 81.0 us,
    // conv 3x3/2 14x14x512 203 -> 174 us).
    const bool deep = nch > 2 && tiles(64, 64) <= cus;
    return G32Tile{64, 64, deep ? 3 : 2};
}

template <int BM, int BN, int NST, bool CONV, int KS = 1, int KC = 64>
bool launch_g32(int M, int N, int K, const float* A, int lda, const float* B, int ldb, float* C,
                int ldc, const float* bias, int act, hipStream_t s, const float* res, int ldr,
                const G32Conv& cv) {
    const int nch = ((K + KC - 1) / KC + KS - 1) / KS;
    // LDS holds only the stages that can be in use (per group); with K groups
    // the partial tiles of groups 1..KS-1 are summed through the same memory
    const int stages = KS > 1 ? NST : (nch < NST ? (nch < 1 ? 1 : nch) : NST);
    constexpr size_t kPart = (size_t)(KS - 1) * BM * BN * 4;
    const size_t lds0 = (size_t)KS * stages * g32_stage(BM, BN, KC) * 4;
    const size_t lds = lds0 > kPart ? lds0 : kPart;
    constexpr size_t kMax = (size_t)KS * NST * g32_stage(BM, BN, KC) * 4;
    static_assert(kMax >= kPart && kMax <= 160 * 1024, "LDS budget");
    // set once per process, thread-safely, before any launch below
    static const bool attr = [&] {
        (void)hipFuncSetAttribute((const void*)k_gemm32<BM, BN, NST, CONV, KS, KC>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMax);
        return true;
    }();
    (void)attr;
    dim3 grid((unsigned)(((N + BN - 1) / BN) * ((M + BM - 1) / BM)));
    ACFUN_LAUNCH("k_gemm32", (k_gemm32<BM, BN, NST, CONV, KS, KC>), grid, dim3(256 * KS), lds, s, A, B,
                 C, bias, res, M, N, K, lda, ldb, ldc, ldr, act, cv);
    return check_launch("k_gemm32");
}

// Persistent launch (k_gemm32p): as many workgroups as fit on a CU (four
// with two stages, three with three), at most one per tile, a multiple of 8
// so that each XCD owns a run of tiles.
template <int NST, bool CONV>
bool launch_g32p(int M, int N, int K, const float* A, int lda, const float* B, int ldb, float* C, int ldc,
                 const float* bias, int act, hipStream_t s, const float* res, int ldr, const G32Conv& cv) {
    constexpr size_t lds = (size_t)NST * g32_stage(64, 64, 32) * 4;
    static_assert(lds <= 160 * 1024 / 2, "two workgroups per CU at least");
    // set once per process, thread-safely, before any launch below
    static const bool attr = [&] {
        (void)hipFuncSetAttribute((const void*)k_gemm32p<NST, CONV>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)lds);
        return true;
    }();
    (void)attr;
    const long long tiles = (long long)((M + 63) / 64) * ((N + 63) / 64);
    const long long slots = (NST == 2 ? 4ll : 3ll) * num_cus(), need = (tiles + 7) / 8 * 8;
    const unsigned grid = (unsigned)(slots < need ? slots : need);
    auto al = [](const void* q) { return ((uintptr_t)q & 15u) == 0; };
    const int vec = al(C) && ldc % 4 == 0 && (!bias || al(bias)) && (!res || (al(res) && ldr % 4 == 0));
    const unsigned a_bytes = CONV ? cv.bytes : (unsigned)((long long)M * lda * 4);
    ACFUN_LAUNCH("k_gemm32", (k_gemm32p<NST, CONV>), dim3(grid), dim3(256), lds, s, A, B, C, bias, res, M, N,
                 K, lda, ldb, ldc, ldr, act, vec, a_bytes, cv);
    return check_launch("k_gemm32p");
}

// Tile-search candidates (kind "g32"): 64 x 64 with 2 or 3 stages, 64 x 64
// with two K groups, 128 x 64 with 2 or 3 stages, 128 x 128; then 32-wide
// chunks: 64 x 64 with four K groups (1,024 threads, four waves per SIMD),
// and with two K groups three or four stages deep; then the persistent
// kernel with 2 or 3 stages.
constexpr G32Tile kG32Cand[] = {{64, 64, 2, 1},        {64, 64, 3, 1},        {64, 64, 2, 2},
                                {128, 64, 2, 1},       {128, 64, 3, 1},       {128, 128, 2, 1},
                                {64, 64, 2, 4, 32},    {64, 64, 3, 2, 32},    {64, 64, 4, 2, 32},
                                {64, 64, 2, 1, 32, 1}, {64, 64, 3, 1, 32, 1}};
constexpr int kG32NC = 11;

int g32_index(const G32Tile& t) {
    for (int i = 0; i < kG32NC; ++i)
        if (kG32Cand[i].bm == t.bm && kG32Cand[i].bn == t.bn && kG32Cand[i].nst == t.nst &&
            kG32Cand[i].ks == t.ks && kG32Cand[i].kc == t.kc && kG32Cand[i].pers == t.pers)
            return i;
    return 0;
}
// K groups need chunks for every group: at least two each.
// The persistent kernel addresses A through one 32-bit buffer resource.
bool g32_admits(int c, int K, long long a_bytes) {
    const G32Tile& t = kG32Cand[c];
    if (t.pers) return a_bytes < 0x7fffffffll;
    return t.ks == 1 || (K + t.kc - 1) / t.kc >= 2 * t.ks;
}

template <bool CONV>
bool launch_cand(int c, int M, int N, int K, const float* A, int lda, const float* B, int ldb,
                 float* C, int ldc, const float* bias, int act, hipStream_t s, const float* res,
                 int ldr, const G32Conv& cv) {
    switch (c) {
        case 1: return launch_g32<64, 64, 3, CONV>(M, N, K, A, lda, B, ldb, C, ldc, bias, act, s, res, ldr, cv);
        case 2: return launch_g32<64, 64, 2, CONV, 2>(M, N, K, A, lda, B, ldb, C, ldc, bias, act, s, res, ldr, cv);
        case 3: return launch_g32<128, 64, 2, CONV>(M, N, K, A, lda, B, ldb, C, ldc, bias, act, s, res, ldr, cv);
        case 4: return launch_g32<128, 64, 3, CONV>(M, N, K, A, lda, B, ldb, C, ldc, bias, act, s, res, ldr, cv);
        case 5: return launch_g32<128, 128, 2, CONV>(M, N, K, A, lda, B, ldb, C, ldc, bias, act, s, res, ldr, cv);
        case 6: return launch_g32<64, 64, 2, CONV, 4, 32>(M, N, K, A, lda, B, ldb, C, ldc, bias, act, s, res, ldr, cv);
        case 7: return launch_g32<64, 64, 3, CONV, 2, 32>(M, N, K, A, lda, B, ldb, C, ldc, bias, act, s, res, ldr, cv);
        case 8: return launch_g32<64, 64, 4, CONV, 2, 32>(M, N, K, A, lda, B, ldb, C, ldc, bias, act, s, res, ldr, cv);
        case 9: return launch_g32p<2, CONV>(M, N, K, A, lda, B, ldb, C, ldc, bias, act, s, res, ldr, cv);
        case 10: return launch_g32p<3, CONV>(M, N, K, A, lda, B, ldb, C, ldc, bias, act, s, res, ldr, cv);
        default: return launch_g32<64, 64, 2, CONV>(M, N, K, A, lda, B, ldb, C, ldc, bias, act, s, res, ldr, cv);
    }
}

// The replay the tile search times for a shape: operands of the shape filled
// with a constant
// (A with lda = K for a GEMM, the NHWC input for a convolution), no epilogue.
template <bool CONV>
TuneMaker g32_maker(int M, int N, int K, const G32Conv& cv) {
    return [=]() -> TuneRunner {
        const size_t abytes = CONV ? (size_t)cv.bytes : (size_t)M * K * 4;
        const size_t bbytes = (size_t)K * N * 4, cbytes = (size_t)M * N * 4;
        if (abytes + bbytes + cbytes > ((size_t)2 << 30)) return TuneRunner();
        hipStream_t s = lib_stream();
        auto a = std::make_shared<Scratch>(abytes, s);
        auto b = std::make_shared<Scratch>(bbytes, s);
        auto c = std::make_shared<Scratch>(cbytes, s);
        if (!a->p || !b->p || !c->p || hipMemsetD32Async((hipDeviceptr_t)a->p, kTuneFill, abytes / 4, s) != hipSuccess ||
            hipMemsetD32Async((hipDeviceptr_t)b->p, kTuneFill, bbytes / 4, s) != hipSuccess)
            return TuneRunner();
        return [=](int cand, hipStream_t st) {
            if (cand < 0) cand = g32_index(pick_g32(M, N, K));     // the built-in choice
            if (!g32_admits(cand, K, CONV ? (long long)cv.bytes : (long long)M * K * 4)) return false;
            return launch_cand<CONV>(cand, M, N, K, a->as<float>(), CONV ? cv.Cin : K, b->as<float>(), N,
                                     c->as<float>(), N, nullptr, 0, st, nullptr, 0, cv);
        };
    };
}

template <bool CONV>
bool launch_gemm32(int M, int N, int K, const float* A, int lda, const float* B, int ldb, float* C,
                   int ldc, const float* bias, int act, hipStream_t s, const float* res, int ldr,
                   const G32Conv& cv) {
    if (M <= 0 || N <= 0) return true;
    const std::vector<int> key = CONV ? std::vector<int>{1, M, N, K, cv.H, cv.W, cv.Cin, cv.KW, cv.stride,
                                                         cv.pad, cv.OH, cv.OW}
                                      : std::vector<int>{0, M, N, K};
    bool rec = false;
    int c = tune_lookup("g32", key, kG32NC, &rec);
    if (rec) {
        tune_record("g32", key, kG32NC, g32_maker<CONV>(M, N, K, cv));
        if (autotune_wanted()) {
            autotune_run();
            c = tune_lookup("g32", key, kG32NC, &rec);
        }
    }
    const long long a_bytes = CONV ? (long long)cv.bytes : (long long)M * lda * 4;
    if (c < 0 || !g32_admits(c, K, a_bytes)) c = g32_index(pick_g32(M, N, K));
    if (!g32_admits(c, K, a_bytes)) c = 0;
    return launch_cand<CONV>(c, M, N, K, A, lda, B, ldb, C, ldc, bias, act, s, res, ldr, cv);
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
           M < (1ll << 31) && (long long)((Cout + 63) / 64) * ((M + 63) / 64) < 0x7fffffffll;
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
           (long long)lda * 16 * 4 < 0x7fffffffll &&
           (long long)((N + 63) / 64) * ((M + 63) / 64) < 0x7fffffffll;
}

}  // namespace acfun

namespace acfun {
void gemm32_register(int M, int N, int K) {
    const std::vector<int> key{0, M, N, K};
    bool rec = false;
    if (tune_lookup("g32", key, kG32NC, &rec) < 0 && rec)
        tune_record("g32", key, kG32NC, g32_maker<false>(M, N, K, G32Conv{}));
}
}  // namespace acfun
