// k_wino43.hip -- Winograd F(4,3) for 3x3 / stride 1 / pad 1 convolutions:
// the persistent unit kernel k_wino43p.
//
// F(4,3) turns a 6x6 input tile into 36 transform points, multiplies each by
// the transformed filter (U = G g G^T, 36 points x Cin x Cout) and folds them
// back into a 4x4 output tile (Y = AT M AT^T): 36 multiplies per 16 outputs
// and input channel, against 16 per 4 for F(2,3) -- 1.78x less matrix work.
// The matrices are the reference's (src/winograd43.cpp:33-54, Lavin's).
//
// Unit = 32 tiles (2 tile rows x 16 tile columns of one image) x 32 output
// channels; one 768-thread workgroup per CU runs a list of units.  Wave w
// (0..11) owns transform row ROW = w / 2 and points (ROW, 3 HALF .. 3 HALF + 2),
// HALF = w % 2, for all 32 tiles: 3 accumulators of v_mfma_f32_32x32x2f32
// (M = tiles, N = output channels, K = 2 input channels).  Input channels are
// consumed in chunks of 8.
//
// Per chunk, the chunk's 10 x 66 input pixels (8 channels) are DMA'd into LDS
// by buffer_load ... lds (zeros past the image through the buffer range
// check), two chunks ahead through three buffers, and each wave forms its 3
// transform points from them in registers: t[b] = sum_a BT[ROW][a] d[a][b]
// over the 3 or 4 input rows row ROW of BT uses, for the 5 columns its points
// use, then V[j] = sum_b BT[j][b] t[b].  U goes straight to registers, one
// chunk ahead (3 x 16 bytes per lane).  The pipeline runs on across unit
// boundaries as in k_wino23p (k_wino.hip), whose wait-count argument holds
// here unchanged: a wait that leaves n loads in flight proves every older
// load landed (loads complete in issue order; the inline-asm stores only make
// waits longer).
//
// LDS: X [row 10][plane = col % 4][kk = col / 4, 17][2 quads], the quad at
// slot q ^ ((kk >> 3) & 1), so 16 lanes of one tile row reading one (row,
// column) hit 64 distinct banks; three buffers (66 KB), the epilogue area
// (60 KB) and the bias (one workgroup per CU).
//
// Epilogue, per output column c of the tiles (4 rounds): wave (ROW, HALF)
// writes P = sum_j AT[c][j] M[ROW][j] over its 3 points into LDS; after a
// barrier 256 threads form S_i = P(i,0) + P(i,1) and Y[r][c] = sum_i AT[r][i]
// S_i for one tile and 4 channels, add the bias, apply the activation and
// store 16-byte quads.
#include "rt.hpp"

namespace acfun {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

__host__ __device__ constexpr int bt43(int i, int j) {
    constexpr int t[6][6] = {{4, 0, -5, 0, 1, 0},  {0, -4, -4, 1, 1, 0}, {0, 4, -4, -1, 1, 0},
                             {0, -2, -1, 2, 1, 0}, {0, 2, -1, -2, 1, 0}, {0, 4, 0, -5, 0, 1}};
    return t[i][j];
}
__host__ __device__ constexpr int at43(int i, int j) {
    constexpr int t[4][6] = {{1, 1, 1, 1, 1, 0}, {0, 1, -1, 2, -2, 0}, {0, 1, 1, 4, 4, 0},
                             {0, 1, -1, 8, -8, 1}};
    return t[i][j];
}

struct W43 {
    static constexpr int TC = 16, R = 2;               // unit: R x TC tiles
    static constexpr int NR = 4 * R + 2;               // staged pixel rows (10)
    static constexpr int NC = 4 * TC + 2;              // staged pixel columns (66)
    static constexpr int KK = TC + 1;                  // kk per plane (col = 4 kk + plane)
    static constexpr int SLOTS = NR * 4 * KK * 2;      // 16-byte slots (1360)
    static constexpr int XBLK = (SLOTS + 63) / 64;     // 64-slot DMA blocks (22)
    static constexpr int XFL = XBLK * 256;             // floats per X buffer
    static constexpr int ROWF = 4 * KK * 8;            // floats per staged row
    static constexpr int NW = 12;                      // waves
    static constexpr int EPI = 18 * 32 * 32;           // epilogue floats: 18 planes of 32 x 32
    static constexpr int MAXC = 4096;                  // Cout staged for the bias
    template <int WAVE>                                // X blocks wave WAVE issues per chunk
    static constexpr int nxw() { return (XBLK > WAVE ? 1 : 0) + (XBLK > WAVE + NW ? 1 : 0); }
    static constexpr __device__ int swz(int kk) { return (kk >> 3) & 1; }
};
static_assert(W43::XBLK <= 2 * W43::NW, "two DMA blocks per wave at most");

// s_waitcnt vmcnt(n) for a wave-uniform n in 0..8 (the count is an immediate)
__device__ __forceinline__ void wait_vm(int n) {
    switch (n) {
        case 0: __builtin_amdgcn_s_waitcnt(0x0F70); break;
        case 1: __builtin_amdgcn_s_waitcnt(0x0F71); break;
        case 2: __builtin_amdgcn_s_waitcnt(0x0F72); break;
        case 3: __builtin_amdgcn_s_waitcnt(0x0F73); break;
        case 4: __builtin_amdgcn_s_waitcnt(0x0F74); break;
        case 5: __builtin_amdgcn_s_waitcnt(0x0F75); break;
        case 6: __builtin_amdgcn_s_waitcnt(0x0F76); break;
        case 7: __builtin_amdgcn_s_waitcnt(0x0F77); break;
        default: __builtin_amdgcn_s_waitcnt(0x0F78); break;
    }
}

// acc + C * x and C * x for a compile-time integer C (+-1 without a multiply)
__device__ __forceinline__ float fmac(float c, float x, float a) { return fmaf(c, x, a); }
__device__ __forceinline__ f4 fmac(float c, f4 x, f4 a) {
    return f4{fmaf(c, x[0], a[0]), fmaf(c, x[1], a[1]), fmaf(c, x[2], a[2]), fmaf(c, x[3], a[3])};
}
template <int C, typename T>
__device__ __forceinline__ T axpy(T acc, T x) {
    if constexpr (C == 1) return acc + x;
    else if constexpr (C == -1) return acc - x;
    else return fmac((float)C, x, acc);
}
template <int C, typename T>
__device__ __forceinline__ T scale(T x) {
    if constexpr (C == 1) return x;
    else if constexpr (C == -1) return -x;
    else return x * (float)C;
}
__device__ __forceinline__ f4 fma4(float c, f4 x, f4 a) { return fmac(c, x, a); }
// Row ROW of BT applied to the 6 values d[0..5] (only the ones the row uses
// are read), factored as
//   t0 = 4 d0 - 5 d2 + d4          t1 = -4 (d1 + d2) + (d3 + d4)
//   t2 = 4 (d1 - d2) + (d4 - d3)   t3 = -2 (d1 - d3) + (d4 - d2)
//   t4 = 2 (d1 - d3) + (d4 - d2)   t5 = 4 d1 - 5 d3 + d5
template <int ROW>
__device__ __forceinline__ f4 bt_row(const f4* d) {
    if constexpr (ROW == 0) return fma4(4.f, d[0], fma4(-5.f, d[2], d[4]));
    else if constexpr (ROW == 1) return fma4(-4.f, d[1] + d[2], d[3] + d[4]);
    else if constexpr (ROW == 2) return fma4(4.f, d[1] - d[2], d[4] - d[3]);
    else if constexpr (ROW == 3) return fma4(-2.f, d[1] - d[3], d[4] - d[2]);
    else if constexpr (ROW == 4) return fma4(2.f, d[1] - d[3], d[4] - d[2]);
    else return fma4(4.f, d[1], fma4(-5.f, d[3], d[5]));
}
// Coefficient rows: c(i) for i = 0..N-1
template <int I> struct BTRow { static constexpr int c(int a) { return bt43(I, a); } };
template <int J, int B0> struct BTCol { static constexpr int c(int b) { return bt43(J, b + B0); } };
template <int R> struct ATRow { static constexpr int c(int i) { return at43(R, i); } };
template <int CC, int J0> struct ATPart { static constexpr int c(int k) { return at43(CC, J0 + k); } };
template <typename CF, int N> constexpr int first_nz() {
    for (int i = 0; i < N; ++i)
        if (CF::c(i) != 0) return i;
    return -1;
}
template <typename CF, int I, int N, typename T>
__device__ __forceinline__ void comb_rest(T& acc, const T* v) {
    if constexpr (I < N) {
        constexpr int c = CF::c(I);
        if constexpr (c != 0) acc = axpy<c>(acc, v[I]);
        comb_rest<CF, I + 1, N>(acc, v);
    }
}
// sum_i CF::c(i) v[i] over the nonzero coefficients, in index order
template <typename CF, int N, typename T>
__device__ __forceinline__ T combine(const T* v) {
    constexpr int f = first_nz<CF, N>();
    static_assert(f >= 0, "an all-zero coefficient row");
    T acc = scale<CF::c(f)>(v[f]);
    comb_rest<CF, f + 1, N>(acc, v);
    return acc;
}

template <int ACT>
__global__ __launch_bounds__(768, 1) void k_wino43p(
    const float* __restrict__ in, const float* __restrict__ U, const float* __restrict__ bias,
    float* __restrict__ out, int H, int W, int Cin, int Cinp, int Cout, int rblocks, int gx, int gz,
    int nunits, int in_bytes, int u_bytes) {
    using CF = W43;
    constexpr unsigned kOOB = 0x80000000u;
    extern __shared__ __attribute__((aligned(16))) float smem[];
    float* const epi = smem + 3 * CF::XFL;
    float* const bsm = epi + CF::EPI;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 31, g = lane >> 5;
    const int m = Cinp / 8;                            // chunks per unit (even, >= 4)

    const int nwx = (int)(gridDim.x / 8);
    const int xcd = (int)(blockIdx.x % 8), i0 = (int)(blockIdx.x / 8);
    const int rs = (int)((long long)xcd * nunits / 8), re = (int)((long long)(xcd + 1) * nunits / 8);
    const int nu = rs + i0 < re ? (re - rs - i0 + nwx - 1) / nwx : 0;
    if (nu == 0) return;                               // uniform per workgroup

    for (int c = tid; c < (Cout + 3) / 4 * 4; c += 768) bsm[c] = bias && c < Cout ? bias[c] : 0.f;
    const int etile = (tid & 255) >> 3, ecq = 4 * (tid & 7);   // epilogue (tid < 512): tile x 4 channels
    const bool Cout4 = (Cout & 3) == 0;

    const __amdgpu_buffer_rsrc_t ures =
        __builtin_amdgcn_make_buffer_rsrc((void*)U, (short)0, u_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t xres =
        __builtin_amdgcn_make_buffer_rsrc((void*)in, (short)0, in_bytes, 0x00020000);
    const bool ragged = (Cin & 7) != 0;

    // X read offsets (floats, buffer 0, input row 0 of the tile): tile li =
    // (sr, stx), column b of its 6x6 patch is plane b % 4 at kk = stx + b / 4
    const int sr = li >> 4, stx = li & 15;
    int xo[6];
#pragma unroll
    for (int b = 0; b < 6; ++b) {
        const int kk = stx + (b >> 2), p = b & 3;
        xo[b] = (((4 * sr * 4 + p) * CF::KK + kk) * 2 + (g ^ CF::swz(kk))) * 4;
    }
    // DMA slots of this lane: block wave + 12 k, slot (wave + 12 k) * 64 + lane
    // -> staged pixel (row, col) and channel quad q; xlo: byte offset from the
    // window origin, the same for every unit
    struct Slot { int r, col, q; bool ok; };
    auto slot = [&](int k) {
        const int sl = (wave + CF::NW * k) * 64 + lane;
        const int qs = sl & 1, s1 = sl >> 1;
        const int kk = s1 % CF::KK, rp = s1 / CF::KK;
        const int col = 4 * kk + (rp & 3);
        return Slot{rp >> 2, col, qs ^ CF::swz(kk), sl < CF::SLOTS && col < CF::NC};
    };
    unsigned xlo[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const Slot q = slot(k);
        xlo[k] = q.ok ? (unsigned)(((q.r * W + q.col) * Cin + 4 * q.q) * 4) : 0u;
    }
    // unit u: cob (first output channel), px (window origin pixel (4 ty0 - 1,
    // 4 tx0 - 1) of image n, negative at the first image's top left), rl / cl
    // (pixel rows / columns from the unit's first output row / column to the
    // image's edge)
    struct UnitP { int px, rl, cl, cob; };
    auto decode = [&](int k) {
        const int u = rs + i0 + k * nwx;
        const int bz = u % gz, sp = u / gz;
        const int bx = sp % gx, by = sp / gx;
        const int n = by / rblocks;
        const int ty0 = (by - n * rblocks) * CF::R, tx0 = bx * CF::TC;
        return UnitP{(n * H + 4 * ty0 - 1) * W + 4 * tx0 - 1, H - 4 * ty0, W - 4 * tx0, bz * 32};
    };
    // in-image bits of the lane's two slots for unit P
    auto inimg = [&](const UnitP& P, bool live) {
        unsigned b = 0;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const Slot q = slot(k);
            const bool ok = live && q.ok && q.r >= (P.rl < H ? 0 : 1) && q.r <= P.rl &&
                            q.col >= (P.cl < W ? 0 : 1) && q.col <= P.cl;
            b |= (unsigned)ok << k;
        }
        return b;
    };

    f16v acc[3];
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[a][e] = 0.f;

    auto run = [&](auto wavec) {
        constexpr int WAVE = decltype(wavec)::value;
        constexpr int ROW = WAVE >> 1, HALF = WAVE & 1;
        constexpr int NXW = CF::template nxw<WAVE>();
        constexpr int B0 = HALF ? 1 : 0;               // first of the 5 patch columns used

        // U(j) of unit P for this wave's 3 points (zeros when !live)
        auto ld_u = [&](const UnitP& P, bool live, int j, f4* ub) {
            const unsigned v = live && P.cob + li < Cout ? (unsigned)((P.cob + li) * 32 + 16 * g) : kOOB;
#pragma unroll
            for (int k = 0; k < 3; ++k) {
                const unsigned off = (unsigned)(((live ? j : 0) * 36 + ROW * 6 + 3 * HALF + k) * Cout) * 32u;
                ub[k] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(ures, v, off, 0));
            }
        };
        auto dma_x = [&](const UnitP& P, unsigned ib, int j, float* base) {
            const int ci = 8 * j;
            const int org = P.px * Cin * 4;
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                if (WAVE + CF::NW * k >= CF::XBLK) continue;
                unsigned v = (ib >> k) & 1 ? (unsigned)org + xlo[k] : kOOB;
                if (ragged && ci + 8 > Cin && ci + 4 * slot(k).q >= Cin) v = kOOB;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xres, (lds_void*)(base + (WAVE + CF::NW * k) * 256), 16,
                                                         v, ci * 4, 0, 0);
            }
        };
        // the 3 transform points of this wave from X buffer X
        auto xform = [&](const float* X, f4* dh) {
            // column by column, the reads of column bb + 1 in flight while
            // column bb is combined (two columns of reads live at a time)
            f4 t[5], d[2][6];
            auto rd = [&](int bb, f4* dd) {
#pragma unroll
                for (int a = 0; a < 6; ++a)
                    if (bt43(ROW, a) != 0) dd[a] = *(const f4*)&X[xo[B0 + bb] + a * CF::ROWF];
            };
            rd(0, d[0]);
#pragma unroll
            for (int bb = 0; bb < 5; ++bb) {
                if (bb + 1 < 5) rd(bb + 1, d[(bb + 1) & 1]);
                __builtin_amdgcn_sched_barrier(0);
                t[bb] = bt_row<ROW>(d[bb & 1]);
            }
            // V[j] = sum_b BT[j][b] t[b] over this wave's 5 columns (t[bb] is
            // column bb + B0), sharing the sums the rows have in common
            if constexpr (HALF == 0) {
                dh[0] = fma4(4.f, t[0], fma4(-5.f, t[2], t[4]));
                dh[1] = fma4(-4.f, t[1] + t[2], t[3] + t[4]);
                dh[2] = fma4(4.f, t[1] - t[2], t[4] - t[3]);
            } else {
                const f4 p = t[0] - t[2], q = t[3] - t[1];          // t1 - t3, t4 - t2
                dh[0] = fma4(-2.f, p, q);
                dh[1] = fma4(2.f, p, q);
                dh[2] = fma4(4.f, t[0], fma4(-5.f, t[2], t[4]));   // 4 t1 - 5 t3 + t5
            }
        };
        auto mfma_pt = [&](int a, const f4& d, const f4& bb) {
#pragma unroll
            for (int s2 = 0; s2 < 4; ++s2)
                acc[a] = __builtin_amdgcn_mfma_f32_32x32x2f32(d[s2], bb[s2], acc[a], 0, 0, 0);
        };

        UnitP cur = decode(0), nxt = decode(nu > 1 ? 1 : 0);
        bool nlive = nu > 1;
        unsigned ib = inimg(cur, true) | (inimg(nxt, nlive) << 2);

        // prologue: U(0), X(0), X(1), X(2) of the first unit; wait for U(0)
        // and X(0) (and the bias staging, by the barrier's lgkmcnt)
        f4 uA[3], uB[3];
        ld_u(cur, true, 0, uA);
        dma_x(cur, ib, 0, smem);
        dma_x(cur, ib, 1, smem + CF::XFL);
        dma_x(cur, ib, 2, smem + 2 * CF::XFL);
        wait_vm(2 * NXW);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        f4 dh[3];
        xform(smem, dh);
        int xb = 0;

        // chunk j: MFMAs of V(j) (dh, transformed during chunk j - 1) with
        // U(j) (bf); U(j + 1) into un; then the transform of X(j + 1) into dh
        auto chunk = [&](int j, const f4* bf, f4* un, bool wait) {
            if (wait) wait_vm(NXW);                    // U(j), X(j+1) have landed
            {
                const bool in_cur = j + 1 < m;
                ld_u(in_cur ? cur : nxt, in_cur || nlive, in_cur ? j + 1 : 0, un);
            }
            mfma_pt(0, dh[0], bf[0]);
            mfma_pt(1, dh[1], bf[1]);
            const int xb1 = xb == 2 ? 0 : xb + 1;
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            {                                          // X(j+3) into X(j)'s buffer
                const bool in_cur = j + 3 < m;
                dma_x(in_cur ? cur : nxt, in_cur ? ib : ib >> 2, in_cur ? j + 3 : j + 3 - m,
                      smem + xb * CF::XFL);
            }
            mfma_pt(2, dh[2], bf[2]);
            xform(smem + xb1 * CF::XFL, dh);
            xb = xb1;
        };

        for (int k = 0; k < nu; ++k) {
            for (int j = 0; j < m; j += 2) {
                chunk(j, uA, uB, j != 0 || k == 0);
                chunk(j + 1, uB, uA, true);
            }
            // ---- epilogue of unit cur (the next unit's U(0) and X(1) have
            // landed after this wait; its X(2) may still be in flight)
            wait_vm(NXW);
            const int ec = cur.cob + ecq;
            const f4 bq = *(const f4*)&bsm[ec < Cout ? ec : 0];
            const int esr = etile >> 4, estx = etile & 15;
            const int erl = cur.rl - 4 * esr, ecl = cur.cl - 4 * estx;   // rows / cols left
            const int epx = cur.px + (4 * esr + 1) * W + 4 * estx + 1;
            float* const orow = out + (long long)(erl > 0 && ecl > 0 ? epx : 0) * Cout + ec;
#pragma unroll
            for (int rd = 0; rd < 2; ++rd) {
                // planes [row i][3] of 32 tiles x 32 channels: pass 0 (output
                // columns 0, 2) A = M0+M1+M2, B = M1+M2 (half 0), B' = M3+M4
                // (half 1); pass 1 (columns 1, 3) C = M1-M2 (half 0),
                // C' = M3-M4, D' = M5 (half 1).  Then column 0: S = A + B',
                // 2: S = B + 4 B', 1: S = C + 2 C', 3: S = C + 8 C' + D'.
                {
                    float* const pl = epi + (3 * ROW) * 1024 + (4 * g) * 32 + li;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int o = (8 * (r >> 2) + (r & 3)) * 32;
                        const float m0 = acc[0][r], m1 = acc[1][r], m2 = acc[2][r];
                        if constexpr (HALF == 0) {
                            if (rd == 0) {
                                const float s12 = m1 + m2;
                                pl[o] = m0 + s12;
                                pl[1024 + o] = s12;
                            } else {
                                pl[o] = m1 - m2;
                            }
                        } else {
                            if (rd == 0) {
                                pl[2048 + o] = m0 + m1;
                            } else {
                                pl[1024 + o] = m0 - m1;
                                pl[2048 + o] = m2;
                            }
                        }
                    }
                }
                asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
                if (WAVE < 8) {
                    constexpr int cs = WAVE >> 2;          // 0: column rd, 1: column rd + 2
                    const int cc = rd + 2 * cs;
                    f4 S[6];
#pragma unroll
                    for (int i = 0; i < 6; ++i) {
                        const float* q = epi + (3 * i) * 1024 + etile * 32 + ecq;
                        if (rd == 0) {
                            if constexpr (cs == 0) S[i] = *(const f4*)q + *(const f4*)(q + 2048);
                            else S[i] = fma4(4.f, *(const f4*)(q + 2048), *(const f4*)(q + 1024));
                        } else {
                            if constexpr (cs == 0) S[i] = fma4(2.f, *(const f4*)(q + 1024), *(const f4*)q);
                            else S[i] = fma4(8.f, *(const f4*)(q + 1024), *(const f4*)q) + *(const f4*)(q + 2048);
                        }
                    }
                    if (ec < Cout && cc < ecl) {
                        const f4 s12 = S[1] + S[2], d12 = S[1] - S[2], s34 = S[3] + S[4], d34 = S[3] - S[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            if (r >= erl) continue;
                            f4 v;
                            if (r == 0) v = S[0] + s12 + s34;
                            else if (r == 1) v = fma4(2.f, d34, d12);
                            else if (r == 2) v = fma4(4.f, s34, s12);
                            else v = fma4(8.f, d34, d12) + S[5];
                            v = v + bq;
#pragma unroll
                            for (int e = 0; e < 4; ++e) v[e] = act_apply(v[e], ACT);
                            float* dst = orow + ((long long)r * W + cc) * Cout;
                            if (Cout4) {
                                // s_nop: a VALU write to the data registers of a
                                // store of more than 8 bytes needs a wait state
                                // after it, which the compiler cannot insert after
                                // inline asm
                                asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1" ::"v"(dst), "v"(v)
                                             : "memory");
                            } else {
#pragma unroll
                                for (int e = 0; e < 4; ++e)
                                    if (ec + e < Cout)
                                        asm volatile("global_store_dword %0, %1, off sc1" ::"v"(dst + e), "v"(v[e])
                                                     : "memory");
                            }
                        }
                    }
                }
                // the second round's writes must not overtake these reads
                if (rd == 0) asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            }
#pragma unroll
            for (int a = 0; a < 3; ++a)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[a][e] = 0.f;
            cur = nxt;
            nlive = k + 2 < nu;
            nxt = decode(nlive ? k + 2 : k + 1);
            ib = (ib >> 2) | (inimg(nxt, nlive) << 2);
        }
        wait_vm(0);                                    // out-of-range loads and stores done
    };
    switch (wave) {
        case 0: run(std::integral_constant<int, 0>{}); break;
        case 1: run(std::integral_constant<int, 1>{}); break;
        case 2: run(std::integral_constant<int, 2>{}); break;
        case 3: run(std::integral_constant<int, 3>{}); break;
        case 4: run(std::integral_constant<int, 4>{}); break;
        case 5: run(std::integral_constant<int, 5>{}); break;
        case 6: run(std::integral_constant<int, 6>{}); break;
        case 7: run(std::integral_constant<int, 7>{}); break;
        case 8: run(std::integral_constant<int, 8>{}); break;
        case 9: run(std::integral_constant<int, 9>{}); break;
        case 10: run(std::integral_constant<int, 10>{}); break;
        default: run(std::integral_constant<int, 11>{}); break;
    }
}

size_t wino43p_lds(int Cout) {
    return ((size_t)3 * W43::XFL + W43::EPI + (size_t)(Cout + 3) / 4 * 4) * sizeof(float);
}

}  // namespace

bool run_wino43(const float* in, int N, int H, int W, int Cin, const float* w, const float* bias,
                int Cout, float* out, int act, hipStream_t s, bool* done) {
    *done = false;
    const int tH = (H + 3) / 4, tW = (W + 3) / 4;
    const int Cinp = (Cin + 15) / 16 * 16;
    const long long in_bytes = (long long)N * H * W * Cin * 4;
    const long long u_bytes = 36ll * Cout * Cinp * 4;
    if (Cin % 4 != 0 || Cinp / 8 < 4 || ((uintptr_t)in & 15u) != 0 || tW < 6 || Cout > W43::MAXC ||
        in_bytes >= (1ll << 31) || u_bytes >= (1ll << 31) || N <= 0 || Cout <= 0)
        return true;
    const int rblocks = (tH + W43::R - 1) / W43::R;
    const long long gx = (tW + W43::TC - 1) / W43::TC, gy = (long long)N * rblocks, gz = (Cout + 31) / 32;
    const long long nunits = gx * gy * gz;
    if (nunits >= (1ll << 30)) return true;
    Scratch Us((size_t)u_bytes, s);
    if (!Us.p) return false;
    if (!wino43_filter(w, Cin, Cout, Us.as<float>(), s)) return false;
    const size_t lds = wino43p_lds(Cout);
    // set once per process, thread-safely, before any launch below
    static const bool attr = [&] {
        (void)hipFuncSetAttribute((const void*)k_wino43p<0>, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        (void)hipFuncSetAttribute((const void*)k_wino43p<1>, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        (void)hipFuncSetAttribute((const void*)k_wino43p<2>, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        return true;
    }();
    (void)attr;
    const long long slots = num_cus() / 8, need = (nunits + 7) / 8;
    const unsigned grid = (unsigned)(8 * (slots < need ? slots : need));
    const float* Up = Us.as<float>();
    if (act == 1)
        ACFUN_LAUNCH("k_wino43", (k_wino43p<1>), dim3(grid), dim3(768), lds, s, in, Up, bias, out, H, W,
                     Cin, Cinp, Cout, rblocks, (int)gx, (int)gz, (int)nunits, (int)in_bytes, (int)u_bytes);
    else if (act == 2)
        ACFUN_LAUNCH("k_wino43", (k_wino43p<2>), dim3(grid), dim3(768), lds, s, in, Up, bias, out, H, W,
                     Cin, Cinp, Cout, rblocks, (int)gx, (int)gz, (int)nunits, (int)in_bytes, (int)u_bytes);
    else
        ACFUN_LAUNCH("k_wino43", (k_wino43p<0>), dim3(grid), dim3(768), lds, s, in, Up, bias, out, H, W,
                     Cin, Cinp, Cout, rblocks, (int)gx, (int)gz, (int)nunits, (int)in_bytes, (int)u_bytes);
    if (!check_launch("k_wino43p")) return false;
    *done = true;
    return true;
}

}  // namespace acfun
