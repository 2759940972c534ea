// k_wino.hip -- Winograd F(2,3) and F(4,3) for 3x3 / stride 1 / pad 1 convs.
//
// Replaces acfun_winograd_conv3x3 (src/winograd.cpp:236-251,
// src/winograd_avx512.cpp:186-250) and acfun_winograd43_conv3x3
// (src/winograd43.cpp:239-250, src/winograd43_avx512.cpp:218-280).  The
// matrices are the standard Lavin & Gray ones the reference uses
// (src/winograd.cpp:9-17, src/winograd43.cpp:33-54):
//   d_hat = BT d BT^T (input tile), g_hat = G g G^T (filter), Y = AT M AT^T.
//
// Two kernels per call: the filter transform U = G g G^T (per call, like the
// reference, :195-206) and one fused kernel doing input transform, the P =
// 16 (36) transform-point GEMMs on fp32 MFMA and the output transform with
// bias and ReLU, so the input is read once and the output written once.
#include "rt.hpp"

#include <memory>

#include <type_traits>

namespace acfun {
namespace {

template <int TILE> struct Wino;

template <> struct Wino<2> {
    static constexpr int A = 4;  // input tile edge
    __device__ static void in_tf(const float d[4][4], float out[4][4]) {
        float U[4][4];
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            U[0][l] = d[0][l] - d[2][l];
            U[1][l] = d[1][l] + d[2][l];
            U[2][l] = d[2][l] - d[1][l];
            U[3][l] = d[3][l] - d[1][l];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            out[i][0] = U[i][0] - U[i][2];
            out[i][1] = U[i][1] + U[i][2];
            out[i][2] = U[i][2] - U[i][1];
            out[i][3] = U[i][3] - U[i][1];
        }
    }
    __device__ static void f_tf(const float g[3][3], float out[4][4]) {
        float T[4][3];
#pragma unroll
        for (int y = 0; y < 3; ++y) {
            float a = g[0][y], b = g[1][y], c = g[2][y];
            T[0][y] = a;
            T[1][y] = 0.5f * (a + b + c);
            T[2][y] = 0.5f * (a - b + c);
            T[3][y] = c;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float t0 = T[i][0], t1 = T[i][1], t2 = T[i][2];
            out[i][0] = t0;
            out[i][1] = 0.5f * (t0 + t1 + t2);
            out[i][2] = 0.5f * (t0 - t1 + t2);
            out[i][3] = t2;
        }
    }
    __device__ static void out_tf(const float m[4][4], float y[2][2]) {
        float t[2][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            t[0][j] = m[0][j] + m[1][j] + m[2][j];
            t[1][j] = m[1][j] - m[2][j] + m[3][j];
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            y[i][0] = t[i][0] + t[i][1] + t[i][2];
            y[i][1] = t[i][1] - t[i][2] + t[i][3];
        }
    }
};

__constant__ float kBT43[6][6] = {
    {4.f, 0.f, -5.f, 0.f, 1.f, 0.f},  {0.f, -4.f, -4.f, 1.f, 1.f, 0.f},
    {0.f, 4.f, -4.f, -1.f, 1.f, 0.f}, {0.f, -2.f, -1.f, 2.f, 1.f, 0.f},
    {0.f, 2.f, -1.f, -2.f, 1.f, 0.f}, {0.f, 4.f, 0.f, -5.f, 0.f, 1.f}};
__constant__ float kG43[6][3] = {{0.25f, 0.f, 0.f},
                                 {-1.f / 6.f, -1.f / 6.f, -1.f / 6.f},
                                 {-1.f / 6.f, 1.f / 6.f, -1.f / 6.f},
                                 {1.f / 24.f, 1.f / 12.f, 1.f / 6.f},
                                 {1.f / 24.f, -1.f / 12.f, 1.f / 6.f},
                                 {0.f, 0.f, 1.f}};
__constant__ float kAT43[4][6] = {{1.f, 1.f, 1.f, 1.f, 1.f, 0.f},
                                  {0.f, 1.f, -1.f, 2.f, -2.f, 0.f},
                                  {0.f, 1.f, 1.f, 4.f, 4.f, 0.f},
                                  {0.f, 1.f, -1.f, 8.f, -8.f, 1.f}};

template <> struct Wino<4> {
    static constexpr int A = 6;
    __device__ static void in_tf(const float d[6][6], float out[6][6]) {
        float t[6][6];
#pragma unroll
        for (int i = 0; i < 6; ++i)
#pragma unroll
            for (int b = 0; b < 6; ++b) {
                float s = 0.f;
#pragma unroll
                for (int a = 0; a < 6; ++a) s += kBT43[i][a] * d[a][b];
                t[i][b] = s;
            }
#pragma unroll
        for (int i = 0; i < 6; ++i)
#pragma unroll
            for (int j = 0; j < 6; ++j) {
                float s = 0.f;
#pragma unroll
                for (int b = 0; b < 6; ++b) s += t[i][b] * kBT43[j][b];
                out[i][j] = s;
            }
    }
    __device__ static void f_tf(const float g[3][3], float out[6][6]) {
        float t[6][3];
#pragma unroll
        for (int i = 0; i < 6; ++i)
#pragma unroll
            for (int y = 0; y < 3; ++y) {
                float s = 0.f;
#pragma unroll
                for (int x = 0; x < 3; ++x) s += kG43[i][x] * g[x][y];
                t[i][y] = s;
            }
#pragma unroll
        for (int i = 0; i < 6; ++i)
#pragma unroll
            for (int j = 0; j < 6; ++j) {
                float s = 0.f;
#pragma unroll
                for (int y = 0; y < 3; ++y) s += t[i][y] * kG43[j][y];
                out[i][j] = s;
            }
    }
    __device__ static void out_tf(const float m[6][6], float y[4][4]) {
        float t[4][6];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int j = 0; j < 6; ++j) {
                float s = 0.f;
#pragma unroll
                for (int i = 0; i < 6; ++i) s += kAT43[r][i] * m[i][j];
                t[r][j] = s;
            }
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                float s = 0.f;
#pragma unroll
                for (int j = 0; j < 6; ++j) s += t[r][j] * kAT43[c][j];
                y[r][c] = s;
            }
    }
};

// Filter transform into the fused kernel's layout U[a][Cout][Cinp]: for each
// transform point a and output channel o, the Cinp (= Cin rounded up to 16)
// input channels are contiguous and zero-padded, so one lane fetches four
// k-steps of an MFMA B operand with a single 16-byte load.
template <int TILE>
__global__ void k_wino_filter_t(const float* __restrict__ w, int Cin, int Cinp, int Cout,
                                float* __restrict__ U) {
    constexpr int A = Wino<TILE>::A;
    int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= Cinp * Cout) return;
    int o = idx / Cinp, c = idx - o * Cinp;
    float gh[A][A];
    if (c < Cin) {
        float g[3][3];
#pragma unroll
        for (int kh = 0; kh < 3; ++kh)
#pragma unroll
            for (int kw = 0; kw < 3; ++kw) g[kh][kw] = w[((long long)(kh * 3 + kw) * Cin + c) * Cout + o];
        Wino<TILE>::f_tf(g, gh);
    } else {
#pragma unroll
        for (int i = 0; i < A; ++i)
#pragma unroll
            for (int j = 0; j < A; ++j) gh[i][j] = 0.f;
    }
    long long plane = (long long)Cout * Cinp;
#pragma unroll
    for (int i = 0; i < A; ++i)
#pragma unroll
        for (int j = 0; j < A; ++j) U[(i * A + j) * plane + idx] = gh[i][j];
}

// Filter transform as a tiled transpose: a 256-lane block owns 16 output x 16
// input channels.  Lane (o = l%16, c = l/16) reads its 9 taps with output
// channels fastest (64-byte runs of w), transforms them, and the block writes
// through LDS with input channels fastest: U[a][Cout][Cinp] (64-byte runs).
template <int TILE>
__global__ __launch_bounds__(256) void k_wino_filter_tt(const float* __restrict__ w, int Cin,
                                                         int Cinp, int Cout, float* __restrict__ U) {
    constexpr int A = Wino<TILE>::A, AA = A * A;
    __shared__ float tr[AA][16][17];
    const int o0 = blockIdx.x * 16, c0 = blockIdx.y * 16;
    const int ol = threadIdx.x & 15, cl = threadIdx.x >> 4;
    const int o = o0 + ol, c = c0 + cl;
    float gh[A][A];
    if (c < Cin && o < Cout) {
        float g[3][3];
#pragma unroll
        for (int kh = 0; kh < 3; ++kh)
#pragma unroll
            for (int kw = 0; kw < 3; ++kw) g[kh][kw] = w[((long long)(kh * 3 + kw) * Cin + c) * Cout + o];
        Wino<TILE>::f_tf(g, gh);
    } else {
#pragma unroll
        for (int i = 0; i < A; ++i)
#pragma unroll
            for (int j = 0; j < A; ++j) gh[i][j] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < A; ++i)
#pragma unroll
        for (int j = 0; j < A; ++j) tr[i * A + j][ol][cl] = gh[i][j];
    __syncthreads();
    // write: lane (c = l%16, o = l/16), c fastest
    const int wc = threadIdx.x & 15, wo = threadIdx.x >> 4;
    const long long plane = (long long)Cout * Cinp;
    if (o0 + wo < Cout && c0 + wc < Cinp) {
        const int c = c0 + wc;
#pragma unroll
        for (int a = 0; a < AA; ++a) U[a * plane + (long long)(o0 + wo) * Cinp + c] = tr[a][wo][wc];
    }
}

// The chunked layout U[Cinp/8][a][Cout][8], in which the filter slice one
// 8-channel chunk of a unit kernel needs for one point and 32 output channels
// is a single contiguous kilobyte, written directly: lane (c % 8, o)
// of a 64-thread block transforms one filter and writes its AA points, and
// the 64 lanes of one point store 8 output channels x 8 input channels, 256
// contiguous bytes, without an LDS transpose.  The arithmetic is
// k_wino_filter_tt's (the same f_tf).
template <int TILE>
__global__ __launch_bounds__(64) void k_wino_filter_c8(const float* __restrict__ w, int Cin, int Cout,
                                                      float* __restrict__ U) {
    constexpr int A = Wino<TILE>::A, AA = A * A;
    const int l = threadIdx.x;
    const int c = blockIdx.y * 8 + (l & 7), o = blockIdx.x * 8 + (l >> 3);
    if (o >= Cout) return;
    float gh[A][A];
    if (c < Cin) {
        float g[3][3];
#pragma unroll
        for (int kh = 0; kh < 3; ++kh)
#pragma unroll
            for (int kw = 0; kw < 3; ++kw) g[kh][kw] = w[((long long)(kh * 3 + kw) * Cin + c) * Cout + o];
        Wino<TILE>::f_tf(g, gh);
    } else {
#pragma unroll
        for (int i = 0; i < A; ++i)
#pragma unroll
            for (int j = 0; j < A; ++j) gh[i][j] = 0.f;
    }
    const long long base = (long long)blockIdx.y * AA * Cout * 8 + (long long)o * 8 + (l & 7);
#pragma unroll
    for (int a = 0; a < AA; ++a) U[base + (long long)a * Cout * 8] = gh[a / A][a % A];
}

typedef float f4 __attribute__((ext_vector_type(4)));

// Fused Winograd: one workgroup = TB consecutive tiles (flattened n,ty,tx
// order) x CB = 16*NW output channels; wave w owns output channels
// 16w..16w+15 of the block and every tile of it, so for each transform point
// a its accumulators hold M[a][tile][o] with lane l, register r <-> tile
// 4*(l/16)+r, channel l%16 (the 16x16 MFMA D layout).  Input channels are
// consumed in chunks of KC, software-pipelined:
//   while the MFMAs of chunk k read d_hat (sV) and the filter chunk (sU) from
//   LDS, the raw input patches and the filter slice of chunk k+1 are already
//   in flight into registers; then the patches are transformed into sV and
//   the filter slice stored into sU for the next round.
// LDS rows hold KC channels plus 4 floats of padding, so the 16 rows touched
// by one ds_read_b128 land in distinct banks; one b128 read gives a lane four
// MFMA k-steps (channel 4*(l/16)+s of the chunk, s = 0..3, for both operands).
// After the last chunk the output transform, bias and ReLU run in registers.
template <int TILE, int TB, int NW, int KC>
__global__ __launch_bounds__(64 * NW) void k_wino_fused(
    const float* __restrict__ in, const float* __restrict__ U, const float* __restrict__ bias,
    float* __restrict__ out, int N, int H, int W, int Cin, int Cinp, int Cout, int tH, int tW,
    int act) {
    constexpr int A = Wino<TILE>::A;
    constexpr int P = A * A;
    constexpr int FB = TB / 16;
    constexpr int NT = 64 * NW;
    constexpr int CB = 16 * NW;
    constexpr int LDV = KC + 4;
    constexpr int KQ = KC / 4;                        // float4 per (a, channel-row) of a chunk
    constexpr int VEC = KC / 4;                       // k-steps per LDS read (4: b128, 2: b64)
    constexpr int UV = (P * CB * KQ + NT - 1) / NT;   // filter float4 per thread per chunk
    constexpr int XV = (TB * KC + NT - 1) / NT;       // (tile, channel) patches per thread
    static_assert(KC == 8 || KC == 16, "one LDS read covers the chunk's 4 lane groups");
    __shared__ __attribute__((aligned(16))) float sV[P * TB * LDV];
    __shared__ __attribute__((aligned(16))) float sU[P * CB * LDV];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const long long T = (long long)N * tH * tW;
    const long long tile0 = (long long)blockIdx.x * TB;
    const int cob = blockIdx.y * CB;
    const long long uplane = (long long)Cout * Cinp;

    // ---- per-thread patch bookkeeping (fixed over chunks)
    const float* xbase[XV];
    int xih0[XV], xiw0[XV], xt[XV], xc[XV];
    bool xok[XV];
#pragma unroll
    for (int v = 0; v < XV; ++v) {
        int idx = tid + v * NT;
        int t = idx / KC, c = idx - (idx / KC) * KC;
        xt[v] = t;
        xc[v] = c;
        long long tile = tile0 + t;
        xok[v] = idx < TB * KC && tile < T;
        long long tl = xok[v] ? tile : 0;
        int tx = (int)(tl % tW);
        long long r = tl / tW;
        int ty = (int)(r % tH);
        int n = (int)(r / tH);
        xbase[v] = in + (long long)n * H * W * Cin + c;
        xih0[v] = ty * TILE - 1;
        xiw0[v] = tx * TILE - 1;
    }
    float xr[XV][A][A];
    f4 ur[UV];

    auto load_chunk = [&](int c0) {
#pragma unroll
        for (int v = 0; v < XV; ++v) {
            bool ok = xok[v] && (c0 + xc[v]) < Cin;
#pragma unroll
            for (int i = 0; i < A; ++i)
#pragma unroll
                for (int j = 0; j < A; ++j) {
                    int ih = xih0[v] + i, iw = xiw0[v] + j;
                    xr[v][i][j] = (ok && ih >= 0 && ih < H && iw >= 0 && iw < W)
                                      ? xbase[v][((long long)ih * W + iw) * Cin + c0] : 0.f;
                }
        }
#pragma unroll
        for (int u = 0; u < UV; ++u) {
            int idx = tid + u * NT;                    // (a, co, q) with q fastest
            int q = idx % KQ;
            int row = idx / KQ;                        // a*CB + co_local
            int a = row / CB, col = row - a * CB;
            f4 val = {0.f, 0.f, 0.f, 0.f};
            if (idx < P * CB * KQ && cob + col < Cout)
                val = *(const f4*)(U + a * uplane + (long long)(cob + col) * Cinp + c0 + q * 4);
            ur[u] = val;
        }
    };
    auto store_chunk = [&]() {
#pragma unroll
        for (int v = 0; v < XV; ++v) {
            if (tid + v * NT >= TB * KC) continue;
            float dh[A][A];
            Wino<TILE>::in_tf(xr[v], dh);
#pragma unroll
            for (int i = 0; i < A; ++i)
#pragma unroll
                for (int j = 0; j < A; ++j) sV[((i * A + j) * TB + xt[v]) * LDV + xc[v]] = dh[i][j];
        }
#pragma unroll
        for (int u = 0; u < UV; ++u) {
            int idx = tid + u * NT;
            if (idx >= P * CB * KQ) continue;
            int q = idx % KQ;
            int row = idx / KQ;
            *(f4*)&sU[row * LDV + q * 4] = ur[u];
        }
    };

    f4 acc[P][FB];
#pragma unroll
    for (int a = 0; a < P; ++a)
#pragma unroll
        for (int b = 0; b < FB; ++b) acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};

    const int lr = lane & 15, lg = lane >> 4;
    load_chunk(0);
    for (int c0 = 0; c0 < Cinp; c0 += KC) {
        __syncthreads();          // previous chunk's MFMAs are done with sV / sU
        store_chunk();
        if (c0 + KC < Cinp) load_chunk(c0 + KC);   // in flight during the MFMAs below
        __syncthreads();
        // lane group g = l/16 supplies channel VEC*g + s to MFMA step s
#pragma unroll
        for (int a = 0; a < P; ++a) {
            typedef float fv __attribute__((ext_vector_type(VEC)));
            fv bfr = *(const fv*)&sU[(a * CB + wave * 16 + lr) * LDV + lg * VEC];
#pragma unroll
            for (int b = 0; b < FB; ++b) {
                fv afr = *(const fv*)&sV[(a * TB + b * 16 + lr) * LDV + lg * VEC];
#pragma unroll
                for (int s = 0; s < VEC; ++s)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(afr[s], bfr[s], acc[a][b], 0, 0, 0);
            }
        }
    }

    // ---- output transform + bias + ReLU in registers
    const int co = cob + wave * 16 + lr;
    if (co >= Cout) return;
    const float bv = bias ? bias[co] : 0.f;
#pragma unroll
    for (int b = 0; b < FB; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            long long tile = tile0 + b * 16 + (lane >> 4) * 4 + r;
            if (tile >= T) continue;
            int tx = (int)(tile % tW);
            long long q = tile / tW;
            int ty = (int)(q % tH);
            int n = (int)(q / tH);
            float m[A][A];
#pragma unroll
            for (int i = 0; i < A; ++i)
#pragma unroll
                for (int j = 0; j < A; ++j) m[i][j] = acc[i * A + j][b][r];
            float y[TILE][TILE];
            Wino<TILE>::out_tf(m, y);
#pragma unroll
            for (int i = 0; i < TILE; ++i)
#pragma unroll
                for (int j = 0; j < TILE; ++j) {
                    int oh = ty * TILE + i, ow = tx * TILE + j;
                    if (oh < H && ow < W) {
                        float v = y[i][j] + bv;
                        v = act_apply(v, act);
                        out[(((long long)n * H + oh) * W + ow) * Cout + co] = v;
                    }
                }
        }
}

typedef float f16v __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

// F(2,3) on v_mfma_f32_32x32x2f32, input and filter staged by LDS DMA.
//
// Workgroup (512 threads) = one image's tile rows ty0..ty0+R-1 x tile
// columns tx0..tx0+TC-1 (R*TC <= 128 tile slots) x 32 output channels.
// Waves 2p and 2p+1 form pair p, owning tile slots 32p..32p+31; wave 2p+h
// keeps the accumulators of the 8 transform points in rows i = 2h, 2h+1 of
// the 4x4 transform grid (8 x 16 AGPRs), so two waves share each SIMD and one
// wave's MFMAs overlap the other's LDS reads and transforms.
//
// Input channels are consumed in chunks of 16.  Per chunk the workgroup DMAs
// (buffer_load_dwordx4 ... lds, no data VGPRs) into one of two LDS buffers:
//   X: the 2R+2 pixel rows x 2TC+2 columns the block's 4x4 patches touch,
//      as [row][col%2][col/2][4 channel quads], quad q of pixel column index
//      k stored at quad slot q ^ ((k>>2)&3);
//   U: the filter chunk [16 points][32 channels][4 quads], quad q of channel
//      row co stored at slot q ^ ((co>>2)&3).
// The XOR swizzles keep DMA destinations contiguous while the 16 rows read
// by a ds_read_b128 lane group fall on distinct banks.  Chunk k+1's DMAs are
// issued between chunk k's MFMAs and fly while it is computed.  Per 8-channel
// half, lane l reads the pixel rows of its tile's 4x4 patch that its
// transform rows need (channel quad 4*(l/32)), applies BT per column, and
// each row of d_hat feeds its 4 points x 4 k-steps (k-step s <-> channel
// 4*(l/32)+s, as in the B operand).
// Epilogue: the output transform is linear, so each wave forms the partial
// 2x2 outputs of its 8 points into one of two LDS output tiles; all threads
// then sum the tiles, add bias, apply ReLU and store 16-byte channel quads.
__global__ __launch_bounds__(512) void k_wino23(
    const float* __restrict__ in, const float* __restrict__ U, const float* __restrict__ bias,
    float* __restrict__ out, int N, int H, int W, int Cin, int Cinp, int Cout, int tH, int tW,
    int R, int TC, int act) {
    constexpr int KC = 16;
    constexpr int NT = 512;
    extern __shared__ __attribute__((aligned(16))) float smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: scalar branches
    const int pair = wave >> 1, hr = wave & 1;
    const int g = lane >> 5, li = lane & 31;
    const int TCP = TC + 1;
    const int nrow = 2 * R + 2;
    // X region rounded up to whole 64-slot DMA blocks: the last block's lanes
    // past the region land in this padding, never in the U region.
    const int xfl = (nrow * 2 * TCP * 4 + 63) / 64 * 64 * 4;
    const int bufsz = xfl + 16 * 32 * 16;                // X + U floats per buffer
    const int rblocks = (tH + R - 1) / R;
    const int n = blockIdx.y / rblocks;
    const int ty0 = (blockIdx.y - n * rblocks) * R;
    const int tx0 = blockIdx.x * TC;
    const int cob = blockIdx.z * 32;
    const long long uplane = (long long)Cout * Cinp;
    const float* __restrict__ img = in + (long long)n * H * W * Cin;

    f16v acc[8];                                         // points 8*hr .. 8*hr+7
#pragma unroll
    for (int a = 0; a < 8; ++a)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[a][e] = 0.f;

    // ---- DMA descriptors.  Sources are read through buffer resources, so a
    // byte offset past the resource's size (kOOB) reads zeros: padding pixels
    // and missing output channels cost no branch or select, and the chunk's
    // channel offset rides in the scalar offset.  Wave w issues X blocks w,
    // w+8, ... (64 slots of 16 bytes); lane l of block k covers slot 64k+l,
    // pixel index pix = (row*2 + plane)*TCP + kk = pix0 + 128k.  The byte
    // offsets of this lane's KXM X slots are computed once; xq packs their
    // channel quads (2 bits each) for a last chunk that ends inside a quad
    // row (Cin % 16 != 0).  Filter block t of a wave sits 4t points (4 *
    // Cout * Cinp floats) after block 0, a uniform step.
    constexpr int KXM = 9;
    constexpr unsigned kOOB = 0x80000000u;
    const int xslots = nrow * 2 * TCP * 4;
    const int nxb = (xslots + 63) / 64;                   // X blocks per chunk
    unsigned xv[KXM];
    unsigned xq = 0;
    {
        const int pix0 = (wave * 64 + lane) >> 2;         // < 128: float quotient is exact
        int rp = (int)(((float)pix0 + 0.5f) / (float)TCP), kk = pix0 - rp * TCP;
        const int dk = 128 % TCP, dr = 128 / TCP;
        const int ih0 = 2 * ty0 - 1, iw0 = 2 * tx0 - 1;
#pragma unroll
        for (int k = 0; k < KXM; ++k) {
            int q = (lane & 3) ^ ((kk >> 2) & 3);
            int ih = ih0 + (rp >> 1);
            int iw = iw0 + 2 * kk + (rp & 1);
            bool ok = rp < 2 * nrow && (unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W;
            xv[k] = ok ? (unsigned)((ih * W + iw) * Cin + 4 * q) * 4u : kOOB;
            xq |= (unsigned)q << (2 * k);
            kk += dk;
            rp += dr;
            if (kk >= TCP) { kk -= TCP; ++rp; }
        }
    }
    unsigned uv;
    {
        int row = (wave * 64 + lane) >> 2;                // a*32 + co, a < 4
        int co = row & 31;
        int q = (lane & 3) ^ ((co >> 2) & 3);
        uv = cob + co < Cout ? (unsigned)((row >> 5) * Cout * Cinp + (cob + co) * Cinp + 4 * q) * 4u
                             : kOOB;
    }
    const unsigned ustep = 16u * Cout * Cinp;             // bytes per 4 points
    const __amdgpu_buffer_rsrc_t xres =
        __builtin_amdgcn_make_buffer_rsrc((void*)img, (short)0, H * W * Cin * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t ures =
        __builtin_amdgcn_make_buffer_rsrc((void*)U, (short)0, (int)(16 * uplane * 4), 0x00020000);
    const bool ragged = (Cin & 15) != 0;
    // DMA item t of a chunk: t < KU are this wave's filter blocks (the 16 x
    // 32 x 4 quads of a chunk are 32 blocks, KU = 4 per wave), t >= KU its X
    // block t-KU.
    constexpr int KU = 16 * 32 * 4 / NT;
    constexpr int NITEM = KU + KXM;
    static_assert(NITEM <= 16, "DMA items are issued after the 16 MFMA groups of a chunk");
    auto dma_item = [&](int t, int c0, float* base) {
        if (t < KU) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ures, (lds_void*)(base + xfl + (wave + 8 * t) * 256),
                                                     16, uv, c0 * 4 + t * ustep, 0, 0);
            return;
        }
        const int k = t - KU;
        const int blk = wave + 8 * k;
        if (blk >= nxb) return;
        unsigned v = xv[k];
        if (ragged && c0 + 16 > Cin && c0 + 4 * (int)((xq >> (2 * k)) & 3) >= Cin) v = kOOB;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xres, (lds_void*)(base + blk * 256), 16, v, c0 * 4, 0, 0);
    };

    // first chunk's DMA goes out before the remaining setup
#pragma unroll
    for (int t = 0; t < NITEM; ++t) dma_item(t, 0, smem);

    // this lane's MFMA row (tile slot); slot < 128, so the float quotient
    // (slot + 0.5) / TC sits at least 1/128 from an integer
    const int slot = pair * 32 + li;
    const int sr = (int)(((float)slot + 0.5f) / (float)TC), stx = slot - sr * TC;
    const int srr = sr < R ? sr : 0;
    const int usw = (li >> 2) & 3;                        // U swizzle of row li
    const int rA = 2 * hr, rB = 2 - hr, rC = 1 + 2 * hr;
    const unsigned smask = (unsigned)hr << 31;            // sign flip of dB for hr = 1

    // Compute chunk buffer b; when c0n >= 0 also issue the DMA items of the
    // next chunk (channels c0n.., buffer bn), one after each group of 4 MFMAs,
    // so the address traffic is spread over the chunk instead of stalling all
    // waves after the barrier.
    auto compute = [&](int b, int c0n, int bn) {
        const float* X = smem + b * bufsz;
        float* nbase = smem + bn * bufsz;
        const float* Ub = X + xfl;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int q = 2 * h + g;
            f4 bf[8];
#pragma unroll
            for (int a = 0; a < 8; ++a)
                bf[a] = *(const f4*)&Ub[(((8 * hr + a) * 32 + li) * 4 + (q ^ usw)) * 4];
            // BT rows 2hr, 2hr+1 of each patch column: hr = 0 gives d0-d2 and
            // d1+d2, hr = 1 gives d2-d1 and d3-d1, i.e. dA-dB and dC+(+-dB)
            // with A = 2hr, B = 2-hr, C = 1+2hr: a wave-uniform row choice
            // with no branch between the reads.  (Separate code per hr costs
            // registers here and spills.)
            f4 t[2][4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int k = stx + (j >> 1);
                const int qs = q ^ ((k >> 2) & 3);
                auto px = [&](int i) {
                    return *(const f4*)&X[((((2 * srr + i) * 2 + (j & 1)) * TCP + k) * 4 + qs) * 4];
                };
                f4 dA = px(rA), dB = px(rB), dC = px(rC);
                f4 dBs;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    dBs[e] = __uint_as_float(__float_as_uint(dB[e]) ^ smask);
                t[0][j] = dA - dB;
                t[1][j] = dC + dBs;
            }
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                f4 dh[4];
                dh[0] = t[i][0] - t[i][2];
                dh[1] = t[i][1] + t[i][2];
                dh[2] = t[i][2] - t[i][1];
                dh[3] = t[i][3] - t[i][1];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int a = i * 4 + j;
#pragma unroll
                    for (int s = 0; s < 4; ++s)
                        acc[a] = __builtin_amdgcn_mfma_f32_32x32x2f32(dh[j][s], bf[a][s], acc[a], 0, 0, 0);
                    const int item = h * 8 + a;
                    if (item < NITEM && c0n >= 0) dma_item(item, c0n, nbase);
                }
            }
        }
    };

    const int nch = Cinp / KC;
    for (int ch = 0; ch < nch; ++ch) {
        __builtin_amdgcn_s_waitcnt(0);   // this wave's DMAs for chunk ch have landed
        __syncthreads();                 // ... and every other wave's; buffer ch+1 is free
        compute(ch & 1, ch + 1 < nch ? (ch + 1) * KC : -1, (ch + 1) & 1);
    }

    // ---- epilogue.  Lane l, register r <-> MFMA row 8*(r/4)+4*(l/32)+r%4, channel l%32.
    // S_i[c] = sum_j AT[c][j] M[i][j]; Y[0][c] = S0+S1+S2, Y[1][c] = S1-S2+S3.
    // Wave 2p+h writes the partial 2x2 outputs of its transform rows into
    // output tile h in LDS, slot-major ([128 slots][2x2 pixels][32 channels],
    // so every write is a lane base plus an immediate); then every thread
    // adds the two tiles, bias and ReLU and stores 16-byte channel quads (32
    // output channels = 128 contiguous bytes per pixel).
    __syncthreads();                     // staging buffers are free
    // Slot stride 136 floats: the lane halves (4 slots apart) of a 64-lane
    // write land 32 banks apart.
    constexpr int SS = 136;
    constexpr int TILE = 128 * SS;       // floats per output tile
    {
        float* p = smem + hr * TILE + (pair * 32 + 4 * g) * SS + li;
        if (hr == 0) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float* ps = p + (8 * (r >> 2) + (r & 3)) * SS;
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    // rows 0, 1 of M: S0 and S1
                    float m0 = acc[0][r], m1 = acc[1][r], m2 = acc[2][r], m3 = acc[3][r];
                    float n0 = acc[4][r], n1 = acc[5][r], n2 = acc[6][r], n3 = acc[7][r];
                    float s0 = c == 0 ? m0 + m1 + m2 : m1 - m2 + m3;
                    float s1 = c == 0 ? n0 + n1 + n2 : n1 - n2 + n3;
                    ps[c * 32] = s0 + s1;          // Y[0][c] partial: S0 + S1
                    ps[(2 + c) * 32] = s1;         // Y[1][c] partial: S1
                }
            }
        } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float* ps = p + (8 * (r >> 2) + (r & 3)) * SS;
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    // rows 2, 3 of M: S2 and S3
                    float m0 = acc[0][r], m1 = acc[1][r], m2 = acc[2][r], m3 = acc[3][r];
                    float n0 = acc[4][r], n1 = acc[5][r], n2 = acc[6][r], n3 = acc[7][r];
                    float s2 = c == 0 ? m0 + m1 + m2 : m1 - m2 + m3;
                    float s3 = c == 0 ? n0 + n1 + n2 : n1 - n2 + n3;
                    ps[c * 32] = s2;               // Y[0][c] partial: S2
                    ps[(2 + c) * 32] = s3 - s2;    // Y[1][c] partial: S3 - S2
                }
            }
        }
    }
    __syncthreads();
    const int qd = tid & 7;              // channel quad: fixed, since NT % 8 == 0
    const int c = cob + 4 * qd;
    f4 bq = {0.f, 0.f, 0.f, 0.f};
    if (bias) {
#pragma unroll
        for (int t = 0; t < 4; ++t) bq[t] = c + t < Cout ? bias[c + t] : 0.f;
    }
    // Output pixel (py, px) of the block = slot (py/2)*TC + px/2, sub-pixel
    // 2*(py&1) + (px&1).  py = pxl / (2TC) uses a float reciprocal: pxl < 2^9
    // and the exact quotient sits at least 1/256 from an integer, far above
    // the float rounding error.
    const int OW2 = 2 * TC;
    const float rw2 = 1.0f / (float)OW2;
    const int nq = 2 * R * OW2 * 8;      // float4 quads of the output block (<= 8 * NT)
#pragma unroll
    for (int it = 0; it < 8; ++it) {
        const int e = tid + it * NT;
        if (e >= nq) break;
        int pxl = e >> 3;
        int py = (int)(((float)pxl + 0.5f) * rw2), pxx = pxl - py * OW2;
        int oh = 2 * ty0 + py, ow = 2 * tx0 + pxx;
        if (oh >= H || ow >= W || c >= Cout) continue;
        int so = ((py >> 1) * TC + (pxx >> 1)) * SS + (2 * (py & 1) + (pxx & 1)) * 32 + 4 * qd;
        f4 v = *(const f4*)&smem[so] + *(const f4*)&smem[TILE + so] + bq;
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] = act_apply(v[t], act);
        float* dst = out + (((long long)n * H + oh) * W + ow) * Cout + c;
        if (c + 4 <= Cout && (Cout & 3) == 0) {
            *(f4*)dst = v;
        } else {
            for (int t = 0; t < 4 && c + t < Cout; ++t) dst[t] = v[t];
        }
    }
}

// F(2,3), one 32-tile x 32-channel unit per 256-thread workgroup, three
// workgroups per CU.
//
// Block = R x TC tiles (R*TC = 32, TC = 16 or 8, both compile-time) of one
// image x 32 output channels.  Wave i accumulates the 4 points of row i of
// the 4x4 Winograd grid for all 32 tiles (v_mfma_f32_32x32x2f32, M = tiles,
// N = channels, K = 2 channels: 4 x 16 accumulators).  Input channels are
// consumed in chunks of 8 (one MFMA k-step pair per lane half g = lane/32
// holding a quad of 4 channels).
//
// Software pipeline, per wave and chunk c:
//   wait for the wave's own U(c) and X(c+1) loads;  DMA U(c+1) -- only the
//   wave's 4 points, into its private double buffer, so U needs no barrier;
//   MFMAs of points 0-1;  workgroup barrier (everyone's X(c+1) has landed and
//   nobody reads X(c) any more);  DMA X(c+3) into X(c)'s buffer;  LDS reads
//   of X(c+1);  MFMAs of points 2-3;  input transform of X(c+1) in registers.
// The MFMAs issued before the barrier and after the reads cover the barrier
// and the LDS latency, and X (the (2R+2) x (2TC+2) pixels of a chunk, DMA'd by
// buffer_load ... lds with zeros past the resources' ends) is prefetched two
// chunks ahead through three buffers.  LDS is 53 KB: three workgroups per CU.
//
// LDS layouts (16-byte quads): X [row][plane = col%2][kk = col/2][2 quads]
// with kk padded to TC+1 and quad q at slot q ^ ((kk >> log2(TC/2)) & 1);
// U, per wave, [point][co][2 quads] with quad q at slot q ^ ((co >> 3) & 1).
// Both make every 16-lane ds_read_b128 group hit 64 distinct banks.
//
// Epilogue: wave i reduces its row with AT (S_i[c] = sum_j AT[c][j] M[i][j])
// into LDS; every thread then forms Y[0][c] = S0+S1+S2, Y[1][c] = S1-S2+S3 for
// one tile and 4 channels, adds the bias (loaded at the start), applies the
// activation and stores 16-byte quads.
template <int TC, int ROW>
struct W23Row;   // BT row ROW of a patch column: t = d[A] -/+ d[B]
template <int TC> struct W23Row<TC, 0> { static constexpr int A = 0, B = 2, PLUS = 0; };
template <int TC> struct W23Row<TC, 1> { static constexpr int A = 1, B = 2, PLUS = 1; };
template <int TC> struct W23Row<TC, 2> { static constexpr int A = 2, B = 1, PLUS = 0; };
template <int TC> struct W23Row<TC, 3> { static constexpr int A = 3, B = 1, PLUS = 0; };

// A unit is NB blocks of R x TC tiles (NB * R * TC = 32, the MFMA M side).
// With NB = 2 the blocks are separate 4 x 4-tile squares: the lanes of the
// two alternate (tile li of the unit is tile li >> 1 of block li & 1) and
// block 1's staging starts an odd number of 16-byte slots after block 0's, so
// the transform reads of 16 consecutive lanes cover all 64 banks once.
template <int TC, int NB = 1>
struct W23Cfg {
    static constexpr int R = 32 / (TC * NB);
    static constexpr int BT = R * TC;                  // tiles per block
    static constexpr int NR = 2 * R + 2;               // staged pixel rows
    static constexpr int TCP = TC + 1;                 // kk per plane (padded)
    static constexpr int SWZ = NB == 2 ? -1 : (TC == 16 ? 3 : 2);   // swizzle bit of kk (-1: none)
    static constexpr int BS = NR * 2 * TCP * 2 + (NB == 2 ? 1 : 0);   // slots per block
    static constexpr int XSLOTS = NB * BS;
    static constexpr int XBLK = (XSLOTS + 63) / 64;    // 64-slot DMA blocks
    static constexpr int XFL = XBLK * 256;             // floats: whole DMA blocks (the slots
                                                       // past XSLOTS load zeros, never read)
    static constexpr int KX = (XBLK + 3) / 4;          // X blocks per wave (at most)
    static constexpr int SST = 40;                     // epilogue tile stride (floats)
    static constexpr int EPI = 4 * 2 * 32 * SST;       // epilogue staging (floats)
    static constexpr int LDS = (3 * XFL > EPI ? 3 * XFL : EPI) * 4;  // bytes
    static_assert(3 * LDS <= 160 * 1024, "three workgroups per CU");
    template <int WAVE>                                // X blocks wave WAVE issues per chunk
    static constexpr int nxw() { return XBLK > WAVE + 4 * (KX - 1) ? KX : KX - 1; }
    static constexpr __device__ int swz(int kk) { return SWZ < 0 ? 0 : (kk >> SWZ) & 1; }
    static_assert(NB * R * TC == 32, "32 tiles per unit");
};

// s_waitcnt vmcnt(n) for a wave-uniform n in 0..4 (the count is an immediate)
__device__ __forceinline__ void wait_vmcnt(int n) {
    switch (n) {
        case 0: __builtin_amdgcn_s_waitcnt(0x0F70); break;
        case 1: __builtin_amdgcn_s_waitcnt(0x0F71); break;
        case 2: __builtin_amdgcn_s_waitcnt(0x0F72); break;
        case 3: __builtin_amdgcn_s_waitcnt(0x0F73); break;
        default: __builtin_amdgcn_s_waitcnt(0x0F74); break;
    }
}

template <int TC>
__global__ __launch_bounds__(256, 3) void k_wino23u(
    const float* __restrict__ in, const float* __restrict__ U, const float* __restrict__ bias,
    float* __restrict__ out, int H, int W, int Cin, int Cinp, int Cout, int rblocks, int act,
    int gx, int gy) {
    using CF = W23Cfg<TC>;
    constexpr int R = CF::R, TCP = CF::TCP;
    constexpr unsigned kOOB = 0x80000000u;
    extern __shared__ __attribute__((aligned(16))) float smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // = transform row
    const int li = lane & 31, g = lane >> 5;
    const int nch = Cinp / 8;
    const unsigned upt = 32u * Cout;                   // bytes per point of one chunk
    const __amdgpu_buffer_rsrc_t ures =
        __builtin_amdgcn_make_buffer_rsrc((void*)U, (short)0, (int)(16u * upt * (Cinp >> 3)), 0x00020000);
    const bool ragged = (Cin & 7) != 0;
    // per-lane LDS read offsets (floats, X buffer 0)
    const int sr = li / TC, stx = li % TC;
    int xoff[2][2];                                    // [kk = stx + jj][plane]
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
        const int kk = stx + jj;
        const int qs = g ^ ((kk >> CF::SWZ) & 1);
#pragma unroll
        for (int pl = 0; pl < 2; ++pl) xoff[jj][pl] = (((2 * sr * 2 + pl) * TCP + kk) * 2 + qs) * 4;
    }
    const int etile = tid >> 3, ecq = 4 * (tid & 7);   // epilogue: one tile x 4 channels

    // Unit u, input-channel chunks [c0, c1).  Units are numbered with the
    // column block fastest, then image x row block, then channel block.
    auto unit = [&](int u, int c0, int c1) {
        const int bx = u % gx, byz = u / gx;
        const int by = byz % gy, bz = byz / gy;
        const int n = by / rblocks;
        const int ty0 = (by - n * rblocks) * R;
        const int tx0 = bx * TC;
        const int cob = bz * 32;
        const float* __restrict__ img = in + (long long)n * H * W * Cin;
        const int ec = cob + ecq;
        // bias first, so its latency hides behind the main loop
        f4 bq = {0.f, 0.f, 0.f, 0.f};
        if (bias) {
#pragma unroll
            for (int e = 0; e < 4; ++e) bq[e] = ec + e < Cout ? bias[ec + e] : 0.f;
        }

        // ---- DMA descriptors.  X: wave w issues blocks w, w+4, ... of XSLOTS
        // 16-byte slots; slot -> (row, plane, kk, quad slot) -> pixel + channel
        // quad.  U (chunked layout [Cinp/8][16][Cout][8]) goes straight to
        // registers: wave w loads its own points 4w..4w+3, each one contiguous
        // kilobyte, lane (li, g) the quad g of output channel li -- the MFMA B
        // operand for four k-steps.
        unsigned xv[CF::KX];
        unsigned xq = 0;
#pragma unroll
        for (int k = 0; k < CF::KX; ++k) {
            const int sl = (wave + 4 * k) * 64 + lane;
            const int qslot = sl & 1;
            const int pk = sl >> 1;                     // (row*2 + plane)*TCP + kk
            const int rp = pk / TCP, kk = pk - rp * TCP;
            const int row = rp >> 1, plane = rp & 1;
            const int q = qslot ^ ((kk >> CF::SWZ) & 1);
            const int ih = 2 * ty0 - 1 + row, iw = 2 * tx0 - 1 + 2 * kk + plane;
            const bool ok = sl < CF::XSLOTS && (unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W;
            xv[k] = ok ? (unsigned)((ih * W + iw) * Cin + 4 * q) * 4u : kOOB;
            xq |= (unsigned)q << k;
        }
        const unsigned uv = cob + li < Cout ? (unsigned)((cob + li) * 8 + 4 * g) * 4u : kOOB;
        const __amdgpu_buffer_rsrc_t xres =
            __builtin_amdgcn_make_buffer_rsrc((void*)img, (short)0, H * W * Cin * 4, 0x00020000);
        const int m = c1 - c0;                          // chunks of this range (even)
        // chunk c0 + j goes to X buffer j % 3.  A chunk index j >= m (the
        // pipeline's loads past the range) reads out of range: the loads are
        // still issued, so every step issues the same instructions and wait
        // counts, but they return zeros without touching memory.
        auto ld_u = [&](int j, f4* ub) {               // U(j): this wave's 4 points
            const bool live = j < m;
            const unsigned cbase = (unsigned)(c0 + (live ? j : 0)) * 16u * upt;
            const unsigned v = live ? uv : kOOB;
#pragma unroll
            for (int k = 0; k < 4; ++k)
                ub[k] = __builtin_bit_cast(
                    f4, __builtin_amdgcn_raw_buffer_load_b128(ures, v, cbase + (unsigned)(4 * wave + k) * upt, 0));
        };
        // X(j) into base: blocks WAVE, WAVE+4, ... (a compile-time count per wave,
        // all lanes active, so the compiler's wait counts are exact)
        auto dma_x = [&](auto wavec, int j, float* base) {
            constexpr int WAVE = decltype(wavec)::value;
            const bool live = j < m;
            const int ci = 8 * (c0 + (live ? j : 0));
#pragma unroll
            for (int k = 0; k < CF::KX; ++k) {
                if (WAVE + 4 * k >= CF::XBLK) continue;
                unsigned v = live ? xv[k] : kOOB;
                if (ragged && ci + 8 > Cin && ci + 4 * (int)((xq >> k) & 1) >= Cin) v = kOOB;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xres, (lds_void*)(base + (WAVE + 4 * k) * 256), 16,
                                                         v, ci * 4, 0, 0);
            }
        };

        f16v acc[4];
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[a][e] = 0.f;

        auto run = [&](auto rowc) {
            constexpr int ROW = decltype(rowc)::value;
            using RW = W23Row<TC, ROW>;
            constexpr int NXW = CF::template nxw<ROW>();   // X blocks this wave issues per chunk

            // ---- prologue: U(0), X(0), X(1), X(2) in this order; wait for U(0),
            // X(0).  Loads past the range fill a buffer no one reads with zeros.
            f4 uA[4], uB[4];
            ld_u(0, uA);
            dma_x(rowc, 0, smem);
            dma_x(rowc, 1, smem + CF::XFL);
            dma_x(rowc, 2, smem + 2 * CF::XFL);
            wait_vmcnt(2 * NXW);
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

            // row ROW of BT d for the lane's 4 patch columns (LDS reads), then BT
            // along the columns: dh[j] = (BT d BT^T)[ROW][j]
            auto xread = [&](const float* X, f4* dA, f4* dB) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int o = xoff[j >> 1][j & 1];
                    dA[j] = *(const f4*)&X[o + RW::A * 2 * TCP * 8];
                    dB[j] = *(const f4*)&X[o + RW::B * 2 * TCP * 8];
                }
            };
            auto xform = [&](const f4* dA, const f4* dB, f4* dh) {
                f4 tt[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) tt[j] = RW::PLUS ? dA[j] + dB[j] : dA[j] - dB[j];
                dh[0] = tt[0] - tt[2];
                dh[1] = tt[1] + tt[2];
                dh[2] = tt[2] - tt[1];
                dh[3] = tt[3] - tt[1];
            };
            auto mfma_pt = [&](int a, const f4& d, const f4& bb) {
#pragma unroll
                for (int s2 = 0; s2 < 4; ++s2)
                    acc[a] = __builtin_amdgcn_mfma_f32_32x32x2f32(d[s2], bb[s2], acc[a], 0, 0, 0);
            };
            f4 dh[4];
            {
                f4 dA[4], dB[4];
                xread(smem, dA, dB);
                xform(dA, dB, dh);
            }
            int xb = 0;                                // X buffer of chunk j: j % 3
            // chunk j multiplies with bf = U(j) and loads U(j+1) into un
            auto chunk = [&](int j, const f4* bf, f4* un) {
                // this wave's U(j) and X(j+1) have landed; X(j+2) may stay in flight
                wait_vmcnt(NXW);
                ld_u(j + 1, un);
                mfma_pt(0, dh[0], bf[0]);
                mfma_pt(1, dh[1], bf[1]);
                const int xb1 = xb == 2 ? 0 : xb + 1;  // buffer of X(j+1)
                // LDS-only workgroup barrier: __syncthreads() would also wait for
                // the DMA still in flight.  lgkmcnt(0): this wave's LDS reads are
                // complete; the memory clobber keeps LDS accesses on their side.
                // After it X(j+1) is visible and X(j)'s buffer is free.
                asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
                dma_x(rowc, j + 3, smem + xb * CF::XFL);
                // X(j+1) (after the last chunk: a buffer whose out-of-range loads
                // completed at the wait above, read before any wave reaches the
                // epilogue, results unused) -- unconditional so the transform can
                // interleave with the MFMAs
                f4 dA[4], dB[4];
                xread(smem + xb1 * CF::XFL, dA, dB);
                __builtin_amdgcn_sched_barrier(0);      // the reads go out first
                mfma_pt(2, dh[2], bf[2]);
                mfma_pt(3, dh[3], bf[3]);
                xform(dA, dB, dh);
                // two MFMAs cover the LDS latency, then the transform's 32 VALU
                // operations interleave with the remaining six
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
#pragma unroll
                for (int i = 0; i < 6; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                }
                xb = xb1;
            };
            for (int j = 0; j < m; j += 2) {           // two register sets for U, no copies
                chunk(j, uA, uB);
                chunk(j + 1, uB, uA);
            }
        };
        switch (wave) {
            case 0: run(std::integral_constant<int, 0>{}); break;
            case 1: run(std::integral_constant<int, 1>{}); break;
            case 2: run(std::integral_constant<int, 2>{}); break;
            default: run(std::integral_constant<int, 3>{}); break;
        }

        // ---- epilogue.  Lane l, register r <-> MFMA row (tile) 8*(r/4)+4*(l/32)+r%4,
        // column (channel) l%32.  S layout [row 4][c 2][tile 32][SST floats].
        wait_vmcnt(0);                       // the last (out-of-range) X loads have landed
        __syncthreads();                     // staging buffers are free
        {
            float* pp = smem + (wave * 2) * 32 * CF::SST + (4 * g) * CF::SST + li;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int tt = 8 * (r >> 2) + (r & 3);
                float m0 = acc[0][r], m1 = acc[1][r], m2 = acc[2][r], m3 = acc[3][r];
                pp[tt * CF::SST] = m0 + m1 + m2;                   // S_i[0]
                pp[(32 + tt) * CF::SST] = m1 - m2 + m3;            // S_i[1]
            }
        }
        __syncthreads();
        f4 S[4][2];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int cc = 0; cc < 2; ++cc)
                S[i][cc] = *(const f4*)&smem[((i * 2 + cc) * 32 + etile) * CF::SST + ecq];
        if (ec < Cout) {
            const int tsr = etile / TC, tsx = etile % TC;
            const int oh0 = 2 * (ty0 + tsr), ow0 = 2 * (tx0 + tsx);
#pragma unroll
            for (int r = 0; r < 2; ++r) {
#pragma unroll
                for (int cc = 0; cc < 2; ++cc) {
                    const int oh = oh0 + r, ow = ow0 + cc;
                    if (oh >= H || ow >= W) continue;
                    f4 v = r == 0 ? S[0][cc] + S[1][cc] + S[2][cc] : S[1][cc] - S[2][cc] + S[3][cc];
                    v = v + bq;
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = act_apply(v[e], act);
                    float* dst = out + (((long long)n * H + oh) * W + ow) * Cout + ec;
                    if (ec + 4 <= Cout && (Cout & 3) == 0) {
                        *(f4*)dst = v;
                    } else {
                        for (int e = 0; e < 4 && ec + e < Cout; ++e) dst[e] = v[e];
                    }
                }
            }
        }
    };

    unit(blockIdx.x, 0, nch);
}

template <int TC>
bool launch_wino23u(const float* in, const float* U, const float* bias, float* out, int N, int H,
                    int W, int Cin, int Cinp, int Cout, int tH, int tW, int act, hipStream_t s) {
    using CF = W23Cfg<TC>;
    // set once per process, thread-safely, before any launch below
    static const bool attr = [&] {
        (void)hipFuncSetAttribute((const void*)k_wino23u<TC>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, CF::LDS);
        return true;
    }();
    (void)attr;
    const int rblocks = (tH + CF::R - 1) / CF::R;
    const int gx = (tW + TC - 1) / TC, gy = N * rblocks, gz = (Cout + 31) / 32;
    ACFUN_LAUNCH("k_wino23", k_wino23u<TC>, dim3((unsigned)(gx * gy * gz)), dim3(256), CF::LDS, s, in,
                 U, bias, out, H, W, Cin, Cinp, Cout, rblocks, act, gx, gy);
    return check_launch("k_wino23u");
}

// F(2,3), persistent form of k_wino23u: each workgroup runs a list of
// 32-tile x 32-channel units back to back, and the chunk pipeline runs on
// across unit boundaries -- the loads of the next unit's first chunks are
// issued during the current unit's last ones, so a unit costs no load
// latency up front and no drain at the end.
//
// Unit u (channel block fastest, then column block, then image x row block)
// is assigned by XCD: XCD x = blockIdx.x % 8 owns the contiguous unit range
// [x*U/8, (x+1)*U/8) and its workgroups take it round robin, so the two
// channel blocks of a spatial block and neighbouring row blocks (which share
// two halo rows) are read while still in that XCD's L2.
//
// The per-chunk body is k_wino23u's (same LDS layouts, operands and MFMA
// order).  A lane's X slot offsets relative to a unit's window origin are the
// same for every unit; per unit only the window origin (a scalar) and the
// lane's in-image bits change.  The epilogue runs in two rounds through a
// 20 KB LDS area (output column cc of the 2x2 tiles): each wave stores its
// row sums S_i[cc] (the AT column reduction
// of its transform row) in LDS, and after a barrier every thread forms
// Y[0][cc] = S0 + S1 + S2 and Y[1][cc] = S1 - S2 + S3 for one tile and 4
// channels, adds the bias (staged in LDS at the start), applies the
// activation and stores two 16-byte quads.
//
// Wait counts.  Chunk J issues U(J+1) at its start and X(J+3) after its
// barrier (the next unit's chunks once J+1, J+3 pass the unit's end), and
// waits for U(J), X(J+1) with X(J+2) left in flight, as in k_wino23u.  The
// epilogue after a unit's last chunk J makes the wait of chunk J+1 (X(J+3)
// left in flight) before its stores, so that chunk skips it.  Stores then
// sit between loads in the vmcnt queue: a later wait that leaves n loads in
// flight still proves every older load landed, because loads complete in
// issue order (a store may complete at any time; it only makes the wait
// longer).  The stores are inline asm, so the compiler's own wait insertion
// sees only loads, whose counts are exact, instead of falling back to
// vmcnt(0) for mixed loads and stores.
template <int TC, int NB, int ACT>
__global__ __launch_bounds__(256, 3) void k_wino23p(
    const float* __restrict__ in, const float* __restrict__ U, const float* __restrict__ bias,
    float* __restrict__ out, int H, int W, int Cin, int Cinp, int Cout, int rblocks, int gx, int gz,
    int nunits, int in_bytes, int nblk) {
    using CF = W23Cfg<TC, NB>;
    constexpr int R = CF::R, TCP = CF::TCP;
    constexpr unsigned kOOB = 0x80000000u;
    extern __shared__ __attribute__((aligned(16))) float smem[];
    float* const epi = smem + 3 * CF::XFL;             // [S_i 4][tile 32][SST floats]
    float* const bsm = epi + 4 * 32 * CF::SST;         // bias, Cout floats (padded to 4)
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // = transform row
    const int li = lane & 31, g = lane >> 5;
    const int m = Cinp / 8;                            // chunks per unit (even, >= 4)

    // this workgroup's units: rs + i0, rs + i0 + nwx, ... < re
    const int nwx = (int)(gridDim.x / 8);
    const int xcd = (int)(blockIdx.x % 8), i0 = (int)(blockIdx.x / 8);
    const int rs = (int)((long long)xcd * nunits / 8), re = (int)((long long)(xcd + 1) * nunits / 8);
    const int nu = rs + i0 < re ? (re - rs - i0 + nwx - 1) / nwx : 0;
    if (nu == 0) return;                               // uniform per workgroup

    for (int c = tid; c < (Cout + 3) / 4 * 4; c += 256) bsm[c] = bias && c < Cout ? bias[c] : 0.f;
    const int etile = tid >> 3, ecq = 4 * (tid & 7);   // epilogue: one tile x 4 channels
    const bool Cout4 = (Cout & 3) == 0;

    const unsigned upt = 32u * Cout;                   // bytes per point of one chunk
    const __amdgpu_buffer_rsrc_t ures =
        __builtin_amdgcn_make_buffer_rsrc((void*)U, (short)0, (int)(16u * upt * (Cinp >> 3)), 0x00020000);
    const __amdgpu_buffer_rsrc_t xres =
        __builtin_amdgcn_make_buffer_rsrc((void*)in, (short)0, in_bytes, 0x00020000);
    const bool ragged = (Cin & 7) != 0;
    // per-lane LDS read offsets (floats, X buffer 0): tile li of the unit is
    // tile lt of block lb
    const int lb = NB == 2 ? (li & 1) : 0, lt = NB == 2 ? (li >> 1) : li;
    const int sr = lt / TC, stx = lt % TC;
    int xoff[2][2];                                    // [kk = stx + jj][plane]
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
        const int kk = stx + jj;
        const int qs = g ^ CF::swz(kk);
#pragma unroll
        for (int pl = 0; pl < 2; ++pl)
            xoff[jj][pl] = (lb * CF::BS + ((2 * sr * 2 + pl) * TCP + kk) * 2 + qs) * 4;
    }
    // X DMA slots of this lane: block k holds slot (wave + 4k)*64 + lane ->
    // tile block sb, staged pixel (row, col) of that block's window and
    // channel quad q.  xlo[k]: the slot's byte offset from the window origin
    // (pixel (2 ty0 - 1, 2 tx0 - 1) of the block's image), the same for every
    // unit; bit k of sbits: sb.
    struct Slot { int sb, rp, kk, q; };
    auto slot = [&](int k) {
        const int sl = (wave + 4 * k) * 64 + lane;
        const int sb = NB == 2 && sl >= CF::BS ? 1 : 0;
        const int s1 = sl - sb * CF::BS;
        const int pk = s1 >> 1;                        // (row*2 + plane)*TCP + kk
        const int rp = pk / TCP, kk = pk - rp * TCP;
        return Slot{sb, rp, kk, (s1 & 1) ^ CF::swz(kk)};
    };
    unsigned xlo[CF::KX], sbits = 0;
#pragma unroll
    for (int k = 0; k < CF::KX; ++k) {
        const Slot q = slot(k);
        xlo[k] = (unsigned)((((q.rp >> 1) * W + 2 * q.kk + (q.rp & 1)) * Cin + 4 * q.q) * 4);
        sbits |= (unsigned)q.sb << k;
    }
    // Block b of a unit: px, the index of its window origin pixel (2 ty0 - 1,
    // 2 tx0 - 1) of image n (negative at the first image's top left), and the
    // pixel rows and columns from its first output row and column to the
    // image's edge, rl = H - 2 ty0 and cl = W - 2 tx0 (-1: no block, the
    // last unit's second block when the block count is odd).  A staged row
    // or column i of the window (0 = origin) is in the image when
    // 1 - (rl < H) <= i <= rl (columns: cl, W).
    struct UnitP { int px[NB], rl[NB], cl[NB], cob; };
    auto decode = [&](int k) {                         // k-th unit of this workgroup
        const int u = rs + i0 + k * nwx;
        const int bz = u % gz, sp = u / gz;
        UnitP P;
        P.cob = bz * 32;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int blk = sp * NB + b;               // block: column fastest, then image x row
            const int bx = blk % gx, by = blk / gx;
            const int n = by / rblocks;
            const int ty0 = (by - n * rblocks) * R, tx0 = bx * TC;
            const bool live = NB == 1 || blk < nblk;
            P.px[b] = (n * H + 2 * ty0 - 1) * W + 2 * tx0 - 1;
            P.rl[b] = live ? H - 2 * ty0 : -1;
            P.cl[b] = live ? W - 2 * tx0 : -1;
        }
        return P;
    };
    // in-image bits of the lane's slots for unit P: bit k (k < KX)
    auto inimg = [&](const UnitP& P, bool live) {
        unsigned b = 0;
#pragma unroll
        for (int k = 0; k < CF::KX; ++k) {
            const int sl = (wave + 4 * k) * 64 + lane;
            const Slot q = slot(k);
            const int rl = q.sb ? P.rl[NB - 1] : P.rl[0], cl = q.sb ? P.cl[NB - 1] : P.cl[0];
            const int i = q.rp >> 1, jc = 2 * q.kk + (q.rp & 1);
            const bool ok = live && sl < CF::XSLOTS && i >= (rl < H ? 0 : 1) && i <= rl &&
                            jc >= (cl < W ? 0 : 1) && jc <= cl;
            b |= (unsigned)ok << k;
        }
        return b;
    };
    // byte offset of block b's window origin in unit P (negative at the
    // image's top left; origin + xlo is in range wherever the in-image bit is
    // set)
    auto origin = [&](const UnitP& P, int b) { return P.px[b] * Cin * 4; };
    // U(j) of unit P: this wave's 4 points; out of range (zeros, no memory
    // access) when !live
    auto ld_u = [&](const UnitP& P, bool live, int j, f4* ub) {
        const unsigned cbase = (unsigned)(live ? j : 0) * 16u * upt;
        const unsigned v = live && P.cob + li < Cout ? (unsigned)((P.cob + li) * 8 + 4 * g) * 4u : kOOB;
#pragma unroll
        for (int k = 0; k < 4; ++k)
            ub[k] = __builtin_bit_cast(
                f4, __builtin_amdgcn_raw_buffer_load_b128(ures, v, cbase + (unsigned)(4 * wave + k) * upt, 0));
    };
    // X(j) of the unit with window origin org and in-image bits ib into base:
    // blocks WAVE, WAVE+4, ...
    auto dma_x = [&](auto wavec, const UnitP& P, unsigned ib, int j, float* base) {
        constexpr int WAVE = decltype(wavec)::value;
        const int ci = 8 * j;
        const int org0 = origin(P, 0), org1 = origin(P, NB - 1);
#pragma unroll
        for (int k = 0; k < CF::KX; ++k) {
            if (WAVE + 4 * k >= CF::XBLK) continue;
            const int org = NB == 2 && ((sbits >> k) & 1) ? org1 : org0;
            unsigned v = (ib >> k) & 1 ? (unsigned)org + xlo[k] : kOOB;
            if (ragged && ci + 8 > Cin && ci + 4 * slot(k).q >= Cin) v = kOOB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xres, (lds_void*)(base + (WAVE + 4 * k) * 256), 16, v,
                                                     ci * 4, 0, 0);
        }
    };

    f16v acc[4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[a][e] = 0.f;

    auto run = [&](auto rowc) {
        constexpr int ROW = decltype(rowc)::value;
        using RW = W23Row<TC, ROW>;
        constexpr int NXW = CF::template nxw<ROW>();   // X blocks this wave issues per chunk

        UnitP cur = decode(0), nxt = decode(nu > 1 ? 1 : 0);
        bool nlive = nu > 1;
        // in-image bits of the current (bits 0..3) and next unit (bits 4..7)
        unsigned ib = inimg(cur, true) | (inimg(nxt, nlive) << 4);

        // ---- prologue: U(0), X(0), X(1), X(2) of the first unit; wait for
        // U(0), X(0) (and the bias staging, by the barrier's lgkmcnt)
        f4 uA[4], uB[4];
        ld_u(cur, true, 0, uA);
        dma_x(rowc, cur, ib, 0, smem);
        dma_x(rowc, cur, ib, 1, smem + CF::XFL);
        dma_x(rowc, cur, ib, 2, smem + 2 * CF::XFL);
        wait_vmcnt(2 * NXW);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

        auto xread = [&](const float* X, f4* dA, f4* dB) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int o = xoff[j >> 1][j & 1];
                dA[j] = *(const f4*)&X[o + RW::A * 2 * TCP * 8];
                dB[j] = *(const f4*)&X[o + RW::B * 2 * TCP * 8];
            }
        };
        auto xform = [&](const f4* dA, const f4* dB, f4* dh) {
            f4 tt[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) tt[j] = RW::PLUS ? dA[j] + dB[j] : dA[j] - dB[j];
            dh[0] = tt[0] - tt[2];
            dh[1] = tt[1] + tt[2];
            dh[2] = tt[2] - tt[1];
            dh[3] = tt[3] - tt[1];
        };
        auto mfma_pt = [&](int a, const f4& d, const f4& bb) {
#pragma unroll
            for (int s2 = 0; s2 < 4; ++s2)
                acc[a] = __builtin_amdgcn_mfma_f32_32x32x2f32(d[s2], bb[s2], acc[a], 0, 0, 0);
        };
        f4 dh[4];
        {
            f4 dA[4], dB[4];
            xread(smem, dA, dB);
            xform(dA, dB, dh);
        }
        int xb = 0;                                    // X buffer of the current chunk
        // chunk j of the current unit multiplies with bf and loads the next
        // chunk's U into un
        auto chunk = [&](int j, const f4* bf, f4* un, bool wait) {
            if (wait) wait_vmcnt(NXW);                 // U(j), X(j+1) have landed
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
                dma_x(rowc, in_cur ? cur : nxt, in_cur ? ib : ib >> 4, in_cur ? j + 3 : j + 3 - m,
                      smem + xb * CF::XFL);
            }
            f4 dA[4], dB[4];
            xread(smem + xb1 * CF::XFL, dA, dB);
            __builtin_amdgcn_sched_barrier(0);
            mfma_pt(2, dh[2], bf[2]);
            mfma_pt(3, dh[3], bf[3]);
            xform(dA, dB, dh);
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
#pragma unroll
            for (int i = 0; i < 6; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            }
            xb = xb1;
        };

        for (int k = 0; k < nu; ++k) {
            // two register sets for U, no copies; the first chunk after an
            // epilogue needs no wait (the epilogue's covers it)
            for (int j = 0; j < m; j += 2) {
                chunk(j, uA, uB, j != 0 || k == 0);
                chunk(j + 1, uB, uA, true);
            }
            // ---- epilogue of unit cur.  After this wait only the X(J+3)
            // loads of the last chunk J (the next unit's X(2)) are in flight:
            // the next unit's U(0) and X(1), which its first chunk needs, have
            // landed.  Two rounds (output column cc of each tile): every wave
            // stores its row sum S_ROW[cc] in LDS, then every thread forms
            // Y[0][cc] = S0 + S1 + S2 and Y[1][cc] = S1 - S2 + S3 for one tile
            // and 4 channels and stores two 16-byte quads.
            wait_vmcnt(NXW);
            const int ec = cur.cob + ecq;
            const f4 bq = *(const f4*)&bsm[ec < Cout ? ec : 0];
            const int eb = NB == 2 ? (etile & 1) : 0, et = NB == 2 ? (etile >> 1) : etile;
            const int tsr = et / TC, tsx = et % TC;
            // output rows / columns of this tile left before the image's edge
            const int erl = (eb ? cur.rl[NB - 1] : cur.rl[0]) - 2 * tsr;
            const int ecl = (eb ? cur.cl[NB - 1] : cur.cl[0]) - 2 * tsx;
            const int epx = (eb ? cur.px[NB - 1] : cur.px[0]) + (2 * tsr + 1) * W + 2 * tsx + 1;
            float* const orow = out + (long long)(erl > 0 ? epx : 0) * Cout + ec;
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                {
                    float* pp = epi + (ROW * 32 + 4 * g) * CF::SST + li;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const float m0 = acc[0][r], m1 = acc[1][r], m2 = acc[2][r], m3 = acc[3][r];
                        pp[(8 * (r >> 2) + (r & 3)) * CF::SST] = cc == 0 ? m0 + m1 + m2 : m1 - m2 + m3;
                    }
                }
                asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
                f4 S[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) S[i] = *(const f4*)&epi[(i * 32 + etile) * CF::SST + ecq];
                // the second pass's writes (cc == 1) must not overtake these reads
                if (cc == 0) asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
                if (ec < Cout && cc < ecl) {
#pragma unroll
                    for (int r = 0; r < 2; ++r) {
                        if (r >= erl) continue;
                        f4 v = r == 0 ? S[0] + S[1] + S[2] : S[1] - S[2] + S[3];
                        v = v + bq;
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] = act_apply(v[e], ACT);
                        float* dst = orow + ((long long)r * W + cc) * Cout;
                        if (Cout4) {
                            // s_nop: a VALU write to the data registers of a store
                            // of more than 8 bytes needs a wait state after it,
                            // which the compiler cannot insert after inline asm.
                            // sc1 (device scope): the store writes through L2, so
                            // the output does not wait dirty in L2 for the kernel's
                            // final write-back, and, unlike a non-temporal store,
                            // stays cached for the next kernel (config 2a: step
                            // 42.7 -> 41.0 us)
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
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[a][e] = 0.f;
            cur = nxt;
            nlive = k + 2 < nu;
            nxt = decode(nlive ? k + 2 : k + 1);
            ib = (ib >> 4) | (inimg(nxt, nlive) << 4);
        }
        wait_vmcnt(0);                                 // out-of-range loads and stores done
    };
    switch (wave) {
        case 0: run(std::integral_constant<int, 0>{}); break;
        case 1: run(std::integral_constant<int, 1>{}); break;
        case 2: run(std::integral_constant<int, 2>{}); break;
        default: run(std::integral_constant<int, 3>{}); break;
    }
}

template <int TC, int NB>
size_t wino23p_lds(int Cout) {
    using CF = W23Cfg<TC, NB>;
    return ((size_t)3 * CF::XFL + 4 * 32 * CF::SST + (size_t)(Cout + 3) / 4 * 4) * sizeof(float);
}

// Persistent launch: 3 workgroups per CU (a multiple of 8 workgroups), each
// running its share of the units.  False when the shape does not suit it
// (fewer than 4 chunks per unit, the input past 2 GB or the LDS budget).
template <int TC, int NB = 1>
bool launch_wino23p(const float* in, const float* U, const float* bias, float* out, int N, int H,
                    int W, int Cin, int Cinp, int Cout, int tH, int tW, int act, hipStream_t s,
                    bool* launched) {
    using CF = W23Cfg<TC, NB>;
    *launched = false;
    const size_t lds = wino23p_lds<TC, NB>(Cout);
    const long long in_bytes = (long long)N * H * W * Cin * 4;
    if (Cinp / 8 < 4 || in_bytes >= (1ll << 31) || lds * 3 > 160 * 1024) return true;
    // set once per process, thread-safely, before any launch below
    static const bool attr = [&] {
        (void)hipFuncSetAttribute((const void*)k_wino23p<TC, NB, 0>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024 / 3);
        (void)hipFuncSetAttribute((const void*)k_wino23p<TC, NB, 1>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024 / 3);
        (void)hipFuncSetAttribute((const void*)k_wino23p<TC, NB, 2>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024 / 3);
        return true;
    }();
    (void)attr;
    const int rblocks = (tH + CF::R - 1) / CF::R;
    const long long gx = (tW + TC - 1) / TC, gy = (long long)N * rblocks, gz = (Cout + 31) / 32;
    const long long nblk = gx * gy;                    // R x TC tile blocks
    const long long nunits = (nblk + NB - 1) / NB * gz;
    if (nunits >= (1ll << 30)) return true;
    const long long slots = 3ll * num_cus() / 8, need = (nunits + 7) / 8;
    const unsigned grid = (unsigned)(8 * (slots < need ? slots : need));
    if (act == 1)
        ACFUN_LAUNCH("k_wino23", (k_wino23p<TC, NB, 1>), dim3(grid), dim3(256), lds, s, in, U, bias, out, H,
                     W, Cin, Cinp, Cout, rblocks, (int)gx, (int)gz, (int)nunits, (int)in_bytes, (int)nblk);
    else if (act == 2)
        ACFUN_LAUNCH("k_wino23", (k_wino23p<TC, NB, 2>), dim3(grid), dim3(256), lds, s, in, U, bias, out, H,
                     W, Cin, Cinp, Cout, rblocks, (int)gx, (int)gz, (int)nunits, (int)in_bytes, (int)nblk);
    else
        ACFUN_LAUNCH("k_wino23", (k_wino23p<TC, NB, 0>), dim3(grid), dim3(256), lds, s, in, U, bias, out, H,
                     W, Cin, Cinp, Cout, rblocks, (int)gx, (int)gz, (int)nunits, (int)in_bytes, (int)nblk);
    *launched = true;
    return check_launch("k_wino23p");
}

// Which F(2,3) engine run_wino23 takes for a shape: 1 the unit kernels (their
// filter transform in the chunked layout), 0 k_wino23 (the plain layout), -1
// neither (the implicit GEMM; no filter transform).
int wino23_plan_impl(int N, int H, int W, int Cin, int Cout, const void* in) {
    const int tH = (H + 1) / 2, tW = (W + 1) / 2;
    const int Cinp = (Cin + 15) / 16 * 16;
    // The DMA staging moves whole 4-channel quads from 16-byte aligned rows.
    if (Cin % 4 != 0 || ((uintptr_t)in & 15u) != 0) return -1;
    // 32-tile units (three workgroups per CU) when the image is wide enough to
    // fill them; buffer resources address one image and the filter with 32-bit
    // byte offsets.  Images of at most 4 x 4 tiles (5 to 8 pixels a side,
    // ResNet-50's 7 x 7 stage) run units of two images' tile blocks.
    const bool small = tH >= 3 && tH <= 4 && tW >= 3 && tW <= 4 && Cinp >= 32;
    const bool unit32 = (long long)H * W * Cin * 4 < (1ll << 31) &&
                        16ll * Cout * Cinp * 4 < (1ll << 31) && (long long)N * ((tH + 1) / 2) < 65536 &&
                        (tW >= 6 || small);
    return unit32 ? 1 : 0;
}

// The filter transform for a plan (16 points x Cout x Cinp floats).
bool wino23_filter_impl(const float* w, int Cin, int Cout, int plan, float* U, hipStream_t s) {
    const int Cinp = (Cin + 15) / 16 * 16;
    if (plan == 1)
        ACFUN_LAUNCH("k_wino_filter_t", (k_wino_filter_c8<2>), dim3((Cout + 7) / 8, Cinp / 8), dim3(64), 0, s,
                     w, Cin, Cout, U);
    else
        ACFUN_LAUNCH("k_wino_filter_t", (k_wino_filter_tt<2>), dim3((Cout + 15) / 16, Cinp / 16),
                     dim3(256), 0, s, w, Cin, Cinp, Cout, U);
    return check_launch("k_wino_filter_t");
}

// Tile-search candidates (kind "w23") for the unit kernels (plan 1): 0 the
// persistent 16-wide units, 1 16-wide units one per workgroup, 2 persistent
// 8-wide, 3 8-wide one per workgroup, 4 units of two 4 x 4-tile blocks.  The
// 16-wide units run on images of at least 12 tile columns, the paired blocks
// only on images of at most 4 x 4 tiles (where the heuristic takes them).
constexpr int kW23NC = 5;
bool w23_launch(int c, const float* in, const float* U, const float* bias, float* out, int N, int H,
                int W, int Cin, int Cinp, int Cout, int tH, int tW, int act, hipStream_t s,
                bool* launched) {
    *launched = false;
    const bool small = tH >= 3 && tH <= 4 && tW >= 3 && tW <= 4 && Cinp >= 32;
    if ((c <= 1 && tW < 12) || (c == 4 && !small)) return true;
    switch (c) {
        case 0: return launch_wino23p<16>(in, U, bias, out, N, H, W, Cin, Cinp, Cout, tH, tW, act, s, launched);
        case 2: return launch_wino23p<8>(in, U, bias, out, N, H, W, Cin, Cinp, Cout, tH, tW, act, s, launched);
        case 4: return launch_wino23p<4, 2>(in, U, bias, out, N, H, W, Cin, Cinp, Cout, tH, tW, act, s, launched);
        default: break;
    }
    *launched = true;
    if (c == 1) return launch_wino23u<16>(in, U, bias, out, N, H, W, Cin, Cinp, Cout, tH, tW, act, s);
    return launch_wino23u<8>(in, U, bias, out, N, H, W, Cin, Cinp, Cout, tH, tW, act, s);
}

// The built-in choice of unit kernel for plan 1 (the tile search's candidate -1).
bool w23_default(const float* in, const float* Up, const float* bias, float* out, int N, int H, int W,
                 int Cin, int Cinp, int Cout, int tH, int tW, int act, hipStream_t s) {
    const bool small = tH >= 3 && tH <= 4 && tW >= 3 && tW <= 4 && Cinp >= 32;
    bool launched = false;
    if (small) {
        if (!launch_wino23p<4, 2>(in, Up, bias, out, N, H, W, Cin, Cinp, Cout, tH, tW, act,
                                  s, &launched))
            return false;
        if (launched) return true;
    }
    if (tW >= 12) {
        if (!launch_wino23p<16>(in, Up, bias, out, N, H, W, Cin, Cinp, Cout, tH, tW, act,
                                s, &launched))
            return false;
        if (launched) return true;
        return launch_wino23u<16>(in, Up, bias, out, N, H, W, Cin, Cinp, Cout, tH, tW,
                                  act, s);
    }
    // 8-wide units: the persistent kernel measured faster at 8 chunks per
    // unit and slower at 32 (ResNet-50's 14 x 14 x 256 stage)
    if (Cinp <= 64) {
        if (!launch_wino23p<8>(in, Up, bias, out, N, H, W, Cin, Cinp, Cout, tH, tW, act, s,
                               &launched))
            return false;
        if (launched) return true;
    }
    return launch_wino23u<8>(in, Up, bias, out, N, H, W, Cin, Cinp, Cout, tH, tW, act, s);
}

// The replay the tile search times: input and filter transform of the shape
// filled with a constant, no bias, no activation.
TuneMaker w23_maker(int N, int H, int W, int Cin, int Cout) {
    return [=]() -> TuneRunner {
        const int Cinp = (Cin + 15) / 16 * 16, tH = (H + 1) / 2, tW = (W + 1) / 2;
        const size_t ib = (size_t)N * H * W * Cin * 4, ub = (size_t)16 * Cout * Cinp * 4,
                     ob = (size_t)N * H * W * Cout * 4;
        if (ib + ub + ob > ((size_t)2 << 30)) return TuneRunner();
        hipStream_t s = lib_stream();
        auto x = std::make_shared<Scratch>(ib, s);
        auto u = std::make_shared<Scratch>(ub, s);
        auto o = std::make_shared<Scratch>(ob, s);
        if (!x->p || !u->p || !o->p || hipMemsetD32Async((hipDeviceptr_t)x->p, kTuneFill, ib / 4, s) != hipSuccess ||
            hipMemsetD32Async((hipDeviceptr_t)u->p, kTuneFill, ub / 4, s) != hipSuccess)
            return TuneRunner();
        return [=](int cand, hipStream_t st) {
            if (cand < 0)
                return w23_default(x->as<float>(), u->as<float>(), nullptr, o->as<float>(), N, H, W, Cin,
                                   Cinp, Cout, tH, tW, 0, st);
            bool launched = false;
            if (!w23_launch(cand, x->as<float>(), u->as<float>(), nullptr, o->as<float>(), N, H, W, Cin,
                            Cinp, Cout, tH, tW, 0, st, &launched))
                return false;
            return launched;
        };
    };
}

// Upre: the filter already transformed for this shape's plan (a model's cached
// transform), or null to transform it here.
bool run_wino23(const float* in, int N, int H, int W, int Cin, const float* w, const float* bias,
                int Cout, float* out, int act, hipStream_t s, const float* Upre = nullptr) {
    int tH = (H + 1) / 2, tW = (W + 1) / 2;
    int Cinp = (Cin + 15) / 16 * 16;
    const int plan = wino23_plan_impl(N, H, W, Cin, Cout, in);
    if (plan < 0) {
        ConvShape gs{N, H, W, Cin, 3, 3, 1, 1, H, W};
        return conv_igemm_f32(gs, in, w, bias, Cout, out, act, s);
    }
    Scratch Uown(Upre ? 0 : (size_t)16 * Cout * Cinp * sizeof(float), s);
    if (!Upre && !Uown.p) return false;
    const float* Up = Upre ? Upre : Uown.as<float>();
    if (plan == 1) {
        if (!Upre && !wino23_filter_impl(w, Cin, Cout, 1, Uown.as<float>(), s)) return false;
        // the tile search's choice of unit kernel for this shape, if any
        const std::vector<int> key{N, H, W, Cin, Cout};
        bool rec = false;
        const int c = tune_lookup("w23", key, kW23NC, &rec);
        if (rec) tune_record("w23", key, kW23NC, w23_maker(N, H, W, Cin, Cout));
        if (c >= 0) {
            bool launched = false;
            if (!w23_launch(c, in, Up, bias, out, N, H, W, Cin, Cinp, Cout, tH, tW, act, s, &launched))
                return false;
            if (launched) return true;
        }
        return w23_default(in, Up, bias, out, N, H, W, Cin, Cinp, Cout, tH, tW, act, s);
    }
    if (!Upre && !wino23_filter_impl(w, Cin, Cout, 0, Uown.as<float>(), s)) return false;
    // Block: TC tile columns x R tile rows of one image, R*TC <= 128 slots and
    // two LDS buffers (padded X region + 16*32*16 filter floats) within 160 KB.
    auto buf_floats = [](int R, int TC) {
        return (size_t)(((2 * R + 2) * 2 * (TC + 1) * 4 + 63) / 64 * 64 * 4 + 16 * 32 * 16);
    };
    int TC = tW < 64 ? tW : 64;
    int R = 128 / TC;
    if (R > tH) R = tH;
    while (R > 1 && 2 * sizeof(float) * buf_floats(R, TC) > 160 * 1024) --R;
    size_t lds = 2 * sizeof(float) * buf_floats(R, TC);
    // Each wave issues at most 9 X blocks of 64 slots per chunk; the epilogue
    // stages two 128-slot output tiles (136 KB) in the same LDS; buffer
    // resources address one image and the filter with 32-bit byte offsets.
    size_t xblocks = ((size_t)(2 * R + 2) * 2 * (TC + 1) * 4 + 63) / 64;
    if (lds < 2 * 128 * 136 * sizeof(float)) lds = 2 * 128 * 136 * sizeof(float);
    if (lds > 160 * 1024 || xblocks > 8 * 9 || (long long)H * W * Cin * 4 >= (1ll << 31) ||
        16ll * Cout * Cinp * 4 >= (1ll << 31)) {
        ConvShape gs{N, H, W, Cin, 3, 3, 1, 1, H, W};
        return conv_igemm_f32(gs, in, w, bias, Cout, out, act, s);
    }
    // set once per process, thread-safely, before any launch below
    static const bool attr = [&] {
        (void)hipFuncSetAttribute((const void*)k_wino23, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  160 * 1024);
        return true;
    }();
    (void)attr;
    int rblocks = (tH + R - 1) / R;
    dim3 grid((unsigned)((tW + TC - 1) / TC), (unsigned)(N * rblocks), (unsigned)((Cout + 31) / 32));
    ACFUN_LAUNCH("k_wino23", k_wino23, grid, dim3(512), lds, s, in, Up, bias, out, N, H, W,
                       Cin, Cinp, Cout, tH, tW, R, TC, act);
    return check_launch("k_wino23");
}

template <int TILE, int TB, int NW, int KC>
bool run_fused(const float* in, int N, int H, int W, int Cin, const float* w, const float* bias,
               int Cout, float* out, int act, hipStream_t s) {
    constexpr int A = Wino<TILE>::A;
    constexpr int P = A * A;
    int tH = (H + TILE - 1) / TILE, tW = (W + TILE - 1) / TILE;
    long long T = (long long)N * tH * tW;
    int Cinp = (Cin + KC - 1) / KC * KC;
    Scratch U((size_t)P * Cout * Cinp * sizeof(float), s);
    if (!U.p) return false;
    ACFUN_LAUNCH("k_wino_filter_t", k_wino_filter_t<TILE>, dim3((Cinp * Cout + 255) / 256), dim3(256), 0, s, w,
                       Cin, Cinp, Cout, U.as<float>());
    if (!check_launch("k_wino_filter_t")) return false;
    dim3 grid((unsigned)((T + TB - 1) / TB), (Cout + 16 * NW - 1) / (16 * NW));
    ACFUN_LAUNCH("k_wino_fused", (k_wino_fused<TILE, TB, NW, KC>), grid, dim3(64 * NW), 0, s, in, U.as<float>(),
                       bias, out, N, H, W, Cin, Cinp, Cout, tH, tW, act);
    return check_launch("k_wino_fused");
}

}  // namespace

bool wino43_filter(const float* w, int Cin, int Cout, float* U, hipStream_t s) {
    const int Cinp = (Cin + 15) / 16 * 16;
    ACFUN_LAUNCH("k_wino_filter_t", (k_wino_filter_c8<4>), dim3((Cout + 7) / 8, Cinp / 8), dim3(64), 0, s, w,
                 Cin, Cout, U);
    return check_launch("k_wino_filter_t");
}

int wino23_plan(int N, int H, int W, int Cin, int Cout, const void* in) {
    return wino23_plan_impl(N, H, W, Cin, Cout, in);
}

size_t wino23_filter_bytes(int Cin, int Cout) {
    return (size_t)16 * Cout * ((Cin + 15) / 16 * 16) * sizeof(float);
}

bool wino23_filter(const float* w, int Cin, int Cout, int plan, float* U, hipStream_t s) {
    return wino23_filter_impl(w, Cin, Cout, plan, U, s);
}

bool winograd_f32(int tile, const float* in, int N, int H, int W, int Cin, const float* w,
                  const float* bias, int Cout, float* out, int act, hipStream_t s, const float* Upre) {
    if (N <= 0 || H <= 0 || W <= 0) return true;
    if (tile == 4) {
        bool done = false;
        if (!run_wino43(in, N, H, W, Cin, w, bias, Cout, out, act, s, &done)) return false;
        if (done) return true;
        return run_fused<4, 16, 4, 8>(in, N, H, W, Cin, w, bias, Cout, out, act, s);
    }
    return run_wino23(in, N, H, W, Cin, w, bias, Cout, out, act, s, Upre);
}

bool winograd_route_f32(int tile, const float* in, int N, int H, int W, int Cin, const float* w,
                        const float* bias, int Cout, float* out, int act, hipStream_t s,
                        const float* Upre) {
    // F(4,3) runs on its unit kernel (k_wino43p) where it applies.  Elsewhere
    // the F(2,3) unit kernels take the F(4,3) route too: measured on MI355X at
    // BASELINE config 2(b) they take about half the time of k_wino_fused<4>.
    if (tile == 4 && N > 0) {
        bool done = false;
        if (!run_wino43(in, N, H, W, Cin, w, bias, Cout, out, act, s, &done)) return false;
        if (done) return true;
    }
    const int tW = (W + 1) / 2, tH = (H + 1) / 2;
    const bool small = tH >= 3 && tH <= 4 && tW >= 3 && tW <= 4 && Cin >= 32;
    const bool unit23 = Cin % 4 == 0 && ((uintptr_t)in & 15u) == 0 && (tW >= 6 || small);
    if (tile == 4 && unit23) tile = 2;
    // Other images too narrow for the unit kernels: the implicit GEMM on the
    // LDS-DMA engine.  (Images of at most 4 x 4 tiles, such as ResNet-50's
    // 7 x 7 stage, run units of two images' tile blocks.)
    ConvShape g{N, H, W, Cin, 3, 3, 1, 1, H, W};
    if (!unit23 && conv32_ok(g, Cout, in, w)) return conv32_f32(g, in, w, bias, Cout, out, act, s);
    return winograd_f32(tile, in, N, H, W, Cin, w, bias, Cout, out, act, s, tile == 2 ? Upre : nullptr);
}

}  // namespace acfun
