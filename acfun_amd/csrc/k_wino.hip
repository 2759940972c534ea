// k_wino.hip -- Winograd F(2,3) and F(4,3) for 3x3 / stride 1 / pad 1 convs.
//
// Replaces acfun_winograd_conv3x3 (src/winograd.cpp:236-251,
// src/winograd_avx512.cpp:186-250) and acfun_winograd43_conv3x3
// (src/winograd43.cpp:239-250, src/winograd43_avx512.cpp:218-280).  The
// matrices are the standard Lavin & Gray ones the reference uses
// (src/winograd.cpp:9-17, src/winograd43.cpp:33-54):
//   d_hat = BT d BT^T (input tile), g_hat = G g G^T (filter), Y = AT M AT^T.
//
// Pipeline on the device (T = tiles, A = 16 or 36 transform points):
//   1. filter transform  U[a][Cin][Cout]   (per call, like the reference)
//   2. input transform   V[a][T][Cin]      one lane per (tile, channel)
//   3. A independent GEMMs M[a] = V[a] * U[a] on fp32 MFMA (batched launch)
//   4. output transform  Y = AT M AT^T + bias (+ReLU) written straight to NHWC
#include "rt.hpp"

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

// U[a][c][o], weight[(k*Cin + c)*Cout + o] with k = kh*3 + kw.
template <int TILE>
__global__ void k_wino_filter(const float* __restrict__ w, int Cin, int Cout, float* __restrict__ U) {
    constexpr int A = Wino<TILE>::A;
    int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= Cin * Cout) return;
    int c = idx / Cout, o = idx - c * Cout;
    float g[3][3];
#pragma unroll
    for (int kh = 0; kh < 3; ++kh)
#pragma unroll
        for (int kw = 0; kw < 3; ++kw) g[kh][kw] = w[((long long)(kh * 3 + kw) * Cin + c) * Cout + o];
    float gh[A][A];
    Wino<TILE>::f_tf(g, gh);
    long long plane = (long long)Cin * Cout;
#pragma unroll
    for (int i = 0; i < A; ++i)
#pragma unroll
        for (int j = 0; j < A; ++j) U[(i * A + j) * plane + idx] = gh[i][j];
}

// V[a][t][c]: tile t = (n, ty, tx), origin (TILE*ty - 1, TILE*tx - 1).
template <int TILE>
__global__ void k_wino_input(const float* __restrict__ in, int N, int H, int W, int Cin, int tH,
                             int tW, float* __restrict__ V) {
    constexpr int A = Wino<TILE>::A;
    long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    long long T = (long long)N * tH * tW;
    if (idx >= T * Cin) return;
    int c = (int)(idx % Cin);
    long long t = idx / Cin;
    int tx = (int)(t % tW);
    long long r = t / tW;
    int ty = (int)(r % tH);
    int n = (int)(r / tH);
    const float* img = in + (long long)n * H * W * Cin + c;
    float d[A][A];
    int ih0 = ty * TILE - 1, iw0 = tx * TILE - 1;
#pragma unroll
    for (int i = 0; i < A; ++i)
#pragma unroll
        for (int j = 0; j < A; ++j) {
            int ih = ih0 + i, iw = iw0 + j;
            d[i][j] = (ih >= 0 && ih < H && iw >= 0 && iw < W) ? img[((long long)ih * W + iw) * Cin] : 0.f;
        }
    float dh[A][A];
    Wino<TILE>::in_tf(d, dh);
    long long plane = T * Cin;
#pragma unroll
    for (int i = 0; i < A; ++i)
#pragma unroll
        for (int j = 0; j < A; ++j) V[(i * A + j) * plane + idx] = dh[i][j];
}

template <int TILE>
__global__ void k_wino_output(const float* __restrict__ Mm, int N, int OH, int OW, int Cout,
                              int tH, int tW, const float* __restrict__ bias,
                              float* __restrict__ out, int act) {
    constexpr int A = Wino<TILE>::A;
    long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    long long T = (long long)N * tH * tW;
    if (idx >= T * Cout) return;
    int o = (int)(idx % Cout);
    long long t = idx / Cout;
    int tx = (int)(t % tW);
    long long r = t / tW;
    int ty = (int)(r % tH);
    int n = (int)(r / tH);
    long long plane = T * Cout;
    float m[A][A];
#pragma unroll
    for (int i = 0; i < A; ++i)
#pragma unroll
        for (int j = 0; j < A; ++j) m[i][j] = Mm[(i * A + j) * plane + idx];
    float y[TILE][TILE];
    Wino<TILE>::out_tf(m, y);
    float b = bias ? bias[o] : 0.f;
#pragma unroll
    for (int i = 0; i < TILE; ++i)
#pragma unroll
        for (int j = 0; j < TILE; ++j) {
            int oh = ty * TILE + i, ow = tx * TILE + j;
            if (oh < OH && ow < OW) {
                float v = y[i][j] + b;
                if (act == 1) v = v > 0.f ? v : 0.f;
                out[(((long long)n * OH + oh) * OW + ow) * Cout + o] = v;
            }
        }
}

template <int TILE>
bool run_wino(const float* in, int N, int H, int W, int Cin, const float* w, const float* bias,
              int Cout, float* out, int act, hipStream_t s) {
    constexpr int A = Wino<TILE>::A;
    constexpr int P = A * A;
    int tH = (H + TILE - 1) / TILE, tW = (W + TILE - 1) / TILE;
    long long T = (long long)N * tH * tW;
    Scratch U((size_t)P * Cin * Cout * sizeof(float), s);
    Scratch V((size_t)P * T * Cin * sizeof(float), s);
    Scratch Mm((size_t)P * T * Cout * sizeof(float), s);
    if (!U.p || !V.p || !Mm.p) return false;
    hipLaunchKernelGGL(k_wino_filter<TILE>, dim3((Cin * Cout + 255) / 256), dim3(256), 0, s, w,
                       Cin, Cout, U.as<float>());
    if (!check_launch("k_wino_filter")) return false;
    hipLaunchKernelGGL(k_wino_input<TILE>, dim3((unsigned)((T * Cin + 255) / 256)), dim3(256), 0, s,
                       in, N, H, W, Cin, tH, tW, V.as<float>());
    if (!check_launch("k_wino_input")) return false;
    if (!gemm_f32_batched(P, (int)T, Cout, Cin, V.as<float>(), T * Cin, Cin, U.as<float>(),
                          (long long)Cin * Cout, Cout, Mm.as<float>(), T * Cout, Cout, s))
        return false;
    hipLaunchKernelGGL(k_wino_output<TILE>, dim3((unsigned)((T * Cout + 255) / 256)), dim3(256), 0,
                       s, Mm.as<float>(), N, H, W, Cout, tH, tW, bias, out, act);
    return check_launch("k_wino_output");
}

}  // namespace

bool winograd_f32(int tile, const float* in, int N, int H, int W, int Cin, const float* w,
                  const float* bias, int Cout, float* out, int act, hipStream_t s) {
    if (N <= 0 || H <= 0 || W <= 0) return true;
    return tile == 4 ? run_wino<4>(in, N, H, W, Cin, w, bias, Cout, out, act, s)
                     : run_wino<2>(in, N, H, W, Cin, w, bias, Cout, out, act, s);
}

}  // namespace acfun
