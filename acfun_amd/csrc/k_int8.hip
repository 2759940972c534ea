// k_int8.hip -- int8 convolution/GEMM on CDNA4 int8 MFMA, bit-exact with the
// reference's AVX-512 VNNI host.
//
// The reference (src/conv_int8.cpp:63-148) quantizes activations to u8 with
// zero point 128 and multiplies u8 x s8 into i32.  Here the activation byte is
// stored as s8 = u8 - 128 (an exact bijection; a padded tap, u8 128, becomes
// s8 0), so the products run on v_mfma_i32_16x16x64_i8 (s8 x s8 -> i32) and
//     acc_u = sum(u8 * w) = acc_s + 128 * Sw[j],   Sw[j] = sum_k w[k][j]
// recovers the reference's accumulator exactly (wrapping i32 both sides).
//
// Epilogues (one per reference route):
//   EPI_I32  : C = acc_u                                     (src/gemm_int8.cpp:11-50)
//   EPI_GEMM : out = fl(fl((float)acc_u * alpha[j]) + beta[j]), ReLU = max_ps
//              (src/gemm_int8_avx512.cpp:113-136, -ffp-contract=off)
//   EPI_WINO : out = fmaf((float)(4*acc_s), fl(fl(s_in*0.25)*ws[j]), bias[j]), ReLU = max_ps.
//              The reference's int8 Winograd F(2,3) (src/winograd_int8.cpp:127-171) computes
//              AT*T4*AT^T = 4*acc_s exactly (the integer transforms lose nothing and
//              the zero-point correction of :204,226-229 cancels the 128 offset), so a
//              direct s8 implicit GEMM reproduces it bit for bit.
//
// Scales never visit the host: absmax -> params -> quantize -> GEMM are
// queued back to back, the per-tensor scale living in a small device block.
#include "rt.hpp"

namespace acfun {
namespace {

typedef int i4 __attribute__((ext_vector_type(4)));

constexpr int IBK = 128;       // k bytes per LDS tile (two MFMA k-steps of 64)
constexpr int ILD = IBK + 16;  // padded LDS row (bytes): rows 36 banks apart

enum { EPI_I32 = 0, EPI_GEMM = 1, EPI_WINO = 2 };

struct I8P {
    const int8_t* A;   // s8 (or u8 with a_xor) activations
    const int8_t* Bt;  // weights transposed [N][ldb], zero beyond the real K
    int M, N, K, lda, ldb, a_xor;
    // implicit conv (CONV = true): A is NHWC [N][H][W][Cinp]
    int H, W, Cinp, KW, stride, pad, OH, OW;
    int epi, act;
    const int* Sw;
    const float* alpha;
    const float* beta;
    const float* bias;
    const float* scal;  // device scalars: [0] inv_s [1] sa [2] zero flag (nullable)
    int32_t* C32;
    float* Cf;
    int ldc;
};

__device__ __forceinline__ float vmax(float a, float b) { return a > b ? a : b; }

template <int BM, int BN, bool CONV, bool VA>
__global__ __launch_bounds__(256) void k_igemm_i8(I8P p) {
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int FM = WM / 16, FN = WN / 16;
    constexpr int ACH = BM * (IBK / 16) / 256;  // 16-byte chunks per thread
    constexpr int BCH = BN * (IBK / 16) / 256;
    __shared__ __attribute__((aligned(16))) int8_t sA[2][BM * ILD];
    __shared__ __attribute__((aligned(16))) int8_t sB[2][BN * ILD];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int ntiles = (p.K + IBK - 1) / IBK;
    const int cch = tid & 7;  // chunk index within a 128-byte k tile

    long long abase[ACH];
    int aih0[ACH], aiw0[ACH], arow[ACH];
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
        int r = (tid >> 3) + i * 32;
        arow[i] = r;
        int m = m0 + r;
        if (CONV) {
            int mm = m < p.M ? m : 0;
            int hw = p.OH * p.OW;
            int n = mm / hw, rem = mm - n * hw;
            int oh = rem / p.OW, ow = rem - oh * p.OW;
            abase[i] = (long long)n * p.H * p.W * p.Cinp;
            aih0[i] = oh * p.stride - p.pad;
            aiw0[i] = ow * p.stride - p.pad;
        } else {
            abase[i] = (long long)m * p.lda;
            aih0[i] = aiw0[i] = 0;
        }
    }
    i4 ra[ACH], rb[BCH];
    const unsigned xr = (unsigned)p.a_xor * 0x01010101u;

    auto load_a = [&](int k0) {
        int k = k0 + cch * 16;
        int kh = 0, kw = 0, ic = 0;
        if (CONV) {
            int tap = k / p.Cinp;
            ic = k - tap * p.Cinp;
            kh = tap / p.KW;
            kw = tap - kh * p.KW;
        }
#pragma unroll
        for (int i = 0; i < ACH; ++i) {
            i4 v = {0, 0, 0, 0};
            int m = m0 + arow[i];
            if (m < p.M && k < p.K) {
                if (CONV) {
                    int ih = aih0[i] + kh, iw = aiw0[i] + kw;
                    if (ih >= 0 && ih < p.H && iw >= 0 && iw < p.W)
                        v = *(const i4*)(p.A + abase[i] + ((long long)ih * p.W + iw) * p.Cinp + ic);
                } else if (VA) {
                    v = *(const i4*)(p.A + abase[i] + k);
                } else {
                    unsigned char b[16];
#pragma unroll
                    for (int e = 0; e < 16; ++e)
                        b[e] = (k + e < p.K) ? (unsigned char)p.A[abase[i] + k + e] : (unsigned char)(p.a_xor);
                    v = *(const i4*)b;
                }
                v.x ^= xr; v.y ^= xr; v.z ^= xr; v.w ^= xr;
            }
            ra[i] = v;
        }
    };
    auto load_b = [&](int k0) {
        int k = k0 + cch * 16;
#pragma unroll
        for (int i = 0; i < BCH; ++i) {
            int n = n0 + (tid >> 3) + i * 32;
            i4 v = {0, 0, 0, 0};
            if (n < p.N && k < p.ldb) v = *(const i4*)(p.Bt + (long long)n * p.ldb + k);
            rb[i] = v;
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < ACH; ++i) *(i4*)&sA[buf][arow[i] * ILD + cch * 16] = ra[i];
#pragma unroll
        for (int i = 0; i < BCH; ++i) *(i4*)&sB[buf][((tid >> 3) + i * 32) * ILD + cch * 16] = rb[i];
    };

    i4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = i4{0, 0, 0, 0};

    if (ntiles > 0) {
        load_a(0);
        load_b(0);
        store(0);
        __syncthreads();
    }
    const int lr = lane & 15, lk = (lane >> 4) * 16;
    for (int t = 0; t < ntiles; ++t) {
        const int buf = t & 1;
        const bool more = t + 1 < ntiles;
        if (more) {
            load_a((t + 1) * IBK);
            load_b((t + 1) * IBK);
        }
#pragma unroll
        for (int ks = 0; ks < IBK / 64; ++ks) {
            i4 fa[FM], fb[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i)
                fa[i] = *(const i4*)&sA[buf][(wm0 + i * 16 + lr) * ILD + ks * 64 + lk];
#pragma unroll
            for (int j = 0; j < FN; ++j)
                fb[j] = *(const i4*)&sB[buf][(wn0 + j * 16 + lr) * ILD + ks * 64 + lk];
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
        if (more) store(buf ^ 1);
        __syncthreads();
    }

    const bool zero = p.scal && p.scal[2] != 0.0f;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        int n = n0 + wn0 + j * 16 + lr;
        if (n >= p.N) continue;
        int corr = p.Sw ? 128 * p.Sw[n] : 0;
        float al = 0.f, be = 0.f;
        if (p.epi == EPI_GEMM) { al = p.alpha[n]; be = p.beta[n]; }
        if (p.epi == EPI_WINO) { al = p.alpha[n]; be = p.bias ? p.bias[n] : 0.0f; }
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                int m = m0 + wm0 + i * 16 + (lane >> 4) * 4 + r;
                if (m >= p.M) continue;
                int a = acc[i][j][r];
                long long o = (long long)m * p.ldc + n;
                if (p.epi == EPI_I32) {
                    p.C32[o] = (int)((unsigned)a + (unsigned)corr);
                } else if (p.epi == EPI_GEMM) {
                    float v;
                    if (zero) v = 0.0f;
                    else {
                        int u = (int)((unsigned)a + (unsigned)corr);
                        v = __fadd_rn(__fmul_rn((float)u, al), be);
                        v = act_apply(v, p.act);
                    }
                    p.Cf[o] = v;
                } else {
                    float v;
                    if (zero) v = 0.0f;
                    else {
                        v = fmaf((float)(4LL * (long long)a), al, be);
                        v = act_apply(v, p.act);
                    }
                    p.Cf[o] = v;
                }
            }
    }
}

// ---------------------------------------------------------------- helpers

// max|x| into *bits (as the bit pattern of a non-negative float).  NaN never
// wins a comparison, as with std::max(maxa, fabs(x)) in src/conv_int8.cpp:77.
__global__ void k_absmax(const float* __restrict__ x, size_t n, unsigned* __restrict__ bits) {
    float m = 0.0f;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i0 = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if ((((uintptr_t)x) & 15u) == 0) {
        const float4* x4 = (const float4*)x;
        size_t n4 = n / 4;
        for (size_t i = i0; i < n4; i += stride) {
            float4 v = x4[i];
            float a = fabsf(v.x); m = a > m ? a : m;
            a = fabsf(v.y); m = a > m ? a : m;
            a = fabsf(v.z); m = a > m ? a : m;
            a = fabsf(v.w); m = a > m ? a : m;
        }
        for (size_t i = n4 * 4 + i0; i < n; i += stride) { float a = fabsf(x[i]); m = a > m ? a : m; }
    } else {
        for (size_t i = i0; i < n; i += stride) { float a = fabsf(x[i]); m = a > m ? a : m; }
    }
    for (int off = 32; off > 0; off >>= 1) {
        float o = __shfl_xor(m, off, 64);
        m = o > m ? o : m;
    }
    __shared__ float red[16];
    int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < (int)(blockDim.x >> 6); ++k) m = red[k] > m ? red[k] : m;
        atomicMax(bits, __float_as_uint(m));
    }
}

__global__ void k_fill_u32(unsigned* p, int n, unsigned v) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

// Per-tensor scale and per-channel factors in the reference's operation order
// (src/conv_int8.cpp:78-81,100-107; src/winograd_int8.cpp:155).
__global__ void k_int8_params(const unsigned* __restrict__ bits, const float* __restrict__ ws,
                              const float* __restrict__ bias, const int* __restrict__ Sw, int Cout,
                              float* __restrict__ alpha, float* __restrict__ beta,
                              float* __restrict__ alpha_w, float* __restrict__ scal) {
    float maxa = __uint_as_float(*bits);
    float inv_s = 127.0f / maxa;
    float sa = maxa / 127.0f;
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        scal[0] = inv_s;
        scal[1] = sa;
        scal[2] = (maxa < 1e-12f) ? 1.0f : 0.0f;
    }
    int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= Cout) return;
    float a = __fmul_rn(sa, ws[j]);
    alpha[j] = a;
    float t = __fmul_rn(a, 128.0f);
    t = __fmul_rn(t, (float)Sw[j]);
    beta[j] = __fsub_rn(bias ? bias[j] : 0.0f, t);
    alpha_w[j] = __fmul_rn(__fmul_rn(sa, 0.25f), ws[j]);
}

// Activation quantization into s8 = u8 - 128, channels padded to Cinp with 0.
// mode 0: RNE (src/int8_quantize_avx512.cpp:15-20)
// mode 2: Winograd route: channels < cvec use trunc(t + copysign(0.5,t)) with the
//         add rounded in float (src/winograd_int8.cpp:306-319), the rest lroundf (:321-325)
__global__ void k_quant_act(const float* __restrict__ x, long long pix, int Cin, int Cinp,
                            int8_t* __restrict__ q, const float* __restrict__ scal, int mode,
                            int cvec) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= pix * Cinp) return;
    long long p = i / Cinp;
    int c = (int)(i - p * Cinp);
    int8_t out = 0;
    if (c < Cin && scal[2] == 0.0f) {
        float t = __fmul_rn(x[p * Cin + c], scal[0]);
        int r;
        if (mode == 0) r = (int)rintf(t);
        else if (c < cvec) r = (int)truncf(__fadd_rn(t, copysignf(0.5f, t)));
        else r = (int)roundf(t);
        int v = r + 128;
        v = v < 0 ? 0 : (v > 255 ? 255 : v);
        out = (int8_t)(v - 128);
    }
    q[i] = out;
}

// Winograd-route quantization with caller-supplied inv_s (acfun_winograd_conv3x3_int8).
__global__ void k_quant_act_inv(const float* __restrict__ x, long long pix, int Cin, int Cinp,
                                int8_t* __restrict__ q, float inv_s, int cvec) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= pix * Cinp) return;
    long long p = i / Cinp;
    int c = (int)(i - p * Cinp);
    int8_t out = 0;
    if (c < Cin) {
        float t = __fmul_rn(x[p * Cin + c], inv_s);
        int r = (c < cvec) ? (int)truncf(__fadd_rn(t, copysignf(0.5f, t))) : (int)roundf(t);
        int v = r + 128;
        v = v < 0 ? 0 : (v > 255 ? 255 : v);
        out = (int8_t)(v - 128);
    }
    q[i] = out;
}

// fl(fl(s_in*0.25f)*ws[j]): the Winograd-route multiplier (src/winograd_int8.cpp:155).
__global__ void k_alpha_w(const float* __restrict__ ws, float s_in, int Cout, float* __restrict__ aw) {
    int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j < Cout) aw[j] = __fmul_rn(__fmul_rn(s_in, 0.25f), ws[j]);
}

// u8 NHWC -> s8 with channel padding (for the quantized-input API entries).
__global__ void k_u8_to_s8(const uint8_t* __restrict__ x, long long pix, int Cin, int Cinp,
                           int8_t* __restrict__ q) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= pix * Cinp) return;
    long long p = i / Cinp;
    int c = (int)(i - p * Cinp);
    q[i] = c < Cin ? (int8_t)(x[p * Cin + c] ^ 0x80u) : (int8_t)0;
}

// wq [taps*Cin][N] -> Bt [N][ldb], row k' = tap*Cinp + ic (zero for ic >= Cin
// and for k' >= taps*Cinp), and Sw[n] = sum_k wq[k][n] (exact i32).  One
// 256-thread block per output channel n: the row is written contiguously and
// summed in the same pass.
__global__ __launch_bounds__(256) void k_prep_weights(const int8_t* __restrict__ wq, int taps,
                                                      int Cin, int Cinp, int N,
                                                      int8_t* __restrict__ Bt, int ldb,
                                                      int* __restrict__ Sw) {
    const int n = blockIdx.x;
    int sum = 0;
    for (int kp = threadIdx.x; kp < ldb; kp += 256) {
        int tap = kp / Cinp, ic = kp - tap * Cinp;
        int8_t v = 0;
        if (tap < taps && ic < Cin) v = wq[((long long)tap * Cin + ic) * N + n];
        Bt[(long long)n * ldb + kp] = v;
        sum += v;
    }
    __shared__ int red[4];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = sum;
    __syncthreads();
    if (threadIdx.x == 0) Sw[n] = red[0] + red[1] + red[2] + red[3];
}

// acfun_quantize_weights (src/conv_int8.cpp:24-37): one lane per column.
__global__ void k_quant_weights(const float* __restrict__ w, int K, int N, float* __restrict__ sc,
                                int8_t* __restrict__ wq) {
    int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= N) return;
    float maxa = 0.0f;
    for (int k = 0; k < K; ++k) { float a = fabsf(w[(long long)k * N + j]); maxa = maxa < a ? a : maxa; }
    float s = maxa / 127.0f;
    if (s <= 0.0f) s = 1.0f;
    sc[j] = s;
    for (int k = 0; k < K; ++k) {
        float r = roundf(w[(long long)k * N + j] / s);
        int v = r > 127.0f ? 127 : (r < -128.0f ? -128 : (int)r);
        wq[(long long)k * N + j] = (int8_t)v;
    }
}

// acfun_quantize_u8 (RNE rule).
__global__ void k_quant_u8(const float* __restrict__ x, uint8_t* __restrict__ out, size_t n,
                           float inv_s, int zp) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float t = __fmul_rn(x[i], inv_s);
    int v = (int)rintf(t) + zp;
    out[i] = (uint8_t)(v < 0 ? 0 : (v > 255 ? 255 : v));
}

inline dim3 g1(long long n) { return dim3((unsigned)((n + 255) / 256)); }
inline int rup(int x, int a) { return (x + a - 1) / a * a; }

// Tile choice: the largest tile that still yields at least one workgroup per CU.
void pick_tile(int M, int N, int* bm, int* bn) {
    const int cus = num_cus();
    const int cand[4][2] = {{128, 128}, {128, 64}, {64, 128}, {64, 64}};
    for (auto& c : cand) {
        long long t = (long long)((M + c[0] - 1) / c[0]) * ((N + c[1] - 1) / c[1]);
        if (t >= cus) { *bm = c[0]; *bn = c[1]; return; }
    }
    *bm = 64; *bn = 64;
}

template <bool CONV, bool VA>
bool launch_i8_v(const I8P& p, int bm, int bn, hipStream_t s) {
    dim3 grid((p.N + bn - 1) / bn, (p.M + bm - 1) / bm);
    if (bm == 128 && bn == 128) ACFUN_LAUNCH("k_igemm_i8", (k_igemm_i8<128, 128, CONV, VA>), grid, dim3(256), 0, s, p);
    else if (bm == 128) ACFUN_LAUNCH("k_igemm_i8", (k_igemm_i8<128, 64, CONV, VA>), grid, dim3(256), 0, s, p);
    else if (bn == 128) ACFUN_LAUNCH("k_igemm_i8", (k_igemm_i8<64, 128, CONV, VA>), grid, dim3(256), 0, s, p);
    else ACFUN_LAUNCH("k_igemm_i8", (k_igemm_i8<64, 64, CONV, VA>), grid, dim3(256), 0, s, p);
    return check_launch("k_igemm_i8");
}

bool launch_i8(const I8P& p, bool conv, bool va, hipStream_t s) {
    if (p.M <= 0 || p.N <= 0) return true;
    int bm, bn;
    pick_tile(p.M, p.N, &bm, &bn);
    if (conv) return launch_i8_v<true, true>(p, bm, bn, s);
    if (va) return launch_i8_v<false, true>(p, bm, bn, s);
    return launch_i8_v<false, false>(p, bm, bn, s);
}

// Prepared weights: Bt [N][ldb] and Sw [N] in pooled device memory.
struct PrepW {
    Scratch bt, sw;
    int ldb = 0;
};
bool prep_weights(const int8_t* wq, int taps, int Cin, int Cinp, int N, hipStream_t s, PrepW& w) {
    w.ldb = rup(taps * Cinp, 16);
    w.bt = Scratch((size_t)N * w.ldb, s);
    w.sw = Scratch((size_t)N * sizeof(int), s);
    if (!w.bt.p || !w.sw.p) return false;
    hipLaunchKernelGGL(k_prep_weights, dim3(N), dim3(256), 0, s, wq, taps, Cin, Cinp, N,
                       w.bt.as<int8_t>(), w.ldb, w.sw.as<int>());
    return check_launch("k_prep_weights");
}

}  // namespace

bool quantize_weights_dev(const float* w, int K, int N, float* scales, int8_t* wq, hipStream_t s) {
    if (K <= 0 || N <= 0) return true;
    hipLaunchKernelGGL(k_quant_weights, g1(N), dim3(256), 0, s, w, K, N, scales, wq);
    return check_launch("k_quant_weights");
}

bool quantize_u8_dev(const float* in, uint8_t* out, size_t n, float inv_s, int zp, hipStream_t s) {
    if (!n) return true;
    hipLaunchKernelGGL(k_quant_u8, g1((long long)n), dim3(256), 0, s, in, out, n, inv_s, zp);
    return check_launch("k_quant_u8");
}

bool gemm_int8_dev(int M, int N, int K, const uint8_t* A, const int8_t* B, int32_t* C,
                   const float* alpha, const float* beta, float* Cf, int act, hipStream_t s) {
    if (M <= 0 || N <= 0) return true;
    PrepW w;
    if (!prep_weights(B, K, 1, 1, N, s, w)) return false;
    I8P p{};
    p.A = (const int8_t*)A; p.Bt = w.bt.as<int8_t>(); p.M = M; p.N = N; p.K = K; p.lda = K;
    p.ldb = w.ldb; p.a_xor = 0x80; p.Sw = w.sw.as<int>();
    p.epi = C ? EPI_I32 : EPI_GEMM; p.act = act; p.alpha = alpha; p.beta = beta;
    p.C32 = C; p.Cf = Cf; p.ldc = N;
    bool va = (K % 16 == 0) && (((uintptr_t)A & 15u) == 0);
    return launch_i8(p, false, va, s);
}

bool conv1x1_int8_dev(const uint8_t* inQ, int M, int K, int Cout, const int8_t* wq,
                      const float* alpha, const float* beta, float* out, int act, hipStream_t s) {
    return gemm_int8_dev(M, Cout, K, inQ, wq, nullptr, alpha, beta, out, act, s);
}

bool conv_int8_direct_dev(const uint8_t* inQ, const ConvShape& g, const int8_t* wq,
                          const float* alpha, const float* beta, int Cout, float* out, int act,
                          hipStream_t s) {
    if (g.OH <= 0 || g.OW <= 0 || Cout <= 0) return true;
    int Cinp = rup(g.Cin, 16);
    long long pix = (long long)g.N * g.H * g.W;
    Scratch q((size_t)pix * Cinp, s);
    if (!q.p) return false;
    hipLaunchKernelGGL(k_u8_to_s8, g1(pix * Cinp), dim3(256), 0, s, inQ, pix, g.Cin, Cinp, q.as<int8_t>());
    if (!check_launch("k_u8_to_s8")) return false;
    PrepW w;
    if (!prep_weights(wq, g.KH * g.KW, g.Cin, Cinp, Cout, s, w)) return false;
    I8P p{};
    p.A = q.as<int8_t>(); p.Bt = w.bt.as<int8_t>(); p.M = g.N * g.OH * g.OW; p.N = Cout;
    p.K = g.KH * g.KW * Cinp; p.ldb = w.ldb;
    p.H = g.H; p.W = g.W; p.Cinp = Cinp; p.KW = g.KW; p.stride = g.stride; p.pad = g.pad;
    p.OH = g.OH; p.OW = g.OW; p.epi = EPI_GEMM; p.act = act; p.Sw = w.sw.as<int>();
    p.alpha = alpha; p.beta = beta; p.Cf = out; p.ldc = Cout;
    return launch_i8(p, true, true, s);
}

bool conv2d_int8_dev(const float* in, const ConvShape& g, const int8_t* wq, const float* ws,
                     const float* bias, int Cout, float* out, int act, hipStream_t s,
                     const I8Weights* pre) {
    if (g.OH <= 0 || g.OW <= 0 || Cout <= 0 || g.N <= 0) return true;
    const bool wino = g.KH == 3 && g.KW == 3 && g.stride == 1 && g.pad == 1 && g.H >= 3 &&
                      g.W >= 3 && g.Cin >= 4 && Cout >= 4;
    int Cinp = rup(g.Cin, 16);
    long long pix = (long long)g.N * g.H * g.W;
    size_t inN = (size_t)pix * g.Cin;
    // device block: [0..3] scalars+maxbits, then alpha, beta, alpha_w
    Scratch par((size_t)(8 + 3 * Cout) * sizeof(float), s);
    Scratch q((size_t)pix * Cinp, s);
    if (!par.p || !q.p) return false;
    float* scal = par.as<float>();
    unsigned* bits = (unsigned*)(scal + 4);
    float* alpha = scal + 8;
    float* beta = alpha + Cout;
    float* alpha_w = beta + Cout;
    PrepW w;
    const int8_t* bt;
    const int* sw;
    int ldb;
    if (pre && pre->bt && pre->taps == g.KH * g.KW && pre->Cin == g.Cin && pre->N == Cout) {
        bt = pre->bt; sw = pre->sw; ldb = pre->ldb;
    } else {
        if (!prep_weights(wq, g.KH * g.KW, g.Cin, Cinp, Cout, s, w)) return false;
        bt = w.bt.as<int8_t>(); sw = w.sw.as<int>(); ldb = w.ldb;
    }
    hipLaunchKernelGGL(k_fill_u32, dim3(1), dim3(64), 0, s, bits, 1, 0u);
    if (!check_launch("k_fill_u32")) return false;
    int nb = (int)((inN / 4 + 255) / 256);
    nb = nb < 1 ? 1 : (nb > 4 * num_cus() ? 4 * num_cus() : nb);
    hipLaunchKernelGGL(k_absmax, dim3(nb), dim3(256), 0, s, in, inN, bits);
    if (!check_launch("k_absmax")) return false;
    hipLaunchKernelGGL(k_int8_params, g1(Cout), dim3(256), 0, s, bits, ws, bias, sw,
                       Cout, alpha, beta, alpha_w, scal);
    if (!check_launch("k_int8_params")) return false;
    hipLaunchKernelGGL(k_quant_act, g1(pix * Cinp), dim3(256), 0, s, in, pix, g.Cin, Cinp,
                       q.as<int8_t>(), scal, wino ? 2 : 0, g.Cin & ~15);
    if (!check_launch("k_quant_act")) return false;
    I8P p{};
    p.A = q.as<int8_t>(); p.Bt = bt; p.M = g.N * g.OH * g.OW; p.N = Cout;
    p.K = g.KH * g.KW * Cinp; p.ldb = ldb;
    p.H = g.H; p.W = g.W; p.Cinp = Cinp; p.KW = g.KW; p.stride = g.stride; p.pad = g.pad;
    p.OH = g.OH; p.OW = g.OW; p.act = act; p.scal = scal; p.Cf = out; p.ldc = Cout;
    if (wino) {
        p.epi = EPI_WINO; p.alpha = alpha_w; p.bias = bias;
    } else {
        p.epi = EPI_GEMM; p.alpha = alpha; p.beta = beta; p.Sw = sw;
    }
    return launch_i8(p, true, true, s);
}

bool winograd_int8_dev(const float* in, int N, int H, int W, int Cin, const int8_t* wq,
                       const float* ws, const float* bias, int Cout, float s_in, float inv_s,
                       float* out, int act, hipStream_t s) {
    if (N <= 0 || H <= 0 || W <= 0 || Cout <= 0) return true;
    int Cinp = rup(Cin, 16);
    long long pix = (long long)N * H * W;
    Scratch q((size_t)pix * Cinp, s);
    Scratch aw((size_t)Cout * sizeof(float), s);
    if (!q.p || !aw.p) return false;
    hipLaunchKernelGGL(k_quant_act_inv, g1(pix * Cinp), dim3(256), 0, s, in, pix, Cin, Cinp,
                       q.as<int8_t>(), inv_s, Cin & ~15);
    if (!check_launch("k_quant_act_inv")) return false;
    hipLaunchKernelGGL(k_alpha_w, g1(Cout), dim3(256), 0, s, ws, s_in, Cout, aw.as<float>());
    if (!check_launch("k_alpha_w")) return false;
    PrepW w;
    if (!prep_weights(wq, 9, Cin, Cinp, Cout, s, w)) return false;
    I8P p{};
    p.A = q.as<int8_t>(); p.Bt = w.bt.as<int8_t>(); p.M = N * H * W; p.N = Cout;
    p.K = 9 * Cinp; p.ldb = w.ldb;
    p.H = H; p.W = W; p.Cinp = Cinp; p.KW = 3; p.stride = 1; p.pad = 1; p.OH = H; p.OW = W;
    p.act = act; p.Cf = out; p.ldc = Cout; p.epi = EPI_WINO; p.alpha = aw.as<float>(); p.bias = bias;
    return launch_i8(p, true, true, s);
}

bool i8_prepare(const int8_t* wq, int taps, int Cin, int N, I8Weights& w, hipStream_t s) {
    i8_release(w);
    int Cinp = rup(Cin, 16);
    w.ldb = rup(taps * Cinp, 16);
    if (!check(hipMalloc((void**)&w.bt, (size_t)N * w.ldb), "hipMalloc(int8 weights)") ||
        !check(hipMalloc((void**)&w.sw, (size_t)N * sizeof(int)), "hipMalloc(int8 sums)")) {
        i8_release(w);
        return false;
    }
    w.taps = taps; w.Cin = Cin; w.N = N;
    hipLaunchKernelGGL(k_prep_weights, dim3(N), dim3(256), 0, s, wq, taps, Cin, Cinp, N, w.bt,
                       w.ldb, w.sw);
    return check_launch("k_prep_weights");
}

void i8_release(I8Weights& w) {
    if (w.bt) (void)hipFree(w.bt);
    if (w.sw) (void)hipFree(w.sw);
    w = I8Weights{};
}

}  // namespace acfun
