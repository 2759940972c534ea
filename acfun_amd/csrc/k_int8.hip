// k_int8.hip -- int8 convolution/GEMM on CDNA4 int8 MFMA, bit-exact with the
// reference's AVX-512 VNNI host.
//
// The reference (src/conv_int8.cpp:63-148) quantizes activations to u8 with
// zero point 128 and multiplies u8 x s8 into i32.  Here the activation byte is
// stored as s8 = u8 - 128 (an exact bijection; a padded tap, u8 128, becomes
// s8 0), so the products run on s8 x s8 -> i32 MFMA and
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
// Kernels.  The convolution routes (acfun_conv2d_int8 and its direct/Winograd
// entries) run k_i8mm: an LDS-DMA staged implicit GEMM on
// v_mfma_i32_32x32x32_i8 whose epilogue forms the per-channel factors from
// the device scalars.  Scales never visit the host: absmax (in the same launch
// as the per-call weight preparation) -> quantize (which reduces the absmax
// partials into the scalars) -> k_i8mm are queued back to back.  The u8-input
// GEMM entries (acfun_gemm_int8*, acfun_conv1x1_int8) and operands too large
// for k_i8mm's 32-bit offsets run k_igemm_i8 (register-staged,
// v_mfma_i32_16x16x64_i8).
#include "i8mm.hpp"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <memory>
#include <mutex>

namespace acfun {
namespace {

typedef int i4 __attribute__((ext_vector_type(4)));

constexpr int IBK = 128;       // k bytes per LDS tile (two MFMA k-steps of 64)
constexpr int ILD = IBK + 16;  // padded LDS row (bytes): rows 36 banks apart


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

// Block blk of nblk: max|x| over its grid-stride share into part[blk] (same
// NaN rule as k_absmax).  Each lane keeps four independent 16-byte loads in
// flight per iteration.
__device__ void absmax_block(const float* __restrict__ x, size_t n, float* __restrict__ part,
                             int blk, int nblk) {
    float m = 0.0f;
    const size_t nth = (size_t)nblk * 256;
    const size_t i0 = (size_t)blk * 256 + threadIdx.x;
    auto upd = [&](float v) { float a = fabsf(v); m = a > m ? a : m; };
    if ((((uintptr_t)x) & 15u) == 0) {
        const float4* x4 = (const float4*)x;
        const size_t n4 = n / 4;
        size_t i = i0;
        for (; i + 3 * nth < n4; i += 4 * nth) {
            float4 v0 = x4[i], v1 = x4[i + nth], v2 = x4[i + 2 * nth], v3 = x4[i + 3 * nth];
            upd(v0.x); upd(v0.y); upd(v0.z); upd(v0.w);
            upd(v1.x); upd(v1.y); upd(v1.z); upd(v1.w);
            upd(v2.x); upd(v2.y); upd(v2.z); upd(v2.w);
            upd(v3.x); upd(v3.y); upd(v3.z); upd(v3.w);
        }
        for (; i < n4; i += nth) { float4 v = x4[i]; upd(v.x); upd(v.y); upd(v.z); upd(v.w); }
        for (size_t k = n4 * 4 + i0; k < n; k += nth) upd(x[k]);
    } else {
        for (size_t k = i0; k < n; k += nth) upd(x[k]);
    }
    for (int off = 32; off > 0; off >>= 1) {
        float o = __shfl_xor(m, off, 64);
        m = o > m ? o : m;
    }
    __shared__ float red[4];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < 4; ++k) m = red[k] > m ? red[k] : m;
        part[blk] = m;
    }
}

// Activation quantization into s8 = u8 - 128 (k_quant_act's rules), 16
// channels of one pixel per lane and one 16-byte store.  Every block first
// reduces the absmax partials to the tensor's max|x| and forms inv_s =
// 127/max (src/conv_int8.cpp:78-81); block 0 also writes the device scalars
// scal = {inv_s, sa = max/127, zero flag, max}.  MODE 0: RNE; 2: the
// Winograd route's rule.  The grid is bounded (the partials are reduced by at
// most that many blocks) and strides over the groups, each lane loading its
// next group while the current one is converted and stored.
template <int MODE>
__global__ __launch_bounds__(256) void k_quant16(const float* __restrict__ x, long long pix,
                                                 int Cin, int Cinp, int8_t* __restrict__ q,
                                                 const float* __restrict__ part, int nparts,
                                                 float* __restrict__ scal, int cvec) {
    const int groups = Cinp >> 4;
    const long long total = pix * groups, stride = (long long)gridDim.x * 256;
    const bool vec = (Cin & 3) == 0 && (((uintptr_t)x) & 15u) == 0;
    auto load = [&](long long g, float* v) {
        const long long pp = g / groups;
        const int c0 = (int)(g - pp * groups) * 16;
        const float* src = x + pp * Cin + c0;
        if (vec && c0 + 16 <= Cin) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float4 f = ((const float4*)src)[k];
                v[4 * k] = f.x; v[4 * k + 1] = f.y; v[4 * k + 2] = f.z; v[4 * k + 3] = f.w;
            }
        } else {
#pragma unroll
            for (int k = 0; k < 16; ++k) v[k] = c0 + k < Cin ? src[k] : 0.0f;
        }
    };
    // the first group's values load while the partials are reduced
    long long g = (long long)blockIdx.x * 256 + threadIdx.x;
    float v[16];
    if (g < total) load(g, v);
    float m = 0.0f;
    for (int i = threadIdx.x; i < nparts; i += 256) { float a = part[i]; m = a > m ? a : m; }
    for (int off = 32; off > 0; off >>= 1) {
        float o = __shfl_xor(m, off, 64);
        m = o > m ? o : m;
    }
    __shared__ float red[4];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    float maxa = red[0];
    for (int k = 1; k < 4; ++k) maxa = red[k] > maxa ? red[k] : maxa;
    const bool zero = maxa < 1e-12f;
    const float inv_s = 127.0f / maxa;
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        scal[0] = inv_s;
        scal[1] = maxa / 127.0f;
        scal[2] = zero ? 1.0f : 0.0f;
        scal[3] = maxa;
    }
    for (; g < total; g += stride) {
        const long long pp = g / groups;
        const int c0 = (int)(g - pp * groups) * 16;
        unsigned w[4] = {0u, 0u, 0u, 0u};
        if (!zero) {
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const int c = c0 + k;
                int out = 0;
                if (c < Cin) {
                    const float t = __fmul_rn(v[k], inv_s);
                    int r;
                    if (MODE == 0) r = x86_cvt(rintf(t));
                    else if (c < cvec) r = x86_cvt(truncf(__fadd_rn(t, copysignf(0.5f, t))));
                    else r = x86_lround(t);
                    out = x86_u8(r, 128) - 128;
                }
                w[k >> 2] |= ((unsigned)out & 0xffu) << (8 * (k & 3));
            }
        }
        if (g + stride < total) load(g + stride, v);
        *(i4*)(q + pp * Cinp + c0) = i4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
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
        if (mode == 0) r = x86_cvt(rintf(t));
        else if (c < cvec) r = x86_cvt(truncf(__fadd_rn(t, copysignf(0.5f, t))));
        else r = x86_lround(t);
        out = (int8_t)(x86_u8(r, 128) - 128);
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
        int r = (c < cvec) ? x86_cvt(truncf(__fadd_rn(t, copysignf(0.5f, t)))) : x86_lround(t);
        out = (int8_t)(x86_u8(r, 128) - 128);
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
__device__ void prep_row(const int8_t* __restrict__ wq, int taps, int Cin, int Cinp, int N,
                         int8_t* __restrict__ Bt, int ldb, int* __restrict__ Sw, int n) {
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

__global__ __launch_bounds__(256) void k_prep_weights(const int8_t* __restrict__ wq, int taps,
                                                      int Cin, int Cinp, int N,
                                                      int8_t* __restrict__ Bt, int ldb,
                                                      int* __restrict__ Sw) {
    prep_row(wq, taps, Cin, Cinp, N, Bt, ldb, Sw, blockIdx.x);
}

__global__ __launch_bounds__(256) void k_absmax_part(const float* __restrict__ x, size_t n,
                                                     float* __restrict__ part) {
    absmax_block(x, n, part, blockIdx.x, gridDim.x);
}

// The activation absmax (blocks < nb) and, in the same launch, the per-call
// weight preparation (one block per output channel after them).
__global__ __launch_bounds__(256) void k_absmax_prep(const float* __restrict__ x, size_t n,
                                                     float* __restrict__ part, int nb,
                                                     const int8_t* __restrict__ wq, int taps,
                                                     int Cin, int Cinp, int N,
                                                     int8_t* __restrict__ Bt, int ldb,
                                                     int* __restrict__ Sw) {
    if ((int)blockIdx.x < nb) absmax_block(x, n, part, blockIdx.x, nb);
    else prep_row(wq, taps, Cin, Cinp, N, Bt, ldb, Sw, blockIdx.x - nb);
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
        // ((int)lroundf, then the clamp: |w / s| <= 127 apart from NaN, which gives 0)
        int v = x86_lround(w[(long long)k * N + j] / s);
        v = v > 127 ? 127 : (v < -128 ? -128 : v);
        wq[(long long)k * N + j] = (int8_t)v;
    }
}

// acfun_quantize_u8 (RNE rule).
__global__ void k_quant_u8(const float* __restrict__ x, uint8_t* __restrict__ out, size_t n,
                           float inv_s, int zp) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float t = __fmul_rn(x[i], inv_s);
    out[i] = (uint8_t)x86_u8(x86_cvt(rintf(t)), zp);
}

// The s8 requantization of y [M][N], the fp32 output (activation applied) of a
// k_i8mm pass that also wrote its per-workgroup maxima of |y| (parts): the
// values and forms of k_i8mm's s8 pass, so the same result bit for bit.
// max from the partials, q = clamp(form(y * 127/max)) per 16 columns (rule 0:
// RNE; rule 1: add-then-truncate below N & ~15, lroundf's half-away above,
// NaN converted as the reference's x86 code does), columns N..ldq-1 and an
// all-zero y give 0, s_out = max/127 (0 for an all-zero y).  Bounded grid.
__global__ __launch_bounds__(256) void k_requant_s8(const float* __restrict__ y, int M, int N,
                                                    int8_t* __restrict__ q, int ldq,
                                                    const float* __restrict__ parts, int nparts,
                                                    float* __restrict__ s_out, int rule) {
    const int groups = ldq >> 4, cvec = N & ~15;
    const bool vec = (N & 3) == 0;
    const long long total = (long long)M * groups, stride = (long long)gridDim.x * 256;
    auto load = [&](long long gi, float* v) {
        const long long r = gi / groups;
        const int c0 = (int)(gi - r * groups) * 16;
        const float* src = y + r * N + c0;
        if (vec && c0 + 16 <= N) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float4 f = ((const float4*)src)[k];
                v[4 * k] = f.x; v[4 * k + 1] = f.y; v[4 * k + 2] = f.z; v[4 * k + 3] = f.w;
            }
        } else {
#pragma unroll
            for (int k = 0; k < 16; ++k) v[k] = c0 + k < N ? src[k] : 0.0f;
        }
    };
    // the first group's values load while the partials are reduced
    long long gi = (long long)blockIdx.x * 256 + threadIdx.x;
    float v[16];
    if (gi < total) load(gi, v);
    float m = 0.0f;
    for (int i = threadIdx.x; i < nparts; i += 256) { const float a = parts[i]; m = a > m ? a : m; }
    for (int off = 32; off > 0; off >>= 1) {
        const float o = __shfl_xor(m, off, 64);
        m = o > m ? o : m;
    }
    __shared__ float red[4];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    float maxa = red[0];
    for (int k = 1; k < 4; ++k) maxa = red[k] > maxa ? red[k] : maxa;
    const bool qzero = maxa < 1e-12f;            // as src/conv_int8.cpp:78 for the consumer
    const float qinv = 127.0f / maxa;
    if (blockIdx.x == 0 && threadIdx.x == 0) s_out[0] = qzero ? 0.0f : maxa / 127.0f;
    for (; gi < total; gi += stride) {
        const long long r = gi / groups;
        const int c0 = (int)(gi - r * groups) * 16;
        unsigned w[4] = {0u, 0u, 0u, 0u};
        if (!qzero) {
            const int form = rule == 0 ? 0 : (c0 < cvec ? 1 : 2);
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const float t = __fmul_rn(v[k], qinv);
                float rq = form == 0 ? rintf(t)
                         : form == 1 ? truncf(__fadd_rn(t, copysignf(0.5f, t)))
                                     : (t != t ? 0.0f : roundf(t));
                rq = fminf(fmaxf(rq, -128.0f), 127.0f);
                const int qv = c0 + k < N ? (int)rq : 0;
                w[k >> 2] |= ((unsigned)qv & 0xffu) << (8 * (k & 3));
            }
        }
        *(uint4*)(q + r * ldq + c0) = make_uint4(w[0], w[1], w[2], w[3]);
        if (gi + stride < total) load(gi + stride, v);
    }
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

// k_i8mm tile choice.  ACFUN_I8_TILE="BMxBNxNST" overrides the tile and
// ACFUN_I8_GRID=<workgroups per CU> the persistent grid (0: one tile per
// workgroup); both exist for tile sweeps.
I8Tile pick_i8mm_tile(int M, int N, int K) {
    // the overrides, read once per process (thread-safe initialization)
    struct Env { bool forced = false; I8Tile ft{64, 64, 3, 0}; int grid_cap = 3; };
    static const Env env = [] {
        Env v;
        if (const char* e = getenv("ACFUN_I8_TILE")) {
            int a, b, c;
            if (sscanf(e, "%dx%dx%d", &a, &b, &c) == 3 && (a == 64 || a == 128) &&
                (b == 64 || b == 128) && c >= 2 && c <= 4) {
                v.ft = I8Tile{a, b, c, 0};
                v.forced = true;
            }
        }
        if (const char* e = getenv("ACFUN_I8_GRID")) v.grid_cap = atoi(e);
        return v;
    }();
    const bool forced = env.forced;
    const I8Tile ft = env.ft;
    const int grid_cap = env.grid_cap;
    I8Tile t;
    if (forced) {
        t = ft;
    } else {
        // Measured on configs 3a/3b and the ResNet-50 int8 model: 64 x 64 tiles
        // with three stages in three persistent workgroups per CU (each runs
        // its tiles back to back, the next tile's chunks loading during the
        // current one's) beat larger tiles, two stages and one tile per
        // workgroup: the short K loops leave a one-tile workgroup too little
        // work to cover its launch, its first loads and its epilogue.
        (void)M; (void)N; (void)K;
        t = I8Tile{64, 64, 3, 0};
    }
    t.per_cu = grid_cap;
    return t;
}

// Whether k_i8mm's 32-bit buffer offsets cover the operands.
bool i8mm_fits(long long a_bytes, long long n, int ldb) {
    return a_bytes < 0x7fffffffll && n * ldb < 0x7fffffffll;
}

// The addressing mode k_i8mm uses for p's A operand.
int i8mm_am(const I8M& p) {
    const int KH = p.K / p.Cinp / p.KW;
    const bool small = p.KW <= 8 && KH <= 4;    // the fast modes' tap bitmask: 4 rows x 8 columns
    if (small && p.Cinp % 128 == 0) return AM_C128;
    if (small && p.Cinp == 64) return AM_C64;
    return AM_GEN;
}

// Tile-search candidates (kind "i8mm", the fp32-output kernel): 64 x 64 with 2
// or 3 stages, 128 x 64, 64 x 128 (3 stages), 128 x 128 (2 stages).
constexpr int kI8NC = 5;
I8Tile i8mm_cand(int c, int per_cu) {
    static const int t[kI8NC][3] = {{64, 64, 2}, {64, 64, 3}, {128, 64, 3}, {64, 128, 3}, {128, 128, 2}};
    return I8Tile{t[c][0], t[c][1], t[c][2], per_cu};
}

// The replay the tile search times for an int8 conv shape: constant s8
// activations and weights, zero scales (EPI_GEMM), fp32 output.
TuneMaker i8mm_maker(const I8M& q, int am) {
    I8M g = q;
    return [g, am]() -> TuneRunner {
        hipStream_t s = lib_stream();
        const size_t cb = (size_t)g.M * g.N * 4;
        if ((size_t)g.a_bytes + g.b_bytes + cb > ((size_t)2 << 30)) return TuneRunner();
        auto a = std::make_shared<Scratch>(g.a_bytes, s);
        auto b = std::make_shared<Scratch>(g.b_bytes, s);
        auto c = std::make_shared<Scratch>(cb, s);
        auto v = std::make_shared<Scratch>((size_t)(3 * g.N + 64) * 4, s);   // ws, bias, Sw, scal
        if (!a->p || !b->p || !c->p || !v->p || hipMemsetAsync(a->p, 0x11, g.a_bytes, s) != hipSuccess ||
            hipMemsetAsync(b->p, 0x11, g.b_bytes, s) != hipSuccess ||
            hipMemsetAsync(v->p, 0, (size_t)(3 * g.N + 64) * 4, s) != hipSuccess)
            return TuneRunner();
        return [=](int cand, hipStream_t st) {
            I8M p = g;
            p.A = a->as<int8_t>(); p.Bt = b->as<int8_t>(); p.Cf = c->as<float>(); p.ldc = p.N;
            float* vf = v->as<float>();
            p.ws = vf; p.bias = vf + p.N; p.Sw = (const int*)(vf + 2 * p.N); p.scal = vf + 3 * p.N;
            p.s_in = nullptr; p.alpha = p.beta = nullptr; p.res = nullptr; p.amax = nullptr;
            p.epi = EPI_GEMM; p.act = 0; p.vec = 1;
            const I8Tile d = pick_i8mm_tile(p.M, p.N, p.K);
            const I8Tile t = cand < 0 ? d : i8mm_cand(cand, d.per_cu);
            return launch_i8mm_f32(p, t, am, st);
        };
    };
}

bool launch_i8mm(I8M& p, hipStream_t s) {
    if (p.M <= 0 || p.N <= 0) return true;
    I8Tile t = pick_i8mm_tile(p.M, p.N, p.K);
    auto al16 = [](const void* q) { return ((uintptr_t)q & 15u) == 0; };
    p.vec = al16(p.Cf) && p.ldc % 4 == 0 && (!p.res || (al16(p.res) && p.ldr % 4 == 0));
    const int am = i8mm_am(p);
    if (!getenv("ACFUN_I8_TILE")) {
        const std::vector<int> key{am, p.M, p.N, p.K, p.H, p.W, p.Cinp, p.KW, p.stride, p.pad, p.OH, p.OW};
        bool rec = false;
        const int c = tune_lookup("i8mm", key, kI8NC, &rec);
        if (rec) tune_record("i8mm", key, kI8NC, i8mm_maker(p, am));
        if (c >= 0) t = i8mm_cand(c, t.per_cu);
    }
    return launch_i8mm_f32(p, t, am, s);
}

// A requantized s8 output.  Without ybuf: the first pass writes the
// per-workgroup maxima of the float output into parts (kAmaxParts floats), the
// second recomputes the tile and stores clamp(rule(v * 127/max)) with s_out =
// max/127.  With ybuf (M x N floats): one fp32 pass into ybuf with the maxima,
// then k_requant_s8.
bool launch_i8mm_rq(I8M& p, float* parts, float* ybuf, hipStream_t s) {
    if (p.M <= 0 || p.N <= 0) return true;
    if (ybuf) {
        // One pass: the fp32 output (activation applied) and its per-workgroup
        // maxima, then k_requant_s8 over it.  The values requantized are the ones
        // the s8 pass would form, so the result is the same bit for bit.
        I8M f = p;
        f.Cf = ybuf;
        f.ldc = p.N;
        f.res = nullptr;
        f.amax = parts;
        f.Cq = nullptr;
        if (!launch_i8mm(f, s)) return false;
        const long long groups = (long long)p.M * (p.ldq / 16);
        const long long blocks = std::min((groups + 255) / 256, 8ll * num_cus());
        ACFUN_LAUNCH("k_requant_s8", k_requant_s8, dim3((unsigned)blocks), dim3(256), 0, s, ybuf, p.M,
                     p.N, p.Cq, p.ldq, parts, f.grid, p.s_out, p.rule);
        return check_launch("k_requant_s8");
    }
    I8Tile t = pick_i8mm_tile(p.M, p.N, p.K);
    t.bm = t.bn = 64;                           // the s8 epilogue stages 64 x 64 tiles
    if (t.per_cu <= 0) t.per_cu = 3;
    p.vec = 0;
    p.res = nullptr;
    p.amax = parts;
    const int am = i8mm_am(p);
    if (!launch_i8mm_q8(p, t, am, OUT_AMAX, s)) return false;
    p.amax = nullptr;
    p.qparts = parts;
    p.nqparts = i8mm_grid(p, t);
    return launch_i8mm_q8(p, t, am, OUT_Q8, s);
}

// Fills the convolution part of k_i8mm's arguments.
void i8mm_conv(I8M& p, const int8_t* q, const ConvShape& g, int Cinp, const int8_t* bt, int ldb,
               int Cout) {
    p.A = q; p.Bt = bt; p.M = g.N * g.OH * g.OW; p.N = Cout; p.K = g.KH * g.KW * Cinp;
    p.ldb = ldb; p.H = g.H; p.W = g.W; p.Cinp = Cinp; p.KW = g.KW; p.stride = g.stride;
    p.pad = g.pad; p.OH = g.OH; p.OW = g.OW;
    p.a_bytes = (unsigned)((long long)g.N * g.H * g.W * Cinp);
    p.b_bytes = (unsigned)((long long)Cout * ldb);
    p.ldc = Cout;
}

// Prepared weights: Bt [N][ldb] and Sw [N] in pooled device memory.
struct PrepW {
    Scratch bt, sw;
    int ldb = 0;
};
bool alloc_weights(int taps, int Cinp, int N, hipStream_t s, PrepW& w) {
    w.ldb = rup(taps * Cinp, 128);
    w.bt = Scratch((size_t)N * w.ldb, s);
    w.sw = Scratch((size_t)N * sizeof(int), s);
    return w.bt.p && w.sw.p;
}
bool prep_weights(const int8_t* wq, int taps, int Cin, int Cinp, int N, hipStream_t s, PrepW& w) {
    if (!alloc_weights(taps, Cinp, N, s, w)) return false;
    ACFUN_LAUNCH("k_prep_weights", k_prep_weights, dim3(N), dim3(256), 0, s, wq, taps, Cin, Cinp, N,
                       w.bt.as<int8_t>(), w.ldb, w.sw.as<int>());
    return check_launch("k_prep_weights");
}

}  // namespace

bool quantize_weights_dev(const float* w, int K, int N, float* scales, int8_t* wq, hipStream_t s) {
    if (K <= 0 || N <= 0) return true;
    ACFUN_LAUNCH("k_quant_weights", k_quant_weights, g1(N), dim3(256), 0, s, w, K, N, scales, wq);
    return check_launch("k_quant_weights");
}

bool quantize_u8_dev(const float* in, uint8_t* out, size_t n, float inv_s, int zp, hipStream_t s) {
    if (!n) return true;
    ACFUN_LAUNCH("k_quant_u8", k_quant_u8, g1((long long)n), dim3(256), 0, s, in, out, n, inv_s, zp);
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
    ACFUN_LAUNCH("k_u8_to_s8", k_u8_to_s8, g1(pix * Cinp), dim3(256), 0, s, inQ, pix, g.Cin, Cinp, q.as<int8_t>());
    if (!check_launch("k_u8_to_s8")) return false;
    PrepW w;
    if (!prep_weights(wq, g.KH * g.KW, g.Cin, Cinp, Cout, s, w)) return false;
    if (i8mm_fits(pix * Cinp, Cout, w.ldb)) {
        I8M p{};
        i8mm_conv(p, q.as<int8_t>(), g, Cinp, w.bt.as<int8_t>(), w.ldb, Cout);
        p.epi = EPI_GEMM; p.act = act; p.Sw = w.sw.as<int>(); p.alpha = alpha; p.beta = beta;
        p.Cf = out;
        return launch_i8mm(p, s);
    }
    I8P p{};
    p.A = q.as<int8_t>(); p.Bt = w.bt.as<int8_t>(); p.M = g.N * g.OH * g.OW; p.N = Cout;
    p.K = g.KH * g.KW * Cinp; p.ldb = w.ldb;
    p.H = g.H; p.W = g.W; p.Cinp = Cinp; p.KW = g.KW; p.stride = g.stride; p.pad = g.pad;
    p.OH = g.OH; p.OW = g.OW; p.epi = EPI_GEMM; p.act = act; p.Sw = w.sw.as<int>();
    p.alpha = alpha; p.beta = beta; p.Cf = out; p.ldc = Cout;
    return launch_i8(p, true, true, s);
}

namespace {
// p (the conv, fp32 factors set up) with its output requantized to s8 as o
// describes: two k_i8mm passes, or for K >= 512 one fp32 pass into a scratch
// buffer and k_requant_s8 (launch_i8mm_rq).
bool launch_q8out(I8M& p, const I8Out& o, Arena& ar, hipStream_t s) {
    if (o.ldo % 16 != 0 || o.ldo < p.N || (((uintptr_t)o.q) & 15u) ||
        (long long)p.M * o.ldo >= 0x7fffffffll) {
        set_error("conv2d_int8: bad s8 output layout");
        return false;
    }
    float* parts = (float*)ar.get((size_t)kAmaxParts * sizeof(float));
    if (!parts) return false;
    p.Cf = nullptr; p.res = nullptr; p.amax = nullptr;
    p.Cq = o.q; p.ldq = o.ldo; p.rule = o.rule; p.s_out = o.s_out;
    float* ybuf = nullptr;
    if (p.K >= 512 || !o.recompute) {
        ybuf = (float*)ar.get((size_t)p.M * p.N * sizeof(float));
        if (!ybuf) return false;
    }
    return launch_i8mm_rq(p, parts, ybuf, s);
}

// acfun_conv2d_int8 on device with every temporary taken from `ar`.
bool conv2d_int8_run(const float* in, const ConvShape& g, const int8_t* wq, const float* ws,
                     const float* bias, int Cout, float* out, int act, hipStream_t s, Arena& ar,
                     bool region, const I8Weights* pre, const float* res, float* amax_out,
                     const float* amax_in, I8Quant* shared = nullptr,
                     const I8Out* q8out = nullptr) {
    if (g.OH <= 0 || g.OW <= 0 || Cout <= 0 || g.N <= 0) return true;
    const bool wino = g.KH == 3 && g.KW == 3 && g.stride == 1 && g.pad == 1 && g.H >= 3 &&
                      g.W >= 3 && g.Cin >= 4 && Cout >= 4;
    int Cinp = rup(g.Cin, 16);
    long long pix = (long long)g.N * g.H * g.W;
    size_t inN = (size_t)pix * g.Cin;
    const int8_t* bt;
    const int* sw;
    int8_t* nbt = nullptr;       // weights prepared by this call
    int* nsw = nullptr;
    int ldb;
    const bool prepared = pre && pre->bt && pre->taps == g.KH * g.KW && pre->Cin == g.Cin &&
                          pre->N == Cout;
    if (prepared) {
        bt = pre->bt; sw = pre->sw; ldb = pre->ldb;
    } else {
        ldb = rup(g.KH * g.KW * Cinp, 128);
        nbt = (int8_t*)ar.get((size_t)Cout * ldb);
        nsw = (int*)ar.get((size_t)Cout * sizeof(int));
        if (!nbt || !nsw) return false;
        bt = nbt; sw = nsw;
    }
    if (i8mm_fits(pix * Cinp, Cout, ldb)) {
        // absmax partials -> quantize (reduces them, writes the scalars) -> k_i8mm,
        // whose epilogue forms the per-channel factors from the scalars
        constexpr int kParts = 512;
        const int mode = wino ? 2 : 0;
        // A shared tensor already quantized with this rule: no absmax, no quantizer.
        const bool reuse = shared && shared->ready && shared->mode == mode;
        if (!reuse && !q8out && !wino && (Cout + 63) / 64 <= kI8AmaxParts && conv_smallc_ok(g, Cout, in)) {
            // a stem (7x7 or 3x3 on 3 channels): the absmax partials (unless the
            // producer supplied them), the input quantized once as dense s8, then
            // k_i8stem with the [K][Cout] weights as they are
            float* part = nullptr;
            int nb = 0;
            if (!amax_in) {
                nb = (int)((inN / 4 + 1023) / 1024);
                nb = nb < 1 ? 1 : (nb > kParts ? kParts : nb);
                part = (float*)ar.get((size_t)kParts * sizeof(float));
                if (!part) return false;
                ACFUN_LAUNCH("k_absmax_prep", k_absmax_prep, dim3(nb), dim3(256), 0, s, in, inN, part, nb, wq,
                             g.KH * g.KW, g.Cin, Cinp, Cout, nbt, ldb, nsw);
                if (!check_launch("k_absmax_prep")) return false;
            }
            int8_t* q8 = (int8_t*)ar.get((size_t)inN);
            if (!q8) return false;
            return conv_i8stem(g, in, wq, ws, bias, Cout, out, act, amax_in ? amax_in : part,
                               amax_in ? kAmaxParts : nb, amax_out, nullptr, q8, s);
        }
        if (!reuse && !q8out && !wino && g.KH == 1 && g.KW == 1 && g.stride == 1 && g.pad == 0 &&
            Cinp <= kI8Q1MaxCinp && i8q1_route(Cout)) {
            // 1x1 / stride 1 / pad 0 into at most 64 channels: the absmax
            // partials (unless the producer supplied them) with the weight
            // preparation, then k_i8q1, which quantizes the rows as it stages
            // them (a shared tensor is left to its other readers)
            float* part = nullptr;
            int nb = 0;
            if (!amax_in) {
                nb = (int)((inN / 4 + 1023) / 1024);
                nb = nb < 1 ? 1 : (nb > kParts ? kParts : nb);
                part = (float*)ar.get((size_t)kParts * sizeof(float));
                if (!part) return false;
            }
            if (nb + (prepared ? 0 : Cout) > 0) {
                ACFUN_LAUNCH("k_absmax_prep", k_absmax_prep, dim3(nb + (prepared ? 0 : Cout)), dim3(256), 0, s,
                             in, inN, part, nb, wq, 1, g.Cin, Cinp, Cout, nbt, ldb, nsw);
                if (!check_launch("k_absmax_prep")) return false;
            }
            I8Q1 a{};
            a.x = in; a.Bt = bt; a.Sw = sw; a.ws = ws; a.bias = bias;
            a.part = amax_in ? amax_in : part;
            a.nparts = amax_in ? kAmaxParts : nb;
            a.scal = nullptr;
            a.res = res; a.Cf = out; a.amax = amax_out;
            a.M = (int)pix; a.N = Cout; a.Cin = g.Cin; a.Cinp = Cinp; a.ldb = ldb;
            a.ldc = Cout; a.ldr = Cout; a.act = act;
            return launch_i8q1(a, s);
        }
        float* scal = reuse || shared ? nullptr : (float*)ar.get((size_t)(8 + kParts) * sizeof(float));
        int8_t* q = reuse || shared ? nullptr : (int8_t*)ar.get((size_t)pix * Cinp);
        float* part = nullptr;
        if (shared) {
            q = shared->q;
            scal = shared->scal;
            if (!reuse && !amax_in) {
                part = (float*)ar.get((size_t)kParts * sizeof(float));
                if (!part) return false;
            }
        } else {
            part = scal ? scal + 8 : nullptr;
        }
        if (!scal || !q) return false;
        long long n4 = (long long)(inN / 4);
        // With amax_in (the producing layer folded its output's max|x| in) the
        // absmax pass is skipped and the quantizer reads that one "partial".
        int nb = amax_in || reuse ? 0 : (int)((n4 + 1023) / 1024);
        if (!amax_in && !reuse) nb = nb < 1 ? 1 : (nb > kParts ? kParts : nb);
        if (nb + (prepared ? 0 : Cout) > 0) {
            ACFUN_LAUNCH("k_absmax_prep", k_absmax_prep, dim3(nb + (prepared ? 0 : Cout)), dim3(256), 0, s, in,
                               inN, part, nb, wq, g.KH * g.KW, g.Cin, Cinp, Cout, nbt, ldb, nsw);
            if (!check_launch("k_absmax_prep")) return false;
        }
        if (!reuse) {
            const long long groups = pix * (Cinp / 16);
            const long long qb = std::min((groups + 255) / 256, 8ll * num_cus());
            if (mode == 0)
                ACFUN_LAUNCH("k_quant16", k_quant16<0>, dim3((unsigned)qb), dim3(256), 0, s, in, pix, g.Cin,
                             Cinp, q, amax_in ? amax_in : part, amax_in ? kAmaxParts : nb, scal,
                             g.Cin & ~15);
            else
                ACFUN_LAUNCH("k_quant16", k_quant16<2>, dim3((unsigned)qb), dim3(256), 0, s, in, pix, g.Cin,
                             Cinp, q, amax_in ? amax_in : part, amax_in ? kAmaxParts : nb, scal,
                             g.Cin & ~15);
            if (!check_launch("k_quant16")) return false;
            if (shared) {
                shared->mode = mode;
                shared->ready = true;
            }
        }
        I8M p{};
        i8mm_conv(p, q, g, Cinp, bt, ldb, Cout);
        p.act = act; p.scal = scal; p.ws = ws; p.bias = bias; p.Cf = out;
        p.res = res; p.ldr = Cout;
        p.amax = amax_out;
        if (wino) p.epi = EPI_WINO;
        else { p.epi = EPI_GEMM; p.Sw = sw; }
        if (q8out) return launch_q8out(p, *q8out, ar, s);
        return launch_i8mm(p, s);
    }
    if (q8out) {
        set_error("conv2d_int8: an s8 output needs operands within 32-bit offsets");
        return false;
    }
    // (operands past 32-bit offsets: amax_in is not needed, the absmax pass
    // below runs; amax_out is filled by a pass over the output at the end)
    if (region) {
        set_error("conv2d_int8: operands past 32-bit offsets need the allocating entry point");
        return false;
    }
    if (res) {
        set_error("conv2d_int8: a fused residual needs operands within 32-bit offsets");
        return false;
    }
    if (!prepared) {
        ACFUN_LAUNCH("k_prep_weights", k_prep_weights, dim3(Cout), dim3(256), 0, s, wq, g.KH * g.KW, g.Cin,
                           Cinp, Cout, nbt, ldb, nsw);
        if (!check_launch("k_prep_weights")) return false;
    }
    // device block: [0..3] scalars+maxbits, then alpha, beta, alpha_w
    float* scal = (float*)ar.get((size_t)(8 + 3 * Cout) * sizeof(float));
    int8_t* q = (int8_t*)ar.get((size_t)pix * Cinp);
    if (!scal || !q) return false;
    unsigned* bits = (unsigned*)(scal + 4);
    float* alpha = scal + 8;
    float* beta = alpha + Cout;
    float* alpha_w = beta + Cout;
    ACFUN_LAUNCH("k_fill_u32", k_fill_u32, dim3(1), dim3(64), 0, s, bits, 1, 0u);
    if (!check_launch("k_fill_u32")) return false;
    int nb = (int)((inN / 4 + 255) / 256);
    nb = nb < 1 ? 1 : (nb > 4 * num_cus() ? 4 * num_cus() : nb);
    ACFUN_LAUNCH("k_absmax", k_absmax, dim3(nb), dim3(256), 0, s, in, inN, bits);
    if (!check_launch("k_absmax")) return false;
    ACFUN_LAUNCH("k_int8_params", k_int8_params, g1(Cout), dim3(256), 0, s, bits, ws, bias, sw,
                       Cout, alpha, beta, alpha_w, scal);
    if (!check_launch("k_int8_params")) return false;
    ACFUN_LAUNCH("k_quant_act", k_quant_act, g1(pix * Cinp), dim3(256), 0, s, in, pix, g.Cin, Cinp,
                       q, scal, wino ? 2 : 0, g.Cin & ~15);
    if (!check_launch("k_quant_act")) return false;
    I8P p{};
    p.A = q; p.Bt = bt; p.M = g.N * g.OH * g.OW; p.N = Cout;
    p.K = g.KH * g.KW * Cinp; p.ldb = ldb;
    p.H = g.H; p.W = g.W; p.Cinp = Cinp; p.KW = g.KW; p.stride = g.stride; p.pad = g.pad;
    p.OH = g.OH; p.OW = g.OW; p.act = act; p.scal = scal; p.Cf = out; p.ldc = Cout;
    if (wino) {
        p.epi = EPI_WINO; p.alpha = alpha_w; p.bias = bias;
    } else {
        p.epi = EPI_GEMM; p.alpha = alpha; p.beta = beta; p.Sw = sw;
    }
    if (!launch_i8(p, true, true, s)) return false;
    if (amax_out) {       // the partials by a pass over the output (nb <= kAmaxParts)
        const size_t outN = (size_t)g.N * g.OH * g.OW * Cout;
        int nbo = (int)((outN / 4 + 1023) / 1024);
        nbo = nbo < 1 ? 1 : (nbo > kAmaxParts ? kAmaxParts : nbo);
        ACFUN_LAUNCH("k_absmax_part", k_absmax_part, dim3(nbo), dim3(256), 0, s, out, outN, amax_out);
        if (!check_launch("k_absmax_part")) return false;
    }
    return true;
}

// The file-scope scratch of the allocation-free entry point: one copy per
// device, for the life of the process.  Host code never passes `scratch`
// itself to a kernel: its device address on the current device comes from
// hipGetSymbolAddress (noalloc_region), taken once per device.
constexpr size_t kNoAllocBytes = size_t(64) << 20;
__device__ __align__(256) char scratch[kNoAllocBytes];

constexpr int kNoAllocDev = 16;
void* g_scratch_ptr[kNoAllocDev] = {};
std::mutex g_scratch_mu;

void* noalloc_region() {
    int d = -1;
    if (!check(hipGetDevice(&d), "hipGetDevice")) return nullptr;
    if (d < 0 || d >= kNoAllocDev) {
        set_error("device %d: no scratch slot", d);
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[d]) {
        void* ptr = nullptr;
        if (!check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)"))
            return nullptr;
        g_scratch_ptr[d] = ptr;
    }
    return g_scratch_ptr[d];
}
}  // namespace

bool conv2d_int8_dev(const float* in, const ConvShape& g, const int8_t* wq, const float* ws,
                     const float* bias, int Cout, float* out, int act, hipStream_t s,
                     const I8Weights* pre, const float* res, float* amax_out,
                     const float* amax_in, I8Quant* shared, const I8Out* q8out) {
    Arena ar(s);
    const long long pix = (long long)g.N * g.H * g.W;
    if (shared && !i8mm_fits(pix * rup(g.Cin, 16), Cout, rup(g.KH * g.KW * rup(g.Cin, 16), 128)))
        shared = nullptr;   // (the large-operand path quantizes per call)
    return conv2d_int8_run(in, g, wq, ws, bias, Cout, out, act, s, ar, false, pre, res, amax_out,
                           amax_in, shared, q8out);
}

bool conv2d_int8_s8in_dev(const int8_t* q, const float* s_in, const ConvShape& g,
                          const I8Weights& pre, const float* ws, const float* bias, int Cout,
                          float* out, int act, hipStream_t s, const float* res, float* amax_out,
                          const I8Out* q8out) {
    if (g.OH <= 0 || g.OW <= 0 || Cout <= 0 || g.N <= 0) return true;
    const int Cinp = rup(g.Cin, 16);
    const long long pix = (long long)g.N * g.H * g.W;
    if (!pre.bt || pre.taps != g.KH * g.KW || pre.Cin != g.Cin || pre.N != Cout ||
        !i8mm_fits(pix * Cinp, Cout, pre.ldb) || (((uintptr_t)q) & 15u)) {
        set_error("conv2d_int8_s8in: needs prepared weights, a 16-byte aligned s8 input and "
                  "operands within 32-bit offsets");
        return false;
    }
    const bool wino = g.KH == 3 && g.KW == 3 && g.stride == 1 && g.pad == 1 && g.H >= 3 &&
                      g.W >= 3 && g.Cin >= 4 && Cout >= 4;
    I8M p{};
    i8mm_conv(p, q, g, Cinp, pre.bt, pre.ldb, Cout);
    p.act = act; p.s_in = s_in; p.ws = ws; p.bias = bias;
    if (wino) p.epi = EPI_WINO;
    else { p.epi = EPI_GEMM; p.Sw = pre.sw; }
    if (q8out) {
        Arena ar(s);
        return launch_q8out(p, *q8out, ar, s);
    }
    p.Cf = out; p.res = res; p.ldr = Cout; p.amax = amax_out;
    return launch_i8mm(p, s);
}

size_t i8_quant_bytes(long long pix, int Cin) {
    return Arena::aligned((size_t)pix * rup(Cin, 16)) + 8 * sizeof(float);
}

size_t conv2d_int8_noalloc_need(const ConvShape& g, int Cout) {
    const int Cinp = rup(g.Cin, 16);
    const size_t ldb = (size_t)rup(g.KH * g.KW * Cinp, 128);
    return Arena::aligned((size_t)Cout * ldb) + Arena::aligned((size_t)Cout * sizeof(int)) +
           Arena::aligned((size_t)(8 + 512) * sizeof(float)) +
           Arena::aligned((size_t)g.N * g.H * g.W * Cinp);
}

size_t conv2d_int8_noalloc_max() { return kNoAllocBytes; }

bool conv2d_int8_noalloc(const float* in, const ConvShape& g, const int8_t* wq, const float* ws,
                         const float* bias, int Cout, float* out, int act, hipStream_t s) {
    if (g.OH <= 0 || g.OW <= 0 || Cout <= 0 || g.N <= 0) return true;
    const size_t need = conv2d_int8_noalloc_need(g, Cout);
    if (need > kNoAllocBytes) {
        set_error("conv2d_int8_noalloc: this shape needs %zu bytes of scratch, more than the "
                  "%zu-byte static region (use acfun_dev_conv2d_int8)", need, kNoAllocBytes);
        return false;
    }
    void* region = noalloc_region();
    if (!region) return false;
    Arena ar(s, region, kNoAllocBytes);
    return conv2d_int8_run(in, g, wq, ws, bias, Cout, out, act, s, ar, true, nullptr, nullptr,
                           nullptr, nullptr);
}

namespace {
// [pix][Cin] s8 -> [pix][Cinp] s8 with zero channel padding, and back.
__global__ void k_s8_repad(const int8_t* __restrict__ x, long long pix, int Cx, int Cy,
                           int8_t* __restrict__ y) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= pix * Cy) return;
    long long p = i / Cy;
    int c = (int)(i - p * Cy);
    y[i] = c < Cx ? x[p * Cx + c] : (int8_t)0;
}
}  // namespace

bool conv2d_int8_q8_dev(const int8_t* q, int ldq_in, const float* s_in, const ConvShape& g,
                        const int8_t* wq, const float* ws, const float* bias, int Cout,
                        int8_t* out, int ldo, float* s_out, int act, int rule, hipStream_t s,
                        const I8Weights* pre) {
    if (g.OH <= 0 || g.OW <= 0 || Cout <= 0 || g.N <= 0) return true;
    const int Cinp = rup(g.Cin, 16);
    if (ldq_in != Cinp || ldo % 16 != 0 || ldo < Cout || (((uintptr_t)q | (uintptr_t)out) & 15u)) {
        set_error("conv2d_int8_q8: s8 rows must be 16-byte aligned and padded to 16 channels");
        return false;
    }
    const long long pix = (long long)g.N * g.H * g.W;
    const bool wino = g.KH == 3 && g.KW == 3 && g.stride == 1 && g.pad == 1 && g.H >= 3 &&
                      g.W >= 3 && g.Cin >= 4 && Cout >= 4;
    Arena ar(s);
    const int8_t* bt;
    const int* sw;
    int ldb;
    const bool prepared = pre && pre->bt && pre->taps == g.KH * g.KW && pre->Cin == g.Cin &&
                          pre->N == Cout;
    if (prepared) {
        bt = pre->bt; sw = pre->sw; ldb = pre->ldb;
    } else {
        ldb = rup(g.KH * g.KW * Cinp, 128);
        int8_t* nbt = (int8_t*)ar.get((size_t)Cout * ldb);
        int* nsw = (int*)ar.get((size_t)Cout * sizeof(int));
        if (!nbt || !nsw) return false;
        ACFUN_LAUNCH("k_prep_weights", k_prep_weights, dim3(Cout), dim3(256), 0, s, wq, g.KH * g.KW, g.Cin,
                           Cinp, Cout, nbt, ldb, nsw);
        if (!check_launch("k_prep_weights")) return false;
        bt = nbt; sw = nsw;
    }
    if (!i8mm_fits(pix * Cinp, Cout, ldb) ||
        (long long)g.N * g.OH * g.OW * ldo >= 0x7fffffffll) {
        set_error("conv2d_int8_q8: operands past 32-bit offsets");
        return false;
    }
    float* parts = (float*)ar.get((size_t)kAmaxParts * sizeof(float));
    if (!parts) return false;
    I8M p{};
    i8mm_conv(p, q, g, Cinp, bt, ldb, Cout);
    p.act = act; p.s_in = s_in; p.ws = ws; p.bias = bias;
    p.Cq = out; p.ldq = ldo; p.rule = rule; p.s_out = s_out;
    if (wino) p.epi = EPI_WINO;
    else { p.epi = EPI_GEMM; p.Sw = sw; }
    // Long K: store the fp32 output once and requantize it (a pass over 9 bytes
    // per output) rather than recompute every tile in a second pass.
    float* ybuf = nullptr;
    if (p.K >= 512) {
        ybuf = (float*)ar.get((size_t)p.M * p.N * sizeof(float));
        if (!ybuf) return false;
    }
    return launch_i8mm_rq(p, parts, ybuf, s);
}

bool conv2d_int8_q8_api(const int8_t* in, const float* s_in, const ConvShape& g,
                        const int8_t* wq, const float* ws, const float* bias, int Cout,
                        int8_t* out, float* s_out, int act, int rule, hipStream_t s) {
    if (g.OH <= 0 || g.OW <= 0 || Cout <= 0 || g.N <= 0) return true;
    if (rule != 0 && rule != 1) {
        set_error("acfun_dev_conv2d_int8_q: out_rule must be 0 or 1 (got %d)", rule);
        return false;
    }
    const int Cinp = rup(g.Cin, 16), Coutp = rup(Cout, 16);
    const long long pix = (long long)g.N * g.H * g.W, pixo = (long long)g.N * g.OH * g.OW;
    Arena ar(s);
    const int8_t* qin = in;
    if (g.Cin != Cinp || ((uintptr_t)in & 15u)) {
        int8_t* t = (int8_t*)ar.get((size_t)pix * Cinp);
        if (!t) return false;
        ACFUN_LAUNCH("k_s8_repad", k_s8_repad, g1(pix * Cinp), dim3(256), 0, s, in, pix, g.Cin, Cinp, t);
        if (!check_launch("k_s8_repad")) return false;
        qin = t;
    }
    const bool direct = Cout == Coutp && ((uintptr_t)out & 15u) == 0;
    int8_t* qo = out;
    if (!direct) {
        qo = (int8_t*)ar.get((size_t)pixo * Coutp);
        if (!qo) return false;
    }
    if (!conv2d_int8_q8_dev(qin, Cinp, s_in, g, wq, ws, bias, Cout, qo, Coutp, s_out, act, rule,
                            s, nullptr))
        return false;
    if (!direct) {
        ACFUN_LAUNCH("k_s8_repad", k_s8_repad, g1(pixo * Cout), dim3(256), 0, s, qo, pixo, Coutp, Cout, out);
        if (!check_launch("k_s8_repad")) return false;
    }
    return true;
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
    ACFUN_LAUNCH("k_quant_act_inv", k_quant_act_inv, g1(pix * Cinp), dim3(256), 0, s, in, pix, Cin, Cinp,
                       q.as<int8_t>(), inv_s, Cin & ~15);
    if (!check_launch("k_quant_act_inv")) return false;
    ACFUN_LAUNCH("k_alpha_w", k_alpha_w, g1(Cout), dim3(256), 0, s, ws, s_in, Cout, aw.as<float>());
    if (!check_launch("k_alpha_w")) return false;
    PrepW w;
    if (!prep_weights(wq, 9, Cin, Cinp, Cout, s, w)) return false;
    if (i8mm_fits(pix * Cinp, Cout, w.ldb)) {
        ConvShape g{N, H, W, Cin, 3, 3, 1, 1, H, W};
        I8M p{};
        i8mm_conv(p, q.as<int8_t>(), g, Cinp, w.bt.as<int8_t>(), w.ldb, Cout);
        p.epi = EPI_WINO; p.act = act; p.alpha = aw.as<float>(); p.bias = bias; p.Cf = out;
        return launch_i8mm(p, s);
    }
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
    w.ldb = rup(taps * Cinp, 128);
    if (!check(hipMalloc((void**)&w.bt, (size_t)N * w.ldb), "hipMalloc(int8 weights)") ||
        !check(hipMalloc((void**)&w.sw, (size_t)N * sizeof(int)), "hipMalloc(int8 sums)")) {
        i8_release(w);
        return false;
    }
    w.taps = taps; w.Cin = Cin; w.N = N;
    ACFUN_LAUNCH("k_prep_weights", k_prep_weights, dim3(N), dim3(256), 0, s, wq, taps, Cin, Cinp, N, w.bt,
                       w.ldb, w.sw);
    return check_launch("k_prep_weights");
}

void i8_release(I8Weights& w) {
    if (w.bt) (void)hipFree(w.bt);
    if (w.sw) (void)hipFree(w.sw);
    w = I8Weights{};
}

}  // namespace acfun
