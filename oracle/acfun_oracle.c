/*
 * acfun_oracle.c -- CPU restatement of the reference's arithmetic for the
 * convolution/GEMM path.  TEST INFRASTRUCTURE ONLY: it is the checker for the
 * HIP kernels in acfun_amd/ and the "port" CPU baseline.  The product library
 * never links, loads or calls it.
 *
 * Every function cites the reference file:line it restates (paths are relative
 * to the reference repository root).  Where the reference's result depends on
 * the host ISA, this file restates the path an AVX-512F/BW/VNNI host takes
 * (the hosts the reference publishes from and the build container), and says so.
 *
 * Build: see oracle/Makefile (-ffp-contract=off, so every a*b+c below is two
 * roundings unless fmaf() is written explicitly).
 *
 * Pinning (how each function is checked against the compiled reference,
 * oracle/_ref, in tests/test_oracle_pins.py, tests/test_route_pins.py and
 * tests/test_model_pins.py):
 *   - oracle_gemm, oracle_gemm_epi ... bit-exact against acfun_gemm_ref /
 *     acfun_gemm_ref_epi (same loop order); oracle_gemm_f64 and
 *     oracle_conv2d_f64 are the f64 closed forms the fp32 routes are held to.
 *   - oracle_conv2d_route ... per shape, acfun_conv2d of the reference is
 *     bit-identical to the entry point of the route this function names, and
 *     differs from the other routes' results.
 *   - int8 functions, quantizers, oracle_requantize_s8 ... bit-exact against
 *     the reference's own entry points on seeded inputs and exact ties.
 *   - oracle_conv_int8_centered_acc + oracle_wino_int8_epilogue ... the
 *     Winograd identity AT*T4*AT^T = 4*A: together they reproduce the
 *     reference's acfun_winograd_conv3x3_int8 bit for bit.
 *   - oracle_fold_bn ... the folded weights and biases read back exactly from
 *     the reference's own loader + executor (one-hot inputs of 2^30).
 *   - dw / grouped / maxpool / bn ... bit-exact against oracle/_ref.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------------ */
/* fp32 GEMM                                                                */
/* ------------------------------------------------------------------------ */

/* C = A*B, i-k-j order with float accumulation, zero rows of A skipped.
 * Restates acfun_gemm_ref_ld (src/gemm_ref.cpp:5-20). */
EXPORT void oracle_gemm(int M, int N, int K, const float* A, const float* B, float* C) {
    #pragma omp parallel for schedule(static)
    for (int i = 0; i < M; ++i) {
        const float* a = A + (size_t)i * K;
        float* c = C + (size_t)i * N;
        for (int j = 0; j < N; ++j) c[j] = 0.0f;
        for (int k = 0; k < K; ++k) {
            float av = a[k];
            if (av == 0.0f) continue;
            const float* b = B + (size_t)k * N;
            for (int j = 0; j < N; ++j) c[j] += av * b[j];
        }
    }
}

/* GEMM then bias[j] and optional ReLU applied once after the full K
 * reduction.  Restates acfun_gemm_ref_epi (src/gemm_ref.cpp:39-63). */
EXPORT void oracle_gemm_epi(int M, int N, int K, const float* A, const float* B, float* C,
                            const float* bias, int act) {
    oracle_gemm(M, N, K, A, B, C);
    #pragma omp parallel for schedule(static)
    for (int i = 0; i < M; ++i) {
        float* c = C + (size_t)i * N;
        for (int j = 0; j < N; ++j) {
            float v = c[j];
            if (bias) v += bias[j];
            if (act && v < 0.0f) v = 0.0f;
            c[j] = v;
        }
    }
}

/* Exact-math yardstick: the same product accumulated in double.  Not a
 * reference restatement; used to bound the error of both the reference and
 * the GPU (the closed form C = A*B). */
EXPORT void oracle_gemm_f64(int M, int N, int K, const float* A, const float* B, double* C) {
    #pragma omp parallel for schedule(static)
    for (int i = 0; i < M; ++i) {
        double* c = C + (size_t)i * N;
        for (int j = 0; j < N; ++j) c[j] = 0.0;
        for (int k = 0; k < K; ++k) {
            double av = A[(size_t)i * K + k];
            const float* b = B + (size_t)k * N;
            for (int j = 0; j < N; ++j) c[j] += av * (double)b[j];
        }
    }
}

/* fp32 -> bf16 as acfun_gemm_bf16 packs its operands (src/gemm_bf16_avx512.cpp:
 * 37-44): add 0x7fff plus bit 16 to the fp32 bits (32-bit wrap-around, so
 * some NaNs become infinities or zero, as there), keep the upper half.  y gets
 * the bf16 value widened back to fp32. */
EXPORT void oracle_bf16_round(const float* x, float* y, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        uint32_t u;
        memcpy(&u, &x[i], 4);
        u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
        memcpy(&y[i], &u, 4);
    }
}

/* ------------------------------------------------------------------------ */
/* fp32 convolution                                                          */
/* ------------------------------------------------------------------------ */

/* Route codes of conv2d_impl (src/layers.cpp:106-195). */
enum {
    ROUTE_NONE = 0,       /* output empty: returns without writing (:71,:121,:180) */
    ROUTE_DW = 1,         /* groups==Cin==Cout -> acfun_conv2d_dw (:112-116) */
    ROUTE_GROUPED = 2,    /* Cin_per<=64 && Cout_per<=128 -> acfun_conv2d_grouped (:126-130) */
    ROUTE_GROUP_SPLIT = 3,/* per-group recursion (:134-153) */
    ROUTE_1X1 = 4,        /* conv1x1_impl (:157-160) */
    ROUTE_WINO43 = 5,     /* F(4,3) (:171-172) */
    ROUTE_WINO23 = 6,     /* F(2,3) (:173-174) */
    ROUTE_IM2COL = 7      /* im2col + GEMM (:178-194) */
};

/* Which route conv2d_impl takes for a shape (src/layers.cpp:106-195). */
EXPORT int oracle_conv2d_route(int N, int H, int W, int Cin, int KH, int KW, int Cout,
                               int stride, int pad, int groups) {
    (void)N;
    if (groups > 1) {
        if (groups == Cin && groups == Cout) return ROUTE_DW;
        int Cin_per = Cin / groups, Cout_per = Cout / groups;
        int OH = (H + 2 * pad - KH) / stride + 1;
        int OW = (W + 2 * pad - KW) / stride + 1;
        if (OH <= 0 || OW <= 0) return ROUTE_NONE;
        if (Cin_per <= 64 && Cout_per <= 128) return ROUTE_GROUPED;
        return ROUTE_GROUP_SPLIT;
    }
    if (KH == 1 && KW == 1) {
        int OH = (H + 2 * pad - 1) / stride + 1;
        int OW = (W + 2 * pad - 1) / stride + 1;
        return (OH <= 0 || OW <= 0) ? ROUTE_NONE : ROUTE_1X1;
    }
    if (KH == 3 && KW == 3 && stride == 1 && pad == 1 && H >= 3 && W >= 3 && Cin >= 4 && Cout >= 4) {
        if (H >= 112 && W >= 112 && Cin >= 64 && Cout >= 64) return ROUTE_WINO43;
        return ROUTE_WINO23;
    }
    int OH = (H + 2 * pad - KH) / stride + 1;
    int OW = (W + 2 * pad - KW) / stride + 1;
    return (OH <= 0 || OW <= 0) ? ROUTE_NONE : ROUTE_IM2COL;
}

/* Direct (grouped) convolution accumulated in double, bias, optional ReLU.
 * The closed form every fp32 conv route of conv2d_impl computes
 * (src/layers.cpp:106-195); weights [groups][KH*KW*Cin_per][Cout_per]
 * (src/group_conv.cpp:8-11; groups=1 gives the [KH*KW*Cin, Cout] layout of
 * include/acfun/acfun.h:54-64).  Depthwise uses [C,KH,KW], which is the same
 * memory layout with Cin_per=Cout_per=1. */
EXPORT void oracle_conv2d_f64(const float* in, int N, int H, int W, int Cin,
                              const float* w, const float* bias, int KH, int KW, int Cout,
                              int stride, int pad, int groups, double* out, int act) {
    if (groups < 1) groups = 1;
    int OH = (H + 2 * pad - KH) / stride + 1;
    int OW = (W + 2 * pad - KW) / stride + 1;
    if (OH <= 0 || OW <= 0) return;
    int Cin_p = Cin / groups, Cout_p = Cout / groups;
    #pragma omp parallel for collapse(2) schedule(static)
    for (int n = 0; n < N; ++n)
        for (int oh = 0; oh < OH; ++oh)
            for (int ow = 0; ow < OW; ++ow)
                for (int co = 0; co < Cout; ++co) {
                    int g = co / Cout_p, oc = co % Cout_p;
                    const float* wg = w + (size_t)g * Cout_p * KH * KW * Cin_p;
                    double s = bias ? (double)bias[co] : 0.0;
                    for (int kh = 0; kh < KH; ++kh) {
                        int ih = oh * stride - pad + kh;
                        if (ih < 0 || ih >= H) continue;
                        for (int kw = 0; kw < KW; ++kw) {
                            int iw = ow * stride - pad + kw;
                            if (iw < 0 || iw >= W) continue;
                            const float* px = in + (((size_t)n * H + ih) * W + iw) * Cin + (size_t)g * Cin_p;
                            const float* wp = wg + (size_t)((kh * KW + kw) * Cin_p) * Cout_p + oc;
                            for (int ic = 0; ic < Cin_p; ++ic)
                                s += (double)px[ic] * (double)wp[(size_t)ic * Cout_p];
                        }
                    }
                    if (act && s < 0.0) s = 0.0;
                    out[(((size_t)n * OH + oh) * OW + ow) * Cout + co] = s;
                }
}

/* AVX-512 max_ps(a,b) = a > b ? a : b (returns b for NaN or equal zeros). */
static inline float vmax(float a, float b) { return a > b ? a : b; }

/* Depthwise conv as an AVX-512F host runs it: acc starts at bias, then one
 * fmaf per tap in (kh,kw) order, out-of-range taps contribute fmaf(0,w,acc);
 * ReLU is max_ps(acc,0).  Restates acfun_conv2d_dw_avx512
 * (src/dw_avx512.cpp:20-69, dispatched by src/dw.cpp:42-54). */
EXPORT void oracle_conv2d_dw(const float* input, int N, int H, int W, int C,
                             const float* weight, const float* bias, int KH, int KW,
                             int stride, int pad, float* output, int act) {
    if (KH <= 0 || KW <= 0) return;
    int OH = (H + 2 * pad - KH) / stride + 1;
    int OW = (W + 2 * pad - KW) / stride + 1;
    if (OH <= 0 || OW <= 0) return;
    #pragma omp parallel for collapse(2) schedule(static)
    for (int n = 0; n < N; ++n)
        for (int oh = 0; oh < OH; ++oh)
            for (int ow = 0; ow < OW; ++ow)
                for (int c = 0; c < C; ++c) {
                    float acc = bias ? bias[c] : 0.0f;
                    for (int kh = 0; kh < KH; ++kh)
                        for (int kw = 0; kw < KW; ++kw) {
                            int ih = oh * stride - pad + kh, iw = ow * stride - pad + kw;
                            float v = (ih >= 0 && ih < H && iw >= 0 && iw < W)
                                ? input[(((size_t)n * H + ih) * W + iw) * C + c] : 0.0f;
                            acc = fmaf(v, weight[(size_t)c * KH * KW + kh * KW + kw], acc);
                        }
                    if (act == 1) acc = vmax(acc, 0.0f);
                    output[(((size_t)n * OH + oh) * OW + ow) * C + c] = acc;
                }
}

/* Grouped direct conv as an AVX-512F host runs it (src/group_conv.cpp:60-79):
 *   Cout_per >= 16 -> acfun_group_conv_avx512 (src/group_conv_avx512.cpp:12-79):
 *                     every channel fmaf-accumulated from bias in (kh,kw,ic) order,
 *                     out-of-range taps skipped, ReLU = max_ps;
 *   Cout_per >= 8  -> acfun_group_conv_avx2 (src/group_conv_avx2.cpp:10-73): the
 *                     first Cout_per&~7 channels as above; the tail channels run the
 *                     scalar loop of :55-68, which gcc contracts to fmaf in that
 *                     -mfma translation unit, ReLU = (s<0 -> 0);
 *   otherwise      -> acfun_group_conv_scalar (src/group_conv.cpp:16-55): mul then
 *                     add (generic TU, no FMA), ReLU = (s<0 -> 0).
 * The contraction claim for the AVX2 tail is pinned against oracle/_ref. */
EXPORT void oracle_conv2d_grouped(const float* input, int N, int H, int W, int Cin,
                                  const float* weight, const float* bias, int KH, int KW,
                                  int Cout, int stride, int pad, int groups,
                                  float* output, int act) {
    if (groups <= 1 || KH <= 0 || KW <= 0) return;
    int OH = (H + 2 * pad - KH) / stride + 1;
    int OW = (W + 2 * pad - KW) / stride + 1;
    if (OH <= 0 || OW <= 0) return;
    int Cin_p = Cin / groups, Cout_p = Cout / groups;
    int mode = Cout_p >= 16 ? 2 : (Cout_p >= 8 ? 1 : 0);
    int vec_end = mode == 2 ? Cout_p : (mode == 1 ? (Cout_p & ~7) : 0);
    size_t wg_stride = (size_t)Cout_p * KH * KW * Cin_p;
    #pragma omp parallel for collapse(2) schedule(static)
    for (int n = 0; n < N; ++n)
        for (int oh = 0; oh < OH; ++oh)
            for (int ow = 0; ow < OW; ++ow)
                for (int g = 0; g < groups; ++g)
                    for (int oc = 0; oc < Cout_p; ++oc) {
                        const float* wg = weight + (size_t)g * wg_stride;
                        float s = bias ? bias[(size_t)g * Cout_p + oc] : 0.0f;
                        int use_fma = (oc < vec_end) || mode == 1;
                        for (int kh = 0; kh < KH; ++kh) {
                            int ih = oh * stride - pad + kh;
                            if (ih < 0 || ih >= H) continue;
                            for (int kw = 0; kw < KW; ++kw) {
                                int iw = ow * stride - pad + kw;
                                if (iw < 0 || iw >= W) continue;
                                const float* px = input + (((size_t)n * H + ih) * W + iw) * Cin + (size_t)g * Cin_p;
                                const float* wp = wg + (size_t)((kh * KW + kw) * Cin_p) * Cout_p + oc;
                                for (int ic = 0; ic < Cin_p; ++ic) {
                                    if (use_fma) s = fmaf(px[ic], wp[(size_t)ic * Cout_p], s);
                                    else         s = s + px[ic] * wp[(size_t)ic * Cout_p];
                                }
                            }
                        }
                        if (act == 1) {
                            if (oc < vec_end) s = vmax(s, 0.0f);
                            else if (s < 0.0f) s = 0.0f;
                        }
                        output[(((size_t)n * OH + oh) * OW + ow) * Cout + (size_t)g * Cout_p + oc] = s;
                    }
}

/* MaxPool over in-range taps from a -1e30 sentinel, optional ReLU after.
 * Channels below the vector width run max_ps semantics
 * (src/maxpool_avx512.cpp:15-62 for C>=16, src/maxpool_avx2.cpp for C>=8),
 * the tail channels and C<8 run the scalar compare (src/layers.cpp:221-246);
 * the two differ only for NaN and signed zeros.  Dispatch: src/layers.cpp:250-258. */
EXPORT void oracle_maxpool(const float* in, int N, int H, int W, int C, int pool, int stride,
                           int pad, float* out, int post_relu) {
    int OH = (H + 2 * pad - pool) / stride + 1;
    int OW = (W + 2 * pad - pool) / stride + 1;
    if (OH <= 0 || OW <= 0) return;
    int vec_end = C >= 16 ? (C & ~15) : (C >= 8 ? (C & ~7) : 0);
    #pragma omp parallel for collapse(2) schedule(static)
    for (int n = 0; n < N; ++n)
        for (int oh = 0; oh < OH; ++oh)
            for (int ow = 0; ow < OW; ++ow)
                for (int c = 0; c < C; ++c) {
                    float mx = -1e30f;
                    for (int ph = 0; ph < pool; ++ph) {
                        int ih = oh * stride - pad + ph;
                        if (ih < 0 || ih >= H) continue;
                        for (int pw = 0; pw < pool; ++pw) {
                            int iw = ow * stride - pad + pw;
                            if (iw < 0 || iw >= W) continue;
                            float v = in[(((size_t)n * H + ih) * W + iw) * C + c];
                            if (c < vec_end) mx = vmax(mx, v);
                            else if (v > mx) mx = v;
                        }
                    }
                    if (post_relu) {
                        if (c < vec_end) mx = vmax(mx, 0.0f);
                        else if (mx < 0.0f) mx = 0.0f;
                    }
                    out[(((size_t)n * OH + oh) * OW + ow) * C + c] = mx;
                }
}

/* acfun_relu / acfun_relu6 (src/layers.cpp:10-17). */
EXPORT void oracle_relu(float* d, size_t len) {
    for (size_t i = 0; i < len; ++i) if (d[i] < 0.0f) d[i] = 0.0f;
}
EXPORT void oracle_relu6(float* d, size_t len) {
    for (size_t i = 0; i < len; ++i) {
        float v = d[i];
        if (v < 0.0f) v = 0.0f; else if (v > 6.0f) v = 6.0f;
        d[i] = v;
    }
}

/* Row softmax: max, expf(x-max), sum, x*(1/sum) (src/layers.cpp:272-283). */
EXPORT void oracle_softmax(const float* in, int rows, int cols, float* out) {
    for (int r = 0; r < rows; ++r) {
        const float* ri = in + (size_t)r * cols;
        float* ro = out + (size_t)r * cols;
        float mx = ri[0];
        for (int c = 1; c < cols; ++c) if (ri[c] > mx) mx = ri[c];
        float sum = 0.0f;
        for (int c = 0; c < cols; ++c) { float e = expf(ri[c] - mx); ro[c] = e; sum += e; }
        float inv = 1.0f / sum;
        for (int c = 0; c < cols; ++c) ro[c] *= inv;
    }
}

/* Unfused BN: (d-mean)*(gamma/sqrtf(var+eps)) + beta, two roundings each
 * (src/layers.cpp:285-296, generic TU). */
EXPORT void oracle_batchnorm(float* d, int size, int channels, const float* mean, const float* var,
                             const float* gamma, const float* beta, float eps) {
    int spatial = size / channels;
    for (int c = 0; c < channels; ++c) {
        float scale = gamma ? gamma[c] : 1.0f;
        float shift = beta ? beta[c] : 0.0f;
        float inv = scale / sqrtf(var[c] + eps);
        for (int s = 0; s < spatial; ++s) {
            float t = d[(size_t)s * channels + c] - mean[c];
            t = t * inv;
            d[(size_t)s * channels + c] = t + shift;
        }
    }
}

/* fold_bn_into (src/model.cpp:69-95): scale=gamma/sqrtf(var+1e-5f),
 * shift=beta-mean*scale, w*=scale at the group-aware offset, b'=b*scale+shift. */
EXPORT void oracle_fold_bn(float* w, float* b, int has_bias, int Cout, size_t wn, int groups,
                           const float* mean, const float* var, const float* gamma, const float* beta) {
    int Cout_per = (groups > 1) ? Cout / groups : Cout;
    size_t per_in = wn / (size_t)Cout;
    for (int c = 0; c < Cout; ++c) {
        float scale = gamma[c] / sqrtf(var[c] + 1e-5f);
        float ms = mean[c] * scale;
        float shift = beta[c] - ms;
        int gc = (groups > 1) ? c / Cout_per : 0;
        int oc = (groups > 1) ? c % Cout_per : c;
        for (size_t t = 0; t < per_in; ++t) {
            size_t off = (size_t)gc * (size_t)Cout_per * per_in + t * (size_t)Cout_per + oc;
            w[off] *= scale;
        }
        float bs = (has_bias ? b[c] : 0.0f) * scale;
        b[c] = bs + shift;
    }
}

/* ------------------------------------------------------------------------ */
/* int8                                                                      */
/* ------------------------------------------------------------------------ */

/* Per-output-column symmetric weight quantization (src/conv_int8.cpp:24-37):
 * s=max|w|/127 (s<=0 -> 1), q=clamp(lroundf(w/s),-128,127). */
EXPORT void oracle_quantize_weights(const float* w, int K, int N, float* scales, int8_t* wq) {
    for (int j = 0; j < N; ++j) {
        float maxa = 0.0f;
        for (int k = 0; k < K; ++k) {
            float a = fabsf(w[(size_t)k * N + j]);
            maxa = (maxa < a) ? a : maxa;          /* std::max(maxa, a) */
        }
        float s = maxa / 127.0f;
        if (s <= 0.0f) s = 1.0f;
        scales[j] = s;
        for (int k = 0; k < K; ++k) {
            int v = (int)lroundf(w[(size_t)k * N + j] / s);    /* as the reference: int first */
            if (v > 127) v = 127; else if (v < -128) v = -128;
            wq[(size_t)k * N + j] = (int8_t)v;
        }
    }
}

/* max|x| over a tensor, std::max order (src/conv_int8.cpp:75-77). */
EXPORT float oracle_absmax(const float* x, size_t n) {
    float maxa = 0.0f;
    for (size_t i = 0; i < n; ++i) { float a = fabsf(x[i]); maxa = (maxa < a) ? a : maxa; }
    return maxa;
}

/* The three activation rounding rules of the reference (mode):
 *   0 RNE  : _mm512_cvtps_epi32 (src/int8_quantize_avx512.cpp:15-20), avx512f+bw hosts
 *   1 LROUND: lroundf (src/int8_quantize.cpp:31-36, scalar hosts; Winograd tail channels
 *            src/winograd_int8.cpp:321-325)
 *   2 HALFAWAY_ADD: trunc(t + copysign(0.5,t)) with t+0.5 rounded in float
 *            (src/winograd_int8.cpp:306-319)
 * Returns clamp(q + zp, 0, 255). */
static inline int quant_one(float x, float inv_s, int zp, int mode) {
    float t = x * inv_s;
    int q;
    if (mode == 0) q = (int)rintf(t);
    else if (mode == 1) q = (int)lroundf(t);
    else { float r = t + copysignf(0.5f, t); q = (int)truncf(r); }
    int v = q + zp;
    return v < 0 ? 0 : (v > 255 ? 255 : v);
}

EXPORT void oracle_quantize_u8(const float* in, uint8_t* out, size_t n, float inv_s, int zp, int mode) {
    for (size_t i = 0; i < n; ++i) out[i] = (uint8_t)quant_one(in[i], inv_s, zp, mode);
}

/* u8 x s8 -> i32 GEMM (src/gemm_int8.cpp:11-30). */
EXPORT void oracle_gemm_int8(int M, int N, int K, const uint8_t* A, const int8_t* B, int32_t* C) {
    #pragma omp parallel for schedule(static)
    for (int i = 0; i < M; ++i) {
        int32_t* c = C + (size_t)i * N;
        for (int j = 0; j < N; ++j) c[j] = 0;
        for (int k = 0; k < K; ++k) {
            int av = A[(size_t)i * K + k];
            if (av == 0) continue;
            const int8_t* b = B + (size_t)k * N;
            for (int j = 0; j < N; ++j) c[j] += av * (int32_t)b[j];
        }
    }
}

/* The non-Winograd int8 epilogue: (float)acc*alpha[j] then +beta[j], two
 * roundings (-ffp-contract=off, CMakeLists.txt:54-66), ReLU = max_ps
 * (src/gemm_int8_avx512.cpp:113-136; src/conv1x1_int8_avx512.cpp:85;
 * src/conv_int8_direct_avx512.cpp:162). */
static inline float epi_mul_add(int32_t acc, float alpha, float beta, int act) {
    float p = (float)acc * alpha;
    float v = p + beta;
    if (act) v = vmax(v, 0.0f);
    return v;
}

/* acfun_gemm_int8_epi (src/gemm_int8.cpp:53-75). */
EXPORT void oracle_gemm_int8_epi(int M, int N, int K, const uint8_t* A, const int8_t* B, float* C,
                                 const float* alpha, const float* beta, int act) {
    #pragma omp parallel for schedule(static)
    for (int i = 0; i < M; ++i) {
        int32_t* acc = (int32_t*)malloc(sizeof(int32_t) * (size_t)(N > 0 ? N : 1));
        for (int j = 0; j < N; ++j) acc[j] = 0;
        for (int k = 0; k < K; ++k) {
            int av = A[(size_t)i * K + k];
            const int8_t* b = B + (size_t)k * N;
            for (int j = 0; j < N; ++j) acc[j] += av * (int32_t)b[j];
        }
        for (int j = 0; j < N; ++j) C[(size_t)i * N + j] = epi_mul_add(acc[j], alpha[j], beta[j], act);
        free(acc);
    }
}

/* acfun_conv1x1_int8 (src/conv1x1_int8.cpp:21-49): the GEMM epilogue on the
 * zero-copy [M,K] activation matrix. */
EXPORT void oracle_conv1x1_int8(const uint8_t* inQ, int M, int K, int Cout, const int8_t* wq,
                                const float* alpha, const float* beta, float* out, int act) {
    oracle_gemm_int8_epi(M, Cout, K, inQ, wq, out, alpha, beta, act);
}

/* acfun_conv2d_int8_direct (src/conv_int8_direct.cpp:20-59): all KH*KW*Cin
 * taps, out-of-range taps read the zero point 128, same epilogue. */
EXPORT void oracle_conv2d_int8_direct(const uint8_t* inQ, int N, int H, int W, int Cin,
                                      const int8_t* wq, const float* alpha, const float* beta,
                                      int KH, int KW, int Cout, int stride, int pad,
                                      int OH, int OW, float* output, int act) {
    #pragma omp parallel for collapse(2) schedule(static)
    for (int n = 0; n < N; ++n)
        for (int oh = 0; oh < OH; ++oh)
            for (int ow = 0; ow < OW; ++ow)
                for (int j = 0; j < Cout; ++j) {
                    int32_t acc = 0;
                    for (int kh = 0; kh < KH; ++kh) {
                        int ih = oh * stride - pad + kh;
                        for (int kw = 0; kw < KW; ++kw) {
                            int iw = ow * stride - pad + kw;
                            int ok = ih >= 0 && ih < H && iw >= 0 && iw < W;
                            const uint8_t* ip = ok ? inQ + (((size_t)n * H + ih) * W + iw) * Cin : NULL;
                            const int8_t* wp = wq + (size_t)((kh * KW + kw) * Cin) * Cout + j;
                            for (int ic = 0; ic < Cin; ++ic)
                                acc += (ok ? (int)ip[ic] : 128) * (int)wp[(size_t)ic * Cout];
                        }
                    }
                    output[(((size_t)n * OH + oh) * OW + ow) * Cout + j] = epi_mul_add(acc, alpha[j], beta[j], act);
                }
}

/* im2col of the quantized input with the zero point 128 in padded taps, then
 * acfun_gemm_int8_epi per image (src/conv_int8.cpp:42-61,133-147).  The
 * result equals the direct form above, so this restates it through that. */
static void int8_im2col_gemm(const uint8_t* inQ, int N, int H, int W, int Cin, const int8_t* wq,
                             const float* alpha, const float* beta, int KH, int KW, int Cout,
                             int stride, int pad, int OH, int OW, float* out, int act) {
    oracle_conv2d_int8_direct(inQ, N, H, W, Cin, wq, alpha, beta, KH, KW, Cout, stride, pad,
                              OH, OW, out, act);
}

/* ---- int8 Winograd F(2,3) (src/winograd_int8.cpp) ---------------------- */

/* d_hat = BT d BT^T on one 4x4 u8 block, int16 (src/winograd_int8.cpp:54-70). */
static void wino_in_u8(const uint8_t* d, int16_t dh[16]) {
    int16_t U[4][4];
    for (int l = 0; l < 4; ++l) {
        int16_t c0 = d[l], c1 = d[4 + l], c2 = d[8 + l], c3 = d[12 + l];
        U[0][l] = (int16_t)(c0 - c2);
        U[1][l] = (int16_t)(c1 + c2);
        U[2][l] = (int16_t)(-c1 + c2);
        U[3][l] = (int16_t)(-c1 + c3);
    }
    for (int i = 0; i < 4; ++i) {
        int16_t u0 = U[i][0], u1 = U[i][1], u2 = U[i][2], u3 = U[i][3];
        dh[i * 4 + 0] = (int16_t)(u0 - u2);
        dh[i * 4 + 1] = (int16_t)(u1 + u2);
        dh[i * 4 + 2] = (int16_t)(-u1 + u2);
        dh[i * 4 + 3] = (int16_t)(-u1 + u3);
    }
}

/* g_hat2 = Gt g Gt^T with Gt = 2G integral (src/winograd_int8.cpp:74-90). */
static void wino_filter_i8(const int8_t g[9], int16_t gh2[16]) {
    int16_t T[4][3];
    for (int y = 0; y < 3; ++y) {
        int16_t a = g[y], b = g[3 + y], c = g[6 + y];
        T[0][y] = (int16_t)(2 * a);
        T[1][y] = (int16_t)(a + b + c);
        T[2][y] = (int16_t)(a - b + c);
        T[3][y] = (int16_t)(2 * c);
    }
    for (int i = 0; i < 4; ++i) {
        int16_t t0 = T[i][0], t1 = T[i][1], t2 = T[i][2];
        gh2[i * 4 + 0] = (int16_t)(2 * t0);
        gh2[i * 4 + 1] = (int16_t)(t0 + t1 + t2);
        gh2[i * 4 + 2] = (int16_t)(t0 - t1 + t2);
        gh2[i * 4 + 3] = (int16_t)(2 * t2);
    }
}

/* acfun_winograd_conv3x3_int8 (src/winograd_int8.cpp:245-350): quantize while
 * padding (HALFAWAY_ADD on 16-channel chunks, lroundf on the tail, pads = 128),
 * T4[ij][o] = sum_c dh*g_hat2 - 128*Q[ij]*Sgh[ij][o] (Q[5]=4) in wrapping int32,
 * output transform in int64 with the AT sign table (:104-121), then
 * fma((float)acc64, fl(fl(s_in*0.25)*ws), bias) and max_ps ReLU (:154-170). */
EXPORT void oracle_winograd_conv3x3_int8(const float* input, int N, int H, int W, int Cin,
                                         const int8_t* wq, const float* wscale, const float* bias,
                                         int Cout, float s_in, float inv_s, float* output, int act) {
    const int OH = H, OW = W, tH = (OH + 1) / 2, tW = (OW + 1) / 2;
    int16_t* gh = (int16_t*)malloc(sizeof(int16_t) * 16 * (size_t)Cin * Cout);
    int32_t* Sgh = (int32_t*)calloc((size_t)16 * Cout, sizeof(int32_t));
    for (int c = 0; c < Cin; ++c)
        for (int o = 0; o < Cout; ++o) {
            int8_t g[9]; int16_t g2[16];
            for (int k = 0; k < 9; ++k) g[k] = wq[((size_t)k * Cin + c) * Cout + o];
            wino_filter_i8(g, g2);
            for (int ij = 0; ij < 16; ++ij) {
                gh[((size_t)ij * Cin + c) * Cout + o] = g2[ij];
                Sgh[(size_t)ij * Cout + o] += g2[ij];
            }
        }
    int AT[2][4] = {{1, 1, 1, 0}, {0, 1, -1, 1}};
    int cvec = Cin & ~15;
    size_t PW = (size_t)W + 2, PH = (size_t)H + 2;
    uint8_t* pad = (uint8_t*)malloc(PH * PW * Cin);
    for (int n = 0; n < N; ++n) {
        const float* x = input + (size_t)n * H * W * Cin;
        memset(pad, 128, PH * PW * Cin);
        for (int ih = 0; ih < H; ++ih)
            for (int iw = 0; iw < W; ++iw)
                for (int c = 0; c < Cin; ++c)
                    pad[(((size_t)ih + 1) * PW + iw + 1) * Cin + c] =
                        (uint8_t)quant_one(x[((size_t)ih * W + iw) * Cin + c], inv_s, 128, c < cvec ? 2 : 1);
        #pragma omp parallel for collapse(2) schedule(static)
        for (int ty = 0; ty < tH; ++ty)
            for (int tx = 0; tx < tW; ++tx) {
                int16_t* dh = (int16_t*)malloc(sizeof(int16_t) * 16 * (size_t)Cin);
                for (int c = 0; c < Cin; ++c) {
                    uint8_t blk[16];
                    for (int k = 0; k < 4; ++k)
                        for (int l = 0; l < 4; ++l) {
                            int pr = 2 * ty + k, pc = 2 * tx + l;
                            blk[k * 4 + l] = (pr < OH + 2 && pc < OW + 2)
                                ? pad[((size_t)pr * PW + pc) * Cin + c] : (uint8_t)128;
                        }
                    int16_t d16[16];
                    wino_in_u8(blk, d16);
                    for (int ij = 0; ij < 16; ++ij) dh[(size_t)ij * Cin + c] = d16[ij];
                }
                for (int o = 0; o < Cout; ++o) {
                    int32_t T4[16];
                    for (int ij = 0; ij < 16; ++ij) {
                        uint32_t acc = 0;   /* wrapping int32 as the vector adds wrap */
                        for (int c = 0; c < Cin; ++c)
                            acc += (uint32_t)((int32_t)dh[(size_t)ij * Cin + c] *
                                              (int32_t)gh[((size_t)ij * Cin + c) * Cout + o]);
                        if (ij == 5) acc -= (uint32_t)(512 * Sgh[(size_t)ij * Cout + o]);
                        T4[ij] = (int32_t)acc;
                    }
                    float wso = (s_in * 0.25f) * wscale[o];
                    float bv = bias ? bias[o] : 0.0f;
                    for (int e = 0; e < 4; ++e) {
                        int r = e >> 1, cc = e & 1;
                        int oh = 2 * ty + r, ow = 2 * tx + cc;
                        if (oh >= OH || ow >= OW) continue;
                        int64_t a64 = 0;
                        for (int ij = 0; ij < 16; ++ij) {
                            int s = AT[r][ij >> 2] * AT[cc][ij & 3];
                            if (s > 0) a64 += T4[ij]; else if (s < 0) a64 -= T4[ij];
                        }
                        float v = fmaf((float)a64, wso, bv);
                        if (act == 1) v = vmax(v, 0.0f);
                        output[(((size_t)n * OH + oh) * OW + ow) * Cout + o] = v;
                    }
                }
                free(dh);
            }
    }
    free(pad); free(gh); free(Sgh);
}

/* The exact direct integer A = sum (u8-128)*wq that the identity
 * AT*T4*AT^T = 4*A says the Winograd route computes (pads contribute 0).
 * Brute force, used to pin the identity. */
EXPORT void oracle_conv_int8_centered_acc(const uint8_t* inQ, int N, int H, int W, int Cin,
                                          const int8_t* wq, int KH, int KW, int Cout, int stride,
                                          int pad, int OH, int OW, int32_t* acc) {
    #pragma omp parallel for collapse(2) schedule(static)
    for (int n = 0; n < N; ++n)
        for (int oh = 0; oh < OH; ++oh)
            for (int ow = 0; ow < OW; ++ow)
                for (int j = 0; j < Cout; ++j) {
                    int32_t a = 0;
                    for (int kh = 0; kh < KH; ++kh)
                        for (int kw = 0; kw < KW; ++kw) {
                            int ih = oh * stride - pad + kh, iw = ow * stride - pad + kw;
                            if (ih < 0 || ih >= H || iw < 0 || iw >= W) continue;
                            const uint8_t* ip = inQ + (((size_t)n * H + ih) * W + iw) * Cin;
                            const int8_t* wp = wq + (size_t)((kh * KW + kw) * Cin) * Cout + j;
                            for (int ic = 0; ic < Cin; ++ic)
                                a += ((int)ip[ic] - 128) * (int)wp[(size_t)ic * Cout];
                        }
                    acc[(((size_t)n * OH + oh) * OW + ow) * Cout + j] = a;
                }
}

/* The Winograd route's epilogue applied to direct accumulators A (M rows of
 * Cout): the reference forms 4*A exactly as AT*T4*AT^T and computes
 * fmaf((float)(4A), fl(fl(s_in*0.25)*ws[j]), b[j]), then max_ps ReLU
 * (src/winograd_int8.cpp:154-170).  With oracle_conv_int8_centered_acc this
 * is the closed form the identity predicts. */
EXPORT void oracle_wino_int8_epilogue(const int32_t* acc, size_t M, int Cout, float s_in,
                                      const float* wscale, const float* bias, float* out, int act) {
    for (int j = 0; j < Cout; ++j) {
        float wso = (s_in * 0.25f) * wscale[j];
        float bv = bias ? bias[j] : 0.0f;
        for (size_t i = 0; i < M; ++i) {
            int64_t a4 = 4 * (int64_t)acc[i * (size_t)Cout + j];
            float v = fmaf((float)a4, wso, bv);
            if (act == 1) v = vmax(v, 0.0f);
            out[i * (size_t)Cout + j] = v;
        }
    }
}

/* int8 route codes of acfun_conv2d_int8 (src/conv_int8.cpp:63-148) on an
 * avx512f host. */
enum { I8_NONE = 0, I8_ZERO = 1, I8_WINO = 2, I8_DIRECT = 3, I8_1X1 = 4, I8_GEMM = 5 };

EXPORT int oracle_conv2d_int8_route(int H, int W, int Cin, int KH, int KW, int Cout, int stride, int pad) {
    int OH = (H + 2 * pad - KH) / stride + 1;
    int OW = (W + 2 * pad - KW) / stride + 1;
    if (OH <= 0 || OW <= 0) return I8_NONE;
    int K = KH * KW * Cin;
    if (KH == 3 && KW == 3 && stride == 1 && pad == 1 && H >= 3 && W >= 3 && Cin >= 4 && Cout >= 4)
        return I8_WINO;
    int zc = (KH == 1 && KW == 1 && stride == 1 && pad == 0);
    if (K <= 64 && !zc) return I8_DIRECT;
    if (zc) return I8_1X1;
    return I8_GEMM;
}

/* acfun_conv2d_int8 (src/conv_int8.cpp:63-148) as an avx512f+bw+vnni host
 * runs it: s_in ignored; maxa=max|x|; maxa<1e-12 -> zero output (no bias);
 * inv_s=127/maxa, sa=maxa/127; Winograd route for 3x3/s1/p1 with channels>=4;
 * otherwise RNE-quantize, alpha=sa*ws[j], beta=b-(alpha*128)*Sw[j] (float Sw),
 * then the direct / 1x1 / im2col+GEMM route, all with the mul-then-add epilogue. */
EXPORT void oracle_conv2d_int8(const float* input, int N, int H, int W, int Cin,
                               const int8_t* wq, const float* wscale, const float* bias,
                               int KH, int KW, int Cout, int stride, int pad,
                               float s_in, float* output, int act) {
    (void)s_in;
    int OH = (H + 2 * pad - KH) / stride + 1;
    int OW = (W + 2 * pad - KW) / stride + 1;
    if (OH <= 0 || OW <= 0) return;
    int K = KH * KW * Cin;
    size_t M = (size_t)N * OH * OW;
    size_t inN = (size_t)N * H * W * Cin;
    float maxa = oracle_absmax(input, inN);
    if (maxa < 1e-12f) { memset(output, 0, M * Cout * sizeof(float)); return; }
    float inv_s = 127.0f / maxa;
    float sa = maxa / 127.0f;
    int route = oracle_conv2d_int8_route(H, W, Cin, KH, KW, Cout, stride, pad);
    if (route == I8_WINO) {
        oracle_winograd_conv3x3_int8(input, N, H, W, Cin, wq, wscale, bias, Cout, sa, inv_s, output, act);
        return;
    }
    uint8_t* inQ = (uint8_t*)malloc(inN ? inN : 1);
    oracle_quantize_u8(input, inQ, inN, inv_s, 128, 0);
    float* alpha = (float*)malloc(sizeof(float) * Cout);
    float* beta = (float*)malloc(sizeof(float) * Cout);
    for (int j = 0; j < Cout; ++j) {
        float Swj = 0.0f;
        for (int k = 0; k < K; ++k) Swj += (float)wq[(size_t)k * Cout + j];
        float a = sa * wscale[j];
        alpha[j] = a;
        float t = a * 128.0f;
        t = t * Swj;
        beta[j] = (bias ? bias[j] : 0.0f) - t;
    }
    if (route == I8_DIRECT)
        oracle_conv2d_int8_direct(inQ, N, H, W, Cin, wq, alpha, beta, KH, KW, Cout, stride, pad, OH, OW, output, act);
    else if (route == I8_1X1)
        oracle_conv1x1_int8(inQ, (int)M, K, Cout, wq, alpha, beta, output, act);
    else
        int8_im2col_gemm(inQ, N, H, W, Cin, wq, alpha, beta, KH, KW, Cout, stride, pad, OH, OW, output, act);
    free(inQ); free(alpha); free(beta);
}

/* Per-tensor requantization of a float tensor to int8 (the build-defined
 * int8 output): q = clamp(RNE(y*inv_s_out), -128, 127), inv_s_out=127/max|y|,
 * which equals acfun_quantize_u8_avx512(y, inv_s_out, 128) - 128
 * (src/int8_quantize_avx512.cpp:15-20; src/conv_int8.cpp:75-81). */
EXPORT float oracle_requantize_s8(const float* y, size_t n, int8_t* q) {
    float maxa = oracle_absmax(y, n);
    if (maxa < 1e-12f) { memset(q, 0, n); return 0.0f; }
    float inv = 127.0f / maxa;
    for (size_t i = 0; i < n; ++i) q[i] = (int8_t)(quant_one(y[i], inv, 128, 0) - 128);
    return maxa / 127.0f;
}

/* The int8-in / int8-out convolution (the build-defined requantized output,
 * no reference counterpart of its own).  Input: s8 activations q [N,H,W,Cin]
 * with per-tensor scale s_in (x = q * s_in; s_in == 0 marks an all-zero
 * input).  The float result y is exactly what acfun_conv2d_int8
 * (src/conv_int8.cpp:63-148) computes from u8 = q + 128 with its activation
 * scale sa = s_in: the Winograd route's fmaf((float)(4A), fl(fl(sa*0.25)*ws), b)
 * (src/winograd_int8.cpp:154-170) for 3x3/s1/p1, else the direct / 1x1 /
 * im2col+GEMM epilogue fl(fl((float)acc_u*alpha)+beta) with
 * alpha = fl(sa*ws), beta = fl(b - fl(fl(alpha*128)*Sw)) (:100-107); every
 * image computed from its own pixels.  Then y is requantized per tensor:
 * maxy = max|y|; maxy < 1e-12 -> out = 0 and *s_out = 0; else
 * inv = 127/maxy, *s_out = maxy/127, out = clamp(rule(y*inv), -128, 127) with
 * rule 0 = RNE (acfun_quantize_u8, src/int8_quantize_avx512.cpp:15-20) and
 * rule 1 = the rule the Winograd route applies to its own input
 * (half-away-by-add on channels below Cout & ~15, lroundf above,
 * src/winograd_int8.cpp:306-325), so the s8 tensor is what the next layer
 * would have quantized the float tensor to. */
EXPORT void oracle_conv2d_int8_q(const int8_t* q, float s_in, int N, int H, int W, int Cin,
                                 const int8_t* wq, const float* wscale, const float* bias,
                                 int KH, int KW, int Cout, int stride, int pad, int8_t* out,
                                 float* s_out, int act, int rule) {
    int OH = (H + 2 * pad - KH) / stride + 1;
    int OW = (W + 2 * pad - KW) / stride + 1;
    if (OH <= 0 || OW <= 0) return;
    size_t M = (size_t)N * OH * OW;
    size_t inN = (size_t)N * H * W * Cin;
    float* y = (float*)malloc(sizeof(float) * (M * (size_t)Cout > 0 ? M * (size_t)Cout : 1));
    if (s_in == 0.0f) {
        memset(y, 0, sizeof(float) * M * Cout);
    } else {
        uint8_t* u = (uint8_t*)malloc(inN ? inN : 1);
        for (size_t i = 0; i < inN; ++i) u[i] = (uint8_t)((int)q[i] + 128);
        int route = oracle_conv2d_int8_route(H, W, Cin, KH, KW, Cout, stride, pad);
        if (route == I8_WINO) {
            int32_t* acc = (int32_t*)malloc(sizeof(int32_t) * (M * (size_t)Cout > 0 ? M * (size_t)Cout : 1));
            oracle_conv_int8_centered_acc(u, N, H, W, Cin, wq, 3, 3, Cout, 1, 1, OH, OW, acc);
            oracle_wino_int8_epilogue(acc, M, Cout, s_in, wscale, bias, y, act);
            free(acc);
        } else {
            int K = KH * KW * Cin;
            float* alpha = (float*)malloc(sizeof(float) * Cout);
            float* beta = (float*)malloc(sizeof(float) * Cout);
            for (int j = 0; j < Cout; ++j) {
                float Swj = 0.0f;
                for (int k = 0; k < K; ++k) Swj += (float)wq[(size_t)k * Cout + j];
                float a = s_in * wscale[j];
                alpha[j] = a;
                float t = a * 128.0f;
                t = t * Swj;
                beta[j] = (bias ? bias[j] : 0.0f) - t;
            }
            if (route == I8_1X1)
                oracle_conv1x1_int8(u, (int)M, K, Cout, wq, alpha, beta, y, act);
            else
                oracle_conv2d_int8_direct(u, N, H, W, Cin, wq, alpha, beta, KH, KW, Cout, stride,
                                          pad, OH, OW, y, act);
            free(alpha); free(beta);
        }
        free(u);
    }
    float maxy = oracle_absmax(y, M * Cout);
    if (maxy < 1e-12f) {
        memset(out, 0, M * Cout);
        *s_out = 0.0f;
    } else {
        float inv = 127.0f / maxy;
        int cvec = Cout & ~15;
        for (size_t i = 0; i < M; ++i)
            for (int c = 0; c < Cout; ++c) {
                int mode = rule == 0 ? 0 : (c < cvec ? 2 : 1);
                out[i * Cout + c] = (int8_t)(quant_one(y[i * Cout + c], inv, 128, mode) - 128);
            }
        *s_out = maxy / 127.0f;
    }
    free(y);
}
