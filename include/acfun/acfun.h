/*
 * acfun.h -- C ABI of libacfun_amd.so, the MI355X (gfx950) implementation of
 * Acfun's convolution/GEMM path.
 *
 * Every function of the reference's public header (include/acfun/acfun.h:15-148
 * of the reference) is declared here with the same name, signature, argument
 * meaning and error behaviour; each carries the reference line it replaces.
 * Behind them, host C++ stages the caller's buffers to HBM (or uses them in
 * place when they already are device pointers), launches hand-written HIP
 * kernels on the library stream and synchronizes before returning, so a
 * caller of the reference sees the same synchronous semantics.
 *
 * The second block holds the reference's internal entry points that its own
 * tests bind (src/internal.h of the reference).
 *
 * The third block is new: device-pointer variants that run asynchronously on a
 * caller-supplied HIP stream (passed as void*, NULL = the library stream),
 * a batched model call, and an error string.  Plain pointers and sizes only.
 *
 * Conventions kept from the reference:
 *   - all tensors NHWC, row-major; conv weights [KH*KW*Cin, Cout];
 *   - invalid shapes (empty output) return without writing;
 *   - no error codes: acfun_last_error() reports the last failure (new).
 */
#ifndef ACFUN_AMD_ACFUN_H
#define ACFUN_AMD_ACFUN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ===================== reference public API (27 functions) ===================== */

/* ref acfun.h:20 -- sets the host thread count used by the CPU-side helpers
 * (the GPU path does not use OpenMP); 0 = all cores. */
void acfun_set_threads(int n);

/* ref acfun.h:23-24 -- backend query.  Returns 4 ("MI355X-gfx950") when a
 * gfx950 device is present; 0 / "none" otherwise (the GPU path has no CPU
 * fallback: entry points then fail and set acfun_last_error()). */
int acfun_backend(void);
const char* acfun_backend_name(void);

/* ref acfun.h:29-30 -- runs the MFMA tile-shape search for the configured GEMM
 * shapes and caches the result (ACFUN_AUTOTUNE=1 triggers it at first use). */
void acfun_autotune(void);
const char* acfun_tune_status(void);

/* ref acfun.h:33-34 -- C[M,N] = A[M,K] * B[K,N], row-major, C overwritten. */
void acfun_gemm(int M, int N, int K, const float* A, const float* B, float* C);

/* ref acfun.h:43-45 -- GEMM, then +bias[j] (NULL = none) and ReLU if act. */
void acfun_gemm_epi(int M, int N, int K, const float* A, const float* B, float* C,
                    const float* bias, int act);

/* ref acfun.h:51-52 -- A and B rounded to bf16 (RNE), fp32 accumulation. */
void acfun_gemm_bf16(int M, int N, int K, const float* A, const float* B, float* C);

/* ref acfun.h:61-64 -- convolution, routed exactly like the reference's
 * conv2d_impl (src/layers.cpp:106-195): 1x1 -> GEMM, 3x3/s1/p1 -> Winograd
 * F(4,3) or F(2,3), else implicit-GEMM (im2col semantics). */
void acfun_conv2d(const float* input, int N, int H, int W, int Cin,
                  const float* weight, const float* bias,
                  int KH, int KW, int Cout, int stride, int pad, float* output);

/* ref acfun.h:67-70 -- the same with fused ReLU. */
void acfun_conv2d_relu(const float* input, int N, int H, int W, int Cin,
                       const float* weight, const float* bias,
                       int KH, int KW, int Cout, int stride, int pad, float* output);

/* ref acfun.h:77-80 -- depthwise conv, weights [C,KH,KW]. */
void acfun_conv2d_dw(const float* input, int N, int H, int W, int C,
                     const float* weight, const float* bias,
                     int KH, int KW, int stride, int pad, float* output, int act);

/* ref acfun.h:86-89 -- grouped conv, weights [groups][KH*KW*Cin_per][Cout_per]
 * (the layout the reference's kernels read, src/group_conv.cpp:8-11). */
void acfun_conv2d_g(const float* input, int N, int H, int W, int Cin,
                    const float* weight, const float* bias,
                    int KH, int KW, int Cout, int stride, int pad, int groups,
                    float* output, int act);

/* ref acfun.h:92-93 / 97-98 -- fully connected, out[N,Cout] = in[N,Cin]*W[Cin,Cout]+b. */
void acfun_fc(const float* input, int N, int Cin, const float* weight, const float* bias,
              int Cout, float* output);
void acfun_fc_relu(const float* input, int N, int Cin, const float* weight, const float* bias,
                   int Cout, float* output);

/* ref acfun.h:101-102 -- in-place activations. */
void acfun_relu(float* data, size_t len);
void acfun_relu6(float* data, size_t len);

/* ref acfun.h:105-111 -- NHWC max pooling (square window), optional ReLU after. */
void acfun_maxpool(const float* input, int N, int H, int W, int C,
                   int pool, int stride, int pad, float* output);
void acfun_maxpool_relu(const float* input, int N, int H, int W, int C,
                        int pool, int stride, int pad, float* output);

/* ref acfun.h:114 -- row softmax. */
void acfun_softmax(const float* input, int rows, int cols, float* output);

/* ref acfun.h:117-119 -- in-place BN: (x-mean)*(gamma/sqrt(var+eps))+beta. */
void acfun_batchnorm(float* data, int size, int channels, const float* mean, const float* var,
                     const float* gamma, const float* beta, float eps);

/* ref acfun.h:126-127 -- per-column symmetric int8 weight quantization. */
void acfun_quantize_weights(const float* w, int K, int N, float* scales, int8_t* wq);

/* ref acfun.h:128-131 -- int8 conv with float I/O.  As in the reference, s_in
 * is ignored and the activation scale is max|x|/127 (src/conv_int8.cpp:63-81);
 * results are bit-identical to the reference on an AVX-512 VNNI host. */
void acfun_conv2d_int8(const float* input, int N, int H, int W, int Cin,
                       const int8_t* wq, const float* wscale, const float* bias,
                       int KH, int KW, int Cout, int stride, int pad,
                       float s_in, float* output, int act);

/* ref acfun.h:136-144 -- ACFUN0 models (src/model.cpp of the reference), the
 * same load-time fusion; weights are uploaded to HBM once at load. */
typedef struct AcfunModel AcfunModel;
AcfunModel* acfun_model_load(const char* path);
void acfun_model_destroy(AcfunModel* m);
int acfun_model_infer(AcfunModel* m, const float* input, float* output);
int acfun_model_output_size(AcfunModel* m);
void acfun_model_input_dims(AcfunModel* m, int* Cin, int* Hin, int* Win);

/* ============ reference internal entry points its tests bind (src/internal.h) ============ */

/* ref internal.h:119-120 -- u8 x s8 -> i32 GEMM. */
void acfun_gemm_int8(int M, int N, int K, const uint8_t* A, const int8_t* B, int32_t* C);
/* ref internal.h:137-139 -- fused (float)acc*alpha[j]+beta[j] (+ReLU) epilogue. */
void acfun_gemm_int8_epi(int M, int N, int K, const uint8_t* A, const int8_t* B, float* C,
                         const float* alpha, const float* beta, int act);
/* ref internal.h:152 -- out = clamp(round(in*inv_s)+zp, 0, 255), round-to-nearest-even
 * (the AVX-512BW rule of src/int8_quantize_avx512.cpp:15-20). */
void acfun_quantize_u8(const float* in, uint8_t* out, size_t n, float inv_s, int zp);
/* ref internal.h:164-167 -- small-K int8 direct conv, pads read zp=128. */
void acfun_conv2d_int8_direct(const uint8_t* inQ, int N, int H, int W, int Cin,
                              const int8_t* wq, const float* alpha, const float* beta,
                              int KH, int KW, int Cout, int stride, int pad,
                              int OH, int OW, float* output, int act);
/* ref internal.h:185-187 -- 1x1/s1/p0 int8 conv on the [M,K] activation matrix. */
void acfun_conv1x1_int8(const uint8_t* inQ, int M, int K, int Cout, const int8_t* wq,
                        const float* alpha, const float* beta, float* output, int act);
/* ref internal.h:198-200 -- int8 3x3/s1/p1 conv, float input quantized in-kernel. */
void acfun_winograd_conv3x3_int8(const float* input, int N, int H, int W, int Cin,
                                 const int8_t* wq, const float* wscale, const float* bias, int Cout,
                                 float s_in, float inv_s, float* output, int act);
/* ref internal.h:50-52 / 59-61 -- Winograd F(2,3) / F(4,3), 3x3/s1/p1. */
void acfun_winograd_conv3x3(const float* input, int N, int H, int W, int Cin,
                            const float* weight, const float* bias, int Cout, float* output, int act);
void acfun_winograd43_conv3x3(const float* input, int N, int H, int W, int Cin,
                              const float* weight, const float* bias, int Cout, float* output,
                              int act);
/* ref internal.h:93-96 -- grouped direct conv (groups>1, not depthwise). */
void acfun_conv2d_grouped(const float* input, int N, int H, int W, int Cin,
                          const float* weight, const float* bias, int KH, int KW, int Cout,
                          int stride, int pad, int groups, float* output, int act);
/* ref internal.h:111-112, 223 -- host thread knobs kept for API compatibility. */
void acfun_set_num_threads_runtime(int n);
int acfun_get_num_threads_runtime(void);
int acfun_effective_cores(void);

/* ===================== new: device pointers, streams, batch ===================== */

/* Last failure as text ("" if none).  Not thread-safe, like the reference's state. */
const char* acfun_last_error(void);

/* Synchronize the library stream of the current device. Returns 0 on success. */
int acfun_sync(void);

/* Device-pointer variants: every pointer must be device memory; work is queued
 * on `stream` (a hipStream_t, NULL = the library stream) and NOT synchronized.
 * Return 0 on success, -1 on a shape or launch error (see acfun_last_error()). */
int acfun_dev_gemm_epi(int M, int N, int K, const float* A, const float* B, float* C,
                       const float* bias, int act, void* stream);
/* acfun_gemm_bf16 on device pointers (bf16 MFMA; operands rounded as the reference's
 * gemm_bf16_avx512.cpp:37-44). */
int acfun_dev_gemm_bf16(int M, int N, int K, const float* A, const float* B, float* C,
                        void* stream);
int acfun_dev_conv2d(const float* input, int N, int H, int W, int Cin,
                     const float* weight, const float* bias, int KH, int KW, int Cout,
                     int stride, int pad, int groups, float* output, int act, void* stream);
int acfun_dev_conv2d_int8(const float* input, int N, int H, int W, int Cin,
                          const int8_t* wq, const float* wscale, const float* bias,
                          int KH, int KW, int Cout, int stride, int pad, float* output,
                          int act, void* stream);
/* The int8-in / int8-out convolution: the requantized int8 output the
 * reference's int8 path has no entry point for (it returns float,
 * src/conv_int8.cpp:63-148), so int8 layers can chain without float tensors.
 * input: s8 NHWC [N,H,W,Cin], the activations quantized with per-tensor scale
 * *s_in (a device float; x = q * s_in, and *s_in == 0 marks an all-zero
 * input).  The float result y is exactly acfun_conv2d_int8's on x with its
 * activation scale equal to *s_in (same routes, epilogues, bias and ReLU);
 * output: s8 NHWC [N,OH,OW,Cout] = clamp(round(y * 127/max|y|), -128, 127)
 * with max over the whole output, and *s_out = max|y|/127 (device; 0 and an
 * all-zero output when max|y| < 1e-12).  out_rule 0 rounds half to even (the
 * rule of acfun_quantize_u8, src/int8_quantize_avx512.cpp:15-20); 1 rounds as
 * the Winograd route quantizes its input (src/winograd_int8.cpp:306-325), so
 * the output equals what a following 3x3/s1/p1 int8 conv would have made of
 * y.  Returns 0, or -1 with acfun_last_error(). */
int acfun_dev_conv2d_int8_q(const int8_t* input, const float* s_in, int N, int H, int W,
                            int Cin, const int8_t* wq, const float* wscale, const float* bias,
                            int KH, int KW, int Cout, int stride, int pad, int8_t* output,
                            float* s_out, int act, int out_rule, void* stream);
/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): acfun_dev_conv2d_int8 with every temporary (quantized
 * activations, prepared weights, absmax partials, scale scalars) carved out of
 * a 64 MiB static device region that each GPU holds for the life of the
 * process; it calls no hipMalloc/hipFree.  A shape needing more than 64 MiB
 * of temporaries (about N*H*W*roundup(Cin,16) + Cout*roundup(KH*KW*
 * roundup(Cin,16),128) bytes) returns -1 with the reason in acfun_last_error().
 * Every call on a device shares that device's region: calls that overlap on one
 * device (two streams, two threads) race; serialize them. */
int acfun_dev_conv2d_int8_noalloc(const float* input, int N, int H, int W, int Cin,
                                  const int8_t* wq, const float* wscale, const float* bias,
                                  int KH, int KW, int Cout, int stride, int pad, float* output,
                                  int act, void* stream);
/* acfun_conv2d_dw (ref acfun.h:77-80, act 0/1) followed by acfun_maxpool or
 * acfun_maxpool_relu (ref acfun.h:105-111, post_relu) on its output: the same
 * result bit for bit, computed in one pass (3x3 depthwise with stride 1 or 2,
 * 3x3 / stride-2 pool with padding 0 or 1, C % 4 == 0, 16-byte aligned
 * buffers) without the depthwise output ever written; other shapes run the
 * two kernels.  output: [N, PH, PW, C]. */
int acfun_dev_conv2d_dw_maxpool(const float* input, int N, int H, int W, int C,
                                const float* weight, const float* bias, int KH, int KW, int stride,
                                int pad, int act, int pool, int pool_stride, int pool_pad,
                                float* output, int post_relu, void* stream);
/* acfun_conv2d_g (ref acfun.h:86-89, act 0/1) followed by acfun_maxpool or
 * acfun_maxpool_relu (ref acfun.h:105-111, post_relu) on its output: the same
 * result bit for bit in one pass for 3x3 grouped convs with 4 or 8 input
 * channels per group and at least 8 (a multiple of 4) output channels per
 * group, a 3x3 / stride-2 pool with padding 0 or 1 and 16-byte aligned
 * buffers; other shapes run the conv and the pool.  output: [N, PH, PW, Cout]. */
int acfun_dev_conv2d_g_maxpool(const float* input, int N, int H, int W, int Cin,
                               const float* weight, const float* bias, int KH, int KW, int Cout,
                               int stride, int pad, int groups, int act, int pool, int pool_stride,
                               int pool_pad, float* output, int post_relu, void* stream);
int acfun_dev_maxpool(const float* input, int N, int H, int W, int C, int pool, int stride,
                      int pad, float* output, int post_relu, void* stream);
int acfun_dev_fc(const float* input, int N, int Cin, const float* weight, const float* bias,
                 int Cout, float* output, int act, void* stream);
int acfun_dev_softmax(const float* input, int rows, int cols, float* output, void* stream);

/* acfun_model_load with options: flags & 1 quantizes every dense conv (type 1)
 * to int8 at load (per-output-channel weights, acfun_quantize_weights rule) and
 * runs it through the acfun_conv2d_int8 rules; other layers stay fp32.  The
 * activation scale of each int8 conv is dynamic and per tensor, i.e. max|x|
 * over the whole batch, exactly as acfun_conv2d_int8 computes it for an N-image
 * input (src/conv_int8.cpp:75-81 of the reference).  flags & 2 (with flags & 1)
 * makes the batched calls run an int8 model image by image instead, so each
 * image gets its own scales and acfun_model_infer's result, as the reference's
 * one-image executor gives it (src/model.cpp:274-349), at lower throughput. */
AcfunModel* acfun_model_load_ex(const char* path, int flags);

/* Batched inference: input [N, inH, inW, inC], output [N, outSize].  Returns
 * outSize (per image), 0 on error.  For fp32 models each image's result is
 * that of acfun_model_infer on it alone, up to the kernels' fp32 rounding (the
 * arithmetic per output element does not depend on the batch).  For int8
 * models (acfun_model_load_ex flags & 1) it is not: every int8 conv quantizes
 * its input with one scale for the whole batch, so an image's result depends
 * on the other images of its batch; with N = 1, or for a model loaded with
 * flags & 2, it is acfun_model_infer's for each image. */
int acfun_model_infer_batch(AcfunModel* m, int N, const float* input, float* output);
/* The same on device pointers, queued on `stream` (not synchronized).  A model
 * holds per-layer device state (Winograd filter transforms made at first use),
 * so one model runs one inference at a time: calls on the same model from
 * different streams must not overlap. */
int acfun_dev_model_infer_batch(AcfunModel* m, int N, const float* input, float* output,
                                void* stream);

/* Kernel timing for measurement.  acfun_prof_enable(1) clears the records and
 * starts launching every kernel of the library with HIP start/stop events that
 * the dispatch itself signals; acfun_prof_enable(0) stops.
 * acfun_prof_kernel_ms() waits for the recorded events and returns the mean
 * execution time in ms of the named kernel (0 if none, -1 on a HIP error) and
 * the launch count in *launches (may be NULL). */
void acfun_prof_enable(int on);
double acfun_prof_kernel_ms(const char* kernel, int* launches);
/* The records as text, one line each, tab-separated:
 *   K  tag  kernel  launches  total_ms    per (tag, kernel name)
 *   L  i type N H W C OH OW OC KH KW stride pad groups int8 fused_into act residual
 *                                         per layer a model ran while timing
 * tag is the model layer (fused index i of an L line) the launch belongs to,
 * -1 outside model inference.  Writes at most len bytes (NUL-terminated) and
 * returns the length the whole report needs (with the NUL), -1 on a HIP error. */
int acfun_prof_report(char* buf, int len);

#ifdef __cplusplus
}
#endif

#endif /* ACFUN_AMD_ACFUN_H */
