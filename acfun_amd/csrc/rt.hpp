// rt.hpp -- runtime shared by the HIP kernels and the C-ABI layer of
// libacfun_amd.so: device state, the library stream, a stream-ordered caching
// memory pool, host<->device staging for the synchronous reference API, and
// the launchers each kernel file exports.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <functional>
#include <vector>

namespace acfun {

// ----------------------------------------------------------------- errors
void set_error(const char* fmt, ...);
const char* last_error();
// Records `what` + the HIP error string and returns false when e != success.
bool check(hipError_t e, const char* what);
// Checks the launch status of the last kernel.
bool check_launch(const char* kernel);

// ----------------------------------------------------------------- timing
// Kernel timing for measurement.  While enabled (acfun_prof_enable),
// ACFUN_LAUNCH starts a kernel with hipExtLaunchKernelGGL, whose start/stop
// events the dispatch itself signals; acfun_prof_kernel_ms averages, per name,
// the time from the later of its start and the previous timed kernel's stop
// on the same stream to its stop.  Disabled: a plain launch.
bool prof_events(const char* kernel, hipStream_t s, hipEvent_t* start, hipEvent_t* stop);
// Tag for the launches that follow (a model executor sets its layer index;
// -1 outside a model), and one text record per executed model layer; both
// are reported by acfun_prof_report while timing is enabled.
void prof_tag(int tag);
bool prof_on();
void prof_layer(const char* record);
#define ACFUN_LAUNCH(NAME, KERNEL, GRID, BLOCK, SHMEM, STREAM, ...)                               \
    do {                                                                                        \
        hipEvent_t acfun_ev0_, acfun_ev1_;                                                      \
        if (::acfun::prof_events(NAME, STREAM, &acfun_ev0_, &acfun_ev1_))                       \
            hipExtLaunchKernelGGL(KERNEL, GRID, BLOCK, SHMEM, STREAM, acfun_ev0_, acfun_ev1_, 0,  \
                                  __VA_ARGS__);                                                 \
        else                                                                                    \
            hipLaunchKernelGGL(KERNEL, GRID, BLOCK, SHMEM, STREAM, __VA_ARGS__);                \
    } while (0)

// ----------------------------------------------------------------- activation
// Epilogue activation codes: 0 none; 1 ReLU as the reference's fused epilogues
// compute it (max_ps: v > 0 ? v : 0, so NaN and -0.0 become +0); 2 ReLU as a
// separate layer computes it (acfun_relu, src/layers.cpp:10-12: v < 0 -> 0,
// keeping NaN and -0.0), used when the model executor fuses a ReLU layer or a
// residual Add's ReLU into the conv before it.
__device__ __forceinline__ float act_apply(float v, int act) {
    return act == 1 ? (v > 0.f ? v : 0.f) : (act == 2 ? (v < 0.f ? 0.f : v) : v);
}
// The same for a runtime code in a loop over many elements: both ReLU forms
// are computed and picked by the wave-uniform flags (relu1: code 1, relu2:
// code 2), which compiles to selects instead of branches per element.
__device__ __forceinline__ float act_select(float v, bool relu1, bool relu2) {
    const float r1 = v > 0.f ? v : 0.f;
    const float r2 = v < 0.f ? 0.f : v;
    const float r = relu2 ? r2 : v;
    return relu1 ? r1 : r;
}

// ----------------------------------------------------------------- quantization
// The reference's float -> int conversions as its x86 code performs them, so
// that the GPU quantizers agree on every input, NaN included:
// _mm512_cvtps_epi32 / _mm512_cvttps_epi32 (src/int8_quantize_avx512.cpp:15-20,
// src/winograd_int8.cpp:306-319) give the integer indefinite INT_MIN for NaN
// and for |x| >= 2^31; (int)std::lroundf (src/int8_quantize.cpp:33,
// src/winograd_int8.cpp:322) keeps the low 32 bits of glibc's long result,
// which is LONG_MIN (low bits 0) for NaN and |x| >= 2^63.
// x86_cvt(r) takes an already rounded float (rintf / truncf of the value).
__device__ __forceinline__ int x86_cvt(float r) {
    return (r != r || fabsf(r) >= 2147483648.0f) ? (int)0x80000000 : (int)r;
}
__device__ __forceinline__ int x86_lround(float t) {
    if (!(fabsf(t) < 9.2233720368547758e18f)) return 0;
    if (fabsf(t) < 2147483648.0f) return (int)roundf(t);
    return (int)(unsigned)(unsigned long long)(long long)t;   // integral here: the low 32 bits
}
// clamp(r + zp, 0, 255) with the reference's wrapping 32-bit add (_mm512_add_epi32)
__device__ __forceinline__ int x86_u8(int r, int zp) {
    const int v = (int)((unsigned)r + (unsigned)zp);
    return v < 0 ? 0 : (v > 255 ? 255 : v);
}

// ----------------------------------------------------------------- device
// Initializes the current device once (verifies it is gfx950, creates the
// library stream).  Returns false (and sets the error) when no usable GPU.
bool ensure_device();
hipStream_t lib_stream();
int num_cus();
// Resolves a user stream argument: NULL -> library stream.
inline hipStream_t resolve(void* s) { return s ? (hipStream_t)s : lib_stream(); }

// ----------------------------------------------------------------- memory
// Stream-ordered caching pool (policy in pool.hpp): a block returned with
// pool_free(p, s) is handed out again for work on s (ordered after every
// kernel that used it); blocks cached on other streams, including streams
// the caller has since destroyed, are reclaimed for any stream by one device
// synchronization once they add up to 64 MiB.
void* pool_alloc(size_t bytes, hipStream_t s);
void pool_free(void* p, hipStream_t s);
size_t pool_cached_bytes();   // bytes held in the free lists

// RAII scratch buffer from the pool.
struct Scratch {
    void* p = nullptr;
    hipStream_t s = nullptr;
    Scratch() = default;
    Scratch(size_t bytes, hipStream_t st) : s(st) { p = bytes ? pool_alloc(bytes, st) : nullptr; }
    ~Scratch() { if (p) pool_free(p, s); }
    Scratch(const Scratch&) = delete;
    Scratch& operator=(const Scratch&) = delete;
    Scratch(Scratch&& o) noexcept : p(o.p), s(o.s) { o.p = nullptr; }
    Scratch& operator=(Scratch&& o) noexcept {
        if (this != &o) {
            if (p) pool_free(p, s);
            p = o.p;
            s = o.s;
            o.p = nullptr;
        }
        return *this;
    }
    template <class T> T* as() const { return static_cast<T*>(p); }
};

// Device memory for the buffers of one call: taken from the stream-ordered
// pool (and returned to it when the arena goes out of scope), or -- region
// mode -- carved out of a caller-provided device region of `cap` bytes, which
// allocates nothing.  Every buffer starts on a 256-byte boundary.  get()
// returns nullptr (and sets the error) when the pool cannot allocate or the
// region is exhausted.
class Arena {
  public:
    explicit Arena(hipStream_t s) : s_(s) {}
    Arena(hipStream_t s, void* region, size_t cap) : s_(s), base_((char*)region), cap_(cap) {}
    void* get(size_t bytes);
    // Bytes get() has handed out in region mode (with alignment), for size checks.
    size_t used() const { return used_; }
    static size_t aligned(size_t b) { return (b + 255) & ~size_t(255); }

  private:
    hipStream_t s_;
    char* base_ = nullptr;
    size_t cap_ = 0, used_ = 0;
    std::vector<Scratch> owned_;
};

bool is_device_ptr(const void* p);

// Staging for the synchronous host-pointer API (the reference's contract):
// inputs that are host memory are copied to pooled device buffers, outputs
// are allocated on the device and copied back by finish(), which then
// synchronizes the stream.  Device pointers pass through untouched.
class HostCall {
  public:
    explicit HostCall(hipStream_t s) : s_(s) {}
    ~HostCall();
    const void* in(const void* host, size_t bytes);   // read-only operand
    void* out(void* host, size_t bytes);              // write-only result
    void* inout(void* host, size_t bytes);            // read-modify-write
    bool finish();                                    // D2H + sync
    hipStream_t stream() const { return s_; }
    bool failed() const { return failed_; }

  private:
    struct Back { void* host; void* dev; size_t bytes; };
    hipStream_t s_;
    std::vector<void*> owned_;
    std::vector<Back> back_;
    bool failed_ = false;
};

// ----------------------------------------------------------------- launchers
// All launchers take device pointers and a stream and return false on error.

// fp32 implicit GEMM on MFMA: C = A*B (+bias, ReLU).  For conv, A is the
// im2col view of an NHWC tensor, never materialized.
struct ConvShape {
    int N, H, W, Cin, KH, KW, stride, pad, OH, OW;
};
// 64x64-tile 32x32x2-MFMA GEMM with LDS-DMA staging (k_gemm32.hip); gemm32_ok
// says whether its alignment and size conditions hold.
bool gemm32_ok(int M, int N, int K, const float* A, int lda, const float* B, int ldb);
bool gemm32_f32(int M, int N, int K, const float* A, int lda, const float* B, int ldb, float* C,
                int ldc, const float* bias, int act, hipStream_t s, const float* res = nullptr,
                int ldr = 0);
// The same engine as an implicit-GEMM convolution (im2col never materialized)
// when Cin is a multiple of 64 and KH, KW <= 8 (conv32_ok).
bool conv32_ok(const ConvShape& g, int Cout, const float* in, const float* w);
bool conv32_f32(const ConvShape& g, const float* in, const float* w, const float* bias, int Cout,
                float* out, int act, hipStream_t s, const float* res = nullptr, int ldr = 0);
bool gemm_f32(int M, int N, int K, const float* A, int lda, const float* B, int ldb, float* C,
              int ldc, const float* bias, int act, hipStream_t s);
bool conv_igemm_f32(const ConvShape& g, const float* in, const float* w, const float* bias,
                    int Cout, float* out, int act, hipStream_t s);
// Convolutions with few input channels (k_stem.hip): the instantiated (KH, KW,
// Cin) shapes whose input window fits the kernel's LDS, with W * Cin a multiple
// of 4 and a 16-byte aligned input.
bool conv_smallc_ok(const ConvShape& g, int Cout, const float* in);
bool conv_smallc_f32(const ConvShape& g, const float* in, const float* w, const float* bias, int Cout, float* out,
                     int act, hipStream_t s);
// The int8 form (acfun_conv2d_int8's GEMM route, RNE quantization) for the same
// shapes: wq [K][Cout] s8 as the API takes it, the activation scale from nparts
// absmax partials, q8 (16-byte aligned, N*H*W*Cin bytes) a temporary for the
// quantized input; amax (nullable) receives one output-maximum partial per
// workgroup, *grid of them (at most kI8AmaxParts).
bool conv_i8stem(const ConvShape& g, const float* in, const int8_t* wq, const float* ws, const float* bias,
                 int Cout, float* out, int act, const float* part, int nparts, float* amax, int* grid,
                 int8_t* q8, hipStream_t s);
// Batched GEMM (batch = gridDim.z) with fixed strides, no epilogue.
bool gemm_f32_batched(int batch, int M, int N, int K, const float* A, long long sA, int lda,
                      const float* B, long long sB, int ldb, float* C, long long sC, int ldc,
                      hipStream_t s);
bool round_bf16(const float* in, float* out, size_t n, hipStream_t s);
// acfun_gemm_bf16 on bf16 MFMA (k_bf16.hip): C = bf16(A) * bf16(B), fp32 accumulation.
bool gemm_bf16_dev(int M, int N, int K, const float* A, const float* B, float* C, hipStream_t s);

// Winograd 3x3/s1/p1 (tile = 2 for F(2,3), 4 for F(4,3)).
// Upre (F(2,3) only, nullable): the filter transform prepared by wino23_filter
// for this shape's wino23_plan, instead of transforming it in the call.
bool winograd_f32(int tile, const float* in, int N, int H, int W, int Cin, const float* w,
                  const float* bias, int Cout, float* out, int act, hipStream_t s,
                  const float* Upre = nullptr);
// The F(2,3) filter transform, prepared once for repeated calls (a model):
// wino23_plan says which engine and filter layout a shape takes (1 or 0; -1:
// no Winograd engine), wino23_filter writes the transform (wino23_filter_bytes).
int wino23_plan(int N, int H, int W, int Cin, int Cout, const void* in);
size_t wino23_filter_bytes(int Cin, int Cout);
bool wino23_filter(const float* w, int Cin, int Cout, int plan, float* U, hipStream_t s);
// F(4,3): the filter transform in the chunked layout U[Cinp/8][36][Cout][8]
// (Cinp = Cin rounded up to 16, zero-padded), and the persistent unit kernel
// (k_wino43p), which reads it.  run_wino43 sets *done when the shape suits the
// unit kernel and it ran (Cin % 4 == 0, Cin >= 32, a 16-byte aligned input,
// images at least 24 pixels wide, operands within 2 GB, Cout <= 4096);
// otherwise it leaves the call to another engine.
bool wino43_filter(const float* w, int Cin, int Cout, float* U, hipStream_t s);
bool run_wino43(const float* in, int N, int H, int W, int Cin, const float* w, const float* bias,
                int Cout, float* out, int act, hipStream_t s, bool* done);
// The conv2d route's Winograd step: the route names the tile the reference
// would use; both tiles compute the direct convolution exactly over the
// rationals, so the faster kernel for the shape runs (within the Winograd
// tolerance of the reference either way).
bool winograd_route_f32(int tile, const float* in, int N, int H, int W, int Cin, const float* w,
                        const float* bias, int Cout, float* out, int act, hipStream_t s,
                        const float* Upre = nullptr);

// Bandwidth kernels.
bool dwconv_f32(const float* in, int N, int H, int W, int C, const float* w, const float* bias,
                int KH, int KW, int stride, int pad, float* out, int act, hipStream_t s);
// Depthwise 3x3 + activation fused with a following 3x3/2 MaxPool (pool pad 0
// or 1, post_relu): the result of dwconv_f32 then maxpool_f32, bit for bit,
// without the depthwise output in HBM (dwconv_pool_ok says when it applies).
bool dwconv_pool_ok(int H, int W, int C, int KH, int KW, int stride, int pad, int pool,
                    int pstride, int ppad, const void* in, const void* w, const void* out);
bool dwconv_pool_f32(const float* in, int N, int H, int W, int C, const float* w,
                     const float* bias, int stride, int pad, int act, int ppad, float* out,
                     int post_relu, hipStream_t s);
// Grouped 3x3 conv + activation fused with a following 3x3/2 MaxPool (pool
// pad 0 or 1, post_relu): gconv_f32 then maxpool_f32, bit for bit, without the
// conv output in memory (gconv_pool_ok says when it applies: Cin/groups 4 or 8,
// Cout/groups >= 8 and a multiple of 4, 16-byte aligned buffers).
bool gconv_pool_ok(int N, int H, int W, int Cin, int KH, int KW, int Cout, int stride, int pad,
                   int groups, int pool, int pstride, int ppad, const void* in, const void* w,
                   const void* out);
bool gconv_pool_f32(const float* in, int N, int H, int W, int Cin, const float* w,
                    const float* bias, int Cout, int stride, int pad, int groups, int act, int ppad,
                    float* out, int post_relu, hipStream_t s);
bool gconv_f32(const float* in, int N, int H, int W, int Cin, const float* w, const float* bias,
               int KH, int KW, int Cout, int stride, int pad, int groups, float* out, int act,
               hipStream_t s);
bool maxpool_f32(const float* in, int N, int H, int W, int C, int pool, int stride, int pad,
                 float* out, int post_relu, hipStream_t s);
bool relu_f32(float* d, size_t n, int six, hipStream_t s);
bool softmax_f32(const float* in, int rows, int cols, float* out, hipStream_t s);
bool batchnorm_f32(float* d, int size, int channels, const float* mean, const float* var,
                   const float* gamma, const float* beta, float eps, hipStream_t s);
bool fill_f32(float* d, size_t n, float v, hipStream_t s);
// y = a + b (ReLU if act): the residual Add record of version-2 models.
bool add_relu_f32(const float* a, const float* b, float* y, size_t n, int act, hipStream_t s);
// Global average pool [N][HW][C] -> [N][C]: sequential sum over HW, then / HW.
bool gap_f32(const float* x, int N, int HW, int C, float* y, hipStream_t s);
bool group_split_copy(const float* src, int pix, int srcC, int off, int cnt, float* dst,
                      int dstC, int dstOff, hipStream_t s);

// int8 family.
enum class RoundMode : int { RNE = 0, LROUND = 1, WINO = 2 };
bool quantize_weights_dev(const float* w, int K, int N, float* scales, int8_t* wq, hipStream_t s);
bool quantize_u8_dev(const float* in, uint8_t* out, size_t n, float inv_s, int zp, hipStream_t s);
bool gemm_int8_dev(int M, int N, int K, const uint8_t* A, const int8_t* B, int32_t* C,
                   const float* alpha, const float* beta, float* Cf, int act, hipStream_t s);
bool conv1x1_int8_dev(const uint8_t* inQ, int M, int K, int Cout, const int8_t* wq,
                      const float* alpha, const float* beta, float* out, int act, hipStream_t s);
bool conv_int8_direct_dev(const uint8_t* inQ, const ConvShape& g, const int8_t* wq,
                          const float* alpha, const float* beta, int Cout, float* out, int act,
                          hipStream_t s);
// acfun_conv2d_int8 end to end on device (absmax, params, quantize, conv).
// int8 conv weights prepared once for k_igemm_i8: Bt [N][ldb] (row k' = tap*Cinp + ic,
// zero padded) and Sw[N] = the quantized weights' column sums, in memory owned
// by the handle (hipMalloc) until i8_release (hipFree, which waits for the device).
struct I8Weights {
    int8_t* bt = nullptr;
    int* sw = nullptr;
    int ldb = 0, taps = 0, Cin = 0, N = 0;
};
bool i8_prepare(const int8_t* wq, int taps, int Cin, int N, I8Weights& w, hipStream_t s);
void i8_release(I8Weights& w);
// res (nullable): a residual [pixels][Cout] added before the activation (a
// model's Add fused into the conv; the same two roundings as a separate Add).
// amax_out (nullable; kI8AmaxParts floats, zeroed by the caller): per-part
// maxima of the output's |v|, written by the producing kernel itself.
// amax_in (nullable): such partials of the input, from its producer, used in
// place of the absmax pass.
constexpr int kI8AmaxParts = 768;
// A quantized activation tensor shared by several int8 convs that read the same
// input with the same rounding rule (a model's projection shortcut and the
// first conv of its block): q [pix][Cinp] s8 and its 8-float scalar block,
// in memory the caller owns (i8_quant_bytes).  The first call with ready ==
// false quantizes into it and sets ready; later calls skip the absmax and
// quantize passes.  mode: 0 RNE (GEMM routes), 2 the Winograd route's rule.
struct I8Quant {
    int8_t* q = nullptr;
    float* scal = nullptr;
    int mode = -1;
    bool ready = false;
};
size_t i8_quant_bytes(long long pix, int Cin);      // q plus the scalar block
// A requantized s8 output (a model's int8 chain): q [pixo][ldo], ldo = Cout
// rounded up to 16 (columns Cout.. written 0), *s_out = max|y|/127 (0 for an
// all-zero y), rounded with rule (0 RNE; 1 the Winograd route's input rule),
// the values acfun_conv2d_int8's consumer would quantize y to.
struct I8Out {
    int8_t* q = nullptr;
    int ldo = 0;
    float* s_out = nullptr;
    int rule = 0;
    // true: for K < 512 recompute the tile in a second pass instead of storing
    // and requantizing the fp32 output (the API entry's choice); false: always
    // one fp32 pass and the requantizer (what a model's chain measured faster)
    bool recompute = true;
};
// q8out (nullable): write the s8 output instead of out (res and amax_out unused).
bool conv2d_int8_dev(const float* in, const ConvShape& g, const int8_t* wq, const float* ws,
                     const float* bias, int Cout, float* out, int act, hipStream_t s,
                     const I8Weights* pre = nullptr, const float* res = nullptr,
                     float* amax_out = nullptr, const float* amax_in = nullptr,
                     I8Quant* shared = nullptr, const I8Out* q8out = nullptr);
// The same on an s8 input of a chain: q [pix][Cin rounded up to 16] with scale
// *s_in (device; 0 = all-zero input) and prepared weights; fp32 output (out,
// res, amax_out as above) or, with q8out, s8.
bool conv2d_int8_s8in_dev(const int8_t* q, const float* s_in, const ConvShape& g,
                          const I8Weights& pre, const float* ws, const float* bias, int Cout,
                          float* out, int act, hipStream_t s, const float* res, float* amax_out,
                          const I8Out* q8out);
// The int8-in / int8-out convolution (a requantized s8 output): s8 activations
// q [pix][ldq_in = roundup(Cin,16)] with per-tensor scale *s_in (device; 0 =
// all-zero input) -> s8 out [pixo][ldo] (ldo a multiple of 16, columns Cout..
// zero) and *s_out = max|y|/127, y being what acfun_conv2d_int8's route computes
// with activation scale *s_in.  rule 0 rounds y*127/max|y| to nearest even;
// rule 1 as the Winograd route quantizes its input.  Two passes of k_i8mm.
bool conv2d_int8_q8_dev(const int8_t* q, int ldq_in, const float* s_in, const ConvShape& g,
                        const int8_t* wq, const float* ws, const float* bias, int Cout,
                        int8_t* out, int ldo, float* s_out, int act, int rule, hipStream_t s,
                        const I8Weights* pre = nullptr);
// The same on unpadded NHWC s8 tensors [N,H,W,Cin] -> [N,OH,OW,Cout].
bool conv2d_int8_q8_api(const int8_t* in, const float* s_in, const ConvShape& g,
                        const int8_t* wq, const float* ws, const float* bias, int Cout,
                        int8_t* out, float* s_out, int act, int rule, hipStream_t s);
// The same on a file-scope static device region (no allocation, no free):
// conv2d_int8_noalloc_need bytes must not exceed conv2d_int8_noalloc_max().
// Calls that overlap on one device share the region and race.
bool conv2d_int8_noalloc(const float* in, const ConvShape& g, const int8_t* wq, const float* ws,
                         const float* bias, int Cout, float* out, int act, hipStream_t s);
size_t conv2d_int8_noalloc_need(const ConvShape& g, int Cout);
size_t conv2d_int8_noalloc_max();
// The int8 Winograd-route entry with caller-supplied scales.
bool winograd_int8_dev(const float* in, int N, int H, int W, int Cin, const int8_t* wq,
                       const float* ws, const float* bias, int Cout, float s_in, float inv_s,
                       float* out, int act, hipStream_t s);

// fp32 convolution routing exactly as the reference's conv2d_impl
// (src/layers.cpp:106-195).
// wino_U (nullable): a prepared F(2,3) filter transform, used when the route
// is Winograd and the shape's plan matches the one it was prepared for.
bool conv2d_route_f32(const float* in, int N, int H, int W, int Cin, const float* w,
                      const float* bias, int KH, int KW, int Cout, int stride, int pad,
                      int groups, float* out, int act, hipStream_t s,
                      const float* wino_U = nullptr);

// The tile search (tune.cpp).  A kernel family (kind "g32", "i8mm", "w23",
// "f32") asks tune_lookup for the searched candidate of a shape (key) among its
// ncand candidates: -1 when the search has not covered (arch, kind, key,
// ncand), and then *record is set the
// first time the shape is seen in this process, so that the caller registers
// it with tune_record: ncand candidates and a maker that, called by the
// search, allocates scratch operands of the shape and returns a runner that
// launches candidate c on them (false: the shape does not admit c).
using TuneRunner = std::function<bool(int cand, hipStream_t s)>;
using TuneMaker = std::function<TuneRunner()>;
const char* device_arch();      // the current device's gfx name, e.g. "gfx950"
int tune_lookup(const char* kind, const std::vector<int>& key, int ncand, bool* record);
void tune_record(const char* kind, const std::vector<int>& key, int ncand, TuneMaker maker);
bool autotune_wanted();         // ACFUN_AUTOTUNE=1: true at the first ask of a process
// The replays fill their fp32 operands with this bit pattern (0.01f), not
// zeros, so the MFMA units see ordinary data.
constexpr unsigned kTuneFill = 0x3c23d70au;
void gemm32_register(int M, int N, int K);   // a GEMM shape for the next search
void autotune_run();
const char* tune_status();

// k_gemm_f32 tiles (the unaligned fallback).
struct TileCfg { int bm, bn, split; };
TileCfg default_f32_tile(int M, int N, int K, int batch = 1);
TileCfg tuned_f32_tile(int M, int N, int K, int batch = 1);
// Runs one fp32 GEMM with an explicit tile config (used by the tile search).
bool gemm_f32_cfg(int M, int N, int K, const float* A, const float* B, float* C,
                  const TileCfg& cfg, hipStream_t s);

}  // namespace acfun
