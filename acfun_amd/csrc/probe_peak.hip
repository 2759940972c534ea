// Attainable-peak probe for gfx950: what this chip's MFMA units and HBM deliver
// to a kernel that does nothing else, beside which the library's roofline
// fractions (quoted against the published peaks) can be read.
//
//   make -C acfun_amd/csrc probe   ->  acfun_amd/probe_peak
//
// MFMA: every wave of every block keeps four independent accumulator chains of
// one MFMA shape busy for `iters` x 32 instructions; FLOPs = waves x MFMAs x
// the instruction's 2*M*N*K.  s_memtime / s_memrealtime (100 MHz) give the
// shader clock over the run.
// fp32 MFMA beside VALU work: whether v_mfma_f32_32x32x2f32 and v_fma_f32
// share the SIMD's time (the transforms of a Winograd kernel are fp32 VALU
// work next to its fp32 MFMAs).  Per iteration 8 MFMAs (independent
// accumulators) and/or 8 x V fmas (16 independent chains), either in one
// wave interleaved MFMA, V fmas, MFMA, ... or in two waves of one SIMD.
// HBM: a grid-stride float4 read (sum) and copy over buffers of 4 GiB, far
// beyond the 256 MB last-level cache, timed after one untimed pass.
// Launch floor: 500 back-to-back launches of a kernel that does nothing (its
// one store is never taken), at several grid / block / dynamic-LDS shapes,
// between two events on the null stream; and the same launches replayed
// from a HIP graph of 20.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

#define CHECK(x)                                                                        \
  do {                                                                                  \
    hipError_t e_ = (x);                                                                \
    if (e_ != hipSuccess) {                                                             \
      std::fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
      std::exit(1);                                                                     \
    }                                                                                   \
  } while (0)

typedef float f16v __attribute__((ext_vector_type(16)));
typedef int i16v __attribute__((ext_vector_type(16)));
typedef int i4v __attribute__((ext_vector_type(4)));
typedef __bf16 bf8v __attribute__((ext_vector_type(8)));

__global__ void k_nothing(float* p) {
  if (p && threadIdx.x == 1u << 30) p[0] = 1.f;
}

template <int KIND>
__global__ __launch_bounds__(256) void k_peak(float* out, int iters, unsigned long long* clk) {
  const int l = threadIdx.x;
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  float r = 0.f;
  if constexpr (KIND == 0) {
    f16v a0 = {}, a1 = {}, a2 = {}, a3 = {};
    const float x = (float)l * 1e-3f, y = 1.0001f;
    for (int i = 0; i < iters; ++i) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        a0 = __builtin_amdgcn_mfma_f32_32x32x2f32(x, y, a0, 0, 0, 0);
        a1 = __builtin_amdgcn_mfma_f32_32x32x2f32(x, y, a1, 0, 0, 0);
        a2 = __builtin_amdgcn_mfma_f32_32x32x2f32(x, y, a2, 0, 0, 0);
        a3 = __builtin_amdgcn_mfma_f32_32x32x2f32(x, y, a3, 0, 0, 0);
      }
    }
    for (int e = 0; e < 16; ++e) r += a0[e] + a1[e] + a2[e] + a3[e];
  } else if constexpr (KIND == 1) {
    i16v a0 = {}, a1 = {}, a2 = {}, a3 = {};
    const i4v x = {l, l + 1, l + 2, l + 3}, y = {1, 2, 3, 4};
    for (int i = 0; i < iters; ++i) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        a0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(x, y, a0, 0, 0, 0);
        a1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(x, y, a1, 0, 0, 0);
        a2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(x, y, a2, 0, 0, 0);
        a3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(x, y, a3, 0, 0, 0);
      }
    }
    for (int e = 0; e < 16; ++e) r += (float)(a0[e] + a1[e] + a2[e] + a3[e]);
  } else {
    f16v a0 = {}, a1 = {}, a2 = {}, a3 = {};
    bf8v x, y;
    for (int e = 0; e < 8; ++e) {
      x[e] = (__bf16)(float)(l + e);
      y[e] = (__bf16)1.0f;
    }
    for (int i = 0; i < iters; ++i) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        a0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, y, a0, 0, 0, 0);
        a1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, y, a1, 0, 0, 0);
        a2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, y, a2, 0, 0, 0);
        a3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, y, a3, 0, 0, 0);
      }
    }
    for (int e = 0; e < 16; ++e) r += a0[e] + a1[e] + a2[e] + a3[e];
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
  out[blockIdx.x * 256 + l] = r;
  if (l == 0 && blockIdx.x == 0) {
    clk[0] = t1 - t0;
    clk[1] = r1 - r0;
  }
}

// MODE 0: MFMA only, 1: fma only, 2: both in each wave, 3: waves 0-3 MFMA and
// waves 4-7 fma (512 threads: two waves per SIMD); MODE 0-2 use waves 0-3
template <int MODE, int V>
__global__ __launch_bounds__(512, 1) void k_overlap(float* out, int iters) {
  const int w = threadIdx.x >> 6;
  const bool mf = MODE == 0 || MODE == 2 || (MODE == 3 && w < 4);
  const bool va = MODE == 1 || MODE == 2 || (MODE == 3 && w >= 4);
  if (MODE != 3 && w >= 4) return;
  f16v acc[8];
  for (int k = 0; k < 8; ++k)
    for (int e = 0; e < 16; ++e) acc[k][e] = 0.f;
  float x[16];
  for (int i = 0; i < 16; ++i) x[i] = threadIdx.x * 1e-3f + i;
  const float a = threadIdx.x * 0.5f, b = 1.0f / (threadIdx.x + 1);
  for (int it = 0; it < iters; ++it) {
    if (mf && va) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        acc[k] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[k], 0, 0, 0);
#pragma unroll
        for (int v = 0; v < V; ++v) x[(k * V + v) & 15] = fmaf(x[(k * V + v) & 15], 1.0001f, 0.5f);
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, V, 0);
      }
    } else if (mf) {
#pragma unroll
      for (int k = 0; k < 8; ++k) acc[k] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[k], 0, 0, 0);
    } else if (va) {
#pragma unroll
      for (int k = 0; k < 8 * V; ++k) x[k & 15] = fmaf(x[k & 15], 1.0001f, 0.5f);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  float r = 0.f;
  for (int k = 0; k < 8; ++k) r += acc[k][0] + acc[k][15];
  for (int i = 0; i < 16; ++i) r += x[i];
  out[blockIdx.x * 512 + threadIdx.x] = r;
}

// grid-stride float4 sum: one partial per thread, so the loads cannot be elided
__global__ __launch_bounds__(256) void k_read(const float4* __restrict__ a, size_t n4,
                                              float* __restrict__ part) {
  const size_t stride = (size_t)gridDim.x * 256;
  float s = 0.f;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride) {
    const float4 v = a[i];
    s += v.x + v.y + v.z + v.w;
  }
  part[(size_t)blockIdx.x * 256 + threadIdx.x] = s;
}

__global__ __launch_bounds__(256) void k_copy(const float4* __restrict__ a, float4* __restrict__ b,
                                              size_t n4) {
  const size_t stride = (size_t)gridDim.x * 256;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride) b[i] = a[i];
}

int main() {
  hipDeviceProp_t pr;
  CHECK(hipGetDeviceProperties(&pr, 0));
  const int cus = pr.multiProcessorCount;
  std::printf("device %s, %d CUs, clockRate %d kHz\n", pr.gcnArchName, cus, pr.clockRate);
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));

  float* out;
  unsigned long long* clk;
  CHECK(hipMalloc(&out, (size_t)2 * cus * 256 * sizeof(float)));
  CHECK(hipMalloc(&clk, 16));
  const int iters = 2000;
  const char* names[3] = {"fp32 mfma_f32_32x32x2f32  ", "int8 mfma_i32_32x32x32_i8 ",
                          "bf16 mfma_f32_32x32x16_bf16"};
  const double ops[3] = {32. * 32 * 2 * 2, 32. * 32 * 32 * 2, 32. * 32 * 16 * 2};
  const double published[3] = {157.3, 5000.0, 2500.0};
  for (int kind = 0; kind < 3; ++kind) {
    for (int bpc : {1, 2}) {
      const int blocks = cus * bpc;
      auto run = [&]() {
        if (kind == 0) hipLaunchKernelGGL(k_peak<0>, dim3(blocks), dim3(256), 0, 0, out, iters, clk);
        if (kind == 1) hipLaunchKernelGGL(k_peak<1>, dim3(blocks), dim3(256), 0, 0, out, iters, clk);
        if (kind == 2) hipLaunchKernelGGL(k_peak<2>, dim3(blocks), dim3(256), 0, 0, out, iters, clk);
        CHECK(hipGetLastError());
      };
      run();
      CHECK(hipDeviceSynchronize());
      CHECK(hipEventRecord(e0, 0));
      run();
      CHECK(hipEventRecord(e1, 0));
      CHECK(hipEventSynchronize(e1));
      float ms;
      CHECK(hipEventElapsedTime(&ms, e0, e1));
      unsigned long long h[2];
      CHECK(hipMemcpy(h, clk, 16, hipMemcpyDeviceToHost));
      const double mfmas = (double)blocks * 4 * iters * 32;
      const double rate = mfmas * ops[kind] / (ms * 1e-3) / 1e12;
      std::printf("%s  blocks/CU %d: %8.3f ms  %8.1f T(FL)OP/s  (%.3f of published %.1f)  "
                  "shader clock %.3f GHz\n",
                  names[kind], bpc, ms, rate, rate / published[kind], published[kind],
                  (double)h[0] / ((double)h[1] * 10.0));
    }
  }

  {
    // fp32 MFMA beside fp32 VALU: one workgroup per CU, MFMA work on four waves
    const int it2 = 20000;
    auto timed = [&](auto launch) {
      launch(10);
      CHECK(hipGetLastError());
      CHECK(hipDeviceSynchronize());
      CHECK(hipEventRecord(e0, 0));
      launch(it2);
      CHECK(hipEventRecord(e1, 0));
      CHECK(hipEventSynchronize(e1));
      float ms;
      CHECK(hipEventElapsedTime(&ms, e0, e1));
      return ms;
    };
#define ACFUN_OVL(MODE, V)                                                                        \
  timed([&](int n) { hipLaunchKernelGGL((k_overlap<MODE, V>), dim3(cus), dim3(512), 0, 0, out2, n); })
    float* out2;
    CHECK(hipMalloc(&out2, (size_t)cus * 512 * sizeof(float)));
    const float m0 = ACFUN_OVL(0, 8);
    std::printf("fp32 MFMA / VALU overlap, %d iterations of 8 MFMAs and/or 8 x V v_fma_f32 per wave:\n", it2);
    std::printf("  MFMA only            %7.3f ms\n", m0);
    const float v4 = ACFUN_OVL(1, 4), v8 = ACFUN_OVL(1, 8), v15 = ACFUN_OVL(1, 15);
    const float b4 = ACFUN_OVL(2, 4), b8 = ACFUN_OVL(2, 8), b15 = ACFUN_OVL(2, 15);
    const float w4 = ACFUN_OVL(3, 4), w8 = ACFUN_OVL(3, 8), w15 = ACFUN_OVL(3, 15);
#undef ACFUN_OVL
    const float vs[3] = {v4, v8, v15}, bs[3] = {b4, b8, b15}, ws[3] = {w4, w8, w15};
    const int Vs[3] = {4, 8, 15};
    for (int i = 0; i < 3; ++i)
      std::printf("  V=%2d: fma only %7.3f ms | one wave, interleaved %7.3f ms | MFMA wave + fma wave "
                  "%7.3f ms | sum %7.3f, max %7.3f\n",
                  Vs[i], vs[i], bs[i], ws[i], m0 + vs[i], m0 > vs[i] ? m0 : vs[i]);
    CHECK(hipFree(out2));
  }

  const size_t bytes = (size_t)4 << 30;
  const size_t n4 = bytes / sizeof(float4);
  float4 *a, *b;
  float* part;
  CHECK(hipMalloc(&a, bytes));
  CHECK(hipMalloc(&b, bytes));
  CHECK(hipMemset(a, 0, bytes));
  for (int bpc : {4, 8, 16}) {
    const int blocks = cus * bpc;
    CHECK(hipMalloc(&part, (size_t)blocks * 256 * sizeof(float)));
    for (int pass = 0; pass < 2; ++pass) {
      hipLaunchKernelGGL(k_read, dim3(blocks), dim3(256), 0, 0, a, n4, part);
      CHECK(hipGetLastError());
      hipLaunchKernelGGL(k_copy, dim3(blocks), dim3(256), 0, 0, a, b, n4);
      CHECK(hipGetLastError());
    }
    CHECK(hipDeviceSynchronize());
    float ms_r, ms_c;
    CHECK(hipEventRecord(e0, 0));
    hipLaunchKernelGGL(k_read, dim3(blocks), dim3(256), 0, 0, a, n4, part);
    CHECK(hipEventRecord(e1, 0));
    CHECK(hipEventSynchronize(e1));
    CHECK(hipEventElapsedTime(&ms_r, e0, e1));
    CHECK(hipEventRecord(e0, 0));
    hipLaunchKernelGGL(k_copy, dim3(blocks), dim3(256), 0, 0, a, b, n4);
    CHECK(hipEventRecord(e1, 0));
    CHECK(hipEventSynchronize(e1));
    CHECK(hipEventElapsedTime(&ms_c, e0, e1));
    std::printf("hbm read 4 GiB   blocks/CU %2d: %8.3f ms  %7.1f GB/s (%.3f of 8000)\n", bpc, ms_r,
                bytes / (ms_r * 1e-3) / 1e9, bytes / (ms_r * 1e-3) / 8e12);
    std::printf("hbm copy 4+4 GiB blocks/CU %2d: %8.3f ms  %7.1f GB/s (%.3f of 8000)\n", bpc, ms_c,
                2.0 * bytes / (ms_c * 1e-3) / 1e9, 2.0 * bytes / (ms_c * 1e-3) / 8e12);
    CHECK(hipFree(part));
  }
  CHECK(hipFree(a));
  CHECK(hipFree(b));

  {
    CHECK(hipFuncSetAttribute((const void*)k_nothing, hipFuncAttributeMaxDynamicSharedMemorySize, 64 * 1024));
    const int shapes[][3] = {{1, 64, 0}, {224, 256, 0}, {224, 512, 60000}, {1024, 256, 0}, {2048, 256, 0}};
    for (const auto& sh : shapes) {
      auto launch = [&](hipStream_t st) {
        hipLaunchKernelGGL(k_nothing, dim3(sh[0]), dim3(sh[1]), sh[2], st, nullptr);
      };
      for (int i = 0; i < 20; ++i) launch(0);
      CHECK(hipGetLastError());
      CHECK(hipDeviceSynchronize());
      CHECK(hipEventRecord(e0, 0));
      for (int i = 0; i < 500; ++i) launch(0);
      CHECK(hipEventRecord(e1, 0));
      CHECK(hipEventSynchronize(e1));
      float ms;
      CHECK(hipEventElapsedTime(&ms, e0, e1));
      std::printf("empty kernel, grid %5d x %4d threads, %5d B LDS: %.2f us per launch back to back\n",
                  sh[0], sh[1], sh[2], ms * 1e3 / 500);
    }
    hipStream_t st;
    CHECK(hipStreamCreate(&st));
    hipGraph_t g;
    hipGraphExec_t ge;
    CHECK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal));
    for (int i = 0; i < 20; ++i) hipLaunchKernelGGL(k_nothing, dim3(224), dim3(512), 60000, st, nullptr);
    CHECK(hipStreamEndCapture(st, &g));
    CHECK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
    for (int i = 0; i < 5; ++i) CHECK(hipGraphLaunch(ge, st));
    CHECK(hipStreamSynchronize(st));
    CHECK(hipEventRecord(e0, st));
    for (int i = 0; i < 25; ++i) CHECK(hipGraphLaunch(ge, st));
    CHECK(hipEventRecord(e1, st));
    CHECK(hipEventSynchronize(e1));
    float ms;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    std::printf("empty kernel, grid   224 x  512 threads, 60000 B LDS: %.2f us per launch in a graph of 20\n",
                ms * 1e3 / 500);
    CHECK(hipGraphExecDestroy(ge));
    CHECK(hipGraphDestroy(g));
    CHECK(hipStreamDestroy(st));
  }
  CHECK(hipFree(out));
  CHECK(hipFree(clk));
  return 0;
}
