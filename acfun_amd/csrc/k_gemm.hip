// k_gemm.hip -- fp32 GEMM and implicit-GEMM convolution on CDNA4 MFMA.
//
// Replaces the reference's blocked AVX-512 GEMM (src/gemm_avx512.cpp:245-337),
// its im2col conv route (src/layers.cpp:39-58,178-194) and the 1x1 route
// (src/layers.cpp:66-101): C[M,N] = A[M,K] * B[K,N] (+bias[n], ReLU).
//
// Kernel shape: 256 threads = 4 waves in a 2x2 grid over a BM x BN tile; each
// wave owns (BM/2) x (BN/2) as (BM/32) x (BN/32) blocks of
// v_mfma_f32_16x16x4f32.  LDS holds A as [BM][BK] and B as [BN][BK], both
// k-contiguous with a 4-float pad, so one ds_read_b128 per block gives a lane
// its operands for four MFMA k-steps: in step j, lane l carries k = 4*(l/16)+j
// for row/col l%16 (A and B use the same k assignment, so every product is
// paired correctly).  Global tiles are prefetched into registers while the
// current LDS tile is consumed (two LDS buffers, one barrier per k-tile).
//
// For convolution A is the im2col view of the NHWC input: row m = output pixel
// (n,oh,ow), column k = (kh,kw,ic); out-of-range taps read 0.  Nothing is
// materialized.  Split-K writes partial tiles to a workspace that a second
// kernel reduces in fixed split order (deterministic) before bias and ReLU.
#include "rt.hpp"

#include <memory>

namespace acfun {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int BK = 16;
constexpr int LDK = BK + 4;  // padded row (floats): rows land 20 banks apart

struct GemmP {
    const float* A;
    const float* B;
    float* C;
    const float* bias;
    long long sA, sB, sC;  // batch strides in elements
    int M, N, K, lda, ldb, ldc;
    int act;
    int splits, kchunk;  // split-K: K range per split (multiple of BK)
    // implicit-conv geometry (CONV = true)
    int H, W, Cin, KW, stride, pad, OH, OW;
};


// Decodes a k index into (kh, kw, ic).
struct Tap {
    int kh, kw, ic;
};
__device__ __forceinline__ Tap decode_k(int k, int Cin, int KW) {
    int tap = k / Cin;
    Tap t;
    t.ic = k - tap * Cin;
    t.kh = tap / KW;
    t.kw = tap - t.kh * KW;
    return t;
}

template <int BM, int BN, bool CONV, bool VA, bool VB>
__global__ __launch_bounds__(256) void k_gemm_f32(GemmP p) {
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int FM = WM / 16, FN = WN / 16;
    // A tile loads: BM rows x 4 float4 (VA) or BM x 16 scalars.
    constexpr int A_VEC_PER_T = BM * 4 / 256;   // float4 per thread
    constexpr int A_SC_PER_T = BM * BK / 256;   // scalars per thread
    constexpr int B_VEC_PER_T = BN * 4 / 256;   // BK rows x BN/4 float4
    constexpr int B_SC_PER_T = BN * BK / 256;
    static_assert(A_VEC_PER_T >= 1 && B_VEC_PER_T >= 1, "tile too small");

    __shared__ __attribute__((aligned(16))) float sA[2][BM * LDK];
    __shared__ __attribute__((aligned(16))) float sB[2][BN * LDK];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm0 = (wave >> 1) * WM;
    const int wn0 = (wave & 1) * WN;

    const int zb = blockIdx.z;
    const int batch = zb / p.splits;
    const int split = zb - batch * p.splits;
    const float* __restrict__ A = p.A + (long long)batch * p.sA;
    const float* __restrict__ B = p.B + (long long)batch * p.sB;

    const int m0 = blockIdx.y * BM;
    const int n0 = blockIdx.x * BN;
    const int kbeg = split * p.kchunk;
    const int kend = min(p.K, kbeg + p.kchunk);
    const int ntiles = (kend - kbeg + BK - 1) / BK;

    // ---- per-thread A row bookkeeping (fixed across the K loop) ----
    constexpr int AR = VA ? A_VEC_PER_T : A_SC_PER_T;
    int arow[AR];
    long long abase[AR];  // CONV: image base offset; plain: row offset
    int aih0[AR], aiw0[AR];
    const int akq = VA ? (tid & 3) * 4 : (tid & 15);
#pragma unroll
    for (int i = 0; i < AR; ++i) {
        int r = VA ? (tid >> 2) + i * 64 : (tid >> 4) + i * 16;
        arow[i] = r;
        int m = m0 + r;
        if (CONV) {
            int mm = m < p.M ? m : 0;
            int hw = p.OH * p.OW;
            int n = mm / hw;
            int rem = mm - n * hw;
            int oh = rem / p.OW;
            int ow = rem - oh * p.OW;
            abase[i] = (long long)n * p.H * p.W * p.Cin;
            aih0[i] = oh * p.stride - p.pad;
            aiw0[i] = ow * p.stride - p.pad;
        } else {
            abase[i] = (long long)m * p.lda;
            aih0[i] = 0;
            aiw0[i] = 0;
        }
    }

    f4 ra[VA ? A_VEC_PER_T : 1];
    float rsa[VA ? 1 : A_SC_PER_T];
    f4 rb[VB ? B_VEC_PER_T : 1];
    float rsb[VB ? 1 : B_SC_PER_T];

    auto load_a = [&](int k0) {
        if (VA) {
            int k = k0 + akq;
            Tap t;
            if (CONV) t = decode_k(k, p.Cin, p.KW);
#pragma unroll
            for (int i = 0; i < A_VEC_PER_T; ++i) {
                f4 v = {0.f, 0.f, 0.f, 0.f};
                int m = m0 + arow[i];
                if (m < p.M && k < kend) {
                    if (CONV) {
                        int ih = aih0[i] + t.kh, iw = aiw0[i] + t.kw;
                        if (ih >= 0 && ih < p.H && iw >= 0 && iw < p.W)
                            v = *(const f4*)(A + abase[i] + ((long long)ih * p.W + iw) * p.Cin + t.ic);
                    } else {
                        v = *(const f4*)(A + abase[i] + k);
                    }
                }
                ra[i] = v;
            }
        } else {
            int k = k0 + akq;
            Tap t;
            if (CONV) t = decode_k(k, p.Cin, p.KW);
#pragma unroll
            for (int i = 0; i < A_SC_PER_T; ++i) {
                float v = 0.f;
                int m = m0 + arow[i];
                if (m < p.M && k < kend) {
                    if (CONV) {
                        int ih = aih0[i] + t.kh, iw = aiw0[i] + t.kw;
                        if (ih >= 0 && ih < p.H && iw >= 0 && iw < p.W)
                            v = A[abase[i] + ((long long)ih * p.W + iw) * p.Cin + t.ic];
                    } else {
                        v = A[abase[i] + k];
                    }
                }
                rsa[i] = v;
            }
        }
    };
    auto store_a = [&](int buf) {
        if (VA) {
#pragma unroll
            for (int i = 0; i < A_VEC_PER_T; ++i) *(f4*)&sA[buf][arow[i] * LDK + akq] = ra[i];
        } else {
#pragma unroll
            for (int i = 0; i < A_SC_PER_T; ++i) sA[buf][arow[i] * LDK + akq] = rsa[i];
        }
    };
    auto load_b = [&](int k0) {
        if (VB) {
#pragma unroll
            for (int i = 0; i < B_VEC_PER_T; ++i) {
                int idx = tid + i * 256;
                int kr = idx / (BN / 4);
                int n4 = (idx - kr * (BN / 4)) * 4;
                int k = k0 + kr, n = n0 + n4;
                f4 v = {0.f, 0.f, 0.f, 0.f};
                if (k < kend && n < p.N) v = *(const f4*)(B + (long long)k * p.ldb + n);
                rb[i] = v;
            }
        } else {
#pragma unroll
            for (int i = 0; i < B_SC_PER_T; ++i) {
                int idx = tid + i * 256;
                int kr = idx / BN;
                int nn = idx - kr * BN;
                int k = k0 + kr, n = n0 + nn;
                rsb[i] = (k < kend && n < p.N) ? B[(long long)k * p.ldb + n] : 0.f;
            }
        }
    };
    auto store_b = [&](int buf) {
        if (VB) {
#pragma unroll
            for (int i = 0; i < B_VEC_PER_T; ++i) {
                int idx = tid + i * 256;
                int kr = idx / (BN / 4);
                int n4 = (idx - kr * (BN / 4)) * 4;
                sB[buf][(n4 + 0) * LDK + kr] = rb[i].x;
                sB[buf][(n4 + 1) * LDK + kr] = rb[i].y;
                sB[buf][(n4 + 2) * LDK + kr] = rb[i].z;
                sB[buf][(n4 + 3) * LDK + kr] = rb[i].w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < B_SC_PER_T; ++i) {
                int idx = tid + i * 256;
                int kr = idx / BN;
                int nn = idx - kr * BN;
                sB[buf][nn * LDK + kr] = rsb[i];
            }
        }
    };

    f4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

    if (ntiles > 0) {
        load_a(kbeg);
        load_b(kbeg);
        store_a(0);
        store_b(0);
        __syncthreads();
    }
    const int lr = lane & 15;
    const int lk = (lane >> 4) * 4;
    for (int t = 0; t < ntiles; ++t) {
        const int buf = t & 1;
        const bool more = (t + 1) < ntiles;
        if (more) {
            load_a(kbeg + (t + 1) * BK);
            load_b(kbeg + (t + 1) * BK);
        }
        f4 fa[FM], fb[FN];
#pragma unroll
        for (int i = 0; i < FM; ++i) fa[i] = *(const f4*)&sA[buf][(wm0 + i * 16 + lr) * LDK + lk];
#pragma unroll
        for (int j = 0; j < FN; ++j) fb[j] = *(const f4*)&sB[buf][(wn0 + j * 16 + lr) * LDK + lk];
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[i][s], fb[j][s], acc[i][j], 0, 0, 0);
        if (more) {
            store_a(buf ^ 1);
            store_b(buf ^ 1);
        }
        __syncthreads();
    }

    // ---- epilogue: D layout of 16x16 MFMA: lane l, reg r -> row 4*(l/16)+r, col l%16
    float* __restrict__ Cb = p.C + (long long)zb * p.sC;
    const bool final_out = (p.splits == 1);
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        int n = n0 + wn0 + j * 16 + lr;
        if (n >= p.N) continue;
        float bv = (final_out && p.bias) ? p.bias[n] : 0.f;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                int m = m0 + wm0 + i * 16 + (lane >> 4) * 4 + r;
                if (m < p.M) {
                    float v = acc[i][j][r];
                    if (final_out) {
                        v = v + bv;
                        v = act_apply(v, p.act);
                    }
                    Cb[(long long)m * p.ldc + n] = v;
                }
            }
        }
    }
}

// Sums split-K partial tiles in split order, then bias and ReLU.
__global__ void k_splitk_reduce(const float* __restrict__ ws, int splits, long long plane, int M,
                                int N, float* __restrict__ C, int ldc, const float* __restrict__ bias,
                                int act) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    long long total = (long long)M * N;
    if (i >= total) return;
    int m = (int)(i / N), n = (int)(i - (long long)m * N);
    float v = ws[i];
    for (int s = 1; s < splits; ++s) v += ws[(long long)s * plane + i];
    if (bias) v = v + bias[n];
    v = act_apply(v, act);
    C[(long long)m * ldc + n] = v;
}

__global__ void k_round_bf16(const float* __restrict__ in, float* __restrict__ out, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    uint32_t u = __float_as_uint(in[i]);
    if ((u & 0x7f800000u) != 0x7f800000u) {   // finite: round to nearest even on bit 16
        u += 0x7fffu + ((u >> 16) & 1u);
    } else if (u & 0x007fffffu) {
        u |= 0x00400000u;                        // quiet NaN
    }
    out[i] = __uint_as_float(u & 0xffff0000u);
}

template <int BM, int BN, bool CONV, bool VA, bool VB>
bool launch_t(const GemmP& p, int batch, hipStream_t s) {
    dim3 grid((p.N + BN - 1) / BN, (p.M + BM - 1) / BM, batch * p.splits);
    {
        ACFUN_LAUNCH("k_gemm_f32", (k_gemm_f32<BM, BN, CONV, VA, VB>), grid, dim3(256), 0, s, p);
    }
    return check_launch("k_gemm_f32");
}

template <int BM, int BN, bool CONV>
bool launch_v(const GemmP& p, int batch, bool va, bool vb, hipStream_t s) {
    if (va && vb) return launch_t<BM, BN, CONV, true, true>(p, batch, s);
    if (va) return launch_t<BM, BN, CONV, true, false>(p, batch, s);
    if (vb) return launch_t<BM, BN, CONV, false, true>(p, batch, s);
    return launch_t<BM, BN, CONV, false, false>(p, batch, s);
}

template <bool CONV>
bool launch_cfg(const GemmP& p, int batch, bool va, bool vb, const TileCfg& c, hipStream_t s) {
    if (c.bm == 128 && c.bn == 128) return launch_v<128, 128, CONV>(p, batch, va, vb, s);
    if (c.bm == 128 && c.bn == 64) return launch_v<128, 64, CONV>(p, batch, va, vb, s);
    if (c.bm == 64 && c.bn == 128) return launch_v<64, 128, CONV>(p, batch, va, vb, s);
    return launch_v<64, 64, CONV>(p, batch, va, vb, s);
}

bool aligned16(const void* q) { return ((uintptr_t)q & 15u) == 0; }

// Runs one (possibly split-K) GEMM problem described by p.
template <bool CONV>
bool run(GemmP p, int batch, bool va, bool vb, hipStream_t s, const TileCfg* force = nullptr) {
    if (p.M <= 0 || p.N <= 0) return true;
    TileCfg c = force ? *force : tuned_f32_tile(p.M, p.N, p.K, batch);
    if (batch > 1) c.split = 1;
    int splits = c.split < 1 ? 1 : c.split;
    int kchunk = (p.K + splits - 1) / splits;
    kchunk = (kchunk + BK - 1) / BK * BK;
    splits = kchunk > 0 ? (p.K + kchunk - 1) / kchunk : 1;
    if (splits < 1) splits = 1;
    if (splits == 1) {
        p.splits = 1;
        p.kchunk = p.K > 0 ? p.K : 1;
        return launch_cfg<CONV>(p, batch, va, vb, c, s);
    }
    long long plane = (long long)p.M * p.N;
    Scratch ws(sizeof(float) * plane * splits, s);
    if (!ws.p) return false;
    float* C = p.C;
    int ldc = p.ldc;
    const float* bias = p.bias;
    int act = p.act;
    p.C = ws.as<float>();
    p.ldc = p.N;
    p.sC = plane;
    p.splits = splits;
    p.kchunk = kchunk;
    p.bias = nullptr;
    p.act = 0;
    if (!launch_cfg<CONV>(p, 1, va, vb, c, s)) return false;
    long long total = plane;
    ACFUN_LAUNCH("k_splitk_reduce", k_splitk_reduce, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                       ws.as<float>(), splits, plane, p.M, p.N, C, ldc, bias, act);
    return check_launch("k_splitk_reduce");
}

}  // namespace

TileCfg default_f32_tile(int M, int N, int K, int batch) {
    const int cus = num_cus();
    const int cand[4][2] = {{128, 128}, {128, 64}, {64, 128}, {64, 64}};
    for (auto& c : cand) {
        if (c[1] > 64 && N <= 64) continue;   // half of every tile would be padding
        if (c[0] > 64 && M <= 64) continue;
        long long tiles = (long long)((M + c[0] - 1) / c[0]) * ((N + c[1] - 1) / c[1]) * batch;
        if (tiles >= cus) return TileCfg{c[0], c[1], 1};
    }
    if (batch > 1) return TileCfg{64, 64, 1};
    long long tiles = (long long)((M + 63) / 64) * ((N + 63) / 64);
    int split = 1;
    if (tiles * 2 <= cus && K >= 512) {
        split = (int)((cus + tiles - 1) / tiles);
        int maxs = K / 256;
        if (split > maxs) split = maxs;
        if (split < 1) split = 1;
    }
    return TileCfg{64, 64, split};
}

// Tile-search candidates (kind "f32"): the four tiles x split-K 1, 2, 4, 8
// (split s needs K >= 256 s).
TileCfg f32_cand(int c) {
    static const int tiles[4][2] = {{128, 128}, {128, 64}, {64, 128}, {64, 64}};
    static const int splits[4] = {1, 2, 4, 8};
    return TileCfg{tiles[c / 4][0], tiles[c / 4][1], splits[c % 4]};
}

TileCfg tuned_f32_tile(int M, int N, int K, int batch) {
    const TileCfg d = default_f32_tile(M, N, K, batch);
    if (batch != 1) return d;
    const std::vector<int> key{M, N, K};
    bool rec = false;
    const int c = tune_lookup("f32", key, 16, &rec);
    if (rec)
        tune_record("f32", key, 16, [M, N, K]() -> TuneRunner {
            const size_t ab = (size_t)M * K * 4, bb = (size_t)K * N * 4, cb = (size_t)M * N * 4;
            if (ab + bb + cb > ((size_t)2 << 30)) return TuneRunner();
            hipStream_t s = lib_stream();
            auto a = std::make_shared<Scratch>(ab, s);
            auto b = std::make_shared<Scratch>(bb, s);
            auto cc = std::make_shared<Scratch>(cb, s);
            if (!a->p || !b->p || !cc->p || hipMemsetD32Async((hipDeviceptr_t)a->p, kTuneFill, ab / 4, s) != hipSuccess ||
                hipMemsetD32Async((hipDeviceptr_t)b->p, kTuneFill, bb / 4, s) != hipSuccess)
                return TuneRunner();
            return [=](int cand, hipStream_t st) {
                const TileCfg t = cand < 0 ? default_f32_tile(M, N, K) : f32_cand(cand);
                if (t.split > 1 && K < 256 * t.split) return false;
                return gemm_f32_cfg(M, N, K, a->as<float>(), b->as<float>(), cc->as<float>(), t, st);
            };
        });
    return c >= 0 ? f32_cand(c) : d;
}

bool gemm_f32(int M, int N, int K, const float* A, int lda, const float* B, int ldb, float* C,
              int ldc, const float* bias, int act, hipStream_t s) {
    GemmP p{};
    p.A = A; p.B = B; p.C = C; p.bias = bias;
    p.M = M; p.N = N; p.K = K; p.lda = lda; p.ldb = ldb; p.ldc = ldc; p.act = act;
    bool va = (K % 4 == 0) && (lda % 4 == 0) && aligned16(A);
    bool vb = (N % 4 == 0) && (ldb % 4 == 0) && aligned16(B);
    if (K <= 0) {  // empty reduction: C = bias / 0 (then ReLU), like the reference loops
        p.K = 0;
    }
    // Few output tiles and a long K (an FC layer): the split-K register-staged
    // kernel spreads K over the CUs that k_gemm32's tiles leave idle (batch-64
    // FC 2048 -> 1000: 40.8 -> 16.7 us; 4096 -> 4096: 76 -> 44 us).
    // ACFUN_FC_SPLITK=0 turns it off.
    static const bool fcs = [] {
        const char* e = getenv("ACFUN_FC_SPLITK");
        return !(e && atoi(e) == 0);
    }();
    const long long t64 = (long long)((M + 63) / 64) * ((N + 63) / 64);
    const bool fc_split = fcs && K >= 1024 && t64 * 4 <= num_cus();
    if (K > 0 && !fc_split && gemm32_ok(M, N, K, A, lda, B, ldb))
        return gemm32_f32(M, N, K, A, lda, B, ldb, C, ldc, bias, act, s);
    return run<false>(p, 1, va, vb, s);
}

bool gemm_f32_cfg(int M, int N, int K, const float* A, const float* B, float* C,
                  const TileCfg& cfg, hipStream_t s) {
    GemmP p{};
    p.A = A; p.B = B; p.C = C; p.M = M; p.N = N; p.K = K; p.lda = K; p.ldb = N; p.ldc = N;
    bool va = (K % 4 == 0) && aligned16(A);
    bool vb = (N % 4 == 0) && aligned16(B);
    return run<false>(p, 1, va, vb, s, &cfg);
}

bool gemm_f32_batched(int batch, int M, int N, int K, const float* A, long long sA, int lda,
                      const float* B, long long sB, int ldb, float* C, long long sC, int ldc,
                      hipStream_t s) {
    GemmP p{};
    p.A = A; p.B = B; p.C = C; p.sA = sA; p.sB = sB; p.sC = sC;
    p.M = M; p.N = N; p.K = K; p.lda = lda; p.ldb = ldb; p.ldc = ldc;
    bool va = (K % 4 == 0) && (lda % 4 == 0) && (sA % 4 == 0) && aligned16(A);
    bool vb = (N % 4 == 0) && (ldb % 4 == 0) && (sB % 4 == 0) && aligned16(B);
    return run<false>(p, batch, va, vb, s);
}

bool conv_igemm_f32(const ConvShape& g, const float* in, const float* w, const float* bias,
                    int Cout, float* out, int act, hipStream_t s) {
    int M = g.N * g.OH * g.OW;
    int K = g.KH * g.KW * g.Cin;
    if (g.KH == 1 && g.KW == 1 && g.stride == 1 && g.pad == 0)
        return gemm_f32(M, Cout, K, in, g.Cin, w, Cout, out, Cout, bias, act, s);
    if (conv32_ok(g, Cout, in, w)) return conv32_f32(g, in, w, bias, Cout, out, act, s);
    if (conv_smallc_ok(g, Cout, in)) return conv_smallc_f32(g, in, w, bias, Cout, out, act, s);
    GemmP p{};
    p.A = in; p.B = w; p.C = out; p.bias = bias;
    p.M = M; p.N = Cout; p.K = K; p.lda = K; p.ldb = Cout; p.ldc = Cout; p.act = act;
    p.H = g.H; p.W = g.W; p.Cin = g.Cin; p.KW = g.KW; p.stride = g.stride; p.pad = g.pad;
    p.OH = g.OH; p.OW = g.OW;
    bool va = (g.Cin % 4 == 0) && aligned16(in);
    bool vb = (Cout % 4 == 0) && aligned16(w);
    return run<true>(p, 1, va, vb, s);
}

bool round_bf16(const float* in, float* out, size_t n, hipStream_t s) {
    if (!n) return true;
    ACFUN_LAUNCH("k_round_bf16", k_round_bf16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, in, out, n);
    return check_launch("k_round_bf16");
}

}  // namespace acfun
