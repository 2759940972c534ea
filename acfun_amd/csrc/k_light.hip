// k_light.hip -- bandwidth-bound kernels: depthwise conv, grouped conv,
// MaxPool, ReLU/ReLU6, softmax, unfused BatchNorm and small copies.
//
// These move bytes, not FLOPs, so there is no MFMA here: every kernel maps one
// lane to one output element with the channel index fastest, so a wavefront
// reads and writes contiguous NHWC channel runs (coalesced HBM access).
//
// Rounding follows the reference's AVX-512 host paths operation for operation
// (the library is built with -ffp-contract=off, fmaf is written where the
// reference fuses), so results are bit-identical, not just close:
//   depthwise  src/dw_avx512.cpp:20-69      bias, then fmaf per tap (kh,kw), OOB tap = 0
//   grouped    src/group_conv.cpp:60-79     fmaf chain from bias over (kh,kw,ic) for the
//                                           vector channels, mul+add for the scalar path
//   maxpool    src/maxpool_avx512.cpp:15-62 max from -1e30 over in-range taps
#include "rt.hpp"

namespace acfun {
namespace {

__device__ __forceinline__ float vmax(float a, float b) { return a > b ? a : b; }  // max_ps
typedef float f4 __attribute__((ext_vector_type(4)));

// Depthwise conv: weights [C][KH][KW]; act==1 -> ReLU (max_ps semantics).
__global__ void k_dwconv(const float* __restrict__ in, int N, int H, int W, int C,
                         const float* __restrict__ w, const float* __restrict__ bias, int KH,
                         int KW, int stride, int pad, int OH, int OW, float* __restrict__ out,
                         int act) {
    long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    long long total = (long long)N * OH * OW * C;
    if (idx >= total) return;
    int c = (int)(idx % C);
    long long p = idx / C;
    int ow = (int)(p % OW);
    p /= OW;
    int oh = (int)(p % OH);
    int n = (int)(p / OH);
    const float* wc = w + (long long)c * KH * KW;
    float acc = bias ? bias[c] : 0.0f;
    const float* img = in + (long long)n * H * W * C + c;
    for (int kh = 0; kh < KH; ++kh) {
        int ih = oh * stride - pad + kh;
        for (int kw = 0; kw < KW; ++kw) {
            int iw = ow * stride - pad + kw;
            float v = (ih >= 0 && ih < H && iw >= 0 && iw < W) ? img[((long long)ih * W + iw) * C] : 0.0f;
            acc = fmaf(v, wc[kh * KW + kw], acc);
        }
    }
    if (act == 1) acc = vmax(acc, 0.0f);
    out[idx] = acc;
}

// Depthwise 3x3 for C % 4 == 0: one lane computes 4 channels with float4
// loads (same per-channel arithmetic as k_dwconv).
__global__ void k_dwconv3_c4(const float4* __restrict__ in, int N, int H, int W, int C4,
                             const float* __restrict__ w, const float* __restrict__ bias,
                             int stride, int pad, int OH, int OW, float4* __restrict__ out,
                             int act) {
    long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    long long total = (long long)N * OH * OW * C4;
    if (idx >= total) return;
    int c4 = (int)(idx % C4);
    long long p = idx / C4;
    int ow = (int)(p % OW);
    p /= OW;
    int oh = (int)(p % OH);
    int n = (int)(p / OH);
    int c = c4 * 4;
    float4 acc = bias ? make_float4(bias[c], bias[c + 1], bias[c + 2], bias[c + 3])
                      : make_float4(0.f, 0.f, 0.f, 0.f);
    const float4* img = in + (long long)n * H * W * C4 + c4;
#pragma unroll
    for (int kh = 0; kh < 3; ++kh) {
        int ih = oh * stride - pad + kh;
#pragma unroll
        for (int kw = 0; kw < 3; ++kw) {
            int iw = ow * stride - pad + kw;
            float4 v = (ih >= 0 && ih < H && iw >= 0 && iw < W) ? img[((long long)ih * W + iw) * C4]
                                                                 : make_float4(0.f, 0.f, 0.f, 0.f);
            int t = kh * 3 + kw;
            acc.x = fmaf(v.x, w[(c + 0) * 9 + t], acc.x);
            acc.y = fmaf(v.y, w[(c + 1) * 9 + t], acc.y);
            acc.z = fmaf(v.z, w[(c + 2) * 9 + t], acc.z);
            acc.w = fmaf(v.w, w[(c + 3) * 9 + t], acc.w);
        }
    }
    if (act == 1) {
        acc.x = vmax(acc.x, 0.f); acc.y = vmax(acc.y, 0.f);
        acc.z = vmax(acc.z, 0.f); acc.w = vmax(acc.w, 0.f);
    }
    out[idx] = acc;
}

// Depthwise 3x3, stride S (1 or 2), C % 4 == 0: a lane owns 4 channels and an
// OHB x OWB = 2 x 4 block of outputs.  Its 36 weights stay in registers and
// each of the (OHB-1)*S+3 input rows is loaded once, as (OWB-1)*S+3 columns,
// for every output it feeds.  Per channel the arithmetic is the reference's
// AVX-512 path (src/dw_avx512.cpp:20-69): acc = bias, then one fmaf per
// in-range tap in kh, kw order; out-of-range taps are skipped.
// Lane index = ((n*nOHB + ohb)*nOWB + owb)*C4 + c4 (channel quads fastest,
// so a wave's loads and stores cover whole pixels).
template <int S>
__global__ __launch_bounds__(256) void k_dwconv3_blk(const float4* __restrict__ in, int H, int W,
                                                     int C4, const float* __restrict__ w,
                                                     const float* __restrict__ bias, int pad,
                                                     int OH, int OW, int nOHB, int nOWB,
                                                     int total, float4* __restrict__ out, int act) {
    constexpr int OWB = 4, OHB = 2, NCOL = (OWB - 1) * S + 3, NROW = (OHB - 1) * S + 3;
    const int t = blockIdx.x * 256 + threadIdx.x;
    if (t >= total) return;
    int q = t / C4;
    const int c4 = t - q * C4;
    const int owb = q % nOWB;
    q /= nOWB;
    const int ohb = q % nOHB;
    const int n = q / nOHB;
    const int ow0 = owb * OWB, oh0 = ohb * OHB;
    const int c = c4 * 4;
    float wk[4][9];
    {
        const float4* w4 = (const float4*)(w + (size_t)c * 9);   // 36 floats, 16-byte aligned
#pragma unroll
        for (int i = 0; i < 9; ++i) {
            float4 v = w4[i];
            wk[(4 * i + 0) / 9][(4 * i + 0) % 9] = v.x;
            wk[(4 * i + 1) / 9][(4 * i + 1) % 9] = v.y;
            wk[(4 * i + 2) / 9][(4 * i + 2) % 9] = v.z;
            wk[(4 * i + 3) / 9][(4 * i + 3) % 9] = v.w;
        }
    }
    float4 b4 = bias ? make_float4(bias[c], bias[c + 1], bias[c + 2], bias[c + 3])
                     : make_float4(0.f, 0.f, 0.f, 0.f);
    float4 acc[OHB][OWB];
#pragma unroll
    for (int r = 0; r < OHB; ++r)
#pragma unroll
        for (int o = 0; o < OWB; ++o) acc[r][o] = b4;
    const float4* img = in + (size_t)n * H * W * C4 + c4;
    const int iw0 = ow0 * S - pad, ih0 = oh0 * S - pad;
#pragma unroll
    for (int ir = 0; ir < NROW; ++ir) {
        const int ih = ih0 + ir;
        const bool rok = (unsigned)ih < (unsigned)H;
        float4 col[NCOL];
        bool cok[NCOL];
#pragma unroll
        for (int j = 0; j < NCOL; ++j) {
            const int iw = iw0 + j;
            cok[j] = rok && (unsigned)iw < (unsigned)W;
            col[j] = cok[j] ? img[((size_t)ih * W + iw) * C4] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int r = 0; r < OHB; ++r) {
            const int kh = ir - r * S;                   // tap row of output row oh0 + r
            if (kh < 0 || kh > 2) continue;
#pragma unroll
            for (int o = 0; o < OWB; ++o) {
#pragma unroll
                for (int kw = 0; kw < 3; ++kw) {
                    const int j = o * S + kw;
                    const int tp = kh * 3 + kw;
                    if (cok[j]) {
                        acc[r][o].x = fmaf(col[j].x, wk[0][tp], acc[r][o].x);
                        acc[r][o].y = fmaf(col[j].y, wk[1][tp], acc[r][o].y);
                        acc[r][o].z = fmaf(col[j].z, wk[2][tp], acc[r][o].z);
                        acc[r][o].w = fmaf(col[j].w, wk[3][tp], acc[r][o].w);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < OHB; ++r) {
        if (oh0 + r >= OH) break;
        float4* dst = out + (((size_t)n * OH + oh0 + r) * OW + ow0) * C4 + c4;
#pragma unroll
        for (int o = 0; o < OWB; ++o) {
            if (ow0 + o >= OW) break;
            float4 v = acc[r][o];
            if (act == 1) {
                v.x = vmax(v.x, 0.f); v.y = vmax(v.y, 0.f); v.z = vmax(v.z, 0.f); v.w = vmax(v.w, 0.f);
            }
            dst[(size_t)o * C4] = v;
        }
    }
}

// MaxPool 3x3 stride 2 for C % 4 == 0 with every channel on the max_ps rule
// (vec_end == C): a lane owns 4 channels and 4 consecutive outputs of a row;
// in-range taps only, initial -1e30 (src/maxpool_avx512.cpp:15-62).
// Lane index = ((n*OH + oh)*nOWB + owb)*C4 + c4.
__global__ __launch_bounds__(256) void k_maxpool3s2_row(const float4* __restrict__ in, int H,
                                                        int W, int C4, int pad, int OH, int OW,
                                                        int nOWB, int total,
                                                        float4* __restrict__ out, int post_relu) {
    constexpr int OWB = 4, S = 2, NCOL = (OWB - 1) * S + 3;
    const int t = blockIdx.x * 256 + threadIdx.x;
    if (t >= total) return;
    int q = t / C4;
    const int c4 = t - q * C4;
    const int owb = q % nOWB;
    const int row = q / nOWB;                        // n*OH + oh
    const int n = row / OH, oh = row - n * OH;
    const int ow0 = owb * OWB;
    float4 mx[OWB];
#pragma unroll
    for (int o = 0; o < OWB; ++o) mx[o] = make_float4(-1e30f, -1e30f, -1e30f, -1e30f);
    const float4* img = in + (size_t)n * H * W * C4 + c4;
    const int iw0 = ow0 * S - pad;
#pragma unroll
    for (int kh = 0; kh < 3; ++kh) {
        const int ih = oh * S - pad + kh;
        if ((unsigned)ih >= (unsigned)H) continue;
        float4 col[NCOL];
        bool cok[NCOL];
#pragma unroll
        for (int j = 0; j < NCOL; ++j) {
            const int iw = iw0 + j;
            cok[j] = (unsigned)iw < (unsigned)W;
            col[j] = cok[j] ? img[((size_t)ih * W + iw) * C4] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int o = 0; o < OWB; ++o) {
#pragma unroll
            for (int kw = 0; kw < 3; ++kw) {
                const int j = o * S + kw;
                if (cok[j]) {
                    mx[o].x = vmax(mx[o].x, col[j].x);
                    mx[o].y = vmax(mx[o].y, col[j].y);
                    mx[o].z = vmax(mx[o].z, col[j].z);
                    mx[o].w = vmax(mx[o].w, col[j].w);
                }
            }
        }
    }
    float4* dst = out + ((size_t)row * OW + ow0) * C4 + c4;
#pragma unroll
    for (int o = 0; o < OWB; ++o) {
        if (ow0 + o >= OW) break;
        float4 v = mx[o];
        if (post_relu) {
            v.x = vmax(v.x, 0.f); v.y = vmax(v.y, 0.f); v.z = vmax(v.z, 0.f); v.w = vmax(v.w, 0.f);
        }
        dst[(size_t)o * C4] = v;
    }
}

// Depthwise 3x3 (stride S) + activation fused with the 3x3 / stride-2 MaxPool
// that follows it (pool padding PP), for C % 4 == 0: the depthwise output
// never reaches HBM.  A workgroup (5 waves) owns image n, pool rows
// ph0, ph0+1, pool columns pw0 .. pw0+13 and 8 channel quads.  Phase 1: wave
// w computes depthwise output row y0 + w (y0 = 2*ph0 - PP) for columns
// x0 .. x0+28 (x0 = 2*pw0 - PP) into LDS, a lane owning 4 consecutive columns
// of one quad (the column loads shared between them); the arithmetic per
// channel is k_dwconv3_blk's (the reference's: bias, fmaf per in-range tap in
// kh, kw order, then the activation).  Phase 2: each pooled value is the max
// from -1e30 over its in-range taps in kh, kw order (max_ps), then the optional
// ReLU -- the two reference calls' results bit for bit.
constexpr int DWP_ROWS = 5, DWP_PWB = 14, DWP_COLS = 2 * DWP_PWB + 1, DWP_Q = 8;
template <int S>
__global__ __launch_bounds__(320) void k_dwconv3_pool(const float4* __restrict__ in, int H, int W,
                                                      int C4, const float* __restrict__ w,
                                                      const float* __restrict__ bias, int pad,
                                                      int OH, int OW, int act, int PP, int PH,
                                                      int PW, int nPHB, int nPWB, int nQG,
                                                      int nblk, int pvec_end,
                                                      float4* __restrict__ out, int post_relu) {
    __shared__ float4 ys[DWP_ROWS][DWP_COLS][DWP_Q];
    // XCD-ordered work: workgroup i of XCD x (blockIdx.x = 8 i + x) takes item
    // x * per + i, so each XCD runs a contiguous range of items, and the
    // blocks of neighbouring pool rows (which stage the same halo input rows)
    // run on one XCD at about the same time: the second read of a halo row
    // hits that XCD's L2 instead of going to memory again.
    const int per = (int)(gridDim.x >> 3);
    int b = (int)(blockIdx.x & 7u) * per + (int)(blockIdx.x >> 3);
    if (b >= nblk) return;                               // uniform per workgroup
    const int qg = b % nQG;
    b /= nQG;
    const int pwb = b % nPWB;
    b /= nPWB;
    const int phb = b % nPHB;
    const int n = b / nPHB;
    const int ph0 = 2 * phb, pw0 = DWP_PWB * pwb;
    const int y0 = 2 * ph0 - PP, x0 = 2 * pw0 - PP;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    // ---- phase 1: depthwise row y0 + wave, lane = (column run r, quad q)
    {
        const int q = lane & 7, run = lane >> 3;         // 8 runs of 4 columns cover 29
        const int c4 = qg * DWP_Q + q;
        const int yr = y0 + wave;
        const int yc0 = x0 + 4 * run;
        const bool live = c4 < C4 && (unsigned)yr < (unsigned)OH;
        float4 acc[4];
        if (live) {
            const int c = 4 * c4;
            float wk[4][9];
            const float4* w4 = (const float4*)(w + (size_t)c * 9);
#pragma unroll
            for (int i = 0; i < 9; ++i) {
                const float4 v = w4[i];
                wk[(4 * i + 0) / 9][(4 * i + 0) % 9] = v.x;
                wk[(4 * i + 1) / 9][(4 * i + 1) % 9] = v.y;
                wk[(4 * i + 2) / 9][(4 * i + 2) % 9] = v.z;
                wk[(4 * i + 3) / 9][(4 * i + 3) % 9] = v.w;
            }
            const float4 b4 = bias ? make_float4(bias[c], bias[c + 1], bias[c + 2], bias[c + 3])
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int o = 0; o < 4; ++o) acc[o] = b4;
            const float4* img = in + (size_t)n * H * W * C4 + c4;
            constexpr int NCOL = 3 * S + 3;              // input columns of 4 outputs
            const int iw0 = yc0 * S - pad;
#pragma unroll
            for (int kh = 0; kh < 3; ++kh) {
                const int ih = yr * S - pad + kh;
                if ((unsigned)ih >= (unsigned)H) continue;
                float4 col[NCOL];
                bool cok[NCOL];
#pragma unroll
                for (int j = 0; j < NCOL; ++j) {
                    const int iw = iw0 + j;
                    cok[j] = (unsigned)iw < (unsigned)W;
                    col[j] = cok[j] ? img[((size_t)ih * W + iw) * C4] : make_float4(0.f, 0.f, 0.f, 0.f);
                }
#pragma unroll
                for (int o = 0; o < 4; ++o) {
#pragma unroll
                    for (int kw = 0; kw < 3; ++kw) {
                        const int j = o * S + kw;
                        const int tp = kh * 3 + kw;
                        if (cok[j]) {
                            acc[o].x = fmaf(col[j].x, wk[0][tp], acc[o].x);
                            acc[o].y = fmaf(col[j].y, wk[1][tp], acc[o].y);
                            acc[o].z = fmaf(col[j].z, wk[2][tp], acc[o].z);
                            acc[o].w = fmaf(col[j].w, wk[3][tp], acc[o].w);
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int o = 0; o < 4; ++o) {
            const int cc = 4 * run + o;
            if (cc >= DWP_COLS) break;
            float4 v = acc[o];
            v.x = act_apply(v.x, act); v.y = act_apply(v.y, act);
            v.z = act_apply(v.z, act); v.w = act_apply(v.w, act);
            if (live) ys[wave][cc][q] = v;
        }
    }
    __syncthreads();
    // ---- phase 2: 2 pool rows x 14 pool columns x 8 quads
    if (tid < 2 * DWP_PWB * DWP_Q) {
        const int q = tid & 7, pc = (tid >> 3) % DWP_PWB, pr = (tid >> 3) / DWP_PWB;
        const int ph = ph0 + pr, pw = pw0 + pc, c4 = qg * DWP_Q + q;
        if (ph < PH && pw < PW && c4 < C4) {
            // k_maxpool's per-channel compare: max_ps below pvec_end, else "v > m"
            const bool pv = 4 * c4 < pvec_end;          // pvec_end is a multiple of 8
            auto mx = [pv](float a, float v) { return pv ? vmax(a, v) : (v > a ? v : a); };
            float4 m = make_float4(-1e30f, -1e30f, -1e30f, -1e30f);
#pragma unroll
            for (int kh = 0; kh < 3; ++kh) {
                const int yr = 2 * ph - PP + kh;
                if ((unsigned)yr >= (unsigned)OH) continue;
#pragma unroll
                for (int kw = 0; kw < 3; ++kw) {
                    const int yc = 2 * pw - PP + kw;
                    if ((unsigned)yc >= (unsigned)OW) continue;
                    const float4 v = ys[yr - y0][yc - x0][q];
                    m.x = mx(m.x, v.x); m.y = mx(m.y, v.y); m.z = mx(m.z, v.z); m.w = mx(m.w, v.w);
                }
            }
            if (post_relu) {
                auto rl = [pv](float a) { return pv ? vmax(a, 0.f) : (a < 0.f ? 0.f : a); };
                m.x = rl(m.x); m.y = rl(m.y); m.z = rl(m.z); m.w = rl(m.w);
            }
            out[(((size_t)n * PH + ph) * PW + pw) * C4 + c4] = m;
        }
    }
}

// Grouped direct conv, weights [g][KH*KW*Cin_p][Cout_p].  vec_end / fma_all
// encode which channels the reference's dispatcher (src/group_conv.cpp:60-79)
// runs through a fused-multiply-add vector kernel.
__global__ void k_gconv(const float* __restrict__ in, int N, int H, int W, int Cin,
                        const float* __restrict__ w, const float* __restrict__ bias, int KH,
                        int KW, int Cout, int stride, int pad, int groups, int OH, int OW,
                        float* __restrict__ out, int act, int vec_end, int fma_all) {
    long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    long long total = (long long)N * OH * OW * Cout;
    if (idx >= total) return;
    int co = (int)(idx % Cout);
    long long p = idx / Cout;
    int ow = (int)(p % OW);
    p /= OW;
    int oh = (int)(p % OH);
    int n = (int)(p / OH);
    int Cin_p = Cin / groups, Cout_p = Cout / groups;
    int g = co / Cout_p, oc = co - g * Cout_p;
    const float* wg = w + (long long)g * Cout_p * KH * KW * Cin_p;
    float s = bias ? bias[co] : 0.0f;
    bool use_fma = fma_all || oc < vec_end;
    for (int kh = 0; kh < KH; ++kh) {
        int ih = oh * stride - pad + kh;
        if (ih < 0 || ih >= H) continue;
        for (int kw = 0; kw < KW; ++kw) {
            int iw = ow * stride - pad + kw;
            if (iw < 0 || iw >= W) continue;
            const float* px = in + (((long long)n * H + ih) * W + iw) * Cin + (long long)g * Cin_p;
            const float* wp = wg + (long long)((kh * KW + kw) * Cin_p) * Cout_p + oc;
            if (use_fma) {
                for (int ic = 0; ic < Cin_p; ++ic) s = fmaf(px[ic], wp[(long long)ic * Cout_p], s);
            } else {
                for (int ic = 0; ic < Cin_p; ++ic) s = s + px[ic] * wp[(long long)ic * Cout_p];
            }
        }
    }
    if (act == 1) {
        if (oc < vec_end) s = vmax(s, 0.0f);
        else if (s < 0.0f) s = 0.0f;
    }
    out[idx] = s;
}

// k_gconv for Cin_p and Cout_p multiples of 4 with the all-FMA rule
// (Cout_p >= 8): a lane owns one output pixel x 4 consecutive output channels
// of one group.  Per in-range tap it loads the group's Cin_p input channels
// as 16-byte quads and, per input channel, the 4 weights as one quad; each
// output keeps the reference's order (bias, then taps kh-major, then input
// channels, one fmaf each).  Lanes run channel-quad fastest, so a wave's
// stores cover whole output pixels.
__global__ __launch_bounds__(256) void k_gconv4(const float* __restrict__ in, int N, int H, int W,
                                                int Cin, const float* __restrict__ w,
                                                const float* __restrict__ bias, int KH, int KW,
                                                int Cout, int stride, int pad, int groups, int OH,
                                                int OW, float* __restrict__ out, int act,
                                                int vec_end) {
    const int cq = Cout >> 2;
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long total = (long long)N * OH * OW * cq;
    if (idx >= total) return;
    const int q = (int)(idx % cq);
    long long p = idx / cq;
    const int ow = (int)(p % OW);
    p /= OW;
    const int oh = (int)(p % OH);
    const int n = (int)(p / OH);
    const int Cin_p = Cin / groups, Cout_p = Cout / groups;
    const int co = 4 * q;
    const int g = co / Cout_p, oc = co - g * Cout_p;
    const float* wg = w + (long long)g * Cout_p * KH * KW * Cin_p + oc;
    f4 s = {0.f, 0.f, 0.f, 0.f};
    if (bias) s = *(const f4*)(bias + co);
    for (int kh = 0; kh < KH; ++kh) {
        const int ih = oh * stride - pad + kh;
        if (ih < 0 || ih >= H) continue;
        for (int kw = 0; kw < KW; ++kw) {
            const int iw = ow * stride - pad + kw;
            if (iw < 0 || iw >= W) continue;
            const float* px = in + (((long long)n * H + ih) * W + iw) * Cin + (long long)g * Cin_p;
            const float* wp = wg + (long long)((kh * KW + kw) * Cin_p) * Cout_p;
            for (int i4 = 0; i4 < Cin_p; i4 += 4) {
                const f4 x = *(const f4*)(px + i4);
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const f4 wv = *(const f4*)(wp + (long long)(i4 + u) * Cout_p);
                    s.x = fmaf(x[u], wv.x, s.x);
                    s.y = fmaf(x[u], wv.y, s.y);
                    s.z = fmaf(x[u], wv.z, s.z);
                    s.w = fmaf(x[u], wv.w, s.w);
                }
            }
        }
    }
    if (act == 1) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (oc + u < vec_end) s[u] = vmax(s[u], 0.0f);
            else if (s[u] < 0.0f) s[u] = 0.0f;
        }
    }
    *(f4*)(out + (((long long)n * OH + oh) * OW + ow) * Cout + co) = s;
}

// k_gconv4 for 3x3 kernels and Cin_p = 4*CINQ: every load of the lane (the
// in-image taps' input quads and all weight quads) is issued before the first
// fmaf, so the lane waits for memory once instead of once per tap.  Taps
// outside the image are skipped (not multiplied by zero), as in the reference.
template <int CINQ>
__global__ __launch_bounds__(256) void k_gconv4_3x3(const float* __restrict__ in, int N, int H,
                                                    int W, int Cin, const float* __restrict__ w,
                                                    const float* __restrict__ bias, int Cout,
                                                    int stride, int pad, int groups, int OH, int OW,
                                                    float* __restrict__ out, int act, int vec_end) {
    constexpr int CP = 4 * CINQ;
    const int cq = Cout >> 2;
    // 32-bit index math (the launcher checks N*OH*OW*Cout/4 < 2^31)
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= N * OH * OW * cq) return;
    const int q = idx % cq;
    int p = idx / cq;
    const int ow = p % OW;
    p /= OW;
    const int oh = p % OH;
    const int n = p / OH;
    const int Cout_p = Cout / groups;
    const int co = 4 * q;
    const int g = co / Cout_p, oc = co - g * Cout_p;
    const float* wg = w + (long long)g * Cout_p * 9 * CP + oc;
    const float* img = in + (long long)n * H * W * Cin + (long long)g * CP;
    f4 x[9][CINQ], wv[9][CP];
    bool ok[9];
#pragma unroll
    for (int t = 0; t < 9; ++t) {
        const int ih = oh * stride - pad + t / 3, iw = ow * stride - pad + t % 3;
        ok[t] = (unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W;
        const float* px = img + ((long long)(ok[t] ? ih : 0) * W + (ok[t] ? iw : 0)) * Cin;
#pragma unroll
        for (int c = 0; c < CINQ; ++c) x[t][c] = *(const f4*)(px + 4 * c);
#pragma unroll
        for (int i = 0; i < CP; ++i) wv[t][i] = *(const f4*)(wg + (long long)(t * CP + i) * Cout_p);
    }
    f4 s = {0.f, 0.f, 0.f, 0.f};
    if (bias) s = *(const f4*)(bias + co);
#pragma unroll
    for (int t = 0; t < 9; ++t) {
        if (!ok[t]) continue;
#pragma unroll
        for (int i = 0; i < CP; ++i) {
            const float xi = x[t][i >> 2][i & 3];
            s.x = fmaf(xi, wv[t][i].x, s.x);
            s.y = fmaf(xi, wv[t][i].y, s.y);
            s.z = fmaf(xi, wv[t][i].z, s.z);
            s.w = fmaf(xi, wv[t][i].w, s.w);
        }
    }
    if (act == 1) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (oc + u < vec_end) s[u] = vmax(s[u], 0.0f);
            else if (s[u] < 0.0f) s[u] = 0.0f;
        }
    }
    *(f4*)(out + (((long long)n * OH + oh) * OW + ow) * Cout + co) = s;
}

// Depthwise 3x3 / stride 2 + activation + 3x3 / stride-2 MaxPool, row-streaming
// form: a lane owns 4 channels of one pooled column and walks a strip of RP
// pooled rows down the image.  Per depthwise row y it loads the two new input
// rows (7 columns: those of depthwise columns 2 pw - pp .. 2 pw - pp + 2), and
// keeps only running sums: the depthwise accumulators of row y + 1 started
// from the row the two share, and the maxima of the (at most two) pool rows
// row y belongs to.  Every value is folded in the reference's order (bias, then
// one fmaf per in-range tap kh-major; pool taps kh-major, max_ps from -1e30),
// out-of-range taps skipped by selects, so the result is bit for bit
// k_dwconv3_blk then k_maxpool3s2_row.  No LDS, no barriers: lanes stream
// independently, and workgroups are XCD-ordered so the strips that share
// input rows read them through one L2.
constexpr int DWR_RP = 4;                               // pooled rows per strip
__global__ __launch_bounds__(256) void k_dwconv3_pool_rs(
    const float* __restrict__ in, int H, int W, int C4, const float* __restrict__ w,
    const float* __restrict__ bias, int pad, int OH, int OW, int act, int PP, int PH, int PW,
    int nstrip, int items, int in_bytes, int pvec_end, float4* __restrict__ out, int post_relu) {
    constexpr unsigned kOOB = 0x80000000u;
    const int per = (int)(gridDim.x >> 3);
    const int blk = (int)(blockIdx.x & 7u) * per + (int)(blockIdx.x >> 3);
    const int idx = blk * 256 + (int)threadIdx.x;
    if (idx >= items) return;
    // a strip's lanes are padded to whole waves, so every wave walks one way
    const int lps = (PW * C4 + 63) & ~63, li = idx % lps;
    if (li >= PW * C4) return;
    const int q = li % C4, pw = li / C4;
    const int t = idx / lps;
    const int st = t % nstrip;
    const int n = t / nstrip;
    const int ph0 = st * DWR_RP, ph1 = ph0 + DWR_RP < PH ? ph0 + DWR_RP : PH;
    const int c = 4 * q;
    float wk[4][9];
    {
        const float4* w4 = (const float4*)(w + (size_t)c * 9);   // 36 floats, 16-byte aligned
#pragma unroll
        for (int i = 0; i < 9; ++i) {
            const float4 v = w4[i];
            wk[(4 * i + 0) / 9][(4 * i + 0) % 9] = v.x;
            wk[(4 * i + 1) / 9][(4 * i + 1) % 9] = v.y;
            wk[(4 * i + 2) / 9][(4 * i + 2) % 9] = v.z;
            wk[(4 * i + 3) / 9][(4 * i + 3) % 9] = v.w;
        }
    }
    const f4 b4 = bias ? f4{bias[c], bias[c + 1], bias[c + 2], bias[c + 3]} : f4{0.f, 0.f, 0.f, 0.f};
    // depthwise columns x_j = 2 pw - PP + j; their input columns cb + l, l < 7
    const int x0 = 2 * pw - PP, cb = 2 * x0 - pad;
    bool xok[3], cok[7];
#pragma unroll
    for (int j = 0; j < 3; ++j) xok[j] = (unsigned)(x0 + j) < (unsigned)OW;
#pragma unroll
    for (int l = 0; l < 7; ++l) cok[l] = (unsigned)(cb + l) < (unsigned)W;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)in, (short)0, in_bytes, 0x00020000);
    auto ldrow = [&](int r, f4* v) {                     // input row r, the 7 columns
        const bool rok = (unsigned)r < (unsigned)H;
        const int base = ((n * H + r) * W + cb) * C4 + q;
#pragma unroll
        for (int l = 0; l < 7; ++l) {
            const unsigned off = rok && cok[l] ? (unsigned)((base + l * C4) * 16) : kOOB;
            v[l] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
        }
        return rok;
    };
    // acc[j] += row's taps kh of depthwise column j, in kw order (in-range only)
    auto fold = [&](f4* acc, const f4* v, bool rok, int kh) {
#pragma unroll
        for (int j = 0; j < 3; ++j)
#pragma unroll
            for (int kw = 0; kw < 3; ++kw) {
                const bool ok = rok && cok[2 * j + kw];
                const f4 x = v[2 * j + kw];
                const int tp = kh * 3 + kw;
                acc[j].x = ok ? fmaf(x.x, wk[0][tp], acc[j].x) : acc[j].x;
                acc[j].y = ok ? fmaf(x.y, wk[1][tp], acc[j].y) : acc[j].y;
                acc[j].z = ok ? fmaf(x.z, wk[2][tp], acc[j].z) : acc[j].z;
                acc[j].w = ok ? fmaf(x.w, wk[3][tp], acc[j].w) : acc[j].w;
            }
    };
    // k_maxpool's per-channel compare: max_ps below pvec_end, else "v > m"
    bool pv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) pv[e] = c + e < pvec_end;
    auto pmax = [&](f4& m, const f4* d, bool yok) {      // the row's 3 taps, kw order
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const bool ok = yok && xok[j];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float v = d[j][e];
                const float r = pv[e] ? vmax(m[e], v) : (v > m[e] ? v : m[e]);
                m[e] = ok ? r : m[e];
            }
        }
    };
    const f4 lo = {-1e30f, -1e30f, -1e30f, -1e30f};
    // depthwise rows yA .. yB feed pool rows ph0 .. ph1 - 1
    const int yA = 2 * ph0 - PP, yB = 2 * (ph1 - 1) - PP + 2;
    if (st & 1) {
        // Odd strips walk up, so each halo shared with a neighbour is read by
        // both strips at the same time (both at their start, or both at their
        // end) and the second read hits L2.  Row y folds its input rows in kh
        // order (r0, r1, then r2 = the row below, kept from the previous step);
        // its activated values go to a per-lane ring of the last three rows in
        // LDS, and pool row ph is formed, in kh order, once its top row 2 ph - PP
        // arrives.  Same arithmetic in the same order as the downward walk.
        __shared__ f4 ring[9][256];
        const int lt = (int)threadIdx.x;
        f4 r2[7];
        bool ok2 = ldrow(2 * yB - pad + 2, r2);
        int ph = ph1 - 1;
        for (int y = yB; y >= yA; --y) {
            f4 r1[7], r0[7];
            const bool ok1 = ldrow(2 * y - pad + 1, r1);
            const bool ok0 = ldrow(2 * y - pad, r0);
            f4 d[3] = {b4, b4, b4};
            fold(d, r0, ok0, 0);
            fold(d, r1, ok1, 1);
            fold(d, r2, ok2, 2);
            const int slot = (y - yA) % 3;
#pragma unroll
            for (int j = 0; j < 3; ++j) {
                d[j].x = act_apply(d[j].x, act); d[j].y = act_apply(d[j].y, act);
                d[j].z = act_apply(d[j].z, act); d[j].w = act_apply(d[j].w, act);
                ring[slot * 3 + j][lt] = d[j];
            }
            if (y == 2 * ph - PP) {
                f4 m = lo;
#pragma unroll
                for (int kh = 0; kh < 3; ++kh) {
                    const int yy = y + kh, sl = (yy - yA) % 3;
                    const f4 dd[3] = {ring[sl * 3][lt], ring[sl * 3 + 1][lt], ring[sl * 3 + 2][lt]};
                    pmax(m, dd, (unsigned)yy < (unsigned)OH);
                }
                if (ph < PH) {
                    if (post_relu) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) m[e] = pv[e] ? vmax(m[e], 0.f) : (m[e] < 0.f ? 0.f : m[e]);
                    }
                    out[(((size_t)n * PH + ph) * PW + pw) * C4 + q] = float4{m.x, m.y, m.z, m.w};
                }
                --ph;
            }
#pragma unroll
            for (int l = 0; l < 7; ++l) r2[l] = r0[l];
            ok2 = ok0;
        }
        return;
    }
    f4 part[3], rowa[7], rowb[7];
    {
        f4 acc0[3] = {b4, b4, b4};
        const bool ok0 = ldrow(2 * yA - pad, rowb);
        fold(acc0, rowb, ok0, 0);
#pragma unroll
        for (int j = 0; j < 3; ++j) part[j] = acc0[j];
    }
    f4 mA = lo, mB = lo;                                  // pool rows ph, ph + 1
    int ph = ph0;
    for (int y = yA; y <= yB; ++y) {
        const bool oka = ldrow(2 * y - pad + 1, rowa);
        const bool okb = ldrow(2 * y - pad + 2, rowb);
        f4 d[3] = {part[0], part[1], part[2]};
        fold(d, rowa, oka, 1);
        fold(d, rowb, okb, 2);
        // the next row's accumulators start from the shared input row
        part[0] = part[1] = part[2] = b4;
        fold(part, rowb, okb, 0);
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            d[j].x = act_apply(d[j].x, act); d[j].y = act_apply(d[j].y, act);
            d[j].z = act_apply(d[j].z, act); d[j].w = act_apply(d[j].w, act);
        }
        const bool yok = (unsigned)y < (unsigned)OH;
        // row y is tap kh = y - (2 ph - PP) of pool row ph and, when that is 2,
        // tap 0 of pool row ph + 1
        const int kh = y - (2 * ph - PP);
        pmax(mA, d, yok);
        if (kh == 2) {
            pmax(mB, d, yok);
            if (ph < PH) {
                f4 m = mA;
                if (post_relu) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) m[e] = pv[e] ? vmax(m[e], 0.f) : (m[e] < 0.f ? 0.f : m[e]);
                }
                out[(((size_t)n * PH + ph) * PW + pw) * C4 + q] = float4{m.x, m.y, m.z, m.w};
            }
            mA = mB;
            mB = lo;
            ++ph;
        }
    }
}

// Grouped 3x3 conv (Cin_p = 4 CINQ, the all-FMA rule) + activation fused with
// a 3x3 / stride-2 MaxPool: a lane owns one pooled pixel x 4 channels, computes
// the conv outputs of its pool window with k_gconv4_3x3's arithmetic (bias,
// then one fmaf per in-range tap and input channel, in order) and reduces them
// with k_maxpool's per-channel compare (max_ps below pvec_end), so the result
// is bit for bit the two kernels' without the conv output in memory.  The
// lane's 9 x CP weight quads are loaded once.
template <int CINQ>
__global__ __launch_bounds__(256) void k_gconv3_pool(const float* __restrict__ in, int N, int H,
                                                     int W, int Cin, const float* __restrict__ w,
                                                     const float* __restrict__ bias, int Cout,
                                                     int stride, int pad, int groups, int OH,
                                                     int OW, int act, int vec_end, int PP, int PH,
                                                     int PW, int pvec_end,
                                                     float* __restrict__ out, int post_relu) {
    constexpr int CP = 4 * CINQ;
    const int cq = Cout >> 2;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= N * PH * PW * cq) return;
    const int q = idx % cq;
    int p = idx / cq;
    const int pw = p % PW;
    p /= PW;
    const int ph = p % PH;
    const int n = p / PH;
    const int Cout_p = Cout / groups;
    const int co = 4 * q;
    const int g = co / Cout_p, oc = co - g * Cout_p;
    const float* wg = w + (long long)g * Cout_p * 9 * CP + oc;
    const float* img = in + (long long)n * H * W * Cin + (long long)g * CP;
    f4 wv[9][CP];
#pragma unroll
    for (int t = 0; t < 9; ++t)
#pragma unroll
        for (int i = 0; i < CP; ++i) wv[t][i] = *(const f4*)(wg + (long long)(t * CP + i) * Cout_p);
    const f4 b4 = bias ? *(const f4*)(bias + co) : f4{0.f, 0.f, 0.f, 0.f};
    f4 m = {-1e30f, -1e30f, -1e30f, -1e30f};
    for (int kh = 0; kh < 3; ++kh) {
        const int oh = 2 * ph - PP + kh;
        if ((unsigned)oh >= (unsigned)OH) continue;
        for (int kw = 0; kw < 3; ++kw) {
            const int ow = 2 * pw - PP + kw;
            if ((unsigned)ow >= (unsigned)OW) continue;
            f4 x[9][CINQ];
            bool ok[9];
#pragma unroll
            for (int t = 0; t < 9; ++t) {
                const int ih = oh * stride - pad + t / 3, iw = ow * stride - pad + t % 3;
                ok[t] = (unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W;
                const float* px = img + ((long long)(ok[t] ? ih : 0) * W + (ok[t] ? iw : 0)) * Cin;
#pragma unroll
                for (int c = 0; c < CINQ; ++c) x[t][c] = *(const f4*)(px + 4 * c);
            }
            f4 sv = b4;
#pragma unroll
            for (int t = 0; t < 9; ++t) {
                if (!ok[t]) continue;
#pragma unroll
                for (int i = 0; i < CP; ++i) {
                    const float xi = x[t][i >> 2][i & 3];
                    sv.x = fmaf(xi, wv[t][i].x, sv.x);
                    sv.y = fmaf(xi, wv[t][i].y, sv.y);
                    sv.z = fmaf(xi, wv[t][i].z, sv.z);
                    sv.w = fmaf(xi, wv[t][i].w, sv.w);
                }
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                float v = sv[u];
                if (act == 1) {
                    if (oc + u < vec_end) v = vmax(v, 0.0f);
                    else if (v < 0.0f) v = 0.0f;
                }
                if (co + u < pvec_end) m[u] = vmax(m[u], v);
                else if (v > m[u]) m[u] = v;
            }
        }
    }
    if (post_relu) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (co + u < pvec_end) m[u] = vmax(m[u], 0.0f);
            else if (m[u] < 0.0f) m[u] = 0.0f;
        }
    }
    *(f4*)(out + (((long long)n * PH + ph) * PW + pw) * Cout + co) = m;
}

// The same fused pair for a small image: one 256-thread workgroup per (image,
// group) stages the group's input channels of the whole image in LDS, computes
// the group's conv outputs into LDS (a thread keeps one output-channel quad's
// 9 x CP weight quads in registers and walks the pixels) and then pools them;
// the arithmetic per value is k_gconv3_pool's.  LDS: H*W*CP + OH*OW*Cout_p
// floats (gconv_pool_img_lds).
template <int CINQ>
__global__ __launch_bounds__(256) void k_gconv3_pool_img(
    const float* __restrict__ in, int H, int W, int Cin, const float* __restrict__ w,
    const float* __restrict__ bias, int Cout, int stride, int pad, int groups, int OH, int OW,
    int act, int vec_end, int PP, int PH, int PW, int pvec_end, float* __restrict__ out,
    int post_relu) {
    constexpr int CP = 4 * CINQ;
    extern __shared__ __attribute__((aligned(16))) float lds[];
    // workgroup -> (image, group), XCD-ordered (workgroup id mod 8 picks the XCD):
    // the groups of one image share its pixels' cache lines, so they run on one L2
    const int G = (int)gridDim.x, b = (int)blockIdx.x;
    const int L = (G & 7) == 0 ? (b & 7) * (G >> 3) + (b >> 3) : b;
    const int n = L / groups, g = L - n * groups;
    const int Cout_p = Cout / groups, nq = Cout_p >> 2;
    f4* const xs = (f4*)lds;                               // [H*W][CINQ]
    f4* const ys = xs + H * W * CINQ;                      // [OH*OW][nq]
    const int tid = threadIdx.x;
    const float* img = in + (long long)n * H * W * Cin + (long long)g * CP;
    // conv: thread -> output-channel quad qo = tid % nq, pixels tid / nq, + 256 / nq, ...
    // (its weights and bias are loaded while the image is staged)
    const int per = 256 / nq;
    const int qo = tid % nq, p0 = tid / nq;
    const int oc = 4 * qo, co = g * Cout_p + oc;
    f4 wv[9][CP];
    {
        const float* wg = w + (long long)g * Cout_p * 9 * CP + oc;
#pragma unroll
        for (int t = 0; t < 9; ++t)
#pragma unroll
            for (int i = 0; i < CP; ++i) wv[t][i] = *(const f4*)(wg + (long long)(t * CP + i) * Cout_p);
    }
    const f4 b4 = bias ? *(const f4*)(bias + co) : f4{0.f, 0.f, 0.f, 0.f};
    for (int i = tid; i < H * W * CINQ; i += 256) {
        const int px = i / CINQ, c = i - px * CINQ;
        xs[i] = *(const f4*)(img + (long long)px * Cin + 4 * c);
    }
    __syncthreads();
    if (p0 < per) {
        for (int pix = p0; pix < OH * OW; pix += per) {
            const int oh = pix / OW, ow = pix - oh * OW;
            f4 sv = b4;
#pragma unroll
            for (int t = 0; t < 9; ++t) {
                const int ih = oh * stride - pad + t / 3, iw = ow * stride - pad + t % 3;
                if ((unsigned)ih >= (unsigned)H || (unsigned)iw >= (unsigned)W) continue;
                const f4* xp = xs + (ih * W + iw) * CINQ;
#pragma unroll
                for (int i = 0; i < CP; ++i) {
                    const float xi = xp[i >> 2][i & 3];
                    sv.x = fmaf(xi, wv[t][i].x, sv.x);
                    sv.y = fmaf(xi, wv[t][i].y, sv.y);
                    sv.z = fmaf(xi, wv[t][i].z, sv.z);
                    sv.w = fmaf(xi, wv[t][i].w, sv.w);
                }
            }
            if (act == 1) {
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    if (oc + u < vec_end) sv[u] = vmax(sv[u], 0.0f);
                    else if (sv[u] < 0.0f) sv[u] = 0.0f;
                }
            }
            ys[pix * nq + qo] = sv;
        }
    }
    __syncthreads();
    // pool: thread -> (pooled pixel, quad)
    for (int i = tid; i < PH * PW * nq; i += 256) {
        const int q = i % nq, pp = i / nq;
        const int ph = pp / PW, pw = pp - ph * PW;
        const int co = g * Cout_p + 4 * q;
        f4 m = {-1e30f, -1e30f, -1e30f, -1e30f};
        for (int kh = 0; kh < 3; ++kh) {
            const int oh = 2 * ph - PP + kh;
            if ((unsigned)oh >= (unsigned)OH) continue;
            for (int kw = 0; kw < 3; ++kw) {
                const int ow = 2 * pw - PP + kw;
                if ((unsigned)ow >= (unsigned)OW) continue;
                const f4 v = ys[(oh * OW + ow) * nq + q];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    if (co + u < pvec_end) m[u] = vmax(m[u], v[u]);
                    else if (v[u] > m[u]) m[u] = v[u];
                }
            }
        }
        if (post_relu) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                if (co + u < pvec_end) m[u] = vmax(m[u], 0.0f);
                else if (m[u] < 0.0f) m[u] = 0.0f;
            }
        }
        *(f4*)(out + (((long long)n * PH + ph) * PW + pw) * Cout + co) = m;
    }
}

// The same fused pair by rows: one 512-thread workgroup per (image, pooled
// row) stages, for every group at once, the input rows its three conv rows
// read (2 * stride + 3 rows, each pixel's channels read once) and the whole
// weight tensor in LDS.  Conv task t is output-channel quad t / (3 OW) of
// pixel t % (3 OW) of the three conv rows: the lanes of a wave share one or
// two quads, so their weight reads are LDS broadcasts.  The conv rows go to
// LDS and are pooled.  The arithmetic per value is k_gconv3_pool's: bias,
// then taps (kh, kw) in order with the in-range ones only, input channels in
// order, fmaf; the same activation and max rules.
// LDS (floats): IR * W * Cin + Cout * 9 * CP + 3 * OW * Cout + Cout.
template <int CINQ>
__global__ __launch_bounds__(512) void k_gconv3_pool_row(
    const float* __restrict__ in, int H, int W, int Cin, const float* __restrict__ w,
    const float* __restrict__ bias, int Cout, int stride, int pad, int groups, int OH, int OW,
    int act, int vec_end, int PP, int PH, int PW, int pvec_end, float* __restrict__ out,
    int post_relu) {
    constexpr int CP = 4 * CINQ;
    extern __shared__ __attribute__((aligned(16))) float lds[];
    // workgroup -> (image, pooled row), XCD-ordered: the pooled rows of an image,
    // which share input rows, run on one L2
    const int G = (int)gridDim.x, b = (int)blockIdx.x;
    const int L = (G & 7) == 0 ? (b & 7) * (G >> 3) + (b >> 3) : b;
    const int n = L / PH, ph = L - n * PH;
    const int IR = 2 * stride + 3;                         // input rows of three conv rows
    const int oh0 = 2 * ph - PP;                           // first conv row (may be -1)
    const int ih0 = oh0 * stride - pad;                    // first staged input row
    const int Cout_p = Cout / groups, nqa = Cout >> 2;
    const int rowf4 = W * Cin / 4, npix = 3 * OW;
    float* const xs = lds;                                 // [IR][W][Cin]
    float* const wsm = xs + IR * W * Cin;                  // [groups][9 * CP][Cout_p], as w
    float* const ys = wsm + Cout * 9 * CP;                 // [3][OW][Cout]
    float* const bsm = ys + 3 * OW * Cout;                 // [Cout] bias (0 without one)
    const int tid = threadIdx.x;
    const float* img = in + (long long)n * H * W * Cin;
    for (int i = tid; i < Cout; i += 512) bsm[i] = bias ? bias[i] : 0.0f;
    for (int i = tid; i < IR * rowf4; i += 512) {
        const int r = i / rowf4, ih = ih0 + r;
        if ((unsigned)ih < (unsigned)H)                  // rows past the image are never read
            ((f4*)xs)[i] = ((const f4*)(img + (long long)ih * W * Cin))[i - r * rowf4];
    }
    for (int i = tid; i < Cout * 9 * CP / 4; i += 512) ((f4*)wsm)[i] = ((const f4*)w)[i];
    __syncthreads();
    for (int t = tid; t < npix * nqa; t += 512) {
        const int q = t / npix, pix = t - q * npix;
        const int r = pix / OW, ow = pix - r * OW;
        const int oh = oh0 + r;
        if ((unsigned)oh >= (unsigned)OH) continue;         // (the pool skips this row)
        const int co = 4 * q, g = co / Cout_p, oc = co - g * Cout_p;
        const float* wg = wsm + g * Cout_p * 9 * CP + oc;
        f4 sv = *(const f4*)(bsm + co);
#pragma unroll
        for (int kt = 0; kt < 9; ++kt) {
            const int ih = oh * stride - pad + kt / 3, iw = ow * stride - pad + kt % 3;
            if ((unsigned)ih >= (unsigned)H || (unsigned)iw >= (unsigned)W) continue;
            const f4* xp = (const f4*)(xs + ((ih - ih0) * W + iw) * Cin + g * CP);
            f4 xv[CINQ];
#pragma unroll
            for (int c = 0; c < CINQ; ++c) xv[c] = xp[c];
#pragma unroll
            for (int i = 0; i < CP; ++i) {
                const float xi = xv[i >> 2][i & 3];
                const f4 wq = *(const f4*)(wg + (kt * CP + i) * Cout_p);
                sv.x = fmaf(xi, wq.x, sv.x);
                sv.y = fmaf(xi, wq.y, sv.y);
                sv.z = fmaf(xi, wq.z, sv.z);
                sv.w = fmaf(xi, wq.w, sv.w);
            }
        }
        if (act == 1) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                if (oc + u < vec_end) sv[u] = vmax(sv[u], 0.0f);
                else if (sv[u] < 0.0f) sv[u] = 0.0f;
            }
        }
        *(f4*)(ys + (r * OW + ow) * Cout + co) = sv;
    }
    __syncthreads();
    for (int t = tid; t < PW * nqa; t += 512) {
        const int q = t % nqa, pw = t / nqa;
        const int co = 4 * q;
        f4 m = {-1e30f, -1e30f, -1e30f, -1e30f};
        for (int kh = 0; kh < 3; ++kh) {
            const int oh = oh0 + kh;
            if ((unsigned)oh >= (unsigned)OH) continue;
            for (int kw = 0; kw < 3; ++kw) {
                const int ow = 2 * pw - PP + kw;
                if ((unsigned)ow >= (unsigned)OW) continue;
                const f4 v = *(const f4*)(ys + (kh * OW + ow) * Cout + co);
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    if (co + u < pvec_end) m[u] = vmax(m[u], v[u]);
                    else if (v[u] > m[u]) m[u] = v[u];
                }
            }
        }
        if (post_relu) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                if (co + u < pvec_end) m[u] = vmax(m[u], 0.0f);
                else if (m[u] < 0.0f) m[u] = 0.0f;
            }
        }
        *(f4*)(out + (((long long)n * PH + ph) * PW + pw) * Cout + co) = m;
    }
}

// MaxPool: channels below vec_end use max_ps semantics, the rest the scalar
// compare of src/layers.cpp:221-246 (they differ only for NaN / signed zero).
__global__ void k_maxpool(const float* __restrict__ in, int N, int H, int W, int C, int pool,
                          int stride, int pad, int OH, int OW, float* __restrict__ out,
                          int post_relu, int vec_end) {
    long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    long long total = (long long)N * OH * OW * C;
    if (idx >= total) return;
    int c = (int)(idx % C);
    long long p = idx / C;
    int ow = (int)(p % OW);
    p /= OW;
    int oh = (int)(p % OH);
    int n = (int)(p / OH);
    const float* img = in + (long long)n * H * W * C + c;
    bool vec = c < vec_end;
    float mx = -1e30f;
    for (int ph = 0; ph < pool; ++ph) {
        int ih = oh * stride - pad + ph;
        if (ih < 0 || ih >= H) continue;
        for (int pw = 0; pw < pool; ++pw) {
            int iw = ow * stride - pad + pw;
            if (iw < 0 || iw >= W) continue;
            float v = img[((long long)ih * W + iw) * C];
            if (vec) mx = vmax(mx, v);
            else if (v > mx) mx = v;
        }
    }
    if (post_relu) {
        if (vec) mx = vmax(mx, 0.0f);
        else if (mx < 0.0f) mx = 0.0f;
    }
    out[idx] = mx;
}

__global__ void k_relu(float* __restrict__ d, size_t n, int six) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float v = d[i];
    if (v < 0.0f) v = 0.0f;
    else if (six && v > 6.0f) v = 6.0f;
    d[i] = v;
}

__global__ void k_fill(float* __restrict__ d, size_t n, float v) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) d[i] = v;
}

// Row softmax: one 256-thread block per row (src/layers.cpp:272-283).
__global__ void k_softmax(const float* __restrict__ in, int cols, float* __restrict__ out) {
    __shared__ float red[256];
    const float* ri = in + (long long)blockIdx.x * cols;
    float* ro = out + (long long)blockIdx.x * cols;
    float mx = ri[0];
    for (int c = threadIdx.x; c < cols; c += 256) mx = ri[c] > mx ? ri[c] : mx;
    red[threadIdx.x] = mx;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (threadIdx.x < s) red[threadIdx.x] = vmax(red[threadIdx.x], red[threadIdx.x + s]);
        __syncthreads();
    }
    mx = red[0];
    __syncthreads();
    float sum = 0.0f;
    for (int c = threadIdx.x; c < cols; c += 256) {
        float e = expf(ri[c] - mx);
        ro[c] = e;
        sum += e;
    }
    red[threadIdx.x] = sum;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
        __syncthreads();
    }
    float inv = 1.0f / red[0];
    for (int c = threadIdx.x; c < cols; c += 256) ro[c] = ro[c] * inv;
}

// Unfused BN, two roundings per step like src/layers.cpp:285-296.
__global__ void k_batchnorm(float* __restrict__ d, long long total, int channels,
                            const float* __restrict__ mean, const float* __restrict__ var,
                            const float* __restrict__ gamma, const float* __restrict__ beta,
                            float eps) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    int c = (int)(i % channels);
    float scale = gamma ? gamma[c] : 1.0f;
    float shift = beta ? beta[c] : 0.0f;
    float inv = scale / sqrtf(var[c] + eps);
    float t = d[i] - mean[c];
    t = t * inv;
    d[i] = t + shift;
}

// dst[p*dstC + dstOff + i] = src[p*srcC + off + i], i < cnt (per-group copies).
__global__ void k_chan_copy(const float* __restrict__ src, int pix, int srcC, int off, int cnt,
                            float* __restrict__ dst, int dstC, int dstOff) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)pix * cnt) return;
    long long p = i / cnt;
    int c = (int)(i - p * cnt);
    dst[p * dstC + dstOff + c] = src[p * srcC + off + c];
}

__global__ void k_add_relu(const float* __restrict__ a, const float* __restrict__ b,
                           float* __restrict__ y, size_t n, int act) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float v = a[i] + b[i];
    if (act && v < 0.0f) v = 0.0f;
    y[i] = v;
}

__global__ void k_gap(const float* __restrict__ x, int N, int HW, int C, float* __restrict__ y) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)N * C) return;
    int n = (int)(i / C), c = (int)(i - (long long)n * C);
    const float* p = x + (long long)n * HW * C + c;
    float s = 0.0f;
    for (int k = 0; k < HW; ++k) s += p[(long long)k * C];
    y[i] = s / (float)HW;
}

inline dim3 grid1d(long long n, int bs = 256) { return dim3((unsigned)((n + bs - 1) / bs)); }

}  // namespace

bool dwconv_f32(const float* in, int N, int H, int W, int C, const float* w, const float* bias,
                int KH, int KW, int stride, int pad, float* out, int act, hipStream_t s) {
    int OH = (H + 2 * pad - KH) / stride + 1;
    int OW = (W + 2 * pad - KW) / stride + 1;
    if (OH <= 0 || OW <= 0 || KH <= 0 || KW <= 0) return true;
    bool al = (((uintptr_t)in | (uintptr_t)out) & 15u) == 0;
    const bool w_al = ((uintptr_t)w & 15u) == 0;
    const int C4 = C / 4;
    const long long nblk = (long long)N * ((OH + 1) / 2) * ((OW + 3) / 4) * C4;
    if (KH == 3 && KW == 3 && C % 4 == 0 && al && w_al && (stride == 1 || stride == 2) &&
        nblk < (1ll << 31) && (long long)N * H * W * C < (1ll << 31)) {
        const int nOHB = (OH + 1) / 2, nOWB = (OW + 3) / 4, total = (int)nblk;
        if (stride == 1)
            ACFUN_LAUNCH("k_dwconv", k_dwconv3_blk<1>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                               s, (const float4*)in, H, W, C4, w, bias, pad, OH, OW, nOHB, nOWB,
                               total, (float4*)out, act);
        else
            ACFUN_LAUNCH("k_dwconv", k_dwconv3_blk<2>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                               s, (const float4*)in, H, W, C4, w, bias, pad, OH, OW, nOHB, nOWB,
                               total, (float4*)out, act);
        return check_launch("k_dwconv3_blk");
    }
    if (KH == 3 && KW == 3 && C % 4 == 0 && al) {
        long long total = (long long)N * OH * OW * (C / 4);
        ACFUN_LAUNCH("k_dwconv", k_dwconv3_c4, grid1d(total), dim3(256), 0, s, (const float4*)in, N, H,
                           W, C / 4, w, bias, stride, pad, OH, OW, (float4*)out, act);
        return check_launch("k_dwconv3_c4");
    }
    long long total = (long long)N * OH * OW * C;
    ACFUN_LAUNCH("k_dwconv", k_dwconv, grid1d(total), dim3(256), 0, s, in, N, H, W, C, w, bias, KH, KW,
                       stride, pad, OH, OW, out, act);
    return check_launch("k_dwconv");
}

bool dwconv_pool_ok(int H, int W, int C, int KH, int KW, int stride, int pad, int pool,
                    int pstride, int ppad, const void* in, const void* w, const void* out) {
    const int OH = (H + 2 * pad - KH) / stride + 1, OW = (W + 2 * pad - KW) / stride + 1;
    return KH == 3 && KW == 3 && (stride == 1 || stride == 2) && C % 4 == 0 && pool == 3 &&
           pstride == 2 && (ppad == 0 || ppad == 1) && OH > 0 && OW > 0 &&
           (OH + 2 * ppad - 3) / 2 + 1 > 0 && (OW + 2 * ppad - 3) / 2 + 1 > 0 &&
           ((((uintptr_t)in) | ((uintptr_t)w) | ((uintptr_t)out)) & 15u) == 0;
}

bool dwconv_pool_f32(const float* in, int N, int H, int W, int C, const float* w,
                     const float* bias, int stride, int pad, int act, int ppad, float* out,
                     int post_relu, hipStream_t s) {
    const int OH = (H + 2 * pad - 3) / stride + 1, OW = (W + 2 * pad - 3) / stride + 1;
    const int PH = (OH + 2 * ppad - 3) / 2 + 1, PW = (OW + 2 * ppad - 3) / 2 + 1;
    if (OH <= 0 || OW <= 0 || PH <= 0 || PW <= 0 || N <= 0) return true;
    const int C4 = C / 4;
    const int nPHB = (PH + 1) / 2, nPWB = (PW + DWP_PWB - 1) / DWP_PWB,
              nQG = (C4 + DWP_Q - 1) / DWP_Q;
    const long long items = (long long)N * nPHB * nPWB * nQG;
    if (items >= (1ll << 30)) {
        set_error("dwconv_pool: grid too large");
        return false;
    }
    // maxpool_f32's per-channel rule (max_ps below pvec_end)
    const int pvec_end = C >= 16 ? (C & ~15) : (C >= 8 ? (C & ~7) : 0);
    const long long in_bytes = (long long)N * H * W * C * 4;
    if (stride == 2 && in_bytes < (1ll << 31)) {
        const int nstrip = (PH + DWR_RP - 1) / DWR_RP;
        const long long lanes = (long long)N * nstrip * ((PW * C4 + 63) / 64 * 64);
        const long long wgs = (lanes + 255) / 256;
        if (lanes < (1ll << 30)) {
            ACFUN_LAUNCH("k_dwconv_pool", k_dwconv3_pool_rs, dim3((unsigned)(8 * ((wgs + 7) / 8))), dim3(256),
                         0, s, in, H, W, C4, w, bias, pad, OH, OW, act, ppad, PH, PW, nstrip, (int)lanes,
                         (int)in_bytes, pvec_end, (float4*)out, post_relu);
            return check_launch("k_dwconv3_pool_rs");
        }
    }
    const unsigned blocks = (unsigned)(8 * ((items + 7) / 8));   // 8 equal XCD ranges
    if (stride == 1)
        ACFUN_LAUNCH("k_dwconv_pool", k_dwconv3_pool<1>, dim3(blocks), dim3(320), 0, s,
                     (const float4*)in, H, W, C4, w, bias, pad, OH, OW, act, ppad, PH, PW, nPHB,
                     nPWB, nQG, (int)items, pvec_end, (float4*)out, post_relu);
    else
        ACFUN_LAUNCH("k_dwconv_pool", k_dwconv3_pool<2>, dim3(blocks), dim3(320), 0, s,
                     (const float4*)in, H, W, C4, w, bias, pad, OH, OW, act, ppad, PH, PW, nPHB,
                     nPWB, nQG, (int)items, pvec_end, (float4*)out, post_relu);
    return check_launch("k_dwconv3_pool");
}

bool gconv_pool_ok(int N, int H, int W, int Cin, int KH, int KW, int Cout, int stride, int pad,
                   int groups, int pool, int pstride, int ppad, const void* in, const void* w,
                   const void* out) {
    if (groups <= 1 || Cin % groups || Cout % groups || stride <= 0) return false;
    const int Cin_p = Cin / groups, Cout_p = Cout / groups;
    const int OH = (H + 2 * pad - KH) / stride + 1, OW = (W + 2 * pad - KW) / stride + 1;
    if (OH <= 0 || OW <= 0) return false;
    const int PH = (OH + 2 * ppad - 3) / 2 + 1, PW = (OW + 2 * ppad - 3) / 2 + 1;
    return KH == 3 && KW == 3 && (Cin_p == 4 || Cin_p == 8) && Cout_p >= 8 && Cout_p % 4 == 0 &&
           pool == 3 && pstride == 2 && (ppad == 0 || ppad == 1) && PH > 0 && PW > 0 &&
           (long long)N * PH * PW * (Cout / 4) < (1ll << 31) &&
           ((((uintptr_t)in) | ((uintptr_t)w) | ((uintptr_t)out)) & 15u) == 0;
}

bool gconv_pool_f32(const float* in, int N, int H, int W, int Cin, const float* w,
                    const float* bias, int Cout, int stride, int pad, int groups, int act, int ppad,
                    float* out, int post_relu, hipStream_t s) {
    const int OH = (H + 2 * pad - 3) / stride + 1, OW = (W + 2 * pad - 3) / stride + 1;
    const int PH = (OH + 2 * ppad - 3) / 2 + 1, PW = (OW + 2 * ppad - 3) / 2 + 1;
    if (N <= 0 || OH <= 0 || OW <= 0 || PH <= 0 || PW <= 0) return true;
    const int Cout_p = Cout / groups, Cin_p = Cin / groups;
    // the conv's and the pool's per-channel rules, as gconv_f32 and maxpool_f32 pick them
    const int vec_end = Cout_p >= 16 ? Cout_p : (Cout_p >= 8 ? (Cout_p & ~7) : 0);
    const int pvec_end = Cout >= 16 ? (Cout & ~15) : (Cout >= 8 ? (Cout & ~7) : 0);
    // one workgroup per (image, pooled row) with its input rows, the weights and
    // its three conv rows in LDS
    const size_t row_lds = ((size_t)(2 * stride + 3) * W * Cin + (size_t)Cout * 9 * Cin_p +
                            (size_t)3 * OW * Cout + Cout) * sizeof(float);
    if (row_lds <= 64 * 1024 && (long long)N * PH < (1ll << 31) && W * Cin % 4 == 0) {
        // set once per process, thread-safely, before any launch below
        static const bool attr = [&] {
            (void)hipFuncSetAttribute((const void*)k_gconv3_pool_row<1>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, 64 * 1024);
            (void)hipFuncSetAttribute((const void*)k_gconv3_pool_row<2>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, 64 * 1024);
            return true;
        }();
        (void)attr;
        const dim3 grid((unsigned)(N * PH));
        if (Cin_p == 4)
            ACFUN_LAUNCH("k_gconv_pool", k_gconv3_pool_row<1>, grid, dim3(512), row_lds, s, in, H, W, Cin,
                         w, bias, Cout, stride, pad, groups, OH, OW, act, vec_end, ppad, PH, PW,
                         pvec_end, out, post_relu);
        else
            ACFUN_LAUNCH("k_gconv_pool", k_gconv3_pool_row<2>, grid, dim3(512), row_lds, s, in, H, W, Cin,
                         w, bias, Cout, stride, pad, groups, OH, OW, act, vec_end, ppad, PH, PW,
                         pvec_end, out, post_relu);
        return check_launch("k_gconv3_pool_row");
    }
    // small images: one workgroup per (image, group) with the image in LDS
    const size_t img_lds = ((size_t)H * W * Cin_p + (size_t)OH * OW * Cout_p) * sizeof(float);
    if (img_lds <= 48 * 1024 && Cout_p / 4 <= 256 && (long long)N * groups < (1ll << 31)) {
        const dim3 grid((unsigned)(N * groups));
        if (Cin_p == 4)
            ACFUN_LAUNCH("k_gconv_pool", k_gconv3_pool_img<1>, grid, dim3(256), img_lds, s, in, H, W, Cin,
                         w, bias, Cout, stride, pad, groups, OH, OW, act, vec_end, ppad, PH, PW,
                         pvec_end, out, post_relu);
        else
            ACFUN_LAUNCH("k_gconv_pool", k_gconv3_pool_img<2>, grid, dim3(256), img_lds, s, in, H, W, Cin,
                         w, bias, Cout, stride, pad, groups, OH, OW, act, vec_end, ppad, PH, PW,
                         pvec_end, out, post_relu);
        return check_launch("k_gconv3_pool_img");
    }
    const long long total = (long long)N * PH * PW * (Cout / 4);
    if (Cin_p == 4)
        ACFUN_LAUNCH("k_gconv_pool", k_gconv3_pool<1>, grid1d(total), dim3(256), 0, s, in, N, H, W, Cin, w,
                     bias, Cout, stride, pad, groups, OH, OW, act, vec_end, ppad, PH, PW, pvec_end, out,
                     post_relu);
    else
        ACFUN_LAUNCH("k_gconv_pool", k_gconv3_pool<2>, grid1d(total), dim3(256), 0, s, in, N, H, W, Cin, w,
                     bias, Cout, stride, pad, groups, OH, OW, act, vec_end, ppad, PH, PW, pvec_end, out,
                     post_relu);
    return check_launch("k_gconv3_pool");
}

bool gconv_f32(const float* in, int N, int H, int W, int Cin, const float* w, const float* bias,
               int KH, int KW, int Cout, int stride, int pad, int groups, float* out, int act,
               hipStream_t s) {
    if (groups <= 1 || KH <= 0 || KW <= 0) return true;
    int OH = (H + 2 * pad - KH) / stride + 1;
    int OW = (W + 2 * pad - KW) / stride + 1;
    if (OH <= 0 || OW <= 0) return true;
    int Cout_p = Cout / groups;
    // src/group_conv.cpp:60-79 on an AVX-512 host: >=16 -> all-FMA kernel,
    // >=8 -> AVX2 kernel (vector part + contracted scalar tail), else scalar.
    int vec_end = Cout_p >= 16 ? Cout_p : (Cout_p >= 8 ? (Cout_p & ~7) : 0);
    int fma_all = Cout_p >= 8 ? 1 : 0;
    const int Cin_p = Cin / groups;
    auto al = [](const void* q) { return ((uintptr_t)q & 15u) == 0; };
    if (fma_all && Cin_p % 4 == 0 && Cout_p % 4 == 0 && al(in) && al(w) && al(out) &&
        (!bias || al(bias))) {
        const long long total4 = (long long)N * OH * OW * (Cout / 4);
        if (KH == 3 && KW == 3 && (Cin_p == 4 || Cin_p == 8) && total4 < (1ll << 31)) {
            if (Cin_p == 4)
                ACFUN_LAUNCH("k_gconv", k_gconv4_3x3<1>, grid1d(total4), dim3(256), 0, s, in, N, H, W, Cin,
                             w, bias, Cout, stride, pad, groups, OH, OW, out, act, vec_end);
            else
                ACFUN_LAUNCH("k_gconv", k_gconv4_3x3<2>, grid1d(total4), dim3(256), 0, s, in, N, H, W, Cin,
                             w, bias, Cout, stride, pad, groups, OH, OW, out, act, vec_end);
            return check_launch("k_gconv4_3x3");
        }
        ACFUN_LAUNCH("k_gconv", k_gconv4, grid1d(total4), dim3(256), 0, s, in, N, H, W, Cin, w, bias, KH,
                     KW, Cout, stride, pad, groups, OH, OW, out, act, vec_end);
        return check_launch("k_gconv4");
    }
    long long total = (long long)N * OH * OW * Cout;
    ACFUN_LAUNCH("k_gconv", k_gconv, grid1d(total), dim3(256), 0, s, in, N, H, W, Cin, w, bias, KH, KW,
                       Cout, stride, pad, groups, OH, OW, out, act, vec_end, fma_all);
    return check_launch("k_gconv");
}

bool maxpool_f32(const float* in, int N, int H, int W, int C, int pool, int stride, int pad,
                 float* out, int post_relu, hipStream_t s) {
    int OH = (H + 2 * pad - pool) / stride + 1;
    int OW = (W + 2 * pad - pool) / stride + 1;
    if (OH <= 0 || OW <= 0) return true;
    int vec_end = C >= 16 ? (C & ~15) : (C >= 8 ? (C & ~7) : 0);
    const long long nq = (long long)N * OH * ((OW + 3) / 4) * (C / 4);
    if (pool == 3 && stride == 2 && vec_end == C && C % 4 == 0 &&
        (((uintptr_t)in | (uintptr_t)out) & 15u) == 0 && nq < (1ll << 31) &&
        (long long)N * H * W * C < (1ll << 31)) {
        const int total = (int)nq;
        ACFUN_LAUNCH("k_maxpool", k_maxpool3s2_row, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                           (const float4*)in, H, W, C / 4, pad, OH, OW, (OW + 3) / 4, total,
                           (float4*)out, post_relu);
        return check_launch("k_maxpool3s2_row");
    }
    long long total = (long long)N * OH * OW * C;
    ACFUN_LAUNCH("k_maxpool", k_maxpool, grid1d(total), dim3(256), 0, s, in, N, H, W, C, pool, stride,
                       pad, OH, OW, out, post_relu, vec_end);
    return check_launch("k_maxpool");
}

bool relu_f32(float* d, size_t n, int six, hipStream_t s) {
    if (!n) return true;
    ACFUN_LAUNCH("k_relu", k_relu, grid1d((long long)n), dim3(256), 0, s, d, n, six);
    return check_launch("k_relu");
}

bool fill_f32(float* d, size_t n, float v, hipStream_t s) {
    if (!n) return true;
    ACFUN_LAUNCH("k_fill", k_fill, grid1d((long long)n), dim3(256), 0, s, d, n, v);
    return check_launch("k_fill");
}

bool add_relu_f32(const float* a, const float* b, float* y, size_t n, int act, hipStream_t s) {
    if (!n) return true;
    ACFUN_LAUNCH("k_add_relu", k_add_relu, grid1d((long long)n), dim3(256), 0, s, a, b, y, n, act);
    return check_launch("k_add_relu");
}

bool gap_f32(const float* x, int N, int HW, int C, float* y, hipStream_t s) {
    if (N <= 0 || C <= 0 || HW <= 0) return true;
    ACFUN_LAUNCH("k_gap", k_gap, grid1d((long long)N * C), dim3(256), 0, s, x, N, HW, C, y);
    return check_launch("k_gap");
}

bool softmax_f32(const float* in, int rows, int cols, float* out, hipStream_t s) {
    if (rows <= 0 || cols <= 0) return true;
    ACFUN_LAUNCH("k_softmax", k_softmax, dim3(rows), dim3(256), 0, s, in, cols, out);
    return check_launch("k_softmax");
}

bool batchnorm_f32(float* d, int size, int channels, const float* mean, const float* var,
                   const float* gamma, const float* beta, float eps, hipStream_t s) {
    if (size <= 0 || channels <= 0) return true;
    long long total = (long long)(size / channels) * channels;
    ACFUN_LAUNCH("k_batchnorm", k_batchnorm, grid1d(total), dim3(256), 0, s, d, total, channels, mean, var,
                       gamma, beta, eps);
    return check_launch("k_batchnorm");
}

bool group_split_copy(const float* src, int pix, int srcC, int off, int cnt, float* dst, int dstC,
                      int dstOff, hipStream_t s) {
    long long total = (long long)pix * cnt;
    if (!total) return true;
    ACFUN_LAUNCH("k_chan_copy", k_chan_copy, grid1d(total), dim3(256), 0, s, src, pix, srcC, off, cnt, dst,
                       dstC, dstOff);
    return check_launch("k_chan_copy");
}

}  // namespace acfun
