// k_i8q1.hip -- the float-input 1x1 int8 convolution with the activation
// quantization fused into the staging of the A operand.
//
// acfun_conv2d_int8 (src/conv_int8.cpp:63-148) quantizes its fp32 input to u8
// with the tensor's scale 127/max|x| (src/conv_int8.cpp:77-81, rounded as
// src/int8_quantize_avx512.cpp:15-20 does) and multiplies it with the s8
// weights.  For a 1x1 / stride-1 / pad-0 convolution (the GEMM
// out[pixel][channel]) this kernel forms those values (as s8 = u8 - 128)
// while it stages the operand: no quantized tensor goes through HBM and no
// quantize pass runs between the absmax partials and the product.
//
// Work unit: a block of 64 pixels and a group of up to ngt 64-channel output
// tiles.  The workgroup (256 threads; 2 x 2 waves, one 32 x 32
// v_mfma_i32_32x32x32_i8 block each per tile) loads the block's fp32 rows
// once, quantizes them and keeps them in LDS as s8 for all the unit's tiles.
// The weight tiles stream through NST stages by LDS DMA (buffer_load ... lds)
// as a (tile, chunk) item stream that runs NST - 1 chunks ahead, across
// units.  Every workgroup reduces the absmax partials to the tensor's max
// itself.  The epilogue is k_i8mm's GEMM route (i8mm.hpp): the reference's
// factors in its operation order, the fused residual and activation, rows
// stored as 16-byte quads through a 64 x 64 LDS stage, and the per-workgroup
// output maximum.
#include "i8mm.hpp"

#include <algorithm>
#include <cstdio>
#include <cstdlib>

namespace acfun {
namespace i8k {
namespace {

// Launch-derived fields of k_i8q1.
struct Q1L {
    int gn;          // 64-channel output tiles
    int ngt;         // tiles per unit
    int nug;         // units per pixel block: ceil(gn / ngt)
    int units;       // pixel blocks * nug
    int vec;         // Cf (and res) rows allow 16-byte stores / loads
    int xvec;        // x allows 16-byte loads (16-byte aligned, Cin % 4 == 0)
    unsigned b_bytes;
};

// LDS of k_i8q1: the s8 block of 64 rows (nch chunks of 128 channels), NST
// weight stages of 64 rows x 128 bytes, the 64 x 64 fp32 epilogue stage and
// three per-column parameter arrays of the unit's ngt tiles.
constexpr size_t q1_lds(int nch, int nst, int ngt) {
    return (size_t)(nch + nst) * 8192 + 16384 + (size_t)3 * ngt * 64 * 4;
}
constexpr int kQ1MaxNgt = 8;

// OCC: the workgroups per CU the build targets (2 or 3; the register budget
// for 3 is 168 VGPRs, which the staging of two groups per round keeps to)
template <int NST, int OCC>
__global__ __launch_bounds__(256, OCC) void k_i8q1(I8Q1 p, Q1L l) {
    constexpr int AHEAD = NST - 1;
    constexpr int QG = OCC >= 3 ? 2 : 4;         // 16-channel groups per thread per staging round
    constexpr int BIT = 2;                       // DMA instructions per wave per weight chunk
    constexpr unsigned kOOB = 0x80000000u;
    typedef __attribute__((address_space(3))) void lds_void;
    typedef int i16v __attribute__((ext_vector_type(16)));
    extern __shared__ __attribute__((aligned(16))) int8_t sm8[];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nch = (p.Cinp + 127) >> 7;        // 128-channel chunks of K
    int8_t* const ablk = sm8;                    // chunk c, row r, quad q at c*8192 + r*128 + 16*(q ^ swz(r))
    int8_t* const bst = sm8 + nch * 8192;        // NST stages, the same layout
    float* const stg = (float*)(bst + NST * 8192);
    float* const pal = stg + 4096;               // per column of the unit: alpha,
    float* const pbe = pal + l.ngt * 64;         // beta,
    int* const pco = (int*)(pbe + l.ngt * 64);   // 128 * (column sum of the weights)

    // ---- units of this workgroup: t0, t0 + tstr, ... (cnt of them); the
    // units are cut into 8 contiguous runs, one per XCD (workgroup id mod 8),
    // so the units of one pixel block share an L2
    const int total = l.units, G = gridDim.x, b = blockIdx.x;
    int t0, tstr, cnt;
    if ((G & 7) == 0) {
        const int x = b & 7, i = b >> 3, gx = G >> 3;
        const int sx = (int)(((long long)x * total) >> 3);
        const int ex = (int)(((long long)(x + 1) * total) >> 3);
        t0 = sx + i;
        tstr = gx;
        cnt = ex > t0 ? (ex - t0 + gx - 1) / gx : 0;
    } else {
        t0 = b;
        tstr = G;
        cnt = b < total ? (total - b + G - 1) / G : 0;
    }
    auto ntl_of = [&](int u) {                   // output tiles of unit u
        const int r = l.gn - (u % l.nug) * l.ngt;
        return r < l.ngt ? r : l.ngt;
    };
    int nit = 0;
    for (int k = 0; k < cnt; ++k) nit += ntl_of(t0 + k * tstr) * nch;

    // ---- weight DMA: row 8*(wave + 4t) + lane/8 of a stage, quad slot lane%8
    // holding data quad bk/16 of the chunk
    const __amdgpu_buffer_rsrc_t bres =
        __builtin_amdgcn_make_buffer_rsrc((void*)p.Bt, (short)0, (int)l.b_bytes, 0x00020000);
    const int sl = lane & 7, rl = lane >> 3;
    int bk[BIT];
#pragma unroll
    for (int t = 0; t < BIT; ++t) bk[t] = 16 * (sl ^ i8swz(8 * (wave + 4 * t) + rl));
    unsigned bv[BIT];                            // byte offsets of this lane's rows at chunk 0
    int iu = 0, ik = 0, ic = 0, intl = 0;        // issue cursor: unit, tile in it, chunk; its tiles
    auto setup = [&]() {
        const int u = t0 + iu * tstr;
        intl = ntl_of(u);
        const int tn = (u % l.nug) * l.ngt + ik;
#pragma unroll
        for (int t = 0; t < BIT; ++t) {
            const int n = tn * 64 + 8 * (wave + 4 * t) + rl;
            bv[t] = n < p.N ? (unsigned)(n * p.ldb + bk[t]) : kOOB;
        }
    };
    // DMA item t of the issue cursor's chunk into stage st.  A chunk past the
    // end (live false) is issued all out of range: it writes zeros to a stage
    // no chunk reads again and keeps the number of loads per iteration fixed,
    // so every wait of the loop is the same.
    auto issue = [&](int t, int8_t* st, bool live) {
        const unsigned v = live ? bv[t] + (unsigned)(ic << 7) : kOOB;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(bres, (lds_void*)(st + (wave + 4 * t) * 1024), 16, v, 0,
                                                 0, 0);
    };
    auto advance = [&]() {
        if (++ic < nch) return;
        ic = 0;
        if (++ik == intl) {
            ik = 0;
            ++iu;
        }
        if (iu < cnt) setup();
    };

    // ---- prologue: the first AHEAD chunks of the item stream
    if (nit > 0) setup();
#pragma unroll
    for (int a = 0; a < AHEAD; ++a) {
        const bool live = a < nit;
#pragma unroll
        for (int t = 0; t < BIT; ++t) issue(t, bst + a * 8192, live);
        if (live) advance();
    }

    // ---- the tensor's scale from the absmax partials, as k_quant16 forms it
    // (the partial loads sit behind the prologue's DMA in the counter)
    float maxa;
    {
        __shared__ float red[4];
        float m = 0.0f;
        for (int i = tid; i < p.nparts; i += 256) {
            const float a = p.part[i];
            m = a > m ? a : m;
        }
        for (int off = 32; off > 0; off >>= 1) {
            const float o = __shfl_xor(m, off, 64);
            m = o > m ? o : m;
        }
        if (lane == 0) red[wave] = m;
        __syncthreads();
        maxa = red[0];
        for (int k = 1; k < 4; ++k) maxa = red[k] > maxa ? red[k] : maxa;
    }
    const bool zero = maxa < 1e-12f;             // an all-zero input: output 0 (src/conv_int8.cpp:78)
    const float inv_s = 127.0f / maxa, sa = maxa / 127.0f;
    if (b == 0 && tid == 0 && p.scal) {
        p.scal[0] = inv_s;
        p.scal[1] = sa;
        p.scal[2] = zero ? 1.0f : 0.0f;
        p.scal[3] = maxa;
    }

    // ---- a unit's 64 pixel rows, quantized into the s8 block: thread t takes
    // 16-channel groups t, t + 256, ... of the block (consecutive threads read
    // consecutive 64-byte pieces of a row), QG groups in flight per round.
    // s8 = clamp(cvt(rint(x * inv_s)) + 128, 0, 255) - 128 with the x86
    // conversion's NaN rule; channels past Cin and rows past M give 0.
    const int gpr = p.Cinp >> 4, gtot = 64 * gpr;
    // (wave-uniform) every group is 16 whole channels at a 16-byte aligned address
    const bool xfast = l.xvec && (p.Cin & 15) == 0;
    auto stage_a = [&](int m0) {
        for (int j0 = 0; j0 < gtot; j0 += 256 * QG) {
            float v[QG][16];
            bool in[QG], kv[QG];
            // group j0 + 256k + tid exists for the whole wave or for none of it
            // (gtot is a multiple of 64): a scalar branch, and every load
            // issued is consumed (a load left in flight would make the
            // compiler wait for all memory before reusing its registers)
#pragma unroll
            for (int k = 0; k < QG; ++k) kv[k] = j0 + 256 * k + 64 * wave < gtot;
            if (xfast) {
                // the round's 16-byte loads all in flight; a lane past the
                // block's rows loads the tensor's first group and drops it
#pragma unroll
                for (int k = 0; k < QG; ++k) {
                    if (!kv[k]) continue;
                    const int j = j0 + 256 * k + tid;
                    const int r = j / gpr, c0 = 16 * (j - r * gpr);
                    const int m = m0 + r;
                    in[k] = j < gtot && m < p.M;
                    const float4* src = (const float4*)(p.x + (in[k] ? (long long)m * p.Cin + c0 : 0));
#pragma unroll
                    for (int q4 = 0; q4 < 4; ++q4) {
                        const float4 f = src[q4];
                        v[k][4 * q4] = f.x;
                        v[k][4 * q4 + 1] = f.y;
                        v[k][4 * q4 + 2] = f.z;
                        v[k][4 * q4 + 3] = f.w;
                    }
                }
            } else {
#pragma unroll
                for (int k = 0; k < QG; ++k) {
                    if (!kv[k]) continue;
                    const int j = j0 + 256 * k + tid;
                    const int r = j / gpr, c0 = 16 * (j - r * gpr);
                    const int m = m0 + r;
                    in[k] = j < gtot && m < p.M;
                    const float* src = p.x + (in[k] ? (long long)m * p.Cin + c0 : 0);
#pragma unroll
                    for (int e = 0; e < 16; ++e) v[k][e] = in[k] && c0 + e < p.Cin ? src[e] : 0.0f;
                }
            }
#pragma unroll
            for (int k = 0; k < QG; ++k) {
                if (!kv[k]) continue;
                const int j = j0 + 256 * k + tid;
                const int r = j / gpr, gq = j - r * gpr, c0 = 16 * gq;
                unsigned w[4] = {0u, 0u, 0u, 0u};
                if (!zero) {
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const float t = __fmul_rn(in[k] ? v[k][e] : 0.0f, inv_s);
                        const int out = c0 + e < p.Cin ? x86_u8(x86_cvt(rintf(t)), 128) - 128 : 0;
                        w[e >> 2] |= ((unsigned)out & 0xffu) << (8 * (e & 3));
                    }
                }
                *(i4*)(ablk + (gq >> 3) * 8192 + r * 128 + 16 * ((gq & 7) ^ i8swz(r))) =
                    i4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
            }
        }
    };
    // ---- the unit's per-column factors (src/conv_int8.cpp:100-107: alpha =
    // sa * ws; beta = b - (alpha * 128) * Sw), formed as k_i8mm's GEMM route does
    auto params = [&](int tn0, int ntl) {
        for (int i = tid; i < ntl * 64; i += 256) {
            const int n = tn0 * 64 + i;
            float a = 0.0f, be = 0.0f;
            int co = 0;
            if (n < p.N) {
                const int sw = p.Sw[n];
                co = 128 * sw;
                a = __fmul_rn(sa, p.ws[n]);
                be = __fsub_rn(p.bias ? p.bias[n] : 0.0f, __fmul_rn(__fmul_rn(a, 128.0f), (float)sw));
                if (zero) {
                    a = 0.0f;
                    be = 0.0f;
                }
            }
            pal[i] = a;
            pbe[i] = be;
            pco[i] = co;
        }
    };

    // ---- LDS read offsets (bytes within a chunk) of this lane, per k-step
    const int r32 = lane & 31, hq = lane >> 5;
    const int wm = wave >> 1, wn = wave & 1;
    int rda[4], rdb[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const int ra = wm * 32 + r32, rb = wn * 32 + r32;
        rda[s] = ra * 128 + 16 * ((2 * s + hq) ^ i8swz(ra));
        rdb[s] = rb * 128 + 16 * ((2 * s + hq) ^ i8swz(rb));
    }
    i16v acc;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0;
    // the epilogue stage: quad q of row r at quad q ^ (8 * bit 2 of r)
    auto sidx = [](int r, int c) { return r * 64 + ((((c >> 2) ^ (((r >> 2) & 1) << 3))) << 2) + (c & 3); };

    int st = 0, cu = 0, ck = 0, cc = 0;          // compute cursor: stage, unit, tile, chunk
    int m0 = 0, tn0 = 0, cntl = 0;
    float amx = 0.0f;                            // max|stored value| of this lane
    for (int g = 0; g < nit; ++g) {
        // Every iteration issues BIT loads (chunk g + AHEAD, real or out of
        // range), so AHEAD - 1 chunks issued after chunk g account for
        // (AHEAD - 1) * BIT loads; anything else queued after chunk g (a unit's
        // row loads, residual loads, stores) only makes the wait longer (loads
        // and stores complete in issue order).
        __builtin_amdgcn_s_waitcnt(vmcnt_enc((AHEAD - 1) * BIT));
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (cc == 0 && ck == 0) {
            // a new unit (every wave is past the previous unit's last reads of
            // the s8 block and the parameters: the barrier above)
            const int u = t0 + cu * tstr;
            m0 = (u / l.nug) * 64;
            tn0 = (u % l.nug) * l.ngt;
            cntl = ntl_of(u);
            stage_a(m0);
            params(tn0, cntl);
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        }
        const int8_t* S = bst + st * 8192;
        const int8_t* A = ablk + cc * 8192;
        int8_t* NB = bst + (st == 0 ? NST - 1 : st - 1) * 8192;   // stage (g + AHEAD) % NST
        const bool more = g + AHEAD < nit;
        const int n0 = (tn0 + ck) * 64;
        const bool full = m0 + 64 <= p.M && n0 + 64 <= p.N;
        i4 fa[4], fb[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            fa[s] = *(const i4*)(A + rda[s]);
            fb[s] = *(const i4*)(S + rdb[s]);
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[s], fb[s], acc, 0, 0, 0);
            if (s == 0) issue(0, NB, more);
            if (s == 2) issue(1, NB, more);
        }
        if (more) advance();
        st = st == NST - 1 ? 0 : st + 1;
        if (++cc < nch) continue;

        // ---- epilogue of tile ck of the unit: lane l, register e <-> row
        // m0 + wm*32 + 8(e/4) + 4(l/32) + e%4, column n0 + wn*32 + l%32
        {
            const int col = wn * 32 + r32;
            const float al = pal[ck * 64 + col], be = pbe[ck * 64 + col];
            const int corr = pco[ck * 64 + col];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int r = wm * 32 + 8 * (e >> 2) + 4 * hq + (e & 3);
                // fl(fl(acc_u * alpha) + beta), acc_u = acc_s + 128 * Sw
                stg[sidx(r, col)] =
                    __fadd_rn(__fmul_rn((float)(int)((unsigned)acc[e] + (unsigned)corr), al), be);
                acc[e] = 0;
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        {
            // thread t: quad t%16 of rows t/16 + 16i; one loop per activation
            // form, with or without the workgroup maximum (I8Q1::amax)
            const int q = tid & 15;
            const bool fast = full && l.vec;
            auto rows = [&](auto actc, auto trackc, auto fastc) {
                constexpr int ACT = decltype(actc)::value;
                constexpr bool TRACK = decltype(trackc)::value, FAST = decltype(fastc)::value;
                // a full tile's four residual rows load together (the stores
                // below are inline asm, which no load is moved across)
                f4v rres[4];
                if (FAST && p.res) {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        rres[i] = *(const f4v*)(p.res + (long long)(m0 + (tid >> 4) + 16 * i) * p.ldr + n0 + 4 * q);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = (tid >> 4) + 16 * i;
                    const int m = m0 + r, n = n0 + 4 * q;
                    f4v v = *(const f4v*)&stg[sidx(r, 4 * q)];
                    float* dst = p.Cf + (long long)m * p.ldc + n;
                    if (FAST || (l.vec && m < p.M && n + 4 <= p.N)) {
                        if (p.res) {
                            const f4v rv = FAST ? rres[i] : *(const f4v*)(p.res + (long long)m * p.ldr + n);
                            v = v + rv;          // fl(v + res) per lane, as a separate Add
                        }
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            v[k] = act_apply(v[k], ACT);
                            if (TRACK) {
                                const float av = fabsf(v[k]);
                                amx = av > amx ? av : amx;
                            }
                        }
                        // s_nop: a VALU write to the data registers of a store of
                        // more than 8 bytes needs a wait state after it
                        asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1" ::"v"(dst), "v"(v)
                                     : "memory");
                    } else if (!FAST && m < p.M) {
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            if (n + k >= p.N) continue;
                            float w = v[k];
                            if (p.res) w = __fadd_rn(w, p.res[(long long)m * p.ldr + n + k]);
                            w = act_apply(w, ACT);
                            if (TRACK) {
                                const float av = fabsf(w);
                                amx = av > amx ? av : amx;
                            }
                            asm volatile("global_store_dword %0, %1, off sc1" ::"v"(dst + k), "v"(w) : "memory");
                        }
                    }
                }
            };
            with_act(p.act, [&](auto actc) {
                if (fast) {
                    if (p.amax) rows(actc, std::true_type{}, std::true_type{});
                    else rows(actc, std::false_type{}, std::true_type{});
                } else {
                    if (p.amax) rows(actc, std::true_type{}, std::false_type{});
                    else rows(actc, std::false_type{}, std::false_type{});
                }
            });
        }
        cc = 0;
        if (++ck == cntl) {
            ck = 0;
            ++cu;
        }
    }
    // this workgroup's max|v| of the output, a partial of the next layer's absmax
    if (p.amax) {
        __shared__ float wmax[4];
        for (int off = 32; off > 0; off >>= 1) {
            const float o = __shfl_xor(amx, off, 64);
            amx = o > amx ? o : amx;
        }
        if (lane == 0) wmax[wave] = amx;
        __syncthreads();
        if (tid == 0) {
            float mm = wmax[0];
            for (int w = 1; w < 4; ++w) mm = wmax[w] > mm ? wmax[w] : mm;
            p.amax[blockIdx.x] = mm;
        }
    }
    // (stores issued by inline asm: drain them before the wave ends)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// ACFUN_I8Q1: "0" turns the fused kernel off (the quantize pass and k_i8mm
// run instead, with the same results); "ngt,nst,per_cu" takes it for every
// output width with that many tiles per unit (1-8), weight stages (2-4) and
// workgroups per CU, for sweeps.  Read once per process.
struct Q1Env {
    bool on = true;
    bool forced = false;
    int ngt = 0, nst = 2, per_cu = 3;
};
const Q1Env& q1_env() {
    static const Q1Env env = [] {
        Q1Env v;
        if (const char* e = std::getenv("ACFUN_I8Q1")) {
            int a = 0, b = 0, c = 0;
            if (*e == '0' && e[1] == 0) v.on = false;
            else if (std::sscanf(e, "%d,%d,%d", &a, &b, &c) == 3 && a >= 1 && a <= kQ1MaxNgt && b >= 2 &&
                     b <= 4 && c >= 1 && c <= 8) {
                v.forced = true;
                v.ngt = a;
                v.nst = b;
                v.per_cu = c;
            }
        }
        return v;
    }();
    return env;
}

template <int NST, int OCC>
bool launch_nst(I8Q1& a, const Q1L& l, int per_cu, hipStream_t s) {
    const int nch = (a.Cinp + 127) >> 7;
    const size_t lds = q1_lds(nch, NST, l.ngt);
    // set once per process, thread-safely, before any launch below: the
    // largest dynamic LDS a launch of this instantiation asks for
    static const bool attr = [] {
        (void)hipFuncSetAttribute((const void*)k_i8q1<NST, OCC>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)q1_lds(kI8Q1MaxCinp / 128, NST, kQ1MaxNgt));
        return true;
    }();
    (void)attr;
    // persistent workgroups: at most per_cu per CU and as many as LDS allows,
    // a multiple of 8 (the per-XCD runs), at most kAmaxParts (one output
    // maximum partial each)
    const int fit = (int)((160 * 1024) / (lds + 256));
    long long g = std::min<long long>(l.units, (long long)std::min(per_cu, std::max(fit, 1)) * num_cus());
    if (g >= 8) g &= ~7ll;
    if (g > kAmaxParts) g = kAmaxParts;
    a.grid = (int)g;
    ACFUN_LAUNCH("k_i8q1", (k_i8q1<NST, OCC>), dim3((unsigned)g), dim3(256), lds, s, a, l);
    return check_launch("k_i8q1");
}

}  // namespace
}  // namespace i8k

// Measured (batch-64 ResNet-50 shapes): the fused kernel is faster where a
// 64-pixel block feeds one output tile (256 -> 64 at 56 x 56: 83.8 against
// 91.6 us; 64 -> 64: 34.5 against 37.4) and slower where one quantized block
// feeds several (256 -> 512 at 28 x 28: 36.8 against 32.1 us), so it takes
// Cout <= 64 unless forced.
bool i8q1_route(int Cout) {
    const i8k::Q1Env& e = i8k::q1_env();
    return e.on && (e.forced || Cout <= 64);
}

bool launch_i8q1(I8Q1& a, hipStream_t s) {
    using namespace i8k;
    if (a.M <= 0 || a.N <= 0) return true;
    if (a.Cinp <= 0 || a.Cinp % 16 != 0 || a.Cinp > kI8Q1MaxCinp || a.Cin > a.Cinp || a.ldb < a.Cinp ||
        a.ldb % 128 != 0 || (long long)a.N * a.ldb >= 0x7fffffffll || a.nparts < 0 ||
        a.nparts > kAmaxParts) {
        set_error("k_i8q1: unsupported operands (Cin %d, Cinp %d, ldb %d, N %d)", a.Cin, a.Cinp, a.ldb, a.N);
        return false;
    }
    const Q1Env& env = q1_env();
    auto al16 = [](const void* q) { return ((uintptr_t)q & 15u) == 0; };
    Q1L l{};
    l.gn = (a.N + 63) / 64;
    const long long gm = ((long long)a.M + 63) / 64;
    l.vec = al16(a.Cf) && a.ldc % 4 == 0 && (!a.res || (al16(a.res) && a.ldr % 4 == 0));
    l.xvec = al16(a.x) && a.Cin % 4 == 0;
    l.b_bytes = (unsigned)((long long)a.N * a.ldb);
    const int per_cu = env.per_cu;
    int ngt = env.ngt;
    if (ngt <= 0) {
        // the largest group of tiles that still gives every workgroup a unit
        ngt = std::min(l.gn, kQ1MaxNgt);
        const long long slots = (long long)per_cu * num_cus();
        while (ngt > 1 && gm * ((l.gn + ngt - 1) / ngt) < slots) ngt = (ngt + 1) / 2;
    }
    l.ngt = std::min(ngt, l.gn);
    l.nug = (l.gn + l.ngt - 1) / l.ngt;
    if (gm * l.nug >= 0x7fffffffll) {
        set_error("k_i8q1: too many pixel blocks (%lld)", gm);
        return false;
    }
    l.units = (int)(gm * l.nug);
    if (per_cu >= 3) {
        if (env.nst == 2) return launch_nst<2, 3>(a, l, per_cu, s);
        return launch_nst<3, 3>(a, l, per_cu, s);
    }
    if (env.nst == 2) return launch_nst<2, 2>(a, l, per_cu, s);
    if (env.nst == 4) return launch_nst<4, 2>(a, l, per_cu, s);
    return launch_nst<3, 2>(a, l, per_cu, s);
}

}  // namespace acfun
