// model.cpp -- ACFUN0 model loader and device executor.
//
// Format and load-time fusion follow the reference's src/model.cpp:
//   header  "ACFUN0", u32 version, u32 inC, inH, inW, u32 num          (:3-16,117-122)
//   records 1 Conv KH,KW,Cout,s,p,w,b | 2 FC Cout,inDim,w,b | 3 ReLU |
//           4 MaxPool pool,s,p | 5 Softmax | 6 BN ch,mean,var,gamma,beta |
//           7 ConvG KH,KW,Cout,s,p,groups,w,b                           (:130-196)
//   fusion  Conv/FC/ConvG absorb a following ReLU and/or a following BN of
//           matching width (folded by fold_bn_into, :69-95); a ReLU whose
//           next layer is MaxPool is dropped; MaxPool absorbs a following
//           ReLU (:199-247).
// Differences, all stricter or additive:
//   * truncated files and out-of-range records are rejected (nullptr);
//   * version >= 2 files may also hold residual-network records (not in the
//     reference; its loader rejects unknown types at :193):
//       8  Add      u32 from, u32 act   cur = cur + out(from), ReLU if act
//       9  GlobalAvgPool               [H,W,C] -> [1,1,C], sequential sum / (H*W)
//       10 Input    u32 from            cur = out(from) (branch start)
//     `from` is a raw record index whose output the executor keeps alive
//     (0xFFFFFFFF = the model input); it must be the last record of its
//     fused group;
//   * inference runs batched on the device; folded weights live in HBM.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../../include/acfun/acfun.h"
#include "rt.hpp"

using namespace acfun;

namespace {

struct Layer {
    int type = 0;
    int p[8] = {0};
    int act = 0;
    int post_relu = 0;
    int raw_last = -1;  // last raw record this fused layer covers
    int from = -2;      // Add/Input: fused index of the referenced tensor (-1 = input)
    size_t wn = 0;      // weight element count
    float* w = nullptr;  // device
    float* b = nullptr;  // device
    // BN (unfused) parameters live in w: mean|var|gamma|beta
    // int8 variant of a conv: quantized weights and per-channel scales
    int8_t* wq = nullptr;
    float* ws = nullptr;
    I8Weights i8;        // wq prepared for the int8 GEMM once, at load
    // fp32 3x3/s1/p1 convs: the F(2,3) filter transform, made at the first
    // inference that routes the layer to Winograd (for plan U_plan) and reused
    float* U = nullptr;
    int U_plan = -1;
};

struct Raw {
    int type = 0;
    int p[8] = {0};
    const float* w = nullptr;
    const float* b = nullptr;
    int prevC = 0;
    size_t wn = 0;
    int outC = 0;
};

unsigned rd32(const unsigned char* p) {
    return (unsigned)p[0] | ((unsigned)p[1] << 8) | ((unsigned)p[2] << 16) | ((unsigned)p[3] << 24);
}

// fold_bn_into of src/model.cpp:69-95, same operation order (this file is
// compiled with -ffp-contract=off, and x86 host code has no implicit FMA).
void fold_bn(std::vector<float>& nw, std::vector<float>& nb, const float* w, const float* b,
             const Raw& bn, int Cout, size_t wn, int groups) {
    int ch = bn.p[0];
    const float* mean = bn.w;
    const float* var = bn.w + ch;
    const float* gamma = bn.w + 2 * ch;
    const float* beta = bn.w + 3 * ch;
    int Cout_per = (groups > 1) ? Cout / groups : Cout;
    size_t per_in = wn / (size_t)Cout;
    nw.assign(w, w + wn);
    nb.assign(Cout, 0.0f);
    for (int c = 0; c < Cout; ++c) {
        float scale = gamma[c] / sqrtf(var[c] + 1e-5f);
        float shift = beta[c] - mean[c] * scale;
        int gc = (groups > 1) ? c / Cout_per : 0;
        int oc = (groups > 1) ? c % Cout_per : c;
        for (size_t t = 0; t < per_in; ++t) {
            size_t off = (size_t)gc * (size_t)Cout_per * per_in + t * (size_t)Cout_per + oc;
            nw[off] *= scale;
        }
        nb[c] = (b ? b[c] : 0.0f) * scale + shift;
    }
}

bool upload(const float* host, size_t n, float** dev) {
    *dev = nullptr;
    if (!n) return true;
    if (!check(hipMalloc((void**)dev, n * sizeof(float)), "hipMalloc(model weights)")) return false;
    return check(hipMemcpy(*dev, host, n * sizeof(float), hipMemcpyHostToDevice), "H2D weights");
}

// Per-column symmetric int8 quantization on the host, same rule as
// acfun_quantize_weights (src/conv_int8.cpp:24-37).
void quantize_cols(const std::vector<float>& w, int K, int N, std::vector<float>& sc,
                   std::vector<int8_t>& q) {
    sc.assign(N, 1.0f);
    q.assign((size_t)K * N, 0);
    for (int j = 0; j < N; ++j) {
        float maxa = 0.0f;
        for (int k = 0; k < K; ++k) {
            float a = std::fabs(w[(size_t)k * N + j]);
            maxa = maxa < a ? a : maxa;
        }
        float s = maxa / 127.0f;
        if (s <= 0.0f) s = 1.0f;
        sc[j] = s;
        for (int k = 0; k < K; ++k) {
            int v = (int)std::lroundf(w[(size_t)k * N + j] / s);   // int first, as the reference
            if (v > 127) v = 127;
            else if (v < -128) v = -128;
            q[(size_t)k * N + j] = (int8_t)v;
        }
    }
}

// ACFUN_I8_CHAIN=0 turns the int8 models' s8 chain off (read once).
bool int8_chain_enabled() {
    static const int on = [] {
        const char* e = std::getenv("ACFUN_I8_CHAIN");
        return e && *e == '0' ? 0 : 1;
    }();
    return on != 0;
}

}  // namespace

struct AcfunModel {
    int inC = 0, inH = 0, inW = 0;
    int version = 0;
    int int8 = 0;
    int per_image = 0;   // int8 models: batched calls run image by image (load flag 2)
    std::vector<Layer> layers;
    int outSize = 0;
};

namespace {

void free_layers(AcfunModel* m) {
    for (auto& L : m->layers) {
        if (L.w) hipFree(L.w);
        if (L.b) hipFree(L.b);
        if (L.wq) hipFree(L.wq);
        if (L.ws) hipFree(L.ws);
        if (L.U) hipFree(L.U);
        i8_release(L.i8);
    }
    m->layers.clear();
}

AcfunModel* load_impl(const char* path, int flags) {
    if (!ensure_device()) return nullptr;
    FILE* f = fopen(path, "rb");
    if (!f) { set_error("acfun_model_load: cannot open %s", path); return nullptr; }
    fseek(f, 0, SEEK_END);
    long sz = ftell(f);
    fseek(f, 0, SEEK_SET);
    std::vector<unsigned char> blob(sz > 0 ? (size_t)sz : 1);
    if (sz < 0 || fread(blob.data(), 1, (size_t)sz, f) != (size_t)sz) { fclose(f); return nullptr; }
    fclose(f);
    if (sz < 6 + 4 * 5 || memcmp(blob.data(), "ACFUN0", 6) != 0) {
        set_error("acfun_model_load: bad magic or short header");
        return nullptr;
    }
    const unsigned char* B = blob.data();
    size_t o = 6;
    int version = (int)rd32(B + o); o += 4;
    int inC = (int)rd32(B + o); o += 4;
    int inH = (int)rd32(B + o); o += 4;
    int inW = (int)rd32(B + o); o += 4;
    int num = (int)rd32(B + o); o += 4;
    if (num < 0 || inC <= 0 || inH <= 0 || inW <= 0) { set_error("acfun_model_load: bad header"); return nullptr; }

    auto need = [&](size_t bytes) { return o + bytes <= (size_t)sz; };
    std::vector<Raw> raw(num);
    int prevC = inC;
    for (int i = 0; i < num; ++i) {
        Raw& L = raw[i];
        if (!need(4)) { set_error("acfun_model_load: truncated at record %d", i); return nullptr; }
        L.type = (int)rd32(B + o); o += 4;
        auto u32s = [&](int n) -> bool {
            if (!need(4 * (size_t)n)) return false;
            for (int k = 0; k < n; ++k) { L.p[k] = (int)rd32(B + o); o += 4; }
            return true;
        };
        auto floats = [&](size_t n, const float** dst) -> bool {
            if (n > ((size_t)sz) / 4 || !need(4 * n)) return false;
            *dst = (const float*)(B + o);
            o += 4 * n;
            return true;
        };
        bool ok = true;
        switch (L.type) {
            case 1:  // Conv
                ok = u32s(5) && L.p[0] > 0 && L.p[1] > 0 && L.p[2] > 0 && L.p[3] > 0;
                if (ok) {
                    L.prevC = prevC;
                    L.wn = (size_t)L.p[0] * L.p[1] * prevC * L.p[2];
                    ok = floats(L.wn, &L.w) && floats(L.p[2], &L.b);
                    prevC = L.p[2];
                }
                break;
            case 2:  // FC
                ok = u32s(2) && L.p[0] > 0 && L.p[1] > 0;
                if (ok) {
                    L.wn = (size_t)L.p[1] * L.p[0];
                    ok = floats(L.wn, &L.w) && floats(L.p[0], &L.b);
                    prevC = L.p[0];
                }
                break;
            case 7:  // ConvGrouped
                ok = u32s(6) && L.p[0] > 0 && L.p[1] > 0 && L.p[2] > 0 && L.p[3] > 0 && L.p[5] > 0;
                if (ok) {
                    L.prevC = prevC;
                    L.wn = (size_t)L.p[0] * L.p[1] * prevC * L.p[2] / L.p[5];
                    ok = floats(L.wn, &L.w) && floats(L.p[2], &L.b);
                    prevC = L.p[2];
                }
                break;
            case 3: case 5: break;
            case 4: ok = u32s(3) && L.p[0] > 0 && L.p[1] > 0; break;
            case 6:
                ok = u32s(1) && L.p[0] > 0;
                if (ok) { L.wn = (size_t)L.p[0] * 4; ok = floats(L.wn, &L.w); }
                break;
            case 8:
                ok = version >= 2 && u32s(2);
                break;
            case 9:
                ok = version >= 2;
                break;
            case 10:
                ok = version >= 2 && u32s(1);
                if (ok) {
                    int from = L.p[0];
                    if (from == -1) prevC = inC;
                    else if (from >= 0 && from < i) prevC = raw[from].outC;
                    else ok = false;
                }
                break;
            default: ok = false;
        }
        if (!ok) { set_error("acfun_model_load: bad or truncated record %d (type %d)", i, L.type); return nullptr; }
        L.outC = prevC;
    }

    AcfunModel* m = new AcfunModel();
    m->inC = inC; m->inH = inH; m->inW = inW; m->version = version;
    m->int8 = (flags & 1) ? 1 : 0;
    m->per_image = (flags & 2) ? 1 : 0;
    std::vector<char> consumed(num, 0);
    std::vector<int> raw2fused(num, -1);
    bool fail = false;
    for (int i = 0; i < num && !fail; ++i) {
        if (consumed[i]) continue;
        Raw& L = raw[i];
        Layer F;
        F.type = L.type;
        memcpy(F.p, L.p, sizeof(L.p));
        F.raw_last = i;
        if (L.type == 1 || L.type == 2 || L.type == 7) {  // :204-228
            int Cout = (L.type == 2) ? L.p[0] : L.p[2];
            int groups = (L.type == 7) ? L.p[5] : 0;
            std::vector<float> hw(L.w, L.w + L.wn), hb(L.b, L.b + Cout);
            int j = i + 1, reluIdx = -1;
            if (j < num && raw[j].type == 3) { reluIdx = j; j++; }
            if (j < num && raw[j].type == 6 && raw[j].p[0] == Cout) {
                fold_bn(hw, hb, L.w, L.b, raw[j], Cout, L.wn, groups);
                consumed[j] = 1;
                F.raw_last = j;
            }
            if (reluIdx >= 0) {
                if (j < num && raw[j].type == 4) { consumed[reluIdx] = 1; F.act = 0; }
                else { F.act = 1; consumed[reluIdx] = 1; }
                if (reluIdx > F.raw_last) F.raw_last = reluIdx;
            }
            F.wn = L.wn;
            if (!upload(hw.data(), hw.size(), &F.w) || !upload(hb.data(), hb.size(), &F.b)) fail = true;
            if (!fail && m->int8 && L.type == 1) {
                int K = (int)(L.wn / Cout);
                std::vector<float> sc;
                std::vector<int8_t> q;
                quantize_cols(hw, K, Cout, sc, q);
                if (!upload(sc.data(), sc.size(), &F.ws) ||
                    !check(hipMalloc((void**)&F.wq, q.size()), "hipMalloc(wq)") ||
                    !check(hipMemcpy(F.wq, q.data(), q.size(), hipMemcpyHostToDevice), "H2D wq") ||
                    !i8_prepare(F.wq, L.p[0] * L.p[1], K / (L.p[0] * L.p[1]), Cout, F.i8,
                                lib_stream()) ||
                    !check(hipStreamSynchronize(lib_stream()), "int8 weight prep"))
                    fail = true;
            }
        } else if (L.type == 3) {  // :229-233
            if (i + 1 < num && raw[i + 1].type == 4) { consumed[i] = 1; continue; }
        } else if (L.type == 6) {  // :234-235
            F.wn = L.wn;
            if (!upload(L.w, L.wn, &F.w)) fail = true;
        } else if (L.type == 4) {  // :236-242
            if (i + 1 < num && raw[i + 1].type == 3) {
                F.post_relu = 1;
                consumed[i + 1] = 1;
                F.raw_last = i + 1;
            }
        }
        m->layers.push_back(F);
        int fi = (int)m->layers.size() - 1;
        for (int r = i; r <= F.raw_last; ++r) raw2fused[r] = fi;
    }
    // Resolve Add / Input references to fused layers.
    for (auto& F : m->layers) {
        if (F.type != 8 && F.type != 10) continue;
        int from = F.p[0];
        if (from == -1) { F.from = -1; continue; }
        if (from < 0 || from >= num || raw2fused[from] < 0 ||
            m->layers[raw2fused[from]].raw_last != from) {
            set_error("acfun_model_load: record reference %d is not the end of a fused layer", from);
            fail = true;
            break;
        }
        F.from = raw2fused[from];
    }
    if (fail) {
        free_layers(m);
        delete m;
        return nullptr;
    }
    return m;
}

struct Dims { int H, W, C; };

// Runs the fused layers on N images resident in HBM.
int run_model(AcfunModel* m, int N, const float* din, float* dout, hipStream_t s) {
    struct TagReset { ~TagReset() { prof_tag(-1); } } tag_reset;   // launches after the layers are untagged
    const int L = (int)m->layers.size();
    // Shapes and last uses (liveness) of every fused output.
    std::vector<Dims> out(L);
    std::vector<int> last_use(L, -1);
    Dims cur{m->inH, m->inW, m->inC};
    int input_last = 0;
    for (int i = 0; i < L; ++i) {
        Layer& F = m->layers[i];
        Dims in = cur;
        if (F.type == 10) in = F.from < 0 ? Dims{m->inH, m->inW, m->inC} : out[F.from];
        Dims o = in;
        switch (F.type) {
            case 1: case 7: {
                int KH = F.p[0], KW = F.p[1], st = F.p[3], pd = F.p[4];
                o = Dims{(in.H + 2 * pd - KH) / st + 1, (in.W + 2 * pd - KW) / st + 1, F.p[2]};
                break;
            }
            case 2: o = Dims{1, 1, F.p[0]}; break;
            case 4: o = Dims{(in.H + 2 * F.p[2] - F.p[0]) / F.p[1] + 1, (in.W + 2 * F.p[2] - F.p[0]) / F.p[1] + 1, in.C}; break;
            case 9: o = Dims{1, 1, in.C}; break;
            default: break;
        }
        if (o.H <= 0 || o.W <= 0 || o.C <= 0) { set_error("model: empty output at layer %d", i); return 0; }
        if (F.type == 8) {
            Dims r = F.from < 0 ? Dims{m->inH, m->inW, m->inC} : out[F.from];
            if (r.H != in.H || r.W != in.W || r.C != in.C) { set_error("model: Add shape mismatch at layer %d", i); return 0; }
        }
        // consumers
        if (F.type == 10 || F.type == 8) {
            if (F.from < 0) input_last = i; else last_use[F.from] = i;
        }
        if (F.type != 10) {
            if (i == 0) input_last = std::max(input_last, 0);
            else last_use[i - 1] = std::max(last_use[i - 1], i);
        }
        out[i] = o;
        cur = o;
    }
    if (L) last_use[L - 1] = L;  // the result stays until copied out
    // Execution plan: the same arithmetic in fewer passes.
    //  * A ReLU layer that alone consumes a dense conv's output runs in the
    //    conv's epilogue with the layer's own rule (act 2: v < 0 -> 0).
    //  * An Add that alone consumes the output of a 1x1 conv runs in the conv's
    //    epilogue: v = (conv + bias) + residual, then its ReLU -- the same
    //    roundings as the separate Add.  fp32: the GEMM engine (any stride when
    //    Cin is a multiple of 64); int8 models: k_i8mm.
    //  * An Input layer aliases the tensor it names (no copy).
    // A fused or aliasing layer owns no buffer; its tensor is alias[i] (-1 =
    // the model input), kept alive as long as the alias is used.
    auto in_of = [&](int i) { return i > 0 ? out[i - 1] : Dims{m->inH, m->inW, m->inC}; };
    auto fusable_add = [&](const AcfunModel* mm, int i, int Cout, int Cin) {
        const Layer& F = mm->layers[i];
        if (F.type != 1 || F.p[0] != 1 || F.p[1] != 1 || Cout % 4 != 0) return false;
        if (mm->int8 && F.wq) return true;
        if (F.p[3] == 1 && F.p[4] == 0) return Cin % 4 == 0;
        return Cin % 64 == 0;
    };
    std::vector<int> alias(L, -2), act_of(L, -1), res_of(L, -3);
    for (int i = 0; i + 1 < L; ++i) {
        const Layer& F = m->layers[i];
        const Layer& G = m->layers[i + 1];
        if (F.type != 1 || F.act != 0 || last_use[i] != i + 1) continue;
        if (G.type == 3) {
            act_of[i] = 2;                           // the separate layer's ReLU rule
            alias[i + 1] = i;
            ++i;
        } else if (G.type == 8 && G.from != i && fusable_add(m, i, out[i].C, in_of(i).C)) {
            res_of[i] = G.from;
            act_of[i] = G.p[1] ? 2 : 0;              // k_add_relu's rule: v < 0 -> 0
            alias[i + 1] = i;
            ++i;
        }
    }
    for (int i = 0; i < L; ++i)
        if (m->layers[i].type == 10) alias[i] = m->layers[i].from;
    for (int i = L - 1; i >= 0; --i)
        if (alias[i] >= 0) last_use[alias[i]] = std::max(last_use[alias[i]], last_use[i]);
    // Execute.
    std::vector<float*> buf(L, nullptr);
    std::vector<Scratch> hold(L);
    // int8 models: per-layer slots for an output's max|v|.  An int8 conv folds
    // its output's max into its slot (in its own epilogue); an int8 conv whose
    // input is such a tensor quantizes with it and skips its absmax pass.
    Scratch amx;
    float* slot = nullptr;                           // L x kI8AmaxParts partial maxima
    std::vector<int> amax_of(L, -1);                 // slot holding layer i's output max
    if (m->int8 && L > 0) {
        amx = Scratch((size_t)L * kI8AmaxParts * sizeof(float), s);
        if (!amx.p) return 0;
        slot = amx.as<float>();
        if (!fill_f32(slot, (size_t)L * kI8AmaxParts, 0.0f, s)) return 0;
    }
    // int8 convs that read the same tensor with the same rounding rule (a
    // stage's projection shortcut and its first block's 1x1 conv) quantize it
    // once: the first writes a shared s8 tensor, the others reuse it.
    // root(t): the tensor an alias stands for (-1 = the model input).
    auto root = [&](int t) {
        while (t >= 0 && alias[t] != -2) t = alias[t];
        return t;
    };
    std::vector<int> qkey(L, -3), qlast(L, -1);      // per int8 conv: (root input, rule) key
    if (m->int8) {
        Dims c{m->inH, m->inW, m->inC};
        int xt = -1;
        for (int i = 0; i < L; ++i) {
            const Layer& F = m->layers[i];
            Dims in = c;
            if (F.type == 10) { xt = F.from; in = F.from < 0 ? Dims{m->inH, m->inW, m->inC} : out[F.from]; }
            if (F.type == 1 && F.wq && alias[i] == -2) {
                const bool wino = F.p[0] == 3 && F.p[1] == 3 && F.p[3] == 1 && F.p[4] == 1 &&
                                  in.H >= 3 && in.W >= 3 && in.C >= 4 && out[i].C >= 4;
                qkey[i] = 2 * (root(xt) + 1) + (wino ? 1 : 0);   // >= 0
            }
            c = out[i];
            xt = i;
        }
        for (int i = 0; i < L; ++i)
            if (qkey[i] >= 0)
                for (int j = i + 1; j < L; ++j)
                    if (qkey[j] == qkey[i]) qlast[i] = j;    // a later reader of the same quantization
    }
    struct SharedQ { int key = -3, last = -1; Scratch mem; I8Quant q; };
    std::vector<SharedQ> sq;
    // The int8 chain: an int8 conv whose output has one reader, an int8 conv
    // taking it as its input, writes it as s8 with its scale (I8Out: the
    // values and scale the reader's quantizer would form from the fp32 tensor,
    // bit for bit) and the reader multiplies that s8 tensor directly; neither
    // the fp32 tensor nor the reader's absmax/quantize passes exist.  Tensors
    // an Add, a projection shortcut or the model output also read stay fp32.
    // ACFUN_I8_CHAIN=0 keeps every tensor fp32 (the same results).
    std::vector<int> chain_to(L, -1), chain_rule(L, 0);
    if (m->int8 && int8_chain_enabled()) {
        std::vector<int> nread(L + 1, 0), reader(L + 1, -1), rin(L, -2);   // index: root + 1
        auto note = [&](int r, int k) { ++nread[r + 1]; reader[r + 1] = k; };
        int xt = -1;
        for (int k = 0; k < L; ++k) {
            const Layer& F = m->layers[k];
            if (alias[k] == -2) {                    // executes (Input layers always alias)
                rin[k] = root(xt);
                note(rin[k], k);
                if (F.type == 8) note(root(F.from), k);
                if (res_of[k] != -3) note(root(res_of[k]), k);
            }
            xt = k;
        }
        if (L > 0) note(root(L - 1), L);             // the model output
        for (int i = 0; i < L; ++i) {
            const Layer& F = m->layers[i];
            if (!(F.type == 1 && F.wq && alias[i] == -2) || nread[i + 1] != 1) continue;
            const int j = reader[i + 1];
            if (j >= L || rin[j] != i) continue;
            const Layer& G = m->layers[j];
            if (!(G.type == 1 && G.wq)) continue;
            const Dims& d = out[i];                  // the reader's input
            const bool wino = G.p[0] == 3 && G.p[1] == 3 && G.p[3] == 1 && G.p[4] == 1 &&
                              d.H >= 3 && d.W >= 3 && d.C >= 4 && out[j].C >= 4;
            chain_to[i] = j;
            chain_rule[i] = wino ? 1 : 0;
        }
    }
    struct S8T { Scratch q, scale; };
    std::vector<S8T> s8t(L);                        // chained s8 tensors by producer
    auto tensor_of = [&](int idx) -> const float* { return idx < 0 ? din : buf[idx]; };
    cur = Dims{m->inH, m->inW, m->inC};
    const float* x = din;
    int xi = -1;
    const bool prof = prof_on();
    for (int i = 0; i < L; ++i) {
        Layer& F = m->layers[i];
        Dims in = cur;
        if (F.type == 10) { x = tensor_of(F.from); xi = F.from; in = F.from < 0 ? Dims{m->inH, m->inW, m->inC} : out[F.from]; }
        Dims o = out[i];
        size_t cap = (size_t)N * o.H * o.W * o.C;
        if (prof) {
            // i type N H W C -> OH OW OC, kernel, stride, pad, groups, int8, fused-into, act, residual
            char rec[192];
            const bool conv = F.type == 1 || F.type == 7;
            snprintf(rec, sizeof(rec), "%d\t%d\t%d\t%d\t%d\t%d\t%d\t%d\t%d\t%d\t%d\t%d\t%d\t%d\t%d\t%d\t%d\t%d",
                     i, F.type, N, in.H, in.W, in.C, o.H, o.W, o.C, conv ? F.p[0] : 0,
                     conv ? F.p[1] : 0, conv ? F.p[3] : 0, conv ? F.p[4] : 0,
                     F.type == 7 ? F.p[5] : 1, (m->int8 && F.type == 1 && F.wq) ? 1 : 0,
                     alias[i] != -2 && F.type != 10 ? alias[i] : -2,
                     act_of[i] >= 0 ? act_of[i] : F.act, res_of[i] != -3 ? 1 : 0);
            prof_layer(rec);
            prof_tag(i);
        }
        if (alias[i] != -2) {                        // fused into the previous layer, or an Input
            buf[i] = const_cast<float*>(tensor_of(alias[i]));
            if (alias[i] >= 0) amax_of[i] = amax_of[alias[i]];
            for (int j = 0; j < i; ++j)
                if (buf[j] && last_use[j] == i && hold[j].p) { hold[j] = Scratch(); buf[j] = nullptr; }
            cur = o;
            x = buf[i];
            xi = i;
            continue;
        }
        bool inplace = (F.type == 3 || F.type == 5 || F.type == 6 || F.type == 10);
        float* y;
        if (chain_to[i] >= 0) {
            y = nullptr;                             // the output exists only as s8 (s8t[i])
        } else if (inplace && F.type != 10 && xi >= 0 && last_use[xi] == i && hold[xi].p) {
            // take over the input buffer
            y = buf[xi];
            hold[i] = std::move(hold[xi]);
            buf[xi] = nullptr;
        } else {
            hold[i] = Scratch(cap * sizeof(float), s);
            if (!hold[i].p) return 0;
            y = hold[i].as<float>();
            if (inplace && F.type != 10 &&
                !check(hipMemcpyAsync(y, x, cap * sizeof(float), hipMemcpyDeviceToDevice, s), "D2D"))
                return 0;
        }
        buf[i] = y;
        bool ok = true;
        switch (F.type) {
            case 1: case 7: {
                int groups = F.type == 7 ? F.p[5] : 1;
                const int act = act_of[i] >= 0 ? act_of[i] : F.act;
                const long long M = (long long)N * in.H * in.W;
                const float* res = res_of[i] != -3 ? tensor_of(res_of[i]) : nullptr;
                ConvShape g{N, in.H, in.W, in.C, F.p[0], F.p[1], F.p[3], F.p[4], o.H, o.W};
                if (m->int8 && F.type == 1 && F.wq) {
                    const float* ain =
                        xi >= 0 && amax_of[xi] >= 0 ? slot + (size_t)amax_of[xi] * kI8AmaxParts : nullptr;
                    I8Quant* shq = nullptr;
                    for (auto& e : sq)
                        if (e.key == qkey[i]) shq = &e.q;
                    if (!shq && qlast[i] > i) {              // the first of several readers
                        sq.emplace_back();
                        SharedQ& e = sq.back();
                        e.key = qkey[i];
                        e.last = qlast[i];
                        for (int j = i + 1; j < L; ++j)
                            if (qkey[j] == qkey[i]) e.last = j;
                        const long long pix = (long long)N * in.H * in.W;
                        e.mem = Scratch(i8_quant_bytes(pix, in.C), s);
                        if (!e.mem.p) return 0;
                        e.q.q = e.mem.as<int8_t>();
                        e.q.scal = (float*)(e.mem.as<char>() + (i8_quant_bytes(pix, in.C) - 8 * sizeof(float)));
                        shq = &e.q;
                    }
                    I8Out qout;
                    if (chain_to[i] >= 0) {
                        qout.ldo = (o.C + 15) / 16 * 16;
                        qout.rule = chain_rule[i];
                        qout.recompute = false;
                        s8t[i].q = Scratch((size_t)N * o.H * o.W * qout.ldo, s);
                        s8t[i].scale = Scratch(sizeof(float), s);
                        if (!s8t[i].q.p || !s8t[i].scale.p) return 0;
                        qout.q = s8t[i].q.as<int8_t>();
                        qout.s_out = s8t[i].scale.as<float>();
                    }
                    const I8Out* qo = chain_to[i] >= 0 ? &qout : nullptr;
                    const int rx = root(xi);
                    if (rx >= 0 && s8t[rx].q.p) {            // an s8 input from the chain
                        ok = conv2d_int8_s8in_dev(s8t[rx].q.as<int8_t>(), s8t[rx].scale.as<float>(), g,
                                                  F.i8, F.ws, F.b, o.C, y, act, s, res,
                                                  slot + (size_t)i * kI8AmaxParts, qo);
                        s8t[rx] = S8T();                     // its only reader
                    } else {
                        ok = conv2d_int8_dev(x, g, F.wq, F.ws, F.b, o.C, y, act, s, &F.i8, res,
                                             slot + (size_t)i * kI8AmaxParts, ain, shq, qo);
                    }
                    amax_of[i] = qo ? -1 : i;
                    for (auto it = sq.begin(); it != sq.end();)
                        it = it->last <= i ? sq.erase(it) : std::next(it);
                } else if (res && F.p[3] == 1 && F.p[4] == 0 && M < (1ll << 31) &&
                           gemm32_ok((int)M, o.C, in.C, x, in.C, F.w, o.C)) {
                    ok = gemm32_f32((int)M, o.C, in.C, x, in.C, F.w, o.C, y, o.C, F.b, act, s, res,
                                    o.C);
                } else if (res && conv32_ok(g, o.C, x, F.w)) {
                    ok = conv32_f32(g, x, F.w, F.b, o.C, y, act, s, res, o.C);
                } else if (res) {
                    set_error("model: residual fusion precondition failed at layer %d", i);
                    return 0;
                } else {
                    // A Winograd-routed layer keeps its filter transform (the
                    // reference rebuilds it per call, src/winograd_avx512.cpp:195-206;
                    // the weights of a loaded model do not change).
                    const float* U = nullptr;
                    if (groups <= 1 && F.p[0] == 3 && F.p[1] == 3 && F.p[3] == 1 && F.p[4] == 1 &&
                        in.H >= 3 && in.W >= 3 && in.C >= 4 && o.C >= 4) {
                        const int plan = wino23_plan(N, in.H, in.W, in.C, o.C, x);
                        if (plan >= 0 && F.U_plan != plan) {
                            if (F.U) { (void)hipStreamSynchronize(s); hipFree(F.U); F.U = nullptr; }
                            F.U_plan = -1;
                            if (check(hipMalloc((void**)&F.U, wino23_filter_bytes(in.C, o.C)),
                                      "hipMalloc(Winograd filter)") &&
                                wino23_filter(F.w, in.C, o.C, plan, F.U, s))
                                F.U_plan = plan;
                            else
                                return 0;
                        }
                        if (plan >= 0) U = F.U;
                    }
                    ok = conv2d_route_f32(x, N, in.H, in.W, in.C, F.w, F.b, F.p[0], F.p[1], o.C,
                                          F.p[3], F.p[4], groups > 1 ? groups : 1, y, act, s, U);
                }
                break;
            }
            case 2: {
                int inDim = in.H * in.W * in.C;
                if ((size_t)inDim * F.p[0] != F.wn) {
                    set_error("model: FC input %d does not match weights", inDim);
                    return 0;
                }
                ok = gemm_f32(N, o.C, inDim, x, inDim, F.w, o.C, y, o.C, F.b, F.act, s);
                break;
            }
            case 3: ok = relu_f32(y, cap, 0, s); break;
            case 4: ok = maxpool_f32(x, N, in.H, in.W, in.C, F.p[0], F.p[1], F.p[2], y, F.post_relu, s); break;
            case 5: ok = softmax_f32(y, N, (int)(cap / N), y, s); break;
            case 6: {
                int ch = F.p[0];
                size_t per = cap / N;
                const float* P = F.w;
                if (per % ch == 0) ok = batchnorm_f32(y, (int)cap, ch, P, P + ch, P + 2 * ch, P + 3 * ch, 1e-5f, s);
                else
                    for (int n = 0; n < N && ok; ++n)
                        ok = batchnorm_f32(y + n * per, (int)per, ch, P, P + ch, P + 2 * ch, P + 3 * ch, 1e-5f, s);
                break;
            }
            case 8: ok = add_relu_f32(x, tensor_of(F.from), y, cap, F.p[1], s); break;
            case 9: ok = gap_f32(x, N, in.H * in.W, in.C, y, s); break;
            case 10: ok = check(hipMemcpyAsync(y, x, cap * sizeof(float), hipMemcpyDeviceToDevice, s), "D2D"); break;
        }
        if (!ok) return 0;
        // release inputs whose last consumer was this layer
        for (int j = 0; j < i; ++j)
            if (buf[j] && last_use[j] == i) {
                hold[j] = Scratch();
                buf[j] = nullptr;
            }
        cur = o;
        x = y;
        xi = i;
    }
    prof_tag(-1);
    size_t per = (size_t)cur.H * cur.W * cur.C;
    if (L == 0) per = (size_t)m->inH * m->inW * m->inC;
    if (!check(hipMemcpyAsync(dout, x, (size_t)N * per * sizeof(float), hipMemcpyDeviceToDevice, s), "D2D out"))
        return 0;
    m->outSize = (int)per;
    return (int)per;
}

}  // namespace

extern "C" {

AcfunModel* acfun_model_load(const char* path) { return load_impl(path, 0); }

AcfunModel* acfun_model_load_ex(const char* path, int flags) { return load_impl(path, flags); }

void acfun_model_destroy(AcfunModel* m) {
    if (!m) return;
    free_layers(m);
    delete m;
}

int acfun_model_output_size(AcfunModel* m) { return m ? m->outSize : 0; }

void acfun_model_input_dims(AcfunModel* m, int* Cin, int* Hin, int* Win) {
    if (!m) return;
    if (Cin) *Cin = m->inC;
    if (Hin) *Hin = m->inH;
    if (Win) *Win = m->inW;
}

}  // extern "C"

// A batch through the executor.  An int8 model loaded with flag 2 runs its
// images one at a time, so every int8 activation scale is the image's own, as
// the reference's acfun_model_infer computes it (one image per call,
// src/model.cpp:274-349); otherwise the batch runs at once.
static int run_batch(AcfunModel* m, int N, const float* in, float* out, hipStream_t s) {
    if (!(m->int8 && m->per_image) || N == 1) return run_model(m, N, in, out, s);
    const size_t in1 = (size_t)m->inC * m->inH * m->inW;
    int per = run_model(m, 1, in, out, s);
    for (int i = 1; i < N && per > 0; ++i)
        if (run_model(m, 1, in + i * in1, out + (size_t)i * per, s) != per) return 0;
    return per;
}

extern "C" {

int acfun_dev_model_infer_batch(AcfunModel* m, int N, const float* input, float* output,
                                void* stream) {
    if (!m || N <= 0 || !ensure_device()) return 0;
    return run_batch(m, N, input, output, resolve(stream));
}

int acfun_model_infer_batch(AcfunModel* m, int N, const float* input, float* output) {
    if (!m || N <= 0 || !ensure_device()) return 0;
    hipStream_t s = lib_stream();
    // The output size is known only after shape inference; run shape-only
    // pass through run_model on the device result buffer sized generously.
    size_t in_n = (size_t)N * m->inC * m->inH * m->inW;
    HostCall hc(s);
    const float* din = (const float*)hc.in(input, in_n * sizeof(float));
    if (hc.failed()) return 0;
    // Upper bound of the per-image output: the largest tensor in the graph.
    size_t maxper = (size_t)m->inC * m->inH * m->inW;
    {
        int H = m->inH, W = m->inW, C = m->inC;
        std::vector<Dims> outs;
        for (auto& F : m->layers) {
            if (F.type == 10) {
                Dims d = F.from < 0 ? Dims{m->inH, m->inW, m->inC} : outs[F.from];
                H = d.H; W = d.W; C = d.C;
            }
            switch (F.type) {
                case 1: case 7: H = (H + 2 * F.p[4] - F.p[0]) / F.p[3] + 1; W = (W + 2 * F.p[4] - F.p[1]) / F.p[3] + 1; C = F.p[2]; break;
                case 2: H = W = 1; C = F.p[0]; break;
                case 4: H = (H + 2 * F.p[2] - F.p[0]) / F.p[1] + 1; W = (W + 2 * F.p[2] - F.p[0]) / F.p[1] + 1; break;
                case 9: H = W = 1; break;
                default: break;
            }
            outs.push_back(Dims{H, W, C});
            if (H > 0 && W > 0 && C > 0 && (size_t)H * W * C > maxper) maxper = (size_t)H * W * C;
        }
    }
    Scratch dres((size_t)N * maxper * sizeof(float), s);
    if (!dres.p) return 0;
    int per = run_batch(m, N, din, dres.as<float>(), s);
    if (per > 0) {
        void* dst = output;
        if (is_device_ptr(output)) {
            if (!check(hipMemcpyAsync(dst, dres.p, (size_t)N * per * sizeof(float), hipMemcpyDeviceToDevice, s), "D2D")) per = 0;
        } else if (!check(hipMemcpyAsync(dst, dres.p, (size_t)N * per * sizeof(float), hipMemcpyDeviceToHost, s), "D2H")) {
            per = 0;
        }
    }
    if (!check(hipStreamSynchronize(s), "sync")) return 0;
    return per;
}

int acfun_model_infer(AcfunModel* m, const float* input, float* output) {
    return acfun_model_infer_batch(m, 1, input, output);
}

}  // extern "C"
