"""Oracle ACFUN0 executor -- TEST INFRASTRUCTURE ONLY.

Restates the reference's loader and executor (src/model.cpp:106-349): the
record parser (:130-196), the load-time fusion (:199-247: BN folded by
fold_bn_into, ReLU fused, a ReLU before MaxPool dropped, MaxPool absorbing a
following ReLU) and the layer loop (:274-349), run on the oracle operators.
Version-2 residual records (Add/GlobalAvgPool/Input) follow the definitions
the library documents for them.  Batched: for fp32 models image n of a batch
equals a batch-1 run on image n (softmax per image, as the reference runs
rows=1 per image).  In int8 mode every conv is acfun_conv2d_int8 on the whole
batch, whose activation scale is max|x| over all images (src/conv_int8.cpp:75-81),
so an image's int8 result depends on its batch.
"""
import struct

import numpy as np

from . import conv2d_dw, conv2d_f64, conv2d_grouped, conv2d_int8, fold_bn, lib, maxpool, \
    quantize_weights


def parse(blob):
    """Returns (version, inC, inH, inW, raw records) or raises ValueError."""
    if len(blob) < 26 or blob[:6] != b"ACFUN0":
        raise ValueError("bad magic")
    version, inC, inH, inW, num = struct.unpack_from("<5I", blob, 6)
    o = 26
    raw = []
    prevC = inC

    def u32(n):
        nonlocal o
        v = struct.unpack_from(f"<{n}I", blob, o)
        o += 4 * n
        return list(v)

    def f32(n):
        nonlocal o
        if o + 4 * n > len(blob):
            raise ValueError("truncated")
        a = np.frombuffer(blob, "<f4", n, o).astype(np.float32)
        o += 4 * n
        return a

    for i in range(num):
        (t,) = u32(1)
        r = {"type": t, "p": [], "w": None, "b": None}
        if t == 1:
            r["p"] = u32(5)
            KH, KW, Cout = r["p"][:3]
            r["prevC"] = prevC
            r["w"] = f32(KH * KW * prevC * Cout)
            r["b"] = f32(Cout)
            prevC = Cout
        elif t == 2:
            r["p"] = u32(2)
            Cout, inDim = r["p"]
            r["w"] = f32(inDim * Cout)
            r["b"] = f32(Cout)
            prevC = Cout
        elif t == 7:
            r["p"] = u32(6)
            KH, KW, Cout, _, _, g = r["p"]
            r["prevC"] = prevC
            r["w"] = f32(KH * KW * prevC * Cout // g)
            r["b"] = f32(Cout)
            prevC = Cout
        elif t in (3, 5):
            pass
        elif t == 4:
            r["p"] = u32(3)
        elif t == 6:
            r["p"] = u32(1)
            r["w"] = f32(4 * r["p"][0])
        elif t == 8 and version >= 2:
            r["p"] = u32(2)
            r["p"][0] = r["p"][0] - (1 << 32) if r["p"][0] >= (1 << 31) else r["p"][0]
        elif t == 9 and version >= 2:
            pass
        elif t == 10 and version >= 2:
            r["p"] = u32(1)
            f = r["p"][0] - (1 << 32) if r["p"][0] >= (1 << 31) else r["p"][0]
            r["p"][0] = f
            prevC = inC if f == -1 else raw[f]["outC"]
        else:
            raise ValueError(f"unknown record type {t}")
        r["outC"] = prevC
        raw.append(r)
    return version, inC, inH, inW, raw


def fuse(raw):
    """The fusion pass of src/model.cpp:199-247; returns fused layer dicts."""
    num = len(raw)
    consumed = [False] * num
    out = []
    for i, L in enumerate(raw):
        if consumed[i]:
            continue
        t = L["type"]
        F = {"type": t, "p": list(L["p"]), "w": L["w"], "b": L["b"], "act": 0, "post_relu": 0,
             "last": i}
        if t in (1, 2, 7):
            Cout = L["p"][0] if t == 2 else L["p"][2]
            groups = L["p"][5] if t == 7 else 0
            j = i + 1
            relu_idx = -1
            if j < num and raw[j]["type"] == 3:
                relu_idx = j
                j += 1
            if j < num and raw[j]["type"] == 6 and raw[j]["p"][0] == Cout:
                bn = raw[j]["w"]
                ch = Cout
                F["w"], F["b"] = fold_bn(L["w"], L["b"], Cout, groups, bn[:ch].copy(),
                                         bn[ch:2 * ch].copy(), bn[2 * ch:3 * ch].copy(),
                                         bn[3 * ch:].copy())
                consumed[j] = True
                F["last"] = j
            if relu_idx >= 0:
                consumed[relu_idx] = True
                F["act"] = 0 if (j < num and raw[j]["type"] == 4) else 1
                F["last"] = max(F["last"], relu_idx)
        elif t == 3:
            if i + 1 < num and raw[i + 1]["type"] == 4:
                consumed[i] = True
                continue
        elif t == 4:
            if i + 1 < num and raw[i + 1]["type"] == 3:
                F["post_relu"] = 1
                consumed[i + 1] = True
                F["last"] = i + 1
        out.append(F)
    return out


def _conv_fp32(x, F, groups):
    KH, KW, Cout, s, p = F["p"][:5]
    N, H, W, Cin = x.shape
    w = np.ascontiguousarray(F["w"], np.float32)
    b = np.ascontiguousarray(F["b"], np.float32)
    act = F["act"]
    if groups > 1:
        if groups == Cin == Cout:
            return conv2d_dw(x, w, b, KH, KW, s, p, act)
        if Cin // groups <= 64 and Cout // groups <= 128:
            return conv2d_grouped(x, w, b, KH, KW, Cout, s, p, groups, act)
    return conv2d_f64(x, w, b, KH, KW, Cout, s, p, groups, act).astype(np.float32)


def run(blob, x, int8=False):
    """Executes a model file on x [N,H,W,C] float32; returns [N, outSize]."""
    version, inC, inH, inW, raw = parse(blob)
    layers = fuse(raw)
    # Add/Input name a raw record; it resolves to the fused layer ending there.
    covered = {F["last"]: fi for fi, F in enumerate(layers)}
    x = np.ascontiguousarray(x, np.float32)
    N = x.shape[0]
    outs = []
    cur = x
    for fi, F in enumerate(layers):
        t = F["type"]
        if t in (1, 7):
            groups = F["p"][5] if t == 7 else 1
            if int8 and t == 1:
                KH, KW, Cout, s, p = F["p"][:5]
                K = KH * KW * cur.shape[3]
                sc, q = quantize_weights(np.asarray(F["w"], np.float32).reshape(K, Cout))
                y = conv2d_int8(cur, q, sc, np.ascontiguousarray(F["b"], np.float32), KH, KW,
                                Cout, s, p, F["act"])
            else:
                y = _conv_fp32(cur, F, groups)
        elif t == 2:
            Cout = F["p"][0]
            flat = cur.reshape(N, -1).astype(np.float64)
            w = np.asarray(F["w"], np.float64).reshape(flat.shape[1], Cout)
            y = (flat @ w + F["b"].astype(np.float64))
            if F["act"]:
                y = np.maximum(y, 0)
            y = y.astype(np.float32).reshape(N, 1, 1, Cout)
        elif t == 3:
            y = cur.copy()
            lib().oracle_relu(y.reshape(-1), y.size)
        elif t == 4:
            y = maxpool(cur, F["p"][0], F["p"][1], F["p"][2], F["post_relu"])
        elif t == 5:
            y = np.empty_like(cur)
            per = cur[0].size
            for n in range(N):
                src = np.ascontiguousarray(cur[n]).reshape(-1)
                dst = np.empty(per, np.float32)
                lib().oracle_softmax(src, 1, per, dst)
                y[n] = dst.reshape(cur.shape[1:])
        elif t == 6:
            ch = F["p"][0]
            P = F["w"]
            y = cur.copy()
            for n in range(N):
                v = np.ascontiguousarray(y[n]).reshape(-1)
                _bn(v, ch, P)
                y[n] = v.reshape(cur.shape[1:])
        elif t == 8:
            ref = x if F["p"][0] == -1 else outs[covered[F["p"][0]]]
            y = (cur + ref).astype(np.float32)
            if F["p"][1]:
                y[y < 0] = 0.0
        elif t == 9:
            Nn, H, W, C = cur.shape
            flat = cur.reshape(Nn, H * W, C)
            s = np.zeros((Nn, C), np.float32)
            for k in range(H * W):
                s += flat[:, k, :]
            y = (s / np.float32(H * W)).astype(np.float32).reshape(Nn, 1, 1, C)
        elif t == 10:
            y = x if F["p"][0] == -1 else outs[covered[F["p"][0]]]
        else:
            raise ValueError(t)
        outs.append(y)
        cur = y
    return cur.reshape(N, -1)


def _bn(v, ch, P):
    mean = np.ascontiguousarray(P[:ch], np.float32)
    var = np.ascontiguousarray(P[ch:2 * ch], np.float32)
    gamma = np.ascontiguousarray(P[2 * ch:3 * ch], np.float32)
    beta = np.ascontiguousarray(P[3 * ch:], np.float32)
    lib().oracle_batchnorm(v, v.size, ch, mean, var, gamma.ctypes.data, beta.ctypes.data, 1e-5)


# ---- the same graph on the compiled reference's own per-op entry points ----

def prepare_reference(ref, blob, int8=False):
    """Parses and fuses a model (as run() does) and, in int8 mode, quantizes
    every dense conv's folded weights once with the reference's own
    acfun_quantize_weights -- the load-time part of run_reference()."""
    import ctypes as C
    version, inC, inH, inW, raw = parse(blob)
    layers = fuse(raw)
    covered = {F["last"]: fi for fi, F in enumerate(layers)}
    P = lambda a: C.c_void_p(a.ctypes.data)
    prev_c = inC
    for F in layers:
        F["w"] = None if F["w"] is None else np.ascontiguousarray(F["w"], np.float32)
        F["b"] = None if F["b"] is None else np.ascontiguousarray(F["b"], np.float32)
        t = F["type"]
        if t == 10:
            prev_c = inC if F["p"][0] == -1 else layers[covered[F["p"][0]]]["outC"]
        if t in (1, 7):
            F["inC"] = prev_c
            prev_c = F["p"][2]
        elif t == 2:
            prev_c = F["p"][0]
        F["outC"] = prev_c
        if int8 and t == 1:
            KH, KW, Cout = F["p"][:3]
            K = KH * KW * F["inC"]
            F["ws"] = np.empty(Cout, np.float32)
            F["wq"] = np.empty((K, Cout), np.int8)
            ref.acfun_quantize_weights(P(F["w"]), K, Cout, P(F["ws"]), P(F["wq"]))
    return {"layers": layers, "covered": covered, "int8": int8}


def run_reference(ref, prep, x):
    """Executes a prepared model on the compiled reference: every conv, FC,
    pool, ReLU, BN and softmax is one call of the reference's API on the whole
    batch (acfun_conv2d(_relu)/_g, acfun_conv2d_int8, acfun_maxpool(_relu),
    acfun_fc, acfun_relu, acfun_batchnorm, acfun_softmax per image); the
    version-2 Add and GlobalAvgPool records, which the reference has no call
    for, are numpy float32 in the order run() gives them.  This is the CPU
    baseline of a version-2 model and is pinned to run() by the tests."""
    import ctypes as C
    P = lambda a: C.c_void_p(a.ctypes.data)
    layers, covered = prep["layers"], prep["covered"]
    x = np.ascontiguousarray(x, np.float32)
    N = x.shape[0]
    outs = []
    cur = x
    for F in layers:
        t = F["type"]
        if t in (1, 7):
            KH, KW, Cout, s, p = F["p"][:5]
            n, h, w_, ci = cur.shape
            OH, OW = (h + 2 * p - KH) // s + 1, (w_ + 2 * p - KW) // s + 1
            y = np.empty((n, OH, OW, Cout), np.float32)
            if t == 7:
                ref.acfun_conv2d_g(P(cur), n, h, w_, ci, P(F["w"]), P(F["b"]), KH, KW, Cout, s, p,
                                   F["p"][5], P(y), F["act"])
            elif prep["int8"]:
                ref.acfun_conv2d_int8(P(cur), n, h, w_, ci, P(F["wq"]), P(F["ws"]), P(F["b"]),
                                      KH, KW, Cout, s, p, C.c_float(0.0), P(y), F["act"])
            else:
                fn = ref.acfun_conv2d_relu if F["act"] else ref.acfun_conv2d
                fn(P(cur), n, h, w_, ci, P(F["w"]), P(F["b"]), KH, KW, Cout, s, p, P(y))
        elif t == 2:
            Cout = F["p"][0]
            flat = np.ascontiguousarray(cur.reshape(N, -1))
            y = np.empty((N, Cout), np.float32)
            fn = ref.acfun_fc_relu if F["act"] else ref.acfun_fc
            fn(P(flat), N, flat.shape[1], P(F["w"]), P(F["b"]), Cout, P(y))
            y = y.reshape(N, 1, 1, Cout)
        elif t == 3:
            y = cur.copy()
            ref.acfun_relu(P(y), y.size)
        elif t == 4:
            pool, s, p = F["p"][:3]
            n, h, w_, ci = cur.shape
            OH, OW = (h + 2 * p - pool) // s + 1, (w_ + 2 * p - pool) // s + 1
            y = np.empty((n, OH, OW, ci), np.float32)
            fn = ref.acfun_maxpool_relu if F["post_relu"] else ref.acfun_maxpool
            fn(P(cur), n, h, w_, ci, pool, s, p, P(y))
        elif t == 5:
            per = cur[0].size
            y = np.empty_like(cur)
            flat = np.ascontiguousarray(cur.reshape(N, per))
            ref.acfun_softmax(P(flat), N, per, P(y))
        elif t == 6:
            ch = F["p"][0]
            mean, var, gamma, beta = (np.array(F["w"][k * ch:(k + 1) * ch], np.float32)
                                      for k in range(4))
            y = cur.copy()
            ref.acfun_batchnorm(P(y), y.size, ch, P(mean), P(var), P(gamma), P(beta),
                                C.c_float(1e-5))
        elif t == 8:
            other = x if F["p"][0] == -1 else outs[covered[F["p"][0]]]
            y = np.add(cur, other, dtype=np.float32)
            if F["p"][1]:
                np.maximum(y, 0.0, out=y, where=y < 0)
        elif t == 9:
            n, h, w_, ci = cur.shape
            flat = cur.reshape(n, h * w_, ci)
            sm = np.zeros((n, ci), np.float32)
            for k in range(h * w_):
                sm += flat[:, k, :]
            y = (sm / np.float32(h * w_)).astype(np.float32).reshape(n, 1, 1, ci)
        elif t == 10:
            y = x if F["p"][0] == -1 else outs[covered[F["p"][0]]]
        else:
            raise ValueError(t)
        outs.append(y)
        cur = np.ascontiguousarray(y)
    return cur.reshape(N, -1)
