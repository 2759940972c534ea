"""ACFUN0 model files: writer, reader and a ResNet-50-style generator.

The layout is the reference's (src/model.cpp:3-16 and the writer
tools/gen_model.py of the reference): little-endian "ACFUN0", u32 version,
u32 inC, inH, inW, u32 record count, then per record a u32 type and its
fields.  Types 1-7 are the reference's; 8 (Add), 9 (GlobalAvgPool) and
10 (Input) are this library's residual-network extension, valid only in
version >= 2 files (the reference loader rejects them).

Records are tuples:
  ("conv", KH, KW, Cout, stride, pad, w[KH*KW*Cin*Cout], b[Cout])
  ("fc", Cout, inDim, w[inDim*Cout], b[Cout])
  ("relu",) ("softmax",) ("gap",)
  ("maxpool", pool, stride, pad)
  ("bn", ch, mean, var, gamma, beta)
  ("convg", KH, KW, Cout, stride, pad, groups, w, b)
  ("add", from_record, act)     from_record = -1 means the model input
  ("input", from_record)
"""
import struct

import numpy as np

TYPES = {"conv": 1, "fc": 2, "relu": 3, "maxpool": 4, "softmax": 5, "bn": 6, "convg": 7,
         "add": 8, "gap": 9, "input": 10}
NAMES = {v: k for k, v in TYPES.items()}


def _f32(a):
    return np.ascontiguousarray(a, dtype="<f4").tobytes()


def _u32(*vals):
    return b"".join(struct.pack("<I", v & 0xFFFFFFFF) for v in vals)


def encode(inC, inH, inW, records, version=1):
    out = [b"ACFUN0", _u32(version, inC, inH, inW, len(records))]
    for r in records:
        kind = r[0]
        out.append(_u32(TYPES[kind]))
        if kind == "conv":
            _, KH, KW, Cout, s, p, w, b = r
            out += [_u32(KH, KW, Cout, s, p), _f32(w), _f32(b)]
        elif kind == "convg":
            _, KH, KW, Cout, s, p, g, w, b = r
            out += [_u32(KH, KW, Cout, s, p, g), _f32(w), _f32(b)]
        elif kind == "fc":
            _, Cout, inDim, w, b = r
            out += [_u32(Cout, inDim), _f32(w), _f32(b)]
        elif kind == "maxpool":
            out.append(_u32(*r[1:4]))
        elif kind == "bn":
            _, ch, mean, var, gamma, beta = r
            out += [_u32(ch), _f32(mean), _f32(var), _f32(gamma), _f32(beta)]
        elif kind == "add":
            out.append(_u32(r[1], r[2]))
        elif kind == "input":
            out.append(_u32(r[1]))
        elif kind in ("relu", "softmax", "gap"):
            pass
        else:
            raise ValueError(kind)
    return b"".join(out)


def write(path, inC, inH, inW, records, version=1):
    with open(path, "wb") as f:
        f.write(encode(inC, inH, inW, records, version))


def conv_weight(rng, KH, KW, Cin, Cout):
    """He-normal conv weights in the [KH*KW*Cin, Cout] layout."""
    std = np.sqrt(2.0 / (KH * KW * Cin))
    return (rng.standard_normal((KH * KW * Cin, Cout)) * std).astype(np.float32)


def bn_params(rng, ch, gamma_lo=0.5, gamma_hi=1.5):
    mean = (rng.standard_normal(ch) * 0.1).astype(np.float32)
    var = rng.uniform(0.5, 1.5, ch).astype(np.float32)
    gamma = rng.uniform(gamma_lo, gamma_hi, ch).astype(np.float32)
    beta = (rng.standard_normal(ch) * 0.1).astype(np.float32)
    return ("bn", ch, mean, var, gamma, beta)


def resnet50(rng, in_hw=224, width=64, blocks=(3, 4, 6, 3), classes=1000, in_ch=3, head=True):
    """ResNet-50 v1.5 (stride on the 3x3), random init, as version-2 records.

    conv1 7x7/2 -> BN -> 3x3/2 MaxPool -> ReLU (MaxPool absorbs the ReLU, so the
    math is ReLU-then-pool as in ResNet; the reference's loader would drop a
    ReLU placed before the pool), then [3,4,6,3] bottlenecks 1x1 -> 3x3 -> 1x1
    with Conv+BN+ReLU fused at load, projection shortcuts on each stage's first
    block, global average pool, FC and softmax.  The last BN of each residual
    branch draws gamma from U[0.1,0.3] so activations stay O(1) through the
    16 residual additions of a random-init network.  head=False ends the
    model at the last block's Add+ReLU (no pool, FC or softmax).
    """
    R = []

    def add(rec):
        R.append(rec)
        return len(R) - 1

    add(("conv", 7, 7, width, 2, 3, conv_weight(rng, 7, 7, in_ch, width), np.zeros(width, np.float32)))
    add(bn_params(rng, width))
    add(("maxpool", 3, 2, 1))
    last = add(("relu",))
    cin = width
    for stage, nblk in enumerate(blocks):
        mid = width * (2 ** stage)
        cout = mid * 4
        for b in range(nblk):
            stride = 2 if (b == 0 and stage > 0) else 1
            block_in = last
            add(("conv", 1, 1, mid, 1, 0, conv_weight(rng, 1, 1, cin, mid), np.zeros(mid, np.float32)))
            add(bn_params(rng, mid))
            add(("relu",))
            add(("conv", 3, 3, mid, stride, 1, conv_weight(rng, 3, 3, mid, mid), np.zeros(mid, np.float32)))
            add(bn_params(rng, mid))
            add(("relu",))
            add(("conv", 1, 1, cout, 1, 0, conv_weight(rng, 1, 1, mid, cout), np.zeros(cout, np.float32)))
            main = add(bn_params(rng, cout, 0.1, 0.3))
            if b == 0:
                add(("input", block_in))
                add(("conv", 1, 1, cout, stride, 0, conv_weight(rng, 1, 1, cin, cout),
                     np.zeros(cout, np.float32)))
                add(bn_params(rng, cout))
                last = add(("add", main, 1))
            else:
                last = add(("add", block_in, 1))
            cin = cout
    if not head:
        return in_ch, in_hw, in_hw, R
    add(("gap",))
    fcw = (rng.standard_normal((cin, classes)) / np.sqrt(cin)).astype(np.float32)
    add(("fc", classes, cin, fcw, np.zeros(classes, np.float32)))
    add(("softmax",))
    return in_ch, in_hw, in_hw, R


def resnet50_flops(in_hw=224, width=64, blocks=(3, 4, 6, 3), classes=1000, in_ch=3):
    """Multiply-add count x2 of the convolutions and FC of resnet50() per image."""
    fl = 0
    h = (in_hw + 6 - 7) // 2 + 1
    fl += 2 * h * h * 7 * 7 * in_ch * width
    h = (h + 2 - 3) // 2 + 1
    cin = width
    for stage, nblk in enumerate(blocks):
        mid = width * (2 ** stage)
        cout = mid * 4
        for b in range(nblk):
            stride = 2 if (b == 0 and stage > 0) else 1
            ho = (h + 2 - 3) // stride + 1
            fl += 2 * h * h * cin * mid + 2 * ho * ho * 9 * mid * mid + 2 * ho * ho * mid * cout
            if b == 0:
                fl += 2 * ho * ho * cin * cout
            h = ho
            cin = cout
    fl += 2 * cin * classes
    return fl
