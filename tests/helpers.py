"""Shared test helpers: pointers, seeded inputs, comparisons."""
import ctypes as C

import numpy as np


def P(a):
    """void* of a numpy array (None passes through as NULL)."""
    return None if a is None else C.c_void_p(a.ctypes.data)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def u8(rng, shape):
    return rng.integers(0, 256, size=shape, dtype=np.uint8)


def s8(rng, shape, lo=-128, hi=127):
    return rng.integers(lo, hi + 1, size=shape).astype(np.int8)


def rel_err(got, want):
    """Normwise relative error max|got-want| / max|want| (the fp32 tolerance measure)."""
    want = np.asarray(want, np.float64)
    d = np.max(np.abs(np.asarray(got, np.float64) - want)) if want.size else 0.0
    den = np.max(np.abs(want)) if want.size else 1.0
    return d / (den if den > 0 else 1.0)


def assert_bitexact(got, want, what=""):
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    if got.dtype.kind == "f":
        same = (got == want) | (np.isnan(got) & np.isnan(want))
    else:
        same = got == want
    if not np.all(same):
        idx = np.argwhere(~same)[:5]
        raise AssertionError(f"{what}: {np.count_nonzero(~same)} of {got.size} differ; first at "
                             f"{idx.tolist()}: got {got[tuple(idx[0])]!r} want {want[tuple(idx[0])]!r}")


def int8_conv_inputs(rng, N, H, W, Cin, KH, KW, Cout, bias=True):
    """Config-3 style inputs: x = q_a * s_a with q_a ~ U{-127..127}, wq ~ U{-127..127},
    ws ~ U[0.005, 0.05], b ~ N(0, 0.01)."""
    sa = np.float32(rng.uniform(0.005, 0.05))
    x = (rng.integers(-127, 128, size=(N, H, W, Cin)).astype(np.float32) * sa).astype(np.float32)
    wq = rng.integers(-127, 128, size=(KH * KW * Cin, Cout)).astype(np.int8)
    ws = rng.uniform(0.005, 0.05, Cout).astype(np.float32)
    b = (rng.standard_normal(Cout) * 0.01).astype(np.float32) if bias else None
    return x, wq, ws, b


def bf16_probe_values(rng):
    """fp32 inputs for the bf16 rounding check: ties to even and to odd, values
    that round up to the next binade or to infinity, signed zero, infinities,
    NaNs whose 32-bit rounding add wraps (to zero) or lands on infinity, and
    random normals.  No denormals: vdpbf16ps reads bf16 denormals as zero."""
    bits = np.array([0x3F808000, 0x3F818000, 0x3F80C000, 0x3F7FFFFF, 0x7F7FFFFF, 0xFF7FFFFF,
                     0x00000000, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0x7F800001,
                     0xFFFFFFFF, 0xFF800001, 0x7FFFFFFF, 0x00800000, 0x3380FFFF], np.uint32)
    rand = rng.standard_normal(495).astype(np.float32) * np.float32(1e3)
    return np.concatenate([bits.view(np.float32), rand])


def same_or_both_nan(a, b):
    return bool(np.all((a == b) | (np.isnan(a) & np.isnan(b))))


def int8_q_inputs(rng, N, H, W, Cin, KH, KW, Cout, bias=True):
    """s8 activations q (|q| <= 127, with +-127 present) and a scale s_in such
    that the float tensor x = fl(q * s_in) has max|x|/127 == s_in exactly in
    float32: the reference's acfun_conv2d_int8 on x then quantizes x back to q
    with activation scale s_in (its int8-input equivalent).  Returns
    (q, s_in, x, wq, ws, b)."""
    q = rng.integers(-127, 128, size=(N, H, W, Cin)).astype(np.int8)
    q.reshape(-1)[0] = 127
    q.reshape(-1)[-1] = -127
    while True:
        s_in = np.float32(rng.uniform(0.005, 0.05))
        if np.float32(np.float32(127.0) * s_in) / np.float32(127.0) == s_in:
            break
    x = (q.astype(np.float32) * s_in).astype(np.float32)
    wq = rng.integers(-127, 128, size=(KH * KW * Cin, Cout)).astype(np.int8)
    ws = rng.uniform(0.005, 0.05, Cout).astype(np.float32)
    b = (rng.standard_normal(Cout) * 0.01).astype(np.float32) if bias else None
    return q, s_in, x, wq, ws, b
