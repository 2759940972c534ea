"""Pins oracle_conv2d_route (the fp32 conv2d_impl predicate) to the compiled
reference's behaviour rather than to a reading of it: for each shape, the
reference's own acfun_conv2d / acfun_conv2d_relu / acfun_conv2d_g output is
bit-identical to the output of the entry point of the route the oracle names
(src/layers.cpp:106-195), and -- among the routes that compute the same
convolution with different roundings (Winograd F(4,3), Winograd F(2,3),
im2col + GEMM) -- differs from the routes it does not name.  The shapes sit on
both sides of every threshold of the predicate.  CPU only.

The direct depthwise and grouped kernels accumulate taps in the same order, so
where they would agree bit for bit the route between them does not change a
result; they are still each checked for identity with the route's output.
"""
import numpy as np
import pytest

import oracle
from tests.helpers import P

NONE, DW, GROUPED, SPLIT, R1X1, WINO43, WINO23, IM2COL = range(8)


def _call_ref_conv(ref, x, w, b, KH, KW, Cout, s, p, g, act, out):
    N, H, W, Cin = x.shape
    if g > 1:
        ref.acfun_conv2d_g(P(x), N, H, W, Cin, P(w), P(b), KH, KW, Cout, s, p, g, P(out), act)
    elif act:
        ref.acfun_conv2d_relu(P(x), N, H, W, Cin, P(w), P(b), KH, KW, Cout, s, p, P(out))
    else:
        ref.acfun_conv2d(P(x), N, H, W, Cin, P(w), P(b), KH, KW, Cout, s, p, P(out))


def _im2col(x, KH, KW, s, p, OH, OW):
    """col[OH*OW, KH*KW*Cin] of one image, zeros in padded taps (src/layers.cpp:39-58)."""
    H, W, Cin = x.shape
    xp = np.zeros((H + 2 * p + KH, W + 2 * p + KW, Cin), np.float32)
    xp[p:p + H, p:p + W] = x
    cols = [xp[kh:kh + s * (OH - 1) + 1:s, kw:kw + s * (OW - 1) + 1:s, :]
            for kh in range(KH) for kw in range(KW)]
    return np.ascontiguousarray(np.concatenate(cols, axis=2).reshape(OH * OW, KH * KW * Cin))


def run_route(ref, route, x, w, b, KH, KW, Cout, s, p, g, act):
    """The output of the route's own reference entry point (None if the route
    does not apply to the shape)."""
    N, H, W, Cin = x.shape
    OH, OW = oracle.out_hw(H, W, KH, KW, s, p)
    out = np.full((N, max(OH, 0), max(OW, 0), Cout), 7.0, np.float32)
    if route == DW:
        ref.acfun_conv2d_dw(P(x), N, H, W, Cin, P(w), P(b), KH, KW, s, p, P(out), act)
    elif route == GROUPED:
        ref.acfun_conv2d_grouped(P(x), N, H, W, Cin, P(w), P(b), KH, KW, Cout, s, p, g, P(out),
                                 act)
    elif route == SPLIT:               # per group, the dense conv of a contiguous copy
        ci, co = Cin // g, Cout // g
        for k in range(g):
            xg = np.ascontiguousarray(x[..., k * ci:(k + 1) * ci])
            wg = np.ascontiguousarray(w[k * co * KH * KW * ci:(k + 1) * co * KH * KW * ci])
            bg = None if b is None else np.ascontiguousarray(b[k * co:(k + 1) * co])
            og = np.empty((N, OH, OW, co), np.float32)
            _call_ref_conv(ref, xg, wg, bg, KH, KW, co, s, p, 1, act, og)
            out[..., k * co:(k + 1) * co] = og
    elif route == R1X1:                # one GEMM over the whole batch, gathered rows
        A = np.ascontiguousarray(np.stack([_im2col(x[n], 1, 1, s, p, OH, OW) for n in range(N)])
                                 .reshape(N * OH * OW, Cin))
        ref.acfun_gemm_epi(N * OH * OW, Cout, Cin, P(A), P(w), P(out), P(b), act)
    elif route == WINO43:
        ref.acfun_winograd43_conv3x3(P(x), N, H, W, Cin, P(w), P(b), Cout, P(out), act)
    elif route == WINO23:
        ref.acfun_winograd_conv3x3(P(x), N, H, W, Cin, P(w), P(b), Cout, P(out), act)
    elif route == IM2COL:              # one GEMM per image on its im2col matrix
        for n in range(N):
            col = _im2col(x[n], KH, KW, s, p, OH, OW)
            on = np.empty((OH * OW, Cout), np.float32)
            ref.acfun_gemm_epi(OH * OW, Cout, KH * KW * Cin, P(col), P(w), P(on), P(b), act)
            out[n] = on.reshape(OH, OW, Cout)
    return out


# (N, H, W, Cin, KH, KW, Cout, stride, pad, groups), the route the oracle must name
CASES = [
    ((1, 112, 112, 64, 3, 3, 64, 1, 1, 1), WINO43),    # every F(4,3) threshold met exactly
    ((1, 111, 112, 64, 3, 3, 64, 1, 1, 1), WINO23),    # H one below
    ((1, 112, 111, 64, 3, 3, 64, 1, 1, 1), WINO23),    # W one below
    ((1, 112, 112, 63, 3, 3, 64, 1, 1, 1), WINO23),    # Cin one below
    ((1, 112, 112, 64, 3, 3, 63, 1, 1, 1), WINO23),    # Cout one below
    ((2, 9, 10, 4, 3, 3, 4, 1, 1, 1), WINO23),         # smallest Winograd channels
    ((1, 3, 3, 8, 3, 3, 8, 1, 1, 1), WINO23),          # smallest Winograd image
    ((1, 9, 10, 3, 3, 3, 8, 1, 1, 1), IM2COL),         # Cin 3 < 4
    ((1, 9, 10, 8, 3, 3, 3, 1, 1, 1), IM2COL),         # Cout 3 < 4
    ((1, 2, 9, 8, 3, 3, 8, 1, 1, 1), IM2COL),          # H 2 < 3
    ((1, 9, 9, 8, 3, 3, 8, 2, 1, 1), IM2COL),          # stride 2
    ((1, 9, 9, 8, 3, 3, 8, 1, 0, 1), IM2COL),          # pad 0
    ((1, 9, 9, 8, 5, 5, 12, 1, 2, 1), IM2COL),         # 5x5
    ((2, 9, 9, 8, 1, 1, 12, 1, 0, 1), R1X1),           # 1x1, zero copy
    ((2, 9, 9, 8, 1, 1, 12, 2, 0, 1), R1X1),           # 1x1 strided gather
    ((1, 9, 9, 8, 1, 1, 12, 1, 1, 1), R1X1),           # 1x1 padded gather (zero rows)
    ((1, 9, 9, 16, 3, 3, 16, 1, 1, 16), DW),           # groups == Cin == Cout
    ((1, 9, 9, 16, 3, 3, 32, 1, 1, 2), GROUPED),       # Cin_per 8, Cout_per 16
    ((1, 7, 7, 128, 3, 3, 256, 1, 1, 2), GROUPED),     # Cin_per 64, Cout_per 128: at the limits
    ((1, 7, 7, 130, 3, 3, 16, 1, 1, 2), SPLIT),        # Cin_per 65 > 64
    ((1, 7, 7, 16, 3, 3, 258, 1, 1, 2), SPLIT),        # Cout_per 129 > 128
    ((1, 2, 2, 8, 3, 3, 8, 1, 0, 1), NONE),            # empty output
    ((1, 2, 2, 8, 3, 3, 8, 1, 0, 2), NONE),            # empty output, grouped
]

FAMILY = (WINO43, WINO23, IM2COL)    # same convolution, different roundings


@pytest.mark.parametrize("shape,route", CASES)
@pytest.mark.parametrize("act", [0, 1])
def test_route_matches_reference_behaviour(ref, shape, route, act):
    N, H, W, Cin, KH, KW, Cout, s, p, g = shape
    assert oracle.conv2d_route(N, H, W, Cin, KH, KW, Cout, s, p, g) == route
    rng = np.random.default_rng(abs(hash((shape, act))) % (1 << 32))
    x = rng.uniform(-1, 1, (N, H, W, Cin)).astype(np.float32)
    w = (rng.standard_normal(KH * KW * Cin * Cout // g) * 0.2).astype(np.float32)
    b = rng.uniform(-0.5, 0.5, Cout).astype(np.float32)
    OH, OW = oracle.out_hw(H, W, KH, KW, s, p)
    got = np.full((N, max(OH, 0), max(OW, 0), Cout), 7.0, np.float32)
    _call_ref_conv(ref, x, w, b, KH, KW, Cout, s, p, g, act, got)
    if route == NONE:
        assert got.size == 0
        return
    np.testing.assert_array_equal(got, run_route(ref, route, x, w, b, KH, KW, Cout, s, p, g, act))
    if route in FAMILY:
        wino_ok = KH == KW == 3 and s == 1 and p == 1
        for other in FAMILY:
            if other == route or (other != IM2COL and not wino_ok):
                continue
            alt = run_route(ref, other, x, w, b, KH, KW, Cout, s, p, g, act)
            assert not np.array_equal(got, alt), f"route {other} gives the same bits"
