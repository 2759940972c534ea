"""Pins the CPU oracle against the compiled reference (oracle/_ref).

Every oracle function whose result the reference fixes bit for bit is compared
exactly on seeded inputs that exercise its edges (tails, padding, ties, empty
and zero inputs); the shape lists follow the reference's own checks
(tools/test_int8_epi.cpp:48-53, tools/test_int8_direct.cpp:56-92,
tools/test_group_conv.cpp:21-101, src/benchmark.cpp:674-711).  CPU only.
"""
import numpy as np
import pytest

import oracle
from tests.helpers import (P, assert_bitexact, bf16_probe_values, f32, int8_conv_inputs,
                           int8_q_inputs, rel_err, s8, same_or_both_nan, u8)

EPI_SHAPES = [(64, 64, 64), (100, 100, 100), (255, 255, 255), (127, 129, 63), (16, 16, 16),
              (1, 16, 255), (513, 17, 131), (4, 4, 4), (33, 65, 129), (1023, 4, 7), (7, 1023, 5)]


@pytest.mark.parametrize("M,N,K", EPI_SHAPES)
def test_gemm_int8_exact(ref, rng, M, N, K):
    A, B = u8(rng, (M, K)), s8(rng, (K, N))
    want = np.empty((M, N), np.int32)
    ref.acfun_gemm_int8(M, N, K, P(A), P(B), P(want))
    assert_bitexact(oracle.gemm_int8(A, B), want, "gemm_int8")


@pytest.mark.parametrize("M,N,K", EPI_SHAPES)
@pytest.mark.parametrize("act", [0, 1])
def test_gemm_int8_epi_exact(ref, rng, M, N, K, act):
    A, B = u8(rng, (M, K)), s8(rng, (K, N))
    j = np.arange(N)
    alpha = (0.001 + 0.0005 * (j % 13)).astype(np.float32)   # tools/test_int8_epi.cpp:59-62
    beta = (-0.3 + 0.02 * (j % 7)).astype(np.float32)
    want = np.empty((M, N), np.float32)
    ref.acfun_gemm_int8_epi(M, N, K, P(A), P(B), P(want), P(alpha), P(beta), act)
    assert_bitexact(oracle.gemm_int8_epi(A, B, alpha, beta, act), want, "gemm_int8_epi")


@pytest.mark.parametrize("M,K,Cout", [(784, 64, 64), (100, 256, 20), (33, 7, 5)])
def test_conv1x1_int8_exact(ref, olib, rng, M, K, Cout):
    A, B = u8(rng, (M, K)), s8(rng, (K, Cout))
    alpha = rng.uniform(1e-4, 1e-3, Cout).astype(np.float32)
    beta = rng.uniform(-1, 1, Cout).astype(np.float32)
    for act in (0, 1):
        want = np.empty((M, Cout), np.float32)
        got = np.empty((M, Cout), np.float32)
        ref.acfun_conv1x1_int8(P(A), M, K, Cout, P(B), P(alpha), P(beta), P(want), act)
        olib.oracle_conv1x1_int8(A, M, K, Cout, B, alpha, beta, got, act)
        assert_bitexact(got, want, "conv1x1_int8")


# tools/test_int8_direct.cpp:56-92: small-K shapes incl. batch 2, odd Cout, stride 2
DIRECT_SHAPES = [(1, 32, 32, 3, 3, 3, 16, 1, 1), (2, 17, 19, 3, 3, 3, 7, 2, 1),
                 (1, 28, 28, 64, 1, 1, 33, 2, 0), (1, 15, 15, 7, 3, 3, 9, 1, 1),
                 (2, 9, 9, 2, 5, 5, 12, 2, 2), (1, 8, 8, 2, 3, 3, 1, 1, 0)]  # K <= 64 (the route contract)


@pytest.mark.parametrize("N,H,W,Cin,KH,KW,Cout,st,pd", DIRECT_SHAPES)
def test_conv_int8_direct_exact(ref, olib, rng, N, H, W, Cin, KH, KW, Cout, st, pd):
    OH, OW = oracle.out_hw(H, W, KH, KW, st, pd)
    x, w = u8(rng, (N, H, W, Cin)), s8(rng, (KH * KW * Cin, Cout))
    alpha = rng.uniform(1e-4, 1e-3, Cout).astype(np.float32)
    beta = rng.uniform(-1, 1, Cout).astype(np.float32)
    for act in (0, 1):
        want = np.empty((N, OH, OW, Cout), np.float32)
        got = np.empty_like(want)
        ref.acfun_conv2d_int8_direct(P(x), N, H, W, Cin, P(w), P(alpha), P(beta), KH, KW, Cout,
                                     st, pd, OH, OW, P(want), act)
        olib.oracle_conv2d_int8_direct(x, N, H, W, Cin, w, alpha, beta, KH, KW, Cout, st, pd,
                                       OH, OW, got, act)
        assert_bitexact(got, want, "conv2d_int8_direct")


def test_quantize_u8_rne_exact(ref, rng):
    x = rng.uniform(-1.5, 1.5, 10007).astype(np.float32)
    # exact ties k+0.5 and the float just below 0.5 (0.49999997)
    x[:8] = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 0.49999997, -0.49999997], np.float32)
    for inv_s in (np.float32(1.0), np.float32(127.0 / 1.5), np.float32(100.0)):
        want = np.empty(x.size, np.uint8)
        ref.acfun_quantize_u8(P(x), P(want), x.size, inv_s, 128)
        assert_bitexact(oracle.quantize_u8(x, inv_s, 128, 0), want, "quantize_u8")


@pytest.mark.parametrize("N,H,W,Cin,Cout", [(1, 8, 8, 16, 16), (2, 7, 9, 20, 5), (1, 3, 3, 4, 4),
                                            (1, 5, 6, 37, 19), (1, 4, 4, 128, 8)])
@pytest.mark.parametrize("act", [0, 1])
def test_winograd_int8_exact(ref, olib, rng, N, H, W, Cin, Cout, act):
    x, wq, ws, b = int8_conv_inputs(rng, N, H, W, Cin, 3, 3, Cout)
    maxa = np.float32(np.max(np.abs(x)))
    inv_s, s_in = np.float32(127.0) / maxa, maxa / np.float32(127.0)
    want = np.empty((N, H, W, Cout), np.float32)
    got = np.empty_like(want)
    ref.acfun_winograd_conv3x3_int8(P(x), N, H, W, Cin, P(wq), P(ws), P(b), Cout, s_in, inv_s,
                                    P(want), act)
    olib.oracle_winograd_conv3x3_int8(x, N, H, W, Cin, wq, ws, P(b), Cout, s_in, inv_s, got, act)
    assert_bitexact(got, want, "winograd_conv3x3_int8")


# One case per acfun_conv2d_int8 route (src/conv_int8.cpp:63-148)
ROUTE_CASES = [
    ((2, 10, 12, 16, 3, 3, 24, 1, 1), 2),   # Winograd
    ((2, 9, 9, 20, 3, 3, 8, 1, 1), 2),      # Winograd, channel tail (20 = 16 + 4)
    ((1, 12, 12, 3, 3, 3, 16, 1, 1), 3),    # Cin=3 < 4 -> direct (K=27)
    ((2, 14, 14, 32, 1, 1, 48, 1, 0), 4),   # 1x1
    ((1, 14, 14, 96, 1, 1, 40, 1, 0), 4),   # 1x1, K > 64
    ((1, 15, 15, 16, 3, 3, 32, 2, 1), 5),   # 3x3 s2 -> im2col+GEMM (K=144)
    ((2, 11, 11, 8, 1, 1, 16, 2, 0), 3),    # 1x1 s2, K=8 -> direct
    ((1, 13, 13, 24, 7, 7, 8, 2, 3), 5),    # 7x7/2 -> GEMM
]


@pytest.mark.parametrize("shape,route", ROUTE_CASES)
@pytest.mark.parametrize("act", [0, 1])
def test_conv2d_int8_routes_exact(ref, rng, shape, route, act):
    N, H, W, Cin, KH, KW, Cout, st, pd = shape
    assert oracle.conv2d_int8_route(H, W, Cin, KH, KW, Cout, st, pd) == route
    x, wq, ws, b = int8_conv_inputs(rng, N, H, W, Cin, KH, KW, Cout, bias=(act == 1))
    OH, OW = oracle.out_hw(H, W, KH, KW, st, pd)
    want = np.empty((N, OH, OW, Cout), np.float32)
    ref.acfun_conv2d_int8(P(x), N, H, W, Cin, P(wq), P(ws), P(b), KH, KW, Cout, st, pd,
                          np.float32(0.123), P(want), act)
    got = oracle.conv2d_int8(x, wq, ws, b, KH, KW, Cout, st, pd, act)
    assert_bitexact(got, want, f"conv2d_int8 route {route}")


def test_conv2d_int8_zero_input(ref):
    x = np.zeros((1, 6, 6, 8), np.float32)
    wq = np.ones((9 * 8, 8), np.int8)
    ws = np.full(8, 0.01, np.float32)
    b = np.full(8, 0.5, np.float32)
    want = np.full((1, 6, 6, 8), 7.0, np.float32)
    ref.acfun_conv2d_int8(P(x), 1, 6, 6, 8, P(wq), P(ws), P(b), 3, 3, 8, 1, 1, 0.0, P(want), 1)
    got = oracle.conv2d_int8(x, wq, ws, b, 3, 3, 8, 1, 1, 1)
    assert_bitexact(got, want, "zero input")
    assert np.all(got == 0.0)   # bias is not added (src/conv_int8.cpp:78)


# NaN, infinities and values whose scaled form leaves int32: the reference's x86
# conversions (integer indefinite for cvtps/cvttps, lroundf's long cut to int)
SPECIAL = np.array([np.nan, -np.nan, np.inf, -np.inf, 3e9, -3e9, 2147483648.0, -2147483648.0,
                    2147483520.0, 1e20, -1e20, 127.5, -128.5], np.float32)


def test_quantize_u8_special_values(ref):
    for inv_s, zp in ((np.float32(1.0), 128), (np.float32(0.5), 3), (np.float32(2.0), 300)):
        want = np.empty(SPECIAL.size, np.uint8)
        ref.acfun_quantize_u8(P(SPECIAL), P(want), SPECIAL.size, inv_s, zp)
        assert_bitexact(oracle.quantize_u8(SPECIAL, inv_s, zp, 0), want, "quantize_u8 specials")


def test_quantize_weights_special_values(ref, rng):
    w = (rng.standard_normal((40, 6)) * 0.2).astype(np.float32)
    w[3, 0] = np.nan                               # NaN among finite weights
    w[7, 1] = np.inf                               # max|w| = inf: every w/s is 0 or NaN
    w[:, 2] = np.nan                               # an all-NaN column: scale 1
    sw, qw = np.empty(6, np.float32), np.empty((40, 6), np.int8)
    ref.acfun_quantize_weights(P(w), 40, 6, P(sw), P(qw))
    so, qo = oracle.quantize_weights(w)
    assert_bitexact(so, sw, "scales")
    assert_bitexact(qo, qw, "wq")


@pytest.mark.parametrize("shape,route", ROUTE_CASES)
@pytest.mark.parametrize("act", [0, 1])
def test_conv2d_int8_nan_input(ref, rng, shape, route, act):
    """NaN activations: max|x| skips them, and each route's quantizer converts
    them as the reference's x86 code does."""
    N, H, W, Cin, KH, KW, Cout, st, pd = shape
    x, wq, ws, b = int8_conv_inputs(rng, N, H, W, Cin, KH, KW, Cout, bias=(act == 1))
    flat = x.reshape(-1)
    flat[rng.choice(flat.size, max(3, flat.size // 50), replace=False)] = np.nan
    flat[-1] = np.nan                              # the last channel: a route's scalar tail
    OH, OW = oracle.out_hw(H, W, KH, KW, st, pd)
    want = np.empty((N, OH, OW, Cout), np.float32)
    ref.acfun_conv2d_int8(P(x), N, H, W, Cin, P(wq), P(ws), P(b), KH, KW, Cout, st, pd,
                          np.float32(0.123), P(want), act)
    got = oracle.conv2d_int8(x, wq, ws, b, KH, KW, Cout, st, pd, act)
    assert_bitexact(got, want, f"conv2d_int8 route {route} with NaN input")


def test_quantize_weights_exact(ref, rng):
    w = (rng.standard_normal((300, 37)) * 0.2).astype(np.float32)
    w[:, 5] = 0.0                                  # all-zero column -> scale 1
    sw, qw = np.empty(37, np.float32), np.empty((300, 37), np.int8)
    ref.acfun_quantize_weights(P(w), 300, 37, P(sw), P(qw))
    so, qo = oracle.quantize_weights(w)
    assert_bitexact(so, sw, "scales")
    assert_bitexact(qo, qw, "wq")


# Windows up to 4x4 only: src/dw_avx512.cpp:28 keeps the transposed weights in a
# float[16*16] stack array, so KH*KW > 16 overflows it in the reference itself.
@pytest.mark.parametrize("N,H,W,C,K,st,pd", [(2, 13, 11, 96, 3, 2, 1), (1, 9, 9, 20, 3, 1, 1),
                                             (1, 8, 8, 3, 4, 1, 2), (1, 6, 7, 16, 3, 2, 0)])
@pytest.mark.parametrize("act", [0, 1])
def test_depthwise_exact(ref, rng, N, H, W, C, K, st, pd, act):
    x = rng.standard_normal((N, H, W, C)).astype(np.float32)
    w = (rng.standard_normal((C, K, K)) * 0.3).astype(np.float32)
    b = rng.standard_normal(C).astype(np.float32)
    OH, OW = oracle.out_hw(H, W, K, K, st, pd)
    want = np.empty((N, OH, OW, C), np.float32)
    ref.acfun_conv2d_dw(P(x), N, H, W, C, P(w), P(b), K, K, st, pd, P(want), act)
    assert_bitexact(oracle.conv2d_dw(x, w, b, K, K, st, pd, act), want, "depthwise")


@pytest.mark.parametrize("Cin,Cout,g", [(24, 48, 6), (12, 24, 3), (32, 48, 4), (12, 36, 3),
                                        (48, 96, 2), (6, 12, 3), (16, 128, 4)])
@pytest.mark.parametrize("act", [0, 1])
def test_grouped_exact(ref, rng, Cin, Cout, g, act):
    N, H, W, st, pd = 2, 9, 10, 1, 1
    x = rng.standard_normal((N, H, W, Cin)).astype(np.float32)
    w = (rng.standard_normal((g, 9 * (Cin // g), Cout // g)) * 0.3).astype(np.float32)
    b = rng.standard_normal(Cout).astype(np.float32)
    want = np.empty((N, H, W, Cout), np.float32)
    ref.acfun_conv2d_grouped(P(x), N, H, W, Cin, P(w), P(b), 3, 3, Cout, st, pd, g, P(want), act)
    assert_bitexact(oracle.conv2d_grouped(x, w, b, 3, 3, Cout, st, pd, g, act), want, "grouped")


@pytest.mark.parametrize("C", [5, 12, 16, 20, 96])
@pytest.mark.parametrize("pool,st,pd", [(3, 2, 1), (2, 2, 0), (3, 1, 1), (7, 7, 0)])
def test_maxpool_exact(ref, rng, C, pool, st, pd):
    x = rng.standard_normal((2, 14, 14, C)).astype(np.float32) - 0.5
    OH, OW = oracle.out_hw(14, 14, pool, pool, st, pd)
    for relu, fn in ((0, ref.acfun_maxpool), (1, ref.acfun_maxpool_relu)):
        want = np.empty((2, OH, OW, C), np.float32)
        fn(P(x), 2, 14, 14, C, pool, st, pd, P(want))
        assert_bitexact(oracle.maxpool(x, pool, st, pd, relu), want, "maxpool")


def test_batchnorm_relu_exact(ref, olib, rng):
    d = rng.standard_normal(6 * 7 * 13).astype(np.float32)
    mean, var = rng.standard_normal(13).astype(np.float32), rng.uniform(0.5, 1.5, 13).astype(np.float32)
    gamma, beta = rng.uniform(0.5, 1.5, 13).astype(np.float32), rng.standard_normal(13).astype(np.float32)
    want, got = d.copy(), d.copy()
    ref.acfun_batchnorm(P(want), want.size, 13, P(mean), P(var), P(gamma), P(beta), np.float32(1e-5))
    olib.oracle_batchnorm(got, got.size, 13, mean, var, P(gamma), P(beta), 1e-5)
    assert_bitexact(got, want, "batchnorm")
    for six in (0, 1):
        v = (rng.standard_normal(1000) * 5).astype(np.float32)
        a, b2 = v.copy(), v.copy()
        (ref.acfun_relu6 if six else ref.acfun_relu)(P(a), a.size)
        (olib.oracle_relu6 if six else olib.oracle_relu)(b2, b2.size)
        assert_bitexact(b2, a, "relu")


def test_softmax_close(ref, olib, rng):
    x = rng.standard_normal((4, 1000)).astype(np.float32) * 3
    want, got = np.empty_like(x), np.empty_like(x)
    ref.acfun_softmax(P(x), 4, 1000, P(want))
    olib.oracle_softmax(x, 4, 1000, got)
    assert rel_err(got, want) < 1e-6


def test_bf16_rounding_against_reference(ref, rng):
    """oracle.bf16 against the reference's own operand rounding, read back
    exactly: with K = 1, B = 1 and M, N multiples of 16 (all in its bf16
    micro-tiles) the reference computes C = bf16(A) * 1
    (src/gemm_bf16_avx512.cpp:37-44), and a product with 1 is exact."""
    A = bf16_probe_values(rng).reshape(-1, 1)
    assert A.shape[0] % 16 == 0
    B = np.ones((1, 16), np.float32)
    C = np.full((A.shape[0], 16), 7.0, np.float32)
    ref.acfun_gemm_bf16(A.shape[0], 16, 1, P(A), P(B), P(C))
    assert same_or_both_nan(C, np.repeat(oracle.bf16(A), 16, axis=1))


@pytest.mark.parametrize("M,N,K", [(96, 80, 200), (100, 70, 129), (7, 300, 64), (290, 5, 33)])
def test_gemm_bf16_against_reference(ref, rng, M, N, K):
    """The reference's bf16 GEMM against oracle.gemm_bf16_f64 (bf16 region and
    fp32 strips), each region discriminated from the other model, and K = 0
    leaving C untouched (src/gemm_bf16_avx512.cpp:173)."""
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    C = np.empty((M, N), np.float32)
    ref.acfun_gemm_bf16(M, N, K, P(A), P(B), P(C))
    want = oracle.gemm_bf16_f64(A, B)
    assert rel_err(C, want) < 1e-5
    M16, N16 = M // 16 * 16, N // 16 * 16
    rounded, exact = oracle.gemm_f64(oracle.bf16(A), oracle.bf16(B)), oracle.gemm_f64(A, B)
    if M16 and N16:
        assert rel_err(C[:M16, :N16], exact[:M16, :N16]) > 1e-4
    if M16 < M:
        assert rel_err(C[M16:], rounded[M16:]) > 1e-4
    C0 = np.full((M, N), 7.0, np.float32)
    ref.acfun_gemm_bf16(M, N, 0, P(A), P(B), P(C0))
    assert np.all(C0 == 7.0)


@pytest.mark.parametrize("M,N,K", [(64, 64, 64), (127, 129, 63), (256, 64, 1024), (1, 1000, 2048)])
def test_gemm_against_reference(ref, rng, M, N, K):
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    exact = oracle.gemm_f64(A, B)
    want = np.empty((M, N), np.float32)
    ref.acfun_gemm_ref(M, N, K, P(A), P(B), P(want))   # src/gemm_ref.cpp:22-25
    got = oracle.gemm(A, B)
    assert_bitexact(got, want, "oracle_gemm vs acfun_gemm_ref")  # same algorithm, same order
    simd = np.empty((M, N), np.float32)
    ref.acfun_gemm(M, N, K, P(A), P(B), P(simd))
    assert rel_err(simd, exact) < 1e-5 and rel_err(got, exact) < 1e-5


@pytest.mark.parametrize("M,N,K", [(64, 64, 64), (127, 129, 63), (33, 1000, 257), (5, 7, 1)])
@pytest.mark.parametrize("act", [0, 1])
def test_gemm_epi_against_reference(ref, rng, M, N, K, act):
    """oracle_gemm_epi vs the reference's scalar acfun_gemm_ref_epi
    (src/gemm_ref.cpp:39-63): same i-k-j order, bias and ReLU after the full
    reduction, so bit-exact; zeros in A exercise the skipped terms, a NULL
    bias the bias-free path."""
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    A[::3, ::2] = 0.0
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    for bias in (rng.uniform(-1, 1, N).astype(np.float32), None):
        want = np.empty((M, N), np.float32)
        ref.acfun_gemm_ref_epi(M, N, K, P(A), P(B), P(want), P(bias), act)
        assert_bitexact(oracle.gemm_epi(A, B, bias, act), want, "gemm_epi")
        if act:
            assert np.all(want >= 0)


@pytest.mark.parametrize("N,H,W,Cin,Cout", [(1, 8, 8, 16, 16), (2, 7, 9, 20, 5), (1, 3, 3, 4, 4),
                                            (1, 5, 6, 37, 19), (2, 6, 6, 128, 8)])
@pytest.mark.parametrize("act", [0, 1])
def test_winograd_int8_identity(ref, rng, N, H, W, Cin, Cout, act):
    """The identity the int8 Winograd route rests on: AT*T4*AT^T = 4*A with A
    the direct centred accumulator, so the reference's
    acfun_winograd_conv3x3_int8 equals fmaf((float)(4A), fl(fl(s*0.25)*ws), b)
    computed from oracle_conv_int8_centered_acc -- bit for bit, on odd sizes
    (half tiles at the border) and channel tails (lroundf channels)."""
    x, wq, ws, b = int8_conv_inputs(rng, N, H, W, Cin, 3, 3, Cout)
    maxa = np.float32(np.max(np.abs(x)))
    inv_s, s_in = np.float32(127.0) / maxa, maxa / np.float32(127.0)
    want = np.empty((N, H, W, Cout), np.float32)
    ref.acfun_winograd_conv3x3_int8(P(x), N, H, W, Cin, P(wq), P(ws), P(b), Cout, s_in, inv_s,
                                    P(want), act)
    acc = oracle.conv_int8_centered_acc(oracle.quantize_wino_u8(x, inv_s), wq, 3, 3, Cout, 1, 1)
    assert_bitexact(oracle.wino_int8_epilogue(acc, s_in, ws, b, act), want, "4A identity")
    # the accumulator itself against numpy brute force (int64, no wrap)
    if N * H * W * Cin * Cout <= 20000:
        u = oracle.quantize_wino_u8(x, inv_s).astype(np.int64) - 128
        up = np.pad(u, ((0, 0), (1, 1), (1, 1), (0, 0)))
        wk = wq.astype(np.int64).reshape(3, 3, Cin, Cout)
        A = sum(np.einsum("nhwc,cd->nhwd", up[:, i:i + H, j:j + W, :], wk[i, j])
                for i in range(3) for j in range(3))
        np.testing.assert_array_equal(acc, A)


def test_requantize_s8_against_reference(ref, rng):
    """oracle_requantize_s8 (the build-defined int8 output) equals the
    reference's own quantizer with zero point 128, minus 128
    (src/int8_quantize_avx512.cpp:15-20 with inv_s = 127/max|y|,
    src/conv_int8.cpp:75-81), on random values, exact ties and the extremes."""
    y = (rng.standard_normal(4099) * 3).astype(np.float32)
    q, s = oracle.requantize_s8(y)
    maxa = np.float32(np.max(np.abs(y)))
    assert s == maxa / np.float32(127.0)
    u = np.empty(y.size, np.uint8)
    ref.acfun_quantize_u8(P(y), P(u), y.size, np.float32(127.0) / maxa, 128)
    assert_bitexact(q, (u.astype(np.int16) - 128).astype(np.int8), "requantize")
    assert q[np.argmax(np.abs(y))] in (-127, 127)
    # max|y| = 127 gives inv_s = 1: k + 0.5 are exact ties (to even), -127.0 stays -127
    t = np.array([127.0, -127.0, 0.5, 1.5, 2.5, -0.5, -1.5, 126.5, -126.5, 0.49999997, 0.0, -0.0],
                 np.float32)
    q, s = oracle.requantize_s8(t)
    ref.acfun_quantize_u8(P(t), P(u), t.size, np.float32(1.0), 128)
    assert_bitexact(q, (u[:t.size].astype(np.int16) - 128).astype(np.int8), "requantize ties")
    np.testing.assert_array_equal(q, [127, -127, 0, 2, 2, 0, -2, 126, -126, 0, 0, 0])
    z, s0 = oracle.requantize_s8(np.zeros(17, np.float32))
    assert s0 == 0.0 and not np.any(z)


def test_reference_int8_gemm_route_batch_defect(ref, rng):
    """The reference's im2col + int8 GEMM route (src/conv_int8.cpp:133-141)
    builds the im2col rows of image 0 only: for N > 1 the rows of images
    1..N-1 stay zero-initialised (u8 0), so those images come out as beta[j]
    everywhere.  Its own model executor always calls with N = 1 and never
    meets this.  The oracle (and the GPU library) give every image its own
    rows; this pins that to the reference itself: in a 2-image call
    [image n, the image holding max|x|], image 0 is image n computed with the
    whole batch's activation scale, and must equal the oracle's image n."""
    N, H, Cin, Cout = 4, 15, 16, 32
    x, wq, ws, b = int8_conv_inputs(rng, N, H, H, Cin, 3, 3, Cout)
    x = x + rng.uniform(-0.3, 0.3, x.shape).astype(np.float32)   # distinct per image
    assert oracle.conv2d_int8_route(H, H, Cin, 3, 3, Cout, 2, 1) == 5
    OH = (H + 2 - 3) // 2 + 1
    got = oracle.conv2d_int8(x, wq, ws, b, 3, 3, Cout, 2, 1, 0)
    y = np.empty((N, OH, OH, Cout), np.float32)
    ref.acfun_conv2d_int8(P(x), N, H, H, Cin, P(wq), P(ws), P(b), 3, 3, Cout, 2, 1,
                          np.float32(0), P(y), 0)
    assert_bitexact(got[0], y[0], "image 0")
    maxa = np.float32(np.max(np.abs(x)))
    alpha = maxa / np.float32(127.0) * ws
    beta = b - (alpha * np.float32(128.0)) * wq.astype(np.float32).sum(0, dtype=np.float32)
    assert np.array_equal(y[1:], np.broadcast_to(beta.astype(np.float32), y[1:].shape))
    imax = int(np.argmax(np.abs(x).reshape(N, -1).max(1)))
    for n in range(N):
        pair = np.ascontiguousarray(np.stack([x[n], x[imax]]))
        y2 = np.empty((2, OH, OH, Cout), np.float32)
        ref.acfun_conv2d_int8(P(pair), 2, H, H, Cin, P(wq), P(ws), P(b), 3, 3, Cout, 2, 1,
                              np.float32(0), P(y2), 0)
        assert_bitexact(got[n], y2[0], f"image {n} with the batch scale")


# (N, H, W, Cin, KH, KW, Cout, stride, pad): every int8 route; N = 1 on the
# im2col + GEMM route (the reference unrolls image 0 only there)
Q8_CASES = [
    (2, 10, 12, 16, 3, 3, 24, 1, 1),     # Winograd
    (2, 9, 9, 20, 3, 3, 19, 1, 1),       # Winograd, channel tails in and out
    (2, 14, 14, 32, 1, 1, 48, 1, 0),     # 1x1
    (2, 12, 12, 3, 3, 3, 16, 1, 1),      # Cin 3 -> direct
    (1, 15, 15, 16, 3, 3, 32, 2, 1),     # im2col + GEMM
    (2, 11, 11, 8, 1, 1, 16, 2, 0),      # 1x1 s2, K = 8 -> direct
]


@pytest.mark.parametrize("shape", Q8_CASES)
@pytest.mark.parametrize("act", [0, 1])
def test_conv2d_int8_q_against_reference(ref, rng, shape, act):
    """oracle_conv2d_int8_q (s8 in with scale s_in, s8 out requantized per
    tensor) against the reference's own API: its acfun_conv2d_int8 on
    x = fl(q * s_in), which quantizes back to exactly q with activation scale
    s_in (max|x|/127 == s_in), then its acfun_quantize_u8(y, 127/max|y|, 128) - 128
    for rule 0.  Rule 1 (the Winograd route's input rule) is checked with
    oracle.quantize_wino_u8, pinned by test_winograd_int8_identity."""
    N, H, W, Cin, KH, KW, Cout, st, pd = shape
    q, s_in, x, wq, ws, b = int8_q_inputs(rng, N, H, W, Cin, KH, KW, Cout)
    assert np.float32(np.max(np.abs(x))) / np.float32(127) == s_in
    OH, OW = oracle.out_hw(H, W, KH, KW, st, pd)
    y = np.empty((N, OH, OW, Cout), np.float32)
    ref.acfun_conv2d_int8(P(x), N, H, W, Cin, P(wq), P(ws), P(b), KH, KW, Cout, st, pd,
                          np.float32(0), P(y), act)
    maxy = np.float32(np.max(np.abs(y)))
    inv = np.float32(127.0) / maxy
    u = np.empty(y.size, np.uint8)
    ref.acfun_quantize_u8(P(y), P(u), y.size, inv, 128)
    want0 = (u.astype(np.int16) - 128).astype(np.int8).reshape(y.shape)
    got0, s0 = oracle.conv2d_int8_q(q, s_in, wq, ws, b, KH, KW, Cout, st, pd, act, rule=0)
    assert_bitexact(got0, want0, "rule 0")
    assert s0 == maxy / np.float32(127.0)
    got1, s1 = oracle.conv2d_int8_q(q, s_in, wq, ws, b, KH, KW, Cout, st, pd, act, rule=1)
    want1 = (oracle.quantize_wino_u8(y, inv).astype(np.int16) - 128).astype(np.int8)
    assert_bitexact(got1, want1, "rule 1")
    assert s1 == s0


def test_conv2d_int8_q_zero(rng):
    """s_in == 0 marks an all-zero input: zero output and s_out = 0, as the
    reference returns zeros without the bias for max|x| < 1e-12
    (src/conv_int8.cpp:78)."""
    q = np.zeros((1, 6, 6, 8), np.int8)
    wq = rng.integers(-127, 128, (72, 8)).astype(np.int8)
    out, so = oracle.conv2d_int8_q(q, 0.0, wq, np.full(8, 0.01, np.float32),
                                   np.full(8, 0.5, np.float32), 3, 3, 8, 1, 1, 1)
    assert so == 0.0 and not np.any(out)
