"""GPU parity: libacfun_amd.so through its C ABI against the CPU oracle.

Bars: int8 paths bit-exact (i32 accumulators and float
outputs); depthwise / grouped / maxpool / BN / ReLU bit-exact (they follow the
reference's AVX-512 operation order); fp32 GEMM / im2col / 1x1 within 1e-4 and
Winograd within 1e-3, both as normwise relative error max|d| / max|ref|
against the f64 closed form.
"""
import ctypes as C

import numpy as np
import pytest

import oracle
from tests.helpers import (P, assert_bitexact, bf16_probe_values, int8_conv_inputs, rel_err, s8,
                           same_or_both_nan, u8)

pytestmark = pytest.mark.gpu

GEMM_TOL = 1e-4
WINO_TOL = 1e-3


# ------------------------------------------------------------------ fp32 GEMM
@pytest.mark.parametrize("M,N,K", [(1024, 1024, 1024), (127, 129, 63), (1, 1000, 2048),
                                   (64, 1000, 2048), (300, 20, 7), (5, 3, 1), (333, 64, 576),
                                   (2048, 256, 64)])
@pytest.mark.parametrize("epi", [0, 1])
def test_gemm_f32(gpu, rng, M, N, K, epi):
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32) if epi else None
    got = np.full((M, N), np.nan, np.float32)
    if epi:
        gpu.acfun_gemm_epi(M, N, K, P(A), P(B), P(got), P(bias), 1)
    else:
        gpu.acfun_gemm(M, N, K, P(A), P(B), P(got))
    want = oracle.gemm_f64(A, B)
    if epi:
        want = np.maximum(want + bias, 0)
    assert rel_err(got, want) < GEMM_TOL, rel_err(got, want)


@pytest.mark.parametrize("M,N,K", [(2065, 1028, 200), (4096, 512, 64), (8192, 256, 4), (2049, 1040, 1032)])
@pytest.mark.parametrize("epi", [0, 1])
@pytest.mark.parametrize("offset", [0, 1])
def test_gemm_persistent(gpu, rng, M, N, K, epi, offset):
    """Shapes of at least two 64 x 64 tiles per CU take the persistent kernel
    (k_gemm32p): ragged M, N and K against 32-wide chunks, bias and ReLU, and C
    offset by one float so that its rows are not 16-byte aligned (element
    stores) -- through the device entry point, against the f64 product."""
    torch = pytest.importorskip("torch")
    dev = torch.device("cuda:0")
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    tA, tB, tb = (torch.from_numpy(a).to(dev) for a in (A, B, bias))
    buf = torch.full((M * N + 4,), float("nan"), device=dev)
    torch.cuda.synchronize()
    rc = gpu.acfun_dev_gemm_epi(M, N, K, tA.data_ptr(), tB.data_ptr(), buf.data_ptr() + 4 * offset,
                                tb.data_ptr() if epi else None, epi, None)
    torch.cuda.synchronize()
    assert rc == 0
    got = buf.cpu().numpy()[offset:offset + M * N].reshape(M, N)
    want = oracle.gemm_f64(A, B)
    if epi:
        want = np.maximum(want + bias, 0)
    assert rel_err(got, want) < GEMM_TOL, rel_err(got, want)


@pytest.mark.parametrize("M,N,K", [(200, 96, 300), (64, 64, 64), (1, 1, 1), (130, 70, 7),
                                   (1024, 1024, 1024), (33, 40, 0), (7, 300, 64), (290, 5, 33)])
def test_gemm_bf16(gpu, rng, M, N, K):
    """acfun_gemm_bf16 against the reference's arithmetic (oracle.gemm_bf16_f64:
    bf16 operands in the 16-aligned region, fp32 in the ragged strips, each
    pinned to the compiled reference); K = 0 leaves C untouched."""
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    got = np.full((M, N), 7.0, np.float32)
    gpu.acfun_gemm_bf16(M, N, K, P(A), P(B), P(got))
    if K == 0:
        assert np.all(got == 7.0)
        return
    assert rel_err(got, oracle.gemm_bf16_f64(A, B)) < 1e-5


def test_gemm_bf16_rounding_exact(gpu, rng):
    """The operand rounding bit for bit (ties, overflow to infinity, NaNs whose
    rounding add wraps): K = 1, B = 1, all in the bf16 region, so C = bf16(A)."""
    A = bf16_probe_values(rng).reshape(-1, 1)
    B = np.ones((1, 16), np.float32)
    got = np.full((A.shape[0], 16), 7.0, np.float32)
    gpu.acfun_gemm_bf16(A.shape[0], 16, 1, P(A), P(B), P(got))
    assert same_or_both_nan(got, np.repeat(oracle.bf16(A), 16, axis=1))


def test_fc_and_fc_relu(gpu, rng):
    N, Cin, Cout = 64, 2048, 1000
    x = rng.standard_normal((N, Cin)).astype(np.float32)
    w = (rng.standard_normal((Cin, Cout)) / 45).astype(np.float32)
    b = rng.standard_normal(Cout).astype(np.float32)
    for fn, relu in ((gpu.acfun_fc, False), (gpu.acfun_fc_relu, True)):
        got = np.zeros((N, Cout), np.float32)
        fn(P(x), N, Cin, P(w), P(b), Cout, P(got))
        want = oracle.gemm_f64(x, w) + b
        if relu:
            want = np.maximum(want, 0)
        assert rel_err(got, want) < GEMM_TOL


# ------------------------------------------------------------------ fp32 conv routes
CONV_CASES = [
    # N, H, W, Cin, KH, KW, Cout, s, p, groups, expected route, tol
    (2, 14, 14, 32, 1, 1, 48, 1, 0, 1, 4, GEMM_TOL),     # 1x1 zero-copy
    (2, 15, 15, 32, 1, 1, 40, 2, 0, 1, 4, GEMM_TOL),     # 1x1 strided (projection)
    (2, 30, 30, 3, 7, 7, 64, 2, 3, 1, 7, GEMM_TOL),      # conv1 7x7/2, Cin=3 (scalar A path)
    (1, 15, 18, 3, 3, 3, 5, 2, 1, 1, 7, GEMM_TOL),       # stride 2, Cin=3, odd sizes
    (2, 9, 10, 1, 5, 5, 4, 2, 2, 1, 7, GEMM_TOL),        # stride 2, Cin=1, 5x5
    (1, 11, 13, 2, 3, 3, 3, 2, 0, 1, 7, GEMM_TOL),       # stride 2, Cin=2, pad 0
    (1, 12, 12, 3, 4, 4, 4, 2, 1, 1, 7, GEMM_TOL),       # stride 2, even kernel
    (2, 16, 16, 32, 3, 3, 64, 2, 1, 1, 7, GEMM_TOL),     # 3x3/2 im2col
    (1, 9, 11, 6, 3, 3, 5, 1, 0, 1, 7, GEMM_TOL),        # 3x3 pad 0 -> im2col, odd channels
    (2, 20, 18, 16, 3, 3, 24, 1, 1, 1, 6, WINO_TOL),     # F(2,3)
    (1, 7, 9, 5, 3, 3, 6, 1, 1, 1, 6, WINO_TOL),         # F(2,3), odd sizes
    (1, 29, 30, 20, 3, 3, 40, 1, 1, 1, 6, WINO_TOL),     # F(2,3) 16-wide units, odd chunk count
    (3, 14, 13, 64, 3, 3, 64, 1, 1, 1, 6, WINO_TOL),     # F(2,3) 8-wide units, ragged edge
    (2, 8, 8, 24, 3, 3, 36, 1, 1, 1, 6, WINO_TOL),       # F(2,3) small image (128-slot kernel)
    (1, 112, 112, 64, 3, 3, 64, 1, 1, 1, 5, WINO_TOL),   # F(4,3)
    (1, 113, 115, 64, 3, 3, 72, 1, 1, 1, 5, WINO_TOL),   # F(4,3), ragged tiles
    (2, 10, 10, 256, 3, 3, 256, 1, 1, 2, 3, GEMM_TOL),   # grouped, Cin_per=128 > 64 -> split
    # Cin a multiple of 64: the implicit GEMM on the LDS-DMA engine (conv32)
    (2, 15, 15, 64, 1, 1, 40, 2, 0, 1, 4, GEMM_TOL),     # 1x1/2 projection
    (2, 16, 17, 64, 3, 3, 64, 2, 1, 1, 7, GEMM_TOL),     # 3x3/2
    (1, 9, 9, 128, 3, 3, 36, 2, 1, 1, 7, GEMM_TOL),      # 3x3/2, ragged M and Cout
    (1, 12, 11, 64, 5, 5, 32, 1, 2, 1, 7, GEMM_TOL),     # 5x5 pad 2
    (1, 10, 10, 128, 3, 3, 68, 1, 0, 1, 7, GEMM_TOL),    # 3x3 pad 0, two 64-channel chunks per tap
    (3, 7, 7, 128, 3, 3, 64, 1, 1, 1, 6, WINO_TOL),      # F(2,3) route on a 7x7 image
]


@pytest.mark.parametrize("case", CONV_CASES)
@pytest.mark.parametrize("act", [0, 1])
def test_conv2d_fp32_routes(gpu, rng, case, act):
    N, H, W, Cin, KH, KW, Cout, s, p, g, route, tol = case
    assert oracle.conv2d_route(N, H, W, Cin, KH, KW, Cout, s, p, g) == route
    x = rng.uniform(0, 1, (N, H, W, Cin)).astype(np.float32)
    w = (rng.standard_normal((KH * KW * Cin // g, Cout)) * np.sqrt(2 / (KH * KW * Cin / g))).astype(np.float32)
    b = (rng.standard_normal(Cout) * 0.01).astype(np.float32) if act else None
    OH, OW = oracle.out_hw(H, W, KH, KW, s, p)
    got = np.full((N, OH, OW, Cout), np.nan, np.float32)
    if g > 1:
        gpu.acfun_conv2d_g(P(x), N, H, W, Cin, P(w), P(b), KH, KW, Cout, s, p, g, P(got), act)
    elif act:
        gpu.acfun_conv2d_relu(P(x), N, H, W, Cin, P(w), P(b), KH, KW, Cout, s, p, P(got))
    else:
        gpu.acfun_conv2d(P(x), N, H, W, Cin, P(w), P(b), KH, KW, Cout, s, p, P(got))
    want = oracle.conv2d_f64(x, w, b, KH, KW, Cout, s, p, g, act)
    assert rel_err(got, want) < tol, rel_err(got, want)


@pytest.mark.parametrize("fn,tile", [("acfun_winograd_conv3x3", 2), ("acfun_winograd43_conv3x3", 4)])
def test_winograd_entry_points(gpu, rng, fn, tile):
    N, H, W, Cin, Cout = 2, 17, 13, 12, 20
    x = rng.uniform(0, 1, (N, H, W, Cin)).astype(np.float32)
    w = (rng.standard_normal((9 * Cin, Cout)) * 0.2).astype(np.float32)
    b = (rng.standard_normal(Cout) * 0.01).astype(np.float32)
    got = np.zeros((N, H, W, Cout), np.float32)
    getattr(gpu, fn)(P(x), N, H, W, Cin, P(w), P(b), Cout, P(got), 1)
    want = oracle.conv2d_f64(x, w, b, 3, 3, Cout, 1, 1, 1, 1)
    assert rel_err(got, want) < WINO_TOL


def test_conv2d_empty_output_untouched(gpu):
    x = np.ones((1, 2, 2, 4), np.float32)
    w = np.ones((9 * 4, 4), np.float32)
    out = np.full(16, 7.0, np.float32)
    gpu.acfun_conv2d(P(x), 1, 2, 2, 4, P(w), None, 3, 3, 4, 1, 0, P(out))   # OH = 0
    assert np.all(out == 7.0)


# ------------------------------------------------------------------ bandwidth kernels
@pytest.mark.parametrize("N,H,W,C,K,st,pd", [(2, 13, 11, 96, 3, 2, 1), (1, 9, 9, 20, 3, 1, 1),
                                             (1, 8, 8, 3, 5, 1, 2), (1, 6, 7, 18, 3, 2, 0)])
@pytest.mark.parametrize("act", [0, 1])
def test_depthwise_exact(gpu, rng, N, H, W, C, K, st, pd, act):
    x = rng.standard_normal((N, H, W, C)).astype(np.float32)
    w = (rng.standard_normal((C, K, K)) * 0.3).astype(np.float32)
    b = rng.standard_normal(C).astype(np.float32)
    OH, OW = oracle.out_hw(H, W, K, K, st, pd)
    got = np.zeros((N, OH, OW, C), np.float32)
    gpu.acfun_conv2d_dw(P(x), N, H, W, C, P(w), P(b), K, K, st, pd, P(got), act)
    assert_bitexact(got, oracle.conv2d_dw(x, w, b, K, K, st, pd, act), "depthwise")
    # routed through acfun_conv2d_g (groups == Cin == Cout)
    got2 = np.zeros_like(got)
    gpu.acfun_conv2d_g(P(x), N, H, W, C, P(w), P(b), K, K, C, st, pd, C, P(got2), act)
    assert_bitexact(got2, got, "conv2d_g depthwise route")


@pytest.mark.parametrize("Cin,Cout,g", [(24, 48, 6), (12, 24, 3), (32, 48, 4), (12, 36, 3),
                                        (48, 96, 2), (6, 12, 3), (16, 128, 4)])
@pytest.mark.parametrize("act", [0, 1])
@pytest.mark.parametrize("st", [1, 2])
def test_grouped_exact(gpu, rng, Cin, Cout, g, act, st):
    N, H, W = 2, 9, 10
    x = rng.standard_normal((N, H, W, Cin)).astype(np.float32)
    w = (rng.standard_normal((g, 9 * (Cin // g), Cout // g)) * 0.3).astype(np.float32)
    b = rng.standard_normal(Cout).astype(np.float32)
    OH, OW = oracle.out_hw(H, W, 3, 3, st, 1)
    got = np.zeros((N, OH, OW, Cout), np.float32)
    gpu.acfun_conv2d_g(P(x), N, H, W, Cin, P(w), P(b), 3, 3, Cout, st, 1, g, P(got), act)
    assert_bitexact(got, oracle.conv2d_grouped(x, w, b, 3, 3, Cout, st, 1, g, act), "grouped")


@pytest.mark.parametrize("C", [5, 12, 16, 20, 96])
@pytest.mark.parametrize("pool,st,pd", [(3, 2, 1), (2, 2, 0), (3, 1, 1), (7, 7, 0)])
def test_maxpool_exact(gpu, rng, C, pool, st, pd):
    x = rng.standard_normal((2, 14, 14, C)).astype(np.float32) - 0.5
    OH, OW = oracle.out_hw(14, 14, pool, pool, st, pd)
    for relu, fn in ((0, gpu.acfun_maxpool), (1, gpu.acfun_maxpool_relu)):
        got = np.zeros((2, OH, OW, C), np.float32)
        fn(P(x), 2, 14, 14, C, pool, st, pd, P(got))
        assert_bitexact(got, oracle.maxpool(x, pool, st, pd, relu), "maxpool")


def test_elementwise_exact(gpu, olib, rng):
    d = rng.standard_normal(6 * 7 * 13).astype(np.float32) * 4
    mean, var = rng.standard_normal(13).astype(np.float32), rng.uniform(0.5, 1.5, 13).astype(np.float32)
    gamma, beta = rng.uniform(0.5, 1.5, 13).astype(np.float32), rng.standard_normal(13).astype(np.float32)
    got, want = d.copy(), d.copy()
    gpu.acfun_batchnorm(P(got), got.size, 13, P(mean), P(var), P(gamma), P(beta), np.float32(1e-5))
    olib.oracle_batchnorm(want, want.size, 13, mean, var, P(gamma), P(beta), 1e-5)
    assert_bitexact(got, want, "batchnorm")
    for six in (0, 1):
        a, b2 = d.copy(), d.copy()
        (gpu.acfun_relu6 if six else gpu.acfun_relu)(P(a), a.size)
        (olib.oracle_relu6 if six else olib.oracle_relu)(b2, b2.size)
        assert_bitexact(a, b2, "relu")
    x = rng.standard_normal((3, 1000)).astype(np.float32) * 3
    sm, smw = np.zeros_like(x), np.zeros_like(x)
    gpu.acfun_softmax(P(x), 3, 1000, P(sm))
    olib.oracle_softmax(x, 3, 1000, smw)
    assert rel_err(sm, smw) < 1e-6


# ------------------------------------------------------------------ int8
EPI_SHAPES = [(64, 64, 64), (100, 100, 100), (255, 255, 255), (127, 129, 63), (16, 16, 16),
              (1, 16, 255), (513, 17, 131), (4, 4, 4), (33, 65, 129), (1023, 4, 7), (7, 1023, 5),
              (512, 512, 512)]


@pytest.mark.parametrize("M,N,K", EPI_SHAPES)
def test_gemm_int8_exact(gpu, rng, M, N, K):
    A, B = u8(rng, (M, K)), s8(rng, (K, N))
    got = np.zeros((M, N), np.int32)
    gpu.acfun_gemm_int8(M, N, K, P(A), P(B), P(got))
    assert_bitexact(got, oracle.gemm_int8(A, B), "gemm_int8")


@pytest.mark.parametrize("M,N,K", EPI_SHAPES)
@pytest.mark.parametrize("act", [0, 1])
def test_gemm_int8_epi_exact(gpu, rng, M, N, K, act):
    A, B = u8(rng, (M, K)), s8(rng, (K, N))
    j = np.arange(N)
    alpha = (0.001 + 0.0005 * (j % 13)).astype(np.float32)
    beta = (-0.3 + 0.02 * (j % 7)).astype(np.float32)
    got = np.zeros((M, N), np.float32)
    gpu.acfun_gemm_int8_epi(M, N, K, P(A), P(B), P(got), P(alpha), P(beta), act)
    assert_bitexact(got, oracle.gemm_int8_epi(A, B, alpha, beta, act), "gemm_int8_epi")


@pytest.mark.parametrize("M,K,Cout", [(784, 64, 64), (100, 256, 20), (33, 7, 5)])
def test_conv1x1_int8_exact(gpu, olib, rng, M, K, Cout):
    A, B = u8(rng, (M, K)), s8(rng, (K, Cout))
    alpha = rng.uniform(1e-4, 1e-3, Cout).astype(np.float32)
    beta = rng.uniform(-1, 1, Cout).astype(np.float32)
    for act in (0, 1):
        got, want = np.zeros((M, Cout), np.float32), np.zeros((M, Cout), np.float32)
        gpu.acfun_conv1x1_int8(P(A), M, K, Cout, P(B), P(alpha), P(beta), P(got), act)
        olib.oracle_conv1x1_int8(A, M, K, Cout, B, alpha, beta, want, act)
        assert_bitexact(got, want, "conv1x1_int8")


@pytest.mark.parametrize("N,H,W,Cin,KH,KW,Cout,st,pd", [
    (1, 32, 32, 3, 3, 3, 16, 1, 1), (2, 17, 19, 3, 3, 3, 7, 2, 1), (1, 28, 28, 64, 1, 1, 33, 2, 0),
    (1, 15, 15, 7, 3, 3, 9, 1, 1), (2, 9, 9, 4, 5, 5, 12, 2, 2), (1, 8, 8, 2, 3, 3, 1, 1, 0)])
def test_conv_int8_direct_exact(gpu, olib, rng, N, H, W, Cin, KH, KW, Cout, st, pd):
    OH, OW = oracle.out_hw(H, W, KH, KW, st, pd)
    x, w = u8(rng, (N, H, W, Cin)), s8(rng, (KH * KW * Cin, Cout))
    alpha = rng.uniform(1e-4, 1e-3, Cout).astype(np.float32)
    beta = rng.uniform(-1, 1, Cout).astype(np.float32)
    for act in (0, 1):
        got, want = np.zeros((N, OH, OW, Cout), np.float32), np.zeros((N, OH, OW, Cout), np.float32)
        gpu.acfun_conv2d_int8_direct(P(x), N, H, W, Cin, P(w), P(alpha), P(beta), KH, KW, Cout,
                                     st, pd, OH, OW, P(got), act)
        olib.oracle_conv2d_int8_direct(x, N, H, W, Cin, w, alpha, beta, KH, KW, Cout, st, pd,
                                       OH, OW, want, act)
        assert_bitexact(got, want, "conv2d_int8_direct")


def test_quantize_u8_exact(gpu, rng):
    x = rng.uniform(-1.5, 1.5, 10007).astype(np.float32)
    x[:8] = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 0.49999997, -0.49999997], np.float32)
    for inv_s in (np.float32(1.0), np.float32(127.0 / 1.5), np.float32(100.0)):
        got = np.zeros(x.size, np.uint8)
        gpu.acfun_quantize_u8(P(x), P(got), x.size, inv_s, 128)
        assert_bitexact(got, oracle.quantize_u8(x, inv_s, 128, 0), "quantize_u8")


# NaN, infinities and values whose scaled form leaves int32 (the reference's x86
# conversions, pinned in tests/test_oracle_pins.py)
SPECIAL = np.array([np.nan, -np.nan, np.inf, -np.inf, 3e9, -3e9, 2147483648.0, -2147483648.0,
                    2147483520.0, 1e20, -1e20, 127.5, -128.5], np.float32)


def test_quantize_u8_special_values(gpu):
    for inv_s, zp in ((np.float32(1.0), 128), (np.float32(0.5), 3), (np.float32(2.0), 300)):
        got = np.zeros(SPECIAL.size, np.uint8)
        gpu.acfun_quantize_u8(P(SPECIAL), P(got), SPECIAL.size, inv_s, zp)
        assert_bitexact(got, oracle.quantize_u8(SPECIAL, inv_s, zp, 0), "quantize_u8 specials")


def test_quantize_weights_special_values(gpu, rng):
    w = (rng.standard_normal((40, 6)) * 0.2).astype(np.float32)
    w[3, 0], w[7, 1] = np.nan, np.inf
    w[:, 2] = np.nan
    sw, qw = np.zeros(6, np.float32), np.zeros((40, 6), np.int8)
    gpu.acfun_quantize_weights(P(w), 40, 6, P(sw), P(qw))
    so, qo = oracle.quantize_weights(w)
    assert_bitexact(sw, so, "scales")
    assert_bitexact(qw, qo, "wq")


def test_quantize_weights_exact(gpu, rng):
    w = (rng.standard_normal((300, 37)) * 0.2).astype(np.float32)
    w[:, 5] = 0.0
    sw, qw = np.zeros(37, np.float32), np.zeros((300, 37), np.int8)
    gpu.acfun_quantize_weights(P(w), 300, 37, P(sw), P(qw))
    so, qo = oracle.quantize_weights(w)
    assert_bitexact(sw, so, "scales")
    assert_bitexact(qw, qo, "wq")


@pytest.mark.parametrize("N,H,W,Cin,Cout", [(1, 8, 8, 16, 16), (2, 7, 9, 20, 5), (1, 3, 3, 4, 4),
                                            (1, 5, 6, 37, 19), (1, 4, 4, 128, 8)])
@pytest.mark.parametrize("act", [0, 1])
def test_winograd_int8_exact(gpu, olib, rng, N, H, W, Cin, Cout, act):
    x, wq, ws, b = int8_conv_inputs(rng, N, H, W, Cin, 3, 3, Cout)
    maxa = np.float32(np.max(np.abs(x)))
    inv_s, s_in = np.float32(127.0) / maxa, maxa / np.float32(127.0)
    got, want = np.zeros((N, H, W, Cout), np.float32), np.zeros((N, H, W, Cout), np.float32)
    gpu.acfun_winograd_conv3x3_int8(P(x), N, H, W, Cin, P(wq), P(ws), P(b), Cout, s_in, inv_s,
                                    P(got), act)
    olib.oracle_winograd_conv3x3_int8(x, N, H, W, Cin, wq, ws, P(b), Cout, s_in, inv_s, want, act)
    assert_bitexact(got, want, "winograd_conv3x3_int8")


ROUTE_CASES = [
    (2, 10, 12, 16, 3, 3, 24, 1, 1), (2, 9, 9, 20, 3, 3, 8, 1, 1), (1, 12, 12, 3, 3, 3, 16, 1, 1),
    (2, 14, 14, 32, 1, 1, 48, 1, 0), (1, 14, 14, 96, 1, 1, 40, 1, 0), (1, 15, 15, 16, 3, 3, 32, 2, 1),
    (2, 11, 11, 8, 1, 1, 16, 2, 0), (1, 13, 13, 24, 7, 7, 8, 2, 3), (1, 30, 30, 3, 7, 7, 64, 2, 3),
]


@pytest.mark.parametrize("shape", ROUTE_CASES)
@pytest.mark.parametrize("act", [0, 1])
def test_conv2d_int8_exact(gpu, rng, shape, act):
    N, H, W, Cin, KH, KW, Cout, st, pd = shape
    x, wq, ws, b = int8_conv_inputs(rng, N, H, W, Cin, KH, KW, Cout, bias=(act == 1))
    OH, OW = oracle.out_hw(H, W, KH, KW, st, pd)
    got = np.full((N, OH, OW, Cout), np.nan, np.float32)
    gpu.acfun_conv2d_int8(P(x), N, H, W, Cin, P(wq), P(ws), P(b), KH, KW, Cout, st, pd,
                          np.float32(0.5), P(got), act)
    assert_bitexact(got, oracle.conv2d_int8(x, wq, ws, b, KH, KW, Cout, st, pd, act), "conv2d_int8")


@pytest.mark.parametrize("shape", ROUTE_CASES)
@pytest.mark.parametrize("act", [0, 1])
def test_conv2d_int8_nan_input(gpu, rng, shape, act):
    """NaN activations on every route: max|x| skips them and each route's
    quantizer converts them as the reference's x86 code does."""
    N, H, W, Cin, KH, KW, Cout, st, pd = shape
    x, wq, ws, b = int8_conv_inputs(rng, N, H, W, Cin, KH, KW, Cout, bias=(act == 1))
    flat = x.reshape(-1)
    flat[rng.choice(flat.size, max(3, flat.size // 50), replace=False)] = np.nan
    flat[-1] = np.nan
    OH, OW = oracle.out_hw(H, W, KH, KW, st, pd)
    got = np.full((N, OH, OW, Cout), 7.0, np.float32)
    gpu.acfun_conv2d_int8(P(x), N, H, W, Cin, P(wq), P(ws), P(b), KH, KW, Cout, st, pd,
                          np.float32(0.5), P(got), act)
    assert_bitexact(got, oracle.conv2d_int8(x, wq, ws, b, KH, KW, Cout, st, pd, act),
                    f"conv2d_int8 NaN input {shape}")


def test_conv2d_int8_zero_input(gpu):
    x = np.zeros((1, 6, 6, 8), np.float32)
    wq = np.ones((9 * 8, 8), np.int8)
    ws = np.full(8, 0.01, np.float32)
    b = np.full(8, 0.5, np.float32)
    got = np.full((1, 6, 6, 8), 7.0, np.float32)
    gpu.acfun_conv2d_int8(P(x), 1, 6, 6, 8, P(wq), P(ws), P(b), 3, 3, 8, 1, 1, 0.0, P(got), 1)
    assert np.all(got == 0.0)


# ------------------------------------------------------------------ full BASELINE configs
def test_config3a_full_exact(gpu, rng):
    """int8 1x1, N=32, 28x28, 256 -> 512, bias + ReLU: bit-exact at full size."""
    x, wq, ws, b = int8_conv_inputs(rng, 32, 28, 28, 256, 1, 1, 512)
    got = np.zeros((32, 28, 28, 512), np.float32)
    gpu.acfun_conv2d_int8(P(x), 32, 28, 28, 256, P(wq), P(ws), P(b), 1, 1, 512, 1, 0, 0.0, P(got), 1)
    assert_bitexact(got, oracle.conv2d_int8(x, wq, ws, b, 1, 1, 512, 1, 0, 1), "cfg3a")


def test_config3b_full_exact(gpu, rng):
    """int8 3x3/s1/p1, N=32, 28x28, 128 -> 128 (Winograd route): bit-exact at full size."""
    x, wq, ws, b = int8_conv_inputs(rng, 32, 28, 28, 128, 3, 3, 128)
    got = np.zeros((32, 28, 28, 128), np.float32)
    gpu.acfun_conv2d_int8(P(x), 32, 28, 28, 128, P(wq), P(ws), P(b), 3, 3, 128, 1, 1, 0.0, P(got), 1)
    assert_bitexact(got, oracle.conv2d_int8(x, wq, ws, b, 3, 3, 128, 1, 1, 1), "cfg3b")


def _check_images(got, x, w, b, Cout, tol, step=4):
    """Every image against the f64 direct convolution, a few images at a time
    (images are independent)."""
    for n in range(0, x.shape[0], step):
        want = oracle.conv2d_f64(np.ascontiguousarray(x[n:n + step]), w, b, 3, 3, Cout, 1, 1, 1, 1)
        assert rel_err(got[n:n + step], want) < tol, (n, rel_err(got[n:n + step], want))


@pytest.mark.parametrize("N,HW,tol", [(32, 56, WINO_TOL), (8, 112, WINO_TOL)])
def test_config2_full(gpu, rng, N, HW, tol):
    """fp32 3x3 conv + bias + ReLU at config 2a (F(2,3)) / 2b (F(4,3)) size,
    every image checked."""
    C = 64
    x = rng.uniform(0, 1, (N, HW, HW, C)).astype(np.float32)
    w = (rng.standard_normal((9 * C, C)) * np.sqrt(2 / (9 * C))).astype(np.float32)
    b = (rng.standard_normal(C) * 0.01).astype(np.float32)
    got = np.zeros((N, HW, HW, C), np.float32)
    gpu.acfun_conv2d_relu(P(x), N, HW, HW, C, P(w), P(b), 3, 3, C, 1, 1, P(got))
    _check_images(got, x, w, b, C, tol)


# F(2,3) 32-tile units at batch sizes around config 2a, including a ragged
# 20 -> 40 conv (4 chunks, partial output-channel block), 896 units of 16
# chunks (more units than workgroups) and 252 units (fewer units than
# workgroups, not a multiple of 8); every image is checked and a second run
# must repeat the first bit for bit.
@pytest.mark.parametrize("N,Cin,Cout", [(15, 64, 64), (32, 20, 40), (26, 64, 64), (4, 128, 256),
                                        (3, 32, 96)])
def test_wino23_batches(gpu, rng, N, Cin, Cout):
    HW = 56
    x = rng.uniform(0, 1, (N, HW, HW, Cin)).astype(np.float32)
    w = (rng.standard_normal((9 * Cin, Cout)) * np.sqrt(2 / (9 * Cin))).astype(np.float32)
    b = (rng.standard_normal(Cout) * 0.01).astype(np.float32)
    got = np.full((N, HW, HW, Cout), np.nan, np.float32)
    gpu.acfun_conv2d_relu(P(x), N, HW, HW, Cin, P(w), P(b), 3, 3, Cout, 1, 1, P(got))
    _check_images(got, x, w, b, Cout, WINO_TOL)
    again = np.full_like(got, np.nan)
    gpu.acfun_conv2d_relu(P(x), N, HW, HW, Cin, P(w), P(b), 3, 3, Cout, 1, 1, P(again))
    assert_bitexact(again, got, "repeat run")


# F(2,3) units on rectangular images whose tile grid is ragged at the right
# and bottom edges (odd pixel counts, partial 16-tile columns), with ragged
# input and output channel counts.
@pytest.mark.parametrize("N,H,W,Cin,Cout", [(3, 50, 46, 24, 48), (3, 22, 54, 20, 32), (2, 64, 64, 64, 64),
                                            (5, 41, 27, 36, 40)])
def test_wino23_unit_shapes(gpu, rng, N, H, W, Cin, Cout):
    x = rng.uniform(0, 1, (N, H, W, Cin)).astype(np.float32)
    w = (rng.standard_normal((9 * Cin, Cout)) * np.sqrt(2 / (9 * Cin))).astype(np.float32)
    b = (rng.standard_normal(Cout) * 0.01).astype(np.float32)
    got = np.full((N, H, W, Cout), np.nan, np.float32)
    gpu.acfun_conv2d_relu(P(x), N, H, W, Cin, P(w), P(b), 3, 3, Cout, 1, 1, P(got))
    _check_images(got, x, w, b, Cout, WINO_TOL)


# Images of at most 4 x 4 tiles (5 to 8 pixels a side; ResNet-50's 7 x 7 stage)
# run F(2,3) units of two images' 4 x 4-tile blocks: an odd image count leaves
# the last unit's second block empty, and a single image is a unit by itself.
@pytest.mark.parametrize("N,H,W,Cin,Cout", [(6, 7, 7, 64, 96), (5, 8, 8, 32, 40), (3, 5, 6, 36, 32),
                                            (1, 7, 7, 512, 64)])
def test_wino23_small_images(gpu, rng, N, H, W, Cin, Cout):
    x = rng.uniform(0, 1, (N, H, W, Cin)).astype(np.float32)
    w = (rng.standard_normal((9 * Cin, Cout)) * np.sqrt(2 / (9 * Cin))).astype(np.float32)
    b = (rng.standard_normal(Cout) * 0.01).astype(np.float32)
    got = np.full((N, H, W, Cout), np.nan, np.float32)
    gpu.acfun_conv2d_relu(P(x), N, H, W, Cin, P(w), P(b), 3, 3, Cout, 1, 1, P(got))
    _check_images(got, x, w, b, Cout, WINO_TOL)
    again = np.full_like(got, np.nan)
    gpu.acfun_conv2d_relu(P(x), N, H, W, Cin, P(w), P(b), 3, 3, Cout, 1, 1, P(again))
    assert_bitexact(again, got, "repeat run")


# 8-wide F(2,3) units (images 12 to 22 pixels wide): ResNet-50's 28 x 28 stage
# (1024 units, more than the persistent grid) and a ragged 36 -> 72 conv.
@pytest.mark.parametrize("N,HW,Cin,Cout", [(32, 28, 128, 128), (5, 22, 36, 72)])
def test_wino23_narrow(gpu, rng, N, HW, Cin, Cout):
    x = rng.uniform(0, 1, (N, HW, HW, Cin)).astype(np.float32)
    w = (rng.standard_normal((9 * Cin, Cout)) * np.sqrt(2 / (9 * Cin))).astype(np.float32)
    b = (rng.standard_normal(Cout) * 0.01).astype(np.float32)
    got = np.full((N, HW, HW, Cout), np.nan, np.float32)
    gpu.acfun_conv2d_relu(P(x), N, HW, HW, Cin, P(w), P(b), 3, 3, Cout, 1, 1, P(got))
    _check_images(got, x, w, b, Cout, WINO_TOL, step=8)


def test_config4a_full_exact(gpu, rng):
    """Depthwise 3x3/2 (BN folded, ReLU) then 3x3/2 MaxPool at config 4a size."""
    N, H, C = 32, 112, 96
    x = rng.uniform(0, 1, (N, H, H, C)).astype(np.float32)
    w = (rng.standard_normal((C, 3, 3)) * 0.3).astype(np.float32)
    gamma, beta = rng.uniform(0.5, 1.5, C).astype(np.float32), (rng.standard_normal(C) * 0.1).astype(np.float32)
    mean, var = (rng.standard_normal(C) * 0.1).astype(np.float32), rng.uniform(0.5, 1.5, C).astype(np.float32)
    wf, bf = oracle.fold_bn(w, None, C, C, mean, var, gamma, beta)
    wf = wf.reshape(C, 3, 3)
    y = np.zeros((N, 56, 56, C), np.float32)
    gpu.acfun_conv2d_dw(P(x), N, H, H, C, P(wf), P(bf), 3, 3, 2, 1, P(y), 1)
    want_y = oracle.conv2d_dw(x, wf, bf, 3, 3, 2, 1, 1)
    assert_bitexact(y, want_y, "cfg4a depthwise")
    z = np.zeros((N, 28, 28, C), np.float32)
    gpu.acfun_maxpool(P(y), N, 56, 56, C, 3, 2, 1, P(z))
    assert_bitexact(z, oracle.maxpool(want_y, 3, 2, 1, 0), "cfg4a maxpool")


# ------------------------------------------------------------------ device pointers
def test_device_pointer_variants(gpu, rng):
    torch = pytest.importorskip("torch")
    dev = torch.device("cuda:0")
    x, wq, ws, b = int8_conv_inputs(rng, 2, 14, 14, 64, 3, 3, 32)
    want = oracle.conv2d_int8(x, wq, ws, b, 3, 3, 32, 1, 1, 1)
    tx, tw, ts, tb = (torch.from_numpy(a).to(dev) for a in (x, wq, ws, b))
    ty = torch.full((2, 14, 14, 32), float("nan"), device=dev)
    # NULL: the library's own stream, which does not wait for torch's null
    # stream -- so the operands are made complete first
    stream = None
    torch.cuda.synchronize()
    rc = gpu.acfun_dev_conv2d_int8(tx.data_ptr(), 2, 14, 14, 64, tw.data_ptr(), ts.data_ptr(),
                                   tb.data_ptr(), 3, 3, 32, 1, 1, ty.data_ptr(), 1, stream)
    torch.cuda.synchronize()
    assert rc == 0
    assert_bitexact(ty.cpu().numpy(), want, "dev conv2d_int8")
    # host entry point given device pointers runs in place
    ty2 = torch.zeros_like(ty)
    gpu.acfun_conv2d_int8(tx.data_ptr(), 2, 14, 14, 64, tw.data_ptr(), ts.data_ptr(), tb.data_ptr(),
                          3, 3, 32, 1, 1, 0.0, ty2.data_ptr(), 1)
    assert_bitexact(ty2.cpu().numpy(), want, "host entry with device pointers")
    A = torch.rand(300, 200, device=dev)
    B = torch.rand(200, 100, device=dev)
    Cm = torch.zeros(300, 100, device=dev)
    torch.cuda.synchronize()
    assert gpu.acfun_dev_gemm_epi(300, 100, 200, A.data_ptr(), B.data_ptr(), Cm.data_ptr(), None, 0,
                                  stream) == 0
    torch.cuda.synchronize()
    want = oracle.gemm_f64(A.cpu().numpy(), B.cpu().numpy())
    assert rel_err(Cm.cpu().numpy(), want) < GEMM_TOL
