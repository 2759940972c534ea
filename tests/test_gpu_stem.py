"""GPU parity of k_conv_smallc (k_stem.hip), the few-input-channel convolution
of a network's stem (the reference's im2col + GEMM route, src/layers.cpp:178-194,
for 7x7 and 3x3 kernels on 3 channels), through the C ABI against the f64 direct
convolution (oracle.conv2d_f64) within the fp32 GEMM tolerance 1e-4 (relative
to the output's largest magnitude); and of its int8 form k_i8stem
(acfun_conv2d_int8, src/conv_int8.cpp:63-148), bit-exact against
oracle.conv2d_int8.  Each case also checks, through the
library's kernel timing, that k_conv_smallc ran -- or, for rows of W*Cin not a
multiple of 4 floats and inputs not 16-byte aligned (which its 16-byte window
DMA needs), that the general implicit GEMM did."""
import ctypes as C

import numpy as np
import pytest

import oracle
from tests.helpers import P, assert_bitexact, int8_conv_inputs, rel_err

pytestmark = pytest.mark.gpu

GEMM_TOL = 1e-4


def _conv(gpu, x, w, b, KH, KW, Cout, s, p, act):
    N, H, W, Cin = x.shape
    OH, OW = oracle.out_hw(H, W, KH, KW, s, p)
    got = np.full((N, OH, OW, Cout), np.nan, np.float32)
    gpu.acfun_prof_enable(1)
    try:
        if act:
            gpu.acfun_conv2d_relu(P(x), N, H, W, Cin, P(w), P(b), KH, KW, Cout, s, p, P(got))
        else:
            gpu.acfun_conv2d(P(x), N, H, W, Cin, P(w), P(b), KH, KW, Cout, s, p, P(got))
        n = C.c_int(0)
        gpu.acfun_prof_kernel_ms(b"k_conv_smallc", C.byref(n))
    finally:
        gpu.acfun_prof_enable(0)
    return got, n.value


# (N, H, W, KH, Cout, stride, pad): the ResNet-50 stem at full size, ragged
# images whose 64-pixel tiles span two or more output rows, Cout past one
# 64-channel tile (two and three channel tiles) and below 32, stride 1 and 2,
# pad 0; W = 30 and 35 (W*3 not a multiple of 4) take the general kernel
CASES = [
    (1, 224, 224, 7, 64, 2, 3),
    (2, 32, 28, 7, 64, 2, 3),
    (3, 33, 36, 7, 70, 2, 3),
    (1, 19, 20, 7, 16, 2, 0),
    (2, 17, 20, 3, 32, 1, 1),
    (2, 64, 64, 3, 24, 2, 1),
    (1, 9, 12, 3, 130, 1, 1),
    (4, 40, 36, 3, 64, 1, 0),
    (2, 30, 30, 7, 64, 2, 3),
    (1, 13, 35, 3, 20, 1, 1),
]


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("act", [0, 1])
def test_stem_conv(gpu, rng, case, act):
    N, H, W, K, Cout, s, p = case
    x = rng.uniform(0, 1, (N, H, W, 3)).astype(np.float32)
    w = (rng.standard_normal((K * K * 3, Cout)) * np.sqrt(2 / (K * K * 3))).astype(np.float32)
    b = (rng.standard_normal(Cout) * 0.01).astype(np.float32) if act else None
    got, ran = _conv(gpu, x, w, b, K, K, Cout, s, p, act)
    assert (ran > 0) == (W % 4 == 0)
    want = oracle.conv2d_f64(x, w, b, K, K, Cout, s, p, 1, act)
    assert rel_err(got, want) < GEMM_TOL, rel_err(got, want)


def test_stem_special_values(gpu, rng):
    """An infinite input makes every output it reaches infinite or NaN as the
    f64 reference does (no padding product turns an inf into a NaN), and a NaN
    input reaches exactly the outputs whose windows hold it."""
    N, H, W, K, Cout, s, p = 1, 20, 24, 7, 64, 2, 3
    x = rng.uniform(0, 1, (N, H, W, 3)).astype(np.float32)
    x[0, 5, 7, 1] = np.inf
    x[0, 14, 3, 2] = np.nan
    w = (np.abs(rng.standard_normal((K * K * 3, Cout))) * 0.1 + 0.01).astype(np.float32)
    b = (rng.standard_normal(Cout) * 0.01).astype(np.float32)
    got, ran = _conv(gpu, x, w, b, K, K, Cout, s, p, 0)
    assert ran > 0
    want = oracle.conv2d_f64(x, w, b, K, K, Cout, s, p, 1, 0)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isinf(got), np.isinf(want))
    fin = np.isfinite(want)
    assert rel_err(got[fin], want[fin]) < GEMM_TOL


def test_stem_unaligned_input_takes_general_kernel(gpu, rng):
    """A device input one float past 16-byte alignment: the general implicit
    GEMM runs, with the same result within tolerance."""
    torch = pytest.importorskip("torch")
    dev = torch.device("cuda:0")
    N, H, W, K, Cout, s, p = 2, 32, 32, 7, 64, 2, 3
    x = rng.uniform(0, 1, (N, H, W, 3)).astype(np.float32)
    w = (rng.standard_normal((K * K * 3, Cout)) * 0.1).astype(np.float32)
    b = (rng.standard_normal(Cout) * 0.01).astype(np.float32)
    want = oracle.conv2d_f64(x, w, b, K, K, Cout, s, p, 1, 1)
    for off in (0, 1):
        xb = torch.zeros(x.size + 4, device=dev)
        xb[off:off + x.size] = torch.from_numpy(x.reshape(-1)).to(dev)
        tw, tb = torch.from_numpy(w).to(dev), torch.from_numpy(b).to(dev)
        y = torch.full(want.shape, float("nan"), device=dev)
        torch.cuda.synchronize()
        gpu.acfun_prof_enable(1)
        try:
            rc = gpu.acfun_dev_conv2d(xb.data_ptr() + 4 * off, N, H, W, 3, tw.data_ptr(), tb.data_ptr(), K, K,
                                      Cout, s, p, 1, y.data_ptr(), 1, None)
            torch.cuda.synchronize()
            n = C.c_int(0)
            gpu.acfun_prof_kernel_ms(b"k_conv_smallc", C.byref(n))
        finally:
            gpu.acfun_prof_enable(0)
        assert rc == 0
        assert (n.value > 0) == (off == 0)
        assert rel_err(y.cpu().numpy(), want) < GEMM_TOL


def _conv_i8(gpu, x, wq, ws, b, KH, Cout, s, p, act):
    N, H, W, Cin = x.shape
    OH, OW = oracle.out_hw(H, W, KH, KH, s, p)
    got = np.full((N, OH, OW, Cout), np.nan, np.float32)
    gpu.acfun_prof_enable(1)
    try:
        gpu.acfun_conv2d_int8(P(x), N, H, W, Cin, P(wq), P(ws), P(b), KH, KH, Cout, s, p, np.float32(0.5),
                              P(got), act)
        n = C.c_int(0)
        gpu.acfun_prof_kernel_ms(b"k_i8stem", C.byref(n))
    finally:
        gpu.acfun_prof_enable(0)
    return got, n.value


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("act", [0, 1])
def test_stem_int8_exact(gpu, rng, case, act):
    N, H, W, K, Cout, s, p = case
    x, wq, ws, b = int8_conv_inputs(rng, N, H, W, 3, K, K, Cout, bias=(act == 1))
    got, ran = _conv_i8(gpu, x, wq, ws, b, K, Cout, s, p, act)
    assert (ran > 0) == (W % 4 == 0)
    assert_bitexact(got, oracle.conv2d_int8(x, wq, ws, b, K, K, Cout, s, p, act), f"int8 stem {case}")


def test_stem_int8_special_inputs(gpu, rng):
    """Normal-distributed activations with NaNs (the x86 conversion's rule: s8
    -128) and the maximum magnitude negated; then an all-zero input, which
    gives 0 without the bias (src/conv_int8.cpp:78)."""
    N, H, W, K, Cout, s, p = 2, 40, 44, 7, 64, 2, 3
    x = rng.standard_normal((N, H, W, 3)).astype(np.float32)
    flat = x.reshape(-1)
    flat[rng.choice(flat.size, 9, replace=False)] = np.nan
    flat[5] = -flat[np.nanargmax(np.abs(flat))]
    wq = rng.integers(-128, 128, size=(K * K * 3, Cout)).astype(np.int8)
    ws = rng.uniform(0.005, 0.05, Cout).astype(np.float32)
    b = (rng.standard_normal(Cout) * 0.1).astype(np.float32)
    got, ran = _conv_i8(gpu, x, wq, ws, b, K, Cout, s, p, 1)
    assert ran > 0
    assert_bitexact(got, oracle.conv2d_int8(x, wq, ws, b, K, K, Cout, s, p, 1), "int8 stem floats")
    z = np.zeros((1, 16, 16, 3), np.float32)
    got, ran = _conv_i8(gpu, z, wq, ws, np.full(Cout, 3.0, np.float32), K, Cout, s, p, 1)
    assert ran > 0
    assert np.all(got == 0.0) and not np.any(np.signbit(got))
