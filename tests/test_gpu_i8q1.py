"""GPU parity of k_i8q1, the float-input 1x1 int8 convolution that quantizes
its activations while staging them (no quantized tensor, no quantize pass),
through the C ABI, bit-exact against oracle.conv2d_int8 (the reference's
acfun_conv2d_int8, src/conv_int8.cpp:63-148).  Each case also checks, through
the library's kernel timing, which kernel ran: k_i8q1 for at most 64 output
channels and Cin up to 512 (rounded up to 16), the quantize pass and k_i8mm
otherwise.  One test runs tests/gpu_i8q1_forced.py in a child process with
ACFUN_I8Q1 forcing k_i8q1 onto every output width (several tiles per unit)."""
import ctypes as C
import os
import subprocess
import sys

import numpy as np
import pytest

import oracle
from tests.helpers import P, assert_bitexact, int8_conv_inputs

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

pytestmark = pytest.mark.gpu


def _ran(gpu, name):
    n = C.c_int(0)
    gpu.acfun_prof_kernel_ms(name, C.byref(n))
    return n.value


def _conv(gpu, x, wq, ws, b, Cout, act):
    N, H, W, Cin = x.shape
    got = np.full((N, H, W, Cout), np.nan, np.float32)
    gpu.acfun_prof_enable(1)
    try:
        gpu.acfun_conv2d_int8(P(x), N, H, W, Cin, P(wq), P(ws), P(b), 1, 1, Cout, 1, 0,
                              np.float32(0.5), P(got), act)
        ran = (_ran(gpu, b"k_i8q1"), _ran(gpu, b"k_quant16"))
    finally:
        gpu.acfun_prof_enable(0)
    return got, ran


# (N, H, W, Cin, Cout): pixel counts that leave a partial 64-row block, Cin
# below 16, not a multiple of 16 or 4 (element loads), 1 to 4 chunks of 128,
# the 512 limit and one past it, Cout below 64 and at it; wider outputs take
# the quantize pass and k_i8mm
CASES = [
    (1, 5, 7, 16, 8),
    (2, 9, 11, 3, 24),
    (1, 13, 13, 20, 61),
    (2, 14, 14, 64, 64),
    (1, 10, 10, 128, 33),
    (1, 8, 9, 200, 48),
    (2, 7, 7, 256, 64),
    (1, 6, 6, 512, 40),
    (1, 6, 6, 520, 40),
    (3, 28, 28, 96, 64),
    (1, 56, 56, 256, 64),
    (2, 7, 7, 256, 512),
    (1, 9, 7, 64, 65),
]


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("act", [0, 1])
def test_i8q1_exact(gpu, rng, case, act):
    N, H, W, Cin, Cout = case
    x, wq, ws, b = int8_conv_inputs(rng, N, H, W, Cin, 1, 1, Cout, bias=(act == 1))
    got, (q1, qp) = _conv(gpu, x, wq, ws, b, Cout, act)
    assert_bitexact(got, oracle.conv2d_int8(x, wq, ws, b, 1, 1, Cout, 1, 0, act), f"i8q1 {case}")
    fused = (Cin + 15) // 16 * 16 <= 512 and Cout <= 64
    assert (q1 > 0, qp > 0) == (fused, not fused), (q1, qp)


@pytest.mark.parametrize("case", [(2, 9, 11, 48, 40), (1, 7, 9, 130, 64), (1, 5, 8, 16, 3)])
def test_i8q1_general_floats(gpu, rng, case):
    """Normal-distributed activations (every rounding position, ties and
    values near the clamp), NaNs among them, a bias and ReLU."""
    N, H, W, Cin, Cout = case
    x = rng.standard_normal((N, H, W, Cin)).astype(np.float32)
    flat = x.reshape(-1)
    flat[rng.choice(flat.size, 7, replace=False)] = np.nan
    flat[3] = -flat[np.nanargmax(np.abs(flat))]           # the max magnitude, negated
    wq = rng.integers(-128, 128, size=(Cin, Cout)).astype(np.int8)
    ws = rng.uniform(0.005, 0.05, Cout).astype(np.float32)
    b = (rng.standard_normal(Cout) * 0.1).astype(np.float32)
    got, (q1, _) = _conv(gpu, x, wq, ws, b, Cout, 1)
    assert q1 > 0
    assert_bitexact(got, oracle.conv2d_int8(x, wq, ws, b, 1, 1, Cout, 1, 0, 1), f"i8q1 floats {case}")


def test_i8q1_zero_input(gpu):
    """An all-zero input gives 0 without the bias (src/conv_int8.cpp:78)."""
    x = np.zeros((1, 9, 9, 32), np.float32)
    wq = np.ones((32, 24), np.int8)
    ws = np.full(24, 0.01, np.float32)
    b = np.full(24, 3.0, np.float32)
    got, (q1, _) = _conv(gpu, x, wq, ws, b, 24, 1)
    assert q1 > 0
    assert np.all(got == 0.0) and not np.any(np.signbit(got))


@pytest.mark.parametrize("offset", [1, 4])
def test_i8q1_device_offsets(gpu, rng, offset):
    """Device operands at float offsets: x and the output rows lose their
    16-byte alignment at offset 1 (element loads and stores), keep it at 4."""
    torch = pytest.importorskip("torch")
    dev = torch.device("cuda:0")
    N, H, W, Cin, Cout = 2, 11, 13, 64, 36
    x, wq, ws, b = int8_conv_inputs(rng, N, H, W, Cin, 1, 1, Cout)
    want = oracle.conv2d_int8(x, wq, ws, b, 1, 1, Cout, 1, 0, 1)
    xb = torch.zeros(x.size + offset, device=dev)
    xb[offset:] = torch.from_numpy(x.reshape(-1)).to(dev)
    tw, ts, tb = (torch.from_numpy(a).to(dev) for a in (wq, ws, b))
    yb = torch.full((want.size + offset,), float("nan"), device=dev)
    torch.cuda.synchronize()
    gpu.acfun_prof_enable(1)
    try:
        rc = gpu.acfun_dev_conv2d_int8(xb.data_ptr() + 4 * offset, N, H, W, Cin, tw.data_ptr(),
                                       ts.data_ptr(), tb.data_ptr(), 1, 1, Cout, 1, 0,
                                       yb.data_ptr() + 4 * offset, 1, None)
        torch.cuda.synchronize()
        q1 = _ran(gpu, b"k_i8q1")
    finally:
        gpu.acfun_prof_enable(0)
    assert rc == 0 and q1 > 0
    got = yb.cpu().numpy()[offset:].reshape(want.shape)
    assert_bitexact(got, want, f"i8q1 offset {offset}")


@pytest.mark.parametrize("setting", ["4,3,2", "8,2,3", "1,4,2"])
def test_i8q1_forced_all_widths(setting):
    """k_i8q1 forced onto every output width (units of several 64-column
    tiles, partial tile groups, 2 to 4 weight stages, 2 or 3 workgroups per
    CU), bit-exact, in a child process (the setting is read once per process)."""
    env = dict(os.environ, ACFUN_I8Q1=setting)
    r = subprocess.run([sys.executable, os.path.join(ROOT, "tests", "gpu_i8q1_forced.py")], env=env,
                       capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-3000:]
    assert "ok" in r.stdout.splitlines()[-1], r.stdout[-2000:]
