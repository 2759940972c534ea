"""GPU parity of the F(4,3) unit kernel (k_wino43p) through the C ABI: the
explicit acfun_winograd43_conv3x3 entry and the conv route's F(4,3) step,
against the f64 direct convolution (oracle.conv2d_f64), within the Winograd
tolerance 1e-3 (relative to the output's largest magnitude).  Each case also
checks, through the library's kernel timing, that k_wino43p is what ran."""
import ctypes as C

import numpy as np
import pytest

import oracle
from tests.helpers import P, rel_err

pytestmark = pytest.mark.gpu

WINO_TOL = 1e-3


def _ran_wino43(gpu):
    n = C.c_int(0)
    gpu.acfun_prof_kernel_ms(b"k_wino43", C.byref(n))
    return n.value


def _conv(gpu, fn, x, w, b, Cout, act):
    N, H, W, Cin = x.shape
    got = np.full((N, H, W, Cout), np.nan, np.float32)
    gpu.acfun_prof_enable(1)
    try:
        if fn == "route":
            if act:
                gpu.acfun_conv2d_relu(P(x), N, H, W, Cin, P(w), P(b), 3, 3, Cout, 1, 1, P(got))
            else:
                gpu.acfun_conv2d(P(x), N, H, W, Cin, P(w), P(b), 3, 3, Cout, 1, 1, P(got))
        else:
            gpu.acfun_winograd43_conv3x3(P(x), N, H, W, Cin, P(w), P(b), Cout, P(got), act)
        ran = _ran_wino43(gpu)
    finally:
        gpu.acfun_prof_enable(0)
    return got, ran


# (fn, N, H, W, Cin, Cout): tile rows and columns that do not fill a unit,
# channel counts that are not multiples of 8 (in) or 32 (out), several chunk
# counts, more units than workgroups, and the route's shapes (H, W >= 112)
CASES = [
    ("entry", 1, 24, 24, 32, 32),
    ("entry", 1, 30, 26, 36, 40),       # ragged input chunk, partial output block
    ("entry", 2, 25, 70, 20, 8),        # Cin 20 (4 chunks), Cout 8
    ("entry", 3, 41, 37, 128, 96),      # 16 chunks, 3 output blocks
    ("entry", 2, 28, 64, 64, 33),       # Cout not a multiple of 4
    ("entry", 1, 33, 29, 64, 256),
    ("route", 1, 112, 112, 64, 64),
    ("route", 1, 113, 115, 64, 72),
    ("route", 4, 120, 112, 96, 64),
]


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("act", [0, 1])
def test_wino43_unit_kernel(gpu, rng, case, act):
    fn, N, H, W, Cin, Cout = case
    print("wino43 case", case, act, flush=True)
    x = rng.uniform(0, 1, (N, H, W, Cin)).astype(np.float32)
    w = (rng.standard_normal((9 * Cin, Cout)) * np.sqrt(2 / (9 * Cin))).astype(np.float32)
    b = (rng.standard_normal(Cout) * 0.1).astype(np.float32)
    got, ran = _conv(gpu, fn, x, w, b, Cout, act)
    assert ran > 0, "k_wino43p did not run"
    want = oracle.conv2d_f64(x, w, b, 3, 3, Cout, 1, 1, 1, act)
    assert not np.isnan(got).any()
    assert rel_err(got, want) < WINO_TOL, rel_err(got, want)


def test_wino43_repeatable(gpu, rng):
    """Two runs of the same call give the same bits (no dependence on
    workgroup timing)."""
    x = rng.uniform(0, 1, (2, 64, 64, 64)).astype(np.float32)
    w = (rng.standard_normal((9 * 64, 64)) * 0.06).astype(np.float32)
    b = (rng.standard_normal(64) * 0.1).astype(np.float32)
    a, _ = _conv(gpu, "entry", x, w, b, 64, 1)
    c, _ = _conv(gpu, "entry", x, w, b, 64, 1)
    assert np.array_equal(a, c)
