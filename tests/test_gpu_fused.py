"""GPU parity of the fused pairs through the C ABI: acfun_dev_conv2d_dw_maxpool
(depthwise conv + activation, then MaxPool, in one kernel) against the
oracle's depthwise conv followed by its maxpool -- the two reference calls
(acfun_conv2d_dw, acfun_maxpool(_relu)) -- and acfun_dev_conv2d_g_maxpool
(grouped conv + activation, then MaxPool) against the oracle's grouped conv
and maxpool (acfun_conv2d_g, acfun_maxpool(_relu)); all pinned bit-exact in
tests/test_oracle_pins.py.  Bar: bit-exact, NaN propagation included."""
import numpy as np
import pytest

import oracle
from acfun_amd import capi
from tests.helpers import assert_bitexact

pytestmark = pytest.mark.gpu


def run_dwpool(gpu, x, w, b, stride, pad, act, ppad, post_relu):
    import torch
    N, H, W, C = x.shape
    OH, OW = oracle.out_hw(H, W, 3, 3, stride, pad)
    PH, PW = oracle.out_hw(OH, OW, 3, 3, 2, ppad)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        dx, dw = torch.from_numpy(x).cuda(), torch.from_numpy(np.ascontiguousarray(w)).cuda()
        db = torch.from_numpy(b).cuda()
        dy = torch.full((N, PH, PW, C), 7.0, device="cuda")
        rc = gpu.acfun_dev_conv2d_dw_maxpool(dx.data_ptr(), N, H, W, C, dw.data_ptr(),
                                             db.data_ptr(), 3, 3, stride, pad, act, 3, 2, ppad,
                                             dy.data_ptr(), post_relu, s.cuda_stream)
        out = dy.cpu().numpy()
    s.synchronize()
    assert rc == 0, capi.last_error()
    return out


def want_dwpool(x, w, b, stride, pad, act, ppad, post_relu):
    y = oracle.conv2d_dw(x, w, b, 3, 3, stride, pad, act)
    return oracle.maxpool(y, 3, 2, ppad, post_relu)


# (N, H, W, C, stride, pad, act, pool pad, post_relu)
CASES = [
    (2, 17, 19, 32, 2, 1, 1, 1, 0),
    (1, 28, 30, 96, 2, 1, 1, 1, 1),
    (2, 15, 15, 20, 1, 1, 0, 1, 0),      # 5 channel quads: a partial quad group
    (1, 9, 40, 64, 1, 1, 1, 0, 1),       # pool pad 0; 19 pool columns: two column blocks
    (3, 6, 6, 8, 2, 0, 1, 1, 0),         # tiny: most pool windows clipped
    (1, 57, 45, 48, 2, 1, 1, 1, 0),      # odd sizes
    (2, 12, 12, 6, 2, 1, 1, 1, 0),       # C % 4 != 0: the two-kernel path
    (2, 37, 26, 24, 2, 1, 1, 0, 1),      # stride 2, pool pad 0: 3 strips, the middle one walks up
    (1, 40, 18, 12, 2, 0, 0, 0, 0),      # conv pad 0, 9 lanes per strip padded to a wave
]


@pytest.mark.parametrize("shape", CASES)
def test_dw_maxpool_exact(gpu, rng, shape):
    N, H, W, C, st, pd, act, ppad, pr = shape
    print("dw+pool case", shape, flush=True)
    x = rng.standard_normal((N, H, W, C)).astype(np.float32)
    w = (rng.standard_normal((C, 3, 3)) * 0.3).astype(np.float32)
    b = (rng.standard_normal(C) * 0.1).astype(np.float32)
    assert_bitexact(run_dwpool(gpu, x, w, b, st, pd, act, ppad, pr),
                    want_dwpool(x, w, b, st, pd, act, ppad, pr), f"dw+pool {shape}")


def test_dw_maxpool_nan(gpu, rng):
    """NaN inputs propagate as max_ps propagates them (the pool skips
    out-of-range taps rather than comparing against a sentinel)."""
    x = rng.standard_normal((1, 16, 16, 16)).astype(np.float32)
    x[0, 3, 5, 2] = np.nan
    x[0, 0, 0, 7] = np.nan
    x[0, 15, 15, 11] = np.nan
    w = (rng.standard_normal((16, 3, 3)) * 0.3).astype(np.float32)
    b = np.zeros(16, np.float32)
    for act, pr in ((0, 0), (1, 1)):
        got = run_dwpool(gpu, x, w, b, 1, 1, act, 1, pr)
        want = want_dwpool(x, w, b, 1, 1, act, 1, pr)
        assert np.isnan(want).any() or act
        assert_bitexact(got, want, f"NaN act={act}")


@pytest.mark.parametrize("st", [1, 2])
def test_dw_maxpool_nan_partial_vec(gpu, rng, st):
    """C = 20: the pool compares channels 16..19 with the scalar rule (v > m),
    not max_ps; with NaNs the two differ, and the fused kernels keep both."""
    x = rng.standard_normal((2, 14, 15, 20)).astype(np.float32)
    x[0, 3, 4, 17] = np.nan
    x[1, 7, 8, 18] = np.nan
    x[0, 9, 9, 2] = np.nan
    w = (rng.standard_normal((20, 3, 3)) * 0.3).astype(np.float32)
    b = np.zeros(20, np.float32)
    for act, pr in ((0, 0), (0, 1)):
        assert_bitexact(run_dwpool(gpu, x, w, b, st, 1, act, 1, pr),
                        want_dwpool(x, w, b, st, 1, act, 1, pr), f"C=20 NaN s{st} act={act} pr={pr}")


@pytest.mark.parametrize("C", [16, 20])
def test_dw_maxpool_nan_strips(gpu, rng, C):
    """Stride 2 over 3 strips of 4 pooled rows (the row-streaming kernel's
    unit): NaNs in each strip, at strip boundaries and in the halo rows the
    strips share, with full (C = 16) and partial (C = 20) max_ps channel
    groups."""
    x = rng.standard_normal((2, 41, 22, C)).astype(np.float32)
    for (n, r, c, ch) in ((0, 3, 4, 1), (0, 15, 7, 2), (0, 16, 8, C - 1), (1, 17, 9, 3),
                          (1, 24, 20, C - 2), (0, 31, 0, 0), (1, 33, 21, C - 3), (0, 40, 5, 5)):
        x[n, r, c, ch] = np.nan
    w = (rng.standard_normal((C, 3, 3)) * 0.3).astype(np.float32)
    b = (rng.standard_normal(C) * 0.1).astype(np.float32)
    for act, pr in ((0, 0), (1, 0), (0, 1)):
        assert_bitexact(run_dwpool(gpu, x, w, b, 2, 1, act, 1, pr),
                        want_dwpool(x, w, b, 2, 1, act, 1, pr), f"strips C={C} act={act} pr={pr}")


def test_config4a_fused_full_exact(gpu, rng):
    """Config 4(a) at full size: depthwise 3x3/2 (BN folded) + ReLU, then
    MaxPool 3x3/2 pad 1 -- one kernel, bit-exact against the two reference ops."""
    N, H, C = 32, 112, 96
    x = rng.uniform(0, 1, (N, H, H, C)).astype(np.float32)
    w = (rng.standard_normal((C, 3, 3)) * 0.3).astype(np.float32)
    gamma, beta = rng.uniform(0.5, 1.5, C).astype(np.float32), (rng.standard_normal(C) * 0.1).astype(np.float32)
    mean, var = (rng.standard_normal(C) * 0.1).astype(np.float32), rng.uniform(0.5, 1.5, C).astype(np.float32)
    wf, bf = oracle.fold_bn(w, None, C, C, mean, var, gamma, beta)
    wf = wf.reshape(C, 3, 3)
    assert_bitexact(run_dwpool(gpu, x, wf, bf, 2, 1, 1, 1, 0),
                    want_dwpool(x, wf, bf, 2, 1, 1, 1, 0), "cfg4a fused")


def run_gpool(gpu, x, w, b, Cout, stride, pad, groups, act, ppad, post_relu):
    import torch
    N, H, W, Cin = x.shape
    OH, OW = oracle.out_hw(H, W, 3, 3, stride, pad)
    PH, PW = oracle.out_hw(OH, OW, 3, 3, 2, ppad)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        dx, dw = torch.from_numpy(x).cuda(), torch.from_numpy(np.ascontiguousarray(w)).cuda()
        db = torch.from_numpy(b).cuda()
        dy = torch.full((N, PH, PW, Cout), 7.0, device="cuda")
        rc = gpu.acfun_dev_conv2d_g_maxpool(dx.data_ptr(), N, H, W, Cin, dw.data_ptr(), db.data_ptr(),
                                            3, 3, Cout, stride, pad, groups, act, 3, 2, ppad,
                                            dy.data_ptr(), post_relu, s.cuda_stream)
        out = dy.cpu().numpy()
    s.synchronize()
    assert rc == 0, capi.last_error()
    return out


def want_gpool(x, w, b, Cout, stride, pad, groups, act, ppad, post_relu):
    y = oracle.conv2d_grouped(x, w, b, 3, 3, Cout, stride, pad, groups, act)
    return oracle.maxpool(y, 3, 2, ppad, post_relu)


# (N, H, W, Cin, Cout, groups, stride, pad, act, pool pad, post_relu)
GCASES = [
    (32, 14, 14, 24, 48, 6, 1, 1, 1, 1, 0),     # config 4(b)
    (2, 15, 13, 32, 64, 4, 1, 1, 1, 0, 1),      # 8 input channels per group, pool pad 0
    (3, 11, 12, 12, 36, 3, 2, 1, 1, 1, 0),      # stride 2, 12 output channels per group
    (2, 9, 9, 16, 128, 4, 1, 1, 0, 1, 1),       # 32 output channels per group, no activation
    (1, 10, 10, 12, 12, 3, 1, 1, 1, 1, 0),      # 4 output channels per group: the two-kernel path
    (1, 60, 58, 16, 64, 2, 1, 1, 1, 1, 1),      # image too large for LDS: one lane per pooled quad
    (2, 41, 40, 24, 48, 6, 2, 1, 1, 0, 0),      # stride 2, pool pad 0 (row kernel)
    (1, 8, 8, 128, 512, 32, 1, 1, 1, 1, 0),     # rows of all groups too large for LDS: per image x group
    (2, 5, 5, 24, 48, 6, 1, 0, 1, 1, 1),        # conv pad 0: 3 x 3 conv output, 2 x 2 pooled
]


@pytest.mark.parametrize("shape", GCASES)
def test_g_maxpool_exact(gpu, rng, shape):
    N, H, W, Cin, Cout, g, st, pd, act, ppad, pr = shape
    print("gconv+pool case", shape, flush=True)
    x = rng.standard_normal((N, H, W, Cin)).astype(np.float32)
    w = (rng.standard_normal((g, 9 * (Cin // g), Cout // g)) * 0.3).astype(np.float32)
    b = (rng.standard_normal(Cout) * 0.1).astype(np.float32)
    assert_bitexact(run_gpool(gpu, x, w, b, Cout, st, pd, g, act, ppad, pr),
                    want_gpool(x, w, b, Cout, st, pd, g, act, ppad, pr), f"gconv+pool {shape}")


def test_g_maxpool_nan(gpu, rng):
    x = rng.standard_normal((1, 12, 12, 24)).astype(np.float32)
    x[0, 2, 3, 1] = np.nan
    x[0, 11, 0, 17] = np.nan
    w = (rng.standard_normal((6, 36, 8)) * 0.3).astype(np.float32)
    b = np.zeros(48, np.float32)
    for act, pr in ((0, 0), (1, 1)):
        assert_bitexact(run_gpool(gpu, x, w, b, 48, 1, 1, 6, act, 1, pr),
                        want_gpool(x, w, b, 48, 1, 1, 6, act, 1, pr), f"gconv NaN act={act}")
