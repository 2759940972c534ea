"""acfun_dev_conv2d_int8_noalloc (the allocation-free entry point, temporaries
in a 64 MiB static device region) against acfun_dev_conv2d_int8 through the C
ABI: bit-exact on two calls in a row, the second smaller, on each int8 route;
and a shape past the region is refused with an error, writing nothing."""
import numpy as np
import pytest

from acfun_amd import capi
from tests.helpers import int8_conv_inputs

pytestmark = pytest.mark.gpu

LIMIT = 64 << 20

# (N, H, W, Cin, KH, KW, Cout, stride, pad): a larger call, then a smaller one
PAIRS = [
    ((8, 28, 28, 256, 1, 1, 512, 1, 0), (2, 14, 14, 256, 1, 1, 128, 1, 0)),      # 1x1
    ((8, 28, 28, 128, 3, 3, 128, 1, 1), (1, 9, 11, 20, 3, 3, 8, 1, 1)),          # Winograd
    ((4, 30, 30, 64, 3, 3, 96, 2, 1), (1, 13, 13, 24, 7, 7, 8, 2, 3)),           # im2col + GEMM
    ((2, 20, 20, 3, 3, 3, 16, 1, 1), (1, 8, 8, 2, 3, 3, 5, 1, 0)),               # direct
]


def _need(N, H, W, Cin, KH, KW, Cout):
    a = lambda b: (b + 255) // 256 * 256
    cinp = (Cin + 15) // 16 * 16
    ldb = (KH * KW * cinp + 127) // 128 * 128
    return a(Cout * ldb) + a(Cout * 4) + a(520 * 4) + a(N * H * W * cinp)


def _run(gpu, fn, shape, x, wq, ws, b, act):
    """One call on a dedicated (non-null) torch stream: the operands are made,
    the entry point queued and the result read back all on that stream.  (A
    NULL stream argument means the library's own stream, which torch's null
    stream does not wait for.)"""
    import torch
    N, H, W, Cin, KH, KW, Cout, st, pd = shape
    OH, OW = (H + 2 * pd - KH) // st + 1, (W + 2 * pd - KW) // st + 1
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        dx, dq, dws = (torch.from_numpy(a).cuda() for a in (x, wq, ws))
        db = torch.from_numpy(b).cuda() if b is not None else None
        dy = torch.full((N, OH, OW, Cout), float("nan"), device="cuda")
        assert s.cuda_stream != 0
        rc = fn(dx.data_ptr(), N, H, W, Cin, dq.data_ptr(), dws.data_ptr(),
                db.data_ptr() if db is not None else None, KH, KW, Cout, st, pd, dy.data_ptr(),
                act, s.cuda_stream)
        out = dy.cpu().numpy()
    s.synchronize()
    return rc, out


@pytest.mark.parametrize("first,second", PAIRS)
def test_noalloc_matches_allocating_entry(gpu, rng, first, second):
    for shape, act in ((first, 1), (second, 0)):
        N, H, W, Cin, KH, KW, Cout, st, pd = shape
        assert _need(N, H, W, Cin, KH, KW, Cout) <= LIMIT
        print("noalloc case", shape, act, flush=True)
        x, wq, ws, b = int8_conv_inputs(rng, N, H, W, Cin, KH, KW, Cout)
        rc0, want = _run(gpu, gpu.acfun_dev_conv2d_int8, shape, x, wq, ws, b, act)
        rc1, got = _run(gpu, gpu.acfun_dev_conv2d_int8_noalloc, shape, x, wq, ws, b, act)
        assert rc0 == 0 and rc1 == 0, capi.last_error()
        assert not np.any(np.isnan(want))
        np.testing.assert_array_equal(got, want)


def test_noalloc_refuses_oversized_shape(gpu, rng):
    import torch
    shape = (90, 56, 56, 256, 1, 1, 64, 1, 0)           # 72 MB of quantized activations
    N, H, W, Cin, KH, KW, Cout, st, pd = shape
    assert _need(N, H, W, Cin, KH, KW, Cout) > LIMIT
    dx = torch.zeros((N, H, W, Cin), device="cuda")
    dq = torch.zeros((Cin, Cout), dtype=torch.int8, device="cuda")
    dws = torch.ones(Cout, device="cuda")
    dy = torch.full((N, H, W, Cout), 7.0, device="cuda")
    torch.cuda.synchronize()
    rc = gpu.acfun_dev_conv2d_int8_noalloc(dx.data_ptr(), N, H, W, Cin, dq.data_ptr(),
                                           dws.data_ptr(), None, KH, KW, Cout, st, pd,
                                           dy.data_ptr(), 0, None)
    assert gpu.acfun_sync() == 0
    torch.cuda.synchronize()
    assert rc == -1
    assert "static region" in capi.last_error()
    assert bool(torch.all(dy == 7.0))
