"""GPU parity of the int8-in / int8-out convolution (acfun_dev_conv2d_int8_q:
s8 activations with a per-tensor scale in, s8 requantized per tensor out)
through the C ABI, against oracle_conv2d_int8_q, which
tests/test_oracle_pins.py pins to the reference's acfun_conv2d_int8 and
acfun_quantize_u8.  Bar: bit-exact s8 output and bit-exact output scale."""
import numpy as np
import pytest

import oracle
from acfun_amd import capi
from tests.helpers import assert_bitexact, int8_q_inputs

pytestmark = pytest.mark.gpu


def run_q(gpu, q, s_in, wq, ws, b, KH, KW, Cout, st, pd, act, rule):
    """One acfun_dev_conv2d_int8_q call on a dedicated stream; returns (out, s_out)."""
    import torch
    N, H, W, Cin = q.shape
    OH, OW = oracle.out_hw(H, W, KH, KW, st, pd)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        dq, dw, dws = (torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in (q, wq, ws))
        db = torch.from_numpy(b).cuda() if b is not None else None
        dsi = torch.tensor([float(s_in)], dtype=torch.float32, device="cuda")
        dso = torch.full((1,), float("nan"), device="cuda")
        dout = torch.full((N, OH, OW, Cout), 99, dtype=torch.int8, device="cuda")
        rc = gpu.acfun_dev_conv2d_int8_q(dq.data_ptr(), dsi.data_ptr(), N, H, W, Cin,
                                         dw.data_ptr(), dws.data_ptr(),
                                         db.data_ptr() if db is not None else None, KH, KW, Cout,
                                         st, pd, dout.data_ptr(), dso.data_ptr(), act, rule,
                                         s.cuda_stream)
        out, so = dout.cpu().numpy(), np.float32(dso.cpu().numpy()[0])
    s.synchronize()
    assert rc == 0, capi.last_error()
    return out, so


# (N, H, W, Cin, KH, KW, Cout, stride, pad): every int8 route, channel tails in
# and out (the padded-copy paths), batches on every route
CASES = [
    (2, 10, 12, 16, 3, 3, 24, 1, 1),      # Winograd route
    (2, 9, 9, 20, 3, 3, 19, 1, 1),        # Winograd, channel tails in and out
    (3, 28, 28, 128, 3, 3, 64, 1, 1),     # Winograd, 128-channel chunks
    (2, 14, 14, 32, 1, 1, 48, 1, 0),      # 1x1
    (4, 14, 14, 256, 1, 1, 100, 1, 0),    # 1x1, Cout tail
    (2, 12, 12, 3, 3, 3, 16, 1, 1),       # Cin 3 -> direct
    (3, 15, 15, 16, 3, 3, 32, 2, 1),      # im2col + GEMM, batch 3
    (2, 11, 11, 8, 1, 1, 16, 2, 0),       # 1x1 s2, K = 8 -> direct
    (2, 23, 23, 64, 3, 3, 128, 2, 1),     # 3x3/2, 64 channels (two taps per chunk)
    (1, 30, 30, 3, 7, 7, 64, 2, 3),       # 7x7/2 on 3 channels (conv1)
]


@pytest.mark.parametrize("shape", CASES)
@pytest.mark.parametrize("act,rule", [(0, 0), (1, 0), (1, 1)])
def test_conv2d_int8_q_exact(gpu, rng, shape, act, rule):
    N, H, W, Cin, KH, KW, Cout, st, pd = shape
    print("int8_q case", shape, act, rule, flush=True)
    q, s_in, _, wq, ws, b = int8_q_inputs(rng, N, H, W, Cin, KH, KW, Cout)
    got, so = run_q(gpu, q, s_in, wq, ws, b, KH, KW, Cout, st, pd, act, rule)
    want, sw = oracle.conv2d_int8_q(q, s_in, wq, ws, b, KH, KW, Cout, st, pd, act, rule)
    assert_bitexact(got, want, f"int8_q {shape}")
    assert so == sw, (so, sw)
    assert np.max(np.abs(got.astype(np.int32))) == 127      # the max maps to +-127


@pytest.mark.parametrize("shape", [(2, 9, 9, 20, 3, 3, 19, 1, 1), (2, 14, 14, 32, 1, 1, 40, 1, 0),
                                   (2, 9, 9, 64, 3, 3, 19, 1, 1)])   # (K = 576: the one-pass path)
@pytest.mark.parametrize("rule", [0, 1])
def test_conv2d_int8_q_nan_outputs(gpu, rng, shape, rule):
    """NaN biases (no activation) make whole output channels NaN: the output
    maximum skips them, and the requantization converts them as the reference's
    x86 code does (-128 by the RNE and add-then-truncate forms, 0 by lroundf's
    on the channels past N & ~15 under rule 1)."""
    N, H, W, Cin, KH, KW, Cout, st, pd = shape
    q, s_in, _, wq, ws, b = int8_q_inputs(rng, N, H, W, Cin, KH, KW, Cout)
    b[0] = np.nan
    b[Cout - 2] = np.nan                           # past Cout & ~15 for the 19-channel case
    got, so = run_q(gpu, q, s_in, wq, ws, b, KH, KW, Cout, st, pd, 0, rule)
    want, sw = oracle.conv2d_int8_q(q, s_in, wq, ws, b, KH, KW, Cout, st, pd, 0, rule)
    assert_bitexact(got, want, f"int8_q NaN {shape} rule {rule}")
    assert so == sw, (so, sw)


@pytest.mark.parametrize("KK,ci,co,pd", [(1, 256, 512, 0), (3, 128, 128, 1)])
def test_config3_int8_io_full_exact(gpu, rng, KK, ci, co, pd):
    """Configs 3a / 3b with int8 I/O at full size (N=32, 28x28): bit-exact."""
    q, s_in, _, wq, ws, b = int8_q_inputs(rng, 32, 28, 28, ci, KK, KK, co)
    got, so = run_q(gpu, q, s_in, wq, ws, b, KK, KK, co, 1, pd, 1, 0)
    want, sw = oracle.conv2d_int8_q(q, s_in, wq, ws, b, KK, KK, co, 1, pd, 1, 0)
    assert_bitexact(got, want, "cfg3 int8 I/O")
    assert so == sw


def test_int8_q_chain(gpu, rng):
    """Two layers chained on device: 1x1 (output rounded by the Winograd rule
    for its consumer) -> 3x3/s1 (rule 0); the s8 tensor and scale between
    them never leave the device, and both match the oracle's chain."""
    q0, s0, _, w1, ws1, b1 = int8_q_inputs(rng, 2, 14, 14, 64, 1, 1, 48)
    w2 = rng.integers(-127, 128, (9 * 48, 32)).astype(np.int8)
    ws2 = rng.uniform(0.005, 0.05, 32).astype(np.float32)
    b2 = (rng.standard_normal(32) * 0.01).astype(np.float32)
    q1, s1 = run_q(gpu, q0, s0, w1, ws1, b1, 1, 1, 48, 1, 0, 1, 1)
    o1, t1 = oracle.conv2d_int8_q(q0, s0, w1, ws1, b1, 1, 1, 48, 1, 0, 1, 1)
    assert_bitexact(q1, o1, "layer 1")
    assert s1 == t1
    q2, s2 = run_q(gpu, q1, s1, w2, ws2, b2, 3, 3, 32, 1, 1, 1, 0)
    o2, t2 = oracle.conv2d_int8_q(o1, t1, w2, ws2, b2, 3, 3, 32, 1, 1, 1, 0)
    assert_bitexact(q2, o2, "layer 2")
    assert s2 == t2


def test_int8_q_zero_input(gpu, rng):
    """s_in = 0 (an all-zero input): zero output and s_out = 0, no bias."""
    q = np.zeros((1, 8, 8, 16), np.int8)
    wq = rng.integers(-127, 128, (9 * 16, 16)).astype(np.int8)
    got, so = run_q(gpu, q, 0.0, wq, np.full(16, 0.01, np.float32),
                    np.full(16, 0.5, np.float32), 3, 3, 16, 1, 1, 1, 0)
    assert so == 0.0 and not np.any(got)


def test_int8_q_rejects_bad_rule(gpu, rng):
    import torch
    q = torch.zeros((1, 4, 4, 16), dtype=torch.int8, device="cuda")
    w = torch.zeros((16, 16), dtype=torch.int8, device="cuda")
    ws = torch.ones(16, device="cuda")
    sc = torch.ones(2, device="cuda")
    out = torch.zeros((1, 4, 4, 16), dtype=torch.int8, device="cuda")
    torch.cuda.synchronize()
    rc = gpu.acfun_dev_conv2d_int8_q(q.data_ptr(), sc.data_ptr(), 1, 4, 4, 16, w.data_ptr(),
                                     ws.data_ptr(), None, 1, 1, 16, 1, 0, out.data_ptr(),
                                     sc.data_ptr() + 4, 0, 7, None)
    assert rc == -1 and "out_rule" in capi.last_error()
