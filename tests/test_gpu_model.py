"""GPU parity of the ACFUN0 model path (loader fusion + executor, model.cpp)
through the C ABI: against the compiled reference's own executor on version-1
models, against the oracle executor (tests/test_model_pins.py pins it to the
reference) on version-2 residual models and on the int8 mode.

Bars: int8 convolution chains bit-exact; fp32 models within the Winograd
tolerance 1e-3 (normwise, on the model output)."""
import ctypes as C

import numpy as np
import pytest

import oracle
import oracle.model as omodel
from acfun_amd import acfun0, capi
from tests import models
from tests.helpers import P, assert_bitexact, rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _write(tmp_path, name, inC, H, W, recs, version):
    path = str(tmp_path / name)
    acfun0.write(path, inC, H, W, recs, version=version)
    return path


def _infer_each(lib, m, x):
    outs = []
    for img in x:
        y = np.full(1 << 16, np.nan, np.float32)
        n = lib.acfun_model_infer(m, P(np.ascontiguousarray(img)), P(y))
        assert n > 0, capi.last_error()
        outs.append(y[:n].copy())
    return np.stack(outs)


def _load(lib, path, flags=0):
    m = lib.acfun_model_load_ex(path.encode(), flags)
    assert m, capi.last_error()
    return m


def test_model_v1_matches_reference(gpu, ref, rng, tmp_path):
    inC, H, W, recs = models.fusion_v1(rng)
    path = _write(tmp_path, "fusion.acfun", inC, H, W, recs, 1)
    x = rng.uniform(-1, 1, (3, H, W, inC)).astype(np.float32)
    mr = ref.acfun_model_load(path.encode())
    want = _infer_each(ref, mr, x)
    ref.acfun_model_destroy(mr)
    m = gpu.acfun_model_load(path.encode())
    assert m, capi.last_error()
    try:
        assert gpu.acfun_model_output_size(m) == 0       # as the reference: known after infer
        dims = [C.c_int(0), C.c_int(0), C.c_int(0)]
        gpu.acfun_model_input_dims(m, *[C.byref(d) for d in dims])
        assert [d.value for d in dims] == [inC, H, W]
        got = _infer_each(gpu, m, x)
        assert gpu.acfun_model_output_size(m) == want.shape[1]
    finally:
        gpu.acfun_model_destroy(m)
    assert got.shape == want.shape
    assert rel_err(got, want) < TOL, rel_err(got, want)


def test_model_batch_equals_single(gpu, rng, tmp_path):
    inC, H, W, recs = models.fusion_v1(rng)
    path = _write(tmp_path, "fusion.acfun", inC, H, W, recs, 1)
    x = rng.uniform(-1, 1, (4, H, W, inC)).astype(np.float32)
    m = _load(gpu, path)
    try:
        single = _infer_each(gpu, m, x)
        batch = np.full_like(single, np.nan)
        assert gpu.acfun_model_infer_batch(m, 4, P(x), P(batch)) == single.shape[1]
    finally:
        gpu.acfun_model_destroy(m)
    assert rel_err(batch, single) < 1e-5, rel_err(batch, single)


def test_model_device_batch(gpu, rng, tmp_path):
    import torch
    inC, H, W, recs = models.fusion_v1(rng)
    path = _write(tmp_path, "fusion.acfun", inC, H, W, recs, 1)
    x = rng.uniform(-1, 1, (3, H, W, inC)).astype(np.float32)
    m = _load(gpu, path)
    try:
        host = np.full((3, 10), np.nan, np.float32)
        assert gpu.acfun_model_infer_batch(m, 3, P(x), P(host)) == 10
        s = torch.cuda.Stream()               # non-null: NULL would mean the library's stream
        with torch.cuda.stream(s):
            dx = torch.from_numpy(x).cuda()
            dy = torch.full((3, 10), float("nan"), device="cuda")
            assert gpu.acfun_dev_model_infer_batch(m, 3, dx.data_ptr(), dy.data_ptr(),
                                                   s.cuda_stream) == 10
        s.synchronize()
    finally:
        gpu.acfun_model_destroy(m)
    assert_bitexact(dy.cpu().numpy(), host, "device vs host batch")


def test_model_v2_residual_matches_oracle(gpu, rng, tmp_path):
    inC, H, W, recs = models.small_resnet_v2(rng)
    path = _write(tmp_path, "res.acfun", inC, H, W, recs, 2)
    x = rng.uniform(0, 1, (2, H, W, inC)).astype(np.float32)
    m = _load(gpu, path)
    try:
        got = np.full((2, 10), np.nan, np.float32)
        assert gpu.acfun_model_infer_batch(m, 2, P(x), P(got)) == 10, capi.last_error()
    finally:
        gpu.acfun_model_destroy(m)
    want = omodel.run(open(path, "rb").read(), x)
    assert rel_err(got, want) < TOL, rel_err(got, want)


def test_model_int8_chain_exact(gpu, rng, tmp_path):
    """int8 mode (flags=1): every dense conv quantized at load, run through the
    acfun_conv2d_int8 rules with the batch's dynamic activation scale."""
    inC, H, W, recs = models.int8_chain_v1(rng)
    path = _write(tmp_path, "i8.acfun", inC, H, W, recs, 1)
    for n in (1, 3):
        x = rng.uniform(0, 1, (n, H, W, inC)).astype(np.float32)
        want = omodel.run(open(path, "rb").read(), x, int8=True)
        m = _load(gpu, path, 1)
        try:
            got = np.full(want.shape, np.nan, np.float32)
            assert gpu.acfun_model_infer_batch(m, n, P(x), P(got)) == want.shape[1]
        finally:
            gpu.acfun_model_destroy(m)
        assert_bitexact(got, want, f"int8 chain, batch {n}")


def test_model_rejects_truncated_file(gpu, rng, tmp_path):
    inC, H, W, recs = models.fusion_v1(rng)
    blob = acfun0.encode(inC, H, W, recs, version=1)
    for cut in (10, 30, len(blob) // 2, len(blob) - 4):
        path = str(tmp_path / f"cut{cut}.acfun")
        with open(path, "wb") as f:
            f.write(blob[:cut])
        assert not gpu.acfun_model_load(path.encode())
        assert capi.last_error()
    assert not gpu.acfun_model_load(str(tmp_path / "missing.acfun").encode())


@pytest.mark.parametrize("int8", [False, True])
def test_resnet50_224_matches_oracle(gpu, rng, tmp_path, int8):
    """Config 5's full graph (ResNet-50-style v1.5, 224x224) on one image."""
    inC, H, W, recs = acfun0.resnet50(np.random.default_rng(5))
    path = _write(tmp_path, "r50.acfun", inC, H, W, recs, 2)
    x = rng.uniform(0, 1, (1, H, W, inC)).astype(np.float32)
    m = _load(gpu, path, 1 if int8 else 0)
    try:
        got = np.full((1, 1000), np.nan, np.float32)
        assert gpu.acfun_model_infer_batch(m, 1, P(x), P(got)) == 1000, capi.last_error()
    finally:
        gpu.acfun_model_destroy(m)
    want = omodel.run(open(path, "rb").read(), x, int8=int8)
    assert rel_err(got, want) < TOL, rel_err(got, want)
    assert abs(float(got.sum()) - 1.0) < 1e-4


@pytest.mark.parametrize("int8", [True, False])
def test_resnet50_headless_batch8(gpu, rng, tmp_path, int8):
    """Config 5's graph without its head (the output is the last block's
    Add+ReLU, 7 x 7 x 2048 per image) at batch 8.  int8: bit-exact against the
    oracle's chain of acfun_conv2d_int8 calls on the whole batch (one dynamic
    activation scale per tensor over the 8 images), which covers the fused
    residual epilogue and the producer-to-consumer absmax handoff of every
    block; fp32 within the Winograd tolerance."""
    inC, H, W, recs = acfun0.resnet50(np.random.default_rng(5), head=False)
    path = _write(tmp_path, "r50h.acfun", inC, H, W, recs, 2)
    n = 8
    x = rng.uniform(0, 1, (n, H, W, inC)).astype(np.float32)
    m = _load(gpu, path, 1 if int8 else 0)
    try:
        got = np.full((n, 7 * 7 * 2048), np.nan, np.float32)
        assert gpu.acfun_model_infer_batch(m, n, P(x), P(got)) == got.shape[1], capi.last_error()
    finally:
        gpu.acfun_model_destroy(m)
    print("oracle ResNet-50 batch", n, "int8" if int8 else "fp32", flush=True)
    want = omodel.run(open(path, "rb").read(), x, int8=int8)
    assert np.count_nonzero(want) > want.size // 4          # ReLU leaves a live tensor
    if int8:
        assert_bitexact(got, want, "int8 ResNet-50 body, batch 8")
    else:
        assert rel_err(got, want) < TOL, rel_err(got, want)


def test_model_winograd_cache_repeats(gpu, rng, tmp_path):
    """A 3x3 conv whose model keeps its F(2,3) filter transform from the first
    inference, at config 2(a)'s size (32 x 56 x 56 x 64, more units than the
    persistent unit kernel has workgroups): three inferences in a row give the
    entry point's bits on the same weights."""
    C, HW, N = 64, 56, 32
    w = acfun0.conv_weight(rng, 3, 3, C, C)
    b = (rng.standard_normal(C) * 0.1).astype(np.float32)
    path = _write(tmp_path, "wino.acfun", C, HW, HW, [("conv", 3, 3, C, 1, 1, w, b)], 1)
    x = rng.uniform(0, 1, (N, HW, HW, C)).astype(np.float32)
    want = np.full((N, HW, HW, C), np.nan, np.float32)
    gpu.acfun_conv2d(P(x), N, HW, HW, C, P(w.reshape(9 * C, C)), P(b), 3, 3, C, 1, 1, P(want))
    assert rel_err(want[:1], oracle.conv2d_f64(np.ascontiguousarray(x[:1]), w.reshape(9 * C, C), b, 3, 3, C, 1, 1)) < TOL
    m = _load(gpu, path)
    try:
        for i in range(3):
            got = np.full((N, HW, HW, C), np.nan, np.float32)
            assert gpu.acfun_model_infer_batch(m, N, P(x), P(got)) == HW * HW * C, capi.last_error()
            assert_bitexact(got, want, f"model inference {i} vs acfun_conv2d")
    finally:
        gpu.acfun_model_destroy(m)



def test_model_layer_profile_tags(gpu, rng, tmp_path):
    """acfun_prof_report: every kernel a model launches carries its layer's
    index, every executed layer has a record with its shapes, and a launch
    outside the model is untagged."""
    inC, H, W, recs = acfun0.resnet50(rng, in_hw=32, width=8, blocks=(1, 1), classes=10)
    path = _write(tmp_path, "r.acfun", inC, H, W, recs, 2)
    m = _load(gpu, path)
    x = rng.uniform(0, 1, (2, H, W, inC)).astype(np.float32)
    y = np.zeros((2, 10), np.float32)
    try:
        assert gpu.acfun_model_infer_batch(m, 2, P(x), P(y)) == 10, capi.last_error()
        gpu.acfun_prof_enable(1)
        try:
            assert gpu.acfun_model_infer_batch(m, 2, P(x), P(y)) == 10, capi.last_error()
            A = rng.uniform(-1, 1, (64, 64)).astype(np.float32)
            Cm = np.zeros((64, 64), np.float32)
            gpu.acfun_gemm(64, 64, 64, P(A), P(A), P(Cm))
        finally:
            gpu.acfun_prof_enable(0)
        kernels, layers = capi.prof_report()
    finally:
        gpu.acfun_model_destroy(m)
    idx = {L["i"]: L for L in layers}
    assert layers and all(L["N"] == 2 for L in layers)
    tags = {t for (t, _) in kernels}
    assert -1 in tags                                    # the GEMM after the model
    assert tags - {-1} <= set(idx)                       # every tagged launch names a layer
    convs = [L for L in layers if L["type"] == 1 and L["fused_into"] == -2]
    assert convs and all(L["i"] in tags for L in convs)  # every conv launched its kernels
    first = idx[0]
    assert (first["H"], first["W"], first["C"], first["OC"], first["KH"], first["stride"]) == \
        (32, 32, 3, 8, 7, 2)
    assert all(n > 0 and ms > 0 for (n, ms) in kernels.values())


def test_resnet50_int8_head_batch3(gpu, rng, tmp_path):
    """Config 5's full graph in int8 mode at batch 3: the head (global pool,
    FC, softmax) after a body whose int8 convs use one activation scale over
    the batch, against the oracle's chain (Winograd tolerance: the FC runs on
    the fp32 GEMM engine)."""
    inC, H, W, recs = acfun0.resnet50(np.random.default_rng(5))
    path = _write(tmp_path, "r50.acfun", inC, H, W, recs, 2)
    n = 3
    x = rng.uniform(0, 1, (n, H, W, inC)).astype(np.float32)
    m = _load(gpu, path, 1)
    try:
        got = np.full((n, 1000), np.nan, np.float32)
        assert gpu.acfun_model_infer_batch(m, n, P(x), P(got)) == 1000, capi.last_error()
    finally:
        gpu.acfun_model_destroy(m)
    print("oracle ResNet-50 int8 with head, batch", n, flush=True)
    want = omodel.run(open(path, "rb").read(), x, int8=True)
    assert rel_err(got, want) < TOL, rel_err(got, want)
    assert np.allclose(got.sum(axis=1), 1.0, atol=1e-4)


@pytest.mark.parametrize("int8", [True, False])
def test_resnet50_b64_batch_permutation(gpu, rng, int8, tmp_path):
    """Config 5's body at the bench's batch of 64 (no oracle at this size): the
    batch-wide int8 activation scales are maxima over the batch, and every
    kernel's arithmetic per output element is independent of the image's place
    in the batch, so permuting the 64 input images permutes the outputs bit for
    bit (int8), and within 1e-6 (fp32)."""
    import torch
    inC, H, W, recs = acfun0.resnet50(np.random.default_rng(5), head=False)
    path = _write(tmp_path, "r50h.acfun", inC, H, W, recs, 2)
    n = 64
    x = torch.rand((n, H, W, inC), device="cuda", generator=torch.Generator(device="cuda").manual_seed(11))
    perm = torch.from_numpy(np.random.default_rng(2).permutation(n)).cuda()
    xp = x[perm].contiguous()
    y = torch.full((n, 7 * 7 * 2048), float("nan"), device="cuda")
    yp = torch.full_like(y, float("nan"))
    m = _load(gpu, path, 1 if int8 else 0)
    try:
        s = torch.cuda.current_stream().cuda_stream
        assert gpu.acfun_dev_model_infer_batch(m, n, x.data_ptr(), y.data_ptr(), s) == y.shape[1], capi.last_error()
        assert gpu.acfun_dev_model_infer_batch(m, n, xp.data_ptr(), yp.data_ptr(), s) == y.shape[1], capi.last_error()
        torch.cuda.synchronize()
    finally:
        gpu.acfun_model_destroy(m)
    a, b = y[perm].cpu().numpy(), yp.cpu().numpy()
    assert not np.isnan(a).any() and np.count_nonzero(a) > a.size // 4
    if int8:
        assert_bitexact(b, a, "int8 ResNet-50 body, batch 64 permuted")
    else:
        assert rel_err(b, a) < 1e-6, rel_err(b, a)


@pytest.mark.parametrize("int8", [True, False])
@pytest.mark.parametrize("head", [False, True])
def test_resnet50_b64_tiles_equal_batch8(gpu, rng, int8, head, tmp_path):
    """Config 5 at the bench's batch of 64, tied to the oracle-checked batch of
    8: the 64 images are 8 copies of 8 images, so every batch-wide int8
    activation scale (a maximum over the batch) equals the batch-8 run's, and
    each block of 8 outputs must reproduce the batch-8 outputs -- bit for bit
    for the int8 body, within 1e-5 where fp32 kernels may choose other tiles at
    the larger batch.  test_resnet50_headless_batch8 and
    test_resnet50_int8_head_batch3 check the small batches against the oracle."""
    import torch
    inC, H, W, recs = acfun0.resnet50(np.random.default_rng(5), head=head)
    path = _write(tmp_path, "r50t.acfun", inC, H, W, recs, 2)
    x8 = torch.rand((8, H, W, inC), device="cuda", generator=torch.Generator(device="cuda").manual_seed(13))
    x64 = x8.repeat(8, 1, 1, 1).contiguous()
    F = 1000 if head else 7 * 7 * 2048
    y8 = torch.full((8, F), float("nan"), device="cuda")
    y64 = torch.full((64, F), float("nan"), device="cuda")
    m = _load(gpu, path, 1 if int8 else 0)
    try:
        s = torch.cuda.current_stream().cuda_stream
        print("ResNet-50 batch 8 and batch 64 (8 copies), int8", int8, "head", head, flush=True)
        assert gpu.acfun_dev_model_infer_batch(m, 8, x8.data_ptr(), y8.data_ptr(), s) == F, capi.last_error()
        assert gpu.acfun_dev_model_infer_batch(m, 64, x64.data_ptr(), y64.data_ptr(), s) == F, capi.last_error()
        torch.cuda.synchronize()
    finally:
        gpu.acfun_model_destroy(m)
    a = y8.cpu().numpy()
    assert not np.isnan(a).any() and np.count_nonzero(a) > a.size // 4
    b = y64.cpu().numpy().reshape(8, 8, F)
    for k in range(8):
        if int8 and not head:
            assert_bitexact(b[k], a, f"int8 ResNet-50 body, batch 64, copy {k}")
        else:
            assert rel_err(b[k], a) < 1e-5, (k, rel_err(b[k], a))


def test_int8_model_per_image_flag(gpu, rng, tmp_path):
    """acfun_model_load_ex flag 2: an int8 model's batched call gives every
    image its own activation scales -- bit for bit the batch-1 call on that
    image, which test_resnet50_224_matches_oracle[int8] checks against the
    oracle -- while flag 1 alone shares them over the batch."""
    import torch
    inC, H, W, recs = acfun0.resnet50(np.random.default_rng(5), head=False)
    path = _write(tmp_path, "r50p.acfun", inC, H, W, recs, 2)
    n, F = 3, 7 * 7 * 2048
    x = torch.rand((n, H, W, inC), device="cuda", generator=torch.Generator(device="cuda").manual_seed(17))
    x[1] *= 4.0                              # one image's wider range moves a shared scale
    s = torch.cuda.current_stream().cuda_stream
    yb = torch.full((n, F), float("nan"), device="cuda")
    y1 = torch.full((n, F), float("nan"), device="cuda")
    yd = torch.full((n, F), float("nan"), device="cuda")
    print("ResNet-50 body, int8 per-image flag, batch", n, flush=True)
    m = _load(gpu, path, 3)
    try:
        assert gpu.acfun_dev_model_infer_batch(m, n, x.data_ptr(), yb.data_ptr(), s) == F, capi.last_error()
        for i in range(n):
            xi = x[i:i + 1].contiguous()
            assert gpu.acfun_dev_model_infer_batch(m, 1, xi.data_ptr(), y1[i].data_ptr(), s) == F, capi.last_error()
        torch.cuda.synchronize()
    finally:
        gpu.acfun_model_destroy(m)
    m = _load(gpu, path, 1)
    try:
        assert gpu.acfun_dev_model_infer_batch(m, n, x.data_ptr(), yd.data_ptr(), s) == F, capi.last_error()
        torch.cuda.synchronize()
    finally:
        gpu.acfun_model_destroy(m)
    a = y1.cpu().numpy()
    assert not np.isnan(a).any() and np.count_nonzero(a) > a.size // 4
    assert_bitexact(yb.cpu().numpy(), a, "int8 per-image batch against batch-1 calls")
    assert not np.array_equal(yd.cpu().numpy(), a)      # the shared scale changes the batch


def test_int8_model_uses_the_s8_chain(gpu, rng, tmp_path):
    """An int8 model passes a tensor whose only reader is another int8 conv as
    s8 with its device scale: its producer requantizes it (k_requant_s8) and the
    reader runs no quantizer, while tensors an Add or a projection also reads
    stay fp32.  The results are the oracle's bit for bit (the chain changes no
    value: test_resnet50_headless_batch8[int8] at full size)."""
    inC, H, W, recs = acfun0.resnet50(rng, in_hw=32, width=8, blocks=(2, 1), classes=10, head=False)
    path = _write(tmp_path, "r.acfun", inC, H, W, recs, 2)
    m = _load(gpu, path, 1)
    x = rng.uniform(0, 1, (2, H, W, inC)).astype(np.float32)
    n_out = 4 * 4 * 64                                   # 32 -> 16 (conv1) -> 8 (pool) -> 8 -> 4; 16 * 4 channels
    y = np.full((2, n_out), np.nan, np.float32)          # (the call writes N x its output size)
    try:
        gpu.acfun_prof_enable(1)
        try:
            assert gpu.acfun_model_infer_batch(m, 2, P(x), P(y)) == n_out, capi.last_error()
        finally:
            gpu.acfun_prof_enable(0)
        kernels, layers = capi.prof_report()
    finally:
        gpu.acfun_model_destroy(m)
    convs = [L["i"] for L in layers if L["type"] == 1 and L["fused_into"] == -2]
    per = {i: {k for (t, k) in kernels if t == i} for i in convs}
    producers = [i for i in convs if "k_requant_s8" in per[i]]
    readers = [i for i in convs if not per[i] & {"k_quant16", "k_absmax_prep"}]
    assert len(producers) >= 4, per                      # conv a -> b and b -> c in each of 3 blocks
    assert len(readers) >= len(producers), per
    want = omodel.run(open(path, "rb").read(), x, int8=True)
    assert_bitexact(y, want, "int8 chain")
