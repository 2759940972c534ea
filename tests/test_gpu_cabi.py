"""The C ABI from C: tests/c_abi/abi_check.c includes include/acfun/acfun.h,
links libacfun_amd.so like any user of the reference's API would, and runs a
GEMM (exact on integer-valued operands) and a fused conv+ReLU on the GPU."""
import subprocess

import pytest

from tests.test_boundary import build_c_caller

pytestmark = pytest.mark.gpu


def test_c_caller_on_gpu(gpu, tmp_path):
    exe = build_c_caller(tmp_path)
    print("running", exe, "gpu", flush=True)
    r = subprocess.run([exe, "gpu"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "abi ok (MI355X-gfx950)" in r.stdout, r.stdout
