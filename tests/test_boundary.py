"""The drop-in boundary on the CPU: libacfun_amd.so loads, exports every entry
point include/acfun/acfun.h declares (the reference's 27 public functions with
the internal ones its tests bind), and fails loudly -- an error string, no
output written -- when there is no GPU.  No compute calls are made here."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from acfun_amd import capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "acfun", "acfun.h")
REF_HEADER = "/root/reference/include/acfun/acfun.h"


def declared(path):
    text = re.sub(r"/\*.*?\*/", "", open(path).read(), flags=re.S)
    return sorted(set(re.findall(r"\b(acfun_\w+)\s*\(", text)))


def test_header_declares_reference_api():
    names = declared(HEADER)
    assert len(names) >= 27
    if os.path.exists(REF_HEADER):
        missing = set(declared(REF_HEADER)) - set(names)
        assert not missing, missing


def test_library_exports_every_declared_symbol():
    L = C.CDLL(capi.LIB_PATH)
    missing = [n for n in declared(HEADER) if not hasattr(L, n)]
    assert not missing, missing
    assert set(declared(HEADER)) <= set(capi.SIGNATURES), \
        set(declared(HEADER)) - set(capi.SIGNATURES)


def test_fails_loudly_without_gpu():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    L = capi.lib()
    assert L.acfun_backend() == 0
    assert L.acfun_backend_name() == b"none"
    A = np.ones((4, 4), np.float32)
    out = np.full((4, 4), 7.0, np.float32)
    L.acfun_gemm(4, 4, 4, A.ctypes.data, A.ctypes.data, out.ctypes.data)
    assert np.all(out == 7.0)            # nothing written, no silent CPU fallback
    assert "device" in capi.last_error()
    assert L.acfun_model_load(b"/nonexistent.acfun") is None
