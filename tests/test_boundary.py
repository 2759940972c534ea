"""The drop-in boundary on the CPU: libacfun_amd.so loads, exports every entry
point include/acfun/acfun.h declares (the reference's 27 public functions with
the internal ones its tests bind), and fails loudly -- an error string, no
output written -- when there is no GPU.  No compute calls are made here."""
import ctypes as C
import os
import re
import shutil
import subprocess

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


_QUALS = {"const", "struct", "unsigned", "signed"}


def prototypes(path):
    """{name: (return type, [argument types])} of every acfun_* declaration,
    with parameter names dropped and pointer spacing normalised."""
    text = re.sub(r"/\*.*?\*/", "", open(path).read(), flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    out = {}
    for ret, name, args in re.findall(r"([A-Za-z_][\w\s\*]*?)\b(acfun_\w+)\s*\(([^)]*)\)\s*;",
                                      text):
        def norm(t):
            t = re.sub(r"\s*\*\s*", "*", " ".join(t.split()))
            return t.replace("*", " *").strip()
        types = []
        for a in [x.strip() for x in args.split(",")]:
            if a in ("", "void"):
                continue
            toks = re.findall(r"\w+|\*", a)
            if len(toks) > 1 and re.match(r"\w+$", toks[-1]) and toks[-1] not in _QUALS:
                toks = toks[:-1]                  # drop the parameter name
            types.append(norm(" ".join(toks)))
        out[name] = (norm(ret.split(";")[-1].split("}")[-1]), types)
    return out


def test_prototypes_match_reference():
    """Every function of the reference's public header (include/acfun/acfun.h:15-148)
    is declared here with the same return type and argument types, in order."""
    if not os.path.exists(REF_HEADER):
        pytest.skip("reference header not present")
    ours, theirs = prototypes(HEADER), prototypes(REF_HEADER)
    assert len(theirs) == 27, sorted(theirs)
    for name, proto in theirs.items():
        assert ours.get(name) == proto, (name, ours.get(name), proto)
    # spot checks that the parser keeps what matters
    assert theirs["acfun_conv2d_int8"][1][5] == "const int8_t *"
    assert theirs["acfun_model_load"] == ("AcfunModel *", ["const char *"])
    assert theirs["acfun_relu"][1] == ["float *", "size_t"]


def build_c_caller(tmpdir):
    """Compiles tests/c_abi/abi_check.c, a C99 caller that includes
    include/acfun/acfun.h and links libacfun_amd.so; returns its path."""
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    exe = os.path.join(str(tmpdir), "abi_check")
    src = os.path.join(ROOT, "tests", "c_abi", "abi_check.c")
    libdir = os.path.dirname(capi.LIB_PATH)
    subprocess.run([cc, "-std=c99", "-Wall", "-Werror", "-O1", "-I", os.path.join(ROOT, "include"),
                    src, "-L", libdir, "-lacfun_amd", "-Wl,-rpath," + libdir, "-lm", "-o", exe],
                   check=True)
    return exe


def test_c_caller_builds_and_fails_loudly_without_gpu(tmp_path):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present (tests/test_gpu_parity.py runs the caller on it)")
    exe = build_c_caller(tmp_path)
    r = subprocess.run([exe, "nogpu"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "abi ok" in r.stdout


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
