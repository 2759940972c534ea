"""The tile search on the GPU (acfun_autotune; tune.cpp), in child processes
(tests/tune_replay.py) with their own cache file:
  - search: one shape of each family (k_gemm32 GEMM and implicit-GEMM conv,
    k_i8mm, the F(2,3) unit kernels, k_gemm_f32) runs, is searched against its
    built-in choice (adopting a candidate only past a 3% margin), cached under
    the device's arch and each family's name, and still matches the oracle
    with the searched choices;
  - forced: a cache file assigns every candidate of every family to a shape;
    each result matches the oracle (fp32 within 1e-4 / Winograd 1e-3, int8 bit
    for bit), and every case ran with its assigned choice; choice -1 (the
    built-in one kept by the search) loads and runs as well."""
import os
import subprocess
import sys

import pytest

import oracle
from tests import tune_replay as R

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
AM_C64 = 2          # k_i8mm's addressing mode for 64-channel inputs


def _child(mode, cache):
    env = dict(os.environ, ACFUN_TUNE_CACHE=str(cache))
    env.pop("ACFUN_AUTOTUNE", None)
    print("tune child", mode, flush=True)
    r = subprocess.run([sys.executable, "-u", os.path.join(ROOT, "tests", "tune_replay.py"), mode],
                       capture_output=True, text=True, timeout=300, env=env, cwd=ROOT)
    assert r.returncode == 0 and "tune ok" in r.stdout, r.stdout[-3000:] + r.stderr[-3000:]
    return r.stdout


def test_tile_search_caches_and_keeps_parity(gpu, tmp_path):
    out = _child("search", tmp_path / "tune.txt")
    lines = (tmp_path / "tune.txt").read_text().split("\n")
    assert all(ln.split()[0] == "gfx950" for ln in lines if ln.strip()), out


def _forced_cache():
    lines = []
    for c, (M, N, K) in enumerate(R.G32_GEMM):
        lines.append(f"gfx950 g32 11 0,{M},{N},{K} {c}")
    for c, (N, H, W, Cin, KH, KW, Cout, s, p) in enumerate(R.G32_CONV):
        OH, OW = oracle.out_hw(H, W, KH, KW, s, p)
        lines.append(f"gfx950 g32 11 1,{N * OH * OW},{Cout},{KH * KW * Cin},{H},{W},{Cin},{KW},{s},{p},{OH},{OW} {c}")
    for c, (N, H, W, Cin, KH, KW, Cout, s, p) in enumerate(R.I8):
        OH, OW = oracle.out_hw(H, W, KH, KW, s, p)
        Cinp = (Cin + 15) // 16 * 16
        lines.append(f"gfx950 i8mm 5 {AM_C64},{N * OH * OW},{Cout},{KH * KW * Cinp},{H},{W},{Cinp},{KW},"
                     f"{s},{p},{OH},{OW} {c}")
    for c, N, H, W, Cin, Cout in R.W23:
        lines.append(f"gfx950 w23 5 {N},{H},{W},{Cin},{Cout} {c}")
    for c, (M, N, K) in enumerate(R.F32):
        lines.append(f"gfx950 f32 16 {M},{N},{K} {c}")
    M, N, K = R.F32_KEPT
    lines.append(f"gfx950 f32 16 {M},{N},{K} -1")
    return "\n".join(lines) + "\n"


def test_every_candidate_keeps_parity(gpu, tmp_path):
    cache = tmp_path / "forced.txt"
    cache.write_text(_forced_cache())
    _child("forced", cache)
