"""Child process of tests/test_gpu_tune.py (run as a script, one GPU process).

  python tests/tune_replay.py search  -- runs one shape of each tile-search
      family, checks it against the oracle, runs acfun_autotune(), checks the
      cache file ($ACFUN_TUNE_CACHE) and the results again with the searched
      choices;
  python tests/tune_replay.py forced  -- runs shapes to which the cache file
      (written by the parent) assigns every candidate of every family, and
      checks each result against the oracle: every choice the search can make
      computes the same result, including -1 (the search kept the built-in
      choice).

Prints one line per step and "tune ok" at the end; exits non-zero on failure."""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from acfun_amd import capi  # noqa: E402
from tests.helpers import P, int8_conv_inputs, rel_err  # noqa: E402

GEMM_TOL, WINO_TOL = 1e-4, 1e-3

# (kind, shape) -> the cases the forced mode assigns to candidate c: shapes are
# distinct per candidate so one cache file carries all assignments
G32_GEMM = [(96 + 32 * c, 160, 256 + 64 * c) for c in range(11)]         # M, N, K
G32_CONV = [(2, 15 + c, 13, 64, 3, 3, 40, 2, 1) for c in range(11)]        # N,H,W,Cin,KH,KW,Cout,s,p
I8 = [(2, 10 + c, 12, 64, 3, 3, 48, 2, 1) for c in range(5)]              # strided: the GEMM route
W23 = [(0, 2, 40, 36 + 2 * c, 32, 40) for c in range(4)] + [(4, 3, 7, 7, 64, 32)] + \
      [(c, 3, 18, 20, 24, 32) for c in (2, 3)]                             # cand, N, H, W, Cin, Cout
F32 = [(70 + c, 36, 301) for c in range(16)]                               # K % 4 != 0 -> k_gemm_f32
F32_KEPT = (86, 36, 301)         # cached as -1: the search kept the built-in choice


def gemm_case(L, rng, M, N, K):
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    Cm = np.full((M, N), np.nan, np.float32)
    L.acfun_gemm(M, N, K, P(A), P(B), P(Cm))
    return rel_err(Cm, A.astype(np.float64) @ B.astype(np.float64)), "gemm %dx%dx%d" % (M, N, K)


def gemm_ragged_case(L, rng, M, N, K):
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    Cm = np.full((M, N), np.nan, np.float32)
    L.acfun_gemm(M, N, K, P(A), P(B), P(Cm))
    return rel_err(Cm, A.astype(np.float64) @ B.astype(np.float64)), "gemm(f32) %dx%dx%d" % (M, N, K)


def conv_case(L, rng, N, H, W, Cin, KH, KW, Cout, s, p, tol_name="conv"):
    x = rng.uniform(0, 1, (N, H, W, Cin)).astype(np.float32)
    w = (rng.standard_normal((KH * KW * Cin, Cout)) * np.sqrt(2 / (KH * KW * Cin))).astype(np.float32)
    b = (rng.standard_normal(Cout) * 0.01).astype(np.float32)
    OH, OW = oracle.out_hw(H, W, KH, KW, s, p)
    got = np.full((N, OH, OW, Cout), np.nan, np.float32)
    L.acfun_conv2d_relu(P(x), N, H, W, Cin, P(w), P(b), KH, KW, Cout, s, p, P(got))
    want = oracle.conv2d_f64(x, w, b, KH, KW, Cout, s, p, 1, 1)
    return rel_err(got, want), "%s %s" % (tol_name, (N, H, W, Cin, KH, KW, Cout, s, p))


def int8_case(L, rng, N, H, W, Cin, KH, KW, Cout, s, p):
    x, wq, ws, b = int8_conv_inputs(rng, N, H, W, Cin, KH, KW, Cout)
    OH, OW = oracle.out_hw(H, W, KH, KW, s, p)
    got = np.full((N, OH, OW, Cout), np.nan, np.float32)
    L.acfun_conv2d_int8(P(x), N, H, W, Cin, P(wq), P(ws), P(b), KH, KW, Cout, s, p, np.float32(0.0),
                        P(got), 1)
    want = oracle.conv2d_int8(x, wq, ws, b, KH, KW, Cout, s, p, 1)
    return (0.0 if np.array_equal(got.view(np.uint32), want.view(np.uint32)) else 1.0), \
        "int8 %s" % ((N, H, W, Cin, KH, KW, Cout, s, p),)


def check(err, what, tol):
    print(what, "err %.3g" % err, flush=True)
    if not err < tol:
        print("FAILED", what, flush=True)
        sys.exit(1)


def run_all(L, rng, forced):
    for M, N, K in (G32_GEMM if forced else G32_GEMM[:1]):
        check(*gemm_case(L, rng, M, N, K), GEMM_TOL)
    for c in (G32_CONV if forced else G32_CONV[:1]):
        check(*conv_case(L, rng, *c), GEMM_TOL)
    for c in (I8 if forced else I8[:1]):
        check(*int8_case(L, rng, *c), 0.5)
    for c, N, H, W, Cin, Cout in (W23 if forced else W23[:1]):
        check(*conv_case(L, rng, N, H, W, Cin, 3, 3, Cout, 1, 1, "wino23[cand %d]" % c), WINO_TOL)
    for M, N, K in (F32 + [F32_KEPT] if forced else F32[:1]):
        check(*gemm_ragged_case(L, rng, M, N, K), GEMM_TOL)


def main():
    mode = sys.argv[1]
    cache = os.environ["ACFUN_TUNE_CACHE"]
    L = capi.lib()
    if L.acfun_backend() != 4:
        print("no gfx950 device:", capi.last_error())
        sys.exit(1)
    rng = np.random.default_rng(7)
    if mode == "search":
        run_all(L, rng, False)
        L.acfun_autotune()
        status = L.acfun_tune_status().decode()
        print("status:", status, flush=True)
        if "shapes searched" not in status or "cached at" not in status:
            sys.exit(1)
        lines = open(cache).read().split("\n")
        kinds = {ln.split()[1] for ln in lines if ln.strip()}
        arches = {ln.split()[0] for ln in lines if ln.strip()}
        print("cache kinds", sorted(kinds), "arches", sorted(arches), flush=True)
        if not {"g32", "i8mm", "w23", "f32"} <= kinds or arches != {"gfx950"}:
            sys.exit(1)
        run_all(L, rng, False)            # the searched choices give the same results
    else:
        run_all(L, rng, True)
    # every case above ran with its cached (searched or assigned) choice
    status = L.acfun_tune_status().decode()
    hits = int(status.rsplit("; ", 1)[1].split()[0])
    need = 5 if mode == "search" else len(G32_GEMM) + len(G32_CONV) + len(I8) + len(W23) + len(F32) + 1
    print("status:", status, "(need %d)" % need, flush=True)
    if hits < need:
        sys.exit(1)
    print("tune ok", flush=True)


if __name__ == "__main__":
    main()
