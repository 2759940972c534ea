"""Child process of tests/test_gpu_i8q1.py::test_i8q1_forced_all_widths: with
ACFUN_I8Q1 forcing k_i8q1 onto every output width, 1x1 int8 convolutions of
several output tiles are bit-exact against oracle.conv2d_int8 and ran k_i8q1.
Prints the case before each call and "ok" at the end."""
import ctypes as C
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from acfun_amd import capi  # noqa: E402
from tests.helpers import P, assert_bitexact, int8_conv_inputs  # noqa: E402

# (N, H, W, Cin, Cout): more tiles than a unit groups, partial tile groups and
# columns, 1 to 4 chunks, element loads
CASES = [(2, 7, 7, 256, 512), (1, 9, 7, 64, 1000), (1, 10, 10, 128, 130), (3, 28, 28, 96, 200),
         (1, 6, 6, 512, 100), (2, 9, 11, 3, 70), (1, 13, 13, 20, 300)]


def main():
    gpu = capi.lib()
    rng = np.random.default_rng(11)
    for case in CASES:
        for act in (0, 1):
            N, H, W, Cin, Cout = case
            print("case", os.environ.get("ACFUN_I8Q1"), case, act, flush=True)
            x, wq, ws, b = int8_conv_inputs(rng, N, H, W, Cin, 1, 1, Cout, bias=(act == 1))
            got = np.full((N, H, W, Cout), np.nan, np.float32)
            gpu.acfun_prof_enable(1)
            gpu.acfun_conv2d_int8(P(x), N, H, W, Cin, P(wq), P(ws), P(b), 1, 1, Cout, 1, 0,
                                  np.float32(0.5), P(got), act)
            n = C.c_int(0)
            gpu.acfun_prof_kernel_ms(b"k_i8q1", C.byref(n))
            gpu.acfun_prof_enable(0)
            assert n.value > 0, f"k_i8q1 did not run for {case}"
            assert_bitexact(got, oracle.conv2d_int8(x, wq, ws, b, 1, 1, Cout, 1, 0, act), f"forced {case}")
    print("ok", flush=True)


if __name__ == "__main__":
    main()
