"""Benchmark of the MI355X convolution/GEMM path (one GPU).

Headline (the JSON line's metric/value): BASELINE config 2(a) -- fp32 NHWC 3x3
conv, stride 1, pad 1, bias + fused ReLU, N=32, 56x56, 64 -> 64 channels,
which the reference routes to Winograd F(2,3).  One step = one
acfun_dev_conv2d call over the whole batch, inputs resident in HBM.  value is
TFLOPS counted as direct convolution (2*N*OH*OW*Cout*9*Cin = 7.40 GFLOP), the
way the reference quotes conv throughput; roofline.achieved counts the FLOPs
the MFMA units actually execute for F(2,3) (2*tiles*16*Cin*Cout) over the
dominant kernel's time.

The other BASELINE configs are measured the same way and reported under
"configs" (GEMM 1024^3, F(4,3), the two int8 convs, depthwise+pool, grouped,
ResNet-50-style batch 64 fp32 and int8).  Configs 3 and 4 also report
"ms_cold": the same step cycling over copies of its input and output whose
total exceeds the 256 MB MALL, so the operands come from HBM ("ms" reuses one
set, which may stay cached).

cpu_baseline: the reference library itself (oracle/_ref, built from the
reference's sources) timed on this host's cores on the headline config:
3 warmups, then the median of the timed repetitions (src/benchmark.cpp:98-111).
"""
import argparse
import ctypes as C
import json
import os
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP32 = 157.3e12     # dense fp32 MFMA, FLOP/s
PEAK_INT8 = 5.0e15       # dense int8 MFMA, OP/s
PEAK_HBM = 8.0e12        # B/s


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--headline-only", action="store_true", help="skip the other configs")
    ap.add_argument("--traffic", action="store_true",
                    help="for rocprofv3 --pmc runs: 5 headline steps, then 3 plain copies of "
                         "256 MiB (the counter scale reference); prints no JSON line")
    return ap.parse_args()


class Timer:
    """HIP events on the stream the library launches on."""

    def __init__(self, torch, stream):
        self.torch, self.stream = torch, stream

    def run(self, fn, steps, warmup):
        torch = self.torch
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(self.stream)
        for _ in range(steps):
            fn()
        e1.record(self.stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps   # ms per step

    def kernel_ms(self, lib, fn, steps, kernel):
        """Mean duration (ms) of one library kernel over `steps` more steps: the
        library brackets each launch of it with a HIP event pair on its stream."""
        self.torch.cuda.synchronize()
        lib.acfun_prof_enable(1)
        for _ in range(steps):
            fn()
        self.torch.cuda.synchronize()
        lib.acfun_prof_enable(0)
        n = C.c_int(0)
        ms = lib.acfun_prof_kernel_ms(kernel.encode(), C.byref(n))
        return ms if n.value > 0 and ms > 0 else None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the path would shard by batch with no exchange between GPUs", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    from acfun_amd import acfun0, capi

    lib = capi.lib()
    if lib.acfun_backend() != 4:
        raise SystemExit("bench.py: no gfx950 device: " + capi.last_error())
    dev = torch.device("cuda:0")
    # A dedicated (default-priority) stream: the library queues its kernels on
    # the stream it is given, and the timing events are recorded on the same one.
    stream = torch.cuda.Stream(device=dev)
    torch.cuda.set_stream(stream)
    sp = stream.cuda_stream
    T = Timer(torch, stream)
    rng = np.random.default_rng(12345 + 1)

    def cuda(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev)

    def check(rc):
        if rc != 0:
            raise RuntimeError(capi.last_error())

    # ---------------------------------------------------------------- headline: config 2(a)
    N, H, Cin, Cout = 32, 56, 64, 64
    x = rng.uniform(0, 1, (N, H, H, Cin)).astype(np.float32)
    w = (rng.standard_normal((9 * Cin, Cout)) * np.sqrt(2.0 / (9 * Cin))).astype(np.float32)
    b = (rng.standard_normal(Cout) * 0.01).astype(np.float32)
    tx, tw, tb = cuda(x), cuda(w), cuda(b)
    ty = torch.empty((N, H, H, Cout), device=dev)

    def step():
        check(lib.acfun_dev_conv2d(tx.data_ptr(), N, H, H, Cin, tw.data_ptr(), tb.data_ptr(),
                                   3, 3, Cout, 1, 1, 1, ty.data_ptr(), 1, sp))

    if args.traffic:
        for _ in range(5):
            step()
        src = torch.empty(64 << 20, device=dev)        # 256 MiB
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        return

    ms = T.run(step, args.steps, args.warmup)
    kms = T.kernel_ms(lib, step, args.steps, "k_wino23")
    direct_flop = 2.0 * N * H * H * Cout * 9 * Cin
    tiles = N * ((H + 1) // 2) ** 2
    exec_flop = 2.0 * tiles * 16 * Cin * Cout
    value = direct_flop / (ms * 1e-3) / 1e12
    achieved = exec_flop / (kms * 1e-3) if kms else None
    traffic = read_traffic(os.path.join(ROOT, "profiles", "traffic_k_wino23_cfg2a.txt"))

    line = {
        "metric": "fp32 TFLOPS & int8 TOPS (% MI355X peak); ResNet-50-style b64 images/s",
        "value": round(value, 3),
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded; BASELINE config-2 distributions)",
        "config": {"workload": "cfg2a fp32 NHWC conv3x3 s1 p1 +bias+ReLU, N=32, 56x56, 64->64 "
                               "(reference route: Winograd F(2,3))",
                   "flop_count": "direct-conv equivalent 7.40 GFLOP per step",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma",
                     "achieved": round(achieved / 1e12, 3) if achieved else None,
                     "peak": PEAK_FP32 / 1e12, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_FP32, 4) if achieved else None,
                     "traffic": traffic,
                     "kernel": "k_wino23p<16,1,1>", "kernel_ms": round(kms, 5) if kms else None,
                     "work": "executed F(2,3) MFMA FLOPs 3.288 GFLOP per launch (2 * 25088 "
                             "tiles * 16 points * 64 * 64)"},
    }

    # ---------------------------------------------------------------- other configs
    configs = {}
    if not args.headline_only:
        steps = max(5, args.steps // 2)

        # 2a through the reference-compatible host-pointer API (acfun_conv2d_relu on
        # host buffers: H2D staging, kernels, D2H, synchronize) -- PCIe-inclusive rate
        yh = np.empty((N, H, H, Cout), np.float32)
        Ph = lambda a: C.c_void_p(a.ctypes.data)
        hcall = lambda: lib.acfun_conv2d_relu(Ph(x), N, H, H, Cin, Ph(w), Ph(b), 3, 3, Cout, 1, 1,
                                              Ph(yh))
        for _ in range(3):
            hcall()
        th = []
        for _ in range(steps):
            t0 = time.perf_counter()
            hcall()
            th.append(time.perf_counter() - t0)
        th = float(np.median(th)) * 1e3
        configs["cfg2a_host_buffers"] = {"ms": round(th, 4),
                                         "TFLOPS_direct": round(direct_flop / (th * 1e-3) / 1e12, 3),
                                         "note": "acfun_conv2d_relu on host memory, PCIe-inclusive, "
                                                 "median wall time"}

        # 1: GEMM 1024^3
        M = 1024
        A = cuda(rng.uniform(-1, 1, (M, M)).astype(np.float32))
        Bm = cuda(rng.uniform(-1, 1, (M, M)).astype(np.float32))
        Cm = torch.empty((M, M), device=dev)
        s1 = lambda: check(lib.acfun_dev_gemm_epi(M, M, M, A.data_ptr(), Bm.data_ptr(),
                                                  Cm.data_ptr(), None, 0, sp))
        t = T.run(s1, steps, 5)
        k = T.kernel_ms(lib, s1, steps, "k_gemm_f32")
        f = 2.0 * M ** 3 / (t * 1e-3)
        configs["cfg1_gemm_1024"] = {"ms": round(t, 5), "TFLOPS": round(f / 1e12, 3),
                                     "frac_fp32_peak": round(f / PEAK_FP32, 4),
                                     "kernel_ms": {"k_gemm_f32": k}}

        # acfun_gemm_bf16 at 1024^3 on device pointers (bf16 MFMA; not a BASELINE config)
        sb = lambda: check(lib.acfun_dev_gemm_bf16(M, M, M, A.data_ptr(), Bm.data_ptr(),
                                                   Cm.data_ptr(), sp))
        t = T.run(sb, steps, 5)
        k = T.kernel_ms(lib, sb, steps, "k_bf16mm")
        f = 2.0 * M ** 3 / (t * 1e-3)
        configs["gemm_bf16_1024"] = {"ms": round(t, 5), "TFLOPS": round(f / 1e12, 3),
                                     "frac_bf16_peak": round(f / 2.5e15, 4),
                                     "kernel_ms": {"k_bf16mm": k},
                                     "note": "step = two bf16 packing passes + k_bf16mm"}

        # 2b: F(4,3), N=8, 112x112
        x2 = cuda(rng.uniform(0, 1, (8, 112, 112, 64)).astype(np.float32))
        y2 = torch.empty((8, 112, 112, 64), device=dev)
        s2 = lambda: check(lib.acfun_dev_conv2d(x2.data_ptr(), 8, 112, 112, 64, tw.data_ptr(),
                                                tb.data_ptr(), 3, 3, 64, 1, 1, 1,
                                                y2.data_ptr(), 1, sp))
        # The reference routes this shape to F(4,3); the route here runs the faster
        # of this library's two Winograd kernels for it, the F(2,3) unit kernel
        # (k_wino23p), so executed FLOPs are counted for F(2,3).
        t = T.run(s2, steps, 5)
        k = T.kernel_ms(lib, s2, steps, "k_wino23")
        f = direct_flop / (t * 1e-3)
        ex_flop = 2.0 * 8 * 56 * 56 * 16 * 64 * 64
        ex = ex_flop / (t * 1e-3)
        configs["cfg2b_conv3x3_f43"] = {"ms": round(t, 5), "TFLOPS_direct": round(f / 1e12, 3),
                                        "kernel": "k_wino23p (persistent F(2,3) unit kernel) on the F(4,3) route",
                                        "TFLOPS_executed": round(ex / 1e12, 3),
                                        "frac_fp32_peak_executed": round(ex / PEAK_FP32, 4),
                                        "kernel_frac_fp32_peak": round(ex_flop / (k * 1e-3) / PEAK_FP32, 4)
                                        if k else None,
                                        "kernel_ms": {"k_wino23": k}}

        # 3a / 3b: int8 convs with float I/O
        for name, (KK, ci, co, pd) in {"cfg3a_int8_1x1": (1, 256, 512, 0),
                                        "cfg3b_int8_3x3": (3, 128, 128, 1)}.items():
            sa = np.float32(rng.uniform(0.005, 0.05))
            xi = cuda((rng.integers(-127, 128, (32, 28, 28, ci)).astype(np.float32) * sa))
            wq = cuda(rng.integers(-127, 128, (KK * KK * ci, co)).astype(np.int8))
            ws = cuda(rng.uniform(0.005, 0.05, co).astype(np.float32))
            bi = cuda((rng.standard_normal(co) * 0.01).astype(np.float32))
            yi = torch.empty((32, 28, 28, co), device=dev)
            def conv3(xt, yt):
                check(lib.acfun_dev_conv2d_int8(
                    xt.data_ptr(), 32, 28, 28, ci, wq.data_ptr(), ws.data_ptr(), bi.data_ptr(), KK, KK,
                    co, 1, pd, yt.data_ptr(), 1, sp))
            s3 = lambda: conv3(xi, yi)
            t = T.run(s3, steps, 5)
            k = T.kernel_ms(lib, s3, steps, "k_igemm_i8")
            ops = 2.0 * 32 * 28 * 28 * co * KK * KK * ci
            byts = 4.0 * 32 * 28 * 28 * (ci + co)
            xs, ys = rotation_sets(xi, yi)
            tc = T.run(rotating(conv3, xs, ys), steps, 5)
            configs[name] = {"ms": round(t, 5), "TOPS": round(ops / (t * 1e-3) / 1e12, 3),
                             "frac_int8_peak": round(ops / (t * 1e-3) / PEAK_INT8, 4),
                             "float_io_GBps": round(byts / (t * 1e-3) / 1e9, 1),
                             "ms_cold": round(tc, 5), "sets_cold": len(xs),
                             "kernel_ms": {"k_igemm_i8": k}}
            del xs, ys

        # 4a: depthwise 3x3/2 (BN folded) + ReLU, then 3x3/2 maxpool
        C4 = 96
        x4 = cuda(rng.uniform(0, 1, (32, 112, 112, C4)).astype(np.float32))
        w4 = cuda((rng.standard_normal((C4, 9)) * 0.3).astype(np.float32))
        b4 = cuda((rng.standard_normal(C4) * 0.1).astype(np.float32))
        y4 = torch.empty((32, 56, 56, C4), device=dev)
        z4 = torch.empty((32, 28, 28, C4), device=dev)

        def dwpool(xt, zt):
            check(lib.acfun_dev_conv2d(xt.data_ptr(), 32, 112, 112, C4, w4.data_ptr(), b4.data_ptr(),
                                       3, 3, C4, 2, 1, C4, y4.data_ptr(), 1, sp))
            check(lib.acfun_dev_maxpool(y4.data_ptr(), 32, 56, 56, C4, 3, 2, 1, zt.data_ptr(), 0, sp))
        s4 = lambda: dwpool(x4, z4)
        t = T.run(s4, steps, 5)
        kd = T.kernel_ms(lib, s4, steps, "k_dwconv")
        kp = T.kernel_ms(lib, s4, steps, "k_maxpool")
        byts = 4.0 * (32 * 112 * 112 * C4 + 2 * 32 * 56 * 56 * C4 + 32 * 28 * 28 * C4)
        xs, zs = rotation_sets(x4, z4, extra=y4.numel() * 4)
        tc = T.run(rotating(dwpool, xs, zs), steps, 5)
        configs["cfg4a_dw_bn_relu_pool"] = {"ms": round(t, 5),
                                            "GBps": round(byts / (t * 1e-3) / 1e9, 1),
                                            "frac_hbm": round(byts / (t * 1e-3) / PEAK_HBM, 4),
                                            "ms_cold": round(tc, 5), "sets_cold": len(xs),
                                            "frac_hbm_cold": round(byts / (tc * 1e-3) / PEAK_HBM, 4),
                                            "kernel_ms": {"k_dwconv": kd, "k_maxpool": kp}}
        del xs, zs

        # 4b: grouped 3x3 g6, 24 -> 48, N=32, 14x14, then maxpool
        x5 = cuda(rng.uniform(0, 1, (32, 14, 14, 24)).astype(np.float32))
        w5 = cuda((rng.standard_normal((6, 36, 8)) * 0.3).astype(np.float32))
        b5 = cuda((rng.standard_normal(48) * 0.1).astype(np.float32))
        y5 = torch.empty((32, 14, 14, 48), device=dev)
        z5 = torch.empty((32, 7, 7, 48), device=dev)

        def gpool(xt, zt):
            check(lib.acfun_dev_conv2d(xt.data_ptr(), 32, 14, 14, 24, w5.data_ptr(), b5.data_ptr(),
                                       3, 3, 48, 1, 1, 6, y5.data_ptr(), 1, sp))
            check(lib.acfun_dev_maxpool(y5.data_ptr(), 32, 14, 14, 48, 3, 2, 1, zt.data_ptr(), 0, sp))
        s5 = lambda: gpool(x5, z5)
        t = T.run(s5, steps, 5)
        kg = T.kernel_ms(lib, s5, steps, "k_gconv")
        byts = 4.0 * (32 * 14 * 14 * 24 + 2 * 32 * 14 * 14 * 48 + 32 * 7 * 7 * 48)
        xs, zs = rotation_sets(x5, z5, extra=y5.numel() * 4)
        tc = T.run(rotating(gpool, xs, zs), steps, 5)
        configs["cfg4b_grouped_pool"] = {"ms": round(t, 5), "GBps": round(byts / (t * 1e-3) / 1e9, 1),
                                         "ms_cold": round(tc, 5), "sets_cold": len(xs),
                                         "kernel_ms": {"k_gconv": kg}}
        del xs, zs

        # 5: ResNet-50-style, batch 64, fp32 and int8
        inC, inH, inW, recs = acfun0.resnet50(np.random.default_rng(5))
        fd, path = tempfile.mkstemp(suffix=".acfun")
        os.close(fd)
        acfun0.write(path, inC, inH, inW, recs, version=2)
        xin = cuda(rng.uniform(0, 1, (64, 224, 224, 3)).astype(np.float32))
        out = torch.empty((64, 1000), device=dev)
        gfl = acfun0.resnet50_flops()
        for tag, flags in (("fp32", 0), ("int8", 1)):
            m = lib.acfun_model_load_ex(path.encode(), flags)
            if not m:
                configs[f"cfg5_resnet50_b64_{tag}"] = {"error": capi.last_error()}
                continue

            def s6():
                if lib.acfun_dev_model_infer_batch(m, 64, xin.data_ptr(), out.data_ptr(), sp) != 1000:
                    raise RuntimeError(capi.last_error())
            t = T.run(s6, max(3, steps // 5), 2)
            configs[f"cfg5_resnet50_b64_{tag}"] = {"ms": round(t, 3),
                                                   "images_per_s": round(64 / (t * 1e-3), 1),
                                                   "TFLOPS": round(64 * gfl / (t * 1e-3) / 1e12, 3)}
            lib.acfun_model_destroy(m)
        os.unlink(path)
    line["configs"] = configs

    # ---------------------------------------------------------------- CPU baseline
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(x, w, b, direct_flop)
    print(json.dumps(line), flush=True)


def rotation_sets(x, y, extra=0, total=320 << 20):
    """Copies of an input and an output tensor, enough sets that one pass over
    them (plus `extra` bytes of fixed intermediates) exceeds the 256 MB MALL:
    a step on set i % n then finds its operands in HBM, not in the cache."""
    per = x.numel() * x.element_size() + y.numel() * y.element_size()
    n = max(2, -(-(total - extra) // per))
    xs = [x.clone() for _ in range(n)]
    ys = [y.new_empty(y.shape) for _ in range(n)]
    return xs, ys


def rotating(fn, xs, ys):
    """A step function that cycles fn over the rotation sets."""
    state = [0]

    def step():
        i = state[0] % len(xs)
        state[0] += 1
        fn(xs[i], ys[i])
    return step


def read_traffic(path):
    """HBM bytes per launch of the headline kernel from the committed counter
    summary (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, scaled by a plain copy of
    known size), or None when the summary is absent."""
    if not os.path.exists(path):
        return None
    vals = {}
    with open(path) as f:
        for ln in f:
            parts = ln.split()
            if len(parts) == 2 and not ln.startswith("#"):
                try:
                    vals[parts[0]] = float(parts[1])
                except ValueError:
                    pass
    return vals.get("hbm_bytes_per_launch")


def cpu_baseline(x, w, b, flop):
    import numpy as np

    import oracle
    from acfun_amd.capi import bind
    ref = oracle.ref()
    if ref is None:
        return {"value": None, "unit": "TFLOPS", "cores": 0, "kind": "reference",
                "sample": "oracle/_ref/libacfun_ref.so not present"}
    bind(ref)
    N, H, _, Cin = x.shape
    Cout = w.shape[1]
    y = np.empty((N, H, H, Cout), np.float32)
    P = lambda a: C.c_void_p(a.ctypes.data)
    run = lambda: ref.acfun_conv2d_relu(P(x), N, H, H, Cin, P(w), P(b), 3, 3, Cout, 1, 1, P(y))
    for _ in range(3):
        run()
    times = []
    t_end = time.time() + 20.0
    while len(times) < 5 or (time.time() < t_end and len(times) < 50):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    cores = ref.acfun_effective_cores()
    return {"value": round(flop / med / 1e12, 4), "unit": "TFLOPS", "cores": int(cores),
            "kind": "reference",
            "sample": f"full headline batch (N=32) through the reference's acfun_conv2d_relu "
                      f"(Winograd F(2,3), AVX-512/OpenMP), median of {len(times)} runs after 3 "
                      f"warmups: {med * 1e3:.1f} ms/step"}


if __name__ == "__main__":
    main()
