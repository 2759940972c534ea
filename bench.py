"""Benchmark of the MI355X convolution/GEMM path (one GPU).

Headline (the JSON line's metric/value): BASELINE config 2(a) -- fp32 NHWC 3x3
conv, stride 1, pad 1, bias + fused ReLU, N=32, 56x56, 64 -> 64 channels,
which the reference routes to Winograd F(2,3).  One step = one
acfun_dev_conv2d call over the whole batch, inputs resident in HBM.  value is
the FLOP rate the MFMA units execute: F(2,3)'s 2 * tiles * 16 * Cin * Cout =
3.288 GFLOP per step over the step time; the direct-convolution-equivalent rate
(7.40 GFLOP per step, the way the reference quotes conv throughput) is in
config.  roofline divides the same executed FLOPs by the dominant kernel's own
mean duration.

Every other BASELINE config is measured the same way under "configs": its step
time, the dominant kernel's time, a roofline block on the config's algorithmic
work (FLOPs, ops or bytes: the ones the computation needs, not padding or
re-reads, as the config is MFMA- or HBM-bound), and a cpu_baseline: the reference library itself (oracle/_ref,
built from the reference's sources) timed on this host's cores on a bounded
sample of the same workload, 3 warmups then the median (src/benchmark.cpp:98-111).
Configs 3 and 4 also report "ms_cold": the step cycling over copies of its
operands whose total exceeds the 256 MB MALL.

Every timed run (the W warmup steps, then exactly K timed steps) follows a
clock ramp: the step repeated, untimed, for --ramp-ms of wall time (100 ms),
because an idle MI355X takes 10-50 ms of sustained load to raise its shader
clock.  The headline's step time without the ramp is reported beside it as
ms_per_step_without_ramp.

--profile CFG runs only CFG's step (5 times) and then three plain 256 MiB
device copies, for rocprofv3 --pmc passes whose counters the copies scale.
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
PEAK_BF16 = 2.5e15       # dense bf16 MFMA, FLOP/s
PEAK_HBM = 8.0e12        # B/s
CFG_REPS = 5            # timed runs per config step (median)
CPU_BUDGET_S = 5.0       # timed CPU work per configuration (after the warmups)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--ramp-ms", type=float, default=100.0,
                    help="untimed steps for this long (wall time) before each timed run's warmup "
                         "steps, so that the GPU's clock has left its idle state (0: none)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--headline-only", action="store_true", help="skip the other configs")
    ap.add_argument("--profile", metavar="CFG", default=None,
                    help="for rocprofv3 runs: 5 steps of CFG (cfg1, cfg2a, cfg2b, cfg3a, "
                         "cfg3b, cfg3a_q, cfg3b_q, cfg4a, cfg4b), then 3 plain copies of 256 MiB "
                         "(the counter scale reference); prints no JSON line.  cfg5_fp32 / "
                         "cfg5_int8: two batch-64 inferences of the config-5 model (the first "
                         "makes its Winograd filter transforms), the second timed per layer "
                         "(--layers-md)")
    ap.add_argument("--layers-md", metavar="PATH", default=None,
                    help="with --profile cfg5_*: write the per-layer table of the second batch "
                         "(markdown) to PATH and its layers with their launch counts to PATH.json")
    ap.add_argument("--traffic", action="store_true", help="the same as --profile cfg2a")
    ap.add_argument("--tune", action="store_true",
                    help="run the tile search (acfun_autotune) over every config's shapes first, as "
                         "the reference's benchmark --tune does (src/benchmark.cpp:1164-1171)")
    return ap.parse_args()


class Timer:
    """HIP events on the stream the library launches on.  Each run first
    repeats its step, untimed, for ramp_ms of wall time: an idle MI355X
    needs about 10-50 ms of sustained work before its shader clock leaves
    the idle state (config 2a's kernel: 46.7 us per launch in the first
    milliseconds, 39.6 us after 50 ms, 46.7 us again after 1 s idle), so
    without the ramp a few-millisecond measurement times the clock's rise,
    not the kernel."""

    def __init__(self, torch, stream, ramp_ms=100.0):
        self.torch, self.stream, self.ramp_ms = torch, stream, ramp_ms

    def ramp(self, fn):
        if self.ramp_ms <= 0:
            return
        t0, n = time.perf_counter(), 0
        while n < 100000:
            fn()
            n += 1
            if n % 16 == 0 and (time.perf_counter() - t0) * 1e3 >= self.ramp_ms:
                break
        self.torch.cuda.synchronize()

    def run(self, fn, steps, warmup, reps=1):
        """ms per step over `steps` timed steps; with reps > 1 the median of
        reps such runs back to back (the configs' short steps, where one host
        stall moves a single run's mean)."""
        torch = self.torch
        self.ramp(fn)
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        ts = []
        for _ in range(reps):
            e0.record(self.stream)
            for _ in range(steps):
                fn()
            e1.record(self.stream)
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1) / steps)   # ms per step
        return sorted(ts)[len(ts) // 2]

    def kernel_ms(self, lib, fn, steps, kernels):
        """Mean duration (ms) of library kernels over `steps` more steps: the
        library brackets each launch with a HIP event pair on its stream.  An
        untimed pass first: while the library creates those events its
        launches read about 1 us long (config 1: 23.45 against 22.4-22.6 us in
        the passes after it)."""
        self.torch.cuda.synchronize()
        lib.acfun_prof_enable(1)
        for _ in range(steps):
            fn()
        self.torch.cuda.synchronize()
        lib.acfun_prof_enable(0)
        lib.acfun_prof_enable(1)
        for _ in range(steps):
            fn()
        self.torch.cuda.synchronize()
        lib.acfun_prof_enable(0)
        out = {}
        for k in kernels:
            n = C.c_int(0)
            ms = lib.acfun_prof_kernel_ms(k.encode(), C.byref(n))
            out[k] = round(ms, 5) if n.value > 0 and ms > 0 else None
        return out


def read_traffic(name):
    """HBM bytes per launch from a committed counter summary
    (profiles/traffic_<name>.txt: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE,
    scaled by a plain copy of known size), or None when there is none."""
    path = os.path.join(ROOT, "profiles", f"traffic_{name}.txt")
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


def roofline(bound, work, ms, kernel, work_note, traffic_name=None):
    """A roofline block: `work` is FLOP/op (bound mfma-fp32 / mfma-int8) or
    bytes (bound hbm) per launch of `kernel`, `ms` its mean duration."""
    if bound == "hbm":
        peak, unit, scale = PEAK_HBM, "GB/s", 1e9
    elif bound == "mfma-int8":
        peak, unit, scale = PEAK_INT8, "TOP/s", 1e12
    else:
        peak, unit, scale = PEAK_FP32, "TFLOP/s", 1e12
    ach = work / (ms * 1e-3) if ms else None
    return {"bound": "hbm" if bound == "hbm" else "mfma",
            "achieved": round(ach / scale, 3) if ach else None,
            "peak": peak / scale, "unit": unit,
            "frac": round(ach / peak, 4) if ach else None,
            "traffic": read_traffic(traffic_name) if traffic_name else None,
            "kernel": kernel, "kernel_ms": round(ms, 5) if ms else None, "work": work_note}


# ------------------------------------------------------------------ config 5 per layer
LAYER_TYPES = {1: "conv", 2: "fc", 3: "relu", 4: "maxpool", 5: "softmax", 6: "bn", 7: "convg",
               8: "add", 9: "gap", 10: "input"}


def layer_work(L, names):
    """Executed work of one model layer, from its shape and the kernels that
    ran it: (fp32 MFMA FLOPs, int8 MFMA ops, compulsory HBM bytes).
    F(2,3) / F(4,3) layers count the transform-domain products the algorithm
    needs (2 * tiles * points * Cin * Cout, no padding), other convs and the FC
    the direct 2 * M * N * K; bytes are the input read, the output written and
    the weights once (fp32 activations, as the model keeps them)."""
    import math
    N, H, W, C, OH, OW, OC = (L[k] for k in ("N", "H", "W", "C", "OH", "OW", "OC"))
    t = L["type"]
    fp32 = int8 = 0.0
    act_in, act_out = 4.0 * N * H * W * C, 4.0 * N * OH * OW * OC
    wbytes = 0.0
    if t in (1, 7):
        KH, KW, g = L["KH"], L["KW"], max(1, L["groups"])
        direct = 2.0 * N * OH * OW * OC * KH * KW * (C // g)
        wbytes = KH * KW * (C // g) * OC * (1.0 if L["int8"] else 4.0)
        if L["int8"]:
            int8 = direct
        elif any(n.startswith("k_wino23") for n in names):
            fp32 = 2.0 * N * math.ceil(OH / 2) * math.ceil(OW / 2) * 16 * C * OC
        elif any(n.startswith(("k_wino43", "k_wino_fused")) for n in names):
            fp32 = 2.0 * N * math.ceil(OH / 4) * math.ceil(OW / 4) * 36 * C * OC
        else:
            fp32 = direct
        if L["residual"]:
            act_out *= 2
    elif t == 2:
        fp32 = 2.0 * N * H * W * C * OC
        wbytes = 4.0 * H * W * C * OC
    elif t == 8:
        act_in *= 2
    return fp32, int8, act_in + act_out + wbytes


def model_layer_profile(lib, run):
    """Runs `run` (one inference) with kernel timing on and returns the layers
    that launched kernels: shape, kernels with their summed ms, executed work
    and the layer's roofline floor (max of MFMA time at peak and HBM time)."""
    from acfun_amd import capi
    import torch
    for _ in range(2):              # the first pass creates the timing events (Timer.kernel_ms)
        torch.cuda.synchronize()
        lib.acfun_prof_enable(1)
        run()
        torch.cuda.synchronize()
        lib.acfun_prof_enable(0)
    kernels, layers = capi.prof_report()
    rows = []
    for L in layers:
        ks = {name: v for (tag, name), v in kernels.items() if tag == L["i"]}
        if not ks:
            continue
        fp32, int8, byt = layer_work(L, ks)
        ms = sum(v[1] for v in ks.values())
        floor = max(fp32 / PEAK_FP32 + int8 / PEAK_INT8, byt / PEAK_HBM) * 1e3
        rows.append(dict(L, kernels=ks, ms=ms, fp32=fp32, int8=int8, bytes=byt, floor_ms=floor))
    untagged = {name: v for (tag, name), v in kernels.items() if tag < 0}
    return rows, untagged


def layer_table_md(rows, untagged, tag):
    """Markdown: the layers grouped by shape and route, largest time first."""
    groups = {}
    for r in rows:
        shape = (f"{LAYER_TYPES.get(r['type'], r['type'])} {r['KH']}x{r['KW']}/{r['stride']} "
                 f"{r['H']}x{r['W']}x{r['C']} -> {r['OH']}x{r['OW']}x{r['OC']}"
                 + (" +add" if r["residual"] else "") if r["type"] in (1, 7) else
                 f"{LAYER_TYPES.get(r['type'], r['type'])} {r['H']}x{r['W']}x{r['C']} -> "
                 f"{r['OH']}x{r['OW']}x{r['OC']}")
        key = (shape, " + ".join(sorted(r["kernels"])))
        g = groups.setdefault(key, dict(n=0, ms=0.0, fp32=0.0, int8=0.0, bytes=0.0, floor=0.0, kms={}))
        for name, (_, kms) in r["kernels"].items():
            g["kms"][name] = g["kms"].get(name, 0.0) + kms
        g["n"] += 1
        g["ms"] += r["ms"]
        g["fp32"] += r["fp32"]
        g["int8"] += r["int8"]
        g["bytes"] += r["bytes"]
        g["floor"] += r["floor_ms"]
    total = sum(g["ms"] for g in groups.values())
    out = [f"| layer shape (per batch of {rows[0]['N'] if rows else 0}) | kernels (ms) | layers | ms | share | "
           "executed GFLOP fp32 / GOP int8 | TFLOP/s (TOP/s) | frac of peak | floor ms | time / floor |",
           "|---|---|---|---|---|---|---|---|---|---|"]
    for (shape, _), g in sorted(groups.items(), key=lambda kv: -kv[1]["ms"]):
        ks = ", ".join(f"{k} {v:.4f}" for k, v in sorted(g["kms"].items(), key=lambda kv: -kv[1]))
        work = g["int8"] if g["int8"] else g["fp32"]
        peak = PEAK_INT8 if g["int8"] else PEAK_FP32
        rate = work / (g["ms"] * 1e-3) / 1e12 if g["ms"] and work else 0.0
        out.append(f"| {shape} | {ks} | {g['n']} | {g['ms']:.4f} | {g['ms'] / total:.3f} | "
                   + (f"{g['int8'] / 1e9:.2f} (int8)" if g["int8"] else f"{g['fp32'] / 1e9:.2f}")
                   + f" | {rate:.1f} | {rate * 1e12 / peak:.3f} | {g['floor']:.4f} | "
                   f"{g['ms'] / g['floor'] if g['floor'] else 0:.2f} |")
    if untagged:
        out.append("")
        out.append("Launches outside the layers (the model's input/output copies are not kernels): "
                   + ", ".join(f"{k} {v[0]}x {v[1]:.4f} ms" for k, v in sorted(untagged.items())))
    kern = {}
    for r in rows:
        for name, (n, ms) in r["kernels"].items():
            a = kern.setdefault(name, [0, 0.0])
            a[0] += n
            a[1] += ms
    out.append("")
    out.append(f"Per kernel name ({tag}, this batch): | kernel | launches | total ms |")
    out.append("|---|---|---|")
    for name, (n, ms) in sorted(kern.items(), key=lambda kv: -kv[1][1]):
        out.append(f"| {name} | {n} | {ms:.4f} |")
    return "\n".join(out) + "\n"


def cfg5_roofline(rows, step_ms, int8):
    """Config 5's roofline block: the batch's executed MFMA work over the step
    time (fp32 model: fp32 FLOPs; int8 model: the int8 convs' ops), plus the
    sum of per-layer floors over the step time."""
    fp32 = sum(r["fp32"] for r in rows)
    i8 = sum(r["int8"] for r in rows)
    floor = sum(r["floor_ms"] for r in rows)
    kern_ms = sum(r["ms"] for r in rows)
    if int8:
        blk = roofline("mfma-int8", i8, step_ms, "whole batch (every layer's kernels)",
                       f"executed int8 MFMA ops of the int8 convs, {i8 / 1e9:.1f} GOP per batch "
                       f"(the fp32 FC: {fp32 / 1e9:.2f} GFLOP, not counted), over the step time")
    else:
        blk = roofline("mfma-fp32", fp32, step_ms, "whole batch (every layer's kernels)",
                       f"executed fp32 MFMA FLOPs, {fp32 / 1e9:.1f} GFLOP per batch: F(2,3) "
                       "transform-domain products for the Winograd layers, direct 2*M*N*K for "
                       "the others, over the step time")
    blk["frac_of_layer_floors"] = round(floor / step_ms, 4) if step_ms else None
    blk["layer_floor_ms"] = round(floor, 4)
    blk["kernels_ms"] = round(kern_ms, 4)
    return blk


# ------------------------------------------------------------------ the configs
# Each builder returns (step, extras): step() runs one step on the library's
# stream; extras carries what the report needs.

def make_configs(lib, torch, dev, sp, rng, check):
    import numpy as np

    from acfun_amd import acfun0

    def cuda(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev)

    cfg = {}

    # 2(a), the headline: F(2,3), N=32, 56x56, 64 -> 64
    N, H, Cin, Cout = 32, 56, 64, 64
    x2 = rng.uniform(0, 1, (N, H, H, Cin)).astype(np.float32)
    w2 = (rng.standard_normal((9 * Cin, Cout)) * np.sqrt(2.0 / (9 * Cin))).astype(np.float32)
    b2 = (rng.standard_normal(Cout) * 0.01).astype(np.float32)
    tx2, tw2, tb2 = cuda(x2), cuda(w2), cuda(b2)
    ty2 = torch.empty((N, H, H, Cout), device=dev)
    cfg["cfg2a"] = dict(
        step=lambda: check(lib.acfun_dev_conv2d(tx2.data_ptr(), N, H, H, Cin, tw2.data_ptr(),
                                                tb2.data_ptr(), 3, 3, Cout, 1, 1, 1,
                                                ty2.data_ptr(), 1, sp)),
        host=(x2, w2, b2))

    # 1: GEMM 1024^3
    M = 1024
    A1 = rng.uniform(-1, 1, (M, M)).astype(np.float32)
    B1 = rng.uniform(-1, 1, (M, M)).astype(np.float32)
    tA, tB = cuda(A1), cuda(B1)
    tC = torch.empty((M, M), device=dev)
    cfg["cfg1"] = dict(step=lambda: check(lib.acfun_dev_gemm_epi(M, M, M, tA.data_ptr(),
                                                                  tB.data_ptr(), tC.data_ptr(),
                                                                  None, 0, sp)),
                       host=(A1, B1))
    cfg["bf16"] = dict(step=lambda: check(lib.acfun_dev_gemm_bf16(M, M, M, tA.data_ptr(),
                                                                   tB.data_ptr(), tC.data_ptr(),
                                                                   sp)))

    # 2(b): N=8, 112x112, 64 -> 64 (the reference's F(4,3) route)
    x2b = rng.uniform(0, 1, (8, 112, 112, 64)).astype(np.float32)
    tx2b = cuda(x2b)
    ty2b = torch.empty((8, 112, 112, 64), device=dev)
    cfg["cfg2b"] = dict(
        step=lambda: check(lib.acfun_dev_conv2d(tx2b.data_ptr(), 8, 112, 112, 64, tw2.data_ptr(),
                                                tb2.data_ptr(), 3, 3, 64, 1, 1, 1,
                                                ty2b.data_ptr(), 1, sp)),
        host=(x2b, w2, b2))

    # 3(a) / 3(b): int8 convs, float I/O (acfun_conv2d_int8) and int8 I/O (acfun_dev_conv2d_int8_q)
    for name, (KK, ci, co, pd) in {"cfg3a": (1, 256, 512, 0), "cfg3b": (3, 128, 128, 1)}.items():
        q = rng.integers(-127, 128, (32, 28, 28, ci)).astype(np.int8)
        q.reshape(-1)[0] = 127
        while True:
            sa = np.float32(rng.uniform(0.005, 0.05))
            if np.float32(np.float32(127.0) * sa) / np.float32(127.0) == sa:
                break
        xf = (q.astype(np.float32) * sa).astype(np.float32)
        wq = rng.integers(-127, 128, (KK * KK * ci, co)).astype(np.int8)
        ws = rng.uniform(0.005, 0.05, co).astype(np.float32)
        bi = (rng.standard_normal(co) * 0.01).astype(np.float32)
        t = dict(x=cuda(xf), q=cuda(q), wq=cuda(wq), ws=cuda(ws), b=cuda(bi),
                 y=torch.empty((32, 28, 28, co), device=dev),
                 yq=torch.empty((32, 28, 28, co), dtype=torch.int8, device=dev),
                 si=torch.tensor([float(sa)], device=dev), so=torch.zeros(1, device=dev))

        def conv_f(xt, yt, t=t, KK=KK, ci=ci, co=co, pd=pd):
            check(lib.acfun_dev_conv2d_int8(xt.data_ptr(), 32, 28, 28, ci, t["wq"].data_ptr(),
                                            t["ws"].data_ptr(), t["b"].data_ptr(), KK, KK, co, 1,
                                            pd, yt.data_ptr(), 1, sp))

        def conv_q(qt, yt, t=t, KK=KK, ci=ci, co=co, pd=pd):
            check(lib.acfun_dev_conv2d_int8_q(qt.data_ptr(), t["si"].data_ptr(), 32, 28, 28, ci,
                                              t["wq"].data_ptr(), t["ws"].data_ptr(),
                                              t["b"].data_ptr(), KK, KK, co, 1, pd, yt.data_ptr(),
                                              t["so"].data_ptr(), 1, 0, sp))
        cfg[name] = dict(step=lambda f=conv_f, t=t: f(t["x"], t["y"]), rot=(conv_f, t["x"], t["y"]),
                         host=(xf, wq, ws, bi, KK, ci, co, pd),
                         ops=2.0 * 32 * 28 * 28 * co * KK * KK * ci,
                         fbytes=4.0 * 32 * 28 * 28 * (ci + co), qbytes=1.0 * 32 * 28 * 28 * (ci + co))
        cfg[name + "_q"] = dict(step=lambda f=conv_q, t=t: f(t["q"], t["yq"]),
                                rot=(conv_q, t["q"], t["yq"]))

    # 4(a): depthwise 3x3/2 (BN folded) + ReLU, then 3x3/2 MaxPool, fused
    C4 = 96
    x4 = rng.uniform(0, 1, (32, 112, 112, C4)).astype(np.float32)
    w4 = (rng.standard_normal((C4, 3, 3)) * 0.3).astype(np.float32)
    b4 = (rng.standard_normal(C4) * 0.1).astype(np.float32)
    tx4, tw4, tb4 = cuda(x4), cuda(w4), cuda(b4)
    tz4 = torch.empty((32, 28, 28, C4), device=dev)

    def dwpool(xt, zt):
        check(lib.acfun_dev_conv2d_dw_maxpool(xt.data_ptr(), 32, 112, 112, C4, tw4.data_ptr(),
                                              tb4.data_ptr(), 3, 3, 2, 1, 1, 3, 2, 1,
                                              zt.data_ptr(), 0, sp))
    cfg["cfg4a"] = dict(step=lambda: dwpool(tx4, tz4), rot=(dwpool, tx4, tz4),
                        host=(x4, w4, b4), bytes=4.0 * (32 * 112 * 112 * C4 + 32 * 28 * 28 * C4))

    # 4(b): grouped 3x3 g6, 24 -> 48, N=32, 14x14, then 3x3/2 MaxPool
    x5 = rng.uniform(0, 1, (32, 14, 14, 24)).astype(np.float32)
    w5 = (rng.standard_normal((6, 36, 8)) * 0.3).astype(np.float32)
    b5 = (rng.standard_normal(48) * 0.1).astype(np.float32)
    tx5, tw5, tb5 = cuda(x5), cuda(w5), cuda(b5)
    ty5 = torch.empty((32, 14, 14, 48), device=dev)
    tz5 = torch.empty((32, 7, 7, 48), device=dev)

    def gpool2(xt, zt):              # the two reference calls as two launches
        check(lib.acfun_dev_conv2d(xt.data_ptr(), 32, 14, 14, 24, tw5.data_ptr(), tb5.data_ptr(),
                                   3, 3, 48, 1, 1, 6, ty5.data_ptr(), 1, sp))
        check(lib.acfun_dev_maxpool(ty5.data_ptr(), 32, 14, 14, 48, 3, 2, 1, zt.data_ptr(), 0, sp))

    def gpool(xt, zt):               # fused: grouped conv + ReLU + MaxPool in one kernel
        check(lib.acfun_dev_conv2d_g_maxpool(xt.data_ptr(), 32, 14, 14, 24, tw5.data_ptr(),
                                             tb5.data_ptr(), 3, 3, 48, 1, 1, 6, 1, 3, 2, 1,
                                             zt.data_ptr(), 0, sp))
    cfg["cfg4b"] = dict(step=lambda: gpool(tx5, tz5), rot=(gpool, tx5, tz5), host=(x5, w5, b5),
                        two=lambda: gpool2(tx5, tz5),
                        bytes=4.0 * (32 * 14 * 14 * 24 + 32 * 7 * 7 * 48))

    # 5: ResNet-50-style, batch 64
    inC, inH, inW, recs = acfun0.resnet50(np.random.default_rng(5))
    cfg["cfg5"] = dict(recs=(inC, inH, inW, recs))
    return cfg


def load_cfg5(lib, torch, dev, rng, cfg, int8):
    """Writes config 5's version-2 ResNet-50 to a temporary file and loads it
    (int8: flags 1); returns (model, path, input [64,224,224,3], output)."""
    import numpy as np

    from acfun_amd import acfun0
    inC, inH, inW, recs = cfg["cfg5"]["recs"]
    fd, path = tempfile.mkstemp(suffix=".acfun")
    os.close(fd)
    acfun0.write(path, inC, inH, inW, recs, version=2)
    xin = torch.from_numpy(rng.uniform(0, 1, (64, inH, inW, inC)).astype(np.float32)).to(dev)
    out = torch.empty((64, 1000), device=dev)
    m = lib.acfun_model_load_ex(path.encode(), 1 if int8 else 0)
    return m, path, xin, out


def check_infer(lib, m, xin, out, sp):
    from acfun_amd import capi
    if lib.acfun_dev_model_infer_batch(m, 64, xin.data_ptr(), out.data_ptr(), sp) != 1000:
        raise RuntimeError(capi.last_error())


def rotation_sets(x, y, extra=0, total=320 << 20):
    """Copies of an input and an output tensor, enough sets that one pass over
    them (plus `extra` bytes of fixed intermediates) exceeds the 256 MB MALL:
    a step on set i % n then finds its operands in HBM, not in the cache."""
    per = x.numel() * x.element_size() + y.numel() * y.element_size()
    n = max(2, -(-(total - extra) // per))
    return [x.clone() for _ in range(n)], [y.new_empty(y.shape) for _ in range(n)]


def rotating(fn, xs, ys):
    state = [0]

    def step():
        i = state[0] % len(xs)
        state[0] += 1
        fn(xs[i], ys[i])
    return step


# ------------------------------------------------------------------ CPU baselines
def host_cpu():
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_median(fn, budget=CPU_BUDGET_S, warmups=3, min_reps=5):
    """The reference's method (src/benchmark.cpp:98-111): warmups, then the
    median of the timed repetitions (at least min_reps, up to the budget)."""
    import numpy as np
    for _ in range(warmups):
        fn()
    times = []
    t_end = time.time() + budget
    while len(times) < min_reps or (time.time() < t_end and len(times) < 200):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def cpu_baselines(cfg, configs, line):
    """The compiled reference on this host, per configuration."""
    import numpy as np

    import oracle
    import oracle.model as omodel
    from acfun_amd.capi import bind
    ref = oracle.ref()
    if ref is None:
        na = {"value": None, "unit": None, "cores": 0, "kind": "reference",
              "sample": "oracle/_ref/libacfun_ref.so not present"}
        line["cpu_baseline"] = dict(na, unit="TFLOPS")
        return
    bind(ref)
    cores = int(ref.acfun_effective_cores())
    ref.acfun_set_threads(cores)
    host = f"{host_cpu()}, {cores} threads (cgroup-capped, as the reference's own acfun_effective_cores)"
    P = lambda a: C.c_void_p(a.ctypes.data)

    def base(value, unit, sample):
        return {"value": round(value, 4), "unit": unit, "cores": cores, "kind": "reference",
                "sample": sample, "host": host}

    # 2(a) headline
    x, w, b = cfg["cfg2a"]["host"]
    y = np.empty((32, 56, 56, 64), np.float32)
    t, n = cpu_median(lambda: ref.acfun_conv2d_relu(P(x), 32, 56, 56, 64, P(w), P(b), 3, 3, 64, 1,
                                                    1, P(y)))
    line["cpu_baseline"] = base(3.288334336e9 / t / 1e12, "TFLOPS",
                                f"full headline batch (N=32) through the reference's "
                                f"acfun_conv2d_relu (Winograd F(2,3), AVX-512/OpenMP), median of {n} "
                                f"runs after 3 warmups: {t * 1e3:.2f} ms/step; value counts the "
                                f"executed F(2,3) FLOPs as the GPU value does "
                                f"({7.398752256e9 / t / 1e12:.3f} TFLOPS direct-equivalent)")
    if "cfg1_gemm_1024" in configs:
        A, B = cfg["cfg1"]["host"]
        Cm = np.empty((1024, 1024), np.float32)
        t, n = cpu_median(lambda: ref.acfun_gemm(1024, 1024, 1024, P(A), P(B), P(Cm)))
        configs["cfg1_gemm_1024"]["cpu_baseline"] = base(
            2.0 * 1024 ** 3 / t / 1e12, "TFLOPS",
            f"full size through acfun_gemm, median of {n}: {t * 1e3:.2f} ms")
    if "cfg2b_conv3x3_f43" in configs:
        x, w, b = cfg["cfg2b"]["host"]
        y = np.empty(x.shape, np.float32)
        t, n = cpu_median(lambda: ref.acfun_conv2d_relu(P(x), 8, 112, 112, 64, P(w), P(b), 3, 3,
                                                        64, 1, 1, P(y)))
        configs["cfg2b_conv3x3_f43"]["cpu_baseline"] = base(
            1.849688064e9 / t / 1e12, "TFLOPS",
            f"full size through acfun_conv2d_relu (its F(4,3) route), median of {n}: "
            f"{t * 1e3:.2f} ms; value on the executed F(4,3) FLOPs "
            f"({7.398752256e9 / t / 1e12:.3f} TFLOPS direct-equivalent)")
    for name, key in (("cfg3a", "cfg3a_int8_1x1"), ("cfg3b", "cfg3b_int8_3x3")):
        if key not in configs:
            continue
        xf, wq, ws, bi, KK, ci, co, pd = cfg[name]["host"]
        y = np.empty((32, 28, 28, co), np.float32)
        t, n = cpu_median(lambda: ref.acfun_conv2d_int8(P(xf), 32, 28, 28, ci, P(wq), P(ws), P(bi),
                                                        KK, KK, co, 1, pd, C.c_float(0.0), P(y), 1))
        configs[key]["cpu_baseline"] = base(
            cfg[name]["ops"] / t / 1e12, "TOPS",
            f"full size through acfun_conv2d_int8 (float I/O, AVX-512 VNNI), median of {n}: "
            f"{t * 1e3:.2f} ms")
    if "cfg4a_dw_bn_relu_pool" in configs:
        x, w, b = cfg["cfg4a"]["host"]
        y = np.empty((32, 56, 56, 96), np.float32)
        z = np.empty((32, 28, 28, 96), np.float32)

        def dp():
            ref.acfun_conv2d_dw(P(x), 32, 112, 112, 96, P(w), P(b), 3, 3, 2, 1, P(y), 1)
            ref.acfun_maxpool(P(y), 32, 56, 56, 96, 3, 2, 1, P(z))
        t, n = cpu_median(dp)
        configs["cfg4a_dw_bn_relu_pool"]["cpu_baseline"] = base(
            cfg["cfg4a"]["bytes"] / t / 1e9, "GB/s",
            f"full size through acfun_conv2d_dw + acfun_maxpool, median of {n}: {t * 1e3:.2f} ms; "
            f"value on the same 163.8 MB as the GPU figure")
    if "cfg4b_grouped_pool" in configs:
        x, w, b = cfg["cfg4b"]["host"]
        y = np.empty((32, 14, 14, 48), np.float32)
        z = np.empty((32, 7, 7, 48), np.float32)

        def gp():
            ref.acfun_conv2d_g(P(x), 32, 14, 14, 24, P(w), P(b), 3, 3, 48, 1, 1, 6, P(y), 1)
            ref.acfun_maxpool(P(y), 32, 14, 14, 48, 3, 2, 1, P(z))
        t, n = cpu_median(gp)
        configs["cfg4b_grouped_pool"]["cpu_baseline"] = base(
            cfg["cfg4b"]["bytes"] / t / 1e9, "GB/s",
            f"full size through acfun_conv2d_g + acfun_maxpool, median of {n}: {t * 1e3:.3f} ms")
    # 5: the version-2 ResNet-50 through the reference's own per-op calls on a
    # bounded sample of 8 images (its executor cannot load residual records)
    inC, inH, inW, recs = cfg["cfg5"]["recs"]
    from acfun_amd import acfun0
    blob = acfun0.encode(inC, inH, inW, recs, version=2)
    xs = np.random.default_rng(3).uniform(0, 1, (8, inH, inW, inC)).astype(np.float32)
    for tag, int8 in (("fp32", False), ("int8", True)):
        key = f"cfg5_resnet50_b64_{tag}"
        if key not in configs:
            continue
        prep = omodel.prepare_reference(ref, blob, int8)
        t, n = cpu_median(lambda: omodel.run_reference(ref, prep, xs), budget=CPU_BUDGET_S,
                          warmups=1, min_reps=3)
        configs[key]["cpu_baseline"] = base(
            8 / t, "images/s",
            f"8 images (a sample of the batch of 64) through the reference's per-op calls "
            f"(acfun_conv2d(_relu)/acfun_conv2d_int8, acfun_maxpool, acfun_fc, acfun_softmax; "
            f"numpy for the Add and global-pool records), median of {n}: {t * 1e3:.1f} ms"
            + ("; int8 convs are acfun_conv2d_int8 on the batch" if int8 else ""))


def tune_all(lib, torch, dev, sp, cfg, rng):
    """One step of every config (and one batch-64 pass of each config-5 model)
    registers their shapes; acfun_autotune() then searches and caches them."""
    import numpy as np

    from acfun_amd import acfun0
    for k, c in cfg.items():
        for key in ("step", "two"):
            if key in c:
                c[key]()
    inC, inH, inW, recs = cfg["cfg5"]["recs"]
    fd, path = tempfile.mkstemp(suffix=".acfun")
    os.close(fd)
    acfun0.write(path, inC, inH, inW, recs, version=2)
    xin = torch.from_numpy(rng.uniform(0, 1, (64, 224, 224, 3)).astype(np.float32)).to(dev)
    out = torch.empty((64, 1000), device=dev)
    for flags in (0, 1):
        m = lib.acfun_model_load_ex(path.encode(), flags)
        if m:
            lib.acfun_dev_model_infer_batch(m, 64, xin.data_ptr(), out.data_ptr(), sp)
            torch.cuda.synchronize()
            lib.acfun_model_destroy(m)
    os.unlink(path)
    torch.cuda.synchronize()
    lib.acfun_autotune()


# ------------------------------------------------------------------ main
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
    T = Timer(torch, stream, args.ramp_ms)
    rng = np.random.default_rng(12345 + 1)

    def check(rc):
        if rc != 0:
            raise RuntimeError(capi.last_error())

    cfg = make_configs(lib, torch, dev, sp, rng, check)
    if args.tune:
        tune_all(lib, torch, dev, sp, cfg, rng)

    if args.traffic:
        args.profile = "cfg2a"
    if args.profile in ("cfg5_fp32", "cfg5_int8"):
        int8 = args.profile == "cfg5_int8"
        m, path, xin, out = load_cfg5(lib, torch, dev, rng, cfg, int8)
        run = lambda: check_infer(lib, m, xin, out, sp)
        run()                                          # makes the Winograd filter transforms
        T.ramp(run)
        rows, untagged = model_layer_profile(lib, run)
        torch.cuda.synchronize()
        lib.acfun_model_destroy(m)
        os.unlink(path)
        md = layer_table_md(rows, untagged, args.profile)
        if args.layers_md:
            with open(args.layers_md, "w") as f:
                f.write(md)
            # the layers in execution order with their launch counts, so that a
            # kernel trace of the same run can be split by layer
            with open(args.layers_md + ".json", "w") as f:
                json.dump({"layers": [dict({k: v for k, v in r.items() if k != "kernels"},
                                           kernels={n: list(v) for n, v in r["kernels"].items()})
                                      for r in rows],
                           "untagged": {n: list(v) for n, v in untagged.items()}}, f)
        print(md, flush=True)
        return
    if args.profile:
        if args.profile not in cfg or "step" not in cfg[args.profile]:
            raise SystemExit(f"bench.py: no configuration {args.profile!r}")
        T.ramp(cfg[args.profile]["step"])
        for _ in range(5):
            cfg[args.profile]["step"]()
        src = torch.empty(64 << 20, device=dev)        # 256 MiB
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        return

    # ---------------------------------------------------------------- headline
    # first the same steps with no clock ramp (reported beside the headline),
    # then with it
    ramp_ms, T.ramp_ms = T.ramp_ms, 0.0
    ms_no_ramp = T.run(cfg["cfg2a"]["step"], args.steps, args.warmup)
    T.ramp_ms = ramp_ms
    ms = T.run(cfg["cfg2a"]["step"], args.steps, args.warmup)
    k = T.kernel_ms(lib, cfg["cfg2a"]["step"], args.steps, ["k_wino23", "k_wino_filter_t"])
    direct_flop = 7.398752256e9
    exec_flop = 3.288334336e9
    line = {
        "metric": "fp32 TFLOPS & int8 TOPS (% MI355X peak); ResNet-50-style b64 images/s",
        "value": round(exec_flop / (ms * 1e-3) / 1e12, 3),
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "clock_ramp_ms": args.ramp_ms,
        "ms_per_step_without_ramp": round(ms_no_ramp, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded; BASELINE config-2 distributions)",
        "config": {"workload": "cfg2a fp32 NHWC conv3x3 s1 p1 +bias+ReLU, N=32, 56x56, 64->64 "
                               "(reference route: Winograd F(2,3))",
                   "flop_count": "executed F(2,3) MFMA FLOPs, 3.288 GFLOP per step",
                   "TFLOPS_direct_equivalent": round(direct_flop / (ms * 1e-3) / 1e12, 3),
                   "parallelism": "single GPU"},
        "roofline": roofline("mfma-fp32", exec_flop, k["k_wino23"], "k_wino23p<16,1,1>",
                             "executed F(2,3) MFMA FLOPs 3.288 GFLOP per launch (2 * 25088 tiles "
                             "* 16 points * 64 * 64)", "k_wino23_cfg2a"),
    }
    line["roofline"]["other_kernels_ms"] = {"k_wino_filter_t": k["k_wino_filter_t"]}

    configs = {}
    if not args.headline_only:
        steps = args.steps

        # 2(a) through the reference-compatible host-pointer API -- PCIe-inclusive rate
        x, w, b = cfg["cfg2a"]["host"]
        yh = np.empty((32, 56, 56, 64), np.float32)
        Ph = lambda a: C.c_void_p(a.ctypes.data)
        hcall = lambda: lib.acfun_conv2d_relu(Ph(x), 32, 56, 56, 64, Ph(w), Ph(b), 3, 3, 64, 1, 1,
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
                                         "note": "acfun_conv2d_relu on host memory: H2D, kernels, "
                                                 "D2H, synchronize (PCIe-inclusive), median wall "
                                                 "time; never the headline value"}

        # 1: GEMM 1024^3
        t = T.run(cfg["cfg1"]["step"], steps, args.warmup, CFG_REPS)
        k = T.kernel_ms(lib, cfg["cfg1"]["step"], steps, ["k_gemm32"])
        flop = 2.0 * 1024 ** 3
        configs["cfg1_gemm_1024"] = {
            "ms": round(t, 5), "TFLOPS": round(flop / (t * 1e-3) / 1e12, 3),
            "roofline": roofline("mfma-fp32", flop, k["k_gemm32"], "k_gemm32",
                                 "2*1024^3 = 2.147 GFLOP per launch", "k_gemm32_cfg1")}

        # acfun_gemm_bf16 1024^3 (not a BASELINE config)
        t = T.run(cfg["bf16"]["step"], steps, args.warmup, CFG_REPS)
        k = T.kernel_ms(lib, cfg["bf16"]["step"], steps, ["k_bf16mm"])
        configs["gemm_bf16_1024"] = {"ms": round(t, 5), "TFLOPS": round(flop / (t * 1e-3) / 1e12, 3),
                                     "frac_bf16_peak_kernel": round(flop / (k["k_bf16mm"] * 1e-3) / PEAK_BF16, 4)
                                     if k["k_bf16mm"] else None,
                                     "kernel_ms": k, "note": "step = one bf16 packing launch (A and B) + k_bf16mm"}

        # 2(b): F(4,3) route; the fraction counts the F(4,3) work the route needs
        t = T.run(cfg["cfg2b"]["step"], steps, args.warmup, CFG_REPS)
        k = T.kernel_ms(lib, cfg["cfg2b"]["step"], steps, ["k_wino43", "k_wino23", "k_wino_fused",
                                                             "k_wino_filter_t"])
        f43 = 1.849688064e9
        kern = next((n for n in ("k_wino43", "k_wino23", "k_wino_fused") if k[n]), "k_wino43")
        configs["cfg2b_conv3x3_f43"] = {
            "ms": round(t, 5), "TFLOPS_direct_equivalent": round(direct_flop / (t * 1e-3) / 1e12, 3),
            "TFLOPS_f43_work": round(f43 / (t * 1e-3) / 1e12, 3),
            "roofline": roofline("mfma-fp32", f43, k[kern], kern,
                                 "F(4,3) work: 2 * 6272 tiles * 36 points * 64 * "
                                 "64 = 1.850 GFLOP per launch, whichever kernel runs it",
                                 "k_wino_cfg2b"),
            "kernel_ms": k}

        # 3(a) / 3(b)
        for name, key in (("cfg3a", "cfg3a_int8_1x1"), ("cfg3b", "cfg3b_int8_3x3")):
            c = cfg[name]
            t = T.run(c["step"], steps, args.warmup, CFG_REPS)
            k = T.kernel_ms(lib, c["step"], steps, ["k_i8mm"])
            fn, xt, yt = c["rot"]
            xs, ys = rotation_sets(xt, yt)
            tc = T.run(rotating(fn, xs, ys), steps, args.warmup, CFG_REPS)
            del xs, ys
            tq = T.run(cfg[name + "_q"]["step"], steps, args.warmup, CFG_REPS)
            kq = T.kernel_ms(lib, cfg[name + "_q"]["step"], steps,
                             ["k_i8mm_amax", "k_i8mm_q8", "k_i8mm", "k_requant_s8"])
            fn, xt, yt = cfg[name + "_q"]["rot"]
            xs, ys = rotation_sets(xt, yt)
            tqc = T.run(rotating(fn, xs, ys), steps, args.warmup, CFG_REPS)
            del xs, ys
            ops = c["ops"]
            configs[key] = {
                "float_io": {
                    "ms": round(t, 5), "ms_cold": round(tc, 5),
                    "TOPS": round(ops / (t * 1e-3) / 1e12, 3),
                    "roofline": roofline("hbm", c["fbytes"], t, "step (absmax + quantize + k_i8mm)",
                                         f"float I/O {c['fbytes'] / 1e6:.1f} MB per step (fp32 input "
                                         "read, fp32 output written); the int8 fraction is TOPS/5000"),
                    "frac_int8_peak": round(ops / (t * 1e-3) / PEAK_INT8, 4),
                    "kernel_ms": k,
                    "kernel_frac_int8_peak": round(ops / (k["k_i8mm"] * 1e-3) / PEAK_INT8, 4)
                    if k["k_i8mm"] else None},
                "int8_io": {
                    "ms": round(tq, 5), "ms_cold": round(tqc, 5),
                    "TOPS": round(ops / (tq * 1e-3) / 1e12, 3),
                    "roofline": roofline("hbm" if name == "cfg3a" else "mfma-int8",
                                         c["qbytes"] if name == "cfg3a" else ops, tq,
                                         "step (k_i8mm max pass + s8 pass, or for K >= 512 "
                                         "k_i8mm fp32 pass + k_requant_s8)",
                                         (f"int8 I/O {c['qbytes'] / 1e6:.1f} MB per step" if name == "cfg3a"
                                          else f"{ops / 1e9:.2f} GOP per step (MFMA-bound with int8 I/O)")
                                         + " (acfun_dev_conv2d_int8_q)"),
                    "frac_int8_peak": round(ops / (tq * 1e-3) / PEAK_INT8, 4),
                    "kernel_ms": kq}}

        # 4(a): fused depthwise + BN + ReLU + MaxPool
        c = cfg["cfg4a"]
        t = T.run(c["step"], steps, args.warmup, CFG_REPS)
        k = T.kernel_ms(lib, c["step"], steps, ["k_dwconv_pool"])
        fn, xt, zt = c["rot"]
        xs, zs = rotation_sets(xt, zt)
        tc = T.run(rotating(fn, xs, zs), steps, args.warmup, CFG_REPS)
        del xs, zs
        configs["cfg4a_dw_bn_relu_pool"] = {
            "ms": round(t, 5), "ms_cold": round(tc, 5),
            "roofline": roofline("hbm", c["bytes"], k["k_dwconv_pool"], "k_dwconv3_pool_rs",
                                 "163.8 MB per launch: the input read and the pooled output written "
                                 "once (fused)", "k_dwconv_pool_cfg4a"),
            "frac_hbm_cold_step": round(c["bytes"] / (tc * 1e-3) / PEAK_HBM, 4)}

        # 4(b): grouped conv + ReLU + MaxPool fused; the two-launch path beside
        # it; and the fused step replayed from a HIP graph (launch cost removed)
        c = cfg["cfg4b"]
        t = T.run(c["step"], steps, args.warmup, CFG_REPS)
        k = T.kernel_ms(lib, c["step"], steps, ["k_gconv_pool"])
        fn, xt, zt = c["rot"]
        xs, zs = rotation_sets(xt, zt)
        tc = T.run(rotating(fn, xs, zs), steps, args.warmup, CFG_REPS)
        del xs, zs
        t2 = T.run(c["two"], steps, args.warmup, CFG_REPS)
        per_graph = 10
        graph = torch.cuda.CUDAGraph()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            for _ in range(per_graph):
                c["step"]()
        tg = T.run(graph.replay, max(2, steps // 2), 2, CFG_REPS) / per_graph
        configs["cfg4b_grouped_pool"] = {
            "ms": round(t, 5), "ms_cold": round(tc, 5), "ms_graph_replay": round(tg, 5),
            "ms_two_launches": round(t2, 5),
            "roofline": roofline("hbm", c["bytes"], k["k_gconv_pool"], "k_gconv3_pool_row<1>",
                                 f"{c['bytes'] / 1e6:.2f} MB per launch (input once, pooled output "
                                 "once); latency-bound at this size", "k_gconv_pool_cfg4b"),
            "kernel_ms": k}

        # 5: ResNet-50-style, batch 64, fp32 and int8
        for tag, int8 in (("fp32", False), ("int8", True)):
            m, path, xin, out = load_cfg5(lib, torch, dev, rng, cfg, int8)
            if not m:
                configs[f"cfg5_resnet50_b64_{tag}"] = {"error": capi.last_error()}
                continue
            s6 = lambda m=m, xin=xin, out=out: check_infer(lib, m, xin, out, sp)
            t = T.run(s6, max(3, steps // 4), 2, 3)
            rows, _ = model_layer_profile(lib, s6)
            gfl = acfun0.resnet50_flops()
            configs[f"cfg5_resnet50_b64_{tag}"] = {
                "ms": round(t, 3), "images_per_s": round(64 / (t * 1e-3), 1),
                "TFLOPS_direct_equivalent": round(64 * gfl / (t * 1e-3) / 1e12, 3),
                "direct_work": f"{gfl / 1e9:.2f} GFLOP per image (convs and FC, direct count)",
                "roofline": cfg5_roofline(rows, t, int8),
                "per_layer": "profiles/kernels_cfg5_%s.md (bench.py --profile cfg5_%s)" % (tag, tag)}
            lib.acfun_model_destroy(m)
            os.unlink(path)
    line["configs"] = configs
    line["config"]["tile_search"] = lib.acfun_tune_status().decode()

    # ---------------------------------------------------------------- CPU baselines
    if not args.no_cpu:
        cpu_baselines(cfg, configs, line)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
