#!/usr/bin/env python3
"""Benchmark of the int4/int8 quantized-inference path on one MI355X.

Headline (BASELINE.json ``metric``): int4-g128 GEMV HBM GB/s at
M=1 x K=4096 x N=11008 (fp16 activations / scales / output, fp32 accumulate).
A step is one launch of the dequant-matvec over one batch (one activation
row).  The same JSON line carries the prefill GEMM TFLOP/s and the other
configurations under ``extra``.

Method:
  * inputs are uploaded once and resident in HBM before timing;
  * each configuration cycles through R weight/scale replicas whose total
    exceeds MI355X's 256 MB Infinity Cache, so weights stream from HBM;
  * a trial is one replay of a HIP graph holding `--steps` launches
    (torch.cuda.CUDAGraph over the library's launches on the capture stream),
    so host launch cost does not gap the GPU; HIP events on that stream
    bracket each of 21 trials, enqueued back to back; a launch's time is the
    median trial / `--steps`;
  * roofline.achieved = algorithmic bytes (or FLOPs) per launch / that
    median; roofline.achievable = the library's streaming-read kernel over
    the same weight replicas, timed the same way (the rate a pure read of a
    buffer that size reaches on this part).
The CPU baseline is the oracle's restatement of the reference NumPy path
(examples/38_quantized_matmul.py:215-232), timed on this host on the same
inputs, median of timed runs after warm-up as in
examples/38_quantized_matmul.py:300-340.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
LLC_BYTES = 256 << 20
METRIC = "W4 GEMV HBM GB/s (% of peak) @1x4096x11008; W4 prefill GEMM TFLOP/s"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


class Case:
    """One dequant-matmul / dequant configuration with device replicas."""

    def __init__(self, kind, wbits, M, N, K, G, lo, hi, seed=0, min_bytes=LLC_BYTES * 5 // 4,
                 max_replicas=64, xd="f16"):
        """xd: activation dtype "f16" (fp16 scales and outputs), "bf16" (fp16
        scales, bf16 outputs) or "f32" (fp32 scales and outputs, the
        reference's own dtypes)."""
        import torch
        from locomp_amd import synth, _lib
        self.kind, self.wbits, self.M, self.N, self.K, self.G = kind, wbits, M, N, K, G
        self.codes = {"f16": (1, 1, 1), "bf16": (2, 1, 2), "f32": (0, 0, 0)}[xd]
        xt = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[xd]
        if kind == "dequant":
            W, S = synth.dequant_case(wbits, N, K, G, lo, hi, seed=seed)
            X = None
        else:
            X, W, S = synth.matvec_case(wbits, M, N, K, G, lo, hi, seed=seed)
            if xd == "f32":
                S = S.astype(np.float32)
        self.host = (X, W, S)
        self.w_bytes = W.nbytes
        self.s_bytes = S.nbytes
        esz = 4 if xd == "f32" else 2
        if kind == "dequant":
            self.out_elems = N * K
            self.algo_bytes = W.nbytes + S.nbytes + N * K * 2
            self.flops = 0
        else:
            self.out_elems = M * N
            self.algo_bytes = W.nbytes + S.nbytes + M * K * esz + M * N * esz
            self.flops = 2 * M * N * K
        per = W.nbytes + S.nbytes + (self.out_elems * 2 if kind == "dequant" else 0)
        self.R = max(1, min(max_replicas, math.ceil(min_bytes / per)))
        w0, s0 = _dev(W), _dev(S)
        self.W = [w0] + [w0.clone() for _ in range(self.R - 1)]
        self.S = [s0] + [s0.clone() for _ in range(self.R - 1)]
        self.X = _dev(X.astype(np.float32)).to(xt) if X is not None else None
        nout = self.R if kind == "dequant" else 1
        ot = torch.float16 if kind == "dequant" else {"f16": torch.float16, "bf16": torch.bfloat16,
                                                       "f32": torch.float32}[xd]
        self.O = [torch.empty(self.out_elems, dtype=ot, device="cuda") for _ in range(nout)]
        self.lib = _lib.load()
        torch.cuda.synchronize()

    def launch(self, i, stream):
        r = i % self.R
        lib, K, G, N, M = self.lib, self.K, self.G, self.N, self.M
        vp = ctypes.c_void_p
        if self.kind == "dequant":
            fn = lib.locomp_amd_dequant_int4 if self.wbits == 4 else None
            rc = fn(vp(self.W[r].data_ptr()), vp(self.S[r].data_ptr()), vp(self.O[r].data_ptr()),
                    K, K // 2, K // G, G, N, 1, 1, stream)
        elif self.wbits == 4:
            rc = lib.locomp_amd_dequant_matvec_int4(
                vp(self.X.data_ptr()), vp(self.W[r].data_ptr()), vp(self.S[r].data_ptr()),
                vp(self.O[0].data_ptr()), K, K // 2, K // G, G, N, M, *self.codes, stream)
        else:
            rc = lib.locomp_amd_dequant_matvec_int8(
                vp(self.X.data_ptr()), vp(self.W[r].data_ptr()), vp(self.S[r].data_ptr()),
                vp(self.O[0].data_ptr()), K, K // G, G, N, M, *self.codes, stream)
        if rc != 0:
            raise RuntimeError(f"launch failed: {rc}")

    def result(self):
        return self.O[0].cpu().numpy()


class QuantCase:
    """GPU weight producer (quantize_int4 of examples/38:248-271): float32
    weights [N, K] -> packed int4 + float32 scales, weight replicas rotated."""

    def __init__(self, N, K, G, seed=0, min_bytes=LLC_BYTES * 5 // 4):
        import torch
        from locomp_amd import _lib
        self.N, self.K, self.G = N, K, G
        rng = np.random.default_rng(seed)
        w0 = _dev(rng.standard_normal((N, K), dtype=np.float32))
        self.R = max(1, math.ceil(min_bytes / w0.numel() / 4))
        self.W = [w0] + [w0.clone() for _ in range(self.R - 1)]
        self.Q = torch.empty(N * K // 2, dtype=torch.uint8, device="cuda")
        self.S = torch.empty(N * (K // G), dtype=torch.float32, device="cuda")
        self.algo_bytes = N * K * 4 + N * K // 2 + N * (K // G) * 4
        self.flops = 0
        self.lib = _lib.load()
        torch.cuda.synchronize()

    def launch(self, i, stream):
        vp = ctypes.c_void_p
        rc = self.lib.locomp_amd_quantize_int4(vp(self.W[i % self.R].data_ptr()), vp(self.Q.data_ptr()),
                                               vp(self.S.data_ptr()), self.N, self.K, self.G, 0, 0, stream)
        if rc != 0:
            raise RuntimeError(f"launch failed: {rc}")


def time_graph(case, steps, warmup, trials=21, per_graph=None):
    """Median time of one launch, from `trials` replays of a graph of launches.

    `warmup` eager launches come first (first-launch costs), then `per_graph`
    launches (default `steps`, rotating the case's weight replicas) are
    captured in one HIP graph, replayed once untimed, then replayed `trials`
    times with a HIP event recorded on the capture stream before each replay
    and after the last, all enqueued back to back.  Returns (median seconds
    per launch, {"trials", "launches_per_trial", "min_us", "max_us"})."""
    import torch
    per_graph = max(1, per_graph or steps)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(max(1, warmup)):
            case.launch(i, ctypes.c_void_p(s.cuda_stream))
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for i in range(per_graph):
            case.launch(i, ctypes.c_void_p(s.cuda_stream))
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(trials + 1)]
    with torch.cuda.stream(s):
        g.replay()
        torch.cuda.synchronize()
        ev[0].record(s)
        for t in range(trials):
            g.replay()
            ev[t + 1].record(s)
    torch.cuda.synchronize()
    per = sorted(ev[t].elapsed_time(ev[t + 1]) / 1e3 / per_graph for t in range(trials))
    med = per[len(per) // 2]
    del g
    return med, {"trials": trials, "launches_per_trial": per_graph,
                 "min_us": round(per[0] * 1e6, 3), "max_us": round(per[-1] * 1e6, 3)}


class StreamCase:
    """The library's streaming-read kernel over a case's weight replicas: the
    achievable HBM read rate for a buffer of that size on this part."""

    def __init__(self, case):
        import torch
        from locomp_amd import _lib
        self.W, self.R = case.W, case.R
        self.nbytes = case.W[0].numel() // 1024 * 1024
        self.sink = torch.zeros(4, dtype=torch.int32, device="cuda")
        self.lib = _lib.load()

    def launch(self, i, stream):
        rc = self.lib.locomp_amd_stream_read(ctypes.c_void_p(self.W[i % self.R].data_ptr()),
                                             self.nbytes, ctypes.c_void_p(self.sink.data_ptr()),
                                             stream)
        if rc != 0:
            raise RuntimeError(f"stream_read failed: {rc}")


class BigStream:
    """The streaming-read kernel over one buffer of `nbytes` (well above the
    256 MB Infinity Cache): the asymptotic HBM read rate, free of the
    per-launch fixed cost that dominates a 22.5 MB read."""

    def __init__(self, nbytes=512 << 20):
        import torch
        from locomp_amd import _lib
        self.nbytes = nbytes
        self.buf = torch.randint(0, 255, (nbytes,), dtype=torch.uint8, device="cuda")
        self.sink = torch.zeros(4, dtype=torch.int32, device="cuda")
        self.lib = _lib.load()
        self.R = 1

    def launch(self, i, stream):
        rc = self.lib.locomp_amd_stream_read(ctypes.c_void_p(self.buf.data_ptr()), self.nbytes,
                                             ctypes.c_void_p(self.sink.data_ptr()), stream)
        if rc != 0:
            raise RuntimeError(f"stream_read failed: {rc}")


def cpu_baseline(case, budget_s=20.0, unit="GB/s"):
    """Oracle (restated reference NumPy path) on the host, same inputs, timed
    like the reference (examples/38_quantized_matmul.py:300-302, 323-340:
    warm-ups, then the median of repeated calls): the dequant-matmul through
    fast_numpy_matvec_int4 / int8 (:215-241), the dequantize through
    dequant_int4_ref (examples/52_dequantize.py:129-143).  `unit` is the
    metric of the GPU line it sits beside (GB/s of algorithmic bytes, or
    TFLOP/s)."""
    from oracle import quant_ref as ref
    X, W, S = case.host
    try:
        from threadpoolctl import threadpool_info
        blas_threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:
        blas_threads = int(os.environ.get("OPENBLAS_NUM_THREADS", os.environ.get("OMP_NUM_THREADS", "1")))

    if case.kind == "dequant":
        what = "dequant_int4_ref (examples/52_dequantize.py:129-143)"

        def run():
            return ref.dequant_int4_ref(W, S, case.N, case.K, case.G).astype(np.float16)
    else:
        f = ref.fast_numpy_matvec_int4 if case.wbits == 4 else ref.fast_numpy_matvec_int8
        what = (f"fast_numpy_matvec_int{case.wbits} (examples/38_quantized_matmul.py:"
                f"{'215-232' if case.wbits == 4 else '235-241'})")
        Xh = X.astype(np.float32)

        def run():
            return f(Xh if case.M > 1 else Xh[0], W, S.astype(np.float32), case.G)

    t0 = time.perf_counter()
    run()
    one = time.perf_counter() - t0
    warm = 5 if one < budget_s / 20 else 1
    runs = int(max(3, min(15, budget_s / max(one, 1e-3) - warm)))
    for _ in range(warm):
        run()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t0)
    med = sorted(ts)[len(ts) // 2]
    value = case.flops / med / 1e12 if unit == "TFLOP/s" else case.algo_bytes / med / 1e9
    shape = (f"{case.N} x {case.K} g{case.G}" if case.kind == "dequant"
             else f"M={case.M} x {case.K} x {case.N} g{case.G}")
    threads = ("elementwise NumPy only, single-threaded" if case.kind == "dequant" else
               f"elementwise NumPy is single-threaded, the BLAS product used {blas_threads} threads")
    return {
        "value": round(value, 4), "unit": unit,
        "cores": 1 if case.kind == "dequant" else int(blas_threads),
        "kind": "port",
        "sample": (f"oracle {what} on the full {shape} inputs, median of {runs} runs after "
                   f"{warm} warm-up(s), {med * 1e3:.1f} ms/call; {threads}; host "
                   f"os.cpu_count()={os.cpu_count()}, affinity={len(os.sched_getaffinity(0))}"),
    }


def profile_case(name, launches=50):
    """Eager launches of one configuration (rotating replicas), for rocprofv3.

    "copy" copies a 64 MiB device buffer (torch copy_): its FETCH_SIZE /
    WRITE_SIZE per dispatch calibrate the counters against known bytes."""
    import torch
    from locomp_amd import synth
    s = torch.cuda.current_stream()
    if name == "copy":
        a = torch.empty(64 << 20, dtype=torch.uint8, device="cuda").fill_(1)
        b = torch.empty_like(a)
        for _ in range(launches):
            b.copy_(a)
        torch.cuda.synchronize()
        print("copy: 67108864 bytes read + 67108864 written per dispatch")
        return 0
    c3, c2, c4, c5 = synth.CFG3, synth.CFG2, synth.CFG4, synth.CFG5A
    case = {
        "gemv": lambda: Case("matvec", 4, 1, c3["N"], c3["K"], c3["G"], c3["lo"], c3["hi"]),
        "gemv_m16": lambda: Case("matvec", 4, 16, c3["N"], c3["K"], c3["G"], c3["lo"], c3["hi"]),
        "gemm": lambda: Case("matvec", 4, c5["M"], c5["N"], c5["K"], c5["G"], c5["lo"], c5["hi"],
                             min_bytes=0, max_replicas=4),
        "dequant": lambda: Case("dequant", 4, 0, c2["N"], c2["K"], c2["G"], c2["lo"], c2["hi"]),
        "w8a16": lambda: Case("matvec", 8, c4["M"], c4["N"], c4["K"], c4["G"], c4["lo"], c4["hi"]),
    }[name]()
    for i in range(launches):
        case.launch(i, ctypes.c_void_p(s.cuda_stream))
    torch.cuda.synchronize()
    print(f"{name}: {launches} launches, {case.algo_bytes} algorithmic bytes per launch")
    return 0


SWEEP_M = (1, 2, 4, 8, 16, 32, 64, 96, 256, 1024)
SWEEP_SHAPES = ((576, 576), (1536, 576), (576, 1536), (4096, 4096), (11008, 4096), (4096, 11008),
                (14336, 4096), (4096, 14336))   # (N, K): SmolLM2-135M, LLaMA-7B / 8B-class linear layers


def sweep():
    """Microseconds per dequant-matmul launch (graph replays, weights rotated
    through replicas larger than the Infinity Cache) over SWEEP_M x
    SWEEP_SHAPES, int4 G = 32 / 128 and int8 G = 128 / per-channel; one
    Markdown table on stdout."""
    import torch
    print("| bits | N | K | G | " + " | ".join(f"M={m}" for m in SWEEP_M) + " |")
    print("|---|---|---|---|" + "---|" * len(SWEEP_M))
    for wb in (4, 8):
        for N, K in SWEEP_SHAPES:
            for G in ((32, 128) if wb == 4 else (128, K)):
                if K % G:
                    continue
                cells = []
                for M in SWEEP_M:
                    case = Case("matvec", wb, M, N, K, G, 0.001, 0.01, max_replicas=16)
                    t, _ = time_graph(case, max(20, case.R), 5, trials=11)
                    cells.append(f"{t * 1e6:.1f}")
                    del case
                    torch.cuda.empty_cache()
                print(f"| {wb} | {N} | {K} | {G} | " + " | ".join(cells) + " |", flush=True)
    return 0


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200,
                    help="launches per timed trial (the headline's median is over 21 trials)")
    ap.add_argument("--warmup", type=int, default=20, help="eager launches before capture")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", default="", help="comma list of extra cases to run (default all)")
    ap.add_argument("--profile", default="", choices=["", "gemv", "gemv_m16", "gemm", "dequant", "w8a16", "copy"],
                    help="launch one case 50 times eagerly and exit (for rocprofv3 counter passes)")
    ap.add_argument("--sweep", action="store_true",
                    help="time the dequant-matmul over a grid of M and linear-layer shapes, print a table")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        return 2

    import torch
    if not torch.cuda.is_available():
        print("no HIP device visible", file=sys.stderr)
        return 1
    from locomp_amd import synth

    if args.profile:
        return profile_case(args.profile)
    if args.sweep:
        return sweep()

    c3 = synth.CFG3
    log("case gemv_w4a16 M=1")
    head = Case("matvec", 4, 1, c3["N"], c3["K"], c3["G"], c3["lo"], c3["hi"])
    t, tinfo = time_graph(head, args.steps, args.warmup)
    us = t * 1e6
    gbs = head.algo_bytes / t / 1e9
    log("case stream_read (achievable HBM read rate, same weight replicas)")
    sc = StreamCase(head)
    ts, sinfo = time_graph(sc, args.steps, args.warmup)
    stream_gbs = sc.nbytes / ts / 1e9

    extra = {}
    only = set(filter(None, args.only.split(","))) if args.only else None

    def want(name):
        return only is None or name in only

    def run_case(name, case, bound, cpu=False):
        per, info = time_graph(case, max(20, case.R), 5)
        d = {"us_per_launch": round(per * 1e6, 3), "GB_s": round(case.algo_bytes / per / 1e9, 1),
             "replicas": case.R, **info}
        if case.flops:
            d["TFLOP_s"] = round(case.flops / per / 1e12, 2)
        if bound == "hbm":
            d["frac_hbm"] = round(case.algo_bytes / per / 1e9 / HBM_PEAK_GBS, 4)
        else:
            d["frac_mfma_f16"] = round(case.flops / per / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)
        if cpu and not args.no_cpu:
            # the reference's NumPy path beside this line, same inputs
            d["cpu_baseline"] = cpu_baseline(case, 8.0, "GB/s" if bound == "hbm" else "TFLOP/s")
        extra[name] = d
        log(name, d)

    if want("gemm_prefill"):
        c = synth.CFG5A
        run_case("gemm_prefill_w4a16_2048x4096x4096_g128",
                 Case("matvec", 4, c["M"], c["N"], c["K"], c["G"], c["lo"], c["hi"],
                      min_bytes=0, max_replicas=4), "mfma", cpu=True)
    if want("gemm_prefill_w8"):
        c = synth.CFG5A
        run_case("gemm_prefill_w8a16_2048x4096x4096_g128",
                 Case("matvec", 8, c["M"], c["N"], c["K"], c["G"], 0.002, 0.02,
                      min_bytes=0, max_replicas=4), "mfma")
    if want("gemm_prefill_small"):
        c = synth.CFG5A
        for M in (128, 512):      # split-K shapes (fewer output tiles than CUs)
            run_case(f"gemm_prefill_w4a16_{M}x4096x4096_g128",
                     Case("matvec", 4, M, c["N"], c["K"], c["G"], c["lo"], c["hi"]), "mfma")
    for M in (4, 16):
        if want(f"gemv_m{M}"):
            run_case(f"gemv_w4a16_M{M}", Case("matvec", 4, M, c3["N"], c3["K"], c3["G"], c3["lo"],
                                                c3["hi"]), "hbm")
    for xd in ("bf16", "f32"):
        for M in (1, 4, 16):
            if want(f"gemv_{xd}"):
                run_case(f"gemv_w4a{xd}_M{M}", Case("matvec", 4, M, c3["N"], c3["K"], c3["G"],
                                                              c3["lo"], c3["hi"], xd=xd), "hbm")
    if want("gemv_g16"):
        # scale groups of 16 (G % 32 != 0): the row kernel with a scale per 16 k
        # at M = 1, the fp32-FMA / dot2 VALU kernel at M = 16
        for xd, M in (("f16", 1), ("f16", 16), ("f32", 16)):
            run_case(f"gemv_w4a{'16' if xd == 'f16' else xd}_g16_M{M}",
                     Case("matvec", 4, M, c3["N"], c3["K"], 16, c3["lo"], c3["hi"], xd=xd), "hbm")
    if want("gemm_prefill_bf16"):
        c = synth.CFG5A
        run_case("gemm_prefill_w4abf16_2048x4096x4096_g128",
                 Case("matvec", 4, c["M"], c["N"], c["K"], c["G"], c["lo"], c["hi"],
                      min_bytes=0, max_replicas=4, xd="bf16"), "mfma")
    if want("cfg1"):
        # BASELINE cfg 1, the reference's CPU-runnable case: W8A32, X fp32
        # [4, 512], int8 [512, 512], per-channel fp32 scales, fp32 output
        c = synth.CFG1
        run_case("w8a32_M4_512x512_cfg1",
                 Case("matvec", 8, c["M"], c["N"], c["K"], c["G"], c["lo"], c["hi"], xd="f32"), "hbm")
    if want("gemm_prefill_f32"):
        # fp32 activations (the reference's dtype): two round-to-nearest
        # bf16 parts per row as 2 M rows on the bf16 GEMM, each row's pair
        # of part products added in its epilogue
        c = synth.CFG5A
        run_case("gemm_prefill_w4af32_2048x4096x4096_g128",
                 Case("matvec", 4, c["M"], c["N"], c["K"], c["G"], c["lo"], c["hi"],
                      min_bytes=0, max_replicas=4, xd="f32"), "mfma")
    if want("launch_floor"):
        # one 1 KB streaming read per launch: the per-launch cost of a graph
        # node on this part, which bounds a stack of small dependent launches
        class Tiny:
            def __init__(self):
                import torch
                from locomp_amd import _lib
                self.buf = torch.zeros(1024, dtype=torch.uint8, device="cuda")
                self.sink = torch.zeros(4, dtype=torch.int32, device="cuda")
                self.lib = _lib.load()

            def launch(self, i, stream):
                vp = ctypes.c_void_p
                if self.lib.locomp_amd_stream_read(vp(self.buf.data_ptr()), 1024,
                                                   vp(self.sink.data_ptr()), stream) != 0:
                    raise RuntimeError("stream_read failed")
        per, _ = time_graph(Tiny(), 120, 5)
        extra["launch_floor_1KB_read"] = {"us_per_launch": round(per * 1e6, 3)}
        log("launch_floor_1KB_read", extra["launch_floor_1KB_read"])
    if want("gemv_floor") and "launch_floor_1KB_read" in extra:
        # Per-launch lower bounds of the headline GEMV: (a) the graph-node
        # floor plus its algorithmic bytes at the 8 TB/s peak; (b) the same
        # bytes at the asymptotic read rate measured here (a 512 MB streaming
        # read) plus the fixed cost that the 22.5 MB streaming read of the
        # weight replicas shows on top of that rate
        big = BigStream()
        tb, _ = time_graph(big, 4, 2)
        rate = big.nbytes / tb                      # bytes / s
        fixed = ts - sc.nbytes / rate               # s, per 22.5 MB launch
        floor = extra["launch_floor_1KB_read"]["us_per_launch"]
        extra["gemv_w4a16_m1_floor"] = {
            "launch_floor_us": floor,
            "peak_bound_us": round(floor + head.algo_bytes / (HBM_PEAK_GBS * 1e3), 3),
            "stream_read_22MB_us": round(ts * 1e6, 3),
            "stream_read_512MB_us": round(tb * 1e6, 2),
            "asymptotic_read_GB_s": round(rate / 1e9, 1),
            "fixed_cost_us": round(fixed * 1e6, 3),
            "achievable_bound_us": round((fixed + head.algo_bytes / rate) * 1e6, 3),
            "gemv_us": round(us, 3),
            "note": ("peak_bound = graph-node floor + 23,279,104 B at 8 TB/s; achievable_bound = "
                     "fixed cost of a 22.5 MB streaming read + the GEMV's bytes at the 512 MB "
                     "read rate"),
        }
        log("gemv_w4a16_m1_floor", extra["gemv_w4a16_m1_floor"])
    if want("dequant"):
        c = synth.CFG2
        run_case("dequant_int4_4096x4096_g32_f16",
                 Case("dequant", 4, 0, c["N"], c["K"], c["G"], c["lo"], c["hi"]), "hbm", cpu=True)
    if want("quantize"):
        run_case("quantize_int4_4096x4096_g32_from_f32", QuantCase(4096, 4096, 32), "hbm")
    if want("smollm2"):
        # SmolLM2-135M-shaped decode step (locomp_amd.stack), every variant
        # ending with the 49152 x 576 LM head; the chained ones run the
        # reference's per-layer order with the RMSNorms and residual adds
        from locomp_amd.stack import DecodeStack
        # (the _fused_norm_residual ones fold the norms and residual adds
        # into the linears: 4 launches per layer instead of 6)
        for fused, silu, chain, f32, fn in ((False, False, False, False, False),
                                            (True, False, False, False, False),
                                            (True, True, False, False, False),
                                            (True, True, True, False, False),
                                            (True, True, True, True, False),
                                            (True, True, True, False, True),
                                            (True, True, True, True, True)):
            st = DecodeStack(fused=fused, silu=silu, chain=chain, f32=f32, fuse_norm=fn)
            per, _ = time_graph(st, 4, 1)
            d = {"us_per_token": round(per * 1e6, 2), "GB_s": round(st.algo_bytes / per / 1e9, 1),
                 "gemvs_per_token": st.gemvs, "launches_per_token": len(st.links),
                 "algorithmic_bytes": st.algo_bytes,
                 "us_per_launch": round(per * 1e6 / len(st.links), 3)}
            name = "smollm2_135m_int4_g32_decode_step" + ("_qkv_gateup_fused" if fused else "") + \
                ("_silu_epilogue" if silu else "") + \
                ("_chained_fused_norm_residual" if fn else "_chained_rmsnorm_residual" if chain else "") + \
                "_lm_head" + ("_fp32_activations" if f32 else "")
            extra[name] = d
            log(name, d)
    if want("w8a16"):
        c = synth.CFG4
        run_case("w8a16_M64_14336x4096",
                 Case("matvec", 8, c["M"], c["N"], c["K"], c["G"], c["lo"], c["hi"]), "hbm", cpu=True)

    cpu = None if args.no_cpu else cpu_baseline(head)
    traffic = None
    tpath = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "gemv_w4a16_m1_traffic.json")
    if os.path.exists(tpath):   # HBM bytes per launch from the committed rocprofv3 PMC passes
        with open(tpath) as f:
            traffic = int(json.load(f)["traffic_bytes"])

    line = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "trials": tinfo["trials"],
        "ms_per_step": round(us / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded np.random.default_rng(0), draw order X, W, S)",
        "config": {"workload": "gemv_w4a16 int4-g128 M=1 K=4096 N=11008, fp16 X/scales/Y, "
                               "fp32 accumulate", "M": 1, "K": 4096, "N": 11008, "group": 128,
                   "weight_replicas": head.R},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "algorithmic_bytes_per_launch": head.algo_bytes,
                     "median_launch_us": round(us, 3), "min_launch_us": tinfo["min_us"],
                     "max_launch_us": tinfo["max_us"],
                     "achievable": round(stream_gbs, 1),
                     "achievable_note": (f"stream_read of the same {sc.nbytes} B weight replicas, "
                                         f"{ts * 1e6:.3f} us per launch, median of "
                                         f"{sinfo['trials']} trials"),
                     "frac_of_achievable": round(gbs / stream_gbs, 4)},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
