#!/usr/bin/env python3
"""Benchmark of the quantized decode GEMV path on one MI355X.

Workload: the decode-step GEMV set of one
Qwen3.5-0.8B-shaped layer at batch 1 -- Q4_K gate and up (3584x1024),
Q6_K down (1024x3584), Q5_K 2048x1024, 512x1024 and 1024x2048, Q8_0
1024x1024 -- random blocks per the BASELINE recipe, activations already
quantized (Q8_K / Q8_0) and resident in HBM. One step is one fused launch
(hip_matvec_group) over the seven matrices. Steps rotate through enough
distinct weight copies (> 512 MB) that every step streams its weights
from HBM rather than the 256 MB MALL.

metric: GB/s of algorithmic bytes (weights + quantized activations + fp32
outputs, 11,560,856 B per step) over the timed steps.

Also reported under "extra": config 0 (single Q4_K GEMV), config 2 (LM
head with fused argmax / top-40), config 3 (prefill GEMM) when available.
The CPU baseline times the reference's own tensor_matmul_* (oracle/_ref,
compiled from its sources) on this host's cores over a bounded sample.
"""
import argparse
import ctypes as C
import importlib.util
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))

CONFIG1 = [(12, 3584, 1024), (12, 3584, 1024), (14, 1024, 3584), (13, 2048, 1024),
           (13, 512, 1024), (13, 1024, 2048), (8, 1024, 1024)]
HBM_PEAK_GBS = 8000.0
MALL_DEFEAT_BYTES = 512 << 20
# HBM bytes per config-1 launch of the current k_gemv, from rocprofv3 --pmc
# FETCH_SIZE and WRITE_SIZE runs of this script (--copy-probe 256), each
# scaled by its reading for a known-size copy / fill (FETCH x2.000,
# WRITE x1.000); the runs are recorded in profiles/k_gemv_decode_set_lmhead.md.
# None when the kernel has changed since the last counter run.
CONFIG1_TRAFFIC_BYTES = 11_997_184 + 55_296


def _load(rel, name):
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, os.path.join(ROOT, rel))
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def alg_bytes(wtype, n, k):
    bb = {8: 34, 12: 144, 13: 176, 14: 210}[wtype]
    be = 32 if wtype == 8 else 256
    xq = (k // 32) * 34 if wtype == 8 else (k // 256) * 292
    return n * (k // be) * bb + xq + 4 * n


class Events:
    """HIP events on the stream the kernels run on."""

    def __init__(self, torch):
        self.torch = torch

    def time(self, fn, steps, warmup):
        torch = self.torch
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        s = torch.cuda.current_stream()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for i in range(steps):
            fn(warmup + i)
        e1.record(s)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / 1e3            # seconds


def bench_config1(torch, qk, synth, lib, steps, warmup, warm=False):
    """Config 1 (the metric). warm=True: one weight copy, so the 11.5 MB
    stay in the 256 MB MALL between steps (a labelled warm-cache figure,
    never the metric)."""
    per_set = sum(alg_bytes(*s) for s in CONFIG1)
    wbytes = sum(alg_bytes(*s) - ((s[2] // 32) * 34 if s[0] == 8 else (s[2] // 256) * 292) - 4 * s[1] for s in CONFIG1)
    copies = 1 if warm else max(2, -(-MALL_DEFEAT_BYTES // wbytes))
    base = []
    for i, (t, n, k) in enumerate(CONFIG1):
        w = torch.from_numpy(synth.blocks(t, n, k, seed=0, tag=i)).cuda()
        x = torch.from_numpy(synth.activations(1, k, seed=0, tag=i)).cuda()
        xq = lib.quantize_for(t, x)[0]
        base.append((t, w, n, k, xq))
    sets = []
    for c in range(copies):
        items = []
        for (t, w, n, k, xq) in base:
            wc = w if c == 0 else w.clone()
            items.append((t, wc, n, k, xq, torch.empty(n, dtype=torch.float32, device="cuda")))
        sets.append(items)
    descs = []
    for items in sets:
        arr = (qk.GemvDesc * len(items))()
        for i, (t, w, n, k, xq, y) in enumerate(items):
            arr[i] = qk.GemvDesc(t, 0, n, k, w.data_ptr(), xq.data_ptr(), y.data_ptr())
        descs.append(arr)
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    fn = lib.L.hip_matvec_group

    def step(i):
        if fn(descs[i % copies], len(CONFIG1), stream):
            raise RuntimeError(lib.last_error())

    secs = Events(torch).time(step, steps, warmup)
    return per_set, copies, secs


def config1_each(torch, qk, synth, lib, steps):
    """Each distinct config-1 matrix alone (one-descriptor launches), then
    the set, `steps` launches each, for per-kernel counters: a profiling
    aid, not a benchmark figure (one weight copy)."""
    items, seen, out = [], set(), {}
    for i, (t, n, k) in enumerate(CONFIG1):
        w = torch.from_numpy(synth.blocks(t, n, k, seed=0, tag=i)).cuda()
        x = torch.from_numpy(synth.activations(1, k, seed=0, tag=i)).cuda()
        items.append((t, w, n, k, lib.quantize_for(t, x)[0], torch.empty(n, dtype=torch.float32, device="cuda")))
    ev = Events(torch)
    for it in items:
        key = f"{it[0]}_{it[2]}x{it[3]}"
        if key in seen:
            continue
        seen.add(key)
        out[key] = round(ev.time(lambda i: lib.matvec_group([it]), steps, 2) / steps * 1e6, 3)
    out["set"] = round(ev.time(lambda i: lib.matvec_group(items), steps, 2) / steps * 1e6, 3)
    return out


def bench_config0(torch, qk, synth, lib, steps, warmup):
    t, n, k = 12, 3584, 1024
    per = alg_bytes(t, n, k)
    copies = -(-MALL_DEFEAT_BYTES // (per - 292 * 4 - 4 * n))
    w = torch.from_numpy(synth.blocks(t, n, k, seed=0)).cuda()
    ws = [w] + [w.clone() for _ in range(copies - 1)]
    xq = lib.quantize_q8k(torch.from_numpy(synth.activations(1, k, seed=0)).cuda())[0]
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    # direct C calls with prebuilt pointers: a 2 MB GEMV is shorter than
    # the binding's Python-side checks
    wp = [C.c_void_p(x.data_ptr()) for x in ws]
    xp, yp = C.c_void_p(xq.data_ptr()), C.c_void_p(y.data_ptr())
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    fn = lib.L.hip_matvec_q4k

    def step(i):
        if fn(wp[i % copies], n, k, xp, yp, stream):
            raise RuntimeError(lib.last_error())

    secs = Events(torch).time(step, steps, warmup)
    return per, copies, secs


def bench_config2(torch, qk, synth, lib, steps, warmup):
    n, k, topk = 248320, 1024, 40
    w = torch.from_numpy(synth.blocks(14, n, k, seed=0)).cuda()
    copies = 3                                        # 3 x 209 MB > 512 MB
    ws = [w] + [w.clone() for _ in range(copies - 1)]
    xq = lib.quantize_q8k(torch.from_numpy(synth.activations(1, k, seed=0)).cuda())[0]
    logits = torch.empty(n, dtype=torch.float32, device="cuda")
    am = torch.empty(1, dtype=torch.int32, device="cuda")
    ti = torch.empty(topk, dtype=torch.int32, device="cuda")
    tv = torch.empty(topk, dtype=torch.float32, device="cuda")
    lib.lmhead(w, n, k, xq, topk=topk, logits=logits)  # checked once through the binding
    # the timed loop calls the C ABI directly with preallocated outputs, so
    # host-side Python does not pace the launches
    f = lib.L.hip_lmhead_q6k_argmax_topk
    wp = [C.c_void_p(t.data_ptr()) for t in ws]
    xp, lp = C.c_void_p(xq.data_ptr()), C.c_void_p(logits.data_ptr())
    ap, ip, vp = C.c_void_p(am.data_ptr()), C.c_void_p(ti.data_ptr()), C.c_void_p(tv.data_ptr())
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    per = n * 4 * 210 + 4 * 292 + 4 * n
    secs = Events(torch).time(lambda i: f(wp[i % copies], n, k, xp, topk, lp, ap, ip, vp, stream), steps, warmup)
    return per, copies, secs


def bench_config3(torch, qk, synth, lib, steps, warmup, wtype=12, n=3584, k=1024, m=512):
    """Chunked-prefill GEMM (int8 MFMA): xq resident, y fp32. Weight and
    output buffers rotate through > 512 MB so each step reads its weights
    from HBM and writes its outputs to fresh lines. Returns (seconds for
    the GEMM alone, seconds for quantize + GEMM from fp32 x)."""
    per = n * (k // 256) * qk.BLOCK_BYTES[wtype] + 4 * m * n
    copies = max(2, -(-MALL_DEFEAT_BYTES // per))
    w = torch.from_numpy(synth.blocks(wtype, n, k, seed=0)).cuda()
    ws = [w] + [w.clone() for _ in range(copies - 1)]
    ys = [torch.empty((m, n), dtype=torch.float32, device="cuda") for _ in range(copies)]
    x = torch.from_numpy(synth.activations(m, k, seed=0)).cuda()
    xq = lib.quantize_q8k(x)
    fn = {12: lib.L.hip_matmul_q4k, 13: lib.L.hip_matmul_q5k, 14: lib.L.hip_matmul_q6k}[wtype]
    wp = [C.c_void_p(t.data_ptr()) for t in ws]
    yp = [C.c_void_p(t.data_ptr()) for t in ys]
    xp, xqp = C.c_void_p(x.data_ptr()), C.c_void_p(xq.data_ptr())
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    quant = lib.L.hip_quantize_q8k

    def gemm(i):
        if fn(wp[i % copies], n, k, xqp, m, yp[i % copies], stream):
            raise RuntimeError(lib.last_error())

    def both(i):
        if quant(xp, m, k, xqp, stream):
            raise RuntimeError(lib.last_error())
        gemm(i)

    ev = Events(torch)
    return copies, ev.time(gemm, steps, warmup), ev.time(both, steps, warmup)


def cpu_baseline(synth, seconds=10.0):
    """The reference's tensor_matmul_*_f32 (one core, as shipped) over the
    config-1 set, repeated for a bounded time."""
    oracle = _load("oracle/oracle.py", "qk_oracle_py")
    if oracle.Ref.available():
        R = oracle.Ref()
        kind, label = "reference", R.label()
        run = lambda t, w, n, k, x: R.matmul(t, w, n, k, x)
    else:
        R = oracle.Oracle()
        kind, label = "port", "oracle restatement"
        run = lambda t, w, n, k, x: R.matmul(t, w, n, k, x, oracle.EPI_FUSED, threads=1)
    mats = [(t, synth.blocks(t, n, k, seed=0, tag=i), n, k, synth.activations(1, k, seed=0, tag=i))
            for i, (t, n, k) in enumerate(CONFIG1)]
    per_set = sum(alg_bytes(t, n, k) for (t, n, k) in CONFIG1)
    reps = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for (t, w, n, k, x) in mats:
            run(t, w, n, k, x)
        reps += 1
    dt = time.perf_counter() - t0
    return {"value": round(per_set * reps / dt / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": kind,
            "sample": f"{reps} passes of the config-1 GEMV set (7 matrices, fp32 x quantized per call) "
                      f"through tensor_matmul_*_f32, {dt:.1f} s, dispatch {label}"}


def mfma_peak():
    """Dense int8 MFMA throughput measured on this GPU by
    qwen.haiku_amd/mfma_peak (built with libqk), or None if it is not built."""
    import subprocess
    exe = os.path.join(ROOT, "qwen.haiku_amd", "mfma_peak")
    if not os.path.exists(exe):
        return None
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    if r.returncode != 0:
        raise RuntimeError(f"mfma_peak failed: {r.stderr.strip()}")
    return json.loads(r.stdout.strip().splitlines()[-1])


def config3_extras(torch, qk, synth, lib, steps, peak_tops=None):
    """Config 3 at M = 512 / 128 / 2048 (Q4_K) and the Q6_K down projection.
    peak_tops: the measured int8 MFMA throughput, for a second fraction."""
    extra = {}
    for (t, n3, k3, m3) in ((12, 3584, 1024, 512), (12, 3584, 1024, 128), (12, 3584, 1024, 2048),
                            (14, 1024, 3584, 512)):
        c3, sg, sb = bench_config3(torch, qk, synth, lib, steps, 10, t, n3, k3, m3)
        ops = 2.0 * m3 * n3 * k3
        xbytes = 4 * m3 * k3
        alg = xbytes + n3 * (k3 // 256) * qk.BLOCK_BYTES[t] + 4 * m3 * n3
        name = {12: "q4k", 14: "q6k"}[t]
        extra[f"config3_gemm_{name}_m{m3}_n{n3}_k{k3}"] = {
            "TOPS_gemm": round(ops * steps / sg / 1e12, 2), "us_gemm": round(sg / steps * 1e6, 3),
            "TOPS_with_quantize": round(ops * steps / sb / 1e12, 2), "us_with_quantize": round(sb / steps * 1e6, 3),
            "frac_of_5POPS": round(ops * steps / sb / 5.0e15, 4),
            "frac_of_bw_x_ai": round((ops * steps / sb) / (HBM_PEAK_GBS * 1e9 * ops / alg), 4),
            "copies": c3}
        if peak_tops:
            extra[f"config3_gemm_{name}_m{m3}_n{n3}_k{k3}"]["frac_of_measured_mfma_peak"] = round(
                ops * steps / sb / (peak_tops * 1e12), 4)
    return extra


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", choices=["all", "config3", "each"], default="all",
                    help="config3: time only the prefill GEMM cases; each: launch every config-1 "
                         "matrix alone, then the set (profiling aids)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="first run 8 plain device copies of MIB MiB each: the known-size "
                         "kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU: the quantized GEMV path runs on a single MI355X "
              f"(--gpus {a.gpus} is not supported)", file=sys.stderr)
        sys.exit(2)
    import torch
    qk = _load("qwen.haiku_amd/qk.py", "qk_binding")
    synth = _load("qwen.haiku_amd/synth.py", "qk_synth")
    lib = qk.QK().init(0)
    if a.copy_probe > 0:
        src = torch.ones(a.copy_probe << 18, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(8):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    if a.only == "each":
        print(json.dumps({"metric": "config-1 matrices alone, us per launch", "unit": "us",
                          "extra": config1_each(torch, qk, synth, lib, a.steps)}))
        return
    if a.only == "config3":
        print(json.dumps({"metric": "prefill int8 TOPS (config 3)", "unit": "TOPS", "dtype": "int8",
                          "extra": config3_extras(torch, qk, synth, lib, a.steps)}))
        return

    per, copies, secs = bench_config1(torch, qk, synth, lib, a.steps, a.warmup)
    gbs = per * a.steps / secs / 1e9
    us = secs / a.steps * 1e6
    out = {
        "metric": "k-quant GEMV GB/s (% of 8 TB/s); prefill int8 TOPS; decode tok/s",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(us / 1e3, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "config1 decode GEMV set: Q4_K 3584x1024 x2, Q6_K 1024x3584, "
                               "Q5_K 2048x1024/512x1024/1024x2048, Q8_0 1024x1024, batch 1",
                   "weight_copies": copies, "bytes_per_step": per, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": CONFIG1_TRAFFIC_BYTES,
                     "kernel": "k_gemv<true, false> (one launch per step)", "us_per_launch": round(us, 3)},
        "tier": lib.tier_label(),
    }
    if not a.no_extra:
        extra = {}
        pw, cw, sw = bench_config1(torch, qk, synth, lib, a.steps, a.warmup, warm=True)
        extra["config1_warm_mall"] = {"GB/s": round(pw * a.steps / sw / 1e9, 2),
                                      "us_per_launch": round(sw / a.steps * 1e6, 3), "copies": cw,
                                      "note": "one weight copy, resident in the 256 MB MALL; not HBM"}
        p0, c0, s0 = bench_config0(torch, qk, synth, lib, a.steps, a.warmup)
        extra["config0_q4k_gemv"] = {"GB/s": round(p0 * a.steps / s0 / 1e9, 2),
                                     "us_per_launch": round(s0 / a.steps * 1e6, 3), "copies": c0}
        st2 = max(20, a.steps // 20)
        p2, c2, s2 = bench_config2(torch, qk, synth, lib, st2, 5)
        extra["config2_lmhead_q6k_argmax_top40"] = {"GB/s": round(p2 * st2 / s2 / 1e9, 2),
                                                    "us_per_call": round(s2 / st2 * 1e6, 3), "copies": c2}
        peak = mfma_peak()
        if peak:
            extra["mfma_int8_peak_measured"] = peak
        peak_tops = peak["mfma_i32_32x32x32_i8_tops"] if peak else None
        extra.update(config3_extras(torch, qk, synth, lib, max(20, a.steps // 10), peak_tops))
        out["extra"] = extra
    if not a.no_cpu:
        out["cpu_baseline"] = cpu_baseline(synth, a.cpu_seconds)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
