#!/usr/bin/env python3
"""Benchmark of the quantized decode GEMV path on one MI355X.

Workload (configuration 1 of the headline metric): the decode-step GEMV set of one
Qwen3.5-0.8B-shaped layer at batch 1 -- Q4_K gate and up (3584x1024),
Q6_K down (1024x3584), Q5_K 2048x1024, 512x1024 and 1024x2048, Q8_0
1024x1024 -- random blocks as configuration 0 draws them (fp16 d, dmin,
uniform scales and quants), activations already
quantized (Q8_K / Q8_0) and resident in HBM. One launch is one fused
dispatch (hip_matvec_group) over the seven matrices.

Timing. One step is one replay of a HIP graph holding R launches that
rotate through enough distinct weight copies (> 512 MB) that every launch
streams its weights from HBM rather than the 256 MB MALL; R is chosen so
that a replay lasts about a millisecond, so the timed region is GPU-bound
whatever --steps is (20 steps: about 25 ms of back-to-back launches).
Warm-up replays run for at least 0.2 s (and at least --warmup replays).
HIP events on the replay stream bracket the --steps timed replays.

metric: GB/s of algorithmic bytes (weights + quantized activations + fp32
outputs, 11,560,856 B per launch) over the timed launches.

Also reported under "extra": config 1 with its activation quantization in
the step, config 0 (single Q4_K GEMV), config 2 (LM head with fused
argmax / top-40, and its GEMV alone), a Q4_K GEMV of LM-head size
(streaming), config 3 (prefill GEMM), config 4 (end-to-end tok/s of the
drop-in and of the CPU reference), and the CPU reference beside each
config, on one core and on every core this process may use.
"""
import argparse
import ctypes as C
import importlib.util
import json
import os
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))

CONFIG1 = [(12, 3584, 1024), (12, 3584, 1024), (14, 1024, 3584), (13, 2048, 1024),
           (13, 512, 1024), (13, 1024, 2048), (8, 1024, 1024)]
HBM_PEAK_GBS = 8000.0
MFMA_I8_PEAK_TOPS = 5000.0
MALL_DEFEAT_BYTES = 512 << 20
REPLAY_TARGET_S = 1.0e-3          # a graph replay (one step) lasts about this long
WARM_S = 0.2                      # minimum warm-up time
# HBM bytes per config-1 launch of the current k_gemv, from rocprofv3 --pmc
# FETCH_SIZE and WRITE_SIZE runs of this script (--only config1
# --copy-probe 256), each scaled by its reading for a known-size copy / fill
# in the same run (FETCH x2.000: 5870.1 KiB; WRITE x1.000: 54.0 KiB). None
# when the kernel has changed since the last counter run.
CONFIG1_TRAFFIC_BYTES = 12_077_261
E2E_GPU = os.path.join(ROOT, "qwen.haiku_amd", "host", "_build", "qwen_e2e_gpu")
E2E_CPU = os.path.join(ROOT, "oracle", "_ref", "qwen_e2e_cpu")


def _load(rel, name):
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, os.path.join(ROOT, rel))
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def act_bytes(wtype, k):
    return (k // 32) * 34 if wtype == 8 else (k // 256) * 292


def weight_bytes(wtype, n, k):
    bb = {8: 34, 12: 144, 13: 176, 14: 210}[wtype]
    return n * (k // (32 if wtype == 8 else 256)) * bb


def alg_bytes(wtype, n, k):
    return weight_bytes(wtype, n, k) + act_bytes(wtype, k) + 4 * n


def cores_available():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_threads():
    """Threads for the N-core CPU figures: every core this process may use,
    at most 16 (a one-GPU box's share of its host)."""
    return max(1, min(16, cores_available()))


class GraphTimer:
    """Launch sequences captured once in a HIP graph and replayed.

    launch(i, stream) enqueues launch i (0 <= i < R) on `stream` (a
    ctypes void pointer). The graph holds launches 0..R-1 in order; one
    step is one replay."""

    def __init__(self, torch):
        self.torch = torch
        self.warm_s = WARM_S

    def time(self, launch, R, steps, warmup):
        torch = self.torch
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        sp = C.c_void_p(s.cuda_stream)
        with torch.cuda.stream(s):
            for i in range(R):                 # eager pass: the stream's own scratch exists before capture
                launch(i, sp)
        s.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for i in range(R):
                launch(i, sp)
        with torch.cuda.stream(s):
            n, t0 = 0, time.perf_counter()
            while n < warmup or time.perf_counter() - t0 < self.warm_s:
                g.replay()
                n += 1
                if n % 16 == 0:
                    s.synchronize()
            s.synchronize()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(s)
            for _ in range(steps):
                g.replay()
            e1.record(s)
        s.synchronize()
        secs = e0.elapsed_time(e1) / 1e3
        del g
        return secs                            # for steps x R launches


def replays_for(copies, est_us):
    """Launches per replay: whole passes over the copies, about
    REPLAY_TARGET_S long (est_us: estimated microseconds per launch)."""
    per_pass = copies * est_us * 1e-6
    passes = max(1, int(round(REPLAY_TARGET_S / per_pass)))
    return copies * passes


def rate(per_launch, R, steps, secs):
    us = secs / (steps * R) * 1e6
    return per_launch * steps * R / secs / 1e9, us


def config1_mats(torch, synth, lib, copies, shared=False):
    """The config-1 weights (copies of each) with activations. shared=True
    gives the activations a decode layer has: one normed hidden row (k=1024)
    feeds gate, up, both 1024-wide Q5_K projections and the Q8_0 matrix,
    the FFN product (k=3584) feeds down, and a k=2048 row the last Q5_K."""
    base = []
    xs = {}
    for i, (t, n, k) in enumerate(CONFIG1):
        w = torch.from_numpy(synth.blocks(t, n, k, seed=0, tag=i)).cuda()
        key = k if shared else i
        if key not in xs:
            xs[key] = torch.from_numpy(synth.activations(1, k, seed=0, tag=i)).cuda()
        base.append((t, w, n, k, xs[key]))
    sets = []
    for c in range(copies):
        sets.append([(t, w if c == 0 else w.clone(), n, k, x) for (t, w, n, k, x) in base])
    return sets, xs


def bench_config1(torch, qk, synth, lib, steps, warmup, warm=False):
    """Config 1 (the metric). warm=True: one weight copy, so the 11.5 MB
    stay in the 256 MB MALL between launches (a labelled warm-cache figure,
    never the metric)."""
    per = sum(alg_bytes(*s) for s in CONFIG1)
    wbytes = sum(weight_bytes(*s) for s in CONFIG1)
    copies = 1 if warm else max(2, -(-MALL_DEFEAT_BYTES // wbytes))
    sets, _ = config1_mats(torch, synth, lib, copies)
    xq = {}
    descs = []
    for items in sets:
        arr = (qk.GemvDesc * len(items))()
        for i, (t, w, n, k, x) in enumerate(items):
            if (i, t) not in xq:
                xq[(i, t)] = lib.quantize_for(t, x)[0]
            y = torch.empty(n, dtype=torch.float32, device="cuda")
            items[i] = (t, w, n, k, x, y)
            arr[i] = qk.GemvDesc(t, 0, n, k, w.data_ptr(), xq[(i, t)].data_ptr(), y.data_ptr())
        descs.append(arr)
    torch.cuda.synchronize()
    fn = lib.L.hip_matvec_group
    R = replays_for(copies, 5.0) if not warm else 200

    def launch(i, sp):
        if fn(descs[i % copies], len(CONFIG1), sp):
            raise RuntimeError(lib.last_error())

    secs = GraphTimer(torch).time(launch, R, steps, warmup)
    keep = (sets, xq, descs)
    del keep
    return per, copies, R, secs


def bench_config1_quantize(torch, qk, synth, lib, steps, warmup):
    """Config 1 from fp32 activations in one dispatch
    (hip_matvec_group_f32): the workgroups quantize the layer's activation
    rows (Q8_K for k = 1024, 3584, 2048; Q8_0 for the Q8_0 matrix)
    themselves, then run the seven GEMVs. Algorithmic bytes add the fp32
    rows read (4 B per element, once per distinct row) to the config-1
    bytes; the quantized rows are counted once, as in config 1."""
    wbytes = sum(weight_bytes(*s) for s in CONFIG1)
    copies = max(2, -(-MALL_DEFEAT_BYTES // wbytes))
    sets, xs = config1_mats(torch, synth, lib, copies, shared=True)
    per = sum(alg_bytes(*s) for s in CONFIG1) + sum(4 * x.numel() for x in xs.values())
    descs = []
    for items in sets:
        arr = (qk.GemvDesc * len(items))()
        for i, (t, w, n, k, x) in enumerate(items):
            y = torch.empty(n, dtype=torch.float32, device="cuda")
            items[i] = (t, w, n, k, x, y)
            arr[i] = qk.GemvDesc(t, 0, n, k, w.data_ptr(), x.data_ptr(), y.data_ptr())
        descs.append(arr)
    R = replays_for(copies, 5.5)

    def launch(i, sp):
        if lib.L.hip_matvec_group_f32(descs[i % copies], len(CONFIG1), sp):
            raise RuntimeError(lib.last_error())

    secs = GraphTimer(torch).time(launch, R, steps, warmup)
    return per, copies, R, secs, 1


def bench_gemv(torch, qk, synth, lib, steps, warmup, wtype, n, k, est_us):
    """One GEMV (hip_matvec_*) over rotating weight copies."""
    per = alg_bytes(wtype, n, k)
    copies = max(2, -(-MALL_DEFEAT_BYTES // weight_bytes(wtype, n, k)))
    w = torch.from_numpy(synth.blocks(wtype, n, k, seed=0)).cuda()
    ws = [w] + [w.clone() for _ in range(copies - 1)]
    xq = lib.quantize_for(wtype, torch.from_numpy(synth.activations(1, k, seed=0)).cuda())[0]
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    wp = [C.c_void_p(x.data_ptr()) for x in ws]
    xp, yp = C.c_void_p(xq.data_ptr()), C.c_void_p(y.data_ptr())
    fn = {8: lib.L.hip_matvec_q8_0, 12: lib.L.hip_matvec_q4k, 13: lib.L.hip_matvec_q5k,
          14: lib.L.hip_matvec_q6k}[wtype]
    R = replays_for(copies, est_us)

    def launch(i, sp):
        if fn(wp[i % copies], n, k, xp, yp, sp):
            raise RuntimeError(lib.last_error())

    secs = GraphTimer(torch).time(launch, R, steps, warmup)
    return per, copies, R, secs


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
    f = lib.L.hip_lmhead_q6k_argmax_topk
    wp = [C.c_void_p(t.data_ptr()) for t in ws]
    xp, lp = C.c_void_p(xq.data_ptr()), C.c_void_p(logits.data_ptr())
    ap, ip, vp = C.c_void_p(am.data_ptr()), C.c_void_p(ti.data_ptr()), C.c_void_p(tv.data_ptr())
    per = n * 4 * 210 + 4 * 292 + 4 * n
    R = replays_for(copies, 45.0)

    def launch(i, sp):
        if f(wp[i % copies], n, k, xp, topk, lp, ap, ip, vp, sp):
            raise RuntimeError(lib.last_error())

    secs = GraphTimer(torch).time(launch, R, steps, warmup)
    return per, copies, R, secs


def bench_config3(torch, qk, synth, lib, steps, warmup, wtype=12, n=3584, k=1024, m=512, planes=False):
    """Chunked-prefill GEMM (int8 MFMA): xq resident, y fp32. Weight and
    output buffers rotate through > 512 MB so each launch reads its weights
    from HBM and writes its outputs to fresh lines. planes: the GEMM over
    the weights repacked once into int8 MFMA planes (hip_matmul_planes;
    the repacking is not timed). Returns (copies, R, seconds for the GEMM
    alone, seconds for quantize + GEMM from fp32 x)."""
    wbytes = lib.planes_bytes(wtype, n, k) if planes else n * qk.row_bytes(wtype, k)
    per = wbytes + 4 * m * n
    copies = max(2, -(-MALL_DEFEAT_BYTES // per))
    w = torch.from_numpy(synth.blocks(wtype, n, k, seed=0)).cuda()
    pack_us = None
    if planes:
        p0 = lib.pack_planes(wtype, w, n, k)
        ws = [p0] + [p0.clone() for _ in range(copies - 1)]
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        lib.pack_planes(wtype, w, n, k, planes=ws[-1])  # the one-time repacking, timed once
        e1.record()
        torch.cuda.synchronize()
        pack_us = e0.elapsed_time(e1) * 1e3
    else:
        ws = [w] + [w.clone() for _ in range(copies - 1)]
    ys = [torch.empty((m, n), dtype=torch.float32, device="cuda") for _ in range(copies)]
    x = torch.from_numpy(synth.activations(m, k, seed=0)).cuda()
    xq = lib.quantize_q8_0(x) if wtype == qk.Q8_0 else lib.quantize_q8k(x)
    if planes:
        def fn(wp_, n_, k_, xq_, m_, y_, sp_):
            return lib.L.hip_matmul_planes(wtype, wp_, n_, k_, xq_, m_, y_, sp_)
    else:
        fn = {8: lib.L.hip_matmul_q8_0, 12: lib.L.hip_matmul_q4k, 13: lib.L.hip_matmul_q5k,
              14: lib.L.hip_matmul_q6k}[wtype]
    wp = [C.c_void_p(t.data_ptr()) for t in ws]
    yp = [C.c_void_p(t.data_ptr()) for t in ys]
    xp, xqp = C.c_void_p(x.data_ptr()), C.c_void_p(xq.data_ptr())
    quant = lib.L.hip_quantize_q8_0 if wtype == qk.Q8_0 else lib.L.hip_quantize_q8k
    est = 2.0 * m * n * k / 250e12 * 1e6
    R = replays_for(copies, est)

    def gemm(i, sp):
        if fn(wp[i % copies], n, k, xqp, m, yp[i % copies], sp):
            raise RuntimeError(lib.last_error())

    def both(i, sp):
        if quant(xp, m, k, xqp, sp):
            raise RuntimeError(lib.last_error())
        gemm(i, sp)

    gt = GraphTimer(torch)
    return copies, R, gt.time(gemm, R, steps, warmup), gt.time(both, R, steps, warmup), pack_us


# config 3 (Q4_K at three prompt lengths, the Q6_K down projection) and
# the Q8_0 GEMM on config 1's Q8_0 matrix at a 512-token prompt
CONFIG3_CASES = ((12, 3584, 1024, 512), (12, 3584, 1024, 128), (12, 3584, 1024, 2048), (14, 1024, 3584, 512),
                 (8, 1024, 1024, 512))
# the GEMM on int8 MFMA planes (hip_matmul_planes): config 3's K-quant cases,
# the Q6_K down projection at 128 / 2048 tokens and a Q5_K projection
PLANES_CASES = tuple(c for c in CONFIG3_CASES if c[0] != 8) + \
    ((14, 1024, 3584, 128), (14, 1024, 3584, 2048), (13, 2048, 1024, 512), (13, 2048, 1024, 2048))


def config3_extras(torch, qk, synth, lib, steps, warmup, peak_tops=None, native=True):
    """Config 3 at M = 512 / 128 / 2048 (Q4_K) and the Q6_K down projection,
    on the native blocks and on the planes. peak_tops: the measured int8
    MFMA throughput, for a second fraction."""
    extra = {}
    for (t, n3, k3, m3, pl) in ([c + (False,) for c in CONFIG3_CASES] if native else []) + \
            [c + (True,) for c in PLANES_CASES]:
        c3, R, sg, sb, pack_us = bench_config3(torch, qk, synth, lib, steps, warmup, t, n3, k3, m3, planes=pl)
        ops = 2.0 * m3 * n3 * k3
        launches = steps * R
        alg = 4 * m3 * k3 + n3 * qk.row_bytes(t, k3) + 4 * m3 * n3
        tg, tb = ops * launches / sg, ops * launches / sb
        name = {8: "q80", 12: "q4k", 13: "q5k", 14: "q6k"}[t]
        e = {"TOPS_gemm": round(tg / 1e12, 2), "us_gemm": round(sg / launches * 1e6, 3),
             "TOPS_with_quantize": round(tb / 1e12, 2), "us_with_quantize": round(sb / launches * 1e6, 3),
             "frac_of_5POPS_gemm": round(tg / (MFMA_I8_PEAK_TOPS * 1e12), 4),
             "frac_of_5POPS_with_quantize": round(tb / (MFMA_I8_PEAK_TOPS * 1e12), 4),
             "frac_of_bw_x_ai": round(tb / (HBM_PEAK_GBS * 1e9 * ops / alg), 4),
             "copies": c3, "launches_per_step": R}
        if peak_tops:
            e["frac_of_measured_mfma_peak_gemm"] = round(tg / (peak_tops * 1e12), 4)
        if pl:
            e["pack_once_us"] = round(pack_us, 2)
        extra[f"config3_gemm_{name}_m{m3}_n{n3}_k{k3}" + ("_planes" if pl else "")] = e
    return extra


# ---- decode-chain links and the sampler -----------------------------------------

CHAIN_CASES = ((1, 1024), (512, 1024))                 # add + RMSNorm -> Q8_K: decode row, prefill batch
SWIGLU_CASES = ((1, 3584), (512, 3584))
SAMPLERS = {"default_k40": dict(temperature=0.7, top_k=40, top_p=0.9, min_p=0.05, repetition_penalty=1.25,
                                repetition_window=64),
            "k256": dict(temperature=1.0, top_k=0, top_p=0.95, min_p=0.0, repetition_penalty=1.0,
                         repetition_window=0),
            "greedy_rep": dict(temperature=0.0, top_k=40, top_p=0.9, min_p=0.05, repetition_penalty=1.25,
                               repetition_window=64)}


def chain_extras(torch, qk, lib, steps, warmup):
    """Latency of hip_add_rmsnorm_q8k and hip_swiglu_q8k (one graph replay
    of 64 launches per step). The norm's sequential double sum of squares
    (slm/tensor.c:357-360) is one dependent add per element on one lane."""
    out = {}
    gt = GraphTimer(torch)
    g = torch.Generator(device="cuda").manual_seed(0)
    for m, k in CHAIN_CASES:
        h = torch.randn(m, k, device="cuda", generator=g)
        d = torch.randn(m, k, device="cuda", generator=g)
        w = torch.ones(k, device="cuda")
        xq = torch.empty(m, (k // 256) * qk.Q8K_BYTES, dtype=torch.uint8, device="cuda")
        args = (qk._dp(h), qk._dp(d), qk._dp(w), C.c_float(1e-6), m, k, None, None, qk._dp(xq))
        secs = gt.time(lambda i, st: lib.L.hip_add_rmsnorm_q8k(*args, st), 64, steps, warmup)
        out[f"add_rmsnorm_q8k_m{m}_k{k}"] = {"us_per_launch": round(secs / (64 * steps) * 1e6, 3)}
    for m, k in SWIGLU_CASES:
        a = torch.randn(m, k, device="cuda", generator=g)
        b = torch.randn(m, k, device="cuda", generator=g)
        xq = torch.empty(m, (k // 256) * qk.Q8K_BYTES, dtype=torch.uint8, device="cuda")
        args = (qk._dp(a), qk._dp(b), m, k, None, qk._dp(xq))
        secs = gt.time(lambda i, st: lib.L.hip_swiglu_q8k(*args, st), 64, steps, warmup)
        per = 8 * m * k + m * (k // 256) * qk.Q8K_BYTES
        us = secs / (64 * steps) * 1e6
        out[f"swiglu_q8k_m{m}_k{k}"] = {"us_per_launch": round(us, 3), "GB/s": round(per / us / 1e3, 1)}
    return out


def sampler_extras(torch, qk, lib, steps, warmup, vocab=248320):
    """hip_sample at the model's vocabulary: the default chain (top-k 40),
    top-k 256, and greedy with the repetition penalty (16 calls per replay;
    each call penalizes the same logits again, as a decode loop would)."""
    out = {}
    gt = GraphTimer(torch)
    g = torch.Generator(device="cuda").manual_seed(0)
    hist = torch.randint(0, vocab, (64,), dtype=torch.int32, device="cuda", generator=g)
    for name, sp in SAMPLERS.items():
        lg = torch.randn(vocab, device="cuda", generator=g) * 2.5
        st_ = torch.full((2,), 12345, dtype=torch.int64, device="cuda")
        tok = torch.empty(1, dtype=torch.int32, device="cuda")
        s = qk.Sampler(sp["temperature"], sp["top_k"], sp["top_p"], sp["min_p"], sp["repetition_penalty"],
                       sp["repetition_window"])
        args = (qk._dp(lg), vocab, C.byref(s), qk._dp(st_), qk._dp(hist), 64, None, 0, qk._dp(tok))
        secs = gt.time(lambda i, stream: lib.L.hip_sample(*args, stream), 16, steps, warmup)
        out[f"sample_vocab{vocab}_{name}"] = {"us_per_call": round(secs / (16 * steps) * 1e6, 1)}
    return out


def deltanet_extras(torch, lib, steps, warmup, n_tok=512, heads=16, hd=128):
    """hip_deltanet_chunked over one Gated DeltaNet layer of the model: 16
    heads of 128, a 512-token prompt in 8 chunks of 64 (5 kernel launches),
    inputs resident, the state carried in place from call to call."""
    g = torch.Generator(device="cuda").manual_seed(0)
    q = torch.nn.functional.normalize(torch.randn(n_tok, heads, hd, device="cuda", generator=g), dim=2) / hd ** 0.5
    k = torch.nn.functional.normalize(torch.randn(n_tok, heads, hd, device="cuda", generator=g), dim=2)
    v = torch.nn.functional.silu(torch.randn(n_tok, heads, hd, device="cuda", generator=g))
    gl = -torch.nn.functional.softplus(torch.randn(n_tok, heads, device="cuda", generator=g))
    beta = torch.sigmoid(torch.randn(n_tok, heads, device="cuda", generator=g))
    state = torch.zeros(heads, hd, hd, device="cuda")
    out = torch.empty(n_tok, heads, hd, device="cuda")
    args = tuple(C.c_void_p(t.data_ptr()) for t in (q, k, v, gl, beta)) + (n_tok, heads, hd, hd,
                                                                            C.c_void_p(state.data_ptr()),
                                                                            C.c_void_p(out.data_ptr()))
    secs = GraphTimer(torch).time(lambda i, st: lib.L.hip_deltanet_chunked(*args, st), 2, steps, warmup)
    us = secs / (2 * steps) * 1e6
    return {f"deltanet_layer_{heads}x{hd}_n{n_tok}": {"us_per_layer": round(us, 1),
                                                     "tok_s_per_layer": round(n_tok / us * 1e6, 1)}}


# ---- CPU reference ------------------------------------------------------------------

def host_description():
    """CPU model, sockets, cores, SMT, governor and memory of this host."""
    d = {"logical_cpus": os.cpu_count(), "cpus_available": cores_available()}
    try:
        phys, model = set(), None
        pid = cid = None
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "model name" and model is None:
                model = v
            elif k == "physical id":
                pid = v
            elif k == "core id":
                cid = v
            elif not k and pid is not None:
                phys.add((pid, cid))
                pid = cid = None
        if pid is not None:
            phys.add((pid, cid))
        d["model"] = model
        d["sockets"] = len({p for p, _ in phys}) or None
        d["physical_cores"] = len(phys) or None
        if d["physical_cores"]:
            d["threads_per_core"] = round(os.cpu_count() / d["physical_cores"], 2)
    except OSError:
        pass
    try:
        d["governor"] = open("/sys/devices/system/cpu/cpu0/cpufreq/scaling_governor").read().strip()
    except OSError:
        d["governor"] = "unavailable"
    try:
        for line in open("/proc/meminfo"):
            if line.startswith("MemTotal"):
                d["mem_total_gib"] = round(int(line.split()[1]) / 2**20, 1)
    except OSError:
        pass
    return d


def _cpu_backend():
    """(kind, dispatch label, run, stop): run(type, w, n, k, x, threads) is
    the reference's tensor_matmul_*_f32 at threads == 1 and its row dots
    split over a persistent pool of `threads` threads otherwise; stop()
    ends the pool."""
    oracle = _load("oracle/oracle.py", "qk_oracle_py")
    if oracle.Ref.available():
        R = oracle.Ref()
        return "reference", R.label(), (lambda t, w, n, k, x, th: R.matmul(t, w, n, k, x, threads=th)), R.pool_stop
    O = oracle.Oracle()
    return "port", "oracle restatement", (lambda t, w, n, k, x, th: O.matmul(t, w, n, k, x, oracle.EPI_FUSED,
                                                                              threads=th)), (lambda: None)


def _cpu_rate(run, mats, threads, seconds, per_pass):
    reps, t0 = 0, time.perf_counter()
    while True:
        for (t, w, n, k, x) in mats:
            run(t, w, n, k, x, threads)
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= seconds:
            return per_pass * reps / dt, reps, dt


def cpu_baseline(synth, seconds=10.0):
    """The reference's tensor_matmul_*_f32 (one core, as shipped) over the
    config-1 set, repeated for a bounded time."""
    kind, label, run, _ = _cpu_backend()
    mats = [(t, synth.blocks(t, n, k, seed=0, tag=i), n, k, synth.activations(1, k, seed=0, tag=i))
            for i, (t, n, k) in enumerate(CONFIG1)]
    per_set = sum(alg_bytes(t, n, k) for (t, n, k) in CONFIG1)
    bps, reps, dt = _cpu_rate(run, mats, 1, seconds, per_set)
    return {"value": round(bps / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": kind,
            "sample": f"{reps} passes of the config-1 GEMV set (7 matrices, fp32 x quantized per call) "
                      f"through tensor_matmul_*_f32, {dt:.1f} s, dispatch {label}"}


def cpu_extras(synth, seconds=2.0):
    """The CPU reference beside configs 0-3: one core (as shipped,
    LLM_PAR_FOR is a plain loop on Linux) and N cores (the reference's row
    dots split over a persistent pool of N threads by the harness;
    bit-identical, rows are independent). Each figure is a bounded sample
    of about `seconds`."""
    kind, label, run, stop = _cpu_backend()
    nth = cpu_threads()
    out = {"kind": kind, "dispatch": label, "n_core_threads": nth}
    c1 = [(t, synth.blocks(t, n, k, seed=0, tag=i), n, k, synth.activations(1, k, seed=0, tag=i))
          for i, (t, n, k) in enumerate(CONFIG1)]
    per1 = sum(alg_bytes(t, n, k) for (t, n, k) in CONFIG1)
    w0 = synth.blocks(12, 3584, 1024, seed=0)
    x0 = synth.activations(1, 1024, seed=0)
    c0 = [(12, w0, 3584, 1024, x0)]
    per0 = alg_bytes(12, 3584, 1024)
    for name, mats, per in (("config0_q4k_gemv", c0, per0), ("config1_decode_set", c1, per1)):
        for th in (1, nth):
            bps, reps, dt = _cpu_rate(run, mats, th, seconds, per)
            out[f"{name}_{th}core"] = {"GB/s": round(bps / 1e9, 3), "passes": reps, "seconds": round(dt, 2)}
    # config 2: the LM-head GEMV on a bounded slice of the vocabulary, scaled
    # to the full 248320 rows (rows are independent and equally sized)
    n2, k2 = 31040, 1024
    w2 = synth.blocks(14, n2, k2, seed=0)
    x2 = synth.activations(1, k2, seed=0)
    for th in (1, nth):
        bps, reps, dt = _cpu_rate(run, [(14, w2, n2, k2, x2)], th, seconds, alg_bytes(14, n2, k2))
        out[f"config2_lmhead_gemv_{th}core"] = {
            "GB/s": round(bps / 1e9, 3), "us_per_full_call": round(209583248 / bps * 1e6, 1),
            "sample": f"{reps} x {n2} of 248320 rows, {dt:.1f} s"}
    # config 3: the prefill GEMM on a bounded number of tokens (each token is
    # an independent quantize + GEMV in the reference's token loop)
    for (t, n3, k3, m3) in CONFIG3_CASES[:1] + CONFIG3_CASES[3:]:
        ms = 8
        w3 = synth.blocks(t, n3, k3, seed=0)
        x3 = synth.activations(ms, k3, seed=0)
        ops = 2.0 * ms * n3 * k3
        for th in (1, nth):
            r, reps, dt = _cpu_rate(run, [(t, w3, n3, k3, x3)], th, seconds, ops)
            out[f"config3_{'q4k' if t == 12 else 'q6k'}_m{m3}_{th}core"] = {
                "TOPS": round(r / 1e9 / 1e3, 4), "sample": f"{reps} x {ms} tokens of {m3}, {dt:.1f} s"}
    stop()
    # the sampler chain (sample_with, slm/sampler.c:134) at the model's
    # vocabulary, one core, as slm_generate_raw runs it
    oracle = _load("oracle/oracle.py", "qk_oracle_py")
    smp = oracle.Ref() if oracle.Ref.available() else oracle.Oracle()
    logits = synth.activations(1, 248320, seed=3).ravel() * np.float32(2.5)
    hist = np.arange(64, dtype=np.int32) * 977
    for name in ("default_k40", "k256"):
        st_, calls, t0 = smp.rng_seed(11), 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds / 2:
            _, _, st_ = smp.sample(logits, SAMPLERS[name], st_, hist)
            calls += 1
        dt = time.perf_counter() - t0
        out[f"sample_vocab248320_{name}_1core"] = {"us_per_call": round(dt / calls * 1e6, 1), "calls": calls}
    # the chunked DeltaNet step (chunked_ssm_step_f32, slm/chunked.c:287):
    # one head, one chunk of 64, scaled to a 16-head 512-token layer
    rng = np.random.default_rng(0)
    qd = rng.standard_normal((64, 128)).astype(np.float32) * np.float32(0.01)
    kd_ = rng.standard_normal((64, 128)).astype(np.float32) * np.float32(0.08)
    vd_ = rng.standard_normal((64, 128)).astype(np.float32)
    gd = -np.abs(rng.standard_normal(64)).astype(np.float32)
    bd = np.full(64, 0.5, np.float32)
    stt = np.zeros((128, 128), np.float32)
    calls, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds / 2:
        smp.chunked_step(qd, kd_, vd_, gd, bd, stt)
        calls += 1
    dt = time.perf_counter() - t0
    out["deltanet_layer_16x128_n512_1core"] = {"us_per_layer": round(dt / calls * 128 * 1e6, 1),
                                               "sample": f"{calls} chunk steps of 64 tokens x 1 head, "
                                                         f"x 128 for 16 heads x 8 chunks"}
    return out


def e2e(prompt=512, gen=256, seed=0, timeout=600):
    """Config 4: the reference's forward pass on the same model and prompt
    three ways in one run: "gpu_chain" (qk_decode.c: residual stream, norms,
    FFN and the greedy pick on the device, the reference's mixers on the
    host), "gpu_dropin" (the reference's slm_forward_step unchanged, its
    quantized matmuls through the seam, one round trip each) and the CPU
    reference. Prefill is slm_forward_batch through the seam in both GPU
    runs."""
    out = {}
    runs = (("gpu_chain", E2E_GPU, ["--decode", "chain"]), ("gpu_dropin", E2E_GPU, ["--decode", "seam"]),
            ("cpu_reference", E2E_CPU, []),
            ("gpu_chain_sampled", E2E_GPU, ["--decode", "chain", "--sample", "11"]),
            ("cpu_reference_sampled", E2E_CPU, ["--sample", "11"]))
    keys = ("prefill_tok_s", "decode_tok_s", "prefill_s", "decode_s", "tier", "host_syncs_per_token")
    for name, path, extra in runs:
        if not os.path.exists(path):
            out[name] = "not built"
            continue
        r = subprocess.run([path, "--prompt", str(prompt), "--gen", str(gen), "--seed", str(seed)] + extra,
                           capture_output=True, text=True, timeout=timeout)
        if r.returncode != 0:
            raise RuntimeError(f"{path} failed ({r.returncode}): {r.stderr[-1000:]}")
        j = json.loads(r.stdout.strip().splitlines()[-1])
        out[name] = {k: j[k] for k in keys if k in j}
        out[name]["tokens"] = j["tokens"]
        if name == "gpu_chain":
            out[name]["prefetch_misses"] = j["prefetch_misses"]
    pairs = (("gpu_chain", "cpu_reference"), ("gpu_dropin", "cpu_reference"),
             ("gpu_chain_sampled", "cpu_reference_sampled"))
    for gname, cname in pairs:
        g, c = out.get(gname), out.get(cname)
        if isinstance(g, dict) and isinstance(c, dict):
            g["tokens_identical"] = g["tokens"] == c["tokens"]
    for cname in ("cpu_reference", "cpu_reference_sampled"):
        if isinstance(out.get(cname), dict):
            out[cname]["cores"] = 1
            out[cname].pop("host_syncs_per_token", None)
    out["tokens_identical"] = all(out[g]["tokens_identical"] for g, _ in pairs
                                  if isinstance(out.get(g), dict) and "tokens_identical" in out[g])
    for v in out.values():
        if isinstance(v, dict):
            v.pop("tokens", None)
    out["workload"] = (f"random Qwen3.5-0.8B-shaped Q4_K_M model, {prompt}-token prompt, {gen} decode steps: "
                       f"greedy, and *_sampled with slm_sampler_defaults and rng seed 11")
    return out


def mfma_peak():
    """Dense int8 MFMA throughput measured on this GPU by
    qwen.haiku_amd/mfma_peak (built with libqk), or None if it is not built."""
    exe = os.path.join(ROOT, "qwen.haiku_amd", "mfma_peak")
    if not os.path.exists(exe):
        return None
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    if r.returncode != 0:
        raise RuntimeError(f"mfma_peak failed: {r.stderr.strip()}")
    return json.loads(r.stdout.strip().splitlines()[-1])


def main():
    global WARM_S
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-e2e", action="store_true")
    ap.add_argument("--warm-seconds", type=float, default=WARM_S,
                    help="minimum warm-up replay time per case (short values keep profiler traces small)")
    ap.add_argument("--only", choices=["all", "config1", "config3", "config3_planes", "lmhead", "q4k_stream",
                                       "chain", "sampler", "deltanet"],
                    default="all",
                    help="time one case only (profiling aids)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="first run 8 plain device copies of MIB MiB each: the known-size "
                         "kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings")
    a = ap.parse_args()
    WARM_S = a.warm_seconds
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

    def progress(msg):
        print(f"[bench] {msg}", file=sys.stderr, flush=True)

    if a.only in ("config3", "config3_planes"):
        print(json.dumps({"metric": "prefill int8 TOPS (config 3)", "unit": "TOPS", "dtype": "int8",
                          "extra": config3_extras(torch, qk, synth, lib, a.steps, a.warmup,
                                                  native=a.only == "config3")}))
        return
    if a.only == "lmhead":
        p2, c2, R2, s2 = bench_config2(torch, qk, synth, lib, a.steps, a.warmup)
        g, us = rate(p2, R2, a.steps, s2)
        print(json.dumps({"metric": "config2 LM head GB/s", "value": round(g, 2), "us_per_call": round(us, 3)}))
        return
    if a.only == "chain":
        print(json.dumps({"metric": "decode-chain link latency", "extra": chain_extras(torch, qk, lib, a.steps,
                                                                                         a.warmup)}))
        return
    if a.only == "deltanet":
        print(json.dumps({"metric": "chunked DeltaNet layer", "extra": deltanet_extras(torch, lib, a.steps,
                                                                                       a.warmup)}))
        return
    if a.only == "sampler":
        print(json.dumps({"metric": "sampler latency", "extra": sampler_extras(torch, qk, lib, a.steps, a.warmup)}))
        return
    if a.only == "q4k_stream":
        p, c, R, s = bench_gemv(torch, qk, synth, lib, a.steps, a.warmup, 12, 248320, 1024, 30.0)
        g, us = rate(p, R, a.steps, s)
        print(json.dumps({"metric": "Q4_K 248320x1024 GEMV GB/s", "value": round(g, 2), "us_per_launch": round(us, 3)}))
        return

    progress("config 1")
    per, copies, R, secs = bench_config1(torch, qk, synth, lib, a.steps, a.warmup)
    gbs, us = rate(per, R, a.steps, secs)
    out = {
        "metric": "k-quant GEMV GB/s (% of 8 TB/s); prefill int8 TOPS; decode tok/s",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(secs / a.steps * 1e3, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "config1 decode GEMV set: Q4_K 3584x1024 x2, Q6_K 1024x3584, "
                               "Q5_K 2048x1024/512x1024/1024x2048, Q8_0 1024x1024, batch 1",
                   "weight_copies": copies, "bytes_per_launch": per, "launches_per_step": R,
                   "step": "one HIP-graph replay of launches_per_step rotating launches",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": CONFIG1_TRAFFIC_BYTES,
                     "kernel": "k_gemv<true, false> (one launch)", "us_per_launch": round(us, 3)},
        "tier": lib.tier_label(),
    }
    if a.only == "config1":
        print(json.dumps(out))
        return
    if not a.no_extra:
        extra = {}
        progress("config 1 with quantize, warm MALL")
        pq, cq, Rq, sq, nl = bench_config1_quantize(torch, qk, synth, lib, a.steps, a.warmup)
        g, u = rate(pq, Rq, a.steps, sq)
        extra["config1_with_quantize"] = {"GB/s": round(g, 2), "us_per_launch": round(u, 3),
                                          "frac": round(g / HBM_PEAK_GBS, 4), "launches": nl,
                                          "bytes": pq, "copies": cq,
                                          "note": "fp32 rows in, one dispatch: each workgroup quantizes "
                                                  "its row (hip_matvec_group_f32)"}
        pw, cw, Rw, sw = bench_config1(torch, qk, synth, lib, a.steps, a.warmup, warm=True)
        g, u = rate(pw, Rw, a.steps, sw)
        extra["config1_warm_mall"] = {"GB/s": round(g, 2), "us_per_launch": round(u, 3), "copies": cw,
                                      "note": "one weight copy, resident in the 256 MB MALL; not HBM"}
        progress("config 0")
        p0, c0, R0, s0 = bench_gemv(torch, qk, synth, lib, a.steps, a.warmup, 12, 3584, 1024, 3.2)
        g, u = rate(p0, R0, a.steps, s0)
        extra["config0_q4k_gemv"] = {"GB/s": round(g, 2), "us_per_launch": round(u, 3),
                                     "frac": round(g / HBM_PEAK_GBS, 4), "copies": c0, "launches_per_step": R0}
        progress("config 2")
        st2 = max(10, a.steps // 10)
        p2, c2, R2, s2 = bench_config2(torch, qk, synth, lib, st2, 3)
        g, u = rate(p2, R2, st2, s2)
        extra["config2_lmhead_q6k_argmax_top40"] = {"GB/s": round(g, 2), "us_per_call": round(u, 3),
                                                    "frac": round(g / HBM_PEAK_GBS, 4), "copies": c2,
                                                    "launches_per_step": R2, "steps": st2}
        p2g, c2g, R2g, s2g = bench_gemv(torch, qk, synth, lib, st2, 3, 14, 248320, 1024, 37.0)
        g, u = rate(p2g, R2g, st2, s2g)
        extra["config2_lmhead_gemv_only"] = {"GB/s": round(g, 2), "us_per_launch": round(u, 3),
                                             "frac": round(g / HBM_PEAK_GBS, 4), "copies": c2g}
        progress("Q4_K streaming GEMV")
        pq4, cq4, Rq4, sq4 = bench_gemv(torch, qk, synth, lib, st2, 3, 12, 248320, 1024, 30.0)
        g, u = rate(pq4, Rq4, st2, sq4)
        extra["q4k_gemv_248320x1024_stream"] = {"GB/s": round(g, 2), "us_per_launch": round(u, 3),
                                                "frac": round(g / HBM_PEAK_GBS, 4), "copies": cq4,
                                                "bytes": pq4}
        progress("config 3")
        peak = mfma_peak()
        if peak:
            extra["mfma_int8_peak_measured"] = peak
        peak_tops = peak["mfma_i32_32x32x32_i8_tops"] if peak else None
        extra.update(config3_extras(torch, qk, synth, lib, max(10, a.steps // 10), 3, peak_tops))
        progress("decode-chain links and sampler")
        extra["chain_links"] = chain_extras(torch, qk, lib, max(10, a.steps // 10), 3)
        extra["sampler"] = sampler_extras(torch, qk, lib, max(5, a.steps // 20), 2)
        extra["deltanet"] = deltanet_extras(torch, lib, max(5, a.steps // 20), 2)
        if not a.no_e2e:
            progress("config 4 end to end")
            extra["config4_e2e"] = e2e()
        out["extra"] = extra
    if not a.no_cpu:
        progress("CPU reference")
        out["cpu_baseline"] = cpu_baseline(synth, a.cpu_seconds)
        if not a.no_extra:
            out["cpu_extra"] = cpu_extras(synth)
            out["cpu_host"] = host_description()
    print(json.dumps(out))


if __name__ == "__main__":
    main()
