#!/usr/bin/env python3
"""Packed-KV decode benchmark on one MI355X (BASELINE.json metric, configuration C2).

Default (``--workload c2``): one step = one decode step of attention for one Llama-3-8B-shaped
layer: batch 16, 32 query heads, 8 KV heads, head_dim 128, 32768 cached tokens (32640 4-bit
packed + 128 exact bf16 rows), over the packed KIVI cache already resident in HBM.  Prints ONE
JSON line.

The other rows of the path are measured by the same script with ``--workload``:
  c1      the fp32 CPU-runnable configuration (B=1, 8 heads, T=4096, groups of 32)
  c3      mixed 2/4/8-bit 64-token blocks (B=8, Hq=32, Hkv=8, T=16384, group 32)
  c4      eviction: 32 score-accumulating decode steps, top-k 2048 + 256 window, retained decode
  c5      DCT-coded context (B=1, Hq=64, Hkv=8, T=131072): decode, and the encoder
  strata  STRATA strata (per-token 8/4/2-bit tiers) at the C3 shape
  append  streaming append of one token per sequence at the C2 shape (µs/step)
  quant   prefill quantise + pack of the C2 context (kivi_quant of K and V)
  quasar  QUASAR compressed-domain decode (embedded spectral code, 64k context, batch 1)
  micro   the reference's decode-attention microbenchmark: SDPA (full, evicting) vs the packed kernels
  alloc   STRATA rate allocation of one layer (compression side: order, head sum, Lagrangian search)
  snapkv  SnapKV scores of a prefilled layer at the C4 shape (the prefill form of the eviction scores)
  compress  STRATA compression of one Llama-3-8B-shaped layer from its own queries, end to end on the device
Each prints one JSON line of the same form (its own metric, roofline and CPU baseline).

Timing: a settle phase (``settle_ms`` of the same step: the device's clocks rise over the first
~30 ms of sustained load), W untimed warm-up steps, then K steps launched back to back between HIP
events on the launch stream (device synchronisation on both sides).  C1/C2 also report the K steps
timed from idle after only the W warm-ups (``cold_ms_per_step``).  The same step captured once in a HIP graph
(the reference's _time_callable protocol, STRATA_KV.py:3424-3447) is timed too and reported as
``graph_us``: on this ROCm stack a replay of a one-step graph costs more than the eager launches.
The dominant kernel's GPU time per launch (``roofline.kernel_us``, the figure a rocprofv3
kernel-trace average gives; its summary is committed under profiles/) is, where it can run alone
(C1/C2, C3, C5, QUASAR), K launches of it back to back between HIP events; HIP events recorded on the
launch stream right before and after each of its launches inside K more eager steps are reported
beside it (``kernel_us_events``), and for the other workloads they are the kernel figure.  Events
around one launch also count its dispatch latency, a few µs that matter only for short kernels.  The
CPU baseline is the oracle's restatement of the reference path on a bounded sample of the same
workload, scaled to the whole workload, at the box's thread count and at 4 threads; for C1/C2 the
oracle's outputs of the sampled (b, h) pairs are compared with the GPU step's (``parity``), and a
mismatch beyond the bar makes the run exit non-zero.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "kv-project_amd"))

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E peak


def log(m: str) -> None:
    print(f"[bench] {m}", file=sys.stderr, flush=True)


def _events_ms(fn, reps: int) -> float:
    import torch
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


def graph_of(fn):
    """Capture fn once in a HIP graph (as the reference's _time_callable, STRATA_KV.py:3424-3447)."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        fn()
    return gr


def graph_ms(fn, steps: int, warmup: int) -> float:
    g = graph_of(fn)
    for _ in range(warmup):
        g.replay()
    return _events_ms(g.replay, steps)


def graph_k_ms(fn, steps: int, warmup: int) -> float:
    """K back-to-back calls of fn captured in one HIP graph, replayed once untimed and once timed:
    GPU time per call, no host dispatch between the launches (launch-bound kernels included)."""
    import torch
    for _ in range(warmup):
        fn()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        for _ in range(steps):
            fn()
    gr.replay()
    return _events_ms(gr.replay, 1) / steps


def kernel_in_step_ms(kern, steps: int, warmup: int, pre=None, post=None) -> float:
    """Average GPU time of ``kern`` launched inside back-to-back eager steps (pre(); kern(); post()):
    HIP events recorded on the launch stream (torch's current stream, the one every kvq call
    launches on) right before and right after each kern() launch.  The host runs ahead of the GPU,
    so each pair brackets the kernel alone; it is the same eager sequence ms_per_step times (after the
    same settle phase), so the kernel's time cannot exceed the step's."""
    import torch

    def whole():
        if pre is not None:
            pre()
        kern()
        if post is not None:
            post()
    settle(whole, SETTLE_MS)
    for _ in range(warmup):
        whole()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    for a, b in evs:
        if pre is not None:
            pre()
        a.record()
        kern()
        b.record()
        if post is not None:
            post()
    torch.cuda.synchronize()
    return sum(a.elapsed_time(b) for a, b in evs) / steps


def kernel_alone_ms(kern, steps: int, warmup: int) -> float:
    """GPU time per launch of the dominant kernel launched alone, K times back to back on the launch
    stream between HIP events, after a settle phase (each launch recomputes the same partials).  One
    dispatch queues behind the other, so the figure is the kernel's duration plus the small gap
    between dispatches: what a rocprofv3 kernel-trace average gives, where events recorded around a
    single launch inside a step (kernel_in_step_ms) also count that launch's dispatch latency."""
    settle(kern, SETTLE_MS)
    return eager_ms(kern, steps, warmup)


def eager_ms(fn, steps: int, warmup: int) -> float:
    """Back-to-back launches on the current stream between HIP events, after warm-up."""
    for _ in range(warmup):
        fn()
    return _events_ms(fn, steps)


SETTLE_MS = 100.0


def settle(fn, ms: float) -> float:
    """Run fn back to back for about ``ms`` of GPU time (batches timed with HIP events): the device
    raises its clocks over the first ~30 ms of sustained load (per-step times from idle: 113-142 us
    over the first 100 C2 steps, ~106 us after 300), and a decode loop in service runs continuously.
    Returns the GPU time spent."""
    import torch
    spent, batch = 0.0, 8
    while spent < ms:
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(batch):
            fn()
        b.record()
        torch.cuda.synchronize()
        spent += a.elapsed_time(b)
        batch = min(batch * 2, 256)
    return spent


def step_ms(fn, steps: int, warmup: int):
    """(eager ms, graph-replay ms) of one step, each after a settle phase (SETTLE_MS of the same step)
    and ``warmup`` untimed steps.  Eager launches are the figure reported: on this ROCm stack a graph
    replay of these launches measures slower than the same launches issued back to back (an extra
    ~5-20 us per replay), so the graph time is kept as a second figure."""
    settle(fn, SETTLE_MS)
    e = eager_ms(fn, steps, warmup)
    g = graph_ms(fn, steps, warmup)
    return e, g


def _threads() -> int:
    from threadpoolctl import threadpool_info
    return int(max([x.get("num_threads", 1) for x in threadpool_info()] or [1]))


def _result(args, *, metric, value, unit, ms_per_step, workload, config, dtype, roofline, hib=True, **extra):
    res = {"metric": metric, "value": round(value, 3), "unit": unit, "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5), "higher_is_better": hib,
           "scaling": "weak", "vs_baseline": None, "dtype": dtype, "data": "synthetic",
           "config": {"workload": workload, **config}}
    res.update(extra)
    res["roofline"] = roofline
    res["cpu_baseline"] = None
    return res


def _roof(bytes_alg: int, ms: float, kernel: str, traffic=None, events_ms=None) -> dict:
    """``ms``: the kernel's GPU time per launch (kernel_by_difference_ms where the step has other
    launches to leave out); ``events_ms``: the same kernel bracketed by events in the eager step."""
    achieved = bytes_alg / (ms * 1e-3) / 1e9
    res = {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
           "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": kernel,
           "kernel_us": round(ms * 1e3, 3), "kernel_bytes_alg": int(bytes_alg)}
    if events_ms is not None:
        res["kernel_us_events"] = round(events_ms * 1e3, 3)
    return res


def _traffic(name: str):
    tf = ROOT / "profiles" / name
    if tf.exists():
        return json.loads(tf.read_text()).get("hbm_bytes_per_launch")
    return None


def _spread_pairs(B: int, H: int) -> list:
    """Every (b, h) pair, ordered so that any prefix is spread over the batch and the heads (and so
    over the split slots and XCDs the plan maps them to): first and last pairs, then the rest in a
    stride that visits every batch row and head early."""
    allp = [(b, h) for b in range(B) for h in range(H)]
    n = len(allp)
    stride = next(st for st in (H + 1, H + 3, H + 5, 7, 11, 13, 1) if math.gcd(st, n) == 1)
    order = [0, n - 1] + [(i * stride) % n for i in range(1, n)]
    seen, res = set(), []
    for i in order:
        if i not in seen:
            seen.add(i)
            res.append(allp[i])
    return res


def _parity_block(errs, bar: float, oracle: str) -> dict:
    return {"pairs": len(errs), "max_abs_err": max(errs), "bar": bar, "ok": max(errs) <= bar, "oracle": oracle}


# ---------------------------------------------------------------------------------------------
# C2 (default) and C1: packed 4-bit KIVI decode

def cpu_kivi_decode(q, K, V, window, bits, group_k, group_v, bytes_alg, seconds: float, gpu_out=None) -> dict:
    """Oracle decode (kivi dequantisation + chunked_attention, float32) on whole (b, h) pairs, timed
    at the box's BLAS thread count and at 4 threads (the reference's default, STRATA_KV.py:225-226).
    With ``gpu_out`` (B, 1, Hq, d) the oracle's output of every pair it computes is compared with the
    GPU step's (``parity``)."""
    import numpy as np
    from threadpoolctl import threadpool_limits
    from oracle.attention import chunked_attention
    from oracle.kivi import kivi_dequant, kivi_quant
    B, Hkv, T, d = K.shape
    rep = q.shape[1] // Hkv
    W = window
    n_q = T - W
    scaling = d ** -0.5

    def pair(b, h):
        Kbh = K[b:b + 1, h:h + 1].float().cpu().numpy()
        Vbh = V[b:b + 1, h:h + 1].float().cpu().numpy()
        qbh = q[b:b + 1, h * rep:(h + 1) * rep].float().cpu().numpy()
        kq = kivi_quant(Kbh, bits, group_k, True, 0)          # compression: not timed
        vq = kivi_quant(Vbh, bits, group_v, False, 0)
        t0 = time.perf_counter()
        kh = kivi_dequant(kq["codes"], kq["lo"], kq["scale"], group_k, True)[:, :, :n_q]
        vh = kivi_dequant(vq["codes"][:, :, :n_q], vq["lo"][:, :, :n_q], vq["scale"][:, :, :n_q], group_v, False)
        tok = {"k": kh, "v": vh, "b": np.zeros((1, 1, n_q), np.float32), "tau": np.full(n_q, -1)}
        o = chunked_attention(qbh, scaling, np.array([T]), Kbh[:, :, n_q:], Vbh[:, :, n_q:], np.arange(W),
                              np.full(W, 1 << 40), tok, dtype=np.float32)
        return time.perf_counter() - t0, o[0]                   # (1, rep, d)

    pairs = [(b, h) for b in range(B) for h in range(Hkv)]
    times, errs = [], []
    for b, h in pairs:
        dt, o = pair(b, h)
        times.append(dt)
        if gpu_out is not None:
            errs.append(float(np.abs(gpu_out[b, :, h * rep:(h + 1) * rep] - o).max()))
        if sum(times) >= seconds and len(times) >= 2:
            break
    per_pair = float(np.median(times))
    t_layer = per_pair * len(pairs)
    times4 = []
    with threadpool_limits(4):
        for b, h in pairs:
            times4.append(pair(b, h)[0])
            if sum(times4) >= seconds / 2 and len(times4) >= 2:
                break
    t4 = float(np.median(times4)) * len(pairs)
    res = {"value": bytes_alg / t_layer / 1e9, "unit": "GB/s", "cores": _threads(), "kind": "port",
           "us_per_layer": t_layer * 1e6,
           "sample": f"{len(times)} of {len(pairs)} (batch, KV-head) pairs at full context; "
                     f"median per pair x {len(pairs)}; numpy float32 dequantise + chunked_attention",
           "at_4_threads": {"value": bytes_alg / t4 / 1e9, "unit": "GB/s", "cores": 4, "us_per_layer": t4 * 1e6,
                            "sample": f"{len(times4)} of {len(pairs)} pairs, median per pair x {len(pairs)}"}}
    if gpu_out is not None:
        res["parity"] = {"pairs": len(errs), "max_abs_err": max(errs),
                         "oracle": "oracle.kivi kivi_quant + chunked_attention (numpy float32), same inputs"}
    return res


def run_kivi(args, shape_name: str) -> dict:
    import torch
    import kvq
    from kvq.synth import C1, C2, decode_inputs
    shape = C2 if shape_name == "c2" else C1
    log(f"generating {shape.name} inputs on the GPU")
    q, K, V = decode_inputs(shape, device="cuda")
    log("quantising and packing the cache")
    cache = kvq.PackedKIVICache.from_context(K, V, window=shape.window, group_k=shape.group_k,
                                             group_v=shape.group_v)
    scaling = shape.d ** -0.5
    out = torch.empty((shape.B, 1, shape.Hq, shape.d), dtype=shape.dtype, device="cuda")
    ws = torch.zeros((kvq.workspace_floats(shape.B, shape.Hq, shape.Hkv, 1, shape.d, cache.n_q, cache.n_exact,
                                           shape.group_k, shape.group_v, args.split_tokens),), dtype=torch.float32,
                     device="cuda")

    def step():
        kvq.kivi_decode(q, scaling, cache, out=out, workspace=ws, split_tokens=args.split_tokens)

    def split_only():
        kvq.kivi_decode(q, scaling, cache, out=out, workspace=ws, split_tokens=args.split_tokens, phases=1)

    def merge_only():
        kvq.kivi_decode(q, scaling, cache, out=out, workspace=ws, split_tokens=args.split_tokens, phases=2)

    log("timing")
    # from idle: W warm-up steps, then K timed steps, before the clocks have settled
    cold_ms = eager_ms(step, args.steps, args.warmup)
    ms_per_step, g_ms = step_ms(step, args.steps, args.warmup)
    split_ev_ms = kernel_in_step_ms(split_only, args.steps, 0, post=merge_only)
    split_ms = kernel_alone_ms(split_only, args.steps, args.warmup)
    step_gpu_ms = graph_k_ms(step, args.steps, args.warmup)
    io_bytes = q.numel() * q.element_size() + out.numel() * out.element_size()
    bytes_alg = cache.payload_bytes() + io_bytes
    # the split kernel reads the packed rows, the exact rows and q; the output belongs to the merge
    split_bytes = cache.payload_bytes() + q.numel() * q.element_size()
    value = bytes_alg / (ms_per_step * 1e-3) / 1e9
    if shape.name == "C2":
        metric = "packed-KV decode: effective HBM GB/s + µs/layer, 8B-shape 32k ctx b16"
        workload = ("C2: one decode step of one Llama-3-8B-shaped layer over a 4-bit KIVI cache (B=16, Hq=32, "
                    "Hkv=8, d=128, T=32768 = 32640 packed + 128 exact)")
        traffic = _traffic("traffic_kivi_decode_split_c2.json")
    else:
        metric = "packed-KV decode (C1, fp32): effective HBM GB/s + µs/layer"
        workload = ("C1: one fp32 decode step (B=1, Hq=Hkv=8, d=128, T=4096 = 3968 packed + 128 exact, "
                    "groups of 32)")
        traffic = None
    res = _result(args, metric=metric, value=value, unit="GB/s", ms_per_step=ms_per_step, workload=workload,
                  config={"global_batch": shape.B, "seq_len": shape.T, "parallelism": "single GPU",
                          "group_k": shape.group_k, "group_v": shape.group_v, "bits": shape.bits,
                          "split_tokens": args.split_tokens},
                  dtype="bf16" if shape.dtype == torch.bfloat16 else "fp32",
                  roofline=_roof(split_bytes, split_ms, "kivi_decode_split", traffic, events_ms=split_ev_ms),
                  us_per_layer=round(ms_per_step * 1e3, 3),
                  timer="back-to-back launches, HIP events over the timed steps",
                  settle_ms=SETTLE_MS, cold_ms_per_step=round(cold_ms, 5),
                  graph_us=round(g_ms * 1e3, 3), step_gpu_us=round(step_gpu_ms * 1e3, 3), bytes_alg=bytes_alg,
                  packed_code_GBs=round(2 * shape.B * shape.Hkv * cache.n_q * shape.d // 2 / (ms_per_step * 1e-3) / 1e9,
                                        2))
    log(f"decode step {ms_per_step * 1e3:.1f} us, split kernel {split_ms * 1e3:.1f} us")
    # measured cache bytes from the stored format itself (the wire-format export of the layer, context
    # window included) against the analytic bits of state_bits: 2 d (bits + 32/group) per quantised
    # token, 2 d 16 per exact row
    wire = cache.export()
    export_ms = eager_ms(lambda: cache.export(out=wire), max(5, args.steps // 20), 2)
    analytic = shape.B * shape.Hkv * (cache.n_q * 2 * shape.d * (shape.bits + 32.0 / shape.group_k) +
                                      cache.n_exact * 2 * shape.d * 16.0) / 8.0
    res["payload"] = {"bytes": int(wire.numel()), "analytic_bytes": analytic,
                      "payload_vs_analytic": wire.numel() / analytic - 1.0,
                      "export_us": round(export_ms * 1e3, 3),
                      "export_GBs": round(2 * wire.numel() / (export_ms * 1e-3) / 1e9, 2)}
    del wire
    if not args.no_cpu_baseline:
        log("cpu baseline (and the oracle's outputs of the pairs it computes against this step's)")
        step()
        gpu_out = out.float().cpu().numpy()
        cb = cpu_kivi_decode(q, K, V, shape.window, shape.bits, shape.group_k, shape.group_v, bytes_alg,
                             args.cpu_seconds, gpu_out=gpu_out)
        par = cb.pop("parity")
        par["bar"] = 2e-3 if shape.dtype == torch.float32 else 1e-2
        par["ok"] = par["max_abs_err"] <= par["bar"]
        res["parity"] = par
        res["cpu_baseline"] = cb
        log(f"parity over {par['pairs']} (b, h) pairs: max-abs-err {par['max_abs_err']:.3e} (bar {par['bar']})")
    return res


# ---------------------------------------------------------------------------------------------
# C3: mixed-width blocks

def run_c3(args) -> dict:
    import numpy as np
    import torch
    import kvq
    from kvq.synth import C3, c3_inputs
    s = C3
    log("generating C3 inputs")
    q, K, V, imp = c3_inputs("cuda")
    widths = kvq.c3_widths(imp)
    cache = kvq.MixedKIVICache.from_context(K, V, widths, window=0)
    scaling = s.d ** -0.5
    out = torch.empty((s.B, 1, s.Hq, s.d), dtype=s.dtype, device="cuda")
    ws = torch.zeros((kvq.mixed_workspace_floats(s.B, s.Hq, s.Hkv, 1, s.d, cache.nb, 0),), dtype=torch.float32,
                     device="cuda")
    step = lambda: kvq.mixed_decode(q, scaling, cache, out=out, workspace=ws)
    split = lambda: kvq.mixed_decode(q, scaling, cache, out=out, workspace=ws, phases=1)
    merge = lambda: kvq.mixed_decode(q, scaling, cache, out=out, workspace=ws, phases=2)
    ms, g_ms = step_ms(step, args.steps, args.warmup)
    split_ev_ms = kernel_in_step_ms(split, args.steps, 0, post=merge)
    split_ms = kernel_alone_ms(split, args.steps, args.warmup)
    qb = q.numel() * q.element_size()
    bytes_alg = cache.coded_bytes() + qb + out.numel() * out.element_size()
    avg_bits = float(widths.float().mean())
    res = _result(args, metric="mixed-width (2/4/8-bit block) decode: effective HBM GB/s + µs/layer",
                  value=bytes_alg / (ms * 1e-3) / 1e9, unit="GB/s", ms_per_step=ms,
                  workload="C3: one decode step over 64-token blocks of 2/4/8-bit KIVI codes (group 32), widths "
                           "by LogNormal(0,1) block importance 10/30/60% (B=8, Hq=32, Hkv=8, d=128, T=16384)",
                  config={"global_batch": s.B, "seq_len": s.T, "parallelism": "single GPU", "group": 32,
                          "avg_bits": round(avg_bits, 4), "blocks_8_4_2": [int((widths == w).sum()) for w in (8, 4, 2)]},
                  dtype="bf16", roofline=_roof(cache.coded_bytes() + qb, split_ms, "mixed_split", events_ms=split_ev_ms),
                  us_per_layer=round(ms * 1e3, 3), graph_us=round(g_ms * 1e3, 3), bytes_alg=bytes_alg)
    log(f"C3 step {ms * 1e3:.1f} us, split {split_ms * 1e3:.1f} us")
    if not args.no_cpu_baseline:
        from oracle.mixed import dequant_blocks, mixed_decode, mixed_quant
        step()
        gpu_out = out.float().cpu().numpy()                                           # (B, 1, Hq, d)
        pairs = _spread_pairs(s.B, s.Hkv)
        times, errs = [], []
        rep = s.Hq // s.Hkv
        for b, h in pairs:
            Kb = K[b:b + 1, h:h + 1].float().cpu().numpy()
            Vb = V[b:b + 1, h:h + 1].float().cpu().numpy()
            m = mixed_quant(Kb, Vb, widths[b:b + 1, h:h + 1].cpu().numpy())          # compression: not timed
            qb_ = q[b:b + 1, h * rep:(h + 1) * rep].float().cpu().numpy()
            t0 = time.perf_counter()
            xk, xv = dequant_blocks(m["kc"], m["k_lo"], m["k_sc"], m["vc"], m["v_lo"], m["v_sc"])
            o = mixed_decode(qb_, scaling, xk, xv)                                     # (1, 1, rep, d)
            times.append(time.perf_counter() - t0)
            errs.append(float(np.abs(gpu_out[b, 0, h * rep:(h + 1) * rep] - o[0, 0]).max()))
            if sum(times) >= args.cpu_seconds and len(times) >= 4:
                break
        t = float(np.median(times)) * s.B * s.Hkv
        res["cpu_baseline"] = {"value": bytes_alg / t / 1e9, "unit": "GB/s", "cores": _threads(), "kind": "port",
                               "us_per_layer": t * 1e6,
                               "sample": f"{len(times)} of {s.B * s.Hkv} (batch, KV-head) pairs; median per pair x "
                                         f"{s.B * s.Hkv}; numpy per-block dequantise + chunked_attention"}
        res["parity"] = _parity_block(errs, 1e-2, "oracle.mixed mixed_quant + dequant_blocks + mixed_decode "
                                                  "(chunked_attention, float64) of the same pairs, same inputs; the "
                                                  "timed plan (class-major splits)")
    return res


# ---------------------------------------------------------------------------------------------
# A6 at the C3 shape: STRATA strata (per-token widths 8/4/2 by the C3 importance rule)

def run_strata(args) -> dict:
    import numpy as np
    import torch
    import kvq
    from kvq.synth import C3, c3_inputs
    s = C3
    log("generating C3 inputs (per-token strata)")
    q, K, V, imp = c3_inputs("cuda")
    tok_imp = imp.repeat_interleave(64, dim=-1)                       # the block importance, per token
    order = torch.argsort(-tok_imp, dim=-1, stable=True).to(torch.int32)
    n8 = int(0.1 * s.T)
    n4 = int(0.4 * s.T) - n8
    assign = [(8, order[..., :n8].contiguous()), (4, order[..., n8:n8 + n4].contiguous()),
              (2, order[..., n8 + n4:].contiguous())]
    cache = kvq.StrataCache.from_context(K, V, window=0, assign=assign)
    scaling = s.d ** -0.5
    out = torch.empty((s.B, 1, s.Hq, s.d), dtype=s.dtype, device="cuda")
    ws = torch.zeros((kvq.strata_workspace_floats(s.B, s.Hq, s.Hkv, 1, s.d, cache.n_exact, [t.n for t in cache.tiers],
                                                  [t.bits for t in cache.tiers]),), dtype=torch.float32, device="cuda")
    step = lambda: kvq.strata_decode(q, scaling, cache, out=out, workspace=ws)
    ms, g_ms = step_ms(step, args.steps, args.warmup)
    qb = q.numel() * q.element_size()
    bytes_alg = cache.coded_bytes() + qb + out.numel() * out.element_size()
    res = _result(args, metric="STRATA strata decode (per-token 8/4/2-bit tiers): effective HBM GB/s + µs/layer",
                  value=bytes_alg / (ms * 1e-3) / 1e9, unit="GB/s", ms_per_step=ms,
                  workload="A6 at the C3 shape: one decode step over STRATA strata (rotated, per-token scales; "
                           "tokens ranked by the C3 block importance, top 10% 8-bit, next 30% 4-bit, rest 2-bit; "
                           "B=8, Hq=32, Hkv=8, d=128, T=16384, no exact rows)",
                  config={"global_batch": s.B, "seq_len": s.T, "parallelism": "single GPU",
                          "tokens_8_4_2": [n8, n4, s.T - n8 - n4]},
                  # the dominant "kernel" is the whole step (split + merge): timed as the back-to-back
                  # steps themselves, so the roofline cannot run slower than the step it is part of
                  dtype="bf16", roofline=_roof(bytes_alg, ms, "strata_split_all + strata_merge (whole step)"),
                  us_per_layer=round(ms * 1e3, 3), graph_us=round(g_ms * 1e3, 3), bytes_alg=bytes_alg)
    log(f"STRATA step {ms * 1e3:.1f} us")
    if not args.no_cpu_baseline:
        import oracle.strata as os_
        Rm = os_.rotation_matrix(s.d)
        step()
        gpu_out = out.float().cpu().numpy()                                           # (B, 1, Hq, d)
        times, errs = [], []
        for b in range(s.B):
            tiers = []
            for t in cache.tiers:
                tiers.append((t.bits, os_.unpack_planar(t.kc[b].cpu().numpy(), t.bits), t.ks[b, :, :t.n].float().cpu().numpy(),
                              os_.unpack_planar(t.vc[b].cpu().numpy(), t.bits), t.vs[b].float().cpu().numpy()))
            qb_ = q[b:b + 1].float().cpu().numpy()
            empty = np.zeros((s.Hkv, 0, s.d))
            t0 = time.perf_counter()
            o = os_.strata_attend(qb_, scaling, empty, empty, tiers, cache.mu_k[b].float().cpu().numpy(),
                                  cache.mu_v[b].float().cpu().numpy(), Rm)
            times.append(time.perf_counter() - t0)
            errs.append(float(np.abs(gpu_out[b] - o[0]).max()))
            if sum(times) >= args.cpu_seconds and len(times) >= 2:
                break
        t = float(np.median(times)) * s.B
        res["cpu_baseline"] = {"value": bytes_alg / t / 1e9, "unit": "GB/s", "cores": _threads(), "kind": "port",
                               "us_per_layer": t * 1e6,
                               "sample": f"{len(times)} of {s.B} sequences (all 8 KV heads each); median x {s.B}; "
                                         f"numpy tier_reference per stratum + merge (float64)"}
        res["parity"] = _parity_block(errs, 1e-2, "oracle.strata strata_attend (tier_reference per stratum + merge, "
                                                  "float64) over the device's stored strata, whole sequences")
    return res


# ---------------------------------------------------------------------------------------------
# C5: DCT-coded context

def run_c5(args) -> dict:
    import numpy as np
    import torch
    import kvq
    from kvq.synth import C5, c5_inputs
    s = C5
    log("generating C5 inputs (AR(1) series)")
    q, K, V = c5_inputs("cuda")
    cache = kvq.DctCache.from_context(K, V, window=0)
    scaling = s.d ** -0.5
    out = torch.empty((s.B, 1, s.Hq, s.d), dtype=s.dtype, device="cuda")
    ws = torch.zeros((kvq.dct_workspace_floats(s.B, s.Hq, s.Hkv, 1, s.d, cache.T, 0),), dtype=torch.float32,
                     device="cuda")
    step = lambda: kvq.dct_decode(q, scaling, cache, out=out, workspace=ws)
    split = lambda: kvq.dct_decode(q, scaling, cache, out=out, workspace=ws, phases=1)
    merge = lambda: kvq.dct_decode(q, scaling, cache, out=out, workspace=ws, phases=2)
    ms, g_ms = step_ms(step, args.steps, args.warmup)
    split_ev_ms = kernel_in_step_ms(split, args.steps, 0, post=merge)
    split_ms = kernel_alone_ms(split, args.steps, args.warmup)
    # the encoder: keys and values of the whole context, one launch each
    kc, ks = torch.empty_like(cache.kc), torch.empty_like(cache.ks)
    ctab = kvq.dct_table()
    from kvq import _lib

    def enc():
        for x, fv in ((K, 0), (V, 1)):
            _lib.call("kvq_dct_encode", x.data_ptr(), _lib.DTYPE_CODE[x.dtype], s.B * s.Hkv, s.T, s.d, s.T * s.d,
                      ctab.data_ptr(), fv, kc.data_ptr(), ks.data_ptr(), _lib.stream_of(x))
    enc_ms = eager_ms(enc, max(5, args.steps // 5), 2)
    enc_bytes = 2 * (K.numel() * K.element_size() + kc.numel() + ks.numel() * 2)
    qb = q.numel() * q.element_size()
    bytes_alg = cache.coded_bytes() + qb + out.numel() * out.element_size()
    dense = 2 * K.numel() * K.element_size()
    res = _result(args, metric="DCT-coded decode: effective HBM GB/s + µs/layer, 70B-shape 131k ctx",
                  value=bytes_alg / (ms * 1e-3) / 1e9, unit="GB/s", ms_per_step=ms,
                  workload="C5: one decode step over a blockwise-DCT-coded context (16 of 64 coefficients, 4-bit "
                           "absmax, fp16 scales; B=1, Hq=64, Hkv=8, d=128, T=131072, AR(1) rho=0.95 + N(0,0.1))",
                  config={"global_batch": s.B, "seq_len": s.T, "parallelism": "single GPU", "keep": 16, "block": 64},
                  dtype="bf16", roofline=_roof(cache.coded_bytes() + qb, split_ms, "dct_split", events_ms=split_ev_ms),
                  us_per_layer=round(ms * 1e3, 3), graph_us=round(g_ms * 1e3, 3), bytes_alg=bytes_alg,
                  compression_vs_bf16=round(dense / cache.coded_bytes(), 3),
                  encoder={"us": round(enc_ms * 1e3, 3), "bytes": enc_bytes,
                           "GBs": round(enc_bytes / (enc_ms * 1e-3) / 1e9, 2),
                           "frac": round(enc_bytes / (enc_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
    log(f"C5 step {ms * 1e3:.1f} us, split {split_ms * 1e3:.1f} us, encode {enc_ms * 1e3:.1f} us")
    if not args.no_cpu_baseline:
        from oracle.dct import dct_decode, dct_encode
        step()
        gpu_out = out.float().cpu().numpy()                                           # (1, 1, Hq, d)
        times, errs = [], []
        rep = s.Hq // s.Hkv
        for h in (0, s.Hkv - 1) + tuple(range(1, s.Hkv - 1)):
            Kh = K[:, h:h + 1].float().cpu().numpy().reshape(1, s.T, s.d)
            Vh = V[:, h:h + 1].float().cpu().numpy().reshape(1, s.T, s.d)
            kc_, ks_, _ = dct_encode(Kh)                                            # compression: not timed
            vc_, vs_, _ = dct_encode(Vh)
            qh = q[:, h * rep:(h + 1) * rep].float().cpu().numpy()
            t0 = time.perf_counter()
            o = dct_decode(qh, scaling, kc_, ks_, vc_, vs_)                         # (1, 1, rep, d)
            times.append(time.perf_counter() - t0)
            errs.append(float(np.abs(gpu_out[0, 0, h * rep:(h + 1) * rep] - o[0, 0]).max()))
            if sum(times) >= args.cpu_seconds and len(times) >= 2:
                break
        t = float(np.median(times)) * s.Hkv
        res["cpu_baseline"] = {"value": bytes_alg / t / 1e9, "unit": "GB/s", "cores": _threads(), "kind": "port",
                               "us_per_layer": t * 1e6,
                               "sample": f"{len(times)} of {s.Hkv} KV heads; median per head x {s.Hkv}; numpy IDCT "
                                         f"reconstruction + chunked_attention (float64)"}
        res["parity"] = _parity_block(errs, 1e-2, "oracle.dct dct_encode + dct_decode (IDCT reconstruction + "
                                                  "chunked_attention, float64) of the same KV heads at full context")
    return res


# ---------------------------------------------------------------------------------------------
# F2: QUASAR compressed-domain decode

QUASAR_CTX, QUASAR_NC, QUASAR_N0 = 65536, 45056, 656


def run_quasar(args) -> dict:
    import numpy as np
    import torch
    import kvq
    from kvq.quasar import synthetic_packed
    Hq, Hkv, d, stages = 32, 8, 128, (2, 2, 4)
    log("generating the QUASAR stored code (codebooks, embedded quantisation)")
    packed = synthetic_packed(Hkv, d, QUASAR_NC, stages=stages, seed=42)
    g = torch.Generator(device="cuda")
    g.manual_seed(42)
    K = torch.randn((1, Hkv, QUASAR_N0, d), generator=g, device="cuda").to(torch.bfloat16)
    V = torch.randn((1, Hkv, QUASAR_N0, d), generator=g, device="cuda").to(torch.bfloat16)
    q = torch.randn((1, Hq, 1, d), generator=g, device="cuda").to(torch.bfloat16)
    H = QUASAR_CTX
    st = kvq.QuasarState(K, V, packed, stages, 0, H)
    scaling = d ** -0.5
    qpos = torch.tensor([H], device="cuda")
    out = torch.empty((1, 1, Hq, d), dtype=torch.bfloat16, device="cuda")
    step = lambda: st.attend(q, scaling, qpos, out=out)
    split = lambda: st.attend(q, scaling, qpos, out=out, phases=2)
    ms, g_ms = step_ms(step, args.steps, args.warmup)
    step_gpu_ms = graph_k_ms(step, args.steps, args.warmup)
    split_ev_ms = kernel_in_step_ms(split, args.steps, 0, pre=lambda: st.attend(q, scaling, qpos, out=out, phases=1),
                                    post=lambda: st.attend(q, scaling, qpos, out=out, phases=4))
    split_ms = kernel_alone_ms(split, args.steps, args.warmup)
    codes = sum(s_["flat"].numel() for s_ in st.sides)
    rho = 2 * 2 * Hkv * QUASAR_NC
    exact = 2 * K.numel() * K.element_size()
    mats = 4 * (st.T_k.numel() + st.T_v.numel() + st.mu_k.numel() + st.mu_v.numel())
    io = q.numel() * q.element_size() + out.numel() * out.element_size()
    bytes_split = codes + rho + exact
    bytes_alg = bytes_split + mats + io
    res = _result(args, metric="QUASAR compressed-domain decode: µs/layer (64k context, embedded 2+2+4-bit code)",
                  value=step_gpu_ms * 1e3, unit="us", ms_per_step=step_gpu_ms, hib=False,
                  workload=f"F2: one decode step of QuasarState.attend over a {QUASAR_CTX}-token context kept as "
                           f"{QUASAR_NC} coded tokens (12 levels: bands 16/16/32/64 x stages 2/2/4 bits, the level-l "
                           f"prefix holding 1.0 .. 0.1 of them) + {QUASAR_N0} exact rows; B=1, Hq=32, Hkv=8, d=128, "
                           "bf16 exact rows, synthetic N(0, 1) coefficients",
                  config={"global_batch": 1, "seq_len": QUASAR_CTX, "parallelism": "single GPU", "coded": QUASAR_NC,
                          "exact": QUASAR_N0, "stages": list(stages)},
                  dtype="bf16", roofline=_roof(bytes_split, split_ms, "quasar_split", events_ms=split_ev_ms),
                  eager_us=round(ms * 1e3, 3), graph_us=round(g_ms * 1e3, 3), bytes_alg=bytes_alg,
                  code_bytes=codes, context_bytes=st.context_bytes(),
                  reference_published_us_64k="4100-39000 (A100-class MIG slice, STRATA_KV.py:30-32)")
    log(f"QUASAR step {step_gpu_ms * 1e3:.1f} us GPU ({ms * 1e3:.1f} eager), split {split_ms * 1e3:.1f} us")
    if not args.no_cpu_baseline:
        import oracle.quasar as oq
        qn = q.float().cpu().numpy()
        Kn, Vn = K.float().cpu().numpy(), V.float().cpu().numpy()
        step()
        gpu_out = out.float().cpu().numpy()
        times = []
        while sum(times) < args.cpu_seconds or len(times) < 2:
            t0 = time.perf_counter()
            ref = oq.attend(qn, scaling, np.array([H]), Kn, Vn, QUASAR_N0, H, packed, stages)
            times.append(time.perf_counter() - t0)
        t = float(np.median(times))
        res["cpu_baseline"] = {"value": t * 1e6, "unit": "us", "cores": _threads(), "kind": "port",
                               "sample": f"the whole step, {len(times)} runs, median; numpy float64 restatement of "
                                         "QuasarState.attend (byte-table gather + matmul per step)"}
        res["parity"] = _parity_block([float(np.abs(gpu_out - ref).max())], 1e-2,
                                      "oracle.quasar attend (QuasarState.attend restated in float64), the whole step")
    return res


# ---------------------------------------------------------------------------------------------
# F3: decode-attention microbenchmark (the reference's attention_microbench, STRATA_KV.py:3363-3421)

def _graph_median_us(fn, reps: int) -> float:
    """Median µs of one graph replay of fn (captured once after 3 warm-up calls on a side stream),
    each replay bracketed by its own events: the reference's _time_callable (STRATA_KV.py:3424-3444)."""
    import numpy as np
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    for _ in range(10):
        graph.replay()
    ts = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        graph.replay()
        b.record()
        torch.cuda.synchronize()
        ts.append(a.elapsed_time(b) * 1000.0)
    return float(np.median(ts))


def run_micro(args) -> dict:
    import numpy as np
    import torch
    import torch.nn.functional as F
    import kvq
    from kvq.quasar import synthetic_packed
    d, Hkv, rep = args.micro_shape
    keeps = args.micro_keep
    dt = torch.bfloat16
    reps = 50
    g = torch.Generator(device="cpu").manual_seed(42)
    rows = []
    try:
        from torch.nn.attention import SDPBackend, sdpa_kernel
        sdpa_ctx = lambda: sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION])
    except ImportError:                                              # older torch: no backend selection
        sdpa_ctx = None
    for H in args.micro_lengths:
        log(f"microbench H={H}")
        spec = torch.exp(-torch.arange(d) / (d / 8.0))               # decaying key spectrum + shared offset
        Kc = (torch.randn(1, Hkv, H, d, generator=g) * spec.sqrt() + 2.0).to("cuda", dt).contiguous()
        Vc = torch.randn(1, Hkv, H, d, generator=g).to("cuda", dt).contiguous()
        q1 = torch.randn(1, Hkv * rep, 1, d, generator=g).to("cuda", dt)
        scaling = d ** -0.5
        full_bytes = 2 * Kc.numel() * Kc.element_size()
        res = {}

        def sdpa(K_, V_):
            if sdpa_ctx is None:
                raise RuntimeError("no SDPA backend selection in this torch")
            with sdpa_ctx():                                         # fused kernels only, never the math path
                return F.scaled_dot_product_attention(q1, K_, V_, enable_gqa=True)
        try:
            sdpa(Kc, Vc)
            res["full_sdpa"] = (_graph_median_us(lambda: sdpa(Kc, Vc), reps), full_bytes)
            for keep in keeps:
                n_keep = max(1, int(H * keep))
                Ke, Ve = Kc[:, :, :n_keep].contiguous(), Vc[:, :, :n_keep].contiguous()
                res[f"evict_sdpa@{keep:g}"] = (_graph_median_us(lambda Ke=Ke, Ve=Ve: sdpa(Ke, Ve), reps),
                                               2 * Ke.numel() * Ke.element_size())
        except RuntimeError as e:                                    # a fused backend refused: recorded
            log(f"  SDPA rows skipped: {e}")
            res["full_sdpa"] = (float("nan"), full_bytes)
        # the full bf16 cache through this build's exact-row decode (every row exact): the fair
        # full-cache baseline on this GPU (torch's fused SDPA is not a decode kernel here)
        full = kvq.PackedKIVICache.from_context(Kc, Vc, window=H, group_k=64, group_v=64)
        out = torch.empty((1, 1, Hkv * rep, d), dtype=dt, device="cuda")
        fws = torch.zeros((kvq.workspace_floats(1, Hkv * rep, Hkv, 1, d, full.n_q, full.n_exact, 64, 64),),
                          dtype=torch.float32, device="cuda")
        res["full_exact_kernel"] = (_graph_median_us(lambda: kvq.kivi_decode(q1, scaling, full, out=out, workspace=fws), reps),
                                    full_bytes)
        del full, fws
        # packed 4-bit KIVI (window 128, groups of 64): the path's headline kernel
        W = 128
        cache = kvq.PackedKIVICache.from_context(Kc, Vc, window=W, group_k=64, group_v=64)
        ws = torch.zeros((kvq.workspace_floats(1, Hkv * rep, Hkv, 1, d, cache.n_q, cache.n_exact, 64, 64),),
                         dtype=torch.float32, device="cuda")
        res["kivi4_kernel"] = (_graph_median_us(lambda: kvq.kivi_decode(q1, scaling, cache, out=out, workspace=ws), reps),
                               cache.wire_bytes())
        for keep in keeps:
            # STRATA at about keep x the full bytes: a synthetic per-token allocation (tokens ranked by a
            # random importance; the compression-side search is not part of this build)
            imp = torch.rand((1, Hkv, H), generator=g).to("cuda")
            order = torch.argsort(-imp, dim=-1).to(torch.int32)
            frac = {0.25: (0.15, 0.30, 0.45), 0.125: (0.04, 0.10, 0.60)}.get(keep, (0.04, 0.10, 0.60))
            n8, n4, n2 = (int(f * H) for f in frac)
            assign = [(8, order[..., :n8].contiguous()), (4, order[..., n8:n8 + n4].contiguous()),
                      (2, order[..., n8 + n4:n8 + n4 + n2].contiguous())]
            sc = kvq.StrataCache.from_context(Kc, Vc, window=0, assign=assign)
            sws = torch.zeros((kvq.strata_workspace_floats(1, Hkv * rep, Hkv, 1, d, sc.n_exact, [t.n for t in sc.tiers],
                                                           [t.bits for t in sc.tiers]),), dtype=torch.float32, device="cuda")
            res[f"strata_kernel@{keep:g}"] = (_graph_median_us(lambda sc=sc, sws=sws: kvq.strata_decode(q1, scaling, sc, out=out,
                                                                                                   workspace=sws), reps),
                                              sc.coded_bytes())
        # QUASAR at about 1/8 of the full bytes: half the tokens coded (12 embedded levels), 1% exact
        n_c = H // 2
        n0 = max(36, H // 100)
        qs = kvq.QuasarState(Kc[:, :, :n0].contiguous(), Vc[:, :, :n0].contiguous(),
                             synthetic_packed(Hkv, d, n_c, seed=H), (2, 2, 4), 0, H)
        qpos = torch.tensor([H], device="cuda")
        res["quasar_kernel@~0.125"] = (_graph_median_us(lambda: qs.attend(q1, scaling, qpos, out=out), reps),
                                       qs.context_bytes())
        base, fair = res["full_sdpa"][0], res["full_exact_kernel"][0]
        for name, (us, nbytes) in res.items():
            rows.append({"context": H, "method": name, "us_per_step": round(us, 2), "cache_bytes": int(nbytes),
                         "speedup_vs_full": round(base / us, 3) if us > 0 and base == base else None,
                         "speedup_vs_full_exact_kernel": round(fair / us, 3) if us > 0 else None})
        log("  " + ", ".join(f"{k_}={v_[0]:.1f}us/{v_[1] / 2**20:.2f}MiB" for k_, v_ in res.items()))
        del cache, ws, qs
        torch.cuda.empty_cache()
    last = [r for r in rows if r["context"] == args.micro_lengths[-1]]
    kivi = next(r for r in last if r["method"] == "kivi4_kernel")
    res_line = _result(args, metric="decode-attention microbenchmark: packed 4-bit KIVI µs/step at the longest context "
                                    "(full table under rows)",
                       value=kivi["us_per_step"], unit="us", ms_per_step=kivi["us_per_step"] / 1e3, hib=False,
                       workload=f"F3: the reference's attention_microbench (one layer, one decode step, graph replay, "
                                f"median of {reps}) at contexts {list(args.micro_lengths)}, d={d}, Hkv={Hkv}, rep={rep}: "
                                "full and eviction SDPA (fused backends only), the full bf16 cache through this build's exact-row "
                                "decode, packed KIVI-4, STRATA tiers (synthetic allocation) and QUASAR codes (synthetic); keys "
                                "with a decaying spectrum and a shared offset, random values",
                       config={"global_batch": 1, "seq_len": args.micro_lengths[-1], "parallelism": "single GPU",
                               "keep": list(keeps)},
                       dtype="bf16", roofline=_roof(kivi["cache_bytes"], kivi["us_per_step"] / 1e3, "kivi4 step (graph)"),
                       rows=rows, timer="one graph replay per sample, median")
    return res_line


# ---------------------------------------------------------------------------------------------
# C4: eviction

def run_c4(args) -> dict:
    import numpy as np
    import torch
    import kvq
    from kvq.synth import C4, C4_GROUP, C4_KEEP, C4_STEPS, C4_WINDOW, c4_inputs
    s = C4
    log("generating C4 inputs")
    qs, K, V = c4_inputs("cuda")
    cache = kvq.PackedKIVICache.from_context(K, V, window=C4_WINDOW, group_k=C4_GROUP, group_v=C4_GROUP)
    scaling = s.d ** -0.5
    out = torch.empty((s.B, 1, s.Hq, s.d), dtype=s.dtype, device="cuda")
    ws = torch.zeros((kvq.workspace_floats(s.B, s.Hq, s.Hkv, 1, s.d, cache.n_q, cache.n_exact, C4_GROUP, C4_GROUP),),
                     dtype=torch.float32, device="cuda")
    scores = torch.zeros((s.B, s.Hkv, cache.n_q), dtype=torch.float32, device="cuda")
    # the scored step's workspace also holds its logits (spilled by the split, summed by the score
    # kernel): the scores need no second pass over the keys
    ws_s = torch.zeros((kvq.score_workspace_floats(s.B, s.Hq, s.Hkv, 1, s.d, cache.n_q, cache.n_exact, C4_GROUP,
                                                   C4_GROUP),), dtype=torch.float32, device="cuda")
    rep = s.Hq // s.Hkv
    wgt = 1.0 / (rep * C4_STEPS)
    q0 = qs[0]
    plain = lambda: kvq.kivi_decode(q0, scaling, cache, out=out, workspace=ws)
    scored = lambda: kvq.kivi_decode(q0, scaling, cache, out=out, workspace=ws_s, scores=scores, score_weight=wgt)
    scored_decode = lambda: kvq.kivi_decode(q0, scaling, cache, out=out, workspace=ws_s, scores=scores,
                                            score_weight=wgt, phases=3)
    score_only = lambda: kvq.kivi_decode(q0, scaling, cache, out=out, workspace=ws_s, scores=scores,
                                         score_weight=wgt, phases=4)
    reread = lambda: kvq.kivi_decode(q0, scaling, cache, out=out, workspace=ws, scores=scores, score_weight=wgt)
    plain_ms = eager_ms(plain, args.steps, args.warmup)
    scored_ms, g_ms = step_ms(scored, args.steps, args.warmup)
    score_ms = kernel_in_step_ms(score_only, args.steps, 0, pre=scored_decode)
    reread_ms = eager_ms(reread, args.steps, args.warmup)
    # the eviction workload proper: 32 scored decode steps, top-k, gather, decode over the kept rows
    scores.zero_()
    torch.cuda.synchronize()
    for t in range(C4_STEPS):
        kvq.kivi_decode(qs[t], scaling, cache, out=out, workspace=ws_s, scores=scores, score_weight=wgt)
    # top-k over several workgroups per row (a caller's workspace); one workgroup per row beside it
    tk_ws = torch.empty(max(1, kvq.topk_workspace_words(s.B * s.Hkv, cache.n_q)), dtype=torch.int32, device="cuda")
    topk = lambda: kvq.topk_retain(scores, C4_KEEP, workspace=tk_ws)
    topk_ms = eager_ms(topk, args.steps, args.warmup)
    idx = kvq.topk_retain(scores, C4_KEEP, workspace=tk_ws)
    idx_buf = torch.empty_like(idx)
    topk_fixed = lambda: kvq.topk_retain(scores, C4_KEEP, out=idx_buf, workspace=tk_ws)
    topk_one = lambda: kvq.topk_retain(scores, C4_KEEP, out=idx_buf, split=False)
    if not torch.equal(idx, kvq.topk_retain(scores, C4_KEEP, split=False)):
        raise SystemExit("C4: the split top-k and the one-workgroup top-k disagree")
    kept = kvq.retained_cache(cache, idx)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(5):
        kvq.retained_cache(cache, idx)
    torch.cuda.synchronize()
    gather_ms = (time.perf_counter() - t0) * 1e3 / 5
    out_k = torch.empty_like(out)
    ws_k = torch.zeros((kvq.workspace_floats(s.B, s.Hq, s.Hkv, 1, s.d, kept.n_q, kept.n_exact, C4_GROUP, C4_GROUP),),
                       dtype=torch.float32, device="cuda")
    kept_dec = lambda: kvq.kivi_decode(q0, scaling, kept, out=out_k, workspace=ws_k)
    kept_ms = eager_ms(kept_dec, args.steps, args.warmup)
    kept_gpu_ms = graph_k_ms(kept_dec, args.steps, args.warmup)
    # the fused form: the kept rows read straight from the packed cache, no gathered copy
    out_f = torch.empty_like(out)
    ws_f = torch.zeros((kvq.retained_workspace_floats(q0, cache, idx),), dtype=torch.float32, device="cuda")
    fused_dec = lambda: kvq.retained_decode(q0, scaling, cache, idx, out=out_f, workspace=ws_f)
    fused_ms = eager_ms(fused_dec, args.steps, args.warmup)
    fused_gpu_ms = graph_k_ms(fused_dec, args.steps, args.warmup)
    topk_gpu_ms = graph_k_ms(topk_fixed, args.steps, args.warmup)
    topk_one_gpu_ms = graph_k_ms(topk_one, args.steps, args.warmup)
    n_q, BH = cache.n_q, s.B * s.Hkv
    # the score kernel: the spilled logits (rep rows a token) and the scores row read and written
    score_bytes = BH * n_q * rep * 4 + 2 * BH * n_q * 4
    # the episode: the scored steps, the top-k and the first decode over the kept rows (the fused
    # form needs no gather; the gathered form's figure beside it)
    ep_ms = C4_STEPS * scored_ms + topk_ms + fused_ms
    ep_gathered_ms = C4_STEPS * scored_ms + topk_ms + gather_ms + kept_ms
    res = _result(args, metric="eviction decode step: score-accumulating decode µs/layer (C4)",
                  value=scored_ms * 1e3, unit="us", ms_per_step=scored_ms, hib=False,
                  workload="C4: one score-accumulating decode step (decode + probability accumulation per KV head) "
                           "over a 4-bit KIVI cache (B=4, Hq=32, Hkv=8, d=128, T=65536 = 65280 packed + 256 exact, "
                           "group 64; 1% of keys +3); then top-k 2048 and the retained decode",
                  config={"global_batch": s.B, "seq_len": s.T, "parallelism": "single GPU", "keep": C4_KEEP,
                          "window": C4_WINDOW, "steps": C4_STEPS, "group": C4_GROUP},
                  dtype="bf16", roofline=_roof(score_bytes, score_ms, "score_from_logits"),
                  graph_us=round(g_ms * 1e3, 3), plain_decode_us=round(plain_ms * 1e3, 3), score_pass_us=round(score_ms * 1e3, 3),
                  scored_step_reread_us=round(reread_ms * 1e3, 3),
                  topk_us=round(topk_ms * 1e3, 3), gather_us_host_timed=round(gather_ms * 1e3, 3),
                  retained_decode_us=round(fused_ms * 1e3, 3), retained_decode_gpu_us=round(fused_gpu_ms * 1e3, 3),
                  gathered_decode_us=round(kept_ms * 1e3, 3), gathered_decode_gpu_us=round(kept_gpu_ms * 1e3, 3),
                  topk_gpu_us=round(topk_gpu_ms * 1e3, 3), topk_one_wg_gpu_us=round(topk_one_gpu_ms * 1e3, 3),
                  episode_ms=round(ep_ms, 4), episode_gathered_ms=round(ep_gathered_ms, 4),
                  decode_GBs=round((cache.payload_bytes() + 2 * q0.numel() * 2) / (plain_ms * 1e-3) / 1e9, 2))
    log(f"C4 scored step {scored_ms * 1e3:.1f} us (plain {plain_ms * 1e3:.1f}, score kernel {score_ms * 1e3:.1f}, "
        f"with the key-rereading score pass {reread_ms * 1e3:.1f}), "
        f"top-k {topk_ms * 1e3:.1f} us, retained decode {fused_ms * 1e3:.1f} us (over gathered rows "
        f"{kept_ms * 1e3:.1f} us + gather {gather_ms * 1e3:.1f} us)")
    if not args.no_cpu_baseline:
        from oracle.evict import accumulate_decode_scores, decode_step_probs, topk_retain
        from oracle.kivi import kivi_dequant, kivi_quant
        pairs = [(b, h) for b in range(s.B) for h in range(s.Hkv)]
        times = []
        for b, h in pairs:
            Kb = K[b:b + 1, h:h + 1].float().cpu().numpy()
            kq = kivi_quant(Kb, 4, C4_GROUP, True, 0)                               # compression: not timed
            qb = qs[0, b:b + 1, h * rep:(h + 1) * rep].float().cpu().numpy()
            t0 = time.perf_counter()
            kh = kivi_dequant(kq["codes"], kq["lo"], kq["scale"], C4_GROUP, True)[:, :, :n_q]
            p = decode_step_probs(qb, scaling, kh, Kb[:, :, n_q:])
            sc = accumulate_decode_scores(np.zeros((1, 1, n_q)), p, wgt)
            topk_retain(sc, C4_KEEP)
            times.append(time.perf_counter() - t0)
            if sum(times) >= args.cpu_seconds and len(times) >= 2:
                break
        t = float(np.median(times)) * len(pairs)
        res["cpu_baseline"] = {"value": t * 1e6, "unit": "us", "cores": _threads(), "kind": "port",
                               "sample": f"{len(times)} of {len(pairs)} (batch, KV-head) pairs; one scored step "
                                         f"(dequantise keys, softmax probabilities, accumulate) + top-k per pair, "
                                         f"median x {len(pairs)}"}
        res["parity"] = c4_parity(args, qs, K, V, scores, idx, {"fused": out_f, "gathered": out_k}, n_q, scaling,
                                  wgt)
    return res


def c4_parity(args, qs, K, V, scores, idx, outs: dict, n_q: int, scaling: float, wgt: float) -> dict:
    """The eviction episode the C4 line times, against the oracle on sampled (b, h) pairs at full size:
    the scores after all C4_STEPS scored steps (relative to the row's largest score), the retained set
    (equal to the oracle's top-k of its own scores except where both sides' candidates tie with the
    oracle's k-th score within 1e-4 of it, torch.topk leaving tie order unspecified), and the decode over
    the retained rows plus the exact window (q of step 0; oracle: chunked_attention over the oracle's
    dequantised rows at the GPU's retained positions) -- each output of ``outs``: the fused decode
    over the packed cache and the decode over the gathered rows."""
    import numpy as np
    from kvq.synth import C4, C4_GROUP, C4_KEEP
    from oracle.attention import chunked_attention
    from oracle.evict import accumulate_decode_scores, decode_step_probs, topk_retain
    from oracle.kivi import kivi_dequant, kivi_quant
    s = C4
    rep = s.Hq // s.Hkv
    sc_gpu = scores.cpu().numpy()
    idx_gpu = idx.cpu().numpy().astype(np.int64)
    o_gpu = {name: o.float().cpu().numpy() for name, o in outs.items()}  # (B, 1, Hq, d) each
    q_all = qs.float().cpu().numpy()                                      # (steps, B, Hq, 1, d)
    n_steps = q_all.shape[0]
    sc_err, set_diff, tie_gap = [], 0, 0.0
    out_err = {name: [] for name in outs}
    t0 = time.perf_counter()
    for b, h in _spread_pairs(s.B, s.Hkv):
        Kb = K[b:b + 1, h:h + 1].float().cpu().numpy()
        Vb = V[b:b + 1, h:h + 1].float().cpu().numpy()
        kq, vq = kivi_quant(Kb, 4, C4_GROUP, True, 0), kivi_quant(Vb, 4, C4_GROUP, False, 0)
        kh = kivi_dequant(kq["codes"], kq["lo"], kq["scale"], C4_GROUP, True)[:, :, :n_q]
        vh = kivi_dequant(vq["codes"][:, :, :n_q], vq["lo"][:, :, :n_q], vq["scale"][:, :, :n_q], C4_GROUP, False)
        # every step's query rows at once: each row is its own softmax over the packed + exact keys
        qb = q_all[:, b, h * rep:(h + 1) * rep, 0].transpose(1, 0, 2)[None]   # (1, rep, steps, d)
        p = decode_step_probs(qb, scaling, kh, Kb[:, :, n_q:])
        sc = accumulate_decode_scores(np.zeros((1, 1, n_q)), p, wgt)[0, 0]
        sc_err.append(float(np.abs(sc_gpu[b, h] - sc).max() / sc.max()))
        ref = topk_retain(sc[None], C4_KEEP)[0]
        kth = float(np.sort(sc)[::-1][C4_KEEP - 1])
        diff = np.setxor1d(ref, idx_gpu[b, h])
        set_diff += int(diff.size)
        if diff.size:
            tie_gap = max(tie_gap, float(np.abs(sc[diff] - kth).max() / kth))
        keep = idx_gpu[b, h]
        tok = {"k": kh[:, :, keep], "v": vh[:, :, keep], "b": np.zeros((1, 1, keep.size)),
               "tau": np.full(keep.size, -1)}
        W = Kb.shape[2] - n_q
        o = chunked_attention(q_all[0, b:b + 1, h * rep:(h + 1) * rep], scaling, np.array([Kb.shape[2]]),
                              Kb[:, :, n_q:], Vb[:, :, n_q:], np.arange(W), np.full(W, 1 << 40), tok)
        for name, og in o_gpu.items():
            out_err[name].append(float(np.abs(og[b, 0, h * rep:(h + 1) * rep] - o[0, 0]).max()))
        if time.perf_counter() - t0 >= args.cpu_seconds and len(sc_err) >= 3:
            break
    worst = max(max(e) for e in out_err.values())
    ok = max(sc_err) <= 1e-4 and tie_gap <= 1e-4 and worst <= 1e-2
    return {"pairs": len(sc_err), "steps": n_steps, "scores_max_rel_err": max(sc_err),
            "retained_set_differences": set_diff, "differences_max_rel_gap_to_kth": tie_gap,
            **{f"{name}_decode_max_abs_err": max(e) for name, e in out_err.items()},
            "max_abs_err": worst, "bar": 1e-2, "ok": ok,
            "oracle": "oracle.kivi kivi_quant + oracle.evict decode_step_probs / accumulate_decode_scores / "
                      "topk_retain + chunked_attention (float64), same inputs, full context"}


# ---------------------------------------------------------------------------------------------
# A2: streaming append, A1: prefill quantisation

def run_append(args) -> dict:
    import numpy as np
    import torch
    import kvq
    from kvq.synth import C2, decode_inputs
    s = C2
    n_steps = 64 * max(1, args.steps // 64)
    log("building a ring cache at the C2 shape")
    q, K, V = decode_inputs(s, device="cuda", T=s.T - n_steps - 64)
    cache = kvq.PackedKIVICache.from_context(K, V, window=s.window, group_k=s.group_k, group_v=s.group_v,
                                             extra_tokens=n_steps + 128, ring=True)
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    newk = torch.randn((n_steps + 64, s.B, s.Hkv, 1, s.d), generator=g, device="cuda").to(s.dtype)
    newv = torch.randn(newk.shape, generator=g, device="cuda").to(s.dtype)
    for t in range(64):                                   # warm-up, not timed
        cache.append(newk[t], newv[t])
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for t in range(n_steps):
        cache.append(newk[64 + t], newv[64 + t])
    b.record()
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1e3 / n_steps
    # per step and (b, h): write the new K and V rows, read the value row leaving the window and
    # write its codes and (scale, zero) pairs; per 64 steps: read the key group, write its codes
    # and per-channel (scale, zero)
    BH, d = s.B * s.Hkv, s.d
    step_bytes = BH * (2 * d * 2 + d * 2 + d // 2 + (d // s.group_v) * 4) + \
        BH * (s.group_k * d * 2 + s.group_k * d // 2 + d * 4) // s.group_k
    res = _result(args, metric="streaming append (quantise + pack one token per sequence): µs/step",
                  value=us, unit="us", ms_per_step=us * 1e-3, hib=False,
                  workload="A2 at the C2 shape: one appended bf16 token per (b, KV head) per step (B=16, Hkv=8, "
                           "d=128), the token leaving the 128-row window quantised into the packed cache, a key group "
                           "of 64 flushed every 64 steps; mean over whole flush periods, eager launches",
                  config={"global_batch": s.B, "seq_len": s.T, "parallelism": "single GPU", "steps_timed": n_steps},
                  dtype="bf16", roofline=_roof(step_bytes, us * 1e-3, "kivi_append"), us_per_step=round(us, 3))
    log(f"append {us:.2f} us/step")
    if not args.no_cpu_baseline:
        from oracle.kivi import kivi_quant
        Kc = newk[:64].float().cpu().numpy().transpose(1, 2, 0, 3, 4).reshape(s.B, s.Hkv, 64, s.d)
        Vc = newv[:64].float().cpu().numpy().transpose(1, 2, 0, 3, 4).reshape(s.B, s.Hkv, 64, s.d)
        reps = 0
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < min(args.cpu_seconds, 5.0) or reps == 0:
            for t in range(64):
                kivi_quant(Vc[:, :, t:t + 1], 4, s.group_v, False, 0)
            kivi_quant(Kc, 4, s.group_k, True, 0)
            reps += 1
        us_cpu = (time.perf_counter() - t0) / (64 * reps) * 1e6
        res["cpu_baseline"] = {"value": us_cpu, "unit": "us", "cores": _threads(), "kind": "port",
                               "sample": f"{reps} flush periods of 64 steps: numpy kivi_quant of each step's leaving "
                                         f"value rows (B*Hkv) + one 64-token key group per period"}
    return res


def run_quant(args) -> dict:
    import numpy as np
    import torch
    import kvq
    from kvq.synth import C2, decode_inputs
    s = C2
    log("generating C2 inputs")
    q, K, V = decode_inputs(s, device="cuda")
    n = s.T - s.window
    Kq, Vq = K[:, :, :n], V[:, :, :n]
    kq = lambda: kvq.kivi_quant_stored(Kq, 4, s.group_k, True, 0)
    vq = lambda: kvq.kivi_quant_stored(Vq, 4, s.group_v, False, 0)
    warm = max(3, args.warmup // 10)          # ~0.3 ms per call: a few ms of load settles the clocks
    k_ms = eager_ms(kq, max(5, args.steps // 5), warm)
    v_ms = eager_ms(vq, max(5, args.steps // 5), warm)
    xb = Kq.numel() * Kq.element_size()
    k_bytes = xb + Kq.numel() // 2 + (n // s.group_k) * s.B * s.Hkv * s.d * 4
    v_bytes = xb + Vq.numel() // 2 + n * s.B * s.Hkv * (s.d // s.group_v) * 4
    ms = k_ms + v_ms
    res = _result(args, metric="prefill KIVI quantise + pack (K and V of one C2 layer): effective GB/s",
                  value=(k_bytes + v_bytes) / (ms * 1e-3) / 1e9, unit="GB/s", ms_per_step=ms,
                  workload="A1 at the C2 shape: kivi_quant (4-bit, group 64) + MSB-first packing of the 32640 "
                           "quantised rows of K (per channel) and V (per token), bf16 in, codes + fp16 metadata out",
                  config={"global_batch": s.B, "seq_len": s.T, "parallelism": "single GPU", "group": s.group_k},
                  dtype="bf16", roofline=_roof(k_bytes, k_ms, "kivi_quant_keys"),
                  keys_us=round(k_ms * 1e3, 3), values_us=round(v_ms * 1e3, 3),
                  values_GBs=round(v_bytes / (v_ms * 1e-3) / 1e9, 2))
    log(f"quant keys {k_ms * 1e3:.1f} us, values {v_ms * 1e3:.1f} us")
    if not args.no_cpu_baseline:
        from oracle.kivi import kivi_quant
        pairs = [(b, h) for b in range(s.B) for h in range(s.Hkv)]
        times = []
        for b, h in pairs:
            Kb = Kq[b:b + 1, h:h + 1].float().cpu().numpy()
            Vb = Vq[b:b + 1, h:h + 1].float().cpu().numpy()
            t0 = time.perf_counter()
            kivi_quant(Kb, 4, s.group_k, True, 0)
            kivi_quant(Vb, 4, s.group_v, False, 0)
            times.append(time.perf_counter() - t0)
            if sum(times) >= args.cpu_seconds and len(times) >= 2:
                break
        t = float(np.median(times)) * len(pairs)
        res["cpu_baseline"] = {"value": (k_bytes + v_bytes) / t / 1e9, "unit": "GB/s", "cores": _threads(),
                               "kind": "port",
                               "sample": f"{len(times)} of {len(pairs)} (batch, KV-head) pairs; numpy kivi_quant of "
                                         f"K and V, median per pair x {len(pairs)}"}
    return res


# ---------------------------------------------------------------------------------------------
# F1: STRATA rate allocation of one layer (compression side)

def run_alloc(args) -> dict:
    import numpy as np
    import torch
    import kvq
    Hkv, d, H, bits, keep = 8, 128, 32768, (2, 4, 8), 0.125
    rs, re = 4, H - 32
    n, nlev = re - rs, len(bits) + 2
    rng = np.random.default_rng(42)
    imp = np.exp(rng.normal(0, 2.0, (Hkv, n, 1)))
    cols = [imp * rng.uniform(0.5, 2.0, (Hkv, n, 1))]
    cols += [imp * 4.0 ** (-2 * l) * rng.uniform(0.5, 2.0, (Hkv, n, 1)) for l in range(1, nlev - 1)]
    D = np.concatenate(cols + [np.zeros((Hkv, n, 1))], -1).astype(np.float32)
    Dg = torch.from_numpy(D).cuda()
    cost, fixed, budget, hist, _ = kvq.layer_costs(bits, d, Hkv, H, keep, rs, re)
    ws = kvq.AllocWorkspace(Hkv, n, nlev, Dg.device)
    step = lambda: kvq.strata_allocate(Dg, cost, fixed, budget, 4, True, ws)
    ms = eager_ms(step, args.steps, args.warmup)
    bytes_alg = D.nbytes + 4 * Hkv * n + 4 * n * nlev + 2 * 4 * n
    al = kvq.allocate_layer(Dg, bits, d, H, keep, rs, re, workspace=ws)
    res = _result(args, metric="STRATA rate allocation: µs/layer (order, head sum, Lagrangian search, histogram)",
                  value=ms * 1e3, unit="us", ms_per_step=ms, hib=False,
                  workload=f"F1: the allocation steps of StrataMethod.compress_layer for one Llama-3-8B-shaped layer: "
                           f"Hkv=8, {H}-token context, {n} coded candidates, options drop / 2 / 4 / 8 bits / exact, "
                           f"keep {keep}, 4 rounds of 32 multipliers; synthetic distortion table",
                  config={"global_batch": 1, "seq_len": H, "parallelism": "single GPU", "n": n, "nlev": nlev,
                          "keep": keep, "rounds": 4},
                  dtype="f64", roofline=_roof(bytes_alg, ms, "kvq_strata_allocate (whole call, ~30 launches)"),
                  bytes_alg=bytes_alg, counts=al["counts"], bits=al["bits"], budget=budget,
                  distortion=round(al["distortion"], 6))
    # the distortion table the allocation reads (rotation, per-width errors e^T Mt e, D), same layer
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    Kc = torch.randn((Hkv, n, d), generator=g, device="cuda").to(torch.bfloat16)
    Vc = torch.randn((Hkv, n, d), generator=g, device="cuda").to(torch.bfloat16)
    Gm = torch.randn((2, Hkv, d, d), generator=g, device="cuda")
    Sm, Mm = (Gm[0] @ Gm[0].transpose(1, 2) / d).contiguous(), (Gm[1] @ Gm[1].transpose(1, 2) / d).contiguous()
    Am, Wm, DDm = torch.rand((3, Hkv, n), generator=g, device="cuda")
    dist = lambda: kvq.strata_distortion(Kc, Vc, Am, Wm, DDm, Sm, Mm, bits)
    d_ms = eager_ms(dist, max(5, args.steps // 5), 3)
    res["distortion_table_us"] = round(d_ms * 1e3, 3)
    res["distortion_table_tflops"] = round(2 * Hkv * n * len(bits) * 2 * d * d / (d_ms * 1e-3) / 1e12, 2)
    log(f"allocation {ms * 1e3:.1f} us, counts {al['counts']}; distortion table {d_ms * 1e3:.1f} us")
    if not args.no_cpu_baseline:
        import oracle.strata_alloc as oa
        times = []
        while sum(times) < args.cpu_seconds or len(times) < 2:
            t0 = time.perf_counter()
            oa.allocate(D, cost, fixed, budget, rounds=4)
            times.append(time.perf_counter() - t0)
        t = float(np.median(times))
        res["cpu_baseline"] = {"value": t * 1e6, "unit": "us", "cores": _threads(), "kind": "port",
                               "sample": f"the whole allocation, {len(times)} runs, median; numpy restatement "
                                         "(stable argsort, float32 head sum, float64 search)"}
    return res


# ---------------------------------------------------------------------------------------------
# A7 prefill form: SnapKV scores at the C4 shape

def run_snapkv(args) -> dict:
    import numpy as np
    import torch
    import kvq
    from kvq.synth import C4, C4_STEPS, c4_inputs
    s = C4
    w, kern = 64, 5
    log("generating C4-shaped keys and window queries")
    _, K, _ = c4_inputs("cuda", steps=1)
    g = torch.Generator(device="cuda").manual_seed(s.seed + 100)
    q = torch.randn((s.B, s.Hq, w, s.d), generator=g, device="cuda").to(s.dtype)   # the window queries
    H = s.T
    scaling = s.d ** -0.5
    out = torch.empty((s.B, s.Hkv, H), dtype=torch.float32, device="cuda")
    need = kvq._lib.load().kvq_snapkv_scores_workspace(s.B, s.Hq, s.Hkv, w, H, kvq._lib.DTYPE_CODE[s.dtype])
    ws = torch.empty((need,), dtype=torch.float32, device="cuda")

    class Win:                                     # the observation queries at positions H - w .. H - 1
        def at(self, pos):
            return q
    qw = Win()
    step = lambda: kvq.snapkv_scores(qw, K, H, scaling, out=out, workspace=ws)
    ms, g_ms = step_ms(step, args.steps, args.warmup)
    rows = (s.Hq // s.Hkv) * w
    flops = 2 * (2 * rows * H * s.d) * s.B * s.Hkv           # logits twice (statistics, then column sums)
    kbytes = 2 * K.numel() * K.element_size()                # keys read by both passes
    tflops = flops / (ms * 1e-3) / 1e12
    res = _result(args, metric="SnapKV scores (prefill form): TFLOP/s of the logit passes + µs/layer", value=tflops,
                  unit="TFLOP/s", ms_per_step=ms,
                  workload=f"A7 snapkv_scores at the C4 shape: B={s.B}, Hq={s.Hq}, Hkv={s.Hkv}, d={s.d}, H={H}, "
                           f"window {w}, pooling {kern}, bf16",
                  config={"global_batch": s.B, "seq_len": H, "parallelism": "single GPU", "window": w,
                          "kernel": kern},
                  dtype="bf16",
                  roofline={"bound": "mfma", "achieved": round(tflops, 2), "peak": 2500.0, "unit": "TFLOP/s",
                            "frac": round(tflops / 2500.0, 4), "traffic": None, "kernel": "snap_stats + snap_cols",
                            "kernel_us": round(ms * 1e3, 3), "kernel_flops": int(flops),
                            "hbm_GBs_keys": round(kbytes / (ms * 1e-3) / 1e9, 1)},
                  us_per_layer=round(ms * 1e3, 3), graph_us=round(g_ms * 1e3, 3))
    log(f"snapkv {ms * 1e3:.1f} us = {tflops:.0f} TFLOP/s")
    if not args.no_cpu_baseline:
        from oracle.evict import snapkv_scores as oracle_snapkv
        Kb = K[:1, :, :H].float().cpu().numpy()
        qb = np.zeros((1, s.Hq, H, s.d), np.float32)
        qb[:, :, H - w:] = q[:1].float().cpu().numpy()
        t0 = time.perf_counter()
        oracle_snapkv(qb, Kb, H, scaling, w, kern)
        t = (time.perf_counter() - t0) * s.B
        res["cpu_baseline"] = {"value": flops / t / 1e12, "unit": "TFLOP/s", "cores": _threads(), "kind": "port",
                               "us_per_layer": t * 1e6,
                               "sample": f"batch element 0 of {s.B} (all {s.Hkv} KV heads), x {s.B}; numpy float64 "
                                         "window attention, pooling, head means"}
    return res


# ---------------------------------------------------------------------------------------------
# F1: STRATA compression of one layer, end to end on the device

def run_compress(args) -> dict:
    import numpy as np
    import torch
    import kvq
    from kvq.strata_compress import StrataCompressor
    B, Hq, Hkv, d, H, keep = 1, 32, 8, 128, 32768, 0.125
    log("generating one Llama-3-8B-shaped layer (queries at every position, keys, values, output metric)")
    g = torch.Generator(device="cuda").manual_seed(47)
    q = torch.randn((B, Hq, H, d), generator=g, device="cuda").to(torch.bfloat16)
    from kvq.synth import student_t3
    t3 = student_t3((Hkv, 1, d), g, "cuda").abs().clamp(0.2, 8.0)   # seeded: the same layer every run
    k = (torch.randn((B, Hkv, H, d), generator=g, device="cuda") * t3).to(torch.bfloat16)
    v = torch.randn((B, Hkv, H, d), generator=g, device="cuda").to(torch.bfloat16)
    Wo = torch.randn((Hq, 64, d), generator=g, device="cuda") / 8
    M = (Wo.transpose(1, 2) @ Wo).contiguous()
    scaling = d ** -0.5
    comp = StrataCompressor(keep)

    def compress():
        al_ = comp.compress_layer(q, k, v, scaling, H, M)
        return al_, comp.pack(al_)

    for _ in range(2):                                       # warm-up: plans, workspaces, clocks
        compress()
    torch.cuda.synchronize()
    reps = max(3, args.steps // 20)
    t0 = time.perf_counter()
    for _ in range(reps):
        al, packed = compress()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / reps
    # phases, HIP events on the launch stream (each phase's own host work included)
    ev = lambda: torch.cuda.Event(enable_timing=True)
    e = [ev() for _ in range(5)]
    rs, re = al["rs"], al["re"]
    e[0].record()
    st = kvq.coverage_stats(q, k, v, scaling, H, rs, re, M)
    e[1].record()
    dist = kvq.strata_distortion(k[0, :, rs:re], v[0, :, rs:re], st["A"], st["W"], st["DD"], st["S"], st["Mbar"],
                                 comp.bits)
    e[2].record()
    kvq.allocate_layer(dist["D"], comp.bits, d, H, keep, rs, re)
    e[3].record()
    comp.pack(al)
    e[4].record()
    torch.cuda.synchronize()
    phase = {nm: e[i].elapsed_time(e[i + 1]) for i, nm in enumerate(("coverage", "distortion", "allocation", "pack"))}
    # coverage work: logits and value sums of every kept group's rows over its causal keys
    plan = kvq.coverage_plan(H, rs, re, Hq // Hkv, None, False, "cuda")
    cov_flops = sum(2 * 2 * (Hq // Hkv) * len(plan.groups[gi]) * (int(plan.groups[gi].max()) + 1) * d * Hkv
                    for gi in plan.kept)
    dist_flops = 2 * Hkv * (re - rs) * len(comp.bits) * 2 * d * d
    tf_cov = cov_flops / (phase["coverage"] * 1e-3) / 1e12
    # the compressed layer decodes through the native state (one appended token, one query step)
    state = comp.native_state(al, packed, k, v, 4, torch.bfloat16)
    kn = torch.randn((1, Hkv, 1, d), generator=g, device="cuda").to(torch.bfloat16)
    state.append(kn, kn, torch.tensor([H]))
    qn = torch.randn((1, Hq, 1, d), generator=g, device="cuda").to(torch.bfloat16)
    dec_ms = eager_ms(lambda: state.attend(qn, scaling, torch.tensor([H])), 50, 10)
    res = _result(args, metric="STRATA compression of one layer on the device: ms/layer (coverage statistics, "
                               "distortion table, allocation, codes)",
                  value=ms, unit="ms", ms_per_step=ms, hib=False,
                  workload=f"F1: StrataMethod.compress_layer + pack for one Llama-3-8B-shaped layer from its own "
                           f"queries (B=1, Hq={Hq}, Hkv={Hkv}, d={d}, H={H}, bf16, keep {keep}, widths 2/4/8 + "
                           f"drop/exact, 4 rounds), synthetic Student-t keys and random o_proj metric",
                  config={"global_batch": B, "seq_len": H, "parallelism": "single GPU", "keep": keep,
                          "bits": list(comp.bits)},
                  dtype="bf16",
                  roofline={"bound": "mfma", "achieved": round(tf_cov, 2), "peak": 2500.0, "unit": "TFLOP/s",
                            "frac": round(tf_cov / 2500.0, 4), "traffic": None,
                            "kernel": "kvq_coverage_stats (logits and value sums of the coverage groups)",
                            "kernel_us": round(phase["coverage"] * 1e3, 3), "kernel_flops": int(cov_flops)},
                  phases_ms={k_: round(v_, 4) for k_, v_ in phase.items()},
                  distortion_tflops=round(dist_flops / (phase["distortion"] * 1e-3) / 1e12, 2),
                  counts=al["counts"], bits=al["bits"], payload_bytes=comp.payload(packed),
                  payload_vs_bits=comp.payload(packed) * 8 / al["bits"] - 1.0, distortion=round(al["distortion"], 6),
                  native_decode_us=round(dec_ms * 1e3, 3), native_context_bytes=state.context_bytes())
    log(f"compress {ms:.2f} ms/layer ({phase}); counts {al['counts']}; native decode {dec_ms * 1e3:.1f} us")
    if not args.no_cpu_baseline:
        # the oracle chain (float64 numpy) on one KV head at an 8192-token context, scaled to the layer:
        # coverage x (H / Hs)^2 (groups and their causal key ranges both grow with H), the rest x H / Hs,
        # then x Hkv
        import oracle.coverage as oc
        import oracle.strata as os_
        import oracle.strata_alloc as oa
        Hs, rep = 8192, Hq // Hkv
        qs = q[0, :rep, :Hs].float().cpu().numpy()
        ks_, vs_ = k[0, :1, :Hs].float().cpu().numpy(), v[0, :1, :Hs].float().cpu().numpy()
        Ms = M[:rep].double().cpu().numpy()
        c0 = time.perf_counter()
        sto = oc.coverage_stats(qs, np.arange(Hs), ks_, vs_, scaling, Hs, 4, Hs - 32, Ms, oc.CoverageParams())
        c1 = time.perf_counter()
        signs = os_.rotation_signs(d)
        _, Yk = os_.strata_center_rotate(ks_[:, 4:Hs - 32], signs)
        _, Yv = os_.strata_center_rotate(vs_[:, 4:Hs - 32], signs)
        Dt = oa.distortion_table(Yk, Yv, sto["S"], sto["Mbar"], sto["A"], sto["W"], sto["DD"], comp.bits)
        cost, fixed, budget, _, _ = oa.layer_costs(comp.bits, d, 1, Hs, keep, 4, Hs - 32)
        oa.allocate(Dt, cost, fixed, budget, 4)
        c2 = time.perf_counter()
        t_layer = ((c1 - c0) * (H / Hs) ** 2 + (c2 - c1) * (H / Hs)) * Hkv
        res["cpu_baseline"] = {"value": t_layer * 1e3, "unit": "ms", "cores": _threads(), "kind": "port",
                               "sample": f"one KV head at an {Hs}-token context ({c1 - c0:.1f} s coverage, "
                                         f"{c2 - c1:.1f} s distortion table + allocation), scaled to the layer: "
                                         f"coverage x (H/{Hs})^2, the rest x H/{Hs}, x {Hkv} heads; numpy float64"}
    return res


WORKLOADS = {"c2": lambda a: run_kivi(a, "c2"), "c1": lambda a: run_kivi(a, "c1"), "c3": run_c3, "c4": run_c4,
             "c5": run_c5, "strata": run_strata, "append": run_append, "quant": run_quant, "quasar": run_quasar,
             "micro": run_micro, "alloc": run_alloc, "snapkv": run_snapkv, "compress": run_compress}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    # the first few ms of sustained load run at a clock that settles afterwards (either way, box to
    # box): a long untimed warm-up keeps that out of the timed steps
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="c2")
    ap.add_argument("--split-tokens", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--micro-lengths", type=int, nargs="+", default=[4096, 16384, 65536],
                    help="contexts of --workload micro (the reference's MICRO_LENGTHS)")
    ap.add_argument("--micro-shape", type=int, nargs=3, default=[128, 8, 4], metavar=("D", "HKV", "REP"))
    ap.add_argument("--micro-keep", type=float, nargs="+", default=[0.25, 0.125])
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 1 GiB device-to-device copy (profiler counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this path is single-GPU by design (sharding over (batch, KV "
              "head) is a design, not launched); run with --gpus 1", file=sys.stderr)
        return 2
    import torch
    torch.cuda.set_device(0)
    if args.copy_calibration:
        # a copy of known size: FETCH_SIZE / WRITE_SIZE per dispatch of this kernel against the
        # 1 GiB it must read and write gives the counters' scale on this device
        src = torch.ones((1 << 28,), dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": src.numel() * 4, "launches": args.steps}), flush=True)
        return 0
    res = WORKLOADS[args.workload](args)
    print(json.dumps(res), flush=True)
    if res.get("parity") is not None and not res["parity"].get("ok", True):
        log(f"PARITY FAILURE: {res['parity']}")
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
