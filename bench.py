#!/usr/bin/env python3
"""Packed-KV decode benchmark on one MI355X (BASELINE.json metric, configuration C2).

One step = one decode step of attention for one Llama-3-8B-shaped layer: batch 16, 32 query
heads, 8 KV heads, head_dim 128, 32768 cached tokens (32640 4-bit packed + 128 exact bf16
rows), over the packed KIVI cache already resident in HBM.  Prints ONE JSON line.

Timing: the step is captured once in a HIP graph (the reference's _time_callable protocol,
STRATA_KV.py:3424-3447); W untimed warm-up replays, then K replays between HIP events on the
launch stream (device synchronisation on both sides).  The eager (uncaptured) step time is
reported too.  The dominant kernel (the split-K decode kernel) is timed the same way on its own
(phase 1 only) for the roofline figure.  The CPU baseline is the
oracle's restatement of the reference decode (dequantise + chunked_attention in float32) on a
bounded sample of (batch, KV head) pairs of the same cache, scaled to the whole layer.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "kv-project_amd"))

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E peak


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


def cpu_baseline(q, K, V, shape, bytes_alg, seconds: float) -> dict:
    """Oracle decode (kivi dequantisation + chunked_attention, float32) on whole (b, h) pairs."""
    import numpy as np
    from threadpoolctl import threadpool_info
    from oracle.attention import chunked_attention
    from oracle.kivi import kivi_dequant, kivi_quant
    B, Hkv, T, d = K.shape
    rep = q.shape[1] // Hkv
    W = shape.window
    n_q = T - W
    scaling = d ** -0.5
    times = []
    pairs = [(b, h) for b in range(B) for h in range(Hkv)]
    for b, h in pairs:
        Kbh = K[b:b + 1, h:h + 1].float().cpu().numpy()
        Vbh = V[b:b + 1, h:h + 1].float().cpu().numpy()
        qbh = q[b:b + 1, h * rep:(h + 1) * rep].float().cpu().numpy()
        kq = kivi_quant(Kbh, shape.bits, shape.group_k, True, 0)          # compression: not timed
        vq = kivi_quant(Vbh, shape.bits, shape.group_v, False, 0)
        t0 = time.perf_counter()
        kh = kivi_dequant(kq["codes"], kq["lo"], kq["scale"], shape.group_k, True)[:, :, :n_q]
        vh = kivi_dequant(vq["codes"][:, :, :n_q], vq["lo"][:, :, :n_q], vq["scale"][:, :, :n_q],
                          shape.group_v, False)
        tok = {"k": kh, "v": vh, "b": np.zeros((1, 1, n_q), np.float32), "tau": np.full(n_q, -1)}
        chunked_attention(qbh, scaling, np.array([T]), Kbh[:, :, n_q:], Vbh[:, :, n_q:], np.arange(W),
                          np.full(W, 1 << 40), tok, dtype=np.float32)
        times.append(time.perf_counter() - t0)
        if sum(times) >= seconds and len(times) >= 2:
            break
    per_pair = float(np.median(times))
    t_layer = per_pair * len(pairs)
    threads = max([x.get("num_threads", 1) for x in threadpool_info()] or [1])
    return {"value": bytes_alg / t_layer / 1e9, "unit": "GB/s", "cores": int(threads), "kind": "port",
            "us_per_layer": t_layer * 1e6,
            "sample": f"{len(times)} of {len(pairs)} (batch, KV-head) pairs at full context; "
                      f"median per pair x {len(pairs)}; numpy float32 dequantise + chunked_attention"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--split-tokens", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 1 GiB device-to-device copy (profiler counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this path is single-GPU by design (multi-GPU sharding is "
              "described in DESIGN.md, not launched); run with --gpus 1", file=sys.stderr)
        return 2
    import torch
    import kvq
    from kvq.synth import C2, decode_inputs
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
    shape = C2
    log = lambda m: print(f"[bench] {m}", file=sys.stderr, flush=True)
    log("generating C2 inputs on the GPU")
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

    def graph_of(fn):
        """Capture fn once in a HIP graph (as the reference's _time_callable, STRATA_KV.py:3424-3447)."""
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

    log("timing")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    eager_ms = _events_ms(step, args.steps)
    g_step, g_split = graph_of(step), graph_of(split_only)
    for _ in range(args.warmup):
        g_step.replay()
    ms_per_step = _events_ms(g_step.replay, args.steps)
    for _ in range(args.warmup):
        g_split.replay()
    split_ms = _events_ms(g_split.replay, args.steps)

    io_bytes = q.numel() * q.element_size() + out.numel() * out.element_size()
    bytes_alg = cache.payload_bytes() + io_bytes
    # the split kernel reads the packed rows, the exact rows and q; the output belongs to the merge
    split_bytes = cache.payload_bytes() + q.numel() * q.element_size()
    value = bytes_alg / (ms_per_step * 1e-3) / 1e9
    achieved = split_bytes / (split_ms * 1e-3) / 1e9
    traffic = None
    tf = ROOT / "profiles" / "traffic_kivi_decode_split_c2.json"
    if tf.exists():
        traffic = json.loads(tf.read_text()).get("hbm_bytes_per_launch")
    res = {
        "metric": "packed-KV decode: effective HBM GB/s + µs/layer, 8B-shape 32k ctx b16",
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "C2: one decode step of one Llama-3-8B-shaped layer over a 4-bit KIVI "
                               "cache (B=16, Hq=32, Hkv=8, d=128, T=32768 = 32640 packed + 128 exact)",
                   "global_batch": shape.B, "seq_len": shape.T, "parallelism": "single GPU",
                   "group_k": shape.group_k, "group_v": shape.group_v, "bits": shape.bits,
                   "split_tokens": args.split_tokens},
        "us_per_layer": round(ms_per_step * 1e3, 3),
        "timer": "HIP graph replay, HIP events over the timed steps",
        "eager_us_per_layer": round(eager_ms * 1e3, 3),
        "bytes_alg": bytes_alg,
        "packed_code_GBs": round(2 * shape.B * shape.Hkv * cache.n_q * shape.d // 2 / (ms_per_step * 1e-3) / 1e9, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "kivi_decode_split", "kernel_us": round(split_ms * 1e3, 3),
                     "kernel_bytes_alg": split_bytes},
        "cpu_baseline": None,
    }
    log(f"decode step {ms_per_step * 1e3:.1f} us, split kernel {split_ms * 1e3:.1f} us")
    if not args.no_cpu_baseline:
        log("cpu baseline")
        res["cpu_baseline"] = cpu_baseline(q, K, V, shape, bytes_alg, args.cpu_seconds)
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
