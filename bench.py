#!/usr/bin/env python
"""Benchmark of the HCP ring-attention hot path on one MI355X.

Workload (the headline prefill step): Qwen2.5-7B attention shape (28 query
heads, 4 KV heads, head_dim 128, scale 1/sqrt(128)), bf16, one request, one
layer: 8192 local query tokens causal over 8192 local keys (kernel-frame
offset 0: local keys sit at global 8192..16383, after the peer chunk) plus
8192 transient peer keys non-causal, then the LSE merge.  Seeded N(0,1)
inputs with 4 of 128 K channels scaled x8 (logit outliers).  A step is
local pass + peer pass + merge; inputs are resident in HBM before timing.

Also measured in the same run (reported under "decode"): batch-64 split-KV
decode -- 64 sequences, one query token each, a 32768-token contiguous peer
segment plus a paged local segment of U[512, 2048] tokens in
[num_blocks, 4, 16, 256] with a random block table, all segments of a
sequence reduced and merged in one launch.

Prints ONE JSON line.  ``value`` is prefill TFLOP/s (algorithmic FLOPs
4*D*H*pairs over the step time); ``roofline`` is for the dominant kernel
(the non-causal peer pass of the flash-forward kernel), timed with HIP
events on the stream the kernels run on; ``cpu_baseline`` times the CPU
oracle (torch fp32 restatement of the reference's fallback path) on a
bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "prefill TFLOP/s + decode KV GB/s, ring attn+LSE merge, 7B shape 8k+8k bf16"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
H, HKV, D = 28, 4, 128
SCALE = 1.0 / math.sqrt(D)


def causal_pairs(tq: int, tk: int, off: int) -> int:
    """sum_i min(Tk, max(0, off + i + 1)) in closed form."""
    total = 0
    # rows with 0 < off + i + 1 < tk contribute off + i + 1; others 0 or tk
    lo = max(0, -off)                # first row with a visible key
    hi = min(tq, max(0, tk - off - 1))  # rows below this see < tk keys
    if hi > lo:
        a, b = off + lo + 1, off + hi
        total += (a + b) * (hi - lo) // 2
    full_from = max(lo, hi)
    if tq > full_from:
        total += (tq - full_from) * tk
    return total


def prefill_inputs(dev, seed=1, n=8192):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(n, H, D, generator=gen).to(torch.bfloat16)
    kl = torch.randn(n, HKV, D, generator=gen)
    vl = torch.randn(n, HKV, D, generator=gen)
    kp = torch.randn(n, HKV, D, generator=gen)
    vp = torch.randn(n, HKV, D, generator=gen)
    ch = torch.randperm(D, generator=gen)[:4]
    kl[..., ch] *= 8.0
    kp[..., ch] *= 8.0
    cast = lambda t: t.to(torch.bfloat16)
    return tuple(cast(t).to(dev) for t in (q, kl, vl, kp, vp))


def bench_prefill(dev, steps, warmup):
    from hcp_vllm_plugin_amd import merge_attn_states, ring_attn_with_lse

    n = 8192
    q, kl, vl, kp, vp = prefill_inputs(dev)
    out = torch.empty_like(q)

    def step(ev=None):
        if ev is not None:
            ev[0].record()
        o_loc, lse_loc = ring_attn_with_lse(q, kl, vl, SCALE, 0)
        if ev is not None:
            ev[1].record()
        o_peer, lse_peer = ring_attn_with_lse(q, kp, vp, SCALE, None)
        if ev is not None:
            ev[2].record()
        merge_attn_states(out, o_peer, lse_peer, o_loc, lse_loc)
        if ev is not None:
            ev[3].record()

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(evs[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    t_loc = [e[0].elapsed_time(e[1]) for e in evs]
    t_peer = [e[1].elapsed_time(e[2]) for e in evs]
    t_merge = [e[2].elapsed_time(e[3]) for e in evs]
    f_loc = 4 * D * H * causal_pairs(n, n, 0)
    f_peer = 4 * D * H * n * n
    merge_bytes = 3 * n * H * D * 2 + 2 * n * H * 4
    return {
        "wall_s": wall,
        "ms_per_step": wall * 1e3 / steps,
        "flops": f_loc + f_peer,
        "local": {"ms": statistics.mean(t_loc), "flops": f_loc},
        "peer": {"ms": statistics.mean(t_peer), "flops": f_peer},
        "merge": {"ms": statistics.mean(t_merge), "bytes": merge_bytes},
    }


def decode_inputs(dev, seed=3, seqs=64, peer_len=32768, bs=16):
    gen = torch.Generator().manual_seed(seed)
    loc = torch.randint(512, 2049, (seqs,), generator=gen).tolist()
    blocks = [-(-l // bs) for l in loc]
    nb = sum(blocks) + 16
    # big tensors drawn on the device from a seeded device generator
    dgen = torch.Generator(device=dev).manual_seed(seed)
    cache = torch.randn(nb, HKV, bs, 2 * D, generator=dgen, device=dev).to(torch.bfloat16)
    pk = torch.randn(seqs * peer_len, HKV, D, generator=dgen, device=dev).to(torch.bfloat16)
    pv = torch.randn(seqs * peer_len, HKV, D, generator=dgen, device=dev).to(torch.bfloat16)
    q = torch.randn(seqs, H, D, generator=gen).to(torch.bfloat16).to(dev)
    perm = torch.randperm(nb, generator=gen).to(torch.int32)
    bt = torch.zeros(seqs, max(blocks), dtype=torch.int32)
    o = 0
    for r, nbk in enumerate(blocks):
        bt[r, :nbk] = perm[o:o + nbk]
        o += nbk
    return q, cache, bt.to(dev), pk, pv, loc, peer_len


def bench_decode(dev, steps, warmup):
    from hcp_vllm_plugin_amd.varlen import (
        DecodeBatch,
        PagedCache,
        segment_contiguous,
        segment_paged,
    )

    q, cache, bt, pk, pv, loc, peer_len = decode_inputs(dev)
    seqs = q.shape[0]
    pc = PagedCache.from_tensor(cache)
    segs = [[segment_contiguous(pk, pv, s * peer_len, peer_len),
             segment_paged(pc, bt[s], 0, loc[s])] for s in range(seqs)]
    batch = DecodeBatch(segs, H, HKV, D, dev)
    out = torch.empty_like(q)
    for _ in range(warmup):
        batch.run(q, out, None, SCALE)
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps)]
    for i in range(steps):
        evs[i][0].record()
        batch.run(q, out, None, SCALE)
        evs[i][1].record()
    torch.cuda.synchronize()
    ms = statistics.mean(a.elapsed_time(b) for a, b in evs)
    keys = seqs * peer_len + sum(loc)
    kv_bytes = keys * HKV * D * 2 * 2
    qo_bytes = seqs * H * D * 2 * 2
    total = kv_bytes + qo_bytes
    return {
        "ms": ms,
        "bytes": total,
        "gbs": total / (ms * 1e-3) / 1e9,
        "split_tokens": batch.split_tokens,
        "splits": batch.num_splits,
        "seqs": seqs,
        "peer_len": peer_len,
        "local_tokens": sum(loc),
    }


def cpu_baseline(budget_s=30.0):
    """CPU oracle (torch fp32 restatement of the reference's fallback path) on
    the prefill workload itself.

    The whole 8k local causal + 8k peer + merge step runs one KV-head group
    (7 query heads over 1 KV head) at a time, which bounds the fp32 score
    buffers to [7, 8192, 8192] (1.9 GB) per pass.  One warm-up group, then
    full steps (all 4 groups) are timed until `budget_s` is spent (at least
    one); the median full-step time is reported.  Same seeded inputs as the
    GPU step (seed 1, outlier K channels).
    """
    from oracle import ring_oracle as orc

    threads = min(16, os.cpu_count() or 1)
    torch.set_num_threads(threads)
    q, kl, vl, kp, vp = (t.float() for t in prefill_inputs(torch.device("cpu")))
    n, g = q.shape[0], H // HKV

    def run_group(j):
        qs = q[:, j * g:(j + 1) * g]
        sl = slice(j, j + 1)
        o_l, l_l = orc.attn_with_lse(qs, kl[:, sl], vl[:, sl], SCALE, 0)
        o_p, l_p = orc.attn_with_lse(qs, kp[:, sl], vp[:, sl], SCALE, None)
        orc.lse_merge(o_l, l_l, o_p, l_p)

    run_group(0)
    times = []
    t_start = time.perf_counter()
    while not times or (time.perf_counter() - t_start < budget_s * 0.6 and len(times) < 3):
        t0 = time.perf_counter()
        for j in range(HKV):
            run_group(j)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    flops = 4 * D * H * (causal_pairs(n, n, 0) + n * n)
    return {
        "value": flops / t / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"the full prefill step (8192 local causal + 8192 peer + merge, 28/4 heads) "
                   f"on the CPU oracle (torch fp32), one KV-head group at a time; "
                   f"{flops / 1e12:.3f} TFLOP in {t:.2f} s, median of {len(times)} steps, "
                   f"{threads} threads"),
    }


def copy_probe(dev, mib=1024, reps=3):
    """A plain device copy of `mib` MiB (bf16), for scaling HBM byte counters:
    FETCH_SIZE / WRITE_SIZE of this kernel against its known 2 x mib MiB."""
    n = mib * 1024 * 1024 // 2
    x = torch.empty(n, dtype=torch.bfloat16, device=dev).normal_()
    y = torch.empty_like(x)
    for _ in range(reps):
        y.copy_(x)
    torch.cuda.synchronize()
    return {"copy_mib": mib, "reps": reps}


def load_traffic():
    """HBM bytes per launch of the measured kernels, from the committed
    rocprofv3 --pmc summary (profiles/traffic.json), or {}."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f)
    except (OSError, ValueError):
        return {}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--part", choices=("all", "prefill", "decode", "copy"), default="all",
                    help="run one part only (profiler passes); the JSON line needs 'all'")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build's hot path runs on a single "
              "MI355X (multi-GPU sharding is a design note, not built); use --gpus 1",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.part == "copy":
        print(json.dumps(copy_probe(dev)), flush=True)
        return
    if args.part == "decode":
        print(json.dumps(bench_decode(dev, args.steps, args.warmup)), flush=True)
        return
    pre = bench_prefill(dev, args.steps, args.warmup)
    if args.part == "prefill":
        print(json.dumps(pre), flush=True)
        return
    dec = None if args.no_decode else bench_decode(dev, args.steps, args.warmup)
    cpu = None if args.no_cpu_baseline else cpu_baseline()
    traffic = load_traffic()

    value = pre["flops"] / (pre["ms_per_step"] * 1e-3) / 1e12
    peer_tf = pre["peer"]["flops"] / (pre["peer"]["ms"] * 1e-3) / 1e12
    loc_tf = pre["local"]["flops"] / (pre["local"]["ms"] * 1e-3) / 1e12
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(pre["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1), 4 of 128 K channels x8",
        "config": {
            "workload": "ring prefill step: 8192 local causal + 8192 peer non-causal + LSE merge",
            "q_heads": H, "kv_heads": HKV, "head_dim": D,
            "local_tokens": 8192, "peer_tokens": 8192, "causal_frame_offset": 0,
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "fa_fwd_kernel<128,bf16,causal=0> (peer pass)",
            "achieved": round(peer_tf, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(peer_tf / PEAK_BF16_TFLOPS, 4),
            "traffic": traffic.get("fa_fwd_peer", {}).get("bytes"),
        },
        "kernels": {
            "local_causal": {"ms": round(pre["local"]["ms"], 4), "tflops": round(loc_tf, 2),
                             "frac": round(loc_tf / PEAK_BF16_TFLOPS, 4),
                             "traffic": traffic.get("fa_fwd_local", {}).get("bytes")},
            "peer": {"ms": round(pre["peer"]["ms"], 4), "tflops": round(peer_tf, 2),
                     "frac": round(peer_tf / PEAK_BF16_TFLOPS, 4)},
            "merge": {"ms": round(pre["merge"]["ms"], 4),
                      "gbs": round(pre["merge"]["bytes"] / (pre["merge"]["ms"] * 1e-3) / 1e9, 1),
                      "traffic": traffic.get("merge", {}).get("bytes")},
        },
        "cpu_baseline": cpu,
    }
    if dec is not None:
        line["decode"] = {
            "workload": "split-KV decode: 64 seqs x (32768 peer + U[512,2048] paged local)",
            "ms": round(dec["ms"], 4),
            "value": round(dec["gbs"], 1),
            "unit": "GB/s",
            "bytes": dec["bytes"],
            "frac_hbm": round(dec["gbs"] / PEAK_HBM_GBS, 4),
            "split_tokens": dec["split_tokens"],
            "splits": dec["splits"],
            "roofline": {
                "bound": "hbm",
                "kernel": "decode_split_kernel<128,bf16> + decode_reduce_kernel",
                "achieved": round(dec["gbs"], 1),
                "peak": PEAK_HBM_GBS,
                "unit": "GB/s",
                "frac": round(dec["gbs"] / PEAK_HBM_GBS, 4),
                "traffic": traffic.get("decode_split", {}).get("bytes"),
            },
        }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
