#!/usr/bin/env python
"""Benchmark of the HCP ring-attention hot path on one MI355X.

Workload (the headline prefill step): Qwen2.5-7B attention shape (28 query
heads, 4 KV heads, head_dim 128, scale 1/sqrt(128)), bf16, one request, one
layer: 8192 local query tokens causal over 8192 local keys (kernel-frame
offset 0: local keys sit at global 8192..16383, after the peer chunk) plus
8192 transient peer keys non-causal, merged by LSE.  Seeded N(0,1) inputs
with 4 of 128 K channels scaled x8 (logit outliers).  A step is the peer
pass, then the local pass that merges the peer result into the output in the
same launch (bit for bit the local pass + peer pass + merge_attn_states of
the reference's forward, whose separate timing is reported as "two_step");
inputs are resident in HBM before timing.

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


def bench_prefill(dev, steps, warmup, two_step=True):
    """The headline step as the backend runs it: the peer pass, then the local
    causal pass that merges the peer result into the output in the same launch
    (hcp_attn_fwd_lse_merge; equal bit for bit to local pass + peer pass +
    merge_attn_states).  The two-step form's local pass and merge kernel are
    timed as well, for comparison."""
    from hcp_vllm_plugin_amd import merge_attn_states, ring_attn_merged, ring_attn_with_lse

    n = 8192
    q, kl, vl, kp, vp = prefill_inputs(dev)
    out = torch.empty_like(q)

    def step(ev=None):
        if ev is not None:
            ev[0].record()
        o_peer, lse_peer = ring_attn_with_lse(q, kp, vp, SCALE, None)
        if ev is not None:
            ev[1].record()
        ring_attn_merged(q, kl, vl, SCALE, 0, o_peer, lse_peer, output=out)
        if ev is not None:
            ev[2].record()

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(evs[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    t_peer = [e[0].elapsed_time(e[1]) for e in evs]
    t_loc = [e[1].elapsed_time(e[2]) for e in evs]
    # the two-step form: plain local pass and the separate merge kernel
    t_loc_plain = t_merge = float("nan")
    if two_step:
        t_loc_plain = timed(lambda: ring_attn_with_lse(q, kl, vl, SCALE, 0), steps, warmup)
        o_l, l_l = ring_attn_with_lse(q, kl, vl, SCALE, 0)
        o_p, l_p = ring_attn_with_lse(q, kp, vp, SCALE, None)
        t_merge = timed(lambda: merge_attn_states(out, o_p, l_p, o_l, l_l), steps, warmup)
    f_loc = 4 * D * H * causal_pairs(n, n, 0)
    f_peer = 4 * D * H * n * n
    merge_bytes = 3 * n * H * D * 2 + 2 * n * H * 4
    return {
        "wall_s": wall,
        "ms_per_step": wall * 1e3 / steps,
        "flops": f_loc + f_peer,
        "local": {"ms": statistics.mean(t_loc), "flops": f_loc},
        "peer": {"ms": statistics.mean(t_peer), "flops": f_peer},
        "local_plain": {"ms": t_loc_plain, "flops": f_loc},
        "merge": {"ms": t_merge, "bytes": merge_bytes},
    }


def decode_inputs(dev, seed=3, seqs=64, peer_len=32768, bs=16):
    from hcp_vllm_plugin_amd.varlen import head_major

    gen = torch.Generator().manual_seed(seed)
    loc = torch.randint(512, 2049, (seqs,), generator=gen).tolist()
    blocks = [-(-l // bs) for l in loc]
    nb = sum(blocks) + 16
    # big tensors drawn on the device from a seeded device generator
    dgen = torch.Generator(device=dev).manual_seed(seed)
    cache = torch.randn(nb, HKV, bs, 2 * D, generator=dgen, device=dev).to(torch.bfloat16)
    pk = torch.randn(seqs * peer_len, HKV, D, generator=dgen, device=dev).to(torch.bfloat16)
    pv = torch.randn(seqs * peer_len, HKV, D, generator=dgen, device=dev).to(torch.bfloat16)
    # the peer prefix as stage_peer_kv stores staged chunks: head-major
    pk, pv = head_major(pk), head_major(pv)
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


def bench_decode_forward(dev, steps, warmup, seqs=64, peer_len=32768, bs=16, seed=3,
                         layers=4):
    """The batch-64 split-KV decode as the backend runs it:
    ``HcpRingAttentionImpl.forward`` on one decode step of 64 requests whose
    32768-token prefixes are staged peer chunks (``stage_peer_kv`` +
    ``map_request_peer``, one chunk per request and layer) and whose
    U[512, 2048] local tokens are in the paged cache (the block-table rows also
    cover the prefix, whose pool slots the reference never reads: they point
    at one spare block).  Decode-ring off (``HCP_RING_DECODE_RING=0``).
    ``forward_ms`` is the per-layer call over ``layers`` layers of one step
    (metadata shared, as vLLM passes it); ``kernel_ms`` the same launch alone."""
    import types

    from hcp_vllm_plugin_amd import ring_backend as rb
    from hcp_vllm_plugin_amd.varlen import (DecodeBatch, PagedCache, segment_contiguous,
                                            segment_paged)

    os.environ["HCP_RING_DECODE_RING"] = "0"
    gen = torch.Generator().manual_seed(seed)
    loc = torch.randint(512, 2049, (seqs,), generator=gen).tolist()
    pre_blocks = peer_len // bs
    blocks = [-(-n // bs) for n in loc]
    nb = sum(blocks) + 1  # block 0: the prefix slots' spare block
    dgen = torch.Generator(device=dev).manual_seed(seed)
    caches = [torch.randn(nb, HKV, bs, 2 * D, generator=dgen, device=dev).to(torch.bfloat16)
              for _ in range(layers)]
    perm = (torch.randperm(nb - 1, generator=gen) + 1).to(torch.int32)
    bt = torch.zeros(seqs, pre_blocks + max(blocks), dtype=torch.int32)
    o = 0
    for r, nbk in enumerate(blocks):
        bt[r, pre_blocks:pre_blocks + nbk] = perm[o:o + nbk]
        o += nbk
    bt = bt.to(dev)
    q = torch.randn(seqs, H, D, generator=gen).to(torch.bfloat16).to(dev)
    # staged chunks as stage_peer_kv stores them: [n, Hkv, D] views of
    # head-major [Hkv, n, D] storage (stage_peer_kv keeps them without a copy)
    rb.clear_peer_kv()
    names = [f"model.layers.{i}.self_attn.attn" for i in range(layers)]
    stash = []
    for li, name in enumerate(names):
        pk = torch.randn(seqs, HKV, peer_len, D, generator=dgen, device=dev).to(torch.bfloat16)
        pv = torch.randn(seqs, HKV, peer_len, D, generator=dgen, device=dev).to(torch.bfloat16)
        stash.append((pk, pv))
        for r in range(seqs):
            rb.stage_peer_kv(f"req{r}-prefix", name, pk[r].permute(1, 0, 2), pv[r].permute(1, 0, 2))
    # a request is known by its first block id (ring_backend.py:740-754): the
    # prefix blocks are never read, so each row's first entry is its own id
    bt[:, 0] = torch.arange(1000, 1000 + seqs, dtype=torch.int32, device=dev)
    for r in range(seqs):
        rb.map_request_peer(1000 + r, [f"req{r}-prefix"])
    meta = types.SimpleNamespace(
        num_actual_tokens=seqs,
        query_start_loc=torch.arange(seqs + 1, dtype=torch.int32, device=dev),
        seq_lens=torch.tensor([peer_len + n for n in loc], dtype=torch.int32, device=dev),
        block_table=bt)
    impl = rb.HcpRingAttentionImpl(H, D, SCALE, HKV)
    out = torch.empty_like(q)
    layer_objs = [types.SimpleNamespace(layer_name=n) for n in names]

    def step():
        for li in range(layers):
            impl.forward(layer_objs[li], q, None, None, caches[li], meta, out)

    rb.reset_impl_stats()
    ms_step = timed(step, steps, warmup)
    assert rb.IMPL_STATS["decode_hip"] > 0 and rb.IMPL_STATS["attn_torch"] == 0
    # the same launch alone: layer 0's segments
    pc = PagedCache.from_tensor(caches[0])
    pk, pv = stash[0]
    segs = [[segment_paged(pc, bt[r], peer_len, loc[r]),
             segment_contiguous(pk[r].permute(1, 0, 2), pv[r].permute(1, 0, 2))]
            for r in range(seqs)]
    batch = DecodeBatch(segs, H, HKV, D, dev)
    ms_kernel = timed(lambda: batch.run(q, out, None, SCALE), steps, warmup)
    rb.clear_peer_kv()
    del stash, caches
    byts = (seqs * peer_len + sum(loc)) * HKV * D * 2 * 2 + seqs * H * D * 2 * 2
    fwd = ms_step / layers
    return {
        "workload": (f"batch-{seqs} decode through HcpRingAttentionImpl.forward: {peer_len}-token "
                     f"staged peer prefix per request (stage_peer_kv + map_request_peer) + "
                     f"U[512,2048] paged local, {layers} layers of one step"),
        "forward_ms": round(fwd, 4), "kernel_ms": round(ms_kernel, 4),
        "forward_over_kernel": round(fwd / ms_kernel, 4),
        "gbs_forward": round(byts / (fwd * 1e-3) / 1e9, 1), "bytes": byts,
    }


def bench_decode_paged(dev, steps, warmup, seqs=64, keys=34000, bs=16, seed=7):
    """Serving decode with every key in the paged cache (no peer): 64 requests
    of 34000 keys, the layer's cache [nb, 4, 16, 256] bf16 of 4.46 GB (past
    the 4 GiB of 32-bit buffer offsets, so the 64-bit load path).  ``ms`` is
    the split-KV kernel pair; ``forward_ms`` the backend's whole per-layer
    call (HcpRingAttentionImpl.forward: planning + launch), metadata reused
    across calls as vLLM does across the layers of a step."""
    import types

    from hcp_vllm_plugin_amd import ring_backend as rb

    gen = torch.Generator(device=dev).manual_seed(seed)
    nbk = -(-keys // bs)
    nb = seqs * nbk + 4
    cache = torch.empty(nb, HKV, bs, 2 * D, dtype=torch.bfloat16, device=dev)
    cache.normal_(generator=gen)
    perm = torch.randperm(nb, device=dev, generator=gen)[: seqs * nbk].to(torch.int32)
    bt = perm.view(seqs, nbk).contiguous()
    q = torch.randn(seqs, H, D, generator=gen, device=dev).to(torch.bfloat16)
    meta = types.SimpleNamespace(
        num_actual_tokens=seqs,
        query_start_loc=torch.arange(seqs + 1, dtype=torch.int32, device=dev),
        seq_lens=torch.full((seqs,), keys, dtype=torch.int32, device=dev), block_table=bt)
    impl = rb.HcpRingAttentionImpl(H, D, SCALE, HKV)
    layer = types.SimpleNamespace(layer_name="bench")
    out = torch.empty_like(q)
    fwd = lambda: impl.forward(layer, q, None, None, cache, meta, out)
    ms_fwd = timed(fwd, steps, warmup)
    from hcp_vllm_plugin_amd.varlen import DecodeBatch, PagedCache, paged_entry_array

    pc = PagedCache.from_tensor(cache)
    ent = paged_entry_array(pc, bt, range(seqs), range(seqs), 1, 0, [0] * seqs, [keys] * seqs)
    batch = DecodeBatch.from_entries(ent, H, HKV, D, dev, keep=(cache, bt))
    ms = timed(lambda: batch.run(q, out, None, SCALE), steps, warmup)
    byts = seqs * keys * HKV * D * 2 * 2 + seqs * H * D * 2 * 2
    del cache
    return {
        "workload": (f"serving decode, all keys paged: {seqs} requests x {keys} keys, cache "
                     f"[{nb},4,16,256] bf16 ({nb * HKV * bs * 2 * D * 2 / 1e9:.2f} GB)"),
        "ms": round(ms, 4), "gbs": round(byts / (ms * 1e-3) / 1e9, 1),
        "frac_hbm": round(byts / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4), "bytes": byts,
        "forward_ms": round(ms_fwd, 4),
    }


def timed(fn, steps, warmup):
    """Mean ms of fn() over `steps` runs after `warmup`, HIP events on the
    current stream."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps)]
    for a, b in evs:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    return statistics.mean(a.elapsed_time(b) for a, b in evs)


def bench_sustained(dev, seconds=10.0, window=20):
    """The headline step under sustained load: the same step as bench_prefill,
    back to back for about ``seconds`` seconds, timed in consecutive windows
    of ``window`` steps (wall clock around each window, synchronized).  The
    default bench line is the cold-start figure the contract asks for (a few
    warm-up steps, then the timed steps); this part shows how the rate
    settles as the part's power management adapts to the load."""
    from hcp_vllm_plugin_amd import ring_attn_merged, ring_attn_with_lse

    n = 8192
    q, kl, vl, kp, vp = prefill_inputs(dev)
    out = torch.empty_like(q)

    def step():
        o_peer, lse_peer = ring_attn_with_lse(q, kp, vp, SCALE, None)
        ring_attn_merged(q, kl, vl, SCALE, 0, o_peer, lse_peer, output=out)

    flops = 4 * D * H * (causal_pairs(n, n, 0) + n * n)
    windows = []
    t_end = time.perf_counter() + seconds
    torch.cuda.synchronize()
    while time.perf_counter() < t_end:
        t0 = time.perf_counter()
        for _ in range(window):
            step()
        torch.cuda.synchronize()
        windows.append((time.perf_counter() - t0) * 1e3 / window)
    ms = [round(w, 4) for w in windows]
    best = min(windows)
    return {
        "workload": ("the headline ring prefill step back to back for "
                     f"{seconds:.0f} s, {window}-step windows"),
        "windows": len(ms),
        "first_window_ms": ms[0],
        "last_window_ms": ms[-1],
        "median_window_ms": round(statistics.median(windows), 4),
        "best_window_ms": round(best, 4),
        "best_tflops": round(flops / (best * 1e-3) / 1e12, 2),
        "window_ms": ms[:: max(1, len(ms) // 25)],
    }


def bench_varlen(dev, steps, warmup, seed=2, nreq=16, bs=16):
    """Continuous-batch varlen prefill: 16 requests, local lengths U[512, 4096]
    causal over a paged [num_blocks, 4, 16, 256] cache (random block table,
    the row also covers the request's prefix blocks, which are not read),
    peer prefixes 16*U[64, 1024] packed contiguously.  One launch per segment
    kind for the whole batch, then one merge over all rows."""
    from hcp_vllm_plugin_amd import merge_attn_states
    from hcp_vllm_plugin_amd.varlen import (
        PagedCache, VarlenLaunch, make_entry, segment_contiguous, segment_paged)

    gen = torch.Generator().manual_seed(seed)
    loc = torch.randint(512, 4097, (nreq,), generator=gen).tolist()
    pre = (16 * torch.randint(64, 1025, (nreq,), generator=gen)).tolist()
    blocks = [-(-(p + l) // bs) for p, l in zip(pre, loc)]
    nb = sum(blocks) + 8
    dgen = torch.Generator(device=dev).manual_seed(seed)
    cache = torch.randn(nb, HKV, bs, 2 * D, generator=dgen, device=dev).to(torch.bfloat16)
    tq, tp = sum(loc), sum(pre)
    q = torch.randn(tq, H, D, generator=dgen, device=dev).to(torch.bfloat16)
    pk = torch.randn(tp, HKV, D, generator=dgen, device=dev).to(torch.bfloat16)
    pv = torch.randn(tp, HKV, D, generator=dgen, device=dev).to(torch.bfloat16)
    perm = torch.randperm(nb, generator=gen).to(torch.int32)
    bt = torch.zeros(nreq, max(blocks), dtype=torch.int32)
    o = 0
    for r, nbk in enumerate(blocks):
        bt[r, :nbk] = perm[o:o + nbk]
        o += nbk
    bt = bt.to(dev)
    pc = PagedCache.from_tensor(cache)
    loc_e, peer_e = [], []
    qs = ps = 0
    for r in range(nreq):
        loc_e.append(make_entry(qs, loc[r], segment_paged(pc, bt[r], pre[r], loc[r]), 0))
        peer_e.append(make_entry(qs, loc[r], segment_contiguous(pk, pv, ps, pre[r])))
        qs += loc[r]
        ps += pre[r]
    l_launch = VarlenLaunch(loc_e, True, True, dev)
    p_launch = VarlenLaunch(peer_e, False, False, dev)
    o_loc, o_peer, out = (torch.empty_like(q) for _ in range(3))
    lse_loc = torch.empty(H, tq, device=dev)
    lse_peer = torch.empty(H, tq, device=dev)
    # the same local keys gathered into contiguous [T, Hkv, D] tensors (set-up,
    # outside every timed region): the paged launch's contiguous counterpart
    kc_parts, vc_parts, locc_e = [], [], []
    for r in range(nreq):
        tok = torch.arange(pre[r], pre[r] + loc[r], device=dev)
        blk = bt[r][tok // bs].long()
        kc_parts.append(cache[blk, :, tok % bs, :D])
        vc_parts.append(cache[blk, :, tok % bs, D:])
    kc, vc = torch.cat(kc_parts).contiguous(), torch.cat(vc_parts).contiguous()
    qs = cs = 0
    for r in range(nreq):
        locc_e.append(make_entry(qs, loc[r], segment_contiguous(kc, vc, cs, loc[r]), 0))
        qs += loc[r]
        cs += loc[r]
    c_launch = VarlenLaunch(locc_e, True, False, dev)
    t_peer = timed(lambda: p_launch.run(q, o_peer, lse_peer, HKV, SCALE), steps, warmup)
    t_loc = timed(lambda: l_launch.run(q, out, None, HKV, SCALE, acc=(o_peer, lse_peer)),
                  steps, warmup)
    t_loc_c = timed(lambda: c_launch.run(q, o_loc, None, HKV, SCALE, acc=(o_peer, lse_peer)),
                    steps, warmup)
    # the two-step form: plain local launch and the separate merge
    t_loc_plain = timed(lambda: l_launch.run(q, o_loc, lse_loc, HKV, SCALE), steps, warmup)
    t_merge = timed(lambda: merge_attn_states(out, o_peer, lse_peer, o_loc, lse_loc),
                    steps, warmup)
    pairs_l = sum(causal_pairs(l, l, 0) for l in loc)
    pairs_p = sum(l * p for l, p in zip(loc, pre))
    f_l, f_p = 4 * D * H * pairs_l, 4 * D * H * pairs_p
    t = t_loc + t_peer
    tf = (f_l + f_p) / (t * 1e-3) / 1e12
    return {
        "workload": (f"varlen prefill: {nreq} requests, local U[512,4096] causal over a paged "
                     f"[nb,4,16,256] cache + peer 16*U[64,1024] contiguous: the peer launch, "
                     f"then the local launch merging the peer result into the output"),
        "query_tokens": tq, "peer_tokens": tp,
        "ms": round(t, 4), "tflops": round(tf, 2), "frac": round(tf / PEAK_BF16_TFLOPS, 4),
        "local_paged_merged": {"ms": round(t_loc, 4),
                               "tflops": round(f_l / (t_loc * 1e-3) / 1e12, 2)},
        "local_contiguous_merged": {"ms": round(t_loc_c, 4),
                                    "tflops": round(f_l / (t_loc_c * 1e-3) / 1e12, 2),
                                    "paged_tflops_over_contiguous": round(t_loc_c / t_loc, 4)},
        "peer": {"ms": round(t_peer, 4), "tflops": round(f_p / (t_peer * 1e-3) / 1e12, 2)},
        "two_step": {"local_paged_ms": round(t_loc_plain, 4), "merge_ms": round(t_merge, 4),
                     "ms": round(t_loc_plain + t_peer + t_merge, 4)},
        "tflop": round((f_l + f_p) / 1e12, 3),
    }


def bench_kv_cache_write(dev, steps, warmup, seed=2, n=43125, nb=12000, bs=16):
    """Paged KV-cache write (the step before the path): n tokens' K/V [n, 4, 128]
    bf16 into a [nb, 4, 16, 256] cache at a seeded random slot permutation
    (n = the varlen batch's new tokens), and the 64-token decode-step write."""
    from hcp_vllm_plugin_amd.kv_cache import reshape_and_cache

    gen = torch.Generator().manual_seed(seed)
    dgen = torch.Generator(device=dev).manual_seed(seed)
    cache = torch.zeros(nb, HKV, bs, 2 * D, dtype=torch.bfloat16, device=dev)
    key = torch.randn(n, HKV, D, generator=dgen, device=dev).to(torch.bfloat16)
    value = torch.randn(n, HKV, D, generator=dgen, device=dev).to(torch.bfloat16)
    slots = torch.randperm(nb * bs, generator=gen)[:n].to(dev)
    ms = timed(lambda: reshape_and_cache(key, value, cache, slots), steps, warmup)
    ms64 = timed(lambda: reshape_and_cache(key[:64], value[:64], cache, slots[:64]),
                 steps, warmup)
    byts = n * HKV * D * 2 * 2 * 2  # K and V, read and written
    return {
        "workload": (f"paged KV-cache write: {n} tokens [n,4,128] bf16 into [nb,4,16,256] at "
                     f"random slots; and a 64-token decode step"),
        "ms": round(ms, 4), "gbs": round(byts / (ms * 1e-3) / 1e9, 1),
        "frac_hbm": round(byts / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
        "bytes": byts, "decode_step_us": round(ms64 * 1e3, 2),
    }


def bench_peer_ingest(dev, steps, warmup, chunks=(4096, 4096), fmt="k_v"):
    """Peer-KV ingest of one layer: a request's chunk files (ring connector
    {"k","v"}: [n, 4, 128] bf16 safetensors, in the page cache) into one packed
    device buffer, against the reference's way -- safetensors load_file to
    the device per chunk, .contiguous(), torch.cat (ring_connector.py:908-915,
    ring_backend.py:766-772).  Wall clock per layer, copies complete."""
    import tempfile

    import safetensors.torch as st
    from hcp_vllm_plugin_amd.peer_ingest import PeerIngest

    gen = torch.Generator().manual_seed(5)
    tmp = tempfile.mkdtemp(prefix="hcp_ingest_")
    paths = []
    for i, n in enumerate(chunks):
        p = os.path.join(tmp, f"layer0_chunk{i}.safetensors")
        st.save_file({"k": torch.randn(n, HKV, D, generator=gen).to(torch.bfloat16),
                      "v": torch.randn(n, HKV, D, generator=gen).to(torch.bfloat16)}, p)
        paths.append(p)
    ing = PeerIngest(dev, fmt)

    def ours():
        r = ing.load(paths)
        r.event.synchronize()

    def ref():
        parts = [st.load_file(p, device=str(dev)) for p in paths]
        k = torch.cat([t["k"].contiguous() for t in parts])
        v = torch.cat([t["v"].contiguous() for t in parts])
        torch.cuda.synchronize()
        return k, v

    def wall(fn):
        for _ in range(warmup):
            fn()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        return (time.perf_counter() - t0) * 1e3 / steps

    ms, ms_ref = wall(ours), wall(ref)
    byts = sum(chunks) * HKV * D * 2 * 2
    for p in paths:
        os.remove(p)
    os.rmdir(tmp)
    return {
        "workload": (f"peer-KV ingest of one layer: {len(chunks)} chunk files of "
                     f"{list(chunks)} tokens ([n,4,128] bf16 k and v) into one packed device "
                     f"buffer, vs safetensors load_file(device) + torch.cat"),
        "ms": round(ms, 4), "gbs": round(byts / (ms * 1e-3) / 1e9, 2),
        "reference_way_ms": round(ms_ref, 4), "bytes": byts,
    }


def bench_sliding_window(dev, steps, warmup, window=4096, n=8192):
    """The local causal pass of the 8k step with a sliding window (a
    Mistral-style 4096-key window at the 7B attention shape): the kernel
    skips keys below each workgroup's window, so the algorithmic work is the
    visible pairs sum_i min(i + 1, window)."""
    from hcp_vllm_plugin_amd import ring_attn_with_lse

    q, kl, vl, _, _ = prefill_inputs(dev)
    win = lambda: ring_attn_with_lse(q, kl, vl, SCALE, 0, window)
    full = lambda: ring_attn_with_lse(q, kl, vl, SCALE, 0)
    timed(full, 2, warmup)  # clocks settled before either is timed
    ms = timed(win, steps, warmup)
    ms_full = timed(full, steps, warmup)
    pairs = sum(min(i + 1, window) for i in range(n))
    flops = 4 * D * H * pairs
    tf = flops / (ms * 1e-3) / 1e12

    def tile_wgs(w):  # (64-key tile x 128-row workgroup) units the kernel executes
        return H * sum(-(-(qb * 128 + 128 - (0 if w is None else max(0, qb * 128 - w + 1)))
                         // 64) for qb in range(n // 128))

    return {
        "workload": (f"local causal pass, {n} queries x {n} keys, sliding window {window}, "
                     f"28/4 heads, head_dim 128, bf16; the same pass without the window "
                     f"timed right after"),
        "ms": round(ms, 4), "tflops": round(tf, 2), "frac": round(tf / PEAK_BF16_TFLOPS, 4),
        "tflop": round(flops / 1e12, 3),
        "ns_per_tile": round(ms * 1e6 / tile_wgs(window), 2),
        "no_window": {"ms": round(ms_full, 4),
                      "ns_per_tile": round(ms_full * 1e6 / tile_wgs(None), 2)},
    }


def bench_ring_decode_hop(dev, steps, warmup, seed=6, chunk=32768, growth=512):
    """One decode-ring hop at Qwen2.5-7B shape (q [1,28,128] bf16): a node's
    partial over its 32768-key chunk snapshot + 512 growth tokens merged into
    the accumulator with LSE out.  ``ms`` is the device step (split-KV decode
    over [chunk, growth] + merge); ``packet_ms`` the whole ``handle_packet``
    (decode the packet, uploads, the step, one download, re-encode), wall
    clock.  ``reference_way_ms`` runs the reference's structure
    (ring_decode.py:224-237: torch.cat of chunk and growth, the prefill kernel
    with Tq=1, merge_attn_states, the LSE in four torch ops) on this build's
    kernels, for comparison."""
    from hcp_vllm_plugin_amd import ring_decode as rd
    from hcp_vllm_plugin_amd.merge import merge_attn_states
    from hcp_vllm_plugin_amd.ring_attn import ring_attn_with_lse

    dgen = torch.Generator(device=dev).manual_seed(seed)

    def rn(*shape):
        return torch.randn(*shape, generator=dgen, device=dev).to(torch.bfloat16)

    ck, cv = rn(chunk, HKV, D), rn(chunk, HKV, D)
    node = rd.RingDecodeNode("", ["c"], 1, device=str(dev), dtype=torch.bfloat16,
                             background=False)
    node.add_chunk("c", "L", ck, cv)
    node.mark_ready()
    gk, gv = rn(growth, HKV, D), rn(growth, HKV, D)
    node.append_growth("r", "L", gk, gv)
    q, o0 = rn(1, H, D), rn(1, H, D)
    l0 = torch.randn(H, 1, generator=dgen, device=dev)
    sc = 1.0 / math.sqrt(D)
    ms = timed(lambda: node.accumulate(q, o0, l0, sc, "L", "r"), steps, warmup)

    def ref_way():
        k = torch.cat([ck, gk], 0)
        v = torch.cat([cv, gv], 0)
        o_loc, lse_loc = ring_attn_with_lse(q, k, v, sc, None)
        out = torch.empty_like(o0)
        merge_attn_states(out, o0, l0, o_loc, lse_loc)
        m = torch.maximum(l0, lse_loc)
        return out, m + torch.log(torch.exp(l0 - m) + torch.exp(lse_loc - m))

    ms_ref = timed(ref_way, steps, warmup)
    pkt = rd.encode_packet(q, o0, l0, sc, "L", "c", "r")
    for _ in range(warmup):
        node.handle_packet(pkt)
    t0 = time.perf_counter()
    for _ in range(steps):
        node.handle_packet(pkt)
    packet_ms = (time.perf_counter() - t0) * 1e3 / steps
    byts = (chunk + growth) * HKV * D * 2 * 2
    return {
        "workload": (f"decode-ring hop: q [1,28,128] bf16 over a {chunk}-key chunk snapshot + "
                     f"{growth} growth tokens ([n,4,128] k and v), merged with LSE out"),
        "ms": round(ms, 4), "gbs": round(byts / (ms * 1e-3) / 1e9, 1),
        "frac_hbm": round(byts / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
        "bytes": byts, "packet_ms": round(packet_ms, 4),
        "reference_way_ms": round(ms_ref, 4),
    }


def bench_head_dim_256(dev, steps, warmup, seed=7, n=8192, seqs=32, keys=32768):
    """head_dim 256 (a Gemma-2-9B-like attention shape: 16 query heads, 8 KV
    heads, bf16): the ring prefill step (8192 peer keys non-causal, then 8192
    local causal keys merging the peer result) and a split-KV decode of 32
    sequences x 32768 staged keys.  Runs the one-wave-per-SIMD prefill and the
    two-wave decode instantiations; a widening line, not a headline."""
    from hcp_vllm_plugin_amd import ring_attn_merged, ring_attn_with_lse
    from hcp_vllm_plugin_amd.varlen import DecodeBatch, head_major, segment_contiguous

    h, hkv, d = 16, 8, 256
    sc = 1.0 / math.sqrt(d)
    dgen = torch.Generator(device=dev).manual_seed(seed)

    def rn(*shape):
        return torch.randn(*shape, generator=dgen, device=dev).to(torch.bfloat16)

    q, kl, vl, kp, vp = rn(n, h, d), rn(n, hkv, d), rn(n, hkv, d), rn(n, hkv, d), rn(n, hkv, d)
    out = torch.empty_like(q)

    def step():
        o_p, l_p = ring_attn_with_lse(q, kp, vp, sc, None)
        ring_attn_merged(q, kl, vl, sc, 0, o_p, l_p, output=out)

    ms = timed(step, steps, warmup)
    flops = 4 * d * h * (n * n + causal_pairs(n, n, 0))
    del q, kl, vl, kp, vp, out
    kd, vd = head_major(rn(seqs * keys, hkv, d)), head_major(rn(seqs * keys, hkv, d))
    qd = rn(seqs, h, d)
    batch = DecodeBatch([[segment_contiguous(kd, vd, s * keys, keys)] for s in range(seqs)],
                        h, hkv, d, dev)
    od = torch.empty_like(qd)
    dms = timed(lambda: batch.run(qd, od, None, sc), steps, warmup)
    dbytes = seqs * keys * hkv * d * 2 * 2 + seqs * h * d * 2 * 2
    return {
        "workload": (f"head_dim 256 (16 / 8 heads, bf16): ring prefill step {n} peer + {n} "
                     f"local causal keys merged; decode {seqs} x {keys} staged keys"),
        "prefill_ms": round(ms, 4),
        "prefill_tflops": round(flops / (ms * 1e-3) / 1e12, 2),
        "prefill_frac": round(flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
        "decode_ms": round(dms, 4),
        "decode_gbs": round(dbytes / (dms * 1e-3) / 1e9, 1),
        "decode_frac_hbm": round(dbytes / (dms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
    }


def bench_llama70b(dev, steps, warmup, seed=4, n=65536, chunk=8192):
    """Long-context layer at the Llama-3-70B attention shape (64 / 8 heads,
    head_dim 128), bf16: 65536 local query tokens causal over local keys
    (global offset 65536: the peer chunk comes first) + 65536 peer keys,
    processed as 8 query chunks of 8192; chunk c attends local keys
    [0, 8192(c+1)) at offset 8192c and all peer keys: the peer pass, then the
    local causal pass merging the peer result into the chunk's output."""
    from hcp_vllm_plugin_amd import ring_attn_merged, ring_attn_with_lse

    h, hkv = 64, 8
    dgen = torch.Generator(device=dev).manual_seed(seed)
    q = torch.randn(n, h, D, generator=dgen, device=dev).to(torch.bfloat16)
    kl = torch.randn(n, hkv, D, generator=dgen, device=dev)
    kp = torch.randn(n, hkv, D, generator=dgen, device=dev)
    ch = torch.randperm(D, generator=torch.Generator().manual_seed(seed))[:4].to(dev)
    kl[..., ch] *= 8.0
    kp[..., ch] *= 8.0
    kl, kp = kl.to(torch.bfloat16), kp.to(torch.bfloat16)
    vl = torch.randn(n, hkv, D, generator=dgen, device=dev).to(torch.bfloat16)
    vp = torch.randn(n, hkv, D, generator=dgen, device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    nchunk = n // chunk

    def step(ev=None):
        for c in range(nchunk):
            qc = q[c * chunk:(c + 1) * chunk]
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e2 = torch.cuda.Event(enable_timing=True)
            if ev is not None:
                e0.record()
            o_p, l_p = ring_attn_with_lse(qc, kp, vp, SCALE, None)
            if ev is not None:
                e1.record()
            ring_attn_merged(qc, kl[:chunk * (c + 1)], vl[:chunk * (c + 1)], SCALE, chunk * c,
                             o_p, l_p, output=out[c * chunk:(c + 1) * chunk])
            if ev is not None:
                e2.record()
                ev.append((e0, e1, e2))

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    evs = []
    t0 = time.perf_counter()
    for _ in range(steps):
        step(evs)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    peer = sum(a.elapsed_time(b) for a, b, _ in evs) / steps
    local = sum(b.elapsed_time(c) for _, b, c in evs) / steps
    pairs = sum(causal_pairs(chunk, chunk * (c + 1), chunk * c) for c in range(nchunk)) + n * n
    flops = 4 * D * h * pairs
    tf = flops / (wall * 1e-3) / 1e12
    return {
        "workload": ("Llama-3-70B attention shape (64/8 heads, head_dim 128) bf16: 65536 local "
                     "causal + 65536 peer keys, 8 query chunks of 8192, each local pass "
                     "merging its chunk's peer result"),
        "ms": round(wall, 3), "tflops": round(tf, 2), "frac": round(tf / PEAK_BF16_TFLOPS, 4),
        "peer_ms": round(peer, 3), "local_merged_ms": round(local, 3),
        "tflop": round(flops / 1e12, 2),
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

    host = cpu_host_info()
    threads = host["threads"]
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
        "threads": threads,
        "cpu_model": host["cpu_model"],
        "physical_cores": host["physical_cores"],
        "logical_cpus": host["logical_cpus"],
        "cpus_granted": host["cpus_granted"],
        "kind": "port",
        "sample": (f"the full prefill step (8192 local causal + 8192 peer + merge, 28/4 heads) "
                   f"on the CPU oracle (torch fp32), one KV-head group at a time; "
                   f"{flops / 1e12:.3f} TFLOP in {t:.2f} s, median of {len(times)} steps, "
                   f"{threads} threads ({host['threads_rule']})"),
    }


def cpu_baseline_configs(threads: int) -> dict:
    """The CPU oracle on bounded samples of the other workloads, each in the
    unit of its GPU line: the batch-64 split-KV decode (four sequences of its
    shape: 32768 peer + U[512, 2048] local keys, GB/s of K/V read), the
    16-request varlen batch (two requests of its length distribution,
    TFLOP/s) and the Llama-3-70B 128k layer (1024 queries of chunk 0 for one
    KV-head group; the whole layer's CPU time is extrapolated from that rate
    and stated as such).  Seeded CPU inputs of the same shapes: the rate does
    not depend on the values."""
    from oracle import ring_oracle as orc

    host = cpu_host_info()
    common = {"cores": threads, "threads": threads, "cpu_model": host["cpu_model"],
              "kind": "port"}

    def ring_rows(q, kl, vl, kp, vp, off):
        """local causal at `off` over kl/vl, peer over kp/vp, merged (oracle)"""
        o_l, l_l = orc.attn_with_lse(q, kl, vl, SCALE, off)
        o_p, l_p = orc.attn_with_lse(q, kp, vp, SCALE, None)
        return orc.merge_pair(o_p, l_p, o_l, l_l)

    gen = torch.Generator().manual_seed(11)
    res = {}
    # decode: one query per sequence over its peer chunk and local keys
    seqs, peer_len = 4, 32768
    loc = torch.randint(512, 2049, (seqs,), generator=gen).tolist()
    t_dec, nbytes = 0.0, 0
    for s in range(seqs):
        q = torch.randn(1, H, D, generator=gen).to(torch.bfloat16).float()
        kp, vp = (torch.randn(peer_len, HKV, D, generator=gen).to(torch.bfloat16).float()
                  for _ in range(2))
        kl, vl = (torch.randn(loc[s], HKV, D, generator=gen).to(torch.bfloat16).float()
                  for _ in range(2))
        t0 = time.perf_counter()  # the oracle's own time, not the input draws
        ring_rows(q, kl, vl, kp, vp, loc[s] - 1)
        t_dec += time.perf_counter() - t0
        nbytes += (peer_len + loc[s]) * HKV * D * 2 * 2 + H * D * 2 * 2
    res["decode"] = {**common, "value": round(nbytes / t_dec / 1e9, 2), "unit": "GB/s",
                     "ms_per_sequence": round(t_dec * 1e3 / seqs, 1),
                     "sample": (f"{seqs} decode sequences of the batch-64 shape (32768 peer + "
                                f"U[512,2048] local keys, 28/4 heads): local causal + peer + "
                                f"merge per sequence, {nbytes / 1e9:.3f} GB of K/V in "
                                f"{t_dec:.2f} s, {threads} threads")}
    # varlen: two requests, local causal over their own keys + peer prefix
    loc = torch.randint(512, 4097, (2,), generator=gen).tolist()
    pre = (16 * torch.randint(64, 1025, (2,), generator=gen)).tolist()
    flops, t_var = 0, 0.0
    for r in range(2):
        q = torch.randn(loc[r], H, D, generator=gen).to(torch.bfloat16).float()
        kl, vl = (torch.randn(loc[r], HKV, D, generator=gen).to(torch.bfloat16).float()
                  for _ in range(2))
        kp, vp = (torch.randn(pre[r], HKV, D, generator=gen).to(torch.bfloat16).float()
                  for _ in range(2))
        g = H // HKV
        t0 = time.perf_counter()
        for j in range(HKV):  # one KV-head group at a time bounds the score buffers
            sl, hs = slice(j, j + 1), slice(j * g, (j + 1) * g)
            ring_rows(q[:, hs], kl[:, sl], vl[:, sl], kp[:, sl], vp[:, sl], 0)
        t_var += time.perf_counter() - t0
        flops += 4 * D * H * (causal_pairs(loc[r], loc[r], 0) + loc[r] * pre[r])
    res["varlen16_paged"] = {**common, "value": round(flops / t_var / 1e12, 4),
                             "unit": "TFLOP/s",
                             "sample": (f"2 requests of the varlen batch's distribution "
                                        f"(local {loc} causal + peer {pre}, 28/4 heads), one "
                                        f"KV-head group at a time: {flops / 1e12:.3f} TFLOP in "
                                        f"{t_var:.2f} s, {threads} threads")}
    # Llama-3-70B layer: 1024 queries of chunk 0, one KV-head group (8 heads)
    h70, hkv70, rows, n = 64, 8, 1024, 65536
    g = h70 // hkv70
    q = torch.randn(rows, g, D, generator=gen).to(torch.bfloat16).float()
    kl, vl = (torch.randn(rows, 1, D, generator=gen).to(torch.bfloat16).float() for _ in range(2))
    kp, vp = (torch.randn(n, 1, D, generator=gen).to(torch.bfloat16).float() for _ in range(2))
    t0 = time.perf_counter()
    ring_rows(q, kl, vl, kp, vp, 0)
    t70 = time.perf_counter() - t0
    f_sample = 4 * D * g * (causal_pairs(rows, rows, 0) + rows * n)
    pairs_layer = sum(causal_pairs(8192, 8192 * (c + 1), 8192 * c) for c in range(8)) + n * n
    f_layer = 4 * D * h70 * pairs_layer
    rate = f_sample / t70
    res["llama70b_128k"] = {**common, "value": round(rate / 1e12, 4), "unit": "TFLOP/s",
                            "layer_s_extrapolated": round(f_layer / rate, 1),
                            "sample": (f"{rows} queries of chunk 0 (local causal over its {rows} "
                                       f"keys + 65536 peer keys + merge) for one KV-head group "
                                       f"(8 of 64 heads): {f_sample / 1e12:.3f} TFLOP in "
                                       f"{t70:.2f} s, {threads} threads; the whole layer "
                                       f"({f_layer / 1e12:.1f} TFLOP) extrapolated at that rate")}
    return res


def cpu_host_info() -> dict:
    """The host CPU as the CPU baseline uses it.

    ``threads`` is every CPU this process may run on (its affinity set, which
    is what ``os.cpu_count()`` means for it), capped by ``OMP_NUM_THREADS``
    when the machine sets one: a GPU host shared by several GPU jobs grants
    each its CPU share that way.  Model and physical-core count come from
    /proc/cpuinfo (unique (physical id, core id) pairs)."""
    logical = os.cpu_count() or 1
    try:
        granted = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        granted = logical
    threads, rule = granted, "all CPUs granted to the process"
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and 0 < int(omp) < granted:
        threads, rule = int(omp), f"the host's CPU share OMP_NUM_THREADS={omp} of {granted} granted"
    model, cores = "unknown", set()
    try:
        with open("/proc/cpuinfo") as f:
            phys = core = None
            for ln in f:
                k, _, v = ln.partition(":")
                k, v = k.strip(), v.strip()
                if k == "model name" and model == "unknown":
                    model = v
                elif k == "physical id":
                    phys = v
                elif k == "core id":
                    core = v
                elif not k and phys is not None:
                    cores.add((phys, core))
                    phys = core = None
            if phys is not None:
                cores.add((phys, core))
    except OSError:
        pass
    return {"threads": threads, "threads_rule": rule, "cpu_model": model,
            "physical_cores": len(cores) or None, "logical_cpus": logical,
            "cpus_granted": granted}


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


TRAFFIC_SOURCE = ("profiles/traffic.json: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE passes "
                  "over this bench's workload (committed, not measured in this run), scaled "
                  "by a 1 GiB device copy's counts")


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
    ap.add_argument("--no-two-step", action="store_true",
                    help="skip timing the unfused local pass + merge (kernel traces of the step)")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the varlen and 70B long-context measurements")
    ap.add_argument("--part", choices=("all", "prefill", "decode", "varlen", "llama70b",
                                       "kvwrite", "ingest", "ringdec", "window", "pdecode",
                                       "fdecode", "d256", "copy", "sustained"),
                    default="all",
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

    if args.part == "sustained":
        print(json.dumps(bench_sustained(dev)), flush=True)
        return
    if args.part == "copy":
        print(json.dumps(copy_probe(dev)), flush=True)
        return
    if args.part == "decode":
        print(json.dumps(bench_decode(dev, args.steps, args.warmup)), flush=True)
        return
    if args.part == "varlen":
        print(json.dumps(bench_varlen(dev, args.steps, args.warmup)), flush=True)
        return
    if args.part == "ingest":
        print(json.dumps(bench_peer_ingest(dev, args.steps, args.warmup)), flush=True)
        return
    if args.part == "fdecode":
        print(json.dumps(bench_decode_forward(dev, args.steps, args.warmup)), flush=True)
        return
    if args.part == "pdecode":
        print(json.dumps(bench_decode_paged(dev, args.steps, args.warmup)), flush=True)
        return
    if args.part == "window":
        print(json.dumps(bench_sliding_window(dev, args.steps, args.warmup)), flush=True)
        return
    if args.part == "ringdec":
        print(json.dumps(bench_ring_decode_hop(dev, args.steps, args.warmup)), flush=True)
        return
    if args.part == "d256":
        print(json.dumps(bench_head_dim_256(dev, args.steps, args.warmup)), flush=True)
        return
    if args.part == "kvwrite":
        print(json.dumps(bench_kv_cache_write(dev, args.steps, args.warmup)), flush=True)
        return
    if args.part == "llama70b":
        print(json.dumps(bench_llama70b(dev, 2, 1)), flush=True)
        return
    pre = bench_prefill(dev, args.steps, args.warmup, two_step=not args.no_two_step)
    if args.part == "prefill":
        print(json.dumps(pre), flush=True)
        return
    dec = None if args.no_decode else bench_decode(dev, args.steps, args.warmup)
    extra = {}
    if not args.no_configs:
        extra["varlen16_paged"] = bench_varlen(dev, args.steps, args.warmup)
        extra["llama70b_128k"] = bench_llama70b(dev, 2, 1)
        extra["kv_cache_write"] = bench_kv_cache_write(dev, args.steps, args.warmup)
        extra["peer_ingest"] = bench_peer_ingest(dev, args.steps, args.warmup)
        extra["ring_decode_hop"] = bench_ring_decode_hop(dev, args.steps, args.warmup)
        extra["sliding_window"] = bench_sliding_window(dev, args.steps, args.warmup)
        extra["decode_paged"] = bench_decode_paged(dev, args.steps, args.warmup)
        extra["decode_forward_staged"] = bench_decode_forward(dev, args.steps, args.warmup)
        extra["head_dim_256"] = bench_head_dim_256(dev, args.steps, args.warmup)
    cpu = None if args.no_cpu_baseline else cpu_baseline()
    cpu_cfg = (None if args.no_cpu_baseline or (args.no_decode and args.no_configs)
               else cpu_baseline_configs(cpu["threads"]))
    traffic = load_traffic()

    value = pre["flops"] / (pre["ms_per_step"] * 1e-3) / 1e12
    peer_tf = pre["peer"]["flops"] / (pre["peer"]["ms"] * 1e-3) / 1e12
    loc_tf = pre["local"]["flops"] / (pre["local"]["ms"] * 1e-3) / 1e12
    locp_tf = pre["local_plain"]["flops"] / (pre["local_plain"]["ms"] * 1e-3) / 1e12
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
            "workload": ("ring prefill step: 8192 peer keys non-causal, then 8192 local causal "
                         "with the LSE merge in the same launch"),
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
            "traffic_source": TRAFFIC_SOURCE if traffic else None,
        },
        "kernels": {
            "local_causal_merged": {"ms": round(pre["local"]["ms"], 4),
                                    "tflops": round(loc_tf, 2),
                                    "frac": round(loc_tf / PEAK_BF16_TFLOPS, 4),
                                    "traffic": traffic.get("fa_fwd_local_merged", {}).get("bytes")},
            "peer": {"ms": round(pre["peer"]["ms"], 4), "tflops": round(peer_tf, 2),
                     "frac": round(peer_tf / PEAK_BF16_TFLOPS, 4)},
            "two_step": None if math.isnan(pre["merge"]["ms"]) else {
                         "local_causal_ms": round(pre["local_plain"]["ms"], 4),
                         "local_causal_tflops": round(locp_tf, 2),
                         "merge_ms": round(pre["merge"]["ms"], 4),
                         "merge_gbs": round(pre["merge"]["bytes"] / (pre["merge"]["ms"] * 1e-3)
                                            / 1e9, 1),
                         "step_ms": round(pre["local_plain"]["ms"] + pre["peer"]["ms"]
                                          + pre["merge"]["ms"], 4)},
        },
        "cpu_baseline": cpu,
    }
    if dec is not None:
        line["decode"] = {
            "workload": "split-KV decode: 64 seqs x (32768 peer staged head-major + U[512,2048] paged local)",
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
                "traffic_source": TRAFFIC_SOURCE if traffic else None,
            },
        }
        if cpu_cfg:
            line["decode"]["cpu_baseline"] = cpu_cfg["decode"]
    if extra:
        if cpu_cfg:
            for k in ("varlen16_paged", "llama70b_128k"):
                extra[k]["cpu_baseline"] = cpu_cfg[k]
        line["configs"] = extra
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
