"""GPU parity: batched varlen prefill (hcp_attn_fwd_varlen) with the local
segment read in place from the paged cache, the peer segment from packed
contiguous KV, and one merge -- against the oracle's per-request
gather + attention + merge (ring_backend.py:611-832).
"""

import pytest
import torch

from hcp_vllm_plugin_amd import merge_attn_states
from hcp_vllm_plugin_amd.varlen import (
    PagedCache,
    make_entry,
    segment_contiguous,
    segment_paged,
    varlen_attn_with_lse,
)
from oracle import ring_oracle as orc
from tests._util import LSE_TOL, OUT_TOL, max_err, randn, scale_for

pytestmark = pytest.mark.gpu


def _build(dev, layout, lens, peers, h, hkv, d, dtype, bs, seed):
    gen = torch.Generator().manual_seed(seed)
    blocks_per = [-(-(p + l) // bs) for p, l in zip(peers, lens)]
    nb = sum(blocks_per) + 3
    if layout == "v031":
        cache = randn(gen, (nb, hkv, bs, 2 * d), dtype)
    else:
        cache = randn(gen, (nb, 2, bs, hkv, d), dtype)
    perm = torch.randperm(nb, generator=gen).to(torch.int32)
    maxb = max(blocks_per)
    bt = torch.zeros(len(lens), maxb, dtype=torch.int32)
    o = 0
    for r, nbk in enumerate(blocks_per):
        bt[r, :nbk] = perm[o:o + nbk]
        o += nbk
    q = randn(gen, (sum(lens), h, d), dtype)
    peer = randn(gen, (sum(peers), 2, hkv, d), dtype)
    return cache, bt, q, peer


@pytest.mark.parametrize("layout", ["v031", "v023"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_varlen_local_paged_peer_contiguous(dev, layout, dtype):
    h, hkv, d, bs = 28, 4, 128, 16
    lens = [300, 1, 129, 700, 64, 0, 257]
    peers = [512, 48, 1024, 0, 16, 32, 400]
    cache, bt, q, peer = _build(dev, layout, lens, peers, h, hkv, d, dtype, bs, seed=41)
    cd, btd, qd, pd = cache.to(dev), bt.to(dev), q.to(dev), peer.to(dev)
    pc = PagedCache.from_tensor(cd)
    pk, pv = pd[:, 0], pd[:, 1]
    loc_e, peer_e = [], []
    qs, ps = 0, 0
    for r, (L, P) in enumerate(zip(lens, peers)):
        loc_e.append(make_entry(qs, L, segment_paged(pc, btd[r], P, L), 0))
        peer_e.append(make_entry(qs, L, segment_contiguous(pk, pv, ps, P), 0))
        qs += L
        ps += P
    scale = scale_for(d)
    o_loc, lse_loc = varlen_attn_with_lse(qd, loc_e, True, hkv, scale)
    o_peer, lse_peer = varlen_attn_with_lse(qd, peer_e, False, hkv, scale)
    out = torch.empty_like(o_loc)
    merge_attn_states(out, o_peer, lse_peer, o_loc, lse_loc)
    torch.cuda.synchronize()
    qs, ps = 0, 0
    for r, (L, P) in enumerate(zip(lens, peers)):
        qr = q[qs:qs + L].float()
        kl, vl = orc.gather_paged(cache.float(), bt[r], P, L, layout)
        rl, rll = orc.attn_with_lse(qr, kl, vl, scale, 0)
        rp, rpl = orc.attn_with_lse(qr, peer[ps:ps + P, 0].float(), peer[ps:ps + P, 1].float(),
                                    scale, None)
        rm = orc.lse_merge(rl, rll, rp, rpl)
        sl = slice(qs, qs + L)
        assert max_err(o_loc[sl], rl) <= OUT_TOL[dtype], r
        assert max_err(lse_loc[:, sl], rll) <= LSE_TOL, r
        assert max_err(o_peer[sl], rp) <= OUT_TOL[dtype], r
        assert max_err(lse_peer[:, sl], rpl) <= LSE_TOL, r
        assert max_err(out[sl], rm) <= OUT_TOL[dtype], r
        qs += L
        ps += P


def test_varlen_offsets_and_unaligned_starts(dev):
    """Causal offsets != 0 and paged segments starting mid-block."""
    h, hkv, d, bs = 8, 2, 128, 16
    lens = [100, 37, 200]
    peers = [5, 0, 77]   # local segment starts at token P (not block aligned)
    offs = [0, 20, 130]
    cache, bt, q, _ = _build(dev, "v031", lens, peers, h, hkv, d, torch.bfloat16, bs, seed=42)
    cd, btd, qd = cache.to(dev), bt.to(dev), q.to(dev)
    pc = PagedCache.from_tensor(cd)
    ent, qs = [], 0
    kv_lens = [L + o for L, o in zip(lens, offs)]  # keys visible up to offset+row
    # widen the cache view: segment length may exceed q rows when offset > 0
    for r, (L, P, o) in enumerate(zip(lens, peers, offs)):
        kl = min(kv_lens[r], bt.shape[1] * bs - P)
        ent.append(make_entry(qs, L, segment_paged(pc, btd[r], P, kl), o))
        qs += L
    o_, lse_ = varlen_attn_with_lse(qd, ent, True, hkv, scale_for(d))
    torch.cuda.synchronize()
    qs = 0
    for r, (L, P, o) in enumerate(zip(lens, peers, offs)):
        e = ent[r]
        kl, vl = orc.gather_paged(cache.float(), bt[r], P, e.kv.len, "v031")
        ro, rl = orc.attn_with_lse(q[qs:qs + L].float(), kl, vl, scale_for(d), o)
        assert max_err(o_[qs:qs + L], ro) <= OUT_TOL[torch.bfloat16]
        assert max_err(lse_[:, qs:qs + L], rl) <= LSE_TOL
        qs += L


@pytest.mark.parametrize("causal", [True, False])
def test_varlen_paged_cache_past_4gib_nan_outside_segments(dev, causal):
    """Blocks at byte offsets past 4 GiB, segment starts off the 64-key tile
    grid (the kernel aligns tiles down and zero-loads the lead), ragged ends;
    every cache slot outside the segments holds NaN, so reading any of them
    would show in the result."""
    h, hkv, d, bs = 28, 4, 128, 16
    blk_bytes = hkv * bs * 2 * d * 2
    nb = 4_600_000_000 // blk_bytes + 1  # 4.6 GB [nb, 4, 16, 256] bf16 cache
    cache = torch.full((nb, hkv, bs, 2 * d), float("nan"), dtype=torch.bfloat16, device=dev)
    gen = torch.Generator().manual_seed(77)
    reqs = [(37, 300), (0, 129), (64, 1), (15, 700), (100, 33)]  # (segment start, length)
    rows, qs_list, ks, vs = [], [], [], []
    next_hi = nb - 1  # allocate blocks downward from the top of the cache
    for start, ln in reqs:
        nblk = -(-(start + ln) // bs)
        ids = list(range(next_hi - nblk + 1, next_hi + 1))[::-1]
        next_hi -= nblk
        rows.append(ids)
        k = randn(gen, (ln, hkv, d), torch.bfloat16)
        v = randn(gen, (ln, hkv, d), torch.bfloat16)
        for j in range(ln):  # only the segment's slots get data
            pos = start + j
            cache[ids[pos // bs], :, pos % bs, :d] = k[j].to(dev)
            cache[ids[pos // bs], :, pos % bs, d:] = v[j].to(dev)
        ks.append(k)
        vs.append(v)
    assert min(min(r) for r in rows) * blk_bytes > (1 << 32)
    maxb = max(len(r) for r in rows)
    bt = torch.zeros(len(reqs), maxb, dtype=torch.int32)
    for r, ids in enumerate(rows):
        bt[r, :len(ids)] = torch.tensor(ids, dtype=torch.int32)
    btd = bt.to(dev)
    pc = PagedCache.from_tensor(cache)
    q = randn(gen, (sum(ln for _, ln in reqs), h, d), torch.bfloat16)
    qd = q.to(dev)
    ents, qs = [], 0
    for r, (start, ln) in enumerate(reqs):
        ents.append(make_entry(qs, ln, segment_paged(pc, btd[r], start, ln), 0))
        qs += ln
    scale = scale_for(d)
    out, lse = varlen_attn_with_lse(qd, ents, causal, hkv, scale)
    torch.cuda.synchronize()
    assert not torch.isnan(out).any() and not torch.isnan(lse).any()
    qs = 0
    for r, (start, ln) in enumerate(reqs):
        ro, rl = orc.attn_with_lse(q[qs:qs + ln].float(), ks[r].float(), vs[r].float(), scale,
                                   0 if causal else None)
        sl = slice(qs, qs + ln)
        assert max_err(out[sl], ro) <= OUT_TOL[torch.bfloat16], r
        assert max_err(lse[:, sl], rl) <= LSE_TOL, r
        qs += ln
    del cache


@pytest.mark.parametrize("bs", [1, 4, 8])
@pytest.mark.parametrize("layout", ["v031", "v023"])
@pytest.mark.parametrize("causal", [True, False])
def test_varlen_paged_small_blocks(dev, bs, layout, causal):
    """Caches with blocks shorter than 16 tokens (the reference's gather takes
    any block size, ring_backend.py:617-624): the launch gathers the paged
    segments into one contiguous buffer on the device and attends over it.
    Segments start mid-block; one entry is empty; the run is repeated after
    the cache changes, so the gather reads the cache at run time."""
    from hcp_vllm_plugin_amd.varlen import VarlenLaunch

    h, hkv, d, dtype = 14, 2, 128, torch.bfloat16
    lens = [130, 1, 0, 77]
    peers = [5, 16, 3, 41]  # local segment starts at token P of the request's frame
    offs = [0, 0, 0, 20] if causal else [0, 0, 0, 0]
    cache, bt, q, _ = _build(dev, layout, [L + o for L, o in zip(lens, offs)], peers, h, hkv,
                             d, dtype, bs, seed=90 + bs)
    cd, btd, qd = cache.to(dev), bt.to(dev), q[:sum(lens)].to(dev)
    pc = PagedCache.from_tensor(cd)
    ent, qs = [], 0
    for r, (L, P, o) in enumerate(zip(lens, peers, offs)):
        ent.append(make_entry(qs, L, segment_paged(pc, btd[r], P, L + o), o))
        qs += L
    launch = VarlenLaunch(ent, causal, True, dev)
    scale = scale_for(d)
    for rep in range(2):
        if rep == 1:  # new cache contents, same addresses: the next run sees them
            cd.copy_(torch.randn(cd.shape, generator=torch.Generator(device=dev).manual_seed(5),
                                 device=dev).to(dtype))
            cache = cd.cpu()
        o_ = torch.zeros_like(qd)
        lse_ = torch.full((h, qd.shape[0]), float("-inf"), device=dev)
        launch.run(qd, o_, lse_, hkv, scale)
        torch.cuda.synchronize()
        qs = 0
        for r, (L, P, o) in enumerate(zip(lens, peers, offs)):
            kl, vl = orc.gather_paged(cache.float(), bt[r], P, L + o, layout)
            ro, rl = orc.attn_with_lse(q[qs:qs + L].float(), kl, vl, scale,
                                       o if causal else None)
            assert max_err(o_[qs:qs + L], ro) <= OUT_TOL[dtype], (rep, r)
            assert max_err(lse_[:, qs:qs + L], rl) <= LSE_TOL, (rep, r)
            qs += L


@pytest.mark.parametrize("bs", [1, 8, 32])
def test_gather_paged_kv_bit_exact(dev, bs):
    """hcp_gather_paged_kv == the oracle's gather (ring_backend.py:617-624)
    bit for bit, both layouts' strides through one descriptor, head_dim 72 (a
    row that is not a power of two of 16-byte chunks)."""
    import numpy as np

    from hcp_vllm_plugin_amd import _lib
    from hcp_vllm_plugin_amd.varlen import ENTRY_DTYPE, _upload

    for layout in ("v031", "v023"):
        h, hkv, d, dtype = 4, 2, 72, torch.float16
        lens, peers = [50, 0, 3, 200], [7, 0, 31, 16]
        cache, bt, _, _ = _build(dev, layout, lens, peers, h, hkv, d, dtype, bs, seed=bs)
        cd, btd = cache.to(dev), bt.to(dev)
        pc = PagedCache.from_tensor(cd)
        ent = [make_entry(0, 1, segment_paged(pc, btd[r], P, L), 0)
               for r, (L, P) in enumerate(zip(lens, peers))]
        arr = np.concatenate([np.frombuffer(e, dtype=ENTRY_DTYPE) for e in ent])
        starts = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
        keep, (ep, sp) = _upload([arr, starts], dev)
        k = torch.zeros(sum(lens), hkv, d, dtype=dtype, device=dev)
        v = torch.zeros_like(k)
        rc = _lib.lib().hcp_gather_paged_kv(ep, len(ent), sp, max(lens), hkv, d,
                                           _lib.dtype_code(dtype), k.data_ptr(), v.data_ptr(),
                                           _lib.stream_ptr(dev))
        assert rc == 0, _lib.lib().hcp_last_error()
        torch.cuda.synchronize()
        for r, (L, P) in enumerate(zip(lens, peers)):
            kr, vr = orc.gather_paged(cache, bt[r], P, L, layout)
            s = int(starts[r])
            assert torch.equal(k[s:s + L].cpu(), kr.to(dtype)), (layout, r)
            assert torch.equal(v[s:s + L].cpu(), vr.to(dtype)), (layout, r)


def test_varlen_small_blocks_two_streams(dev):
    """A gather-mode launch (block size 8) run on the current stream and on a
    side stream: each stream gets its own contiguous K/V buffer, so runs in
    flight on the two never share one; both results equal the oracle's."""
    from hcp_vllm_plugin_amd.varlen import VarlenLaunch

    h, hkv, d, dtype, bs = 14, 2, 128, torch.bfloat16, 8
    lens, peers = [200, 64], [9, 0]
    cache, bt, q, _ = _build(dev, "v031", lens, peers, h, hkv, d, dtype, bs, seed=77)
    cd, btd, qd = cache.to(dev), bt.to(dev), q.to(dev)
    pc = PagedCache.from_tensor(cd)
    ent, qs = [], 0
    for r, (L, P) in enumerate(zip(lens, peers)):
        ent.append(make_entry(qs, L, segment_paged(pc, btd[r], P, L), 0))
        qs += L
    launch = VarlenLaunch(ent, True, True, dev)
    scale = scale_for(d)
    outs = []
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    for st in (torch.cuda.current_stream(dev), side):
        with torch.cuda.stream(st):
            o_ = torch.zeros_like(qd)
            lse_ = torch.full((h, qd.shape[0]), float("-inf"), device=dev)
            launch.run(qd, o_, lse_, hkv, scale)
            outs.append((o_, lse_))
    torch.cuda.synchronize()
    assert len(launch._gather["bufs"]) == 2
    for o_, lse_ in outs:
        qs = 0
        for r, (L, P) in enumerate(zip(lens, peers)):
            kl, vl = orc.gather_paged(cache.float(), bt[r], P, L, "v031")
            ro, rl = orc.attn_with_lse(q[qs:qs + L].float(), kl, vl, scale, 0)
            assert max_err(o_[qs:qs + L], ro) <= OUT_TOL[dtype], r
            assert max_err(lse_[:, qs:qs + L], rl) <= LSE_TOL, r
            qs += L
