"""GPU parity at the benchmark's full sizes.

The whole output of the full-size launches is compared with the oracle: the
7B 8k + 8k ring step (bf16 and fp16), every request and row of the
16-request varlen batch, and all 64 sequences of the split-KV decode.  The
oracle runs on the host one KV-head group and one block of query rows at a
time (rows are independent; a causal block only takes the keys it can see),
which bounds its fp32 score buffers to about 1 GB.  The 70B 64k + 64k layer
(eight 8192-query chunks; the peer pass alone is 17.6 TFLOP per chunk) is
too large for the host oracle whole: every chunk is checked on sampled rows
at its start, middle and end, and its whole output against a
size-independent identity -- the ring step (peer pass, then the local pass
merging it, ring_backend.py:820-831) equals one causal pass over the
concatenated keys [peer; local] with the queries at positions len(peer)+i.
Inputs are drawn on the device from a seeded generator (the bench's shapes;
N(0,1), K outlier channels x8).
"""

import pytest
import torch

from hcp_vllm_plugin_amd import ring_attn_with_lse
from hcp_vllm_plugin_amd.ring_attn import ring_attn_merged
from hcp_vllm_plugin_amd.varlen import PagedCache, decode_attn, segment_contiguous, segment_paged
from oracle import ring_oracle as orc
from tests._util import LSE_TOL, OUT_TOL, max_err, scale_for

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


def _draw(g, shape, dev, outlier_ch=None, dtype=BF16):
    x = torch.randn(*shape, generator=g, device=dev)
    if outlier_ch is not None:
        x[..., outlier_ch] *= 8.0
    return x.to(dtype)


def _oracle_ring(q, kl, vl, kp, vp, scale, q0, hkv, row_block=2048):
    """The oracle's ring step for every row: the local pass causal at offset
    ``q0`` over kl/vl, merged with the peer pass over kp/vp as prefix
    (``merge_pair``, ring_backend.py:820-831), fp32 on the host, one KV-head
    group and ``row_block`` query rows at a time.  q ``[n, h, d]``, k/v
    ``[tk, hkv, d]`` on any device.  Returns (out ``[n, h, d]``, lse
    ``[h, n]``) float32 on the host."""
    n, h, d = q.shape
    g = h // hkv
    out = torch.empty(n, h, d)
    lse = torch.empty(h, n)
    for j in range(hkv):
        hs, ks = slice(j * g, (j + 1) * g), slice(j, j + 1)
        kl_j, vl_j = kl[:, ks].float().cpu(), vl[:, ks].float().cpu()
        kp_j, vp_j = kp[:, ks].float().cpu(), vp[:, ks].float().cpu()
        for r0 in range(0, n, row_block):
            r1 = min(n, r0 + row_block)
            qb = q[r0:r1, hs].float().cpu()
            vis = max(0, min(kl_j.shape[0], q0 + r1))  # keys some row of the block sees
            o_l, l_l = orc.attn_with_lse(qb, kl_j[:vis], vl_j[:vis], scale, q0 + r0)
            o_p, l_p = orc.attn_with_lse(qb, kp_j, vp_j, scale, None)
            o, lo = orc.merge_pair(o_p, l_p, o_l, l_l)
            out[r0:r1, hs] = o
            lse[hs, r0:r1] = lo
    return out, lse


def _ring_step(q, kl, vl, kp, vp, scale, q0):
    """The ring step as the backend runs it: the peer pass, then the local
    pass merging it in its epilogue."""
    h, n = q.shape[1], q.shape[0]
    o_peer, lse_peer = ring_attn_with_lse(q, kp, vp, scale, None)
    lse = torch.empty(h, n, dtype=torch.float32, device=q.device)
    out = ring_attn_merged(q, kl, vl, scale, q0, o_peer, lse_peer, output_lse=lse)
    return out, lse


@pytest.mark.parametrize("dtype", [BF16, torch.float16])
def test_ring_prefill_step_full_size_every_row(dev, dtype):
    """Qwen2.5-7B shape, 8192 local causal (frame offset 0) + 8192 peer keys:
    every row of out and LSE against the oracle's ring step (bf16 gate 1.5e-2,
    fp16 gate 2e-3 on out; 1e-3 on LSE); the one-pass identity as an extra
    check of the whole output."""
    h, hkv, n, d = 28, 4, 8192, 128
    seed = 28 + n if dtype == BF16 else 16
    g = torch.Generator(device=dev).manual_seed(seed)
    ch = torch.randperm(d, generator=torch.Generator().manual_seed(seed))[:4]
    q = _draw(g, (n, h, d), dev, dtype=dtype)
    kl, vl = _draw(g, (n, hkv, d), dev, ch, dtype), _draw(g, (n, hkv, d), dev, dtype=dtype)
    kp, vp = _draw(g, (n, hkv, d), dev, ch, dtype), _draw(g, (n, hkv, d), dev, dtype=dtype)
    scale = scale_for(d)
    out, lse = _ring_step(q, kl, vl, kp, vp, scale, 0)
    o1, l1 = ring_attn_with_lse(q, torch.cat([kp, kl]), torch.cat([vp, vl]), scale, n)
    torch.cuda.synchronize()
    assert out.dtype == dtype and torch.isfinite(out).all() and torch.isfinite(lse).all()
    ro, rl = _oracle_ring(q, kl, vl, kp, vp, scale, 0, hkv)
    assert max_err(out, ro) <= OUT_TOL[dtype], max_err(out, ro)
    assert max_err(lse, rl) <= LSE_TOL, max_err(lse, rl)
    # both sides are within the tolerance of the exact result, so they agree
    # to twice it: two roundings of one value in [2, 4) can differ by an ulp
    assert max_err(out, o1) <= 2 * OUT_TOL[dtype] and max_err(lse, l1) <= 2 * LSE_TOL


@pytest.mark.parametrize("chunk", range(8))
def test_ring_prefill_70b_chunk(dev, chunk):
    """Llama-3-70B shape (64 / 8 heads), chunk ``chunk`` of the eight
    8192-query chunks of a 65536-token prompt: local keys [0, 8192(c+1))
    causal at offset 8192c, and all 65536 peer keys.  Rows at the chunk's
    start, middle and end against the oracle; the whole output against one
    causal pass over [peer; local]."""
    h, hkv, d, n_q, n_peer = 64, 8, 128, 8192, 65536
    q0 = 8192 * chunk
    n_loc = q0 + n_q
    g = torch.Generator(device=dev).manual_seed(1000 + chunk)
    ch = torch.randperm(d, generator=torch.Generator().manual_seed(h))[:8]
    q = _draw(g, (n_q, h, d), dev)
    kl, vl = _draw(g, (n_loc, hkv, d), dev, ch), _draw(g, (n_loc, hkv, d), dev)
    kp, vp = _draw(g, (n_peer, hkv, d), dev, ch), _draw(g, (n_peer, hkv, d), dev)
    scale = scale_for(d)
    out, lse = _ring_step(q, kl, vl, kp, vp, scale, q0)
    kk, vv = torch.cat([kp, kl]), torch.cat([vp, vl])
    del kp, vp, kl, vl
    o1, l1 = ring_attn_with_lse(q, kk, vv, scale, n_peer + q0)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all() and torch.isfinite(lse).all()
    assert max_err(out, o1) <= 2 * OUT_TOL[BF16], max_err(out, o1)
    assert max_err(lse, l1) <= 2 * LSE_TOL, max_err(lse, l1)
    del o1, l1
    kc, vc = kk.float().cpu(), vv.float().cpu()
    for r0 in (0, 4096 + 16 * chunk, n_q - 16):
        ro, rl = orc.attn_with_lse(q[r0:r0 + 16].float().cpu(), kc, vc, scale, n_peer + q0 + r0)
        assert max_err(out[r0:r0 + 16], ro) <= OUT_TOL[BF16], (r0, max_err(out[r0:r0 + 16], ro))
        assert max_err(lse[:, r0:r0 + 16], rl) <= LSE_TOL, r0


@pytest.mark.parametrize("peer_layout", ["head_major", "token_major"])
def test_split_kv_decode_full_size(dev, peer_layout):
    """64 sequences, each 32768 contiguous peer keys + U[512, 2048] local keys
    in a paged [nb, 4, 16, 256] cache under a random block table; every
    sequence is checked against the oracle (local causal at len - 1, peer,
    merged).  The peers are stored head-major ([Hkv, n, D] behind the
    [n, Hkv, D] view, as stage_peer_kv stores staged chunks: 64-bit head
    offsets of up to 3.7 GB) or token-major (as loaded)."""
    from hcp_vllm_plugin_amd.varlen import head_major

    h, hkv, d, bs, s, n_peer = 28, 4, 128, 16, 64, 32768
    gc = torch.Generator().manual_seed(3)
    loc = torch.randint(512, 2049, (s,), generator=gc).tolist()
    blocks = [-(-n // bs) for n in loc]
    nb = sum(blocks) + 4
    perm = torch.randperm(nb, generator=gc).to(torch.int32)
    bt = torch.zeros(s, max(blocks), dtype=torch.int32)
    o = 0
    for r, n in enumerate(blocks):
        bt[r, :n] = perm[o:o + n]
        o += n
    g = torch.Generator(device=dev).manual_seed(3)
    cache = _draw(g, (nb, hkv, bs, 2 * d), dev)
    q = _draw(g, (s, h, d), dev)
    kp, vp = _draw(g, (s * n_peer, hkv, d), dev), _draw(g, (s * n_peer, hkv, d), dev)
    if peer_layout == "head_major":
        kp, vp = head_major(kp), head_major(vp)
        assert kp.stride() == (d, s * n_peer * d, 1)
    btd = bt.to(dev)
    pc = PagedCache.from_tensor(cache)
    segs = [[segment_contiguous(kp, vp, r * n_peer, n_peer), segment_paged(pc, btd[r], 0, loc[r])]
            for r in range(s)]
    scale = scale_for(d)
    out, lse = decode_attn(q, segs, hkv, scale, with_lse=True)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all() and torch.isfinite(lse).all()
    cache_c = cache.float().cpu()
    for r in range(s):
        kl, vl = orc.gather_paged(cache_c, bt[r], 0, loc[r], "v031")
        sl = slice(r * n_peer, (r + 1) * n_peer)
        ro, rl = _oracle_ring(q[r:r + 1], kl, vl, kp[sl], vp[sl], scale, loc[r] - 1, hkv)
        assert max_err(out[r:r + 1], ro) <= OUT_TOL[BF16], (r, max_err(out[r:r + 1], ro))
        assert max_err(lse[:, r:r + 1], rl) <= LSE_TOL, r


def test_varlen_batch_full_size(dev):
    """16 requests: local U[512, 4096] queries causal over their own keys in a
    paged [nb, 4, 16, 256] cache (the block-table row also covers the
    request's 16*U[64, 1024] prefix blocks, which the local pass does not
    read), peer = the prefix keys packed contiguously.  The peer launch, then
    the local launch merging it; every row of every request against the
    oracle."""
    from hcp_vllm_plugin_amd.varlen import VarlenLaunch, make_entry

    h, hkv, d, bs, nreq = 28, 4, 128, 16, 16
    gc = torch.Generator().manual_seed(2)
    loc = torch.randint(512, 4097, (nreq,), generator=gc).tolist()
    pre = (16 * torch.randint(64, 1025, (nreq,), generator=gc)).tolist()
    blocks = [-(-(p + n) // bs) for p, n in zip(pre, loc)]
    nb = sum(blocks) + 8
    perm = torch.randperm(nb, generator=gc).to(torch.int32)
    bt = torch.zeros(nreq, max(blocks), dtype=torch.int32)
    o = 0
    for r, n in enumerate(blocks):
        bt[r, :n] = perm[o:o + n]
        o += n
    g = torch.Generator(device=dev).manual_seed(2)
    cache = _draw(g, (nb, hkv, bs, 2 * d), dev)
    q = _draw(g, (sum(loc), h, d), dev)
    pk, pv = _draw(g, (sum(pre), hkv, d), dev), _draw(g, (sum(pre), hkv, d), dev)
    btd = bt.to(dev)
    pc = PagedCache.from_tensor(cache)
    loc_e, peer_e, qs, ps = [], [], [0], [0]
    for r in range(nreq):
        loc_e.append(make_entry(qs[-1], loc[r], segment_paged(pc, btd[r], pre[r], loc[r]), 0))
        peer_e.append(make_entry(qs[-1], loc[r], segment_contiguous(pk, pv, ps[-1], pre[r])))
        qs.append(qs[-1] + loc[r])
        ps.append(ps[-1] + pre[r])
    scale = scale_for(d)
    o_peer = torch.empty_like(q)
    lse_peer = torch.empty(h, qs[-1], dtype=torch.float32, device=dev)
    VarlenLaunch(peer_e, False, False, dev).run(q, o_peer, lse_peer, hkv, scale)
    out = torch.empty_like(q)
    lse = torch.empty(h, qs[-1], dtype=torch.float32, device=dev)
    VarlenLaunch(loc_e, True, True, dev).run(q, out, lse, hkv, scale, acc=(o_peer, lse_peer))
    torch.cuda.synchronize()
    assert torch.isfinite(out).all() and torch.isfinite(lse).all()
    cache_c = cache.float().cpu()
    for r in range(nreq):
        kl, vl = orc.gather_paged(cache_c, bt[r], pre[r], loc[r], "v031")
        rows = slice(qs[r], qs[r + 1])
        ro, rl = _oracle_ring(q[rows], kl, vl, pk[ps[r]:ps[r + 1]], pv[ps[r]:ps[r + 1]],
                              scale, 0, hkv)
        assert max_err(out[rows], ro) <= OUT_TOL[BF16], (r, max_err(out[rows], ro))
        assert max_err(lse[:, rows], rl) <= LSE_TOL, r
