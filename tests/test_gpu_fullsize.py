"""GPU parity at the benchmark's full sizes.

Rows of attention are independent, so sampled query rows (or sequences) of a
full-size launch are checked exactly against the oracle run on those rows
alone, and the whole output against a size-independent identity: the ring
step (peer pass, then the local pass merging it, ring_backend.py:820-831)
equals one causal pass over the concatenated keys [peer; local] with the
queries at positions len(peer)+i.  Inputs are drawn on the device from a
seeded generator (the bench's shapes; N(0,1), K outlier channels x8).
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


def _draw(g, shape, dev, outlier_ch=None):
    x = torch.randn(*shape, generator=g, device=dev)
    if outlier_ch is not None:
        x[..., outlier_ch] *= 8.0
    return x.to(BF16)


@pytest.mark.parametrize("h,hkv,n_q,n_loc,n_peer,q0,n_out,blocks", [
    # Qwen2.5-7B shape: 8192 local causal (frame offset 0) + 8192 peer keys
    (28, 4, 8192, 8192, 8192, 0, 4, (0, 2047, 5000, 8176)),
    # Llama-3-70B shape, chunks 0, 3 and 7 of the eight 8192-query chunks of
    # a 65536-token prompt: chunk c sees local keys [0, 8192(c+1)) causal at
    # offset 8192c, and all 65536 peer keys
    (64, 8, 8192, 8192, 65536, 0, 8, (0, 8176)),
    (64, 8, 8192, 32768, 65536, 24576, 8, (0, 4000, 8176)),
    (64, 8, 8192, 65536, 65536, 57344, 8, (0, 8176)),
])
def test_ring_prefill_step_full_size(dev, h, hkv, n_q, n_loc, n_peer, q0, n_out, blocks):
    d = 128
    g = torch.Generator(device=dev).manual_seed(h + n_loc)
    ch = torch.randperm(d, generator=torch.Generator().manual_seed(h))[:n_out]
    q = _draw(g, (n_q, h, d), dev)
    kl, vl = _draw(g, (n_loc, hkv, d), dev, ch), _draw(g, (n_loc, hkv, d), dev)
    kp, vp = _draw(g, (n_peer, hkv, d), dev, ch), _draw(g, (n_peer, hkv, d), dev)
    scale = scale_for(d)
    o_peer, lse_peer = ring_attn_with_lse(q, kp, vp, scale, None)
    lse = torch.empty(h, n_q, dtype=torch.float32, device=dev)
    out = ring_attn_merged(q, kl, vl, scale, q0, o_peer, lse_peer, output_lse=lse)
    del o_peer, lse_peer
    kk, vv = torch.cat([kp, kl]), torch.cat([vp, vl])
    del kp, vp, kl, vl
    o1, l1 = ring_attn_with_lse(q, kk, vv, scale, n_peer + q0)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all() and torch.isfinite(lse).all()
    # both sides are within the tolerance of the exact result (checked on the
    # sampled rows below), so they agree to twice it: two bf16 roundings of
    # one value in [2, 4) can differ by 2^-6
    assert max_err(out, o1) <= 2 * OUT_TOL[BF16], max_err(out, o1)
    assert max_err(lse, l1) <= 2 * LSE_TOL, max_err(lse, l1)
    del o1, l1
    kc, vc = kk.float().cpu(), vv.float().cpu()
    for r0 in blocks:
        ro, rl = orc.attn_with_lse(q[r0:r0 + 16].float().cpu(), kc, vc, scale, n_peer + q0 + r0)
        assert max_err(out[r0:r0 + 16], ro) <= OUT_TOL[BF16], (r0, max_err(out[r0:r0 + 16], ro))
        assert max_err(lse[:, r0:r0 + 16], rl) <= LSE_TOL, r0


def test_ring_prefill_step_full_size_fp16(dev):
    """The 7B 8k + 8k ring step in fp16 (the reference's probe dtype; gate
    2e-3 on out): sampled rows against the oracle, and the whole output
    against one causal pass over [peer; local]."""
    h, hkv, d, n = 28, 4, 128, 8192
    g = torch.Generator(device=dev).manual_seed(16)
    ch = torch.randperm(d, generator=torch.Generator().manual_seed(16))[:4]

    def draw(shape, outlier=False):
        x = torch.randn(*shape, generator=g, device=dev)
        if outlier:
            x[..., ch] *= 8.0
        return x.to(torch.float16)

    q = draw((n, h, d))
    kl, vl, kp, vp = draw((n, hkv, d), True), draw((n, hkv, d)), draw((n, hkv, d), True), draw((n, hkv, d))
    scale = scale_for(d)
    o_peer, lse_peer = ring_attn_with_lse(q, kp, vp, scale, None)
    lse = torch.empty(h, n, dtype=torch.float32, device=dev)
    out = ring_attn_merged(q, kl, vl, scale, 0, o_peer, lse_peer, output_lse=lse)
    kk, vv = torch.cat([kp, kl]), torch.cat([vp, vl])
    o1, l1 = ring_attn_with_lse(q, kk, vv, scale, n)
    torch.cuda.synchronize()
    assert out.dtype == torch.float16 and torch.isfinite(out).all()
    assert max_err(out, o1) <= 2 * OUT_TOL[torch.float16], max_err(out, o1)
    assert max_err(lse, l1) <= 2 * LSE_TOL
    kc, vc = kk.float().cpu(), vv.float().cpu()
    for r0 in (0, 4100, 8176):
        ro, rl = orc.attn_with_lse(q[r0:r0 + 16].float().cpu(), kc, vc, scale, n + r0)
        assert max_err(out[r0:r0 + 16], ro) <= OUT_TOL[torch.float16], (r0, max_err(out[r0:r0 + 16], ro))
        assert max_err(lse[:, r0:r0 + 16], rl) <= LSE_TOL, r0


@pytest.mark.parametrize("peer_layout", ["head_major", "token_major"])
def test_split_kv_decode_full_size(dev, peer_layout):
    """64 sequences, each 32768 contiguous peer keys + U[512, 2048] local keys
    in a paged [nb, 4, 16, 256] cache under a random block table; every
    sequence's output goes through the full launch, eight are checked.  The
    peers are stored head-major ([Hkv, n, D] behind the [n, Hkv, D] view, as
    stage_peer_kv stores staged chunks: 64-bit head offsets of up to 3.7 GB)
    or token-major (as loaded)."""
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
    for r in range(0, s, 9):
        kl, vl = orc.gather_paged(cache_c, bt[r], 0, loc[r], "v031")
        qr = q[r:r + 1].float().cpu()
        ro_l, rl_l = orc.attn_with_lse(qr, kl, vl, scale, loc[r] - 1)
        sl = slice(r * n_peer, (r + 1) * n_peer)
        ro_p, rl_p = orc.attn_with_lse(qr, kp[sl].float().cpu(), vp[sl].float().cpu(), scale, None)
        ro, rl = orc.merge_pair(ro_l, rl_l, ro_p, rl_p)
        assert max_err(out[r:r + 1], ro) <= OUT_TOL[BF16], (r, max_err(out[r:r + 1], ro))
        assert max_err(lse[:, r:r + 1], rl) <= LSE_TOL, r


def test_varlen_batch_full_size(dev):
    """16 requests: local U[512, 4096] queries causal over their own keys in a
    paged [nb, 4, 16, 256] cache (the block-table row also covers the
    request's 16*U[64, 1024] prefix blocks, which the local pass does not
    read), peer = the prefix keys packed contiguously.  The peer launch, then
    the local launch merging it; four requests checked at both ends."""
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
    for r in (0, 5, 10, 15):
        kl, vl = orc.gather_paged(cache_c, bt[r], pre[r], loc[r], "v031")
        kp_r = pk[ps[r]:ps[r + 1]].float().cpu()
        vp_r = pv[ps[r]:ps[r + 1]].float().cpu()
        for i0 in (0, loc[r] - 16):
            rows = slice(qs[r] + i0, qs[r] + i0 + 16)
            qr = q[rows].float().cpu()
            ro_l, rl_l = orc.attn_with_lse(qr, kl, vl, scale, i0)
            ro_p, rl_p = orc.attn_with_lse(qr, kp_r, vp_r, scale, None)
            ro, rl = orc.merge_pair(ro_p, rl_p, ro_l, rl_l)
            assert max_err(out[rows], ro) <= OUT_TOL[BF16], (r, i0, max_err(out[rows], ro))
            assert max_err(lse[:, rows], rl) <= LSE_TOL, (r, i0)
