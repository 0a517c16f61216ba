"""GPU parity: an attention pass and the LSE merge after it in one launch
(hcp_attn_fwd_lse_merge via ring_attn_merged, hcp_attn_fwd_varlen_merge via
VarlenLaunch.run(acc=...)).

The fused result must equal the two-step path -- ring_attn_with_lse /
VarlenLaunch, then merge_attn_states(out, o_peer, lse_peer, o_loc, lse_loc)
as HcpRingAttentionImpl.forward merges (ring_backend.py:349-354,820-831) --
bit for bit, output and merged LSE, for the accumulator on either side of the
merge, and the merged step must match the oracle's float32 ring
decomposition within the output tolerances.
"""

import pytest
import torch

from hcp_vllm_plugin_amd import merge_attn_states, ring_attn_merged, ring_attn_with_lse
from hcp_vllm_plugin_amd.varlen import (
    PagedCache,
    VarlenLaunch,
    make_entry,
    segment_contiguous,
    segment_paged,
)
from oracle import ring_oracle as orc
from tests._util import LSE_TOL, OUT_TOL, max_err, outlier_k, randn, scale_for

pytestmark = pytest.mark.gpu

# (tq, local keys, peer keys, local causal offset, window, head_dim, dtype)
CASES = [
    (1000, 1000, 3000, 0, None, 128, torch.bfloat16),
    (513, 700, 2048, 187, None, 128, torch.float16),
    (300, 900, 64, 600, 128, 128, torch.bfloat16),
    (129, 129, 1, 0, None, 64, torch.float16),
    (257, 300, 1500, 43, 7, 64, torch.bfloat16),
    (64, 64, 0, 0, None, 128, torch.bfloat16),     # empty peer: prefix LSE -inf everywhere
    (100, 60, 500, -20, None, 128, torch.float16),  # first 20 rows see no local key
]


def _inputs(case, seed):
    tq, tl, tp, off, win, d, dt = case
    gen = torch.Generator().manual_seed(seed)
    h, hkv = 28, 4
    q = randn(gen, (tq, h, d), dt)
    kl = outlier_k(randn(gen, (tl, hkv, d), dt), gen).to(dt)
    vl = randn(gen, (tl, hkv, d), dt)
    kp = outlier_k(randn(gen, (tp, hkv, d), dt), gen).to(dt)
    vp = randn(gen, (tp, hkv, d), dt)
    return q, kl, vl, kp, vp


@pytest.mark.parametrize("ci", range(len(CASES)))
def test_merged_pass_equals_two_step(dev, ci):
    case = CASES[ci]
    tq, tl, tp, off, win, d, dt = case
    q, kl, vl, kp, vp = _inputs(case, 70 + ci)
    qd, kld, vld, kpd, vpd = (t.to(dev) for t in (q, kl, vl, kp, vp))
    sc = scale_for(d)
    o_p, l_p = ring_attn_with_lse(qd, kpd, vpd, sc, None)
    o_l, l_l = ring_attn_with_lse(qd, kld, vld, sc, off, win)
    ref = torch.empty_like(o_l)
    ref_lse = torch.empty_like(l_l)
    merge_attn_states(ref, o_p, l_p, o_l, l_l, ref_lse)
    # local pass last, the peer result as the prefix (the backend's order)
    got_lse = torch.empty_like(l_l)
    got = ring_attn_merged(qd, kld, vld, sc, off, o_p, l_p, True, win, output_lse=got_lse)
    # peer pass last, the local result as the suffix
    got2 = ring_attn_merged(qd, kpd, vpd, sc, None, o_l, l_l, False)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    assert torch.equal(got_lse, ref_lse)
    assert torch.equal(got2, ref)
    # and the merged step against the oracle's float32 ring decomposition:
    # both partial outputs are rounded to the dtype before the merge rounds
    # again (as in the reference), so rows attending to few keys (|out| up to
    # ~4 here) get half an ulp of their own magnitude on top of the gate
    rl, rll = orc.attn_with_lse(q.float(), kl.float(), vl.float(), sc, off, win)
    rp, rpl = orc.attn_with_lse(q.float(), kp.float(), vp.float(), sc, None)
    rm = orc.lse_merge(rl, rll, rp, rpl)
    rtol = {torch.float16: 2 ** -11, torch.bfloat16: 2 ** -8}[dt]
    torch.testing.assert_close(got.float().cpu(), rm, atol=OUT_TOL[dt], rtol=rtol)
    rml = torch.logaddexp(rll, rpl)
    assert max_err(got_lse, rml) <= LSE_TOL


def test_merged_inf_and_in_place(dev):
    """Accumulator rows of LSE -inf (weight 0, never read: NaN there must not
    leak) and +inf (counted as -inf), and out / lse aliasing the accumulator."""
    tq, d, dt = 300, 128, torch.bfloat16
    q, kl, vl, kp, vp = _inputs((tq, 400, 800, 100, None, d, dt), 91)
    qd, kld, vld, kpd, vpd = (t.to(dev) for t in (q, kl, vl, kp, vp))
    sc = scale_for(d)
    o_p, l_p = ring_attn_with_lse(qd, kpd, vpd, sc, None)
    l_p[:, :50] = float("-inf")
    o_p[:50] = float("nan")
    l_p[3, 60:70] = float("inf")
    o_p[60:70, 3] = float("nan")
    o_l, l_l = ring_attn_with_lse(qd, kld, vld, sc, 100)
    ref = torch.empty_like(o_l)
    ref_lse = torch.empty_like(l_l)
    merge_attn_states(ref, o_p, l_p, o_l, l_l, ref_lse)
    acc_o, acc_l = o_p.clone(), l_p.clone()
    got = ring_attn_merged(qd, kld, vld, sc, 100, acc_o, acc_l, True, output=acc_o,
                           output_lse=acc_l)
    torch.cuda.synchronize()
    assert got.data_ptr() == acc_o.data_ptr()
    assert not torch.isnan(got).any()
    assert torch.equal(got, ref)
    assert torch.equal(acc_l, ref_lse)


def _paged(dev, lens, peers, layout, dt, seed, h=28, hkv=4, d=128, bs=16):
    gen = torch.Generator().manual_seed(seed)
    blocks_per = [-(-(p + ln) // bs) for p, ln in zip(peers, lens)]
    nb = sum(blocks_per) + 3
    if layout == "v031":
        cache = randn(gen, (nb, hkv, bs, 2 * d), dt)
    else:
        cache = randn(gen, (nb, 2, bs, hkv, d), dt)
    perm = torch.randperm(nb, generator=gen).to(torch.int32)
    bt = torch.zeros(len(lens), max(blocks_per), dtype=torch.int32)
    o = 0
    for r, nbk in enumerate(blocks_per):
        bt[r, :nbk] = perm[o:o + nbk]
        o += nbk
    q = randn(gen, (sum(lens), h, d), dt)
    peer = randn(gen, (sum(peers), 2, hkv, d), dt)
    return cache.to(dev), bt.to(dev), q.to(dev), peer.to(dev)


@pytest.mark.parametrize("layout", ["v031", "v023"])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_varlen_merged_equals_two_step(dev, layout, dt):
    """The backend's prefill: peer launch, then the local paged causal launch
    merging the peer result (prefix) into the output; rows whose request has
    no peer get the local result."""
    lens = [300, 1, 129, 700, 64, 257]
    peers = [512, 48, 1024, 0, 16, 400]
    cache, bt, q, peer = _paged(dev, lens, peers, layout, dt, 97)
    pc = PagedCache.from_tensor(cache)
    pk, pv = peer[:, 0], peer[:, 1]
    loc_e, peer_e = [], []
    qs = ps = 0
    for r, (ln, pn) in enumerate(zip(lens, peers)):
        loc_e.append(make_entry(qs, ln, segment_paged(pc, bt[r], pn, ln), 0))
        if pn:
            peer_e.append(make_entry(qs, ln, segment_contiguous(pk, pv, ps, pn), 0))
        qs += ln
        ps += pn
    sc = scale_for(128)
    T = q.shape[0]
    o_p = torch.empty_like(q)
    l_p = torch.full((28, T), float("-inf"), device=dev)
    VarlenLaunch(peer_e, False, False, dev).run(q, o_p, l_p, 4, sc)
    o_l = torch.empty_like(q)
    l_l = torch.empty(28, T, device=dev)
    local = VarlenLaunch(loc_e, True, True, dev)
    local.run(q, o_l, l_l, 4, sc)
    ref = torch.empty_like(q)
    ref_lse = torch.empty_like(l_l)
    merge_attn_states(ref, o_p, l_p, o_l, l_l, ref_lse)
    got = torch.empty_like(q)
    got_lse = torch.empty_like(l_l)
    local.run(q, got, got_lse, 4, sc, acc=(o_p, l_p), acc_is_prefix=True)
    got_nolse = torch.empty_like(q)
    local.run(q, got_nolse, None, 4, sc, acc=(o_p, l_p))
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    assert torch.equal(got_lse, ref_lse)
    assert torch.equal(got_nolse, ref)
