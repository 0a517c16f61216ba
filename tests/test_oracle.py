"""Pins the CPU oracle (oracle/ring_oracle.py) without retyping its formulas.

Each check uses a different route to the same number: float64 loops over
(query, head) with an explicit max-shifted softmax, torch's SDPA with an
explicit boolean mask, torch.logsumexp, closed forms, and the reference's own
invariant that a KV split merged by LSE equals full attention
(validate_ring_triton_kernel.py:80-94).  Any dropped term, wrong sign, wrong
GQA index or transposed operand in the oracle fails at least one of them.
"""

import math

import numpy as np
import pytest
import torch

from oracle import ring_oracle as orc


def brute(q, k, v, scale, off, window=None):
    """float64 loops: out[i,h] = sum_j w_j v_j, lse = log sum_j exp(s_j)."""
    q = q.double().numpy()
    k = k.double().numpy()
    v = v.double().numpy()
    tq, h, d = q.shape
    tk, hkv = k.shape[0], k.shape[1]
    g = h // hkv
    out = np.zeros((tq, h, d))
    lse = np.full((h, tq), -np.inf)
    for i in range(tq):
        for hh in range(h):
            kh = hh // g
            vis = [j for j in range(tk) if off is None or
                   (j <= off + i and (window is None or j > off + i - window))]
            if not vis:
                continue
            s = np.array([scale * float(np.dot(q[i, hh], k[j, kh])) for j in vis])
            m = s.max()
            w = np.exp(s - m)
            out[i, hh] = (w[:, None] * v[vis, kh]).sum(0) / w.sum()
            lse[hh, i] = m + math.log(w.sum())
    return out, lse


def rnd(gen, *shape):
    return torch.randn(*shape, generator=gen)


CASES = [
    # (tq, tk, offset)
    (1, 1, 0),
    (5, 7, 2),
    (7, 7, 0),
    (3, 9, 6),
    (6, 4, 10),    # offset beyond Tk: every key visible
    (4, 6, -2),    # negative offset: first rows see nothing
    (5, 8, None),  # non-causal
]


@pytest.mark.parametrize("tq,tk,off", CASES)
@pytest.mark.parametrize("h,hkv", [(4, 2), (6, 3), (4, 4)])
def test_attn_vs_float64_brute(tq, tk, off, h, hkv):
    gen = torch.Generator().manual_seed(tq * 100 + tk + h)
    d = 16
    q, k, v = rnd(gen, tq, h, d), rnd(gen, tk, hkv, d), rnd(gen, tk, hkv, d)
    scale = 1 / math.sqrt(d)
    o, lse = orc.attn_with_lse(q, k, v, scale, off)
    ob, lb = brute(q, k, v, scale, off)
    np.testing.assert_allclose(o.numpy(), ob, atol=2e-6, rtol=1e-5)
    np.testing.assert_allclose(lse.numpy(), lb, atol=2e-6, rtol=1e-6)


def _sdpa_ref(q, k, v, scale, off):
    """torch SDPA with an explicit mask + torch.logsumexp (library routines)."""
    tq, h, d = q.shape
    tk, hkv = k.shape[0], k.shape[1]
    g = h // hkv
    kk = torch.stack([k[:, i // g] for i in range(h)], 1)  # explicit head map
    vv = torch.stack([v[:, i // g] for i in range(h)], 1)
    i = torch.arange(tq)[:, None]
    j = torch.arange(tk)[None, :]
    mask = torch.ones(tq, tk, dtype=torch.bool) if off is None else (j <= off + i)
    out = torch.nn.functional.scaled_dot_product_attention(
        q.transpose(0, 1).double(), kk.transpose(0, 1).double(), vv.transpose(0, 1).double(),
        attn_mask=mask, scale=scale,
    ).transpose(0, 1)
    s = torch.matmul(q.transpose(0, 1).double(), kk.permute(1, 2, 0).double()) * scale
    s = s.masked_fill(~mask, float("-inf"))
    lse = torch.logsumexp(s, -1)
    return out, lse


@pytest.mark.parametrize("off", [None, 0, 40, 200])
def test_attn_vs_sdpa(off):
    gen = torch.Generator().manual_seed(7)
    q, k, v = rnd(gen, 64, 28, 128), rnd(gen, 96, 4, 128), rnd(gen, 96, 4, 128)
    scale = 1 / math.sqrt(128)
    o, lse = orc.attn_with_lse(q, k, v, scale, off)
    ro, rl = _sdpa_ref(q, k, v, scale, off)
    torch.testing.assert_close(o.double(), ro, atol=2e-5, rtol=1e-4)
    torch.testing.assert_close(lse.double(), rl, atol=2e-5, rtol=1e-5)


def test_closed_form_single_key():
    gen = torch.Generator().manual_seed(1)
    q, k, v = rnd(gen, 5, 6, 32), rnd(gen, 1, 2, 32), rnd(gen, 1, 2, 32)
    scale = 0.3
    o, lse = orc.attn_with_lse(q, k, v, scale, None)
    for h in range(6):
        kh = h // 3
        torch.testing.assert_close(o[:, h], v[0, kh].expand(5, 32))
        torch.testing.assert_close(lse[h], scale * (q[:, h] @ k[0, kh]))


def test_closed_form_constant_keys():
    """All-zero keys: out = mean of visible V, lse = log(#visible)."""
    gen = torch.Generator().manual_seed(2)
    tq, tk, off = 6, 10, 3
    q, v = rnd(gen, tq, 4, 16), rnd(gen, tk, 2, 16)
    k = torch.zeros(tk, 2, 16)
    o, lse = orc.attn_with_lse(q, k, v, 0.25, off)
    for i in range(tq):
        n = min(tk, off + i + 1)
        for h in range(4):
            torch.testing.assert_close(o[i, h], v[:n, h // 2].mean(0), atol=1e-6, rtol=1e-6)
            assert abs(lse[h, i].item() - math.log(n)) < 1e-6


def test_causal_large_offset_equals_noncausal():
    gen = torch.Generator().manual_seed(3)
    q, k, v = rnd(gen, 9, 4, 16), rnd(gen, 13, 2, 16), rnd(gen, 13, 2, 16)
    a = orc.attn_with_lse(q, k, v, 0.2, 12)
    b = orc.attn_with_lse(q, k, v, 0.2, None)
    torch.testing.assert_close(a[0], b[0])
    torch.testing.assert_close(a[1], b[1])


def test_empty_segment_convention():
    q = torch.randn(3, 4, 16)
    k = torch.zeros(0, 2, 16)
    o, lse = orc.attn_with_lse(q, k, k, 0.1, None)
    assert torch.all(o == 0) and torch.all(torch.isneginf(lse))


@pytest.mark.parametrize("merge", ["lse_merge", "merge_pair"])
def test_split_merge_equals_full(merge):
    """validate_ring_triton_kernel.py:80-94: local causal + peer non-causal,
    merged, equals causal attention over the whole KV."""
    gen = torch.Generator().manual_seed(4)
    tk_full, split, tq = 96, 40, 24
    q, k, v = rnd(gen, tq, 6, 32), rnd(gen, tk_full, 2, 32), rnd(gen, tk_full, 2, 32)
    scale = 1 / math.sqrt(32)
    o_full, lse_full = brute(q, k, v, scale, tk_full - tq)
    o_loc, lse_loc = orc.attn_with_lse(q, k[split:], v[split:], scale, tk_full - tq - split)
    o_peer, lse_peer = orc.attn_with_lse(q, k[:split], v[:split], scale, None)
    if merge == "lse_merge":
        o_m = orc.lse_merge(o_loc, lse_loc, o_peer, lse_peer)
    else:
        o_m, lse_m = orc.merge_pair(o_loc, lse_loc, o_peer, lse_peer)
        np.testing.assert_allclose(lse_m.numpy(), lse_full, atol=3e-6)
    np.testing.assert_allclose(o_m.numpy(), o_full, atol=3e-6)


def test_merge_identities():
    gen = torch.Generator().manual_seed(5)
    o1, o2, o3 = rnd(gen, 7, 3, 8), rnd(gen, 7, 3, 8), rnd(gen, 7, 3, 8)
    l1, l2, l3 = rnd(gen, 3, 7) * 3, rnd(gen, 3, 7) * 3, rnd(gen, 3, 7) * 3
    ninf = torch.full_like(l1, float("-inf"))
    # -inf side carries no weight
    o, lse = orc.merge_pair(o1, l1, o2, ninf)
    torch.testing.assert_close(o, o1)
    torch.testing.assert_close(lse, l1)
    # commutative
    a = orc.merge_pair(o1, l1, o2, l2)
    b = orc.merge_pair(o2, l2, o1, l1)
    torch.testing.assert_close(a[0], b[0])
    torch.testing.assert_close(a[1], b[1])
    # associative: running merge equals one-shot softmax-weighted sum
    r = orc.merge_pair(*orc.merge_pair(o1, l1, o2, l2), o3, l3)
    w = torch.stack([l1, l2, l3]).double().softmax(0)  # [3, H, T]
    ref = sum(w[i].T[..., None] * o.double() for i, o in enumerate((o1, o2, o3)))
    torch.testing.assert_close(r[0].double(), ref, atol=1e-6, rtol=1e-6)
    ref_lse = torch.logsumexp(torch.stack([l1, l2, l3]).double(), 0)
    torch.testing.assert_close(r[1].double(), ref_lse, atol=1e-6, rtol=1e-6)
    # both empty: 0 / -inf
    o, lse = orc.merge_pair(o1, ninf, o2, ninf)
    assert torch.all(o == 0) and torch.all(torch.isneginf(lse))


def test_merge_attn_states_order_and_inf():
    """prefix/suffix order is symmetric; +inf reads as -inf (vLLM semantics)."""
    gen = torch.Generator().manual_seed(6)
    o1, o2 = rnd(gen, 5, 2, 8), rnd(gen, 5, 2, 8)
    l1, l2 = rnd(gen, 2, 5), rnd(gen, 2, 5)
    out = torch.empty(5, 2, 8)
    out_lse = torch.empty(2, 5)
    orc.merge_attn_states(out, o1, l1, o2, l2, out_lse)
    ref = orc.lse_merge(o2, l2, o1, l1)
    torch.testing.assert_close(out, ref)
    pinf = l1.clone()
    pinf[0, 0] = float("inf")
    orc.merge_attn_states(out, o1, pinf, o2, l2, out_lse)
    torch.testing.assert_close(out[0, 0], o2[0, 0])
    assert out_lse[0, 0] == l2[0, 0]


@pytest.mark.parametrize("layout", ["v023", "v031"])
def test_gather_paged(layout):
    gen = torch.Generator().manual_seed(8)
    nb, bs, hkv, d = 12, 4, 2, 8
    if layout == "v023":
        cache = rnd(gen, nb, 2, bs, hkv, d)
    else:
        cache = rnd(gen, nb, hkv, bs, 2 * d)
    row = torch.randperm(nb, generator=gen).to(torch.int32)
    start, length = 3, 17
    k, v = orc.gather_paged(cache, row, start, length, layout)
    for t in range(length):
        x = start + t
        b, o = int(row[x // bs]), x % bs
        for h in range(hkv):
            if layout == "v023":
                ek, ev = cache[b, 0, o, h], cache[b, 1, o, h]
            else:
                ek, ev = cache[b, h, o, :d], cache[b, h, o, d:]
            assert torch.equal(k[t, h], ek) and torch.equal(v[t, h], ev)


@pytest.mark.parametrize("layout", ["v023", "v031"])
def test_kv_cache_update_vs_elementwise_and_gather(layout):
    """kv_cache_update writes slot = block * bs + offset: checked element by
    element against explicit loops, padding (-1) slots left untouched, and
    read back through gather_paged (pinned above) along a block table."""
    gen = torch.Generator().manual_seed(9)
    nb, bs, hkv, d, n = 10, 4, 2, 8, 23
    shape = (nb, 2, bs, hkv, d) if layout == "v023" else (nb, hkv, bs, 2 * d)
    cache = rnd(gen, *shape)
    before = cache.clone()
    key, value = rnd(gen, n + 3, hkv, d), rnd(gen, n + 3, hkv, d)  # padded rows
    slots = torch.randperm(nb * bs, generator=gen)[:n].clone()
    slots[[2, 11]] = -1
    orc.kv_cache_update(key, value, cache, slots, layout)
    written = set()
    for t in range(n):
        s = int(slots[t])
        if s < 0:
            continue
        b, o = s // bs, s % bs
        written.add((b, o))
        for h in range(hkv):
            if layout == "v023":
                gk, gv = cache[b, 0, o, h], cache[b, 1, o, h]
            else:
                gk, gv = cache[b, h, o, :d], cache[b, h, o, d:]
            assert torch.equal(gk, key[t, h]) and torch.equal(gv, value[t, h])
    for b in range(nb):
        for o in range(bs):
            if (b, o) in written:
                continue
            if layout == "v023":
                assert torch.equal(cache[b, :, o], before[b, :, o])
            else:
                assert torch.equal(cache[b, :, o], before[b, :, o])
    # round trip: tokens written along a block table come back from gather_paged
    row = torch.randperm(nb, generator=gen).to(torch.int32)
    length = 13
    tok_slots = torch.tensor([int(row[x // bs]) * bs + x % bs for x in range(length)])
    orc.kv_cache_update(key, value, cache, tok_slots, layout)
    k, v = orc.gather_paged(cache, row, 0, length, layout)
    assert torch.equal(k, key[:length]) and torch.equal(v, value[:length])


def _full_causal(q, k, v, scale, qpos0):
    return brute(q, k, v, scale, qpos0)[0]


@pytest.mark.parametrize("mode", ["vanilla", "split", "staged", "split_n_a"])
def test_ring_forward_equals_full_attention(mode):
    """forward's segmentation reproduces causal attention over all tk keys
    (the check validate_ring_backend.py makes between custom and ref)."""
    gen = torch.Generator().manual_seed(9)
    h, hkv, d, bs, nb = 4, 2, 16, 4, 40
    scale = 1 / math.sqrt(d)
    cache = rnd(gen, nb, hkv, bs, 2 * d)
    reqs = [(6, 22), (1, 31), (9, 9), (5, 17)]  # (tq, tk)
    qsl = [0]
    for tq, _ in reqs:
        qsl.append(qsl[-1] + tq)
    seq_lens = [tk for _, tk in reqs]
    perm = torch.randperm(nb, generator=gen).to(torch.int32)
    bt = torch.stack([perm[i * 10:(i + 1) * 10] for i in range(4)])
    query = rnd(gen, qsl[-1], h, d)
    split, peers = 0, None
    if mode in ("split",):
        split = 8
    if mode == "split_n_a":
        split = 20  # larger than some qpos0: exercises the n_a queries
    if mode == "staged":
        peers = []
        for r, (tq, tk) in enumerate(reqs):
            k_all, v_all = orc.gather_paged(cache, bt[r], 0, tk, "v031")
            p = min(8, tk - tq)
            peers.append((k_all[:p], v_all[:p]) if p > 0 else None)
    out = orc.ring_forward(query, cache, "v031", qsl, seq_lens, bt, scale,
                           peers=peers, split_tokens=split, out_dtype=torch.float32)
    for r, (tq, tk) in enumerate(reqs):
        k_all, v_all = orc.gather_paged(cache, bt[r], 0, tk, "v031")
        ref = _full_causal(query[qsl[r]:qsl[r + 1]], k_all, v_all, scale, tk - tq)
        np.testing.assert_allclose(out[qsl[r]:qsl[r + 1]].numpy(), ref, atol=3e-6)


def test_causal_pairs_and_flops():
    for tq, tk, off in [(7, 9, 2), (5, 5, 0), (4, 3, 10), (6, 8, -3), (8192, 8192, 0)]:
        if tq > 100:
            # closed form for o = 0, Tq = Tk: n(n+1)/2
            assert orc.causal_pairs(tq, tk, off) == tq * (tq + 1) // 2
            continue
        brute_n = sum(1 for i in range(tq) for j in range(tk) if j <= off + i)
        assert orc.causal_pairs(tq, tk, off) == brute_n
    assert orc.causal_pairs(3, 4, None) == 12
    # C2: 8192 local causal (frame offset 0) + 8192 peer keys, 7B shape
    f = orc.attn_flops(28, 128, orc.causal_pairs(8192, 8192, 0) + 8192 * 8192)
    assert abs(f / 1e12 - 1.4432) < 1e-3


# ---------------------------------------------------------------------------
# Decode ring (ring_decode.py:187-259, ring_backend.py:643-722)
# ---------------------------------------------------------------------------
def _brute_t(q, k, v, scale, off):
    o, lse = brute(q, k, v, scale, off)
    return torch.from_numpy(o), torch.from_numpy(lse)


def test_ring_decode_hop_from_empty_accumulator_is_plain_attention():
    """An empty accumulator (o = 0, lse = -inf) merged with one hop is the
    float64 brute-force attention over snapshot + growth."""
    g = torch.Generator().manual_seed(81)
    q = rnd(g, 1, 4, 16)
    ck, cv = rnd(g, 11, 2, 16), rnd(g, 11, 2, 16)
    gk, gv = rnd(g, 3, 2, 16), rnd(g, 3, 2, 16)
    o0 = torch.zeros(1, 4, 16)
    l0 = torch.full((4, 1), float("-inf"))
    o, lse = orc.ring_decode_hop(q, o0, l0, ck, cv, gk, gv, 0.25)
    bo, bl = _brute_t(q, torch.cat([ck, gk]), torch.cat([cv, gv]), 0.25, None)
    assert (o.double() - bo).abs().max() < 1e-5
    assert (lse.double() - bl).abs().max() < 1e-5
    # without growth the hop sees the snapshot alone
    o, lse = orc.ring_decode_hop(q, o0, l0, ck, cv, None, None, 0.25)
    bo, bl = _brute_t(q, ck, cv, 0.25, None)
    assert (o.double() - bo).abs().max() < 1e-5


@pytest.mark.parametrize("n,policy", [(2, "rr"), (3, "rr"), (4, "rr"), (3, "owner")])
def test_decode_ring_protocol_equals_full_attention(n, policy):
    """Memory-split decode is exact: after every step the accumulator the
    owner gets back is attention over ALL keys (every prefix chunk, the own
    chunk and every decode token so far, including the one-step-late growth),
    and each peer holds exactly the positions assigned to it."""
    g = torch.Generator().manual_seed(90 + n)
    H, HKV, D, scale = 4, 2, 16, 0.25
    peers = [(rnd(g, 5 + 3 * i, HKV, D), rnd(g, 5 + 3 * i, HKV, D)) for i in range(n - 1)]
    own = (rnd(g, 6, HKV, D), rnd(g, 6, HKV, D))
    sim = orc.DecodeRingSim(peers, own, scale, policy)
    allk = [k for k, _ in peers] + [own[0]]
    allv = [v for _, v in peers] + [own[1]]
    pos0 = sum(k.shape[0] for k in allk)
    for t in range(3 * n + 2):
        q = rnd(g, 1, H, D)
        kc, vc = rnd(g, 1, HKV, D), rnd(g, 1, HKV, D)
        allk.append(kc)
        allv.append(vc)
        o, lse = sim.step(q, kc, vc, pos0 + t)
        bo, bl = _brute_t(q, torch.cat(allk), torch.cat(allv), scale, None)
        assert (o.double() - bo).abs().max() < 1e-5, t
        assert (lse.double() - bl).abs().max() < 1e-5, t
    # growth placement: position p lives on growth index p % n (rr) or the
    # owner; the last step's token is still pending when it belongs to a peer
    last = pos0 + 3 * n + 1
    for tidx in range(n):
        gi = n - 1 if tidx == 0 else tidx - 1
        want = [p for p in range(pos0, last + 1) if sim.assignee(p) == gi]
        if tidx != 0 and sim.assignee(last) == gi:
            want = want[:-1]
        assert len(sim.growth_of[tidx]) == len(want), (tidx, want)


def test_decode_ring_sim_catches_a_lost_shipment():
    """A planted mistake (the pending token is never shipped) breaks the
    full-attention check above -- the check has teeth."""
    g = torch.Generator().manual_seed(97)
    H, HKV, D, scale = 4, 2, 16, 0.25
    peers = [(rnd(g, 4, HKV, D), rnd(g, 4, HKV, D))]
    own = (rnd(g, 4, HKV, D), rnd(g, 4, HKV, D))

    class Lossy(orc.DecodeRingSim):
        def step(self, q, k_cur, v_cur, pos):
            self.pending = None
            return super().step(q, k_cur, v_cur, pos)

    sim = Lossy(peers, own, scale, "rr")
    allk, allv = [peers[0][0], own[0]], [peers[0][1], own[1]]
    worst = 0.0
    for t in range(4):
        q = rnd(g, 1, H, D)
        kc, vc = rnd(g, 1, HKV, D), rnd(g, 1, HKV, D)
        allk.append(kc)
        allv.append(vc)
        o, _ = sim.step(q, kc, vc, 8 + t)
        bo, _ = _brute_t(q, torch.cat(allk), torch.cat(allv), scale, None)
        worst = max(worst, (o.double() - bo).abs().max().item())
    assert worst > 1e-3



# ---------------------------------------------------------------------------
# Sliding window (ring_backend.py:372,397-398)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("tq,tk,off,w", [(5, 9, 4, 1), (7, 12, 5, 3), (6, 6, 0, 2),
                                         (4, 10, 8, 20), (5, 8, -2, 3), (3, 4, 9, 2)])
def test_window_vs_float64_brute(tq, tk, off, w):
    g = torch.Generator().manual_seed(tq * 31 + w)
    q, k, v = rnd(g, tq, 4, 8), rnd(g, tk, 2, 8), rnd(g, tk, 2, 8)
    o, lse = orc.attn_with_lse(q, k, v, 0.3, off, w)
    bo, bl = brute(q, k, v, 0.3, off, w)
    assert np.abs(o.double().numpy() - bo).max() < 1e-5
    finite = np.isfinite(bl)
    assert np.array_equal(finite, np.isfinite(lse.double().numpy()))
    if finite.any():
        assert np.abs(lse.double().numpy()[finite] - bl[finite]).max() < 1e-5


def test_window_closed_forms():
    """w = 1: every row sees only its own position -- out = v there and
    lse = scale q.k there.  A window wider than the causal range is no
    window at all."""
    g = torch.Generator().manual_seed(12)
    q, k, v = rnd(g, 6, 4, 8), rnd(g, 10, 2, 8), rnd(g, 10, 2, 8)
    o, lse = orc.attn_with_lse(q, k, v, 0.5, 4, 1)
    for i in range(6):
        j = 4 + i
        for h in range(4):
            assert torch.allclose(o[i, h], v[j, h // 2], atol=1e-6)
            assert abs(lse[h, i].item() - 0.5 * float(q[i, h] @ k[j, h // 2])) < 1e-5
    o1, l1 = orc.attn_with_lse(q, k, v, 0.5, 4, 10)
    o2, l2 = orc.attn_with_lse(q, k, v, 0.5, 4, None)
    assert torch.allclose(o1, o2) and torch.allclose(l1, l2)


def test_decode_ring_sim_window_one_sees_the_current_token_locally():
    """With window 1 the owner's local partial is the current token alone,
    so the ring's result is attention over every peer key (snapshots and
    their growth) plus the current token -- not the owner's chunk or its
    growth."""
    g = torch.Generator().manual_seed(77)
    H, HKV, D, scale = 4, 2, 16, 0.25
    peers = [(rnd(g, 5, HKV, D), rnd(g, 5, HKV, D)), (rnd(g, 3, HKV, D), rnd(g, 3, HKV, D))]
    own = (rnd(g, 4, HKV, D), rnd(g, 4, HKV, D))
    sim = orc.DecodeRingSim(peers, own, scale, "rr", window=1)
    peer_keys = [[peers[0]], [peers[1]]]
    pending = None
    for t in range(7):
        pos = 12 + t
        q = rnd(g, 1, H, D)
        kc, vc = rnd(g, 1, HKV, D), rnd(g, 1, HKV, D)
        if pending is not None:
            peer_keys[pending[0]].append(pending[1])
            pending = None
        o, lse = sim.step(q, kc, vc, pos)
        ks = [kv[0] for row in peer_keys for kv in row] + [kc]
        vs = [kv[1] for row in peer_keys for kv in row] + [vc]
        bo, bl = _brute_t(q, torch.cat(ks), torch.cat(vs), scale, None)
        assert (o.double() - bo).abs().max() < 1e-5, t
        assert (lse.double() - bl).abs().max() < 1e-5, t
        if pos % 3 != 2:  # growth index of a peer: shipped next step
            pending = (pos % 3, (kc, vc))
