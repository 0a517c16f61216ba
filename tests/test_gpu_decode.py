"""GPU parity: split-KV decode (hcp_decode_splitkv) against the oracle.

Each sequence has one query token, a contiguous peer segment and a paged
local segment (all keys visible, ring_backend.py:663-679 / :820-830 with
tq == 1); the reference result is local attention and peer attention merged
(ring_backend.py:831, ring_decode.py:46-61).
"""

import pytest
import torch

from hcp_vllm_plugin_amd.varlen import PagedCache, decode_attn, segment_contiguous, segment_paged
from oracle import ring_oracle as orc
from tests._util import LSE_TOL, OUT_TOL, max_err, randn, scale_for

pytestmark = pytest.mark.gpu


def _case(dev, h, hkv, d, dtype, peer_lens, loc_lens, bs, seed, split):
    gen = torch.Generator().manual_seed(seed)
    s = len(peer_lens)
    blocks = [-(-l // bs) for l in loc_lens]
    nb = sum(blocks) + 2
    cache = randn(gen, (nb, hkv, bs, 2 * d), dtype)
    perm = torch.randperm(nb, generator=gen).to(torch.int32)
    bt = torch.zeros(s, max(max(blocks), 1), dtype=torch.int32)
    o = 0
    for r, n in enumerate(blocks):
        bt[r, :n] = perm[o:o + n]
        o += n
    q = randn(gen, (s, h, d), dtype)
    pk = randn(gen, (sum(peer_lens), hkv, d), dtype)
    pv = randn(gen, (sum(peer_lens), hkv, d), dtype)
    cd, btd, qd, pkd, pvd = cache.to(dev), bt.to(dev), q.to(dev), pk.to(dev), pv.to(dev)
    pc = PagedCache.from_tensor(cd)
    segs, ps = [], 0
    for r in range(s):
        segs.append([segment_contiguous(pkd, pvd, ps, peer_lens[r]),
                     segment_paged(pc, btd[r], 0, loc_lens[r])])
        ps += peer_lens[r]
    scale = scale_for(d)
    out, lse = decode_attn(qd, segs, hkv, scale, with_lse=True, split_tokens=split)
    torch.cuda.synchronize()
    ps = 0
    for r in range(s):
        kl, vl = orc.gather_paged(cache.float(), bt[r], 0, loc_lens[r], "v031")
        qr = q[r:r + 1].float()
        ro_l, rl_l = orc.attn_with_lse(qr, kl, vl, scale, loc_lens[r] - 1)
        ro_p, rl_p = orc.attn_with_lse(qr, pk[ps:ps + peer_lens[r]].float(),
                                       pv[ps:ps + peer_lens[r]].float(), scale, None)
        ro, rl = orc.merge_pair(ro_l, rl_l, ro_p, rl_p)
        assert max_err(out[r:r + 1], ro) <= OUT_TOL[dtype], (r, max_err(out[r:r + 1], ro))
        assert max_err(lse[:, r:r + 1], rl) <= LSE_TOL, r
        ps += peer_lens[r]


@pytest.mark.parametrize("split", [None, 32, 64, 256, 1000])
def test_decode_qwen7b_shape(dev, split):
    _case(dev, 28, 4, 128, torch.bfloat16,
          peer_lens=[4096, 0, 1000, 33, 2048, 7],
          loc_lens=[512, 700, 1, 2048, 33, 1500], bs=16, seed=51, split=split)


@pytest.mark.parametrize("split", [None, 16])
def test_decode_llama70b_shape(dev, split):
    _case(dev, 64, 8, 128, torch.bfloat16, peer_lens=[3000, 100], loc_lens=[900, 17],
          bs=16, seed=52, split=split)


def test_decode_fp16_d64(dev):
    _case(dev, 14, 2, 64, torch.float16, peer_lens=[512, 2048, 0], loc_lens=[100, 1, 600],
          bs=16, seed=53, split=128)


@pytest.mark.parametrize("h,hkv,d,dtype", [
    (32, 1, 128, torch.bfloat16),   # MQA: G = 32, two full head chunks
    (28, 1, 128, torch.bfloat16),   # G = 28: chunks of 16 and 12 heads
    (40, 2, 64, torch.float16),     # G = 20
    (17, 1, 64, torch.bfloat16),    # G = 17: a 1-head second chunk
])
@pytest.mark.parametrize("split", [None, 64])
def test_decode_groups_above_16(dev, h, hkv, d, dtype, split):
    """Query-head groups larger than the 16 MFMA columns (any G, as the
    reference's head map h / G, ring_triton_attn.py:64)."""
    _case(dev, h, hkv, d, dtype, peer_lens=[1500, 0, 64], loc_lens=[300, 800, 1],
          bs=16, seed=54 + h + hkv, split=split)


@pytest.mark.parametrize("split", [None, 16, 64])
def test_decode_paged_cache_past_4gib_nan_outside_segments(dev, split):
    """A cache of 4.6 GB (its span from a head's base exceeds 4 GiB, so the
    split kernel loads with 64-bit addresses), the sequences' blocks past
    4 GiB, segments starting mid-block with ragged ends, and every slot
    outside them NaN: reading any of those would show in the result."""
    h, hkv, d, bs = 28, 4, 128, 16
    blk_bytes = hkv * bs * 2 * d * 2
    nb = 4_600_000_000 // blk_bytes + 1
    cache = torch.full((nb, hkv, bs, 2 * d), float("nan"), dtype=torch.bfloat16, device=dev)
    gen = torch.Generator().manual_seed(78)
    seqs = [(37, 300), (0, 5000), (15, 1), (100, 2049)]  # (segment start, length)
    rows, ks, vs = [], [], []
    next_hi = nb - 1  # blocks allocated downward from the top of the cache
    for start, ln in seqs:
        nblk = -(-(start + ln) // bs)
        ids = list(range(next_hi - nblk + 1, next_hi + 1))[::-1]
        next_hi -= nblk
        rows.append(ids)
        k = randn(gen, (ln, hkv, d), torch.bfloat16)
        v = randn(gen, (ln, hkv, d), torch.bfloat16)
        pos = torch.arange(start, start + ln)
        blk = torch.tensor(ids, dtype=torch.long)[pos // bs].to(dev)
        slot = (pos % bs).to(dev)
        cache[blk, :, slot, :d] = k.to(dev)
        cache[blk, :, slot, d:] = v.to(dev)
        ks.append(k)
        vs.append(v)
    assert min(min(r) for r in rows) * blk_bytes > (1 << 32)
    bt = torch.zeros(len(seqs), max(len(r) for r in rows), dtype=torch.int32)
    for r, ids in enumerate(rows):
        bt[r, :len(ids)] = torch.tensor(ids, dtype=torch.int32)
    btd = bt.to(dev)
    pc = PagedCache.from_tensor(cache)
    q = randn(gen, (len(seqs), h, d), torch.bfloat16)
    segs = [[segment_paged(pc, btd[r], start, ln)] for r, (start, ln) in enumerate(seqs)]
    scale = scale_for(d)
    out, lse = decode_attn(q.to(dev), segs, hkv, scale, with_lse=True, split_tokens=split)
    torch.cuda.synchronize()
    assert not torch.isnan(out).any() and not torch.isnan(lse).any()
    for r, (_, ln) in enumerate(seqs):
        ro, rl = orc.attn_with_lse(q[r:r + 1].float(), ks[r].float(), vs[r].float(), scale, ln - 1)
        assert max_err(out[r:r + 1], ro) <= OUT_TOL[torch.bfloat16], r
        assert max_err(lse[:, r:r + 1], rl) <= LSE_TOL, r
    del cache


def test_decode_empty_sequence(dev):
    """A sequence whose segments are all empty gets out 0, lse -inf."""
    h, hkv, d = 28, 4, 128
    q = torch.randn(2, h, d, device=dev).to(torch.bfloat16)
    k = torch.randn(100, hkv, d, device=dev).to(torch.bfloat16)
    segs = [[segment_contiguous(k, k, 0, 100)], [segment_contiguous(k, k, 0, 0)]]
    out, lse = decode_attn(q, segs, hkv, 0.088, with_lse=True)
    torch.cuda.synchronize()
    assert torch.all(out[1] == 0) and torch.all(torch.isneginf(lse[:, 1]))
    ro, rl = orc.attn_with_lse(q[:1].float().cpu(), k.float().cpu(), k.float().cpu(), 0.088, None)
    assert max_err(out[:1], ro) <= OUT_TOL[torch.bfloat16]


# ---------------------------------------------------------------------------
# hcp_decode_splitkv_acc: the decode merged into a running accumulator
# ---------------------------------------------------------------------------
def _acc_case(dev, dtype, seg_lens, split, seed, in_place=False, acc_lse_fill=None):
    h, hkv, d = 28, 4, 128
    gen = torch.Generator().manual_seed(seed)
    s = len(seg_lens)
    q = randn(gen, (s, h, d), dtype)
    o_acc = randn(gen, (s, h, d), dtype)
    l_acc = torch.randn(h, s, generator=gen) * 4
    if acc_lse_fill is not None:
        l_acc[:, 0] = acc_lse_fill
    ks = [[randn(gen, (n, hkv, d), dtype) for n in lens] for lens in seg_lens]
    vs = [[randn(gen, (n, hkv, d), dtype) for n in lens] for lens in seg_lens]
    kd = [[k.to(dev) for k in row] for row in ks]
    vd = [[v.to(dev) for v in row] for row in vs]
    segs = [[segment_contiguous(k, v) for k, v in zip(kr, vr)] for kr, vr in zip(kd, vd)]
    qd, oad, lad = q.to(dev), o_acc.to(dev), l_acc.to(dev)
    scale = scale_for(d)
    if in_place:
        decode_attn(qd, segs, hkv, scale, out=oad, split_tokens=split, acc=(oad, lad))
        # lse in place: run again through the batch API with lse = acc lse
        out, lse = oad, None
    else:
        out, lse = decode_attn(qd, segs, hkv, scale, with_lse=True, split_tokens=split,
                               acc=(oad, lad))
    torch.cuda.synchronize()
    for r in range(s):
        ro, rl = o_acc[r:r + 1].float(), l_acc[:, r:r + 1].clone()
        rl[torch.isposinf(rl)] = float("-inf")
        for k, v in zip(ks[r], vs[r]):
            if k.shape[0] == 0:
                continue
            po, pl = orc.attn_with_lse(q[r:r + 1].float(), k.float(), v.float(), scale, None)
            ro, rl = orc.merge_pair(ro, rl, po, pl)
        assert max_err(out[r:r + 1], ro) <= OUT_TOL[dtype], r
        if lse is not None:
            assert max_err(lse[:, r:r + 1], rl) <= LSE_TOL, r


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("split", [None, 64, 100 * 64])
def test_decode_acc_vs_oracle(dev, dtype, split):
    """Chunk + growth segments of several lengths; split 64 gives one
    sequence 500+ partials, exercising the reduce's 8-wide batches and its
    remainder."""
    _acc_case(dev, dtype, [[32768, 512], [1000, 3], [1, 0], [700]], split, seed=61)


def test_decode_acc_empty_accumulator_and_no_keys(dev):
    """An accumulator LSE of -inf or +inf contributes nothing; a sequence with
    no keys returns the accumulator itself."""
    _acc_case(dev, torch.bfloat16, [[300], [0]], None, seed=62, acc_lse_fill=float("-inf"))
    _acc_case(dev, torch.bfloat16, [[300], [0]], None, seed=63, acc_lse_fill=float("inf"))


def test_decode_acc_in_place(dev):
    """out may be the accumulator's own O (and lse its LSE)."""
    _acc_case(dev, torch.float16, [[5000, 17], [64]], 256, seed=64, in_place=True)
    h, hkv, d = 28, 4, 128
    gen = torch.Generator().manual_seed(65)
    q = randn(gen, (1, h, d), torch.bfloat16).to(dev)
    k = randn(gen, (2000, hkv, d), torch.bfloat16).to(dev)
    v = randn(gen, (2000, hkv, d), torch.bfloat16).to(dev)
    o = randn(gen, (1, h, d), torch.bfloat16).to(dev)
    lse = (torch.randn(h, 1, generator=gen) * 2).to(dev)
    want_o, want_l = decode_attn(q, [[segment_contiguous(k, v)]], hkv, 0.088, with_lse=True,
                                 acc=(o, lse))
    from hcp_vllm_plugin_amd.varlen import DecodeBatch

    DecodeBatch([[segment_contiguous(k, v)]], h, hkv, d, dev).run(q, o, lse, 0.088, acc=(o, lse))
    torch.cuda.synchronize()
    assert torch.equal(o, want_o) and torch.equal(lse, want_l)
