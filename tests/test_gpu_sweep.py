"""GPU parity sweeps over seeded random configurations: of
HcpRingAttentionImpl.forward against the oracle's restated segmentation
(oracle.ring_oracle.ring_forward, ring_backend.py:576-834), and of the
kernel contract (ring_attn_with_lse / ring_attn_merged) against the oracle's
_attn_with_lse and merge (ring_backend.py:366-421, ring_decode.py:46-61).

Each case draws, from its own seed: the head counts (any GQA group), a
head_dim (a multiple of 8 up to 256), the dtype, the cache layout and block
size (1 to 64 tokens), an optional sliding window, and a batch of 1-6
requests -- prefill rows, single-token decode rows or both -- whose peer
prefix is either staged in one to three chunks (stage_peer_kv +
map_request_peer, ring_backend.py:96-123) or taken from a split of the local
cache (HCP_RING_SPLIT_TOKENS, :776-778).  Lengths are ragged on purpose
(partial blocks, partial 64-key tiles, empty requests).  The same checks as
the fixed cases in test_gpu_backend.py apply: every computed row within the
dtype's tolerance of the oracle, padding rows past num_actual_tokens
untouched, and no CPU path taken.
"""

import random
import types

import pytest
import torch

from hcp_vllm_plugin_amd import ring_backend as rb
from oracle import ring_oracle as orc
from tests._util import OUT_TOL, max_err, randn, scale_for

pytestmark = pytest.mark.gpu

N_CASES = 64


@pytest.fixture(autouse=True)
def _clean(monkeypatch):
    rb.clear_peer_kv()
    rb.reset_impl_stats()
    for k in ("HCP_RING_IMPL", "HCP_RING_MERGE", "HCP_RING_SPLIT_TOKENS", "HCP_RING_ENABLED"):
        monkeypatch.delenv(k, raising=False)
    yield
    rb.clear_peer_kv()


def _draw_case(seed):
    """A configuration (plain Python values) drawn from ``seed``."""
    rnd = random.Random(seed)
    hkv = rnd.choice([1, 2, 4, 8])
    group = rnd.choice([1, 2, 3, 4, 7, 8, 16, 24])
    d = rnd.choice([64, 128, 128, 128, 8 * rnd.randint(1, 32)])
    mode = rnd.choice(["prefill", "prefill", "decode", "mixed"])
    nreq = rnd.randint(1, 6)
    reqs = []
    for _ in range(nreq):
        decode = mode == "decode" or (mode == "mixed" and rnd.random() < 0.5)
        tk = rnd.randint(1, 3000)
        tq = 1 if decode else rnd.randint(0, tk)
        reqs.append((tq, tk))
    peer = rnd.choice(["none", "staged", "staged", "split"])
    chunks = None
    split = 0
    if peer == "staged":
        chunks = [[rnd.randint(1, 700) for _ in range(rnd.randint(1, 3))]
                  if rnd.random() < 0.75 else None for _ in reqs]
    elif peer == "split":
        split = rnd.randint(1, 900)
    return dict(
        h=hkv * group, hkv=hkv, d=d,
        dtype=rnd.choice([torch.bfloat16, torch.float16]),
        layout=rnd.choice(["v031", "v023"]),
        bs=rnd.choice([1, 4, 16, 16, 32, 64]),
        window=rnd.choice([None, rnd.randint(1, 600)]),
        reqs=reqs, chunks=chunks, split=split,
    )


@pytest.mark.parametrize("seed", range(N_CASES))
def test_forward_random_configuration(dev, seed, monkeypatch):
    c = _draw_case(1000 + seed)
    h, hkv, d, dtype, bs, layout = c["h"], c["hkv"], c["d"], c["dtype"], c["bs"], c["layout"]
    print(f"sweep case {seed}: {c}", flush=True)
    gen = torch.Generator().manual_seed(seed)
    seq_lens = [tk for _, tk in c["reqs"]]
    qsl = [0]
    for tq, _ in c["reqs"]:
        qsl.append(qsl[-1] + tq)
    nb = sum(-(-tk // bs) for tk in seq_lens) + 3
    if layout == "v031":
        cache = randn(gen, (nb, hkv, bs, 2 * d), dtype)
    else:
        cache = randn(gen, (nb, 2, bs, hkv, d), dtype)
    perm = torch.randperm(nb, generator=gen).to(torch.int32)
    bt = torch.zeros(len(seq_lens), max(-(-tk // bs) for tk in seq_lens) + 1, dtype=torch.int32)
    o = 0
    for r, tk in enumerate(seq_lens):
        n = -(-tk // bs)
        bt[r, :n] = perm[o:o + n]
        o += n
    query = randn(gen, (qsl[-1] + 3, h, d), dtype)  # 3 padding rows past num_actual
    layer = types.SimpleNamespace(layer_name="model.layers.0.self_attn.attn")
    impl = rb.HcpRingAttentionImpl(h, d, scale_for(d), hkv, sliding_window=c["window"])
    if c["split"]:
        monkeypatch.setenv("HCP_RING_SPLIT_TOKENS", str(c["split"]))
    peers = None
    if c["chunks"] is not None:
        peers = []
        for r, chunks in enumerate(c["chunks"]):
            if not chunks:
                peers.append(None)
                continue
            ks, vs, keys = [], [], []
            for j, n in enumerate(chunks):
                k, v = randn(gen, (n, hkv, d), dtype), randn(gen, (n, hkv, d), dtype)
                key = f"sweep{seed}-req{r}-chunk{j}"
                rb.stage_peer_kv(key, layer.layer_name, k.to(dev), v.to(dev))
                keys.append(key)
                ks.append(k)
                vs.append(v)
            rb.map_request_peer(int(bt[r, 0]), keys)
            peers.append((torch.cat(ks).float(), torch.cat(vs).float()))
    output = torch.full((query.shape[0], h, d), 7.0, dtype=dtype, device=dev)
    meta = types.SimpleNamespace(
        num_actual_tokens=qsl[-1],
        query_start_loc=torch.tensor(qsl, dtype=torch.int32, device=dev),
        seq_lens=torch.tensor(seq_lens, dtype=torch.int32, device=dev),
        block_table=bt.to(dev),
    )
    ret = impl.forward(layer, query.to(dev), None, None, cache.to(dev), meta, output)
    torch.cuda.synchronize()
    assert ret is output
    ref = orc.ring_forward(query.float(), cache.float(), layout, qsl, seq_lens, bt,
                           scale_for(d), peers=peers, split_tokens=c["split"],
                           out_dtype=torch.float32, window=c["window"])
    n = qsl[-1]
    assert max_err(output[:n], ref[:n]) <= OUT_TOL[dtype], (c, max_err(output[:n], ref[:n]))
    assert torch.all(output[n:] == 7.0)
    assert rb.IMPL_STATS["attn_torch"] == 0 and rb.IMPL_STATS["merge_torch"] == 0


def _draw_pass(seed):
    """A kernel-contract case (plain Python values) drawn from ``seed``."""
    rnd = random.Random(seed)
    hkv = rnd.choice([1, 2, 4, 8])
    group = rnd.choice([1, 2, 4, 7, 8])
    d = rnd.choice([64, 128, rnd.randint(1, 256)])
    tq = rnd.randint(1, 1200)
    tk = rnd.randint(0, 2000)
    causal = rnd.random() < 0.6
    off = rnd.choice([tk - tq, rnd.randint(-200, tk + 200)]) if causal else None
    window = rnd.choice([None, rnd.randint(1, 800)]) if causal else None
    return dict(h=hkv * group, hkv=hkv, d=d, tq=tq, tk=tk, off=off, window=window,
                dtype=rnd.choice([torch.bfloat16, torch.float16]),
                packed=rnd.random() < 0.3, merged=rnd.random() < 0.5)


@pytest.mark.parametrize("seed", range(48))
def test_pass_random_configuration(dev, seed):
    """``ring_attn_with_lse`` (and, for half the cases, ``ring_attn_merged``
    over a random partial) on random shapes: any head_dim up to 256, causal
    offsets inside, before and past the key range, windows, empty key ranges,
    and q/k/v as views into one packed projection output -- against the
    oracle's ``_attn_with_lse`` / merge restatement."""
    from hcp_vllm_plugin_amd import ring_attn_merged, ring_attn_with_lse
    from tests._util import LSE_TOL

    c = _draw_pass(5000 + seed)
    h, hkv, d, tq, tk, dtype = c["h"], c["hkv"], c["d"], c["tq"], c["tk"], c["dtype"]
    print(f"pass case {seed}: {c}", flush=True)
    gen = torch.Generator().manual_seed(seed)
    # values at half scale: with a handful of keys a row's output is close to
    # one value row, and an N(0,1) row reaches |o| > 4, where bf16's own
    # rounding (half an ulp, 2^-6) is above the 1.5e-2 gate for any
    # implementation
    if c["packed"]:  # one projection output [T, H + 2 Hkv, D]; q, k, v are views
        t = max(tq, tk)
        qkv = randn(gen, (t, h + 2 * hkv, d), torch.float32)
        qkv[:, h + hkv:] *= 0.5
        qkv = qkv.to(dtype).to(dev)
        q, k, v = qkv[:tq, :h], qkv[:tk, h:h + hkv], qkv[:tk, h + hkv:]
    else:
        q = randn(gen, (tq, h, d), dtype).to(dev)
        k = randn(gen, (tk, hkv, d), dtype).to(dev)
        v = (randn(gen, (tk, hkv, d), torch.float32) * 0.5).to(dtype).to(dev)
    scale = scale_for(d)
    ro, rl = orc.attn_with_lse(q.float().cpu(), k.float().cpu(), v.float().cpu(), scale,
                               c["off"], window=c["window"])
    if c["merged"]:
        # a partial output at the same half scale
        po = (randn(gen, (tq, h, d), torch.float32) * 0.5).to(dtype).to(dev)
        pl = (torch.randn(h, tq, generator=gen) * 3).to(dev)
        lse = torch.empty(h, tq, dtype=torch.float32, device=dev)
        out = ring_attn_merged(q, k, v, scale, c["off"], po, pl, window=c["window"],
                               output_lse=lse)
        ro, rl = orc.merge_pair(po.float().cpu(), pl.cpu(), ro, rl)
    else:
        out, lse = ring_attn_with_lse(q, k, v, scale, c["off"], window=c["window"])
    torch.cuda.synchronize()
    assert out.shape == (tq, h, d) and out.dtype == dtype
    assert max_err(out, ro) <= OUT_TOL[dtype], (c, max_err(out, ro))
    assert max_err(lse, rl) <= LSE_TOL, (c, max_err(lse, rl))
