"""GPU parity of the backend contract: HcpRingAttentionImpl.forward.

The impl is driven the way vLLM's Attention layer drives the reference
(ring_backend.py:576-834): a paged KV cache, attention metadata with
``num_actual_tokens`` / ``query_start_loc`` / ``seq_lens`` / ``block_table``,
peer KV staged through ``stage_peer_kv`` + ``map_request_peer``
(ring_backend.py:96-123) or taken from a split of the local cache
(``HCP_RING_SPLIT_TOKENS``, :776-778).  The result is compared with the
oracle's restated segmentation (oracle.ring_oracle.ring_forward), which the
CPU tests pin to full causal attention over all keys.
"""

import types

import pytest
import torch

from hcp_vllm_plugin_amd import ring_backend as rb
from oracle import ring_oracle as orc
from tests._util import OUT_TOL, max_err, randn, scale_for

pytestmark = pytest.mark.gpu

H, HKV, D, BS = 28, 4, 128, 16


def _meta(dev, qsl, seq_lens, bt):
    return types.SimpleNamespace(
        num_actual_tokens=qsl[-1],
        query_start_loc=torch.tensor(qsl, dtype=torch.int32, device=dev),
        seq_lens=torch.tensor(seq_lens, dtype=torch.int32, device=dev),
        block_table=bt.to(dev),
    )


def _cache(gen, layout, nb, dtype, bs=BS):
    if layout == "v031":
        return randn(gen, (nb, HKV, bs, 2 * D), dtype)
    return randn(gen, (nb, 2, bs, HKV, D), dtype)


def _block_table(gen, seq_lens, nb, bs=BS):
    blocks = [-(-tk // bs) for tk in seq_lens]
    perm = torch.randperm(nb, generator=gen).to(torch.int32)
    bt = torch.zeros(len(seq_lens), max(blocks) + 1, dtype=torch.int32)
    o = 0
    for r, n in enumerate(blocks):
        bt[r, :n] = perm[o:o + n]
        o += n
    return bt


@pytest.fixture(autouse=True)
def _clean(monkeypatch):
    rb.clear_peer_kv()
    rb.reset_impl_stats()
    for k in ("HCP_RING_IMPL", "HCP_RING_MERGE", "HCP_RING_SPLIT_TOKENS", "HCP_RING_ENABLED"):
        monkeypatch.delenv(k, raising=False)
    yield
    rb.clear_peer_kv()


def _run(dev, layout, reqs, dtype=torch.bfloat16, seed=61, split=0, staged_chunks=None,
         monkeypatch=None, window=None, bs=BS):
    """reqs: list of (tq, tk).  staged_chunks: per request list of chunk lengths
    (peer prefix = their concatenation) or None."""
    gen = torch.Generator().manual_seed(seed)
    seq_lens = [tk for _, tk in reqs]
    qsl = [0]
    for tq, _ in reqs:
        qsl.append(qsl[-1] + tq)
    nb = sum(-(-tk // bs) for tk in seq_lens) + 4
    cache = _cache(gen, layout, nb, dtype, bs)
    bt = _block_table(gen, seq_lens, nb, bs)
    query = randn(gen, (qsl[-1] + 5, H, D), dtype)  # 5 padding rows past num_actual
    peers = None
    impl = rb.HcpRingAttentionImpl(H, D, scale_for(D), HKV, sliding_window=window)
    layer = types.SimpleNamespace(layer_name="model.layers.3.self_attn.attn")
    if split:
        monkeypatch.setenv("HCP_RING_SPLIT_TOKENS", str(split))
    if staged_chunks is not None:
        peers = []
        for r, chunks in enumerate(staged_chunks):
            if not chunks:
                peers.append(None)
                continue
            ks, vs, keys = [], [], []
            for c, n in enumerate(chunks):
                k = randn(gen, (n, HKV, D), dtype)
                v = randn(gen, (n, HKV, D), dtype)
                key = f"req{r}-chunk{c}"
                rb.stage_peer_kv(key, layer.layer_name, k.to(dev), v.to(dev))
                keys.append(key)
                ks.append(k)
                vs.append(v)
            rb.map_request_peer(int(bt[r, 0]), keys)
            peers.append((torch.cat(ks).float(), torch.cat(vs).float()))
    output = torch.full((query.shape[0], H, D), 7.0, dtype=dtype, device=dev)
    meta = _meta(dev, qsl, seq_lens, bt)
    ret = impl.forward(layer, query.to(dev), None, None, cache.to(dev), meta, output)
    torch.cuda.synchronize()
    assert ret is output
    ref = orc.ring_forward(query.float(), cache.float(), layout, qsl, seq_lens, bt,
                           scale_for(D), peers=peers, split_tokens=split,
                           out_dtype=torch.float32, window=window)
    n = qsl[-1]
    assert max_err(output[:n], ref[:n]) <= OUT_TOL[dtype]
    assert torch.all(output[n:] == 7.0)  # rows past num_actual_tokens untouched
    return output


@pytest.mark.parametrize("layout", ["v031", "v023"])
def test_forward_no_peer_is_causal_over_paged_cache(dev, layout):
    _run(dev, layout, [(300, 300), (17, 517), (1, 40), (0, 64), (129, 1000)])
    assert rb.IMPL_STATS["attn_hip"] == 1 and rb.IMPL_STATS["merge_hip"] == 0
    assert rb.IMPL_STATS["attn_torch"] == 0


@pytest.mark.parametrize("bs", [1, 8])
@pytest.mark.parametrize("layout", ["v031", "v023"])
def test_forward_small_blocks(dev, layout, bs, monkeypatch):
    """Caches with blocks under 16 tokens: prefill gathers the local segments
    on the device first (the reference gathers for every block size,
    ring_backend.py:617-624), decode reads them in place; staged peers and a
    split of the local cache both run."""
    reqs = [(300, 300 + 64), (17, 517), (1, 40), (129, 1000)]
    _run(dev, layout, reqs, staged_chunks=[[64], None, None, None], bs=bs)
    rb.clear_peer_kv()
    _run(dev, layout, [(200, 700), (1, 333), (64, 900)], split=100, monkeypatch=monkeypatch,
         bs=bs)
    _run(dev, layout, [(1, 700), (1, 33), (1, 1500)], bs=bs)  # a decode batch
    assert rb.IMPL_STATS["attn_torch"] == 0


@pytest.mark.parametrize("split", [64, 700])
def test_forward_split_tokens(dev, split, monkeypatch):
    # split 700 > qpos0 of some requests: exercises the n_a queries (:811-817)
    _run(dev, "v031", [(300, 900), (200, 256), (64, 1100), (5, 700)], split=split,
         monkeypatch=monkeypatch)
    assert rb.IMPL_STATS["merge_hip"] >= 1


@pytest.mark.parametrize("layout", ["v031", "v023"])
def test_forward_staged_peer_chunks(dev, layout):
    # peer prefixes are block aligned (ring_connector.py:582-587); request 1 has
    # two ordered chunks, request 2 none
    reqs = [(256, 256 + 512), (100, 100 + 64 + 128), (77, 77), (40, 40 + 2048)]
    staged = [[512], [64, 128], None, [1024, 1024]]
    _run(dev, layout, reqs, staged_chunks=staged)
    assert rb.IMPL_STATS["attn_triton"] == rb.IMPL_STATS["attn_hip"] > 0
    assert rb.IMPL_STATS["attn_torch"] == 0 and rb.IMPL_STATS["merge_torch"] == 0


def test_forward_decode_batch_uses_splitkv(dev):
    # every request has one query token: the split-KV decode path
    reqs = [(1, 513), (1, 2048 + 700), (1, 1), (1, 64 + 33)]
    staged = [[512], [2048], None, [64]]
    _run(dev, "v031", reqs, staged_chunks=staged)
    assert rb.IMPL_STATS["decode_hip"] == 1


@pytest.mark.parametrize("window", [1, 37, 256, 5000])
def test_forward_sliding_window(dev, window, monkeypatch):
    """sliding_window reaches every causal pass (no peer, the split env's n_a
    rows and local rest) and never the peer pass (ring_backend.py:786-830)."""
    _run(dev, "v031", [(300, 300), (17, 517), (1, 40), (129, 1000)], window=window)
    _run(dev, "v023", [(300, 900), (200, 256), (64, 1100), (5, 700)], split=700,
         monkeypatch=monkeypatch, window=window)


@pytest.mark.parametrize("window", [1, 100, 3000])
def test_forward_sliding_window_staged_and_decode(dev, window):
    _run(dev, "v031", [(256, 256 + 512), (100, 100 + 64 + 128), (40, 40 + 2048)],
         staged_chunks=[[512], [64, 128], [1024, 1024]], window=window)
    # decode batch: the local segment is cut to its last `window` keys
    _run(dev, "v031", [(1, 513), (1, 2048 + 700), (1, 1), (1, 64 + 33)],
         staged_chunks=[[512], [2048], None, [64]], window=window)
    assert rb.IMPL_STATS["decode_hip"] == 1


def test_forward_fp16(dev):
    _run(dev, "v031", [(200, 200 + 256), (33, 33 + 16)], dtype=torch.float16,
         staged_chunks=[[256], [16]])


def test_profiling_run_and_switches(dev, monkeypatch):
    impl = rb.HcpRingAttentionImpl(H, D, scale_for(D), HKV)
    out = torch.ones(4, H, D, device=dev)
    assert impl.forward(None, out, None, None, None, None, out) is out
    assert torch.all(out == 0)  # attn_metadata None -> zeros (ring_backend.py:590-592)
    monkeypatch.setenv("HCP_RING_IMPL", "torch")
    gen = torch.Generator().manual_seed(1)
    cache = _cache(gen, "v031", 4, torch.bfloat16).to(dev)
    meta = _meta(dev, [0, 2], [2], torch.zeros(1, 2, dtype=torch.int32))
    q = torch.zeros(2, H, D, dtype=torch.bfloat16, device=dev)
    with pytest.raises(NotImplementedError, match="HIP kernels only"):
        impl.forward(None, q, None, None, cache, meta, torch.empty_like(q))
    monkeypatch.setenv("HCP_RING_IMPL", "triton")  # legacy value: alias of hip
    impl.forward(None, q, None, None, cache, meta, torch.empty_like(q))


def test_backend_type_contract():
    B = rb.HcpRingAttentionBackend
    assert B.get_name() == "CUSTOM"
    assert B.get_impl_cls() is rb.HcpRingAttentionImpl
    assert B.forward_includes_kv_cache_update is False
    with pytest.raises(NotImplementedError):
        rb.HcpRingAttentionImpl(H, D, 0.1, HKV, alibi_slopes=[0.1] * H)
    with pytest.raises(NotImplementedError):
        rb.HcpRingAttentionImpl(H, D, 0.1, HKV, logits_soft_cap=30.0)


@pytest.mark.parametrize("window", [None, 300])
def test_forward_decode_staged_plan_across_layers(dev, window):
    """A pure decode step over three layers (one metadata object, as vLLM
    passes it): the split plan is built at the first layer and reused, each
    layer binding its own cache and its own staged chunks.  Requests: one
    staged chunk, two chunks, none, and a prefix at least as long as the
    context (its query sees the local range only, ring_backend.py:811-817)."""
    gen = torch.Generator().manual_seed(91)
    reqs = [(1, 1024 + 300), (1, 64 + 128 + 40), (1, 700), (1, 256)]
    chunks = [[1024], [64, 128], None, [256, 512]]
    seq_lens = [tk for _, tk in reqs]
    qsl = list(range(len(reqs) + 1))
    nb = sum(-(-tk // BS) for tk in seq_lens) + 4
    bt = _block_table(gen, seq_lens, nb)
    meta = _meta(dev, qsl, seq_lens, bt)
    impl = rb.HcpRingAttentionImpl(H, D, scale_for(D), HKV, sliding_window=window)
    for li in range(3):
        layer = types.SimpleNamespace(layer_name=f"model.layers.{li}.self_attn.attn")
        cache = _cache(gen, "v031", nb, torch.bfloat16)
        query = randn(gen, (len(reqs), H, D), torch.bfloat16)
        peers = []
        for r, cl in enumerate(chunks):
            if not cl:
                peers.append(None)
                continue
            ks, vs, keys = [], [], []
            for c, n in enumerate(cl):
                k, v = randn(gen, (n, HKV, D), torch.bfloat16), randn(gen, (n, HKV, D), torch.bfloat16)
                rb.stage_peer_kv(f"r{r}c{c}", layer.layer_name, k.to(dev), v.to(dev))
                keys.append(f"r{r}c{c}")
                ks.append(k)
                vs.append(v)
            rb.map_request_peer(int(bt[r, 0]), keys)
            peers.append((torch.cat(ks).float(), torch.cat(vs).float()))
        out = torch.full((len(reqs), H, D), 7.0, dtype=torch.bfloat16, device=dev)
        impl.forward(layer, query.to(dev), None, None, cache.to(dev), meta, out)
        torch.cuda.synchronize()
        ref = orc.ring_forward(query.float(), cache.float(), "v031", qsl, seq_lens, bt,
                               scale_for(D), peers=peers, out_dtype=torch.float32,
                               window=window)
        assert max_err(out, ref) <= OUT_TOL[torch.bfloat16], li
    assert rb.IMPL_STATS["decode_hip"] == 3
    assert sum(1 for k in rb._STEP["fast"] if k[0] == "dec_staged") == 1


def test_forward_decode_staged_chunk_arriving_between_layers(dev):
    """One decode request with no request-map entry takes the staged chunks
    through the single-request fallback (ring_backend.py:738-748).  Layer 0
    runs with nothing staged; a chunk is staged before layer 1, which must
    attend to it -- the step's cached decode template is rebuilt when a chunk
    key appears, not reused from layer 0."""
    gen = torch.Generator().manual_seed(92)
    peer, tk = 512, 512 + 300
    seq_lens, qsl = [tk], [0, 1]
    nb = -(-tk // BS) + 4
    bt = _block_table(gen, seq_lens, nb)
    meta = _meta(dev, qsl, seq_lens, bt)
    impl = rb.HcpRingAttentionImpl(H, D, scale_for(D), HKV)
    for li in range(3):
        layer = types.SimpleNamespace(layer_name=f"model.layers.{li}.self_attn.attn")
        cache = _cache(gen, "v031", nb, torch.bfloat16)
        query = randn(gen, (1, H, D), torch.bfloat16)
        peers = [None]
        if li >= 1:
            k, v = randn(gen, (peer, HKV, D), torch.bfloat16), randn(gen, (peer, HKV, D), torch.bfloat16)
            rb.stage_peer_kv("late", layer.layer_name, k.to(dev), v.to(dev))
            peers = [(k.float(), v.float())]
        out = torch.empty(1, H, D, dtype=torch.bfloat16, device=dev)
        impl.forward(layer, query.to(dev), None, None, cache.to(dev), meta, out)
        torch.cuda.synchronize()
        ref = orc.ring_forward(query.float(), cache.float(), "v031", qsl, seq_lens, bt,
                               scale_for(D), peers=peers, out_dtype=torch.float32)
        assert max_err(out, ref) <= OUT_TOL[torch.bfloat16], li
