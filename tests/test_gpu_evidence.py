"""GPU: the validators' evidence counters through the backend.

Every engine validator of the reference resets and reads the same counters
around a ring run (validate_ring_connector.py:205-207,230-235,
validate_ring_concurrent.py:196-199,220-224, validate_ring_closure.py:127-130,
170-178): ``reset_write_tracking`` / ``reset_staging_stats`` /
``reset_impl_stats`` / ``reset_batch_stats``, then ``STAGING_STATS``,
``WRITE_TRACK['overlap']`` / ``['slots']``, ``BATCH_STATS`` and
``IMPL_STATS``.  This test runs that sequence on a consumer that stages a
peer chunk for every layer, writes only its own chunk into the paged pool and
runs the ring forward, and checks the values the validators assert
(ring_backend.py:228-275, the chunk-A probe :790-810); then it plants a
write into the peer region and checks the probe counts it.
"""

import types

import pytest
import torch

from hcp_vllm_plugin_amd import ring_backend as rb
from oracle import ring_oracle as orc
from tests._util import OUT_TOL, max_err, randn, scale_for

pytestmark = pytest.mark.gpu

H, HKV, D, BS = 28, 4, 128, 16
LAYERS = 3


@pytest.fixture(autouse=True)
def _clean():
    rb.clear_peer_kv()
    yield
    rb.clear_peer_kv()
    rb.WRITE_TRACK["enabled"] = False


def _meta(dev, qsl, seq_lens, bt):
    return types.SimpleNamespace(
        num_actual_tokens=qsl[-1],
        query_start_loc=torch.tensor(qsl, dtype=torch.int32, device=dev),
        seq_lens=torch.tensor(seq_lens, dtype=torch.int32, device=dev),
        block_table=bt.to(dev))


def test_validator_counter_sequence(dev):
    gen = torch.Generator().manual_seed(2024)
    peer, tq = 512, 300           # chunk A (staged) + chunk B (this worker's)
    tk = peer + tq
    nblk = -(-tk // BS)
    nb = nblk + 8
    bt = torch.randperm(nb, generator=gen)[:nblk].to(torch.int32)[None, :]
    slots_b = torch.tensor([int(bt[0, p // BS]) * BS + p % BS for p in range(peer, tk)],
                           dtype=torch.int64)
    impl = rb.HcpRingAttentionImpl(H, D, scale_for(D), HKV)
    meta = _meta(dev, [0, tq], [tk], bt)

    rb.reset_write_tracking()
    rb.reset_staging_stats()
    rb.reset_impl_stats()
    rb.reset_batch_stats()
    assert rb.WRITE_TRACK == {"enabled": True, "slots": set(), "overlap": 0, "skipped": 0}

    layers = [types.SimpleNamespace(layer_name=f"model.layers.{i}.self_attn.attn")
              for i in range(LAYERS)]
    caches, peers = [], []
    for ly in layers:  # the connector stages chunk A for every layer first
        k = randn(gen, (peer, HKV, D), torch.bfloat16)
        v = randn(gen, (peer, HKV, D), torch.bfloat16)
        rb.stage_peer_kv("chunkA", ly.layer_name, k.to(dev), v.to(dev))
        peers.append((k.float(), v.float()))
    rb.map_request_peer(int(bt[0, 0]), ["chunkA"])
    assert rb.STAGING_STATS == {"max_concurrent_chunks": 1, "max_staged_layers": LAYERS,
                                "last_chunk_len": peer}

    for i, ly in enumerate(layers):
        # NaN everywhere: a kernel that read a slot outside the request's
        # chunk-B region would fail the comparison below
        cache = torch.full((nb, HKV, BS, 2 * D), float("nan"), dtype=torch.bfloat16)
        cache = cache.to(dev)
        kb = randn(gen, (tq, HKV, D), torch.bfloat16).to(dev)
        vb = randn(gen, (tq, HKV, D), torch.bfloat16).to(dev)
        impl.do_kv_cache_update(ly, kb, vb, cache, slots_b.to(dev))
        q = randn(gen, (tq, H, D), torch.bfloat16)
        out = torch.empty(tq, H, D, dtype=torch.bfloat16, device=dev)
        impl.forward(ly, q.to(dev), None, None, cache, meta, out)
        torch.cuda.synchronize()
        ref = orc.ring_forward(q.float(), cache.float().cpu().nan_to_num(0.0), "v031",
                               [0, tq], [tk], bt, scale_for(D), peers=[peers[i]],
                               out_dtype=torch.float32)
        assert max_err(out, ref) <= OUT_TOL[torch.bfloat16], i
        caches.append(cache)

    # the values validate_ring_connector.py:230-245 asserts on
    assert rb.STAGING_STATS["max_staged_layers"] == LAYERS
    assert rb.STAGING_STATS["last_chunk_len"] == peer
    assert rb.WRITE_TRACK["overlap"] == 0
    assert rb.WRITE_TRACK["slots"] == set(slots_b.tolist())
    assert rb.BATCH_STATS["max_reqs"] == 1
    assert rb.IMPL_STATS["attn_triton"] > 0 and rb.IMPL_STATS["attn_torch"] == 0
    assert rb.IMPL_STATS["merge_triton"] > 0 and rb.IMPL_STATS["merge_torch"] == 0

    # high-water marks survive the cleanup the validators check for
    rb.unmap_request_peer(int(bt[0, 0]))
    rb.drop_chunk_kv("chunkA")
    assert len(rb.PEER_KV_STAGING) == 0 and len(rb.PEER_REQ_MAP) == 0
    assert rb.STAGING_STATS["max_staged_layers"] == LAYERS


def test_overlap_probe_counts_peer_region_writes(dev):
    """A worker that wrote two slots of a request's peer region is caught by
    the probe of every ring forward (two per layer); writes outside it and a
    request without a peer are not counted."""
    gen = torch.Generator().manual_seed(7)
    peer, tq = 64, 40
    tk = peer + tq
    nblk = -(-tk // BS)
    nb = nblk + 20
    bt = torch.randperm(nb, generator=gen)[:nblk].to(torch.int32)[None, :]
    impl = rb.HcpRingAttentionImpl(H, D, scale_for(D), HKV)
    ly = types.SimpleNamespace(layer_name="model.layers.0.self_attn.attn")
    cache = randn(gen, (nb, HKV, BS, 2 * D), torch.bfloat16).to(dev)
    rb.reset_write_tracking()
    pos = [3, 63, 64, 100]  # two inside chunk A, two in chunk B
    slots = torch.tensor([int(bt[0, p // BS]) * BS + p % BS for p in pos], device=dev)
    kv = randn(gen, (len(pos), HKV, D), torch.bfloat16).to(dev)
    impl.do_kv_cache_update(ly, kv, kv, cache, slots)
    k = randn(gen, (peer, HKV, D), torch.bfloat16).to(dev)
    rb.stage_peer_kv("c", ly.layer_name, k, k)
    rb.map_request_peer(int(bt[0, 0]), ["c"])
    q = randn(gen, (tq, H, D), torch.bfloat16).to(dev)
    out = torch.empty_like(q)
    for _ in range(2):
        impl.forward(ly, q, None, None, cache, _meta(dev, [0, tq], [tk], bt), out)
    assert rb.WRITE_TRACK["overlap"] == 4
    # tracking off: the probe does not run
    rb.WRITE_TRACK["enabled"] = False
    impl.forward(ly, q, None, None, cache, _meta(dev, [0, tq], [tk], bt), out)
    assert rb.WRITE_TRACK["overlap"] == 4
