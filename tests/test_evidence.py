"""CPU: the validators' evidence counters (ring_backend.py:228-275, :790-810).

``STAGING_STATS`` keeps high-water marks of the staging dict (entries held,
distinct chunks held, last staged chunk length) across drops, and
``reset_staging_stats`` clears them; ``reset_write_tracking`` enables
tracking and clears every field (``enable_write_tracking`` is the same
call); the chunk-A probe counts written slots of a request's first
``peer_end`` positions through its block-table row, and only those.
"""

import torch

from hcp_vllm_plugin_amd import ring_backend as rb


def test_staging_high_water_marks():
    rb.clear_peer_kv()
    rb.reset_staging_stats()
    k = torch.zeros(48, 2, 8)
    for layer in range(3):
        rb.stage_peer_kv("a", f"l{layer}", k, k)
    assert rb.STAGING_STATS == {"max_concurrent_chunks": 1, "max_staged_layers": 3,
                                "last_chunk_len": 48}
    rb.stage_peer_kv("b", "l0", k[:16], k[:16])
    assert rb.STAGING_STATS == {"max_concurrent_chunks": 2, "max_staged_layers": 4,
                                "last_chunk_len": 16}
    assert rb.drop_chunk_kv("a") == 3
    rb.stage_peer_kv("c", "l0", k[:32], k[:32])  # 2 chunks, 2 entries now held
    assert rb.STAGING_STATS == {"max_concurrent_chunks": 2, "max_staged_layers": 4,
                                "last_chunk_len": 32}
    rb.reset_staging_stats()
    assert rb.STAGING_STATS == {"max_concurrent_chunks": 0, "max_staged_layers": 0,
                                "last_chunk_len": 0}
    rb.clear_peer_kv()


def test_reset_write_tracking():
    rb.WRITE_TRACK.update(enabled=False, slots={1, 2}, overlap=5, skipped=3)
    rb.reset_write_tracking()
    assert rb.WRITE_TRACK == {"enabled": True, "slots": set(), "overlap": 0, "skipped": 0}
    rb.WRITE_TRACK.update(enabled=False, overlap=2)
    rb.enable_write_tracking()
    assert rb.WRITE_TRACK["enabled"] and rb.WRITE_TRACK["overlap"] == 0
    rb.WRITE_TRACK["enabled"] = False


def test_chunk_a_probe():
    bs = 4
    row = torch.tensor([9, 2, 7, 5], dtype=torch.int32)  # positions 0..15
    rb.reset_write_tracking()
    # position p lives in slot row[p // bs] * bs + p % bs
    slot = {p: int(row[p // bs]) * bs + p % bs for p in range(16)}
    rb.WRITE_TRACK["slots"] = {slot[0], slot[5], slot[6], slot[9], slot[10], 1000}
    # peer region of 6 positions: slots of positions 0..5 -> two written (0, 5)
    assert rb._probe_chunk_a_writes(row, 6, bs) == 2
    assert rb.WRITE_TRACK["overlap"] == 2
    # a region ending mid-block counts only positions before peer_end:
    # 0, 5, 6 and 9 of 0..9 (10 is past it)
    assert rb._probe_chunk_a_writes(row, 10, bs) == 4
    assert rb.WRITE_TRACK["overlap"] == 6
    assert rb._probe_chunk_a_writes(row, 1, bs) == 1
    assert rb.WRITE_TRACK["overlap"] == 7
    rb.WRITE_TRACK["enabled"] = False


def test_staging_generation_moves_only_on_key_or_map_changes():
    """The decode-step template stays valid while no chunk key appears or
    leaves and the request map is unchanged: staging a further layer of a
    staged chunk, or re-mapping a request to the same chunks, keeps it."""
    rb.clear_peer_kv()
    k = torch.zeros(16, 2, 8)
    g0 = rb._STAGE_GEN[0]
    rb.stage_peer_kv("a", "l0", k, k)
    g1 = rb._STAGE_GEN[0]
    assert g1 > g0                      # new chunk key
    rb.stage_peer_kv("a", "l1", k, k)
    rb.stage_peer_kv("a", "l1", k, k)   # restage of a staged layer
    assert rb._STAGE_GEN[0] == g1
    rb.map_request_peer(5, ["a"])
    g2 = rb._STAGE_GEN[0]
    assert g2 > g1
    rb.map_request_peer(5, "a")         # same chunks
    assert rb._STAGE_GEN[0] == g2
    rb.map_request_peer(5, ["a", "b"])
    assert rb._STAGE_GEN[0] > g2
    g3 = rb._STAGE_GEN[0]
    rb.unmap_request_peer(99)           # not mapped: nothing changes
    assert rb._STAGE_GEN[0] == g3
    assert rb.drop_chunk_kv("a") == 2
    assert rb._STAGE_GEN[0] > g3
    g4 = rb._STAGE_GEN[0]
    assert rb.drop_chunk_kv("a") == 0
    assert rb._STAGE_GEN[0] == g4
    rb.stage_peer_kv("a", "l0", k, k)   # the key appears again
    assert rb._STAGE_GEN[0] > g4
    rb.clear_peer_kv()


def test_step_metadata_cache_sees_in_place_updates():
    """The host copy of a step's metadata is reused while the same object and
    the same tensor contents (by storage, shape and in-place version) come
    back, and rebuilt when a reused object's tensors are refilled in place
    between steps, or after invalidate_step_cache()."""
    import types

    bt = torch.tensor([[3, 4], [5, 6]], dtype=torch.int32)
    meta = types.SimpleNamespace(query_start_loc=torch.tensor([0, 2, 5], dtype=torch.int32),
                                 seq_lens=torch.tensor([10, 20], dtype=torch.int32),
                                 block_table=bt)
    (qsl, sl, fb), _ = rb._host_metadata(meta)
    assert (qsl, sl, fb) == ([0, 2, 5], [10, 20], [3, 5])
    rb._STEP["fast"]["x"] = 1
    assert rb._host_metadata(meta)[0][1] == [10, 20] and "x" in rb._STEP["fast"]
    meta.seq_lens.copy_(torch.tensor([11, 21]))  # refilled in place: next step
    (qsl, sl, fb), _ = rb._host_metadata(meta)
    assert sl == [11, 21] and "x" not in rb._STEP["fast"]
    meta.block_table[1, 0] = 9
    assert rb._host_metadata(meta)[0][2] == [3, 9]
    with torch.inference_mode():
        qi = torch.tensor([0, 1, 2], dtype=torch.int32)
    meta.query_start_loc = qi  # no version counter: explicit invalidation
    assert rb._host_metadata(meta)[0][0] == [0, 1, 2]
    rb._STEP["fast"]["y"] = 1
    rb.invalidate_step_cache()
    assert rb._host_metadata(meta)[0][0] == [0, 1, 2] and "y" not in rb._STEP["fast"]
