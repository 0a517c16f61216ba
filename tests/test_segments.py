"""Host-side KV segment descriptors (CPU): trimming and the decode window.

A decode query at the last position of its local keys sees, under a sliding
window w, the last w keys of the concatenation of its local segments
(ring_backend.py:397-398 with qpos = len - 1, :672-679 for the decode ring's
own chunk + growth + current token).
"""

import pytest
import torch

from hcp_vllm_plugin_amd.varlen import head_major, segment_contiguous, trim_segment, window_tail


def _segs():
    k = torch.zeros(100, 4, 128, dtype=torch.bfloat16)
    return k, [segment_contiguous(k, k, 0, 40), segment_contiguous(k, k, 40, 25),
               segment_contiguous(k, k, 65, 1)]


def _spans(segs):
    return [(s.start, s.len) for s in segs]


def test_window_tail_keeps_the_last_keys():
    _, (a, b, c) = _segs()
    assert _spans(window_tail([a, None, b, c], 30)) == [(36, 4), (40, 25), (65, 1)]
    assert _spans(window_tail([a, b, c], 1)) == [(65, 1)]
    assert _spans(window_tail([a, b, c], 26)) == [(40, 25), (65, 1)]
    assert _spans(window_tail([a, b, c], 500)) == [(0, 40), (40, 25), (65, 1)]
    assert _spans(window_tail([a, b, c], None)) == [(0, 40), (40, 25), (65, 1)]
    assert window_tail([], 5) == []
    # the total key count equals min(window, keys) -- brute force over windows
    for w in range(1, 70):
        assert sum(s.len for s in window_tail([a, b, c], w)) == min(w, 66)
    with pytest.raises(ValueError):
        window_tail([a], 0)


def test_trim_segment_keeps_the_descriptor():
    k, (a, _, _) = _segs()
    t = trim_segment(a, 15)
    assert (t.start, t.len) == (15, 25)
    assert (t.k_addr, t.v_addr, t.stride_tok, t.stride_head) == \
        (a.k_addr, a.v_addr, a.stride_tok, a.stride_head)
    assert t._keep is a._keep  # the storage stays referenced
    assert trim_segment(a, 40).len == 0
    with pytest.raises(ValueError):
        trim_segment(a, 41)


def test_head_major_view_and_staging():
    """Staged peer KV keeps its values and [n, Hkv, D] shape but is stored
    head-major (each KV head's keys one contiguous run); a tensor already so
    stored is returned as is, and a segment over it carries the strides."""
    from hcp_vllm_plugin_amd import ring_backend as rb

    k = torch.randn(37, 4, 16)
    h = head_major(k)
    assert h.shape == k.shape and torch.equal(h, k)
    assert h.stride() == (16, 37 * 16, 1) and h.is_contiguous() is False
    assert head_major(h) is h
    seg = segment_contiguous(h, h, 5, 20)
    assert (seg.stride_tok, seg.stride_head) == (16, 37 * 16)
    v = torch.randn(37, 4, 16)
    try:
        rb.stage_peer_kv("c0", "layer0", k, v)
        sk, sv = rb.PEER_KV_STAGING[("c0", "layer0")]
        assert torch.equal(sk, k) and torch.equal(sv, v)
        assert sk.stride() == (16, 37 * 16, 1) and sv.stride() == (16, 37 * 16, 1)
    finally:
        rb.clear_peer_kv()
