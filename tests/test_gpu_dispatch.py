"""GPU parity of the dispatch layer ``_attn`` / ``_merge`` (ring_backend.py:309-360).

``_attn(q, k, v, scale, q_pos0_in_kv, window)`` returns (out in q's dtype,
lse [H, Tq] float32); ``_merge(o_loc, lse_loc, o_peer, lse_peer)`` is
``merge_attn_states(out, o_peer, lse_peer, o_loc, lse_loc)`` with out in
o_loc's dtype.  Both read ``HCP_RING_IMPL`` / ``HCP_RING_MERGE`` on every
call and count ``IMPL_STATS``; ``torch`` raises (this build has no torch
path), ``triton`` is an alias of ``hip``.  Checked against the oracle's
``attn_with_lse`` and ``lse_merge`` on the same seeded inputs.
"""

import pytest
import torch

from hcp_vllm_plugin_amd import ring_backend as rb
from oracle import ring_oracle as orc
from tests._util import LSE_TOL, OUT_TOL, max_err, outlier_k, randn, scale_for

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _clean(monkeypatch):
    for k in ("HCP_RING_IMPL", "HCP_RING_MERGE"):
        monkeypatch.delenv(k, raising=False)
    rb.reset_impl_stats()
    yield


def _inputs(gen, tq, tk, h, hkv, d, dtype):
    q = randn(gen, (tq, h, d), dtype)
    k = outlier_k(randn(gen, (tk, hkv, d), torch.float32), gen).to(dtype)
    v = randn(gen, (tk, hkv, d), dtype)
    return q, k, v


# (tq, tk, causal offset or None, window or None)
CASES = [
    (200, 300, None, None),   # non-causal (the peer pass)
    (257, 257, 0, None),      # causal, offset 0 (local chunk after its peer)
    (130, 500, 370, None),    # causal with an offset: queries at the end of the keys
    (300, 300, 0, 64),        # sliding window
    (96, 640, 544, 100),      # window with an offset
]


@pytest.mark.parametrize("impl", ["hip", "triton"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("tq,tk,off,window", CASES)
def test_attn_dispatch(dev, monkeypatch, impl, dtype, tq, tk, off, window):
    monkeypatch.setenv("HCP_RING_IMPL", impl)
    gen = torch.Generator().manual_seed(1000 + tq + tk)
    h, hkv, d = 28, 4, 128
    q, k, v = _inputs(gen, tq, tk, h, hkv, d, dtype)
    before = dict(rb.IMPL_STATS)
    o, lse = rb._attn(q.to(dev), k.to(dev), v.to(dev), scale_for(d), off, window)
    torch.cuda.synchronize()
    assert o.dtype == dtype and o.shape == (tq, h, d) and o.device.type == "cuda"
    assert lse.dtype == torch.float32 and lse.shape == (h, tq)
    o_ref, lse_ref = orc.attn_with_lse(q, k, v, scale_for(d), off, window)
    assert max_err(o, o_ref) <= OUT_TOL[dtype]
    assert max_err(lse, lse_ref) <= LSE_TOL
    # one kernel launch counted, under the new and the legacy key; no torch path
    assert rb.IMPL_STATS["attn_hip"] == before["attn_hip"] + 1
    assert rb.IMPL_STATS["attn_triton"] == before["attn_triton"] + 1
    assert rb.IMPL_STATS["attn_torch"] == 0


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
def test_merge_dispatch(dev, monkeypatch, out_dtype):
    """_merge of a local causal pass and a peer pass over two halves of the
    keys equals attention over all of them (validate_ring_triton_kernel.py:80-94
    on the dispatch layer), out in o_loc's dtype."""
    monkeypatch.setenv("HCP_RING_MERGE", "triton")
    gen = torch.Generator().manual_seed(77)
    h, hkv, d, tq, tp, tl = 14, 2, 64, 160, 192, 160
    q, kp, vp = _inputs(gen, tq, tp, h, hkv, d, out_dtype)
    _, kl, vl = _inputs(gen, 0, tl, h, hkv, d, out_dtype)
    qd = q.to(dev)
    o_peer, lse_peer = rb._attn(qd, kp.to(dev), vp.to(dev), scale_for(d), None)
    o_loc, lse_loc = rb._attn(qd, kl.to(dev), vl.to(dev), scale_for(d), 0)
    before = dict(rb.IMPL_STATS)
    out = rb._merge(o_loc, lse_loc, o_peer, lse_peer)
    torch.cuda.synchronize()
    assert out.dtype == o_loc.dtype and out.shape == o_loc.shape
    # against the oracle's merge of the same two partials ...
    ref = orc.lse_merge(o_loc.float().cpu(), lse_loc.cpu(), o_peer.float().cpu(), lse_peer.cpu())
    assert max_err(out, ref) <= OUT_TOL[out_dtype]
    # ... and against full attention over peer + local keys (the ring identity)
    k_all = torch.cat([kp, kl])
    v_all = torch.cat([vp, vl])
    full, _ = orc.attn_with_lse(q, k_all, v_all, scale_for(d), tp)
    assert max_err(out, full) <= 2 * OUT_TOL[out_dtype]
    assert rb.IMPL_STATS["merge_hip"] == before["merge_hip"] + 1
    assert rb.IMPL_STATS["merge_triton"] == before["merge_triton"] + 1
    assert rb.IMPL_STATS["merge_torch"] == 0


def test_torch_switch_raises(dev, monkeypatch):
    """HCP_RING_IMPL / HCP_RING_MERGE = torch would run the oracle in the
    product path: both raise, read on every call, and count nothing."""
    gen = torch.Generator().manual_seed(5)
    q, k, v = (t.to(dev) for t in _inputs(gen, 64, 64, 28, 4, 128, torch.bfloat16))
    monkeypatch.setenv("HCP_RING_IMPL", "torch")
    with pytest.raises(NotImplementedError):
        rb._attn(q, k, v, scale_for(128), 0)
    monkeypatch.setenv("HCP_RING_IMPL", "hip")
    o, lse = rb._attn(q, k, v, scale_for(128), 0)
    monkeypatch.setenv("HCP_RING_MERGE", "torch")
    with pytest.raises(NotImplementedError):
        rb._merge(o, lse, o, lse)
    assert rb.IMPL_STATS["attn_torch"] == 0 and rb.IMPL_STATS["merge_torch"] == 0
    assert rb.IMPL_STATS["attn_hip"] == 1 and rb.IMPL_STATS["merge_hip"] == 0
