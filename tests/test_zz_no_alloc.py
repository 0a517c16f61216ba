"""GPU parity of the allocation-free decode entry point.

``hcp_decode_splitkv_noalloc`` runs the split-KV decode with its fp32 split
partials in the library's fixed per-GPU scratch instead of a caller
workspace.  Its output and LSE must equal ``hcp_decode_splitkv``'s on the same
plan bit for bit (same kernels, same arithmetic), on two calls in a row, the
second with a smaller batch (the scratch keeps the first call's partials);
and a plan whose partials exceed the scratch is refused on the host before
anything is launched.  Both entry points are called through the C ABI
(``DecodeBatch.run`` binds them with ctypes).
"""

import pytest
import torch

from hcp_vllm_plugin_amd import _lib
from hcp_vllm_plugin_amd.varlen import (
    DecodeBatch,
    PagedCache,
    head_major,
    segment_contiguous,
    segment_paged,
)
from tests._util import randn, scale_for

pytestmark = pytest.mark.gpu

H, HKV, D, BS = 28, 4, 128, 16


def _batch(dev, seqs, peer_len, loc_max, seed):
    gen = torch.Generator().manual_seed(seed)
    loc = torch.randint(1, loc_max + 1, (seqs,), generator=gen).tolist()
    blocks = [-(-n // BS) for n in loc]
    nb = sum(blocks) + 3
    cache = randn(gen, (nb, HKV, BS, 2 * D), torch.bfloat16).to(dev)
    perm = torch.randperm(nb, generator=gen).to(torch.int32)
    bt = torch.zeros(seqs, max(blocks), dtype=torch.int32)
    o = 0
    for r, n in enumerate(blocks):
        bt[r, :n] = perm[o:o + n]
        o += n
    bt = bt.to(dev)
    kp = head_major(randn(gen, (seqs * peer_len, HKV, D), torch.bfloat16).to(dev))
    vp = head_major(randn(gen, (seqs * peer_len, HKV, D), torch.bfloat16).to(dev))
    q = randn(gen, (seqs, H, D), torch.bfloat16).to(dev)
    pc = PagedCache.from_tensor(cache)
    segs = [[segment_contiguous(kp, vp, r * peer_len, peer_len),
             segment_paged(pc, bt[r], 0, loc[r])] for r in range(seqs)]
    return q, DecodeBatch(segs, H, HKV, D, dev), (cache, kp, vp, bt)


def test_noalloc_matches_workspace_entry(dev):
    scale = scale_for(D)
    # first call: 24 sequences of 6000 peer + up to 900 local keys; second: 5
    # sequences, shorter (fewer splits than the first left in the scratch)
    for seqs, peer_len, loc_max, seed in ((24, 6000, 900, 11), (5, 1500, 300, 12)):
        q, batch, keep = _batch(dev, seqs, peer_len, loc_max, seed)
        assert batch.ws_bytes <= _lib.NOALLOC_SCRATCH_BYTES
        out_ws = torch.empty_like(q)
        lse_ws = torch.empty(H, seqs, dtype=torch.float32, device=dev)
        batch.run(q, out_ws, lse_ws, scale)
        out_na = torch.full_like(q, float("nan"))
        lse_na = torch.full((H, seqs), float("nan"), dtype=torch.float32, device=dev)
        batch.run(q, out_na, lse_na, scale, noalloc=True)
        torch.cuda.synchronize()
        assert torch.isfinite(out_ws.float()).all() and torch.isfinite(lse_ws).all()
        assert torch.equal(out_na, out_ws), (seqs, (out_na.float() - out_ws.float()).abs().max())
        assert torch.equal(lse_na, lse_ws), seqs
        del keep


def test_noalloc_rejects_plans_beyond_scratch(dev):
    """1172 splits x 28 heads of fp32 partials need more than 16 MiB (1161 fit): refused
    with EWORKSPACE on the host, the output left as it was."""
    gen = torch.Generator().manual_seed(13)
    n = 1172 * 64
    k = randn(gen, (n, HKV, D), torch.bfloat16).to(dev)
    v = randn(gen, (n, HKV, D), torch.bfloat16).to(dev)
    q = randn(gen, (1, H, D), torch.bfloat16).to(dev)
    batch = DecodeBatch([[segment_contiguous(k, v)]], H, HKV, D, dev, split_tokens=64)
    assert batch.num_splits == 1172 and batch.ws_bytes > _lib.NOALLOC_SCRATCH_BYTES
    out = torch.zeros_like(q)
    with pytest.raises(RuntimeError, match="EWORKSPACE"):
        batch.run(q, out, None, scale_for(D), noalloc=True)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out) == 0
