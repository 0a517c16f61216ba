"""GPU parity of sliding-window attention (the window of _attn_with_lse,
ring_backend.py:372,397-398: query i at p = offset + i sees keys
p - window < j <= p) on the prefill kernel -- single segment and varlen over
the paged cache -- against the oracle, whose window the CPU tests pin to
float64 brute force and closed forms."""

import pytest
import torch

from hcp_vllm_plugin_amd import ring_attn_with_lse
from hcp_vllm_plugin_amd.varlen import (
    PagedCache,
    make_entry,
    segment_paged,
    varlen_attn_with_lse,
)
from oracle import ring_oracle as orc
from tests._util import LSE_TOL, OUT_TOL, max_err, randn, scale_for

pytestmark = pytest.mark.gpu

CASES = [
    # (tq, tk, offset, window)
    (128, 128, 0, 1),
    (300, 1000, 700, 64),
    (256, 4096, 3840, 100),
    (1000, 1000, 0, 257),
    (64, 500, 436, 1000),     # window wider than the keys: no effect
    (70, 100, -5, 10),        # negative offset: first rows see nothing
    (513, 2000, 1487, 130),   # ragged last tile, window across tiles
    (33, 5000, 4967, 4000),
    (200, 700, 900, 50),      # offset past the keys: rows near the end only
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("tq,tk,off,w", CASES)
def test_window_single_segment(dev, tq, tk, off, w, dtype):
    gen = torch.Generator().manual_seed(tq + 3 * tk + w)
    q = randn(gen, (tq, 28, 128), dtype)
    k = randn(gen, (tk, 4, 128), dtype)
    v = randn(gen, (tk, 4, 128), dtype)
    o, lse = ring_attn_with_lse(q.to(dev), k.to(dev), v.to(dev), scale_for(128), off, w)
    torch.cuda.synchronize()
    ro, rl = orc.attn_with_lse(q.float(), k.float(), v.float(), scale_for(128), off, w)
    assert max_err(o, ro) <= OUT_TOL[dtype]
    assert max_err(lse, rl) <= LSE_TOL


def test_window_d64_fp16_and_noncausal_ignores_it(dev):
    gen = torch.Generator().manual_seed(7)
    q = randn(gen, (200, 14, 64), torch.float16)
    k = randn(gen, (900, 2, 64), torch.float16)
    v = randn(gen, (900, 2, 64), torch.float16)
    o, lse = ring_attn_with_lse(q.to(dev), k.to(dev), v.to(dev), 0.125, 700, 33)
    ro, rl = orc.attn_with_lse(q.float(), k.float(), v.float(), 0.125, 700, 33)
    assert max_err(o, ro) <= 2e-3 and max_err(lse, rl) <= LSE_TOL
    # the peer pass is non-causal: a window has no effect there (:828-830)
    o1, l1 = ring_attn_with_lse(q.to(dev), k.to(dev), v.to(dev), 0.125, None, 33)
    o2, l2 = ring_attn_with_lse(q.to(dev), k.to(dev), v.to(dev), 0.125, None)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(l1, l2)


@pytest.mark.parametrize("bs", [16, 4])
@pytest.mark.parametrize("layout", ["v031", "v023"])
@pytest.mark.parametrize("w", [1, 50, 333])
def test_window_varlen_paged(dev, layout, w, bs):
    """Several requests over the paged cache in one causal launch, each with
    its own offset (and a segment starting mid-block), one window; block
    size 4 runs through the device gather."""
    gen = torch.Generator().manual_seed(40 + w)
    h, hkv, d = 28, 4, 128
    reqs = [(300, 300, 0), (17, 517, 0), (129, 1000, 200), (64, 64, 0), (200, 900, 0)]
    nb = sum(-(-(s + tk) // bs) for _, tk, s in reqs) + 2
    cache = randn(gen, (nb, hkv, bs, 2 * d) if layout == "v031" else (nb, 2, bs, hkv, d),
                  torch.bfloat16)
    perm = torch.randperm(nb, generator=gen).to(torch.int32)
    q = randn(gen, (sum(r[0] for r in reqs), h, d), torch.bfloat16)
    cd = cache.to(dev)
    pc = PagedCache.from_tensor(cd)
    rows, entries, o0 = [], [], 0
    qs = 0
    for tq, tk, start in reqs:
        nbk = -(-(start + tk) // bs)
        row = perm[o0:o0 + nbk].clone()
        o0 += nbk
        rows.append(row)
        rd = row.to(dev)
        entries.append(make_entry(qs, tq, segment_paged(pc, rd, start, tk), tk - tq))
        qs += tq
    out, lse = varlen_attn_with_lse(q.to(dev), entries, True, hkv, scale_for(d), window=w)
    torch.cuda.synchronize()
    qs = 0
    for (tq, tk, start), row in zip(reqs, rows):
        kk, vv = orc.gather_paged(cache.float(), row, start, tk, layout)
        ro, rl = orc.attn_with_lse(q[qs:qs + tq].float(), kk, vv, scale_for(d), tk - tq, w)
        assert max_err(out[qs:qs + tq], ro) <= OUT_TOL[torch.bfloat16]
        assert max_err(lse[:, qs:qs + tq], rl) <= LSE_TOL
        qs += tq
