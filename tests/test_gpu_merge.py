"""GPU parity: merge_attn_states / merge_pair (hcp_merge_attn_states).

Mirrors validate_ring_triton_kernel.py:63-94: the HIP merge against the torch
merge on kernel outputs (gate 2e-3), and the two-chunk ring merge of local
causal + peer non-causal against full causal attention (gate 3e-3), both with
the prefix = peer, suffix = local order of ring_backend.py:354.
"""

import pytest
import torch

from hcp_vllm_plugin_amd import merge_attn_states, merge_pair, ring_attn_with_lse
from oracle import ring_oracle as orc
from tests._util import max_err, randn, scale_for

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("odt", [torch.float16, torch.bfloat16, torch.float32])
def test_merge_vs_oracle(dev, odt):
    gen = torch.Generator().manual_seed(31)
    t, h, d = 777, 28, 128
    op = randn(gen, (t, h, d), odt)
    os_ = randn(gen, (t, h, d), odt)
    lp = torch.randn(h, t, generator=gen) * 4
    ls = torch.randn(h, t, generator=gen) * 4
    out = torch.empty(t, h, d, dtype=odt, device=dev)
    out_lse = torch.empty(h, t, device=dev)
    merge_attn_states(out, op.to(dev), lp.to(dev), os_.to(dev), ls.to(dev), out_lse)
    torch.cuda.synchronize()
    ro, rl = orc.merge_pair(op.float(), lp, os_.float(), ls)
    # inputs are N(0,1) partials, so |out| reaches ~4: allow the output
    # dtype's own rounding (half an ulp, relative) on top of the absolute gate
    tol = {torch.float16: 2e-3, torch.bfloat16: 1.5e-2, torch.float32: 1e-5}[odt]
    rtol = {torch.float16: 2 ** -11, torch.bfloat16: 2 ** -8, torch.float32: 1e-6}[odt]
    torch.testing.assert_close(out.float().cpu(), ro, atol=tol, rtol=rtol)
    assert max_err(out_lse, rl) <= 1e-5


def test_merge_mixed_dtypes_and_strides(dev):
    gen = torch.Generator().manual_seed(32)
    t, h, d = 100, 8, 64
    op = randn(gen, (t, h, d), torch.float32).to(dev)
    big = randn(gen, (t, h + 4, d), torch.bfloat16).to(dev)
    os_ = big[:, 2:2 + h]  # strided view
    lp = (torch.randn(h, t, generator=gen) * 3).to(dev)
    ls = (torch.randn(h, t, generator=gen) * 3).to(dev)
    out = torch.empty(t, h, d, dtype=torch.float16, device=dev)
    merge_attn_states(out, op, lp, os_, ls)
    torch.cuda.synchronize()
    ro = orc.lse_merge(op.cpu(), lp.cpu(), os_.float().cpu(), ls.cpu())
    assert max_err(out, ro) <= 2e-3


def test_merge_inf_handling(dev):
    t, h, d = 4, 2, 64
    op = torch.randn(t, h, d, device=dev)
    os_ = torch.randn(t, h, d, device=dev)
    lp = torch.zeros(h, t, device=dev)
    ls = torch.zeros(h, t, device=dev)
    lp[0, 0] = float("inf")     # read as -inf: suffix only
    ls[1, 1] = float("-inf")    # prefix only
    lp[0, 2] = float("-inf")
    ls[0, 2] = float("-inf")    # both empty: 0 / -inf
    os_[0, 1] = float("nan")    # weight-0 side is not read
    ls[1, 0] = float("-inf")
    out = torch.empty_like(op)
    out_lse = torch.empty(h, t, device=dev)
    merge_attn_states(out, op, lp, os_, ls, out_lse)
    torch.cuda.synchronize()
    assert torch.equal(out[0, 0], os_[0, 0])
    assert torch.equal(out[1, 1], op[1, 1])
    assert torch.all(out[2, 0] == 0) and out_lse[0, 2] == float("-inf")
    assert torch.equal(out[0, 1], op[0, 1])
    assert not torch.isnan(out).any()


@pytest.mark.parametrize("dtype,h,hkv,d", [(torch.float16, 14, 2, 64),
                                           (torch.bfloat16, 28, 4, 128)])
def test_ring_two_chunk_merge_equals_full(dev, dtype, h, hkv, d):
    """validate_ring_triton_kernel.py:80-94 on the HIP kernels."""
    gen = torch.Generator().manual_seed(33)
    tk_full, split, tq = 2048, 1024, 512
    q = randn(gen, (tq, h, d), dtype)
    k = randn(gen, (tk_full, hkv, d), dtype)
    v = randn(gen, (tk_full, hkv, d), dtype)
    scale = scale_for(d)
    o_full, lse_full = orc.attn_with_lse(q.float(), k.float(), v.float(), scale, tk_full - tq)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    o_loc, lse_loc = ring_attn_with_lse(qd, kd[split:], vd[split:], scale, tk_full - tq - split)
    o_peer, lse_peer = ring_attn_with_lse(qd, kd[:split], vd[:split], scale, None)
    o_m = torch.empty_like(o_loc)
    merge_attn_states(o_m, o_peer, lse_peer, o_loc, lse_loc)
    o_p, lse_p = merge_pair(o_peer, lse_peer, o_loc, lse_loc)
    torch.cuda.synchronize()
    tol = 3e-3 if dtype == torch.float16 else 1.5e-2
    assert max_err(o_m, o_full) <= tol
    assert torch.equal(o_m, o_p)
    assert max_err(lse_p, lse_full) <= 1e-3
