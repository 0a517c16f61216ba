"""GPU parity: ring_attn_with_lse (hcp_attn_fwd_lse) against the CPU oracle.

Cases follow the reference's kernel probe (validate_ring_triton_kernel.py:41-61:
six (Tq, Tk, offset) shapes, causal and non-causal, H=14 / Hkv=2 / D=64 fp16,
gate 2e-3 on out and LSE) and repeat them at the Qwen2.5-7B attention shape
(28 / 4 / 128) in bf16 and fp16, plus logit outliers, ragged and empty
segments, negative offsets, strided inputs, and scores that rise far above
(or fall far below) a row's first tile.
"""

import pytest
import torch

from hcp_vllm_plugin_amd import ring_attn_with_lse
from hcp_vllm_plugin_amd.ring_attn import COPY_STATS
from oracle import ring_oracle as orc
from tests._util import LSE_TOL, OUT_TOL, max_err, outlier_k, randn, scale_for

pytestmark = pytest.mark.gpu

REF_CASES = [(1, 1, 0), (1, 512, 511), (37, 37, 0), (37, 512, 475), (512, 512, 0),
             (512, 2048, 1536)]


def _run(dev, tq, tk, off, h, hkv, d, dtype, seed, outliers=False):
    gen = torch.Generator().manual_seed(seed)
    q = randn(gen, (tq, h, d), dtype)
    k = randn(gen, (tk, hkv, d), dtype)
    v = randn(gen, (tk, hkv, d), dtype)
    if outliers:
        k = outlier_k(k, gen).to(dtype)
    scale = scale_for(d)
    o, lse = ring_attn_with_lse(q.to(dev), k.to(dev), v.to(dev), scale, off)
    torch.cuda.synchronize()
    ro, rl = orc.attn_with_lse(q.float(), k.float(), v.float(), scale, off)
    assert o.dtype == dtype and o.shape == (tq, h, d)
    assert lse.dtype == torch.float32 and lse.shape == (h, tq)
    return max_err(o, ro), max_err(lse, rl)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("tq,tk,off", REF_CASES)
def test_reference_probe_cases_fp16_d64(dev, tq, tk, off, causal):
    eo, el = _run(dev, tq, tk, off if causal else None, 14, 2, 64, torch.float16, seed=tq + tk)
    assert eo <= 2e-3, eo
    assert el <= 2e-3, el


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("tq,tk,off", REF_CASES)
def test_reference_cases_qwen7b_shape(dev, tq, tk, off, causal, dtype):
    eo, el = _run(dev, tq, tk, off if causal else None, 28, 4, 128, dtype, seed=3 * tq + tk)
    assert eo <= OUT_TOL[dtype], eo
    assert el <= LSE_TOL, el


@pytest.mark.parametrize("tq,tk,off", [(300, 700, 400), (129, 1000, None), (256, 256, 0)])
def test_logit_outliers_bf16(dev, tq, tk, off):
    eo, el = _run(dev, tq, tk, off, 28, 4, 128, torch.bfloat16, seed=11, outliers=True)
    assert eo <= OUT_TOL[torch.bfloat16], eo
    assert el <= LSE_TOL, el


@pytest.mark.parametrize("tq,tk,off", [(200, 63, None), (65, 1, 0), (130, 129, -1),
                                       (70, 100, -40), (3, 5000, 4997)])
def test_ragged_and_negative_offsets(dev, tq, tk, off):
    eo, el = _run(dev, tq, tk, off, 8, 2, 128, torch.bfloat16, seed=tq * 7 + tk)
    assert eo <= OUT_TOL[torch.bfloat16], eo
    assert el <= LSE_TOL, el


def test_empty_kv_segment(dev):
    q = torch.randn(70, 28, 128, device=dev).to(torch.bfloat16)
    k = torch.zeros(0, 4, 128, device=dev, dtype=torch.bfloat16)
    o, lse = ring_attn_with_lse(q, k, k, 0.088, None)
    torch.cuda.synchronize()
    assert torch.all(o == 0)
    assert torch.all(torch.isneginf(lse))


def test_empty_query(dev):
    q = torch.zeros(0, 28, 128, device=dev, dtype=torch.bfloat16)
    k = torch.randn(10, 4, 128, device=dev).to(torch.bfloat16)
    o, lse = ring_attn_with_lse(q, k, k, 0.088, 0)
    assert o.shape == (0, 28, 128) and lse.shape == (28, 0)


def test_strided_qkv_views(dev):
    """q/k/v as views into one packed [T, H + 2*Hkv, D] projection output."""
    gen = torch.Generator().manual_seed(21)
    t, h, hkv, d = 333, 28, 4, 128
    qkv = randn(gen, (t, h + 2 * hkv, d), torch.bfloat16).to(dev)
    q, k, v = qkv[:, :h], qkv[:, h:h + hkv], qkv[:, h + hkv:]
    before = dict(COPY_STATS)
    o, lse = ring_attn_with_lse(q, k, v, scale_for(d), 0)
    torch.cuda.synchronize()
    ro, rl = orc.attn_with_lse(q.float().cpu(), k.float().cpu(), v.float().cpu(), scale_for(d), 0)
    assert max_err(o, ro) <= OUT_TOL[torch.bfloat16]
    assert max_err(lse, rl) <= LSE_TOL
    # these views are loadable in place: no layout copy
    assert COPY_STATS == before


def test_unloadable_layout_is_copied_and_counted(dev):
    """A head stride that is not a multiple of 8 elements is copied contiguous
    first (the reference copies every input, ring_backend.py:328); the copy
    is counted with its bytes, and the result matches the oracle."""
    gen = torch.Generator().manual_seed(22)
    t, h, hkv, d = 200, 28, 4, 128
    qpad = randn(gen, (t, h, d + 4), torch.bfloat16).to(dev)
    q = qpad[..., :d]  # head stride d + 4: not loadable in place
    k = randn(gen, (t, hkv, d), torch.bfloat16).to(dev)
    v = randn(gen, (t, hkv, d), torch.bfloat16).to(dev)
    before = dict(COPY_STATS)
    o, lse = ring_attn_with_lse(q, k, v, scale_for(d), 0)
    torch.cuda.synchronize()
    assert COPY_STATS["tensors"] == before["tensors"] + 1
    assert COPY_STATS["bytes"] == before["bytes"] + t * h * d * 2
    ro, rl = orc.attn_with_lse(q.float().cpu(), k.float().cpu(), v.float().cpu(), scale_for(d), 0)
    assert max_err(o, ro) <= OUT_TOL[torch.bfloat16]
    assert max_err(lse, rl) <= LSE_TOL


def test_invalid_arguments_raise(dev):
    q = torch.randn(8, 6, 128, device=dev).to(torch.bfloat16)
    k = torch.randn(8, 4, 128, device=dev).to(torch.bfloat16)
    with pytest.raises(ValueError):
        ring_attn_with_lse(q, k, k, 0.1, 0)  # 6 % 4 != 0
    q = torch.randn(8, 4, 264, device=dev).to(torch.bfloat16)
    k = torch.randn(8, 4, 264, device=dev).to(torch.bfloat16)
    with pytest.raises(RuntimeError, match="EUNSUPPORTED"):
        ring_attn_with_lse(q, k, k, 0.1, 0)  # head_dim above 256 not built


def test_deterministic_repeat(dev):
    gen = torch.Generator().manual_seed(5)
    q = randn(gen, (500, 28, 128), torch.bfloat16).to(dev)
    k = randn(gen, (900, 4, 128), torch.bfloat16).to(dev)
    v = randn(gen, (900, 4, 128), torch.bfloat16).to(dev)
    a = ring_attn_with_lse(q, k, v, 0.088, 400)
    b = ring_attn_with_lse(q, k, v, 0.088, 400)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def _drift_inputs(gen, tq, tk, h, hkv, d, dtype, slope, spike):
    """Queries and keys sharing one direction u: key j carries slope*j/64 of it
    (scores drift by about slope log2 units per 64-key tile), and key `spike`
    (if any) 40 more."""
    u = torch.randn(d, generator=gen)
    u /= u.norm()
    q = torch.randn(tq, h, d, generator=gen) + 8.0 * u
    w = slope * torch.arange(tk, dtype=torch.float32) / 64.0
    if spike is not None:
        w[spike] += 40.0
    k = torch.randn(tk, hkv, d, generator=gen) + w[:, None, None] * u
    v = torch.randn(tk, hkv, d, generator=gen)
    return q.to(dtype), k.to(dtype), v.to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("off", [None, 1500])
@pytest.mark.parametrize("slope,spike", [(2.0, None), (-2.0, None), (0.0, 1500)])
def test_scores_far_above_first_tile(dev, dtype, off, slope, spike):
    """Rows whose later scores exceed their first tile's maximum by far more
    than the exponent headroom (rising scores, one late spike) must be
    rescaled on the way; falling scores underflow harmlessly."""
    tq, tk, h, hkv, d = 300, 2048, 8, 2, 128
    gen = torch.Generator().manual_seed(int(slope * 10) + 7 * (off or 0) + 3)
    q, k, v = _drift_inputs(gen, tq, tk, h, hkv, d, dtype, slope, spike)
    scale = scale_for(d)
    # the inputs do exercise the rescale: against the first tile's maximum,
    # some later score is more than 12 log2 units higher in every row
    s = torch.einsum("qhd,khd->hqk", q.float(), k.float().repeat_interleave(h // hkv, 1))
    s = s * scale * 1.4426950408889634
    if off is not None:
        s = s.masked_fill(torch.arange(tk)[None, :] > off + torch.arange(tq)[:, None], -torch.inf)
    rise = (s.amax(-1) - s[..., :64].amax(-1)).amin().item()
    assert (rise > 12.0) == (slope > 0 or spike is not None), rise
    o, lse = ring_attn_with_lse(q.to(dev), k.to(dev), v.to(dev), scale, off)
    torch.cuda.synchronize()
    ro, rl = orc.attn_with_lse(q.float(), k.float(), v.float(), scale, off)
    assert max_err(o, ro) <= OUT_TOL[dtype]
    assert max_err(lse, rl) <= LSE_TOL
