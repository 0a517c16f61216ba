"""GPU parity at head_dims other than 64 / 128.

The reference kernel takes any head_dim (BLOCK_D = next power of two with the
columns past head_dim masked, ring_triton_attn.py:69-78,201).  The HIP
kernels compute in 64, 128 or 256 columns and treat the tail as zeros: every
entry point is checked here against the oracle at head_dims that are
multiples of 8 up to 256 other than 64 and 128 (256 itself runs the
one-wave-per-SIMD prefill and two-wave decode instantiations) -- the plain and
merging forward passes, the paged varlen pass, the split-KV decode, the paged
KV write and the backend's forward.  Rows are
packed at their true width ([T, H, head_dim], stride head_dim), so a load
past a row's end would read the neighbouring head or token and show.
"""

import types

import pytest
import torch

from hcp_vllm_plugin_amd import merge_attn_states, ring_attn_merged, ring_attn_with_lse
from hcp_vllm_plugin_amd import ring_backend as rb
from hcp_vllm_plugin_amd.kv_cache import reshape_and_cache
from hcp_vllm_plugin_amd.varlen import (
    PagedCache, make_entry, segment_contiguous, segment_paged, varlen_attn_with_lse)
from oracle import ring_oracle as orc
from tests._util import LSE_TOL, OUT_TOL, max_err, outlier_k, randn, scale_for
from tests.test_gpu_decode import _case as decode_case
from tests.test_gpu_kv_cache import _case as cache_case
from tests.test_gpu_varlen import _build as varlen_build

pytestmark = pytest.mark.gpu

DIMS = [8, 40, 72, 80, 96, 112, 136, 200, 256]


@pytest.mark.parametrize("d", DIMS)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("off", [None, 400, -30])
def test_forward_head_dims(dev, d, dtype, off):
    gen = torch.Generator().manual_seed(d + (off or 0))
    tq, tk, h, hkv = 300, 700, 14, 2
    q = randn(gen, (tq, h, d), dtype)
    k = outlier_k(randn(gen, (tk, hkv, d), dtype), gen, n_channels=min(4, d)).to(dtype)
    v = randn(gen, (tk, hkv, d), dtype)
    scale = scale_for(d)
    o, lse = ring_attn_with_lse(q.to(dev), k.to(dev), v.to(dev), scale, off)
    torch.cuda.synchronize()
    ro, rl = orc.attn_with_lse(q.float(), k.float(), v.float(), scale, off)
    assert o.shape == (tq, h, d)
    assert max_err(o, ro) <= OUT_TOL[dtype], max_err(o, ro)
    assert max_err(lse, rl) <= LSE_TOL


@pytest.mark.parametrize("d", [1, 3, 20, 100, 130, 250])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_kernel_contract_any_head_dim(dev, d, dtype):
    """head_dims that are not a multiple of 8 (the reference's kernel takes any,
    with masked BLOCK_D columns, ring_triton_attn.py:69-78,201): the pass
    (causal and not), the merging pass and merge_attn_states / merge_pair run
    on zero-padded copies and return [T, H, d] results equal to the oracle's."""
    from hcp_vllm_plugin_amd import merge_pair

    gen = torch.Generator().manual_seed(900 + d)
    tq, tk, h, hkv = 150, 333, 6, 2
    q = randn(gen, (tq, h, d), dtype)
    k = randn(gen, (tk, hkv, d), dtype)
    v = randn(gen, (tk, hkv, d), dtype)
    kp, vp = randn(gen, (200, hkv, d), dtype), randn(gen, (200, hkv, d), dtype)
    scale = scale_for(d)
    qd, kd, vd, kpd, vpd = (t.to(dev) for t in (q, k, v, kp, vp))
    o_l, l_l = ring_attn_with_lse(qd, kd, vd, scale, tk - tq)
    o_p, l_p = ring_attn_with_lse(qd, kpd, vpd, scale, None)
    out = torch.empty_like(o_l)
    merge_attn_states(out, o_p, l_p, o_l, l_l)
    mo, ml = merge_pair(o_p, l_p, o_l, l_l)
    fused = ring_attn_merged(qd, kd, vd, scale, tk - tq, o_p, l_p)
    torch.cuda.synchronize()
    assert o_l.shape == (tq, h, d) and out.shape == (tq, h, d) and fused.shape == (tq, h, d)
    rl, rll = orc.attn_with_lse(q.float(), k.float(), v.float(), scale, tk - tq)
    rp, rpl = orc.attn_with_lse(q.float(), kp.float(), vp.float(), scale, None)
    rm = orc.lse_merge(rl, rll, rp, rpl)
    assert max_err(o_l, rl) <= OUT_TOL[dtype] and max_err(l_l, rll) <= LSE_TOL
    assert max_err(o_p, rp) <= OUT_TOL[dtype] and max_err(l_p, rpl) <= LSE_TOL
    assert max_err(out, rm) <= OUT_TOL[dtype]
    assert torch.equal(mo, out) and torch.equal(fused, out)
    assert max_err(ml, torch.logaddexp(rll, rpl)) <= LSE_TOL


@pytest.mark.parametrize("d", [40, 96, 256])
def test_merged_pass_head_dims(dev, d):
    """Local pass merging a peer partial (the acc epilogue) equals pass +
    merge_attn_states bit for bit, and the oracle's merge within tolerance."""
    gen = torch.Generator().manual_seed(70 + d)
    tq, h, hkv, dtype = 260, 28, 4, torch.bfloat16
    q = randn(gen, (tq, h, d), dtype).to(dev)
    kl, vl = (randn(gen, (tq, hkv, d), dtype).to(dev) for _ in range(2))
    kp, vp = (randn(gen, (333, hkv, d), dtype).to(dev) for _ in range(2))
    scale = scale_for(d)
    o_p, l_p = ring_attn_with_lse(q, kp, vp, scale, None)
    o_l, l_l = ring_attn_with_lse(q, kl, vl, scale, 0)
    ref = torch.empty_like(q)
    merge_attn_states(ref, o_p, l_p, o_l, l_l)
    lse = torch.empty_like(l_p)
    out = ring_attn_merged(q, kl, vl, scale, 0, o_p, l_p, output_lse=lse)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    rl, rll = orc.attn_with_lse(q.float().cpu(), kl.float().cpu(), vl.float().cpu(), scale, 0)
    rp, rpl = orc.attn_with_lse(q.float().cpu(), kp.float().cpu(), vp.float().cpu(), scale, None)
    assert max_err(out, orc.lse_merge(rl, rll, rp, rpl)) <= OUT_TOL[dtype]


@pytest.mark.parametrize("layout", ["v031", "v023"])
@pytest.mark.parametrize("d", [80, 40, 192, 256])
def test_varlen_paged_head_dims(dev, layout, d):
    h, hkv, bs, dtype = 28, 4, 16, torch.bfloat16
    lens, peers = [300, 1, 129, 64], [512, 48, 0, 32]
    cache, bt, q, peer = varlen_build(dev, layout, lens, peers, h, hkv, d, dtype, bs, seed=42)
    cd, btd, qd, pd = cache.to(dev), bt.to(dev), q.to(dev), peer.to(dev)
    pc = PagedCache.from_tensor(cd)
    pk, pv = pd[:, 0], pd[:, 1]
    loc_e, peer_e = [], []
    qs = ps = 0
    for r, (L, P) in enumerate(zip(lens, peers)):
        loc_e.append(make_entry(qs, L, segment_paged(pc, btd[r], P, L), 0))
        peer_e.append(make_entry(qs, L, segment_contiguous(pk, pv, ps, P), 0))
        qs += L
        ps += P
    scale = scale_for(d)
    o_loc, lse_loc = varlen_attn_with_lse(qd, loc_e, True, hkv, scale)
    o_peer, lse_peer = varlen_attn_with_lse(qd, peer_e, False, hkv, scale)
    torch.cuda.synchronize()
    qs = ps = 0
    for r, (L, P) in enumerate(zip(lens, peers)):
        qr = q[qs:qs + L].float()
        kl, vl = orc.gather_paged(cache.float(), bt[r], P, L, layout)
        rl, rll = orc.attn_with_lse(qr, kl, vl, scale, 0)
        rp, rpl = orc.attn_with_lse(qr, peer[ps:ps + P, 0].float(), peer[ps:ps + P, 1].float(),
                                    scale, None)
        sl = slice(qs, qs + L)
        assert max_err(o_loc[sl], rl) <= OUT_TOL[dtype], r
        assert max_err(lse_loc[:, sl], rll) <= LSE_TOL, r
        assert max_err(o_peer[sl], rp) <= OUT_TOL[dtype], r
        assert max_err(lse_peer[:, sl], rpl) <= LSE_TOL, r
        qs += L
        ps += P


@pytest.mark.parametrize("h,hkv,d,dtype", [(28, 4, 96, torch.bfloat16),
                                          (14, 2, 80, torch.float16),
                                          (32, 1, 40, torch.bfloat16),
                                          (16, 8, 256, torch.bfloat16),
                                          (24, 2, 256, torch.float16),
                                          (8, 1, 184, torch.bfloat16)])
@pytest.mark.parametrize("split", [None, 64])
def test_decode_head_dims(dev, h, hkv, d, dtype, split):
    decode_case(dev, h, hkv, d, dtype, peer_lens=[1500, 0, 64], loc_lens=[300, 800, 1],
                bs=16, seed=80 + d, split=split)


@pytest.mark.parametrize("layout", ["v031", "v023"])
@pytest.mark.parametrize("d", [96, 40, 200, 256])
def test_cache_write_head_dims(dev, layout, d):
    cache, key, value, slots = cache_case(layout, torch.bfloat16, torch.int64, 333, 41, 16, 4,
                                          d, 90 + d)
    ref = cache.clone()
    orc.kv_cache_update(key, value, ref, slots, layout)
    dcache = cache.to(dev)
    reshape_and_cache(key.to(dev), value.to(dev), dcache, slots.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(dcache.cpu(), ref)


@pytest.mark.parametrize("d", [96, 80, 256])
def test_backend_forward_head_dims(dev, d):
    """HcpRingAttentionImpl.forward at head_size d: prefill rows (with a
    staged peer chunk) and a decode row, paged cache [nb, Hkv, 16, 2d]."""
    rb.clear_peer_kv()
    gen = torch.Generator().manual_seed(100 + d)
    h, hkv, bs, dtype = 28, 4, 16, torch.bfloat16
    reqs = [(200, 200 + 64), (1, 700), (77, 77)]
    seq_lens = [tk for _, tk in reqs]
    qsl = [0]
    for tq, _ in reqs:
        qsl.append(qsl[-1] + tq)
    nb = sum(-(-tk // bs) for tk in seq_lens) + 4
    cache = randn(gen, (nb, hkv, bs, 2 * d), dtype)
    blocks = [-(-tk // bs) for tk in seq_lens]
    perm = torch.randperm(nb, generator=gen).to(torch.int32)
    bt = torch.zeros(len(reqs), max(blocks) + 1, dtype=torch.int32)
    o = 0
    for r, n in enumerate(blocks):
        bt[r, :n] = perm[o:o + n]
        o += n
    query = randn(gen, (qsl[-1], h, d), dtype)
    layer = types.SimpleNamespace(layer_name="model.layers.0.self_attn.attn")
    kp, vp = randn(gen, (96, hkv, d), dtype), randn(gen, (96, hkv, d), dtype)
    rb.stage_peer_kv("c0", layer.layer_name, kp.to(dev), vp.to(dev))
    rb.map_request_peer(int(bt[0, 0]), ["c0"])
    impl = rb.HcpRingAttentionImpl(h, d, scale_for(d), hkv)
    meta = types.SimpleNamespace(
        num_actual_tokens=qsl[-1],
        query_start_loc=torch.tensor(qsl, dtype=torch.int32, device=dev),
        seq_lens=torch.tensor(seq_lens, dtype=torch.int32, device=dev),
        block_table=bt.to(dev))
    out = torch.empty(qsl[-1], h, d, dtype=dtype, device=dev)
    try:
        impl.forward(layer, query.to(dev), None, None, cache.to(dev), meta, out)
        torch.cuda.synchronize()
    finally:
        rb.clear_peer_kv()
    ref = orc.ring_forward(query.float(), cache.float(), "v031", qsl, seq_lens, bt, scale_for(d),
                           peers=[(kp.float(), vp.float()), None, None],
                           out_dtype=torch.float32)
    assert max_err(out, ref) <= OUT_TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("off", [None, 1500])
@pytest.mark.parametrize("slope,spike", [(2.0, None), (0.0, 1500)])
def test_rescale_path_d256(dev, dtype, off, slope, spike):
    """Scores rising far above every row's first tile at head_dim 256: the
    rescale of the output accumulator, which at this width lives in AGPRs,
    runs on most rows (inputs as in test_gpu_attn's drift cases)."""
    from tests.test_gpu_attn import _drift_inputs

    tq, tk, h, hkv, d = 300, 2048, 8, 2, 256
    gen = torch.Generator().manual_seed(int(slope * 10) + 7 * (off or 0) + 256)
    q, k, v = _drift_inputs(gen, tq, tk, h, hkv, d, dtype, slope, spike)
    scale = scale_for(d)
    o, lse = ring_attn_with_lse(q.to(dev), k.to(dev), v.to(dev), scale, off)
    torch.cuda.synchronize()
    ro, rl = orc.attn_with_lse(q.float(), k.float(), v.float(), scale, off)
    assert max_err(o, ro) <= OUT_TOL[dtype]
    assert max_err(lse, rl) <= LSE_TOL


def test_ring_step_d256_full_size(dev):
    """The head_dim 256 bench shape (16 / 8 heads, bf16): the 8192-key peer
    pass, then the 8192-key local causal pass merging it; every row of out and
    LSE against the oracle's ring step, and the whole output against one
    causal pass over [peer; local] (the ring step's identity)."""
    from tests.test_gpu_fullsize import _oracle_ring

    h, hkv, d, n = 16, 8, 256, 8192
    g = torch.Generator(device=dev).manual_seed(256)
    ch = torch.randperm(d, generator=torch.Generator().manual_seed(3))[:4]

    def draw(shape, outlier=False):
        x = torch.randn(*shape, generator=g, device=dev)
        if outlier:
            x[..., ch] *= 8.0
        return x.to(torch.bfloat16)

    q = draw((n, h, d))
    kl, vl, kp, vp = draw((n, hkv, d), True), draw((n, hkv, d)), draw((n, hkv, d), True), draw((n, hkv, d))
    scale = scale_for(d)
    o_p, l_p = ring_attn_with_lse(q, kp, vp, scale, None)
    lse = torch.empty(h, n, dtype=torch.float32, device=dev)
    out = ring_attn_merged(q, kl, vl, scale, 0, o_p, l_p, output_lse=lse)
    kk, vv = torch.cat([kp, kl]), torch.cat([vp, vl])
    o1, l1 = ring_attn_with_lse(q, kk, vv, scale, n)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all() and torch.isfinite(lse).all()
    assert max_err(out, o1) <= 2 * OUT_TOL[torch.bfloat16]
    assert max_err(lse, l1) <= 2 * LSE_TOL
    ro, rl = _oracle_ring(q, kl, vl, kp, vp, scale, 0, hkv)
    assert max_err(out, ro) <= OUT_TOL[torch.bfloat16], max_err(out, ro)
    assert max_err(lse, rl) <= LSE_TOL, max_err(lse, rl)
