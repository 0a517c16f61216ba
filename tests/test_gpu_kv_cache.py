"""GPU parity: paged KV-cache write (hcp_reshape_and_cache) against the oracle's
restatement of do_kv_cache_update (ring_backend.py:501-539), bit-exact, for
both cache layouts, fp16 and bf16, int32 and int64 slot mappings, padded key
rows, padding (-1) slots, and strided key/value views.
"""

import pytest
import torch

from hcp_vllm_plugin_amd.kv_cache import reshape_and_cache
from oracle import ring_oracle as orc
from tests._util import randn

pytestmark = pytest.mark.gpu


def _case(layout, dtype, slot_dtype, n, nb, bs, hkv, d, seed, strided=False):
    gen = torch.Generator().manual_seed(seed)
    shape = (nb, 2, bs, hkv, d) if layout == "v023" else (nb, hkv, bs, 2 * d)
    cache = randn(gen, shape, dtype)
    if strided:  # key/value as views into a fused [N, 2, Hkv, D] buffer
        kv = randn(gen, (n + 5, 2, hkv, d), dtype)
        key, value = kv[:, 0], kv[:, 1]
    else:
        key, value = randn(gen, (n + 5, hkv, d), dtype), randn(gen, (n + 5, hkv, d), dtype)
    slots = torch.randperm(nb * bs, generator=gen)[:n].clone()
    if n > 4:
        slots[[1, n // 2]] = -1
    return cache, key, value, slots.to(slot_dtype)


@pytest.mark.parametrize("layout", ["v031", "v023"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("slot_dtype", [torch.int64, torch.int32])
def test_cache_write_bit_exact(dev, layout, dtype, slot_dtype):
    cache, key, value, slots = _case(layout, dtype, slot_dtype, 777, 97, 16, 4, 128, 31)
    ref = cache.clone()
    orc.kv_cache_update(key, value, ref, slots.long(), layout)
    dcache = cache.to(dev)
    reshape_and_cache(key.to(dev), value.to(dev), dcache, slots.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(dcache.cpu(), ref)


@pytest.mark.parametrize("layout", ["v031", "v023"])
def test_cache_write_small_shapes_and_views(dev, layout):
    # head_dim 64, block_size 1 and 32, strided key/value views, n = 1 (decode)
    for (n, nb, bs, hkv, d, strided) in [(1, 5, 16, 4, 128, False), (50, 70, 1, 2, 64, True),
                                         (130, 9, 32, 8, 128, True)]:
        cache, key, value, slots = _case(layout, torch.bfloat16, torch.int64, n, nb, bs, hkv, d,
                                         n, strided)
        ref = cache.clone()
        orc.kv_cache_update(key, value, ref, slots, layout)
        dcache = cache.to(dev)
        reshape_and_cache(key.to(dev), value.to(dev), dcache, slots.to(dev))
        torch.cuda.synchronize()
        assert torch.equal(dcache.cpu(), ref), (n, nb, bs, hkv, d, strided)


def test_cache_write_then_paged_read(dev):
    """Written along a block table, the cache feeds the paged local-segment
    reader: attention over it equals attention over the contiguous rows."""
    from hcp_vllm_plugin_amd import ring_attn_with_lse
    from hcp_vllm_plugin_amd.varlen import PagedCache, make_entry, segment_paged, varlen_attn_with_lse
    gen = torch.Generator().manual_seed(5)
    h, hkv, d, bs, n = 28, 4, 128, 16, 300
    nb = 40
    cache = torch.zeros(nb, hkv, bs, 2 * d, dtype=torch.bfloat16, device=dev)
    row = torch.randperm(nb, generator=gen).to(torch.int32)
    key = randn(gen, (n, hkv, d), torch.bfloat16).to(dev)
    value = randn(gen, (n, hkv, d), torch.bfloat16).to(dev)
    slots = torch.tensor([int(row[x // bs]) * bs + x % bs for x in range(n)], device=dev)
    reshape_and_cache(key, value, cache, slots)
    q = randn(gen, (n, h, d), torch.bfloat16).to(dev)
    scale = d ** -0.5
    pc = PagedCache.from_tensor(cache)
    row_dev = row.to(dev)
    ent = [make_entry(0, n, segment_paged(pc, row_dev, 0, n), 0)]
    o1, l1 = varlen_attn_with_lse(q, ent, True, hkv, scale)
    o2, l2 = ring_attn_with_lse(q, key, value, scale, 0)
    torch.cuda.synchronize()
    assert torch.equal(o1.cpu(), o2.cpu()) and torch.equal(l1.cpu(), l2.cpu())
