"""Paged KV-cache write on the HIP kernel (the step before the attention path).

``reshape_and_cache(key, value, kv_cache, slot_mapping)`` writes this step's
K/V rows into the paged cache at ``slot_mapping`` (slot = block * block_size
+ offset): the operation of the reference's ``do_kv_cache_update``
(hcp_vllm_plugin/ring_backend.py:501-539), which does it with torch advanced
indexing into the vLLM 0.23 layout ``[nb, 2, bs, Hkv, D]``, and of vLLM's
``reshape_and_cache`` for the 0.31 layout ``[nb, Hkv, bs, 2*D]`` that the
paged local-segment reader consumes (file_connector.py:13-16).  Rows ``t <
len(slot_mapping)`` of key/value are written (key may be padded past that, as
in the reference's ``key[:n]``); a negative slot is a padding token and is
skipped.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .varlen import PagedCache

__all__ = ["reshape_and_cache"]

# Cache descriptors by (address, shape, strides, dtype): the write runs once per
# layer and step, and building the descriptor each time was a third of its
# host cost.  The key fixes every field the descriptor holds, so a descriptor
# found here is the one the tensor would produce.
_DESCS: dict = {}
_MAX_DESCS = 1024


def _cache_desc(kv_cache: torch.Tensor):
    ck = (kv_cache.data_ptr(), tuple(kv_cache.shape), kv_cache.stride(), kv_cache.dtype)
    ent = _DESCS.get(ck)
    if ent is None:
        pc = PagedCache.from_tensor(kv_cache)
        desc = _lib.PagedCacheDesc()
        desc.k_addr = pc.k_addr
        desc.v_addr = pc.v_addr
        desc.stride_block = pc.stride_block
        desc.stride_head = pc.stride_head
        desc.stride_tok = pc.stride_tok
        desc.num_blocks = kv_cache.shape[0]
        desc.block_size = pc.block_size
        if len(_DESCS) >= _MAX_DESCS:
            _DESCS.clear()
        ent = _DESCS[ck] = (desc, ctypes.addressof(desc), pc.num_kv_heads, pc.head_dim)
    return ent


def reshape_and_cache(key: torch.Tensor, value: torch.Tensor, kv_cache: torch.Tensor,
                      slot_mapping: torch.Tensor) -> None:
    """Write ``key``/``value`` ``[N, Hkv, D]`` rows ``[0, n)``, ``n =
    slot_mapping.numel()``, into ``kv_cache`` at ``slot_mapping``."""
    _, desc_addr, hkv, d = _cache_desc(kv_cache)
    n = slot_mapping.numel()
    if key.shape != value.shape or key.dim() != 3:
        raise ValueError("key/value must be [N, Hkv, D] of one shape")
    if key.shape[0] < n:
        raise ValueError(f"{n} slots for {key.shape[0]} key rows")
    if key.shape[1] != hkv or key.shape[2] != d:
        raise ValueError("key/value heads or head_dim do not match the cache")
    if key.dtype != kv_cache.dtype or value.dtype != kv_cache.dtype:
        raise ValueError("key/value dtype must match the cache dtype")
    if key.stride(-1) != 1 or value.stride(-1) != 1:
        raise ValueError("key/value head_dim must be contiguous")
    if slot_mapping.dtype not in (torch.int32, torch.int64):
        raise ValueError("slot_mapping must be int32 or int64")
    if n == 0:
        return
    slots = slot_mapping.contiguous()
    L = _lib.lib()
    args = (key.data_ptr(), key.stride(0), key.stride(1),
            value.data_ptr(), value.stride(0), value.stride(1),
            slots.data_ptr(), _lib.DTYPE_I64 if slots.dtype == torch.int64 else _lib.DTYPE_I32,
            n, hkv, d, desc_addr, _lib.dtype_code(key.dtype))
    dev = key.device
    if dev.index == torch.cuda.current_device():
        rc = L.hcp_reshape_and_cache(*args, torch.cuda.current_stream(dev).cuda_stream)
    else:
        with torch.cuda.device(dev):
            rc = L.hcp_reshape_and_cache(*args, _lib.stream_ptr(dev))
    _lib.check(rc, "hcp_reshape_and_cache")
