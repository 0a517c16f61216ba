"""Flash attention with LSE on the HIP kernels (the ``ring_attn_with_lse`` contract).

Mirrors hcp_vllm_plugin/ring_triton_attn.py:155-207: the same call
``ring_attn_with_lse(q, k, v, scale, causal_offset) -> (out, lse)``, the same
shapes (q ``[Tq, H, D]``, k/v ``[Tk, Hkv, D]``, out ``[Tq, H, D]`` in q.dtype,
lse ``[H, Tq]`` float32 natural log), ``causal_offset=None`` meaning
non-causal and an integer meaning causal with query 0 at that position in the
KV frame.  The work runs in ``hcp_attn_fwd_lse`` (libhcp_mi355x.so).

``ring_attn_merged`` is that pass and the ``merge_attn_states`` after it
(ring_backend.py:820-831) in one launch (``hcp_attn_fwd_lse_merge``).
"""

from __future__ import annotations

import torch

from . import _lib

__all__ = ["ring_attn_with_lse", "ring_attn_merged", "check_qkv", "COPY_STATS",
           "pad_head_dim", "padded_width"]

# Layout copies made on the way into the kernels: an input whose layout the
# kernel cannot load directly (rows not 16-byte aligned, strides not
# multiples of 8 elements, k and v with different strides) is copied
# contiguous first, as the reference's dispatch copies every input
# (ring_backend.py:328).  Counted here so the extra HBM traffic is visible.
COPY_STATS: dict = {"tensors": 0, "bytes": 0}


def _copied(t: torch.Tensor) -> torch.Tensor:
    c = t.contiguous()
    COPY_STATS["tensors"] += 1
    COPY_STATS["bytes"] += c.numel() * c.element_size()
    return c


def check_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    """Shape/dtype/device checks of the kernel contract (ring_triton_attn.py:169-172)."""
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
        raise ValueError("q, k, v must be 3-D: [T, heads, head_dim]")
    if k.shape != v.shape:
        raise ValueError(f"k {tuple(k.shape)} and v {tuple(v.shape)} differ")
    if q.shape[2] != k.shape[2]:
        raise ValueError("q and k head_dim differ")
    if q.shape[1] % k.shape[1] != 0:
        raise ValueError(f"num_heads {q.shape[1]} not a multiple of num_kv_heads {k.shape[1]}")
    if q.dtype not in (torch.float16, torch.bfloat16) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"q/k/v must share dtype float16 or bfloat16, got {q.dtype}/{k.dtype}/{v.dtype}")
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise ValueError("q, k, v must be GPU tensors")
    if q.stride(-1) != 1 or k.stride(-1) != 1 or v.stride(-1) != 1:
        raise ValueError("head_dim must be the contiguous dimension")


def pad_head_dim(t: torch.Tensor, width: int) -> torch.Tensor:
    """t ``[T, heads, d]`` copied into a zero-filled ``[T, heads, width]``
    (counted in COPY_STATS).  The kernels load rows in 16-byte pieces, so a
    head_dim that is not a multiple of 8 runs at the next multiple of 8: zero
    columns in q and k add nothing to the scores, and zero columns of v give
    output columns that are dropped -- the reference's masked ``BLOCK_D``
    columns (ring_triton_attn.py:69-78,201)."""
    out = t.new_zeros((t.shape[0], t.shape[1], width))
    out[..., : t.shape[2]].copy_(t)
    COPY_STATS["tensors"] += 1
    COPY_STATS["bytes"] += out.numel() * out.element_size()
    return out


def padded_width(head_dim: int) -> int:
    """The multiple of 8 a head_dim runs at."""
    return -(-head_dim // 8) * 8


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """Return t, or a contiguous copy when its layout is not kernel-loadable."""
    ok = (
        t.data_ptr() % 16 == 0
        and all(s % 8 == 0 for s in t.stride()[:-1])
        and t.stride(-1) == 1
    )
    return t if ok else _copied(t)


def ring_attn_with_lse(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: float,
    causal_offset: int | None,
    window: int | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Flash-style attention with LSE output (HIP, gfx950).

    causal_offset: absolute position of query token 0 within the KV range
    (None => non-causal, all keys visible).  window: sliding window on the
    causal pass as ``_attn_with_lse`` applies it (ring_backend.py:372,
    397-398): query i at p = causal_offset + i sees keys p - window < j <= p;
    ignored when non-causal.  Returns (out ``[Tq, H, D]`` in q.dtype, lse
    ``[H, Tq]`` float32 natural log).  A query with no visible key (empty KV,
    or a negative offset) gets out 0 and lse -inf.
    """
    check_qkv(q, k, v)
    if window is not None and window <= 0:
        raise ValueError("window must be a positive number of keys")
    if q.shape[2] % 8:
        w = padded_width(q.shape[2])
        out, lse = ring_attn_with_lse(pad_head_dim(q, w), pad_head_dim(k, w), pad_head_dim(v, w),
                                      scale, causal_offset, window)
        return out[..., : q.shape[2]].contiguous(), lse
    q, k, v = _aligned(q), _aligned(k), _aligned(v)
    tq, num_heads, head_dim = q.shape
    tk, num_kv_heads = k.shape[0], k.shape[1]
    out = torch.empty_like(q, memory_format=torch.contiguous_format)
    lse = torch.empty((num_heads, tq), dtype=torch.float32, device=q.device)
    if tq == 0:
        return out, lse
    if k.stride() != v.stride():
        v = v if v.is_contiguous() else _copied(v)
        k = k if k.is_contiguous() else _copied(k)
    L = _lib.lib()
    with torch.cuda.device(q.device):
        rc = L.hcp_attn_fwd_lse(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
            tq, tk, num_heads, num_kv_heads, head_dim,
            q.stride(0), q.stride(1), k.stride(0), k.stride(1),
            v.stride(0), v.stride(1), out.stride(0), out.stride(1), lse.stride(0),
            float(scale), 0 if causal_offset is None else 1,
            0 if causal_offset is None else int(causal_offset),
            0 if (window is None or causal_offset is None) else int(window),
            _lib.dtype_code(q.dtype), _lib.stream_ptr(q.device),
        )
    _lib.check(rc, "hcp_attn_fwd_lse")
    return out, lse


def _check_partial(o: torch.Tensor, lse: torch.Tensor, q: torch.Tensor, name: str) -> None:
    if o.shape != q.shape or o.dtype != q.dtype or o.device != q.device:
        raise ValueError(f"{name} output must match q: {tuple(o.shape)} {o.dtype}")
    if lse.shape != (q.shape[1], q.shape[0]) or lse.dtype != torch.float32 or lse.device != q.device:
        raise ValueError(f"{name} lse must be float32 [H, Tq]")
    if lse.stride(1) != 1:
        raise ValueError(f"{name} lse must be contiguous along tokens")
    if o.stride(-1) != 1 or o.data_ptr() % 16 or any(st % 8 for st in o.stride()[:-1]):
        raise ValueError(f"{name} output layout not loadable (16-byte rows, head_dim contiguous)")


def ring_attn_merged(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: float,
    causal_offset: int | None,
    acc_output: torch.Tensor,
    acc_lse: torch.Tensor,
    acc_is_prefix: bool = True,
    window: int | None = None,
    output: torch.Tensor | None = None,
    output_lse: torch.Tensor | None = None,
) -> torch.Tensor:
    """``ring_attn_with_lse`` over (q, k, v) merged with a partial state, in one launch.

    With ``acc_is_prefix`` the result is ``merge_attn_states(output,
    acc_output, acc_lse, <this pass>)`` -- the local pass taking the peer
    result as the prefix, as ``HcpRingAttentionImpl.forward`` merges them
    (ring_backend.py:349-354,820-831); otherwise this pass is the prefix.
    The arithmetic is the merge kernel's on this pass's output rounded to
    q.dtype, so the result equals the two calls bit for bit.  ``output``
    (default: new) may be ``acc_output`` itself; ``output_lse`` (optional,
    ``[H, Tq]`` float32) receives the merged LSE.  Returns ``output``.
    """
    check_qkv(q, k, v)
    if window is not None and window <= 0:
        raise ValueError("window must be a positive number of keys")
    if q.shape[2] % 8:
        if output is not None and (output.shape != q.shape or output.dtype != q.dtype):
            raise ValueError("output must match q in shape and dtype")
        w = padded_width(q.shape[2])
        res = ring_attn_merged(pad_head_dim(q, w), pad_head_dim(k, w), pad_head_dim(v, w),
                               scale, causal_offset, pad_head_dim(acc_output, w), acc_lse,
                               acc_is_prefix, window, None, output_lse)
        if output is None:
            return res[..., : q.shape[2]].contiguous()
        output.copy_(res[..., : q.shape[2]])
        return output
    q, k, v = _aligned(q), _aligned(k), _aligned(v)
    _check_partial(acc_output, acc_lse, q, "acc")
    tq, num_heads, head_dim = q.shape
    tk, num_kv_heads = k.shape[0], k.shape[1]
    if output is None:
        output = torch.empty_like(q, memory_format=torch.contiguous_format)
    elif output.shape != q.shape or output.dtype != q.dtype or output.stride(-1) != 1:
        raise ValueError("output must match q in shape and dtype, head_dim contiguous")
    if output_lse is not None and (output_lse.shape != (num_heads, tq)
                                   or output_lse.dtype != torch.float32
                                   or output_lse.stride(1) != 1):
        raise ValueError("output_lse must be float32 [H, Tq], contiguous along tokens")
    if tq == 0:
        return output
    if k.stride() != v.stride():
        v = v if v.is_contiguous() else _copied(v)
        k = k if k.is_contiguous() else _copied(k)
    L = _lib.lib()
    with torch.cuda.device(q.device):
        rc = L.hcp_attn_fwd_lse_merge(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), output.data_ptr(),
            0 if output_lse is None else output_lse.data_ptr(),
            tq, tk, num_heads, num_kv_heads, head_dim,
            q.stride(0), q.stride(1), k.stride(0), k.stride(1),
            v.stride(0), v.stride(1), output.stride(0), output.stride(1),
            0 if output_lse is None else output_lse.stride(0),
            float(scale), 0 if causal_offset is None else 1,
            0 if causal_offset is None else int(causal_offset),
            0 if (window is None or causal_offset is None) else int(window),
            acc_output.data_ptr(), acc_output.stride(0), acc_output.stride(1),
            acc_lse.data_ptr(), acc_lse.stride(0), int(bool(acc_is_prefix)),
            _lib.dtype_code(q.dtype), _lib.stream_ptr(q.device),
        )
    _lib.check(rc, "hcp_attn_fwd_lse_merge")
    return output
