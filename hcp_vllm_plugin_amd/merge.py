"""LSE merge on the HIP kernel (the ``merge_attn_states`` contract).

``merge_attn_states(output, prefix_output, prefix_lse, suffix_output,
suffix_lse, output_lse=None)`` with vLLM's semantics as the reference calls it
(ring_backend.py:349-354: prefix = peer, suffix = local; ring_decode.py:55-58),
plus ``merge_pair`` returning the merged LSE as ring_decode.py:46-61 does.
o tensors ``[T, H, D]`` (f16 / bf16 / f32, independently), lse ``[H, T]``
float32.  The work runs in ``hcp_merge_attn_states`` (libhcp_mi355x.so).
"""

from __future__ import annotations

import torch

from . import _lib

__all__ = ["merge_attn_states", "merge_pair"]


def _chk_o(name: str, t: torch.Tensor) -> None:
    if t.dim() != 3:
        raise ValueError(f"{name} must be [T, H, D]")
    if t.stride(-1) != 1 or t.data_ptr() % 16 or any(s % 8 for s in t.stride()[:-1]):
        raise ValueError(f"{name}: last dim must be contiguous, 16-byte aligned rows")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")


def _chk_lse(name: str, t: torch.Tensor, h: int, n: int) -> None:
    if t.dtype != torch.float32 or t.dim() != 2 or tuple(t.shape) != (h, n):
        raise ValueError(f"{name} must be float32 [H={h}, T={n}], got {t.dtype} {tuple(t.shape)}")
    if t.stride(1) != 1:
        raise ValueError(f"{name} must be contiguous along tokens")


def merge_attn_states(
    output: torch.Tensor,
    prefix_output: torch.Tensor,
    prefix_lse: torch.Tensor,
    suffix_output: torch.Tensor,
    suffix_lse: torch.Tensor,
    output_lse: torch.Tensor | None = None,
) -> None:
    """out = (e^{lse_p} o_p + e^{lse_s} o_s) / (e^{lse_p} + e^{lse_s}); in place.

    A head_dim that is not a multiple of 8 runs on zero-padded copies (the
    kernel moves 16-byte pieces), the result copied back into ``output``."""
    if output.dim() == 3 and output.shape[2] % 8:
        from .ring_attn import pad_head_dim, padded_width

        if prefix_output.shape != output.shape or suffix_output.shape != output.shape:
            raise ValueError("output / prefix_output / suffix_output shapes differ")
        w = padded_width(output.shape[2])
        tmp = output.new_empty((output.shape[0], output.shape[1], w))
        merge_attn_states(tmp, pad_head_dim(prefix_output, w), prefix_lse,
                          pad_head_dim(suffix_output, w), suffix_lse, output_lse)
        output.copy_(tmp[..., : output.shape[2]])
        return
    for n, t in (("output", output), ("prefix_output", prefix_output),
                 ("suffix_output", suffix_output)):
        _chk_o(n, t)
    if prefix_output.shape != suffix_output.shape or output.shape != prefix_output.shape:
        raise ValueError("output / prefix_output / suffix_output shapes differ")
    t, h, d = output.shape
    _chk_lse("prefix_lse", prefix_lse, h, t)
    _chk_lse("suffix_lse", suffix_lse, h, t)
    if output_lse is not None:
        _chk_lse("output_lse", output_lse, h, t)
    L = _lib.lib()
    with torch.cuda.device(output.device):
        rc = L.hcp_merge_attn_states(
            output.data_ptr(), output.stride(0), output.stride(1), _lib.dtype_code(output.dtype),
            output_lse.data_ptr() if output_lse is not None else None,
            output_lse.stride(0) if output_lse is not None else 0,
            prefix_output.data_ptr(), prefix_output.stride(0), prefix_output.stride(1),
            _lib.dtype_code(prefix_output.dtype), prefix_lse.data_ptr(), prefix_lse.stride(0),
            suffix_output.data_ptr(), suffix_output.stride(0), suffix_output.stride(1),
            _lib.dtype_code(suffix_output.dtype), suffix_lse.data_ptr(), suffix_lse.stride(0),
            t, h, d, _lib.stream_ptr(output.device),
        )
    _lib.check(rc, "hcp_merge_attn_states")


def merge_pair(
    o1: torch.Tensor, lse1: torch.Tensor, o2: torch.Tensor, lse2: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor]:
    """Merge two partials and return (out, merged lse) -- ring_decode.py:46-61."""
    out = torch.empty_like(o1, memory_format=torch.contiguous_format)
    lse = torch.empty_like(lse1, memory_format=torch.contiguous_format)
    merge_attn_states(out, o1, lse1, o2, lse2, lse)
    return out, lse
