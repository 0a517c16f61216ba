"""ctypes binding of ``libhcp_mi355x.so`` (the C ABI in include/hcp_mi355x.h).

The library is built in-tree by ``hcp_vllm_plugin_amd.build`` (``__graft_entry__.build()``)
and loaded from this package directory.  Loading it after ``import torch`` makes
its ``libamdhip64.so.7`` dependency resolve to the HIP runtime torch already
loaded (same soname), so the raw ``hipStream_t`` of torch's current stream and
torch's device pointers are valid in the library.

There is no fallback: if the library is missing or fails to load, every entry
point raises ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must be loaded first: shares its HIP runtime)

LIB_NAME = "libhcp_mi355x.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

HCP_OK = 0
HCP_EINVAL = -1
HCP_EUNSUPPORTED = -2
HCP_ELAUNCH = -3
HCP_EWORKSPACE = -4

# include/hcp_mi355x.h HCP_NOALLOC_SCRATCH_BYTES
NOALLOC_SCRATCH_BYTES = 16 << 20

DTYPE_F16 = 0
DTYPE_BF16 = 1
DTYPE_F32 = 2
DTYPE_I32 = 3
DTYPE_I64 = 4

_STATUS_NAMES = {
    HCP_EINVAL: "EINVAL",
    HCP_EUNSUPPORTED: "EUNSUPPORTED",
    HCP_ELAUNCH: "ELAUNCH",
    HCP_EWORKSPACE: "EWORKSPACE",
}

# Every symbol include/hcp_mi355x.h declares.
EXPORTED_SYMBOLS = (
    "hcp_abi_version",
    "hcp_last_error",
    "hcp_attn_fwd_lse",
    "hcp_attn_fwd_lse_merge",
    "hcp_varlen_block_m",
    "hcp_plan_varlen_tiles",
    "hcp_attn_fwd_varlen",
    "hcp_attn_fwd_varlen_merge",
    "hcp_plan_decode_splits",
    "hcp_decode_workspace_bytes",
    "hcp_decode_splitkv",
    "hcp_decode_splitkv_acc",
    "hcp_decode_splitkv_noalloc",
    "hcp_merge_attn_states",
    "hcp_reshape_and_cache",
    "hcp_gather_paged_kv",
)

ABI_VERSION = 9


class KvSegment(ctypes.Structure):
    """``hcp_kv_segment`` (include/hcp_mi355x.h)."""

    _fields_ = [
        ("k_addr", ctypes.c_uint64),
        ("v_addr", ctypes.c_uint64),
        ("block_table", ctypes.c_uint64),
        ("stride_tok", ctypes.c_int64),
        ("stride_head", ctypes.c_int64),
        ("stride_block", ctypes.c_int64),
        ("start", ctypes.c_int64),
        ("len", ctypes.c_int64),
        ("block_size", ctypes.c_int32),
        ("num_blocks", ctypes.c_int32),
    ]


class VarlenEntry(ctypes.Structure):
    """``hcp_varlen_entry`` (include/hcp_mi355x.h)."""

    _fields_ = [
        ("q_start", ctypes.c_int64),
        ("q_len", ctypes.c_int64),
        ("causal_offset", ctypes.c_int64),
        ("kv", KvSegment),
    ]


class PagedCacheDesc(ctypes.Structure):
    """``hcp_paged_cache`` (include/hcp_mi355x.h)."""

    _fields_ = [
        ("k_addr", ctypes.c_uint64),
        ("v_addr", ctypes.c_uint64),
        ("stride_block", ctypes.c_int64),
        ("stride_head", ctypes.c_int64),
        ("stride_tok", ctypes.c_int64),
        ("num_blocks", ctypes.c_int64),
        ("block_size", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


class DecodeSplit(ctypes.Structure):
    """``hcp_decode_split`` (include/hcp_mi355x.h)."""

    _fields_ = [
        ("entry", ctypes.c_int32),
        ("key_begin", ctypes.c_int32),
        ("key_end", ctypes.c_int32),
        ("slot", ctypes.c_int32),
    ]


_lock = threading.Lock()
_lib = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_F = ctypes.c_float


def _declare(lib: ctypes.CDLL) -> None:
    lib.hcp_abi_version.restype = ctypes.c_int
    lib.hcp_abi_version.argtypes = []
    lib.hcp_last_error.restype = ctypes.c_char_p
    lib.hcp_last_error.argtypes = []
    lib.hcp_attn_fwd_lse.restype = ctypes.c_int
    lib.hcp_attn_fwd_lse.argtypes = [
        _P, _P, _P, _P, _P, _I64, _I64, _I32, _I32, _I32,
        _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
        _F, _I32, _I64, _I32, _I32, _P,
    ]
    lib.hcp_attn_fwd_lse_merge.restype = ctypes.c_int
    lib.hcp_attn_fwd_lse_merge.argtypes = [
        _P, _P, _P, _P, _P, _I64, _I64, _I32, _I32, _I32,
        _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
        _F, _I32, _I64, _I32, _P, _I64, _I64, _P, _I64, _I32, _I32, _P,
    ]
    lib.hcp_varlen_block_m.restype = ctypes.c_int
    lib.hcp_varlen_block_m.argtypes = [_I32, _I32]
    lib.hcp_plan_varlen_tiles.restype = ctypes.c_int
    lib.hcp_plan_varlen_tiles.argtypes = [_P, _I32, _I32, _I32, _P, _I32]
    lib.hcp_attn_fwd_varlen.restype = ctypes.c_int
    lib.hcp_attn_fwd_varlen.argtypes = [
        _P, _I64, _I64, _P, _I64, _I64, _P, _I64,
        _P, _I32, _P, _I32, _I32, _I32, _I32, _F, _I32, _I32, _I32, _I32, _P,
    ]
    lib.hcp_attn_fwd_varlen_merge.restype = ctypes.c_int
    lib.hcp_attn_fwd_varlen_merge.argtypes = [
        _P, _I64, _I64, _P, _I64, _I64, _P, _I64,
        _P, _I32, _P, _I32, _I32, _I32, _I32, _F, _I32, _I32, _I32,
        _P, _I64, _I64, _P, _I64, _I32, _I32, _P,
    ]
    lib.hcp_plan_decode_splits.restype = ctypes.c_int
    lib.hcp_plan_decode_splits.argtypes = [_P, _I32, _P, _I32, _I32, _I32, _P, _I32, _P]
    lib.hcp_decode_workspace_bytes.restype = ctypes.c_size_t
    lib.hcp_decode_workspace_bytes.argtypes = [_I32, _I32, _I32]
    lib.hcp_decode_splitkv.restype = ctypes.c_int
    lib.hcp_decode_splitkv.argtypes = [
        _P, _I64, _I64, _P, _I32, _P, _I32, _P, _I32, _P, ctypes.c_size_t,
        _P, _I64, _I64, _P, _I64, _I32, _I32, _I32, _F, _I32, _P,
    ]
    lib.hcp_decode_splitkv_acc.restype = ctypes.c_int
    lib.hcp_decode_splitkv_acc.argtypes = [
        _P, _I64, _I64, _P, _I32, _P, _I32, _P, _I32, _P, ctypes.c_size_t,
        _P, _I64, _I64, _P, _I64,
        _P, _I64, _I64, _P, _I64, _I32, _I32, _I32, _F, _I32, _P,
    ]
    lib.hcp_decode_splitkv_noalloc.restype = ctypes.c_int
    lib.hcp_decode_splitkv_noalloc.argtypes = [
        _P, _I64, _I64, _P, _I32, _P, _I32, _P, _I32,
        _P, _I64, _I64, _P, _I64, _I32, _I32, _I32, _F, _I32, _P,
    ]
    lib.hcp_reshape_and_cache.restype = ctypes.c_int
    lib.hcp_reshape_and_cache.argtypes = [
        _P, _I64, _I64, _P, _I64, _I64, _P, _I32, _I64, _I32, _I32, _P, _I32, _P,
    ]
    lib.hcp_gather_paged_kv.restype = ctypes.c_int
    lib.hcp_gather_paged_kv.argtypes = [_P, _I32, _P, _I64, _I32, _I32, _I32, _P, _P, _P]
    lib.hcp_merge_attn_states.restype = ctypes.c_int
    lib.hcp_merge_attn_states.argtypes = [
        _P, _I64, _I64, _I32, _P, _I64,
        _P, _I64, _I64, _I32, _P, _I64,
        _P, _I64, _I64, _I32, _P, _I64,
        _I64, _I32, _I32, _P,
    ]


def lib() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_NAME} is not built ({LIB_PATH} missing); run "
                    "`python -c 'import __graft_entry__ as g; g.build()'` or "
                    "`python -m hcp_vllm_plugin_amd.build`"
                )
            try:
                handle = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_LOCAL)
            except OSError as exc:
                raise RuntimeError(f"cannot load {LIB_PATH}: {exc}") from exc
            _declare(handle)
            ver = handle.hcp_abi_version()
            if ver != ABI_VERSION:
                raise RuntimeError(f"{LIB_NAME} ABI {ver}, expected {ABI_VERSION}")
            _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    """Turn a negative hcp_status into RuntimeError with the library's text."""
    if rc < 0:
        msg = lib().hcp_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({_STATUS_NAMES.get(rc, rc)}): {msg}")


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float16:
        return DTYPE_F16
    if dt == torch.bfloat16:
        return DTYPE_BF16
    if dt == torch.float32:
        return DTYPE_F32
    raise ValueError(f"unsupported dtype {dt}")


def stream_ptr(device: torch.device) -> int:
    """Raw hipStream_t of torch's current stream on ``device``."""
    return torch.cuda.current_stream(device).cuda_stream
