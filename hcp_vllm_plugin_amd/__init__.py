"""MI355X-native HCP ring-attention hot path (drop-in for stark-sim/hcp-vllm-plugin).

The package keeps the reference's Python contracts for the hot path and runs
the work in hand-written gfx950 HIP kernels (``libhcp_mi355x.so``, C ABI in
``include/hcp_mi355x.h``):

* ``ring_attn_with_lse(q, k, v, scale, causal_offset) -> (out, lse)``
  (hcp_vllm_plugin/ring_triton_attn.py:155-207)
* ``merge_attn_states(output, prefix_output, prefix_lse, suffix_output,
  suffix_lse, output_lse=None)`` (vLLM op called at ring_backend.py:349-354)
* ``HcpRingAttentionBackend`` / ``HcpRingAttentionImpl`` registered as the
  vLLM ``CUSTOM`` attention backend by ``register()`` (__init__.py:34-54)
* batched varlen / paged prefill and split-KV decode (``varlen``)

Importing the package does not import vLLM; ``register()`` does.
"""

from __future__ import annotations

from .merge import merge_attn_states, merge_pair
from .ring_attn import ring_attn_merged, ring_attn_with_lse

__all__ = [
    "register",
    "ring_attn_with_lse",
    "ring_attn_merged",
    "merge_attn_states",
    "merge_pair",
    "BACKEND_PATH",
]

BACKEND_PATH = "hcp_vllm_plugin_amd.ring_backend.HcpRingAttentionBackend"


def register() -> None:
    """Register the HIP ring backend as vLLM's CUSTOM attention backend.

    Same registration as hcp_vllm_plugin/__init__.py:51-54 (the reference's
    KV connectors are not part of this package).  Entry point group
    ``vllm.general_plugins``.
    """
    from vllm.v1.attention.backends.registry import (  # type: ignore
        AttentionBackendEnum,
        register_backend,
    )

    register_backend(AttentionBackendEnum.CUSTOM, BACKEND_PATH)
