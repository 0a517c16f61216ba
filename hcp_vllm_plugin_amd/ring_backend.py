"""HCP ring-attention backend on the MI355X HIP kernels.

Drop-in for hcp_vllm_plugin/ring_backend.py's hot path:

* ``HcpRingAttentionBackend`` -- ``get_name() == "CUSTOM"``, ``get_impl_cls``,
  ``get_builder_cls``, ``forward_includes_kv_cache_update = False``
  (ring_backend.py:427-449).  When vLLM is importable it subclasses vLLM's
  ``FlashAttentionBackend`` exactly as the reference does (ring_backend.py:71-74);
  without vLLM it is a plain class with the same static methods.
* ``HcpRingAttentionImpl`` -- ``__init__`` (ring_backend.py:464-498) and
  ``forward(layer, query, key, value, kv_cache, attn_metadata, output,
  output_scale=None, output_block_scale=None)`` (ring_backend.py:576-834) with
  the reference's segmentation: vanilla causal attention when a request has no
  peer, plain causal attention for the ``n_a`` queries inside the peer region,
  and for the rest local causal attention over ``[peer_end, tk)`` at offset
  ``qpos0 + n_a - peer_end`` merged with non-causal attention over the peer.
  Instead of a Python loop with a gather copy and 5-6 launches per request,
  a whole batch runs as one launch over the staged peer KV and one varlen
  launch over the paged cache (read in place) that also merges the peer
  result into the output; a pure decode batch runs the split-KV decode
  kernel.
* ``_attn`` / ``_merge`` (ring_backend.py:309-360) with ``HCP_RING_IMPL`` /
  ``HCP_RING_MERGE`` read on every call.  ``hip`` is the default; ``triton``
  is accepted as an alias so existing launch scripts keep working.  There is
  no torch fallback in this package: ``torch`` raises, and a kernel error
  raises instead of silently switching paths.
* The peer-KV staging input contract (ring_backend.py:78-136):
  ``PEER_KV_STAGING[(chunk_key, layer_name)] = (k, v)`` with k/v
  ``[n, Hkv, D]`` post-RoPE, ``PEER_REQ_MAP[first_block_id] = [chunk keys]``.
* Memory-split decode (accumulator ring, ring_backend.py:140-227, :632-722):
  ``register_decode_ring`` / ``clear_decode_ring`` / ``DECODE_RING_MAP``.  A
  registered request's single-token decode step skips the pool write, and its
  attention is the owner's local partial (own chunk in the pool + owned growth
  + current token) sent around the ring by ``ring_decode.ring_decode_step``;
  decode growth is sharded by ``ring_decode.growth_assignee``.  In a pure
  decode batch the owner partials run in the same split-KV launch as the
  other rows.
* ``IMPL_STATS`` evidence counters (ring_backend.py:295-306).  ``attn_hip`` /
  ``merge_hip`` count kernel launches and merges (a merge done inside the
  local pass counts as one); the legacy keys ``attn_triton`` /
  ``merge_triton`` mirror them so validators that read those names still see
  which path ran, and ``attn_torch`` / ``merge_torch`` stay 0.
* The validators' other evidence (ring_backend.py:228-275, :790-810), same
  names and meaning: ``STAGING_STATS`` / ``reset_staging_stats`` (staging
  high-water marks), ``WRITE_TRACK`` / ``reset_write_tracking`` (pool slots
  written, the chunk-A ``overlap`` probe in ``forward``, decode-ring
  ``skipped`` writes) and ``BATCH_STATS`` / ``reset_batch_stats``.
"""

from __future__ import annotations

import enum
import logging
import os

import numpy as np
import torch

from . import _lib
from .kv_cache import reshape_and_cache
from .merge import merge_attn_states
from .ring_attn import COPY_STATS, ring_attn_with_lse
from .ring_decode import GrowthBuffer, growth_assignee, local_partial, ring_decode_step
from .varlen import (
    ENTRY_DTYPE,
    head_major,
    DecodeBatch,
    PagedCache,
    VarlenLaunch,
    make_entry,
    paged_entry_array,
    segment_contiguous,
    segment_paged,
    trim_segment,
    window_tail,
)

logger = logging.getLogger(__name__)

try:  # optional: the real vLLM base classes, as the reference uses them
    from vllm.v1.attention.backend import AttentionImpl as _ImplBase  # type: ignore
    from vllm.v1.attention.backend import AttentionType  # type: ignore
    from vllm.v1.attention.backends.flash_attn import (  # type: ignore
        FlashAttentionBackend as _BackendBase,
        FlashAttentionMetadataBuilder as _BuilderCls,
    )

    HAVE_VLLM = True
except ImportError:  # vLLM absent: same surface, no base classes
    HAVE_VLLM = False
    _ImplBase = object
    _BackendBase = object
    _BuilderCls = None

    class AttentionType(str, enum.Enum):  # type: ignore[no-redef]
        DECODER = "decoder"
        ENCODER = "encoder"
        ENCODER_ONLY = "encoder_only"
        ENCODER_DECODER = "encoder_decoder"


# ---------------------------------------------------------------------------
# Peer KV staging (input contract; the connector writes, forward reads)
# ---------------------------------------------------------------------------
PEER_KV_STAGING: dict[tuple[str, str], tuple[torch.Tensor, torch.Tensor]] = {}
PEER_REQ_MAP: dict[int, list[str]] = {}
# (chunk_key, layer_name) -> (event recorded after the staged copy was queued,
# streams already ordered after it); a forward on any stream waits on the
# event once before reading the chunk
_STAGE_READY: dict[tuple[str, str], tuple[torch.cuda.Event, set]] = {}
# Bumped whenever a chunk key appears in or leaves the staging dict, or the
# request map changes: which requests take which chunks (the decode-step
# template) is decided from these, and stays valid while the count holds.
# (A further layer of an already staged chunk does not bump it; each layer's
# lookup checks its own entry.)
_STAGE_GEN = [0]
_CHUNK_LAYERS: dict[str, int] = {}  # chunk key -> layers staged


def stage_peer_kv(chunk_key: str, layer_name: str, k: torch.Tensor, v: torch.Tensor,
                  ready: torch.cuda.Event | None = None) -> None:
    """Stage a peer chunk's K/V ``[n, Hkv, D]`` (post-RoPE) for one layer.

    Stored head-major (one copy per chunk and layer): a chunk is staged once
    and read by every decode step, and the split-KV decode streams a KV head's
    keys 5% faster as one contiguous run than as rows interleaved with the
    other heads'; the prefill passes read either layout at the same rate.

    Ordering: the copy is queued on the caller's current stream.  ``ready``
    (e.g. ``IngestedKV.event`` of a ``PeerIngest.load`` on a side stream) is
    waited on by that stream first, so the copy reads landed bytes.  An event
    recorded after the copy is kept with the entry and every forward that
    reads the chunk makes its own stream wait on it, so staging from a
    connector thread's stream and reading from the model's stream is ordered
    on the device without a host synchronisation.
    """
    on_gpu = k.is_cuda
    if on_gpu and ready is not None:
        torch.cuda.current_stream(k.device).wait_event(ready)
    key = (chunk_key, layer_name)
    if key not in PEER_KV_STAGING:
        _CHUNK_LAYERS[chunk_key] = _CHUNK_LAYERS.get(chunk_key, 0) + 1
        if _CHUNK_LAYERS[chunk_key] == 1:
            _STAGE_GEN[0] += 1
    PEER_KV_STAGING[key] = (head_major(k), head_major(v))
    if on_gpu:
        st = torch.cuda.current_stream(k.device)
        ev = torch.cuda.Event()
        ev.record(st)
        _STAGE_READY[key] = (ev, {st})
    else:
        _STAGE_READY.pop(key, None)
    _note_staging(k)


# High-water marks of the staging dict (ring_backend.py:228-251): staging is
# freed when a request finishes, so post-run checks read these instead.
STAGING_STATS: dict = {"max_concurrent_chunks": 0, "max_staged_layers": 0, "last_chunk_len": 0}


def reset_staging_stats() -> None:
    STAGING_STATS["max_concurrent_chunks"] = 0
    STAGING_STATS["max_staged_layers"] = 0
    STAGING_STATS["last_chunk_len"] = 0


def _note_staging(k: torch.Tensor) -> None:
    """Raise the high-water marks after a stage: (chunk, layer) entries held,
    distinct chunks held, and the token count of the chunk just staged."""
    STAGING_STATS["max_staged_layers"] = max(STAGING_STATS["max_staged_layers"],
                                             len(PEER_KV_STAGING))
    chunks = {key[0] for key in PEER_KV_STAGING}
    STAGING_STATS["max_concurrent_chunks"] = max(STAGING_STATS["max_concurrent_chunks"],
                                                 len(chunks))
    STAGING_STATS["last_chunk_len"] = int(k.shape[0])


def _wait_staged(key: tuple[str, str], kv: tuple[torch.Tensor, torch.Tensor]) -> None:
    """Order the current stream after the staging copy of ``key`` (once per
    stream).  A chunk staged on another stream is also marked as used on this
    one, so the caching allocator keeps its memory until this stream's reads
    are done even if the chunk is dropped meanwhile."""
    ent = _STAGE_READY.get(key)
    if ent is None:
        return
    ev, seen = ent
    cur = torch.cuda.current_stream(kv[0].device)
    if cur in seen:
        return
    cur.wait_event(ev)
    for t in kv:
        t.record_stream(cur)
    seen.add(cur)


def drop_chunk_kv(chunk_key: str) -> int:
    keys = [key for key in PEER_KV_STAGING if key[0] == chunk_key]
    for key in keys:
        del PEER_KV_STAGING[key]
        _STAGE_READY.pop(key, None)
    if _CHUNK_LAYERS.pop(chunk_key, None) is not None:
        _STAGE_GEN[0] += 1
    return len(keys)


def map_request_peer(first_block_id: int, chunk_keys) -> None:
    """Bind a request (by its first block id) to its ordered prefix chunks."""
    if isinstance(chunk_keys, str):
        chunk_keys = [chunk_keys]
    chunk_keys = list(chunk_keys)
    if PEER_REQ_MAP.get(first_block_id) != chunk_keys:
        PEER_REQ_MAP[first_block_id] = chunk_keys
        _STAGE_GEN[0] += 1


def unmap_request_peer(first_block_id: int) -> None:
    if PEER_REQ_MAP.pop(first_block_id, None) is not None:
        _STAGE_GEN[0] += 1


def request_peer_chunk(first_block_id: int) -> list[str] | None:
    return PEER_REQ_MAP.get(first_block_id)


def clear_peer_kv() -> None:
    PEER_KV_STAGING.clear()
    PEER_REQ_MAP.clear()
    _STAGE_READY.clear()
    _CHUNK_LAYERS.clear()
    _STAGE_GEN[0] += 1


# ---------------------------------------------------------------------------
# Memory-split decode registry (ring_backend.py:140-227)
# ---------------------------------------------------------------------------
DECODE_RING_MAP: dict[int, dict] = {}
_STAGING_RELEASE_FN = None


def _decode_ring_enabled() -> bool:
    return os.environ.get("HCP_RING_DECODE_RING", "1") == "1"


def _growth_policy() -> str:
    return os.environ.get("HCP_RING_DECODE_GROWTH", "rr")


def set_staging_release_fn(fn) -> None:
    """Connector callback that frees a request's staged prefix KV."""
    global _STAGING_RELEASE_FN
    _STAGING_RELEASE_FN = fn


def register_decode_ring(first_block_id: int, peer_chunks: list[tuple[str, str]],
                         prefix_len: int, transport=None) -> None:
    """Switch a request to memory-split decode (ring_backend.py:175-208).

    ``peer_chunks``: ordered ``(chunk_key, peer_url)`` of the prefix (entries
    with an empty url are dropped); ``prefix_len``: tokens of the prefix;
    ``transport``: the ring transport (``send_packet`` / ``recv_packet``).
    Ring indices: 0..N-2 the prefix peers, N-1 the owner.
    """
    import uuid

    peers = [(ck, u) for ck, u in peer_chunks if u]
    DECODE_RING_MAP[first_block_id] = {
        "peer_chunks": peers,
        "prefix_len": prefix_len,
        "req_tag": f"{first_block_id}:{uuid.uuid4().hex[:8]}",
        "ring_size": len(peers) + 1,
        "own_index": len(peers),
        "own_chunk_len": None,     # set at the first decode step
        "growth": {},              # layer -> GrowthBuffer (owner's share)
        "pending_growth": {},      # layer -> (assignee, k, v), shipped next step
        "growth_policy": _growth_policy(),
        "transport": transport,
    }


def clear_decode_ring(first_block_id: int) -> None:
    DECODE_RING_MAP.pop(first_block_id, None)


def _release_staged_for_request(first_block_id: int) -> None:
    """Free a request's staged prefix KV at its decode-ring transition
    (ring_backend.py:214-225)."""
    if first_block_id not in PEER_REQ_MAP:
        return
    if _STAGING_RELEASE_FN is not None:
        _STAGING_RELEASE_FN(first_block_id)
    else:
        for ck in PEER_REQ_MAP.pop(first_block_id, None) or []:
            drop_chunk_kv(ck)


def _contiguous_record(j: int, seq: int, k: torch.Tensor, v: torch.Tensor):
    """hcp_varlen_entry of decode query row ``seq`` over all of a staged chunk
    (contiguous k/v ``[n, Hkv, D]``), as an ENTRY_DTYPE record value."""
    if k.stride() != v.stride() or k.data_ptr() % 16 or v.data_ptr() % 16 or \
            (k.stride(0) * k.element_size()) % 16 or (k.stride(1) * k.element_size()) % 16 or \
            not 0 < k.stride(0) < (1 << 24):
        raise ValueError(f"staged chunk of entry {j}: k/v layout not loadable")
    return (seq, 1, 0, k.data_ptr(), v.data_ptr(), 0, k.stride(0), k.stride(1), 0, 0,
            int(k.shape[0]), 0, 0)


# Host copy of the step's attention metadata.  vLLM hands every layer the same
# metadata object, so one device->host copy serves all layers of a step (the
# reference syncs three times per layer, ring_backend.py:604-605).  Holding the
# object keeps its identity from being reused by a later step's metadata.
_STEP: dict = {"meta": None, "stamp": None, "host": None, "bt": None, "fast": {}}


def _version_of(t: torch.Tensor) -> int:
    try:
        return t._version
    except RuntimeError:  # inference-mode tensors keep no version counter
        return -1


def _meta_stamp(attn_metadata) -> tuple:
    """What identifies one step's metadata contents without reading them:
    the object, and the storage, shape and in-place version counter of each
    tensor the forward reads.  A caller that keeps one metadata object and
    refills its tensors in place between steps through torch's in-place ops
    bumps the version counters, so the next step does not reuse the previous
    step's host copy or plans.  (vLLM builds a new metadata object every
    step; tensors made under inference mode keep no version counter, and a
    caller that refills such tensors in one reused object calls
    ``invalidate_step_cache`` between steps.)"""
    st = [id(attn_metadata)]
    for t in (attn_metadata.query_start_loc, attn_metadata.seq_lens, attn_metadata.block_table):
        st.extend((t.data_ptr(), tuple(t.shape), _version_of(t)))
    return tuple(st)


def invalidate_step_cache() -> None:
    """Drop the cached host copy of the step's metadata and the plans built
    from it: for a caller that rewrites the metadata tensors behind torch's
    back (a kernel writing into them directly) before reusing the object."""
    _STEP.update(meta=None, stamp=None, host=None, bt=None, fast={})


def _host_metadata(attn_metadata):
    """(query_start_loc, seq_lens, first block ids) as lists, and the block
    table as contiguous int32, for this step's metadata."""
    stamp = _meta_stamp(attn_metadata)
    if _STEP["meta"] is attn_metadata and _STEP.get("stamp") == stamp:
        return _STEP["host"], _STEP["bt"]
    block_table = attn_metadata.block_table
    if block_table.dtype != torch.int32:
        block_table = block_table.to(torch.int32)
    block_table = block_table.contiguous()
    qsl_t = attn_metadata.query_start_loc
    sl_t = attn_metadata.seq_lens
    n = sl_t.shape[0]
    fb = block_table[:, 0] if block_table.shape[1] > 0 else sl_t.new_zeros(n)
    packed = torch.cat([qsl_t.reshape(-1).to(torch.int64), sl_t.reshape(-1).to(torch.int64),
                        fb.reshape(-1).to(torch.int64)]).tolist()
    host = (packed[:n + 1], packed[n + 1:2 * n + 1], packed[2 * n + 1:])
    _STEP.update(meta=attn_metadata, stamp=stamp, host=host, bt=block_table, fast={})
    return host, block_table


def _forward_attn_metadata(layer):
    """This step's attention metadata for ``layer`` from vLLM's forward
    context, or None (no vLLM, or no context)."""
    try:
        from vllm.forward_context import get_forward_context  # type: ignore

        raw = get_forward_context().attn_metadata
    except Exception:  # noqa: BLE001 -- no context: attribute nothing
        return None
    if isinstance(raw, dict):
        return raw.get(layer.layer_name)
    if isinstance(raw, list):
        return raw[0].get(layer.layer_name)
    return raw


# Pool-write evidence (ring_backend.py:254-267), validation only.  While
# enabled, do_kv_cache_update records the pool slots this worker wrote, and
# forward counts in "overlap" every slot of a request's peer (chunk-A) region
# among them: a memory-splitting worker never writes one.  "skipped" counts
# decode-ring tokens whose pool write was skipped (always counted).
WRITE_TRACK: dict = {"enabled": False, "slots": set(), "overlap": 0, "skipped": 0}


def reset_write_tracking() -> None:
    """Enable write tracking and clear its evidence (ring_backend.py:260-265)."""
    WRITE_TRACK["enabled"] = True
    WRITE_TRACK["slots"] = set()
    WRITE_TRACK["overlap"] = 0
    WRITE_TRACK["skipped"] = 0


enable_write_tracking = reset_write_tracking  # earlier name of the same call


def _probe_chunk_a_writes(block_row: torch.Tensor, peer_end: int, block_size: int) -> int:
    """Slots of the first ``peer_end`` positions of a request (its peer region,
    through its block-table row) that this worker wrote; added to
    ``WRITE_TRACK["overlap"]`` with a warning (ring_backend.py:790-810)."""
    nb_a = (peer_end + block_size - 1) // block_size
    blocks = block_row[:nb_a].tolist()
    slots = [b * block_size + o for b in blocks for o in range(block_size)][:peer_end]
    overlap = WRITE_TRACK["slots"].intersection(slots)
    if overlap:
        WRITE_TRACK["overlap"] += len(overlap)
        logger.warning("HCP ring: %d chunk-A pool slots were written locally "
                       "(expected 0 in a memory-splitting worker)", len(overlap))
    return len(overlap)


# ---------------------------------------------------------------------------
# Switches and evidence counters
# ---------------------------------------------------------------------------
BATCH_STATS: dict = {"max_reqs": 0}

IMPL_STATS: dict = {
    "attn_hip": 0,
    "merge_hip": 0,
    "decode_hip": 0,
    "ring_decode_steps": 0,
    "attn_triton": 0,
    "merge_triton": 0,
    "attn_torch": 0,
    "merge_torch": 0,
}

_FAST_IMPLS = ("hip", "triton")


def reset_impl_stats() -> None:
    for key in IMPL_STATS:
        IMPL_STATS[key] = 0
    for key in COPY_STATS:
        COPY_STATS[key] = 0


def reset_batch_stats() -> None:
    BATCH_STATS["max_reqs"] = 0


def _ring_enabled() -> bool:
    return os.environ.get("HCP_RING_ENABLED", "1") == "1"


def _split_tokens() -> int:
    return int(os.environ.get("HCP_RING_SPLIT_TOKENS", "0"))


def _ring_impl() -> str:
    return os.environ.get("HCP_RING_IMPL", "hip")


def _merge_impl() -> str:
    return os.environ.get("HCP_RING_MERGE", "hip")


def _require_fast(kind: str, value: str) -> None:
    if value not in _FAST_IMPLS:
        raise NotImplementedError(
            f"{kind}={value!r}: this build runs the HIP kernels only "
            f"(accepted: {', '.join(_FAST_IMPLS)}); there is no torch path"
        )


def _count(kind: str, n: int = 1) -> None:
    IMPL_STATS[f"{kind}_hip"] += n
    legacy = f"{kind}_triton"
    if legacy in IMPL_STATS:
        IMPL_STATS[legacy] += n


def _attn(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: float,
    q_pos0_in_kv: int | None,
    window: int | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Attention + LSE on the HIP kernel (ring_backend.py:309-336 contract),
    sliding window included (the reference sends windowed calls to its torch
    path, :323,336; here the kernel applies it).

    Returns (out ``[Tq, H, D]`` in q.dtype, lse ``[H, Tq]`` float32).
    """
    _require_fast("HCP_RING_IMPL", _ring_impl())
    o, lse = ring_attn_with_lse(q, k, v, scale, q_pos0_in_kv, window)
    _count("attn")
    return o, lse


def _merge(
    o_loc: torch.Tensor, lse_loc: torch.Tensor, o_peer: torch.Tensor, lse_peer: torch.Tensor
) -> torch.Tensor:
    """Local + peer LSE merge on the HIP kernel (ring_backend.py:339-360).

    Same argument order as the reference: ``merge_attn_states(out, o_peer,
    lse_peer, o_loc, lse_loc)`` with out in ``o_loc.dtype``.
    """
    _require_fast("HCP_RING_MERGE", _merge_impl())
    out = torch.empty_like(o_loc, memory_format=torch.contiguous_format)
    merge_attn_states(out, o_peer, lse_peer, o_loc, lse_loc)
    _count("merge")
    return out


# ---------------------------------------------------------------------------
# Backend class (registered as CUSTOM)
# ---------------------------------------------------------------------------
class HcpRingAttentionBackend(_BackendBase):  # type: ignore[misc,valid-type]
    """Ring-attention backend: FlashAttention cache layout + metadata builder
    (inherited when vLLM is present), HIP attention impl with LSE peer merge.

    ``get_name()`` stays "CUSTOM": vLLM's Attention layer looks the backend up
    by that enum member (ring_backend.py:439-441).
    """

    forward_includes_kv_cache_update: bool = False

    @staticmethod
    def get_name() -> str:
        return "CUSTOM"

    @staticmethod
    def get_impl_cls() -> type["HcpRingAttentionImpl"]:
        return HcpRingAttentionImpl

    @staticmethod
    def get_builder_cls():
        return _BuilderCls


class _Plan:
    """Launch descriptors for one forward call."""

    def __init__(self):
        self.local: list = []           # causal entries over the paged cache
        self.peer_rounds: list = []     # per round: {"contig": [...], "paged": [...]}
        self.any_peer = False
        self.ring: list = []  # decode-ring rows: (r, q row, tk, ring state, bt row, block 0)


class HcpRingAttentionImpl(_ImplBase):  # type: ignore[misc,valid-type]
    """HIP attention + LSE merge with peer chunk KV (ring_backend.py:452-834).

    Reads the paged cache in either vLLM 0.31 ``[nb, Hkv, bs, 2*D]`` or vLLM
    0.23 ``[nb, 2, bs, Hkv, D]`` layout, in place.  Peer KV is consumed from
    the staging dict (or from a split of the local cache) and never written.
    """

    def __init__(
        self,
        num_heads: int,
        head_size: int,
        scale: float,
        num_kv_heads: int | None = None,
        alibi_slopes: list[float] | None = None,
        sliding_window: int | None = None,
        kv_cache_dtype: str = "auto",
        logits_soft_cap: float | None = None,
        attn_type=AttentionType.DECODER,
        kv_sharing_target_layer_name: str | None = None,
        **kwargs,
    ) -> None:
        self.num_heads = num_heads
        self.head_size = head_size
        self.scale = float(scale)
        self.num_kv_heads = num_kv_heads if num_kv_heads is not None else num_heads
        self.kv_cache_dtype = kv_cache_dtype
        self.attn_type = attn_type
        self.kv_sharing_target_layer_name = kv_sharing_target_layer_name
        self.supports_quant_query_input = False
        if alibi_slopes is not None:
            raise NotImplementedError("HCP ring backend: ALiBi not supported")
        if logits_soft_cap:
            raise NotImplementedError("HCP ring backend: soft cap not supported")
        if sliding_window is not None and int(sliding_window) <= 0:
            raise ValueError("sliding_window must be a positive number of keys")
        if kv_cache_dtype not in ("auto", "float16", "bfloat16"):
            raise NotImplementedError(f"kv_cache_dtype {kv_cache_dtype} not supported")
        # the paged cache is read in place in 16-byte pieces (vLLM's flash
        # backends take the same head sizes)
        if head_size % 8 or not 0 < head_size <= 256:
            raise NotImplementedError(
                f"HCP ring backend: head_size {head_size} not supported (a multiple of 8 up to 256)")
        # applied to every causal pass (local segments), never to the
        # non-causal peer pass -- ring_backend.py:490-492,786,815,826-830
        self.sliding_window = int(sliding_window) if sliding_window is not None else None
        self.num_queries_per_kv = self.num_heads // self.num_kv_heads

    # -- paged KV write (the step before the path) ----------------------------
    def do_kv_cache_update(
        self,
        layer,
        key: torch.Tensor,
        value: torch.Tensor,
        kv_cache: torch.Tensor,
        slot_mapping: torch.Tensor,
    ) -> None:
        """Write this step's K/V into the paged cache at ``slot_mapping``.

        ring_backend.py:501-539 on the HIP cache-write kernel: slot = block *
        bs + offset, either cache layout.  The single-token decode steps of
        decode-ring requests are not written (their KV is decode growth,
        routed by the ring): those rows get slot -1, which the kernel skips,
        instead of three gather copies.
        """
        if self.attn_type in (AttentionType.ENCODER_ONLY, AttentionType.ENCODER):
            return
        skip = self._decode_ring_skip_positions(layer, slot_mapping)
        if skip:
            WRITE_TRACK["skipped"] += len(skip)
            slot_mapping = slot_mapping.clone()
            idx = torch.tensor(sorted(skip), dtype=torch.long, device=slot_mapping.device)
            slot_mapping.index_fill_(0, idx, -1)
        reshape_and_cache(key, value, kv_cache, slot_mapping)
        if WRITE_TRACK["enabled"]:
            WRITE_TRACK["slots"].update(s for s in slot_mapping.tolist() if s >= 0)

    def _decode_ring_skip_positions(self, layer, slot_mapping: torch.Tensor) -> set[int]:
        """Rows of this step's slot_mapping that are decode-ring requests'
        single-token decode steps (ring_backend.py:541-574); empty when the
        step's metadata is unavailable (never skip what cannot be attributed)."""
        if not (_decode_ring_enabled() and DECODE_RING_MAP):
            return set()
        meta = _forward_attn_metadata(layer)
        if meta is None:
            return set()
        qsl = meta.query_start_loc.tolist()
        first = meta.block_table[:, 0].tolist() if meta.block_table.shape[1] else []
        return {qsl[r] for r in range(len(qsl) - 1)
                if qsl[r + 1] - qsl[r] == 1 and int(first[r]) in DECODE_RING_MAP
                and qsl[r] < slot_mapping.shape[0]}

    # -- planning -------------------------------------------------------------
    def _peer_for_request(self, first_block: int, layer_name: str, n_reqs: int,
                          probe: bool = False):
        """Ordered staged (k, v) chunks of a request, or None (ring_backend.py:738-772).
        ``probe``: only look (no warning, no stream ordering)."""
        ck_list = PEER_REQ_MAP.get(first_block)
        if ck_list is None and n_reqs == 1:
            chunks = {key[0] for key in PEER_KV_STAGING}
            if len(chunks) == 1:
                ck_list = [next(iter(chunks))]
        if not ck_list:
            return None
        parts = []
        for ck in ck_list:
            kv = PEER_KV_STAGING.get((ck, layer_name))
            if kv is None:
                if not probe:
                    logger.warning(
                        "HCP ring: request mapped to chunks %s but staging incomplete at "
                        "layer %s; falling back to local path", ck_list, layer_name)
                return None
            parts.append(kv)
        if not probe:
            for ck, kv in zip(ck_list, parts):
                _wait_staged((ck, layer_name), kv)
        return parts

    def _write_probe(self, layer_name, qsl, seq_lens, block_table, first_blocks, pc,
                     ring_on: bool, split: int) -> None:
        """With write tracking on: every request that takes the ring path
        (a peer region of ``peer_end > 0`` positions, from staged chunks or the
        split env; decode-ring rows excepted) has its peer region's pool slots
        checked against the slots this worker wrote (ring_backend.py:790-810)."""
        ring_rows = _decode_ring_enabled() and bool(DECODE_RING_MAP)
        n = len(seq_lens)
        for r in range(n):
            tq, tk = qsl[r + 1] - qsl[r], int(seq_lens[r])
            if tq == 0 or (ring_rows and tq == 1 and first_blocks[r] in DECODE_RING_MAP):
                continue
            staged = (self._peer_for_request(first_blocks[r], layer_name, n, probe=True)
                      if ring_on else None)
            if staged is not None:
                peer_end = min(sum(int(kv[0].shape[0]) for kv in staged), tk)
            else:
                peer_end = min(split, tk) if split > 0 else 0
            if peer_end > 0:
                _probe_chunk_a_writes(block_table[r], peer_end, pc.block_size)

    def _plan(self, layer_name, qsl, seq_lens, block_table, first_blocks, pc, split):
        plan = _Plan()
        ring_on = _decode_ring_enabled() and bool(DECODE_RING_MAP)
        for r in range(len(seq_lens)):
            qs, qe = qsl[r], qsl[r + 1]
            tq, tk = qe - qs, seq_lens[r]
            if tq == 0:
                continue
            row = block_table[r]
            if ring_on and tq == 1:
                dr = DECODE_RING_MAP.get(first_blocks[r])
                if dr is not None:
                    plan.ring.append((r, qs, tk, dr, row, first_blocks[r]))
                    continue
            qpos0 = tk - tq
            staged = None
            if _ring_enabled():
                staged = self._peer_for_request(first_blocks[r], layer_name, len(seq_lens))
            peer_segs = []
            if staged is not None:
                total = sum(int(kv[0].shape[0]) for kv in staged)
                peer_end = min(total, tk)
                for kk, vv in staged:
                    if kk.shape[0] > 0:
                        peer_segs.append(segment_contiguous(kk, vv))
            elif split > 0:
                peer_end = min(split, tk)
                peer_segs.append(segment_paged(pc, row, 0, peer_end))
            else:
                peer_end = 0
            if peer_end == 0:
                plan.local.append(make_entry(qs, tq, segment_paged(pc, row, 0, tk), qpos0))
                continue
            n_a = max(0, min(tq, peer_end - qpos0))
            if n_a > 0:
                plan.local.append(make_entry(qs, n_a, segment_paged(pc, row, 0, tk), qpos0))
            if n_a < tq:
                qb0, nb = qs + n_a, tq - n_a
                plan.local.append(make_entry(
                    qb0, nb, segment_paged(pc, row, peer_end, tk - peer_end),
                    qpos0 + n_a - peer_end))
                for i, seg in enumerate(peer_segs):
                    while len(plan.peer_rounds) <= i:
                        plan.peer_rounds.append({"contig": [], "paged": []})
                    kind = "paged" if seg.block_table else "contig"
                    plan.peer_rounds[i][kind].append(make_entry(qb0, nb, seg, 0))
                    plan.any_peer = True
        return plan

    # -- forward ----------------------------------------------------------------
    def forward(
        self,
        layer,
        query: torch.Tensor,
        key: torch.Tensor,
        value: torch.Tensor,
        kv_cache: torch.Tensor,
        attn_metadata,
        output: torch.Tensor,
        output_scale: torch.Tensor | None = None,
        output_block_scale: torch.Tensor | None = None,
    ) -> torch.Tensor:
        if output_scale is not None or output_block_scale is not None:
            raise NotImplementedError("fused output quant not supported")
        if attn_metadata is None:
            return output.fill_(0)  # profiling run
        if self.attn_type != AttentionType.DECODER:
            raise NotImplementedError("HCP ring backend supports decoder attention only")
        _require_fast("HCP_RING_IMPL", _ring_impl())
        _require_fast("HCP_RING_MERGE", _merge_impl())

        num_actual = attn_metadata.num_actual_tokens
        query = query[:num_actual]
        out = output[:num_actual]
        pc = PagedCache.from_tensor(kv_cache)
        if pc.num_kv_heads != self.num_kv_heads or pc.head_dim != self.head_size:
            raise ValueError("kv_cache shape does not match the layer's heads/head_size")
        # small metadata tensors: one host sync per step (see _host_metadata)
        (qsl, seq_lens, first_blocks), block_table = _host_metadata(attn_metadata)
        BATCH_STATS["max_reqs"] = max(BATCH_STATS["max_reqs"], len(seq_lens))
        ring_on = _ring_enabled()
        split = _split_tokens() if ring_on else 0
        layer_name = getattr(layer, "layer_name", "")
        n = len(seq_lens)
        if self._peer_free(ring_on, split, first_blocks, n):
            self._forward_local_only(query, out, qsl, seq_lens, block_table, pc, kv_cache)
            return output
        if WRITE_TRACK["enabled"]:
            self._write_probe(layer_name, qsl, seq_lens, block_table, first_blocks, pc,
                              ring_on, split)

        is_decode = n > 0 and qsl == list(range(n + 1))
        if is_decode and self._forward_decode_staged(query, out, seq_lens, block_table,
                                                     first_blocks, pc, kv_cache, layer_name,
                                                     ring_on, split):
            return output
        plan = self._plan(layer_name, qsl, seq_lens, block_table, first_blocks, pc, split)
        ring_local = self._ring_local_segments(plan, pc, key, value, layer_name)
        if is_decode:
            lse = self._forward_decode(query, out, plan, n, ring_local)
            parts = {r: (out[qs:qs + 1], lse[:, qs:qs + 1]) for (r, qs, *_r) in plan.ring}
        else:
            if plan.local or plan.any_peer:
                self._forward_prefill(query, out, plan)
            parts = {}
            for (r, qs, *_r) in plan.ring:
                parts[r] = self._local_partial(query[qs:qs + 1], ring_local[r])
        for (r, qs, tk, dr, *_r) in plan.ring:
            o_acc, lse_acc = parts[r]
            out[qs:qs + 1] = self._ring_step(dr, layer_name, query[qs:qs + 1],
                                             o_acc, lse_acc)
        return output

    # -- memory-split decode (owner side) ----------------------------------------
    def _ring_local_segments(self, plan: _Plan, pc: PagedCache, key, value, layer_name):
        """Owner-side local segments of each decode-ring row: own chunk in the
        pool, the owner's growth share, the current token (ring_backend.py:
        643-671), with the growth bookkeeping of :652-689 done here (the
        current token joins the owner's growth or waits to be shipped)."""
        segs = {}
        for (r, qs, tk, dr, row, fb) in plan.ring:
            _release_staged_for_request(fb)
            plen = dr["prefix_len"]
            if dr["own_chunk_len"] is None:
                dr["own_chunk_len"] = tk - 1 - plen
            own_len = dr["own_chunk_len"]
            pos = tk - 1
            assignee = growth_assignee(pos, dr["ring_size"], dr["growth_policy"])
            dr["ship"] = dr["pending_growth"].pop(layer_name, None)
            k_cur = key[qs:qs + 1].contiguous()
            v_cur = value[qs:qs + 1].contiguous()
            g = dr["growth"].get(layer_name)
            if g is None:
                g = dr["growth"][layer_name] = GrowthBuffer(
                    self.num_kv_heads, self.head_size, k_cur.dtype, k_cur.device)
            own = segment_paged(pc, row, plen, own_len) if own_len > 0 else None
            if assignee == dr["own_index"]:
                g.append(k_cur, v_cur)
                local = [own, g.segment()]
            else:
                local = [own, g.segment(), segment_contiguous(k_cur, v_cur)]
                dr["pending_growth"][layer_name] = (assignee, k_cur, v_cur)
            # causal at len - 1 over the concatenation (:672-679): every key,
            # or the last `sliding_window` of them
            segs[r] = window_tail(local, self.sliding_window)
        return segs

    def _local_partial(self, q_r, segs):
        o, lse = local_partial(q_r, segs, self.num_kv_heads, self.scale)
        _count("decode")
        return o, lse

    def _ring_step(self, dr, layer_name, q_r, o_acc, lse_acc):
        """Send the owner's accumulator around the ring (ring_backend.py:
        690-722); the returned (O, LSE) is the exact attention of the step."""
        transport = dr.get("transport")
        if transport is None:
            raise RuntimeError("HCP decode ring requires a ring transport "
                               "(register_decode_ring(..., transport=...))")
        ship = dr.pop("ship", None)
        gk = gv = None
        target = -1
        if ship is not None:
            gk, gv = ship[1], ship[2]
            target = ship[0] + 1   # growth index 0..N-2 -> transport index 1..N-1
        first_chunk = dr["peer_chunks"][0][0] if dr["peer_chunks"] else ""
        o, _lse = ring_decode_step(transport, q_r, o_acc, lse_acc, self.scale, layer_name,
                                   first_chunk, req=dr["req_tag"], growth_k=gk,
                                   growth_v=gv, growth_target=target)
        IMPL_STATS["ring_decode_steps"] += 1
        return o

    # -- batches with no peer KV and no decode-ring rows -------------------------
    @staticmethod
    def _peer_free(ring_on: bool, split: int, first_blocks, n: int) -> bool:
        """No request of the batch takes a peer segment or the decode ring:
        the plain causal pass over the paged cache (ring_backend.py:783-789)."""
        if _decode_ring_enabled() and DECODE_RING_MAP and \
                any(fb in DECODE_RING_MAP for fb in first_blocks):
            return False
        if not ring_on:
            return True
        if split > 0:
            return False
        if not PEER_KV_STAGING:
            return True
        return n > 1 and not any(fb in PEER_REQ_MAP for fb in first_blocks)

    # -- pure decode batches with staged peers ------------------------------------
    def _decode_staged_template(self, seq_lens, block_table, first_blocks, pc, layer_name):
        """The step's decode entries with every field that does not change
        from layer to layer (lengths, block-table rows, strides of the cache),
        the split plan over them, and where each layer's addresses go; False
        if some request's staging is incomplete (the general path then
        decides, per layer, as the reference does)."""
        n = len(seq_lens)
        w = self.sliding_window
        seq, kinds, rows, starts, lens, peers = [], [], [], [], [], []
        for r in range(n):
            tk = int(seq_lens[r])
            staged = None
            if _ring_enabled():
                staged = self._peer_for_request(first_blocks[r], layer_name, n)
                if staged is None and PEER_REQ_MAP.get(first_blocks[r]):
                    return False  # staging still arriving: decided per layer
            peer_end = min(sum(int(kv[0].shape[0]) for kv in staged), tk) if staged else 0
            # one query at position tk - 1 (ring_backend.py:626-627): inside the
            # prefix it sees the whole local range (:811-817), else the local
            # keys past the prefix plus every staged chunk (:820-830)
            lo = 0 if peer_end == 0 or peer_end >= tk else peer_end
            if w is not None:  # the causal pass sees the last `w` local keys
                lo = max(lo, tk - w)
            seq.append(r); kinds.append(0); rows.append(r); starts.append(lo); lens.append(tk - lo)
            if 0 < peer_end < tk:
                ck_list = PEER_REQ_MAP.get(first_blocks[r])
                if ck_list is None:  # the single-request fallback of _peer_for_request
                    ck_list = [next(iter({key[0] for key in PEER_KV_STAGING}))]
                for ck, (kk, _vv) in zip(ck_list, staged):
                    if kk.shape[0] > 0:
                        seq.append(r); kinds.append(1); rows.append(r); starts.append(0)
                        lens.append(int(kk.shape[0]))
                        peers.append((len(seq) - 1, ck, int(kk.shape[0])))
        m = len(seq)
        kinds = np.asarray(kinds)
        loc = np.nonzero(kinds == 0)[0]
        tmpl = np.zeros(m, dtype=ENTRY_DTYPE)
        tmpl["q_start"] = seq
        tmpl["q_len"] = 1
        tmpl["start"] = starts
        tmpl["len"] = lens
        if len(loc):
            tmpl[loc] = paged_entry_array(pc, block_table, np.asarray(rows)[loc], tmpl["q_start"][loc],
                                          1, 0, tmpl["start"][loc], tmpl["len"][loc])
        first = tmpl.copy()
        for j, ck, _nt in peers:
            k, v = PEER_KV_STAGING[(ck, layer_name)]
            first[j] = _contiguous_record(j, seq[j], k, v)
        batch = DecodeBatch.from_entries(first, self.num_heads, self.num_kv_heads, self.head_size,
                                         block_table.device, entry_seq=np.asarray(seq, np.int32),
                                         num_seqs=n)
        return {"tmpl": tmpl, "loc": loc, "peers": peers, "batch": batch}

    def _forward_decode_staged(self, query, out, seq_lens, block_table, first_blocks, pc,
                               kv_cache, layer_name, ring_on, split) -> bool:
        """A pure decode batch without decode-ring rows: one split-KV launch
        over every request's local paged segment and staged peer chunks, its
        split plan built once per step and reused by every layer, each layer
        writing only its addresses (the cache, the layer's staged chunks) into
        the entries and uploading them in one small copy.  False when the
        general path must run (split env, decode-ring rows, staging that
        differs from the step's template)."""
        if split > 0 or (_decode_ring_enabled() and DECODE_RING_MAP
                         and any(fb in DECODE_RING_MAP for fb in first_blocks)):
            return False
        # (the staging generation: a chunk staged, dropped or mapped after the
        # template was built -- even for a request the template saw without
        # peers -- makes the next layer build a new one)
        key = ("dec_staged", self.sliding_window, pc.layout, pc.stride_tok, pc.stride_head,
               pc.stride_block, pc.block_size, pc.num_blocks, pc.v_addr - pc.k_addr, ring_on,
               _STAGE_GEN[0])
        st = _STEP["fast"].get(key)
        if st is None:
            st = self._decode_staged_template(seq_lens, block_table, first_blocks, pc, layer_name)
            _STEP["fast"][key] = st
        if st is False:
            return False
        ent = st["tmpl"].copy()
        ent["k_addr"][st["loc"]] = pc.k_addr
        ent["v_addr"][st["loc"]] = pc.v_addr
        keep = [kv_cache, block_table]
        for j, ck, nt in st["peers"]:
            kv = PEER_KV_STAGING.get((ck, layer_name))
            if kv is None or int(kv[0].shape[0]) != nt:
                return False
            _wait_staged((ck, layer_name), kv)
            ent[j] = _contiguous_record(j, int(ent["q_start"][j]), kv[0], kv[1])
            keep.append(kv)
        st["batch"].rebind(ent, keep).run(query, out, None, self.scale)
        _count("decode")
        return True

    def _forward_local_only(self, query, out, qsl, seq_lens, block_table, pc, kv_cache):
        """Causal attention of every request over its paged KV, the batch's
        entries built with array operations (once per step and cache layout,
        then only the layer's cache address changes): a split-KV decode for a
        pure decode batch, else one varlen launch."""
        n = len(seq_lens)
        if n == 0:
            return
        is_decode = qsl == list(range(n + 1))
        w = self.sliding_window
        key = (is_decode, w, pc.layout, pc.stride_tok, pc.stride_head, pc.stride_block,
               pc.block_size, pc.num_blocks, pc.v_addr - pc.k_addr)
        tmpl = _STEP["fast"].get(key)
        if tmpl is None:
            qs = np.asarray(qsl[:-1], dtype=np.int64)
            tq = np.diff(np.asarray(qsl, dtype=np.int64))
            tk = np.asarray(seq_lens, dtype=np.int64)
            rows = np.arange(n, dtype=np.int64)
            if is_decode:
                # one query at the end of its keys: all of them visible, or
                # the last `w` of them (ring_backend.py:397-398)
                start = np.zeros(n, np.int64) if w is None else np.maximum(tk - w, 0)
                tmpl = paged_entry_array(pc, block_table, rows, rows, 1, 0, start, tk - start)
            else:
                sel = tq > 0
                tmpl = paged_entry_array(pc, block_table, rows[sel], qs[sel], tq[sel],
                                         (tk - tq)[sel], 0, tk[sel])
            _STEP["fast"][key] = tmpl
        ent = tmpl.copy()
        ent["k_addr"] = pc.k_addr
        ent["v_addr"] = pc.v_addr
        keep = (kv_cache, block_table)
        if is_decode:
            DecodeBatch.from_entries(ent, self.num_heads, self.num_kv_heads, self.head_size,
                                     query.device, keep=keep).run(query, out, None, self.scale)
            _count("decode")
        else:
            lse = torch.empty((self.num_heads, query.shape[0]), dtype=torch.float32,
                              device=query.device)
            VarlenLaunch(ent, True, True, query.device, keep=keep).run(
                query, out, lse, self.num_kv_heads, self.scale, w)
            _count("attn")

    def _forward_prefill(self, query, out, plan: _Plan) -> None:
        dev = query.device
        h = self.num_heads
        if not plan.any_peer:
            lse = torch.empty((h, query.shape[0]), dtype=torch.float32, device=dev)
            VarlenLaunch(plan.local, True, True, dev).run(query, out, lse, self.num_kv_heads,
                                                         self.scale, self.sliding_window)
            _count("attn")
            return
        o_peer = lse_peer = None
        for rnd in plan.peer_rounds:
            o_r = torch.empty_like(query, memory_format=torch.contiguous_format)
            lse_r = torch.full((h, query.shape[0]), float("-inf"), dtype=torch.float32,
                               device=dev)
            for kind in ("contig", "paged"):
                if rnd[kind]:
                    VarlenLaunch(rnd[kind], False, kind == "paged", dev).run(
                        query, o_r, lse_r, self.num_kv_heads, self.scale)
                    _count("attn")
            if o_peer is None:
                o_peer, lse_peer = o_r, lse_r
            else:  # running merge of further prefix chunks (ring_decode.py:46-61)
                o_m = torch.empty_like(o_peer)
                lse_m = torch.empty_like(lse_peer)
                merge_attn_states(o_m, o_peer, lse_peer, o_r, lse_r, lse_m)
                _count("merge")
                o_peer, lse_peer = o_m, lse_m
        # Local causal pass merged with the peer result in the same launch:
        # merge_attn_states(out, o_peer, lse_peer, o_loc, lse_loc) with prefix
        # = peer, suffix = local (ring_backend.py:354,820-831), bit for bit.
        # The local entries cover every query row of the plan; rows without a
        # peer have lse_peer = -inf and get the local result.
        VarlenLaunch(plan.local, True, True, dev).run(
            query, out, None, self.num_kv_heads, self.scale, self.sliding_window,
            acc=(o_peer, lse_peer), acc_is_prefix=True)
        _count("attn")
        _count("merge")

    def _forward_decode(self, query, out, plan: _Plan, n: int, ring_local=None):
        """One split-KV launch for the whole decode batch; decode-ring rows
        get their owner-local partial (with LSE) from the same launch."""
        segs: list[list] = [[] for _ in range(n)]
        w = self.sliding_window
        for e in plan.local:
            kv = e.kv
            if w is not None:  # the causal local pass sees keys (off - w, off]
                kv = trim_segment(kv, min(kv.len, max(0, e.causal_offset - w + 1)))
            segs[e.q_start].append(kv)
        for rnd in plan.peer_rounds:
            for kind in ("contig", "paged"):
                for e in rnd[kind]:
                    segs[e.q_start].append(e.kv)
        lse = None
        for (r, qs, *_r) in plan.ring:
            segs[qs] = [s for s in ring_local[r] if s is not None and s.len > 0]
        if plan.ring:
            lse = torch.empty((self.num_heads, n), dtype=torch.float32, device=query.device)
        DecodeBatch(segs, self.num_heads, self.num_kv_heads, self.head_size,
                    query.device).run(query, out, lse, self.scale)
        _count("decode")
        return lse
