"""Batched (varlen) prefill and split-KV decode on the HIP kernels.

The reference runs one flash launch per request and segment and gathers the
paged local KV into a contiguous copy first (ring_backend.py:611-832,
:617-624).  This module describes a whole batch as ``hcp_varlen_entry``
records -- query rows plus a KV segment that is either contiguous (staged
peer chunks) or paged (the local KV cache, read in place through the block
table) -- and runs one launch per segment kind:

* ``varlen_attn_with_lse``: causal (local) or non-causal (peer) prefill over
  every entry, tiles ordered longest-first by ``hcp_plan_varlen_tiles``.
* ``decode_attn``: split-KV decode of single-token queries; every segment of a
  sequence (peer and local) is split, and one reduce merges all partials.

Paged layouts the reference reads: vLLM 0.31 ``[nb, Hkv, bs, 2*D]`` with
K in ``[..., :D]`` and V in ``[..., D:]`` (file_connector.py:13-16,175-179),
and vLLM 0.23 ``[nb, 2, bs, Hkv, D]`` (ring_backend.py:601,617-624).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

import torch

from . import _lib
from ._lib import DecodeSplit, KvSegment, VarlenEntry

__all__ = [
    "PagedCache",
    "segment_contiguous",
    "segment_paged",
    "varlen_attn_with_lse",
    "plan_varlen_tiles",
    "DecodeBatch",
    "decode_attn",
    "choose_split_tokens",
    "head_major",
]


@dataclass
class PagedCache:
    """A paged KV cache and its element strides.

    ``layout`` is ``"v031"`` for ``[nb, Hkv, bs, 2*D]`` or ``"v023"`` for
    ``[nb, 2, bs, Hkv, D]``; ``from_tensor`` infers it from the rank.
    """

    cache: torch.Tensor
    layout: str
    num_kv_heads: int
    head_dim: int
    block_size: int
    k_addr: int
    v_addr: int
    stride_tok: int
    stride_head: int
    stride_block: int

    @property
    def num_blocks(self) -> int:
        return int(self.cache.shape[0])

    @classmethod
    def from_tensor(cls, cache: torch.Tensor) -> "PagedCache":
        if cache.stride(-1) != 1:
            raise ValueError("paged cache: last dim must be contiguous")
        es = cache.element_size()
        if cache.dim() == 4:  # [nb, Hkv, bs, 2D]
            nb, hkv, bs, d2 = cache.shape
            d = d2 // 2
            return cls(cache, "v031", hkv, d, bs, cache.data_ptr(),
                       cache.data_ptr() + d * es,
                       cache.stride(2), cache.stride(1), cache.stride(0))
        if cache.dim() == 5 and cache.shape[1] == 2:  # [nb, 2, bs, Hkv, D]
            nb, _, bs, hkv, d = cache.shape
            return cls(cache, "v023", hkv, d, bs, cache.data_ptr(),
                       cache.data_ptr() + cache.stride(1) * es,
                       cache.stride(2), cache.stride(3), cache.stride(0))
        raise ValueError(f"unrecognised paged cache shape {tuple(cache.shape)}")


def segment_contiguous(k: torch.Tensor, v: torch.Tensor, start: int = 0,
                       length: int | None = None) -> KvSegment:
    """Segment over tokens ``[start, start+length)`` of k/v ``[T, Hkv, D]``."""
    if k.shape != v.shape or k.stride() != v.stride():
        raise ValueError("k and v must share shape and strides")
    _check_kv_layout(k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1), 0, k.element_size())
    if k.stride(-1) != 1:
        raise ValueError("k/v head_dim must be contiguous")
    n = k.shape[0] - start if length is None else length
    if start < 0 or n < 0 or start + n > k.shape[0]:
        raise ValueError("segment out of range")
    s = KvSegment()
    s.k_addr = k.data_ptr()
    s.v_addr = v.data_ptr()
    s.block_table = 0
    s.stride_tok = k.stride(0)
    s.stride_head = k.stride(1)
    s.stride_block = 0
    s.start = start
    s.len = n
    s.block_size = 0
    s._keep = (k, v)  # the descriptor holds raw addresses: keep the storage alive
    return s


def _check_kv_layout(k_addr: int, v_addr: int, stride_tok: int, stride_head: int,
                     stride_block: int, esize: int) -> None:
    """Kernel loadability: 16-byte aligned rows, token stride below 2^24 elements."""
    if k_addr % 16 or v_addr % 16:
        raise ValueError("k/v base addresses must be 16-byte aligned")
    if (stride_tok * esize) % 16 or (stride_head * esize) % 16 or (stride_block * esize) % 16:
        raise ValueError("k/v strides must be multiples of 16 bytes")
    if not 0 < stride_tok < (1 << 24):
        raise ValueError("k/v token stride must be in (0, 2^24) elements")


def segment_paged(pc: PagedCache, block_table_row: torch.Tensor, start: int,
                  length: int) -> KvSegment:
    """Segment over tokens ``[start, start+length)`` of one request's paged KV.

    ``block_table_row`` is the request's int32 block-table row on the device
    (contiguous); token x lives in block ``row[x // bs]`` at ``x % bs``.
    """
    if block_table_row.dtype != torch.int32 or block_table_row.stride(-1) != 1:
        raise ValueError("block table row must be contiguous int32")
    _check_kv_layout(pc.k_addr, pc.v_addr, pc.stride_tok, pc.stride_head, pc.stride_block,
                     pc.cache.element_size())
    if pc.block_size <= 0 or pc.block_size & (pc.block_size - 1):
        raise ValueError("block_size must be a power of two")
    if start < 0 or length < 0:
        raise ValueError("negative segment start/length")
    nblk = (start + length + pc.block_size - 1) // pc.block_size
    if length > 0 and nblk > block_table_row.shape[0]:
        raise ValueError("segment extends past the block-table row")
    s = KvSegment()
    s.k_addr = pc.k_addr
    s.v_addr = pc.v_addr
    s.block_table = block_table_row.data_ptr()
    s.stride_tok = pc.stride_tok
    s.stride_head = pc.stride_head
    s.stride_block = pc.stride_block
    s.start = start
    s.len = length
    s.block_size = pc.block_size
    s.num_blocks = pc.num_blocks if pc.num_blocks < (1 << 31) else 0
    s._keep = (pc.cache, block_table_row)  # raw addresses inside: keep them alive
    return s


def trim_segment(seg: KvSegment, skip: int) -> KvSegment:
    """The same keys without the first ``skip`` (0 <= skip <= len)."""
    if not 0 <= skip <= seg.len:
        raise ValueError("trim beyond the segment")
    s = KvSegment()
    ctypes.memmove(ctypes.addressof(s), ctypes.addressof(seg), ctypes.sizeof(KvSegment))
    s.start = seg.start + skip
    s.len = seg.len - skip
    s._keep = getattr(seg, "_keep", None)
    return s


def window_tail(segments: list, window: int | None) -> list:
    """The last ``window`` keys of the concatenation of ``segments`` (in
    order): what a query at the last position sees under a sliding window
    (ring_backend.py:397-398 with qpos = len - 1).  None keeps all keys."""
    segs = [s for s in segments if s is not None and s.len > 0]
    if window is None:
        return segs
    if window <= 0:
        raise ValueError("window must be a positive number of keys")
    out, need = [], window
    for s in reversed(segs):
        if need == 0:
            break
        out.append(s if s.len <= need else trim_segment(s, s.len - need))
        need -= min(need, s.len)
    return out[::-1]


def make_entry(q_start: int, q_len: int, seg: KvSegment, causal_offset: int = 0) -> VarlenEntry:
    e = VarlenEntry()
    e.q_start = q_start
    e.q_len = q_len
    e.causal_offset = causal_offset
    e.kv = seg
    e._keep = getattr(seg, "_keep", None)
    return e


def _nbytes_addr(a) -> tuple[int, int]:
    if isinstance(a, np.ndarray):
        return a.nbytes, a.ctypes.data
    return ctypes.sizeof(a), ctypes.addressof(a)


def _upload(arrays, device: torch.device):
    """Copy ctypes or numpy arrays to the device in one asynchronous copy from
    pinned memory on the current stream.

    Returns (device byte tensor, [address of each array on the device]), each
    array 256-byte aligned.  The pinned block comes from torch's caching host
    allocator, which keeps it until the copy has completed.
    """
    offs, total = [], 0
    for a in arrays:
        offs.append(total)
        total += (_nbytes_addr(a)[0] + 255) & ~255
    host = torch.empty(max(total, 256), dtype=torch.uint8, pin_memory=True)
    base = host.data_ptr()
    for a, o in zip(arrays, offs):
        nb, addr = _nbytes_addr(a)
        ctypes.memmove(base + o, addr, nb)
    dev = host.to(device, non_blocking=True)
    return dev, [dev.data_ptr() + o for o in offs]


# hcp_varlen_entry as a numpy record (include/hcp_mi355x.h), for building a
# whole batch's entries with array operations instead of one object each
ENTRY_DTYPE = np.dtype({
    "names": ["q_start", "q_len", "causal_offset", "k_addr", "v_addr", "block_table",
              "stride_tok", "stride_head", "stride_block", "start", "len", "block_size",
              "num_blocks"],
    "formats": ["<i8", "<i8", "<i8", "<u8", "<u8", "<u8", "<i8", "<i8", "<i8", "<i8", "<i8",
                "<i4", "<i4"],
    "offsets": [0, 8, 16, 24, 32, 40, 48, 56, 64, 72, 80, 88, 92],
    "itemsize": 96,
})
assert ENTRY_DTYPE.itemsize == ctypes.sizeof(VarlenEntry)


def paged_entry_array(pc: "PagedCache", block_table: torch.Tensor, rows, q_start, q_len,
                      causal_offset, start, length) -> np.ndarray:
    """Entries over the paged cache for many requests at once: entry i covers
    query rows [q_start[i], +q_len[i]) and tokens [start[i], +length[i]) of
    block-table row rows[i].  ``block_table`` is the batch's contiguous int32
    table on the device; all checks are done once for the batch."""
    if block_table.dtype != torch.int32 or not block_table.is_contiguous():
        raise ValueError("block table must be contiguous int32")
    _check_kv_layout(pc.k_addr, pc.v_addr, pc.stride_tok, pc.stride_head, pc.stride_block,
                     pc.cache.element_size())
    if pc.block_size <= 0 or pc.block_size & (pc.block_size - 1):
        raise ValueError("block_size must be a power of two")
    rows = np.asarray(rows, dtype=np.int64)
    start = np.asarray(start, dtype=np.int64)
    length = np.asarray(length, dtype=np.int64)
    if (start < 0).any() or (length < 0).any():
        raise ValueError("negative segment start/length")
    nblk = (start + length + pc.block_size - 1) // pc.block_size
    if ((length > 0) & (nblk > block_table.shape[1])).any():
        raise ValueError("segment extends past the block-table row")
    a = np.zeros(len(rows), dtype=ENTRY_DTYPE)
    a["q_start"] = q_start
    a["q_len"] = q_len
    a["causal_offset"] = causal_offset
    a["k_addr"] = pc.k_addr
    a["v_addr"] = pc.v_addr
    a["block_table"] = block_table.data_ptr() + rows * block_table.stride(0) * 4
    a["stride_tok"] = pc.stride_tok
    a["stride_head"] = pc.stride_head
    a["stride_block"] = pc.stride_block
    a["start"] = start
    a["len"] = length
    a["block_size"] = pc.block_size
    a["num_blocks"] = pc.num_blocks if pc.num_blocks < (1 << 31) else 0
    return a


def plan_varlen_tiles(entries: list[VarlenEntry], causal: bool) -> list[tuple[int, int]]:
    """Host tile plan (entry, q_block), longest first (hcp_plan_varlen_tiles)."""
    L = _lib.lib()
    n = len(entries)
    arr = (VarlenEntry * max(n, 1))(*entries)
    bm = L.hcp_varlen_block_m(128, _lib.DTYPE_BF16)
    cap = sum((e.q_len + bm - 1) // bm for e in entries)
    tiles = (ctypes.c_int32 * max(2 * cap, 2))()
    rc = L.hcp_plan_varlen_tiles(ctypes.addressof(arr), n, int(causal), bm,
                                 ctypes.addressof(tiles), cap)
    _lib.check(rc, "hcp_plan_varlen_tiles")
    return [(tiles[2 * i], tiles[2 * i + 1]) for i in range(rc)]


# smallest block_size the paged prefill kernel reads in place (a wave's 16
# rows of a tile must lie in one block); smaller ones are gathered first
_MIN_PAGED_BLOCK = 16


class VarlenLaunch:
    """A planned varlen launch: entries and tile list uploaded to the device.

    Build once per batch layout; ``run`` may be called repeatedly (e.g. per
    layer, or per benchmark step) with any q/out/lse of matching rows.  The
    plan is uploaded asynchronously on the current stream: run it on that
    stream (or synchronise first).
    """

    def __init__(self, entries, causal: bool, paged: bool, device: torch.device, keep=None):
        """``entries``: a list of VarlenEntry, or an ENTRY_DTYPE array (then
        ``keep`` holds the tensors its addresses point into)."""
        L = _lib.lib()
        self.causal = bool(causal)
        self.paged = bool(paged)
        self.num_entries = len(entries)
        bm = L.hcp_varlen_block_m(128, _lib.DTYPE_BF16)
        if isinstance(entries, np.ndarray):
            if entries.dtype != ENTRY_DTYPE or not entries.flags.c_contiguous:
                raise ValueError("entry array must be contiguous ENTRY_DTYPE")
            if ((entries["block_table"] != 0) != self.paged).any():
                raise ValueError("all entries of a launch must share the KV form")
            arr = entries if self.num_entries else np.zeros(1, dtype=ENTRY_DTYPE)
            cap = int(((entries["q_len"] + bm - 1) // bm).sum())
            self._keep = keep
        else:
            for e in entries:
                if (e.kv.block_table != 0) != self.paged:
                    raise ValueError("all entries of a launch must share the KV form")
            arr = (VarlenEntry * max(self.num_entries, 1))(*entries)
            cap = sum((e.q_len + bm - 1) // bm for e in entries)
            # the entries point at K/V / cache / block-table storage by
            # address: hold those tensors for as long as this launch can run
            self._keep = [getattr(e, "_keep", None) for e in entries]
        # Paged prefill reads a wave's 16 rows of a tile from one block: over a
        # cache with shorter blocks the segments are gathered into one
        # contiguous K/V buffer on the device first (hcp_gather_paged_kv, one
        # launch per run), and the attention runs over that copy.
        self._gather = None
        if self.paged and self.num_entries:
            host = np.frombuffer(arr, dtype=ENTRY_DTYPE, count=self.num_entries).copy()
            if int(host["block_size"].min()) < _MIN_PAGED_BLOCK:
                lens = host["len"].astype(np.int64)
                out_start = np.zeros(self.num_entries, dtype=np.int64)
                out_start[1:] = np.cumsum(lens)[:-1]
                cont = host.copy()
                for f in ("block_table", "stride_block", "block_size", "num_blocks",
                          "k_addr", "v_addr"):
                    cont[f] = 0
                cont["start"] = out_start
                self._gather = {"paged": host, "out_start": out_start, "cont": cont,
                                "total": int(lens.sum()), "max_len": int(lens.max()),
                                "bufs": {}}
                arr = cont
                self.paged = False
        tiles = (ctypes.c_int32 * max(2 * cap, 2))()
        rc = L.hcp_plan_varlen_tiles(_nbytes_addr(arr)[1], self.num_entries,
                                     int(self.causal), bm, ctypes.addressof(tiles), cap)
        _lib.check(rc, "hcp_plan_varlen_tiles")
        self.num_tiles = rc
        if self._gather is None:
            self._plan_dev, (self.entries_ptr, self.tiles_ptr) = _upload([arr, tiles], device)
        else:
            g = self._gather
            self._plan_dev, (g["paged_ptr"], g["start_ptr"], self.tiles_ptr) = _upload(
                [g["paged"], g["out_start"], tiles], device)
            self.entries_ptr = None
        self.device = device

    def _gathered(self, q: torch.Tensor, num_kv_heads: int) -> int:
        """Gather mode: copy every entry's paged keys into a contiguous K/V
        buffer on the current stream; returns the device address of the
        entries over that buffer.

        The buffer (and its uploaded entries) is allocated on the first run
        of a (shape, stream) pair and reused by later runs on that stream,
        which the stream orders after each other; a run on another stream
        gets buffers of its own, so runs in flight on two streams never
        overwrite each other's keys.  Each buffer holds ``total * Hkv * D``
        16-bit elements of K and of V for as long as the launch lives."""
        g = self._gather
        head_dim = q.shape[2]
        st = torch.cuda.current_stream(q.device)
        key = (num_kv_heads, head_dim, q.dtype, st.cuda_stream)
        buf = g["bufs"].get(key)
        if buf is None:
            k = torch.empty(max(g["total"], 1), num_kv_heads, head_dim, dtype=q.dtype,
                            device=q.device)
            v = torch.empty_like(k)
            cont = g["cont"].copy()
            cont["k_addr"] = k.data_ptr()
            cont["v_addr"] = v.data_ptr()
            cont["stride_tok"] = num_kv_heads * head_dim
            cont["stride_head"] = head_dim
            cont_dev, (ptr,) = _upload([cont], q.device)
            buf = g["bufs"][key] = (k, v, cont_dev, ptr)
        k, v, _cont_dev, ptr = buf
        L = _lib.lib()
        rc = L.hcp_gather_paged_kv(g["paged_ptr"], self.num_entries, g["start_ptr"],
                                   g["max_len"], num_kv_heads, head_dim,
                                   _lib.dtype_code(q.dtype), k.data_ptr(),
                                   v.data_ptr(), _lib.stream_ptr(q.device))
        _lib.check(rc, "hcp_gather_paged_kv")
        return ptr

    def run(self, q: torch.Tensor, out: torch.Tensor, lse: torch.Tensor | None,
            num_kv_heads: int, scale: float, window: int | None = None,
            acc=None, acc_is_prefix: bool = True) -> None:
        """``window``: sliding window of a causal launch (query at p sees keys
        p - window < j <= p in its entry's frame); ignored when non-causal.

        ``acc=(o, lse)``: a partial state with out's rows, merged into the
        result in the same launch (``hcp_attn_fwd_varlen_merge``): with
        ``acc_is_prefix`` each row gets merge_attn_states(acc, this pass), the
        local pass taking the peer result as the prefix (ring_backend.py:354).
        ``lse`` may then be None; otherwise it receives the merged LSE."""
        if self.num_tiles == 0:
            return
        if window is not None and window <= 0:
            raise ValueError("window must be a positive number of keys")
        num_heads, head_dim = q.shape[1], q.shape[2]
        L = _lib.lib()
        win = int(window or 0) if self.causal else 0
        with torch.cuda.device(q.device):
            entries_ptr = self.entries_ptr
            if self._gather is not None:
                entries_ptr = self._gathered(q, num_kv_heads)
            if acc is None:
                rc = L.hcp_attn_fwd_varlen(
                    q.data_ptr(), q.stride(0), q.stride(1),
                    out.data_ptr(), out.stride(0), out.stride(1),
                    lse.data_ptr(), lse.stride(0),
                    entries_ptr, self.num_entries,
                    self.tiles_ptr, self.num_tiles,
                    num_heads, num_kv_heads, head_dim, float(scale),
                    int(self.causal), win, int(self.paged),
                    _lib.dtype_code(q.dtype), _lib.stream_ptr(q.device),
                )
                _lib.check(rc, "hcp_attn_fwd_varlen")
                return
            a_o, a_lse = acc
            if a_o.dtype != q.dtype or a_o.stride(-1) != 1 or a_lse.dtype != torch.float32:
                raise ValueError("acc must be (out in q.dtype, float32 lse)")
            rc = L.hcp_attn_fwd_varlen_merge(
                q.data_ptr(), q.stride(0), q.stride(1),
                out.data_ptr(), out.stride(0), out.stride(1),
                0 if lse is None else lse.data_ptr(), 0 if lse is None else lse.stride(0),
                entries_ptr, self.num_entries,
                self.tiles_ptr, self.num_tiles,
                num_heads, num_kv_heads, head_dim, float(scale),
                int(self.causal), win, int(self.paged),
                a_o.data_ptr(), a_o.stride(0), a_o.stride(1),
                a_lse.data_ptr(), a_lse.stride(0), int(bool(acc_is_prefix)),
                _lib.dtype_code(q.dtype), _lib.stream_ptr(q.device),
            )
        _lib.check(rc, "hcp_attn_fwd_varlen_merge")


def varlen_attn_with_lse(
    q: torch.Tensor,
    entries: list[VarlenEntry],
    causal: bool,
    num_kv_heads: int,
    scale: float,
    out: torch.Tensor | None = None,
    lse: torch.Tensor | None = None,
    window: int | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """One launch over all entries.  Rows not covered by an entry are left as
    given (``out``/``lse`` allocated here start as 0 / -inf).  ``window``: as
    ``VarlenLaunch.run``."""
    if q.dtype not in (torch.float16, torch.bfloat16) or q.stride(-1) != 1:
        raise ValueError("q must be float16/bfloat16 with contiguous head_dim")
    paged = bool(entries) and entries[0].kv.block_table != 0
    if out is None:
        out = torch.zeros_like(q, memory_format=torch.contiguous_format)
    if lse is None:
        lse = torch.full((q.shape[1], q.shape[0]), float("-inf"), dtype=torch.float32,
                         device=q.device)
    VarlenLaunch(entries, causal, paged, q.device).run(q, out, lse, num_kv_heads, scale, window)
    return out, lse


def head_major(t: torch.Tensor) -> torch.Tensor:
    """``t`` (``[n, Hkv, D]``) as an ``[n, Hkv, D]`` view of an ``[Hkv, n, D]``
    buffer, so each KV head's keys are one contiguous run (returned as is if
    already so stored)."""
    if t.dim() != 3 or t.stride() == (t.shape[2], t.shape[0] * t.shape[2], 1):
        return t
    return t.permute(1, 0, 2).contiguous().permute(1, 0, 2)


def head_chunks(num_heads: int, num_kv_heads: int) -> int:
    """Decode workgroups per (split, KV head): the split kernel takes up to 16
    query heads of a KV group at a time."""
    return -(-(num_heads // num_kv_heads) // 16)


def choose_split_tokens(seg_lens: list[int], num_kv_heads: int, num_cus: int = 256,
                        max_rounds: int = 4, round_keys: int = 2048, minimum: int = 64,
                        maximum: int = 16384) -> int:
    """Split size from the batch's total key count.

    The split kernel runs one workgroup per CU at a time (its chunk buffers
    take 128 KB of LDS), so the launch is planned in whole rounds of
    ``num_cus`` (split, KV head) workgroups: one round while the work is
    small (a single long request -- a decode-ring hop -- spread over the whole
    machine), up to ``max_rounds`` once each workgroup would stream more than
    ``round_keys`` keys, so the launch drains evenly while each split stays
    long enough that its fp32 partial is small next to the K/V it summarises.
    Several rounds: rounded up to 64 keys.  One round: the smallest split
    whose pieces fill at most one workgroup per CU.
    """
    total = sum(seg_lens) * num_kv_heads
    if total == 0:
        return minimum
    rounds = min(max_rounds, max(1, -(-total // (num_cus * round_keys))))
    s = -(-total // (rounds * num_cus))
    if rounds == 1:
        # one round: the smallest split whose pieces (every segment cut into
        # ceil(len / s) of them) fit the machine, so a single long request
        # occupies every CU
        lens = [n for n in seg_lens if n > 0]
        lo, hi = max(minimum, s), max(max(lens), minimum)
        while lo < hi:
            mid = (lo + hi) // 2
            if sum(-(-n // mid) for n in lens) * num_kv_heads <= num_cus:
                hi = mid
            else:
                lo = mid + 1
        return min(maximum, lo)
    s = ((s + 63) // 64) * 64
    return max(minimum, min(maximum, s))


class DecodeBatch:
    """A planned split-KV decode: entries and splits on the device (the fp32
    partials' workspace is taken per run).

    ``segments[s]`` lists the KV segments of sequence ``s`` (all keys visible
    to its single query, e.g. the staged peer prefix and the local paged KV
    including the current token).  The plan is uploaded asynchronously on the
    current stream: run it on that stream (or synchronise first).
    """

    def __init__(self, segments: list[list[KvSegment]], num_heads: int, num_kv_heads: int,
                 head_dim: int, device: torch.device, split_tokens: int | None = None):
        L = _lib.lib()
        entries, seq_of = [], []
        for s, segs in enumerate(segments):
            for seg in segs:
                entries.append(make_entry(s, 1, seg, 0))
                seq_of.append(s)
        self.num_seqs = len(segments)
        self.num_entries = len(entries)
        if split_tokens is None:
            split_tokens = choose_split_tokens([e.kv.len for e in entries],
                                               num_kv_heads * head_chunks(num_heads, num_kv_heads))
        self.split_tokens = split_tokens
        arr = (VarlenEntry * max(self.num_entries, 1))(*entries)
        seq_arr = (ctypes.c_int32 * max(self.num_entries, 1))(*seq_of)
        cap = sum(-(-e.kv.len // split_tokens) for e in entries)
        splits = (DecodeSplit * max(cap, 1))()
        starts = (ctypes.c_int32 * (self.num_seqs + 1))()
        rc = L.hcp_plan_decode_splits(ctypes.addressof(arr), self.num_entries,
                                      ctypes.addressof(seq_arr), self.num_seqs, 0,
                                      split_tokens, ctypes.addressof(splits), cap,
                                      ctypes.addressof(starts))
        _lib.check(rc, "hcp_plan_decode_splits")
        self.num_splits = rc
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self._plan_dev, (self.entries_ptr, self.splits_ptr, self.starts_ptr) = _upload(
            [arr, splits, starts], device)
        self.ws_bytes = int(L.hcp_decode_workspace_bytes(max(rc, 1), num_heads, head_dim))
        self.device = device
        # the segments point at K/V / cache / block-table storage by address
        self._keep = [getattr(e, "_keep", None) for e in entries]

    @classmethod
    def from_entries(cls, entries: np.ndarray, num_heads: int, num_kv_heads: int,
                     head_dim: int, device: torch.device, split_tokens: int | None = None,
                     keep=None, entry_seq: np.ndarray | None = None,
                     num_seqs: int | None = None) -> "DecodeBatch":
        """Entries given as an ENTRY_DTYPE array; ``keep`` holds the tensors
        it points into.  By default one entry per sequence (sequence i = entry
        i = query row i); with ``entry_seq`` (int32, non-decreasing) entry j
        belongs to sequence ``entry_seq[j]`` of ``num_seqs`` -- a sequence's
        peer chunks and its local segment."""
        if entries.dtype != ENTRY_DTYPE or not entries.flags.c_contiguous:
            raise ValueError("entry array must be contiguous ENTRY_DTYPE")
        L = _lib.lib()
        self = cls.__new__(cls)
        n = len(entries)
        if entry_seq is None:
            seq_arr = np.arange(max(n, 1), dtype=np.int32)
            ns = n
        else:
            seq_arr = np.ascontiguousarray(entry_seq, dtype=np.int32)
            if len(seq_arr) != n or num_seqs is None:
                raise ValueError("entry_seq needs one sequence per entry and num_seqs")
            ns = int(num_seqs)
            if n == 0:
                seq_arr = np.zeros(1, dtype=np.int32)
        self.num_seqs = ns
        self.num_entries = n
        lens = entries["len"]
        if split_tokens is None:
            split_tokens = choose_split_tokens([int(lens.sum())],
                                               num_kv_heads * head_chunks(num_heads, num_kv_heads))
        self.split_tokens = split_tokens
        arr = entries if n else np.zeros(1, dtype=ENTRY_DTYPE)
        cap = int(((lens + split_tokens - 1) // split_tokens).sum())
        splits = (DecodeSplit * max(cap, 1))()
        starts = (ctypes.c_int32 * (ns + 1))()
        rc = L.hcp_plan_decode_splits(arr.ctypes.data, n, seq_arr.ctypes.data, ns, 0,
                                      split_tokens, ctypes.addressof(splits), cap,
                                      ctypes.addressof(starts))
        _lib.check(rc, "hcp_plan_decode_splits")
        self.num_splits = rc
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self._plan_dev, (self.entries_ptr, self.splits_ptr, self.starts_ptr) = _upload(
            [arr, splits, starts], device)
        self.ws_bytes = int(L.hcp_decode_workspace_bytes(max(rc, 1), num_heads, head_dim))
        self.device = device
        self._keep = keep
        return self

    def rebind(self, entries: np.ndarray, keep=None) -> "DecodeBatch":
        """The same plan (splits, partial slots) over new entries of the same
        layout and lengths -- another layer's cache and staged chunks: only
        the entries go to the device (one small asynchronous copy)."""
        if entries.dtype != ENTRY_DTYPE or not entries.flags.c_contiguous:
            raise ValueError("entry array must be contiguous ENTRY_DTYPE")
        if len(entries) != self.num_entries:
            raise ValueError("rebind needs the plan's entry count")
        other = object.__new__(type(self))
        other.__dict__.update(self.__dict__)
        arr = entries if len(entries) else np.zeros(1, dtype=ENTRY_DTYPE)
        other._entries_dev, (other.entries_ptr,) = _upload([arr], self.device)
        other._keep = keep
        return other

    def run(self, q: torch.Tensor, out: torch.Tensor, lse: torch.Tensor | None,
            scale: float, acc: tuple[torch.Tensor, torch.Tensor] | None = None,
            noalloc: bool = False) -> None:
        """Decode into ``out`` (and ``lse``).  With ``acc = (o_acc [S, H, D] in
        q's dtype, lse_acc [H, S] float32)`` the accumulator is merged in by the
        same launch (``hcp_decode_splitkv_acc``); ``out`` / ``lse`` may be the
        accumulator's own tensors.

        ``noalloc``: run ``hcp_decode_splitkv_noalloc`` instead, whose partials
        live in the library's fixed per-GPU scratch (no workspace is taken, so
        nothing is allocated; calls overlapping on one GPU race).  Plans whose
        partials exceed ``_lib.NOALLOC_SCRATCH_BYTES`` raise."""
        L = _lib.lib()
        if noalloc:
            if acc is not None:
                raise ValueError("noalloc decode has no accumulator form")
            with torch.cuda.device(q.device):
                rc = L.hcp_decode_splitkv_noalloc(
                    q.data_ptr(), q.stride(0), q.stride(1),
                    self.entries_ptr, self.num_entries,
                    self.splits_ptr, self.num_splits,
                    self.starts_ptr, self.num_seqs,
                    out.data_ptr(), out.stride(0), out.stride(1),
                    lse.data_ptr() if lse is not None else None,
                    lse.stride(0) if lse is not None else 0,
                    self.num_heads, self.num_kv_heads, self.head_dim, float(scale),
                    _lib.dtype_code(q.dtype), _lib.stream_ptr(q.device))
            _lib.check(rc, "hcp_decode_splitkv_noalloc")
            return
        # fp32 partials: stream-ordered scratch from torch's caching allocator
        workspace = torch.empty(self.ws_bytes, dtype=torch.uint8, device=q.device)
        head = (q.data_ptr(), q.stride(0), q.stride(1),
                self.entries_ptr, self.num_entries,
                self.splits_ptr, self.num_splits,
                self.starts_ptr, self.num_seqs,
                workspace.data_ptr(), self.ws_bytes)
        tail = (out.data_ptr(), out.stride(0), out.stride(1),
                lse.data_ptr() if lse is not None else None,
                lse.stride(0) if lse is not None else 0,
                self.num_heads, self.num_kv_heads, self.head_dim, float(scale),
                _lib.dtype_code(q.dtype), _lib.stream_ptr(q.device))
        with torch.cuda.device(q.device):
            if acc is None:
                rc = L.hcp_decode_splitkv(*head, *tail)
                name = "hcp_decode_splitkv"
            else:
                ao, al = acc
                if ao.dtype != q.dtype or tuple(ao.shape) != tuple(q.shape) or ao.stride(-1) != 1:
                    raise ValueError("acc o must match q's dtype and shape, contiguous head_dim")
                if al.dtype != torch.float32 or tuple(al.shape) != (q.shape[1], q.shape[0]) \
                        or al.stride(1) != 1:
                    raise ValueError("acc lse must be float32 [H, S], contiguous along S")
                if not (ao.is_cuda and al.is_cuda):
                    raise ValueError("accumulator must be on the GPU")
                rc = L.hcp_decode_splitkv_acc(
                    *head, ao.data_ptr(), ao.stride(0), ao.stride(1), al.data_ptr(),
                    al.stride(0), *tail)
                name = "hcp_decode_splitkv_acc"
        _lib.check(rc, name)


def decode_attn(
    q: torch.Tensor,
    segments: list[list[KvSegment]],
    num_kv_heads: int,
    scale: float,
    out: torch.Tensor | None = None,
    with_lse: bool = False,
    split_tokens: int | None = None,
    acc: tuple[torch.Tensor, torch.Tensor] | None = None,
):
    """Split-KV decode: q ``[S, H, D]`` (one token per sequence) over all
    segments of each sequence, merged (and merged into ``acc`` when given).
    Returns out (and lse ``[H, S]``)."""
    if q.dtype not in (torch.float16, torch.bfloat16) or q.stride(-1) != 1:
        raise ValueError("q must be float16/bfloat16 with contiguous head_dim")
    if len(segments) != q.shape[0]:
        raise ValueError("one segment list per query row")
    s, h, d = q.shape
    batch = DecodeBatch(segments, h, num_kv_heads, d, q.device, split_tokens)
    if out is None:
        out = torch.empty_like(q, memory_format=torch.contiguous_format)
    lse = torch.empty((h, s), dtype=torch.float32, device=q.device) if with_lse else None
    batch.run(q, out, lse, scale, acc)
    return (out, lse) if with_lse else out
