"""Decode accumulator step of the HCP decode ring, on the device.

In the reference's memory-split decode (hcp_vllm_plugin/ring_decode.py) a query
token's accumulator (O, LSE) travels around the ring; every node adds the
partial attention over its own chunk snapshot plus its share of the decode
growth and forwards the packet (``RingDecodeNode.handle_packet``, :187-259).
Per hop the reference decodes the packet, appends growth with ``torch.cat``
(:213-222, a full re-copy per token), concatenates chunk and growth
(:229-232), runs the prefill kernel with grid (H, 1) (:234-236), merges with
``merge_attn_states`` plus four elementwise ops for the LSE (``_merge_pair``,
:46-61) and re-encodes through three synchronous ``.cpu()`` copies
(:245-247, :340-342).

Here the same step keeps the packet format (:241-259, :336-355) and does:

* growth appended in place into per-(request, layer) device buffers with
  doubling capacity (amortised O(1) per token, no re-copy of the history);
* the local partial over the chunk snapshot and the growth as segments of one
  split-KV decode (all query heads of a KV head share each K/V read, the key
  range split over every CU) -- no concatenation -- whose second kernel also
  merges the accumulator and writes the merged LSE: two launches per hop, the
  split plan cached per (request, layer) until the growth changes;
* the host side of the packet through one pinned staging buffer: inputs go up
  with asynchronous copies, O and LSE come back with one copy pair and one
  stream synchronisation; fields the hop does not change (q, scale, names,
  forwarded growth) are passed through as received.

The ring transport (TCP, ring_transport.py) is not part of this build;
``start_relay`` and ``ring_decode_step`` take any object with
``send_packet(bytes)`` and ``recv_packet(timeout_s) -> bytes``.
"""

from __future__ import annotations

import logging
import os
import threading
import time

import torch

from .packet import Packet, encode, replace
from .packet import _NAMES as _DTYPE_NAMES
from .peer_ingest import PeerIngest
from .varlen import DecodeBatch, decode_attn, head_major, segment_contiguous

logger = logging.getLogger(__name__)

__all__ = [
    "RING_NODES",
    "growth_assignee",
    "encode_packet",
    "decode_packet",
    "GrowthBuffer",
    "RingDecodeNode",
    "ring_decode_step",
    "local_partial",
]


def growth_assignee(pos: int, ring_size: int, policy: str = "rr") -> int:
    """Ring node that keeps the KV of the decode token at global position
    ``pos`` (ring_decode.py:30-43): ``"rr"`` round-robin ``pos % N``,
    ``"owner"`` the owner (index N-1)."""
    if policy == "owner":
        return ring_size - 1
    return pos % ring_size


# ---------------------------------------------------------------------------
# Packet codec (the wire format)
# ---------------------------------------------------------------------------
class _HostStage:
    """One pinned host buffer, grown on demand, for the packet's tensors.

    ``down`` copies device tensors into it (asynchronously, on the current
    stream) and synchronises once; ``up`` stages host tensors into it and
    issues one asynchronous copy of them all to the device, recording an
    event that the next use of the buffer waits for.
    """

    def __init__(self):
        self._buf: torch.Tensor | None = None
        self._busy: torch.cuda.Event | None = None

    def _get(self, nbytes: int) -> torch.Tensor:
        if self._busy is not None:
            self._busy.synchronize()
            self._busy = None
        if self._buf is None or self._buf.numel() < nbytes:
            self._buf = torch.empty(max(nbytes, 1 << 16), dtype=torch.uint8, pin_memory=True)
        return self._buf

    @staticmethod
    def _layout(tensors):
        offs, o = [], 0
        for t in tensors:
            o = (o + 255) & ~255
            offs.append(o)
            o += t.numel() * t.element_size()
        return offs, o

    def _view(self, buf, off, t):
        n = t.numel() * t.element_size()
        return buf[off:off + n].view(t.dtype).view(t.shape)

    def up_bytes(self, fields: list, device) -> tuple[torch.Tensor, list[int]]:
        """``fields``: uint8 arrays (e.g. a packet's byte ranges), staged with
        numpy copies and sent up in one copy.  Returns the device buffer and
        each field's byte offset in it."""
        offs, o = [], 0
        for f in fields:
            o = (o + 255) & ~255
            offs.append(o)
            o += f.size
        buf = self._get(o)
        pin = buf.numpy()
        for off, f in zip(offs, fields):
            pin[off:off + f.size] = f
        dev = torch.empty(max(o, 1), dtype=torch.uint8, device=device)
        dev[:o].copy_(buf[:o], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(device))
        self._busy = ev
        return dev, offs

    def down(self, tensors: list[torch.Tensor]) -> list[torch.Tensor]:
        dev = [t for t in tensors if t.is_cuda]
        offs, total = self._layout(dev)
        buf = self._get(total)
        views = {}
        for off, t in zip(offs, dev):
            v = self._view(buf, off, t)
            v.copy_(t, non_blocking=True)
            views[id(t)] = v
        if dev:
            torch.cuda.current_stream(dev[0].device).synchronize()
        return [views.get(id(t), t) for t in tensors]

    def up(self, tensors: list[torch.Tensor], device) -> list[torch.Tensor]:
        offs, total = self._layout(tensors)
        buf = self._get(total)
        for off, t in zip(offs, tensors):
            self._view(buf, off, t).copy_(t)
        # one host-to-device copy of the whole staging area into a fresh
        # device buffer (so the returned tensors own their memory)
        dev = torch.empty(max(total, 1), dtype=torch.uint8, device=device)
        dev[:total].copy_(buf[:total], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(device))
        self._busy = ev
        return [self._view(dev, off, t) for off, t in zip(offs, tensors)]


def encode_packet(q, o, lse, scale, layer, chunk, req="", growth_k=None, growth_v=None,
                  growth_target=-1, stage: _HostStage | None = None) -> bytes:
    """The accumulator packet in the reference's wire format (ring_decode.py:
    336-355): safetensors of ``chunk``/``layer``/``req`` (uint8 bytes), ``q``,
    ``o``, ``lse``, ``scale`` (float32 [1]) and optional ``growth_k``,
    ``growth_v``, ``growth_target`` (int64 [1]).  Device tensors come down
    through one pinned buffer with one synchronisation."""
    ts = [q.detach().contiguous(), o.detach().contiguous(), lse.detach().contiguous()]
    with_growth = growth_k is not None and growth_v is not None
    if with_growth:
        ts += [growth_k.detach().contiguous(), growth_v.detach().contiguous()]
    if any(t.is_cuda for t in ts):
        ts = (stage or _HostStage()).down(ts)
    d = {"chunk": chunk, "layer": layer, "req": req, "q": ts[0], "o": ts[1], "lse": ts[2],
         "scale": torch.tensor([float(scale)], dtype=torch.float32)}
    if with_growth:
        d["growth_k"], d["growth_v"] = ts[3], ts[4]
        d["growth_target"] = torch.tensor([int(growth_target)], dtype=torch.int64)
    return encode(d)


def decode_packet(payload: bytes) -> dict:
    """Parse a packet: strings decoded, ``scale`` / ``growth_target`` as
    Python numbers, tensors left on the host."""
    pkt = Packet(payload)
    out = {k: pkt.tensor(k) for k in pkt.meta}
    for k in ("chunk", "layer", "req"):
        if k in pkt:
            out[k] = pkt.text(k)
    out.setdefault("req", "")
    out["scale"] = float(pkt.item("scale"))
    if "growth_target" in pkt:
        out["growth_target"] = int(pkt.item("growth_target"))
    return out


# ---------------------------------------------------------------------------
# Growth storage and the local partial
# ---------------------------------------------------------------------------
class GrowthBuffer:
    """Decode-growth K/V ``[len, Hkv, D]`` of one (request, layer), appended
    in place; capacity doubles when full (one copy of the history per
    doubling instead of one per token)."""

    def __init__(self, num_kv_heads: int, head_dim: int, dtype, device, capacity: int = 64):
        self.k = torch.empty(capacity, num_kv_heads, head_dim, dtype=dtype, device=device)
        self.v = torch.empty_like(self.k)
        self.len = 0

    def append(self, k: torch.Tensor, v: torch.Tensor) -> None:
        n = k.shape[0]
        if self.len + n > self.k.shape[0]:
            cap = max(2 * self.k.shape[0], self.len + n)
            nk = torch.empty((cap,) + tuple(self.k.shape[1:]), dtype=self.k.dtype,
                             device=self.k.device)
            nv = torch.empty_like(nk)
            nk[:self.len].copy_(self.k[:self.len])
            nv[:self.len].copy_(self.v[:self.len])
            self.k, self.v = nk, nv
        self.k[self.len:self.len + n].copy_(k)
        self.v[self.len:self.len + n].copy_(v)
        self.len += n

    def segment(self):
        return segment_contiguous(self.k, self.v, 0, self.len) if self.len else None


def local_partial(q: torch.Tensor, segments: list, num_kv_heads: int, scale: float):
    """(O ``[T, H, D]``, LSE ``[H, T]``) of every query row of ``q`` over all
    keys of ``segments`` (non-causal), one split-KV decode launch.  An empty
    key set gives LSE = -inf, which the merge treats as an empty partial."""
    segs = [s for s in segments if s is not None and s.len > 0]
    if not segs:
        o = torch.zeros_like(q, memory_format=torch.contiguous_format)
        lse = torch.full((q.shape[1], q.shape[0]), float("-inf"), dtype=torch.float32,
                         device=q.device)
        return o, lse
    return decode_attn(q, [segs] * q.shape[0], num_kv_heads, scale, with_lse=True)


RING_NODES: list["RingDecodeNode"] = []


class RingDecodeNode:
    """A ring node's decode state and its accumulator step.

    Constructor as the reference's (ring_decode.py:107-121): the node's chunk
    snapshot is ``store_dir/<chunk_key>/<layer>.safetensors`` with
    ``{"k","v"}: [n, Hkv, D]``, complete once ``<chunk_key>/_READY`` exists.
    It is read in a background thread (``background=True``, as the reference)
    through ``PeerIngest`` (pinned parallel reads, asynchronous uploads), or by
    calling ``load()``; ``add_chunk`` installs device tensors directly.
    """

    def __init__(self, store_dir: str, chunk_keys: list[str], ring_index: int,
                 device: str = "cuda", dtype: torch.dtype = torch.float16,
                 background: bool = True):
        self._store_dir = store_dir
        self._chunk_keys = list(chunk_keys)
        self._ring_index = ring_index
        self._device = torch.device(device)
        if self._device.type == "cuda" and self._device.index is None:
            self._device = torch.device("cuda", torch.cuda.current_device())
        self._dtype = dtype
        self._layers: dict[tuple[str, str], tuple[torch.Tensor, torch.Tensor]] = {}
        self._growth: dict[tuple[str, str], GrowthBuffer] = {}
        self._growth_appends: dict[str, int] = {}
        self._plans: dict[tuple[str, str], tuple[tuple, DecodeBatch]] = {}
        self._ready = threading.Event()
        self._calls = 0
        self._running = False
        self._transport = None
        self._stage = _HostStage()
        RING_NODES.append(self)
        if background:
            threading.Thread(target=self.load, daemon=True).start()

    # -- chunk snapshot ------------------------------------------------------
    def load(self, wait_s: float = 3600.0, poll_s: float = 0.5) -> None:
        t0 = time.time()
        torch.cuda.set_device(self._device)
        ing = PeerIngest(self._device, "k_v")
        for ck in self._chunk_keys:
            cdir = os.path.join(self._store_dir, ck)
            waited = 0.0
            while not os.path.exists(os.path.join(cdir, "_READY")) and waited < wait_s:
                time.sleep(poll_s)
                waited += poll_s
            for fname in sorted(os.listdir(cdir)):
                if not fname.endswith(".safetensors"):
                    continue
                got = ing.load([os.path.join(cdir, fname)])
                got.event.synchronize()
                self.add_chunk(ck, fname[: -len(".safetensors")], got.k, got.v)
        logger.info("RingDecodeNode[%d]: chunks %s loaded (%d layers, %.1fs)",
                    self._ring_index, self._chunk_keys, len(self._layers), time.time() - t0)
        self._ready.set()

    def add_chunk(self, chunk_key: str, layer: str, k: torch.Tensor, v: torch.Tensor) -> None:
        """Install one layer of a chunk snapshot (``[n, Hkv, D]`` each), stored
        head-major like staged peer KV: installed once, read at every hop."""
        k = head_major(k.to(self._device, self._dtype))
        v = head_major(v.to(self._device, self._dtype))
        self._layers[(chunk_key, layer)] = (k, v)

    def mark_ready(self) -> None:
        self._ready.set()

    def wait_ready(self, timeout_s: float = 600) -> bool:
        return self._ready.wait(timeout_s)

    def is_ready(self) -> bool:
        return self._ready.is_set()

    @property
    def ring_index(self) -> int:
        return self._ring_index

    @property
    def calls(self) -> int:
        return self._calls

    @property
    def growth_appends(self) -> int:
        return sum(self._growth_appends.values())

    def growth_tokens(self) -> int:
        """Growth tokens per layer, summed over requests."""
        per_req: dict[str, int] = {}
        for (req, _layer), g in self._growth.items():
            per_req[req] = g.len
        return sum(per_req.values())

    def growth_stats(self) -> dict[str, int]:
        """Growth tokens per layer, per request (isolation evidence)."""
        per_req: dict[str, int] = {}
        for (req, _layer), g in self._growth.items():
            per_req[req] = g.len
        return per_req

    def drop_request(self, req: str) -> None:
        """Free a finished request's growth."""
        for key in [k for k in self._growth if k[0] == req]:
            del self._growth[key]
        for key in [k for k in self._plans if k[0] == req]:
            del self._plans[key]
        self._growth_appends.pop(req, None)

    # -- the accumulator step -----------------------------------------------
    def append_growth(self, req: str, layer: str, gk: torch.Tensor, gv: torch.Tensor) -> None:
        key = (req, layer)
        g = self._growth.get(key)
        if g is None:
            g = self._growth[key] = GrowthBuffer(gk.shape[1], gk.shape[2], self._dtype,
                                                 self._device)
        g.append(gk, gv)
        self._growth_appends[req] = self._growth_appends.get(req, 0) + 1

    def _accumulate_into(self, q, o_acc, lse_acc, scale, layer, req, chunk, out, lse) -> None:
        my_chunk = self._chunk_keys[0] if self._chunk_keys else chunk
        k, v = self._layers[(my_chunk, layer)]
        # the packet's q sets the kernel's row width and head count: it must
        # match this node's KV, or the kernel would read rows of another width
        if q.dim() != 3 or q.shape[2] != k.shape[2] or q.shape[1] % k.shape[1] != 0:
            raise ValueError(
                f"decode-ring packet q {tuple(q.shape)} does not match this node's KV "
                f"[n, {k.shape[1]}, {k.shape[2]}] (head_dim must agree, heads a multiple "
                f"of the KV heads)")
        if tuple(o_acc.shape) != tuple(q.shape) or tuple(lse_acc.shape) != (q.shape[1], q.shape[0]):
            raise ValueError("decode-ring packet o/lse shapes do not match q")
        g = self._growth.get((req, layer))
        glen = g.len if g is not None else 0
        sig = (k.data_ptr(), k.shape[0], g.k.data_ptr() if glen else 0, glen, tuple(q.shape))
        plan = self._plans.get((req, layer))
        if plan is None or plan[0] != sig:
            segs = [segment_contiguous(k, v)] + ([g.segment()] if glen else [])
            plan = (sig, DecodeBatch([segs] * q.shape[0], q.shape[1], k.shape[1], q.shape[2],
                                     q.device))
            self._plans[(req, layer)] = plan
        plan[1].run(q, out, lse, scale, acc=(o_acc, lse_acc))

    def accumulate(self, q: torch.Tensor, o_acc: torch.Tensor, lse_acc: torch.Tensor,
                   scale: float, layer: str, req: str = "",
                   chunk: str = "") -> tuple[torch.Tensor, torch.Tensor]:
        """Device-only hop: (O, LSE) of the accumulator merged with this
        node's partial over its chunk snapshot plus this request's growth
        (non-causal), ring_decode.py:224-237.  The node's own chunk key is
        used; ``chunk`` (the packet's) only when the node has none."""
        out = torch.empty_like(q, memory_format=torch.contiguous_format)
        lse = torch.empty((q.shape[1], q.shape[0]), dtype=torch.float32, device=q.device)
        self._accumulate_into(q, o_acc, lse_acc, scale, layer, req, chunk, out, lse)
        return out, lse

    def handle_packet(self, payload: bytes) -> bytes:
        """One hop on a packet (ring_decode.py:187-259): growth addressed to
        this node appended, partial merged into the accumulator, the updated
        packet returned; growth for another node is forwarded unchanged.

        Host side: the packet is parsed in place; q, o, lse (and consumed
        growth) go up in one copy; the new O and LSE land in one device
        buffer and come down in one copy; the reply is the received bytes with
        the ``o`` and ``lse`` ranges rewritten whenever the key set and dtypes
        stay the same (no re-serialisation)."""
        pkt = Packet(payload)
        layer = pkt.text("layer")
        req = pkt.text("req") if "req" in pkt else ""
        dname = _DTYPE_NAMES.get(self._dtype)
        same = (pkt.meta["q"]["dtype"] == dname and pkt.meta["o"]["dtype"] == dname
                and pkt.meta["lse"]["dtype"] == "F32")
        consumed = False
        if "growth_k" in pkt:
            target = int(pkt.item("growth_target")) if "growth_target" in pkt else self._ring_index
            consumed = target == self._ring_index
        names = ["q", "o", "lse"] + (["growth_k", "growth_v"] if consumed else [])
        if same and (not consumed or (pkt.meta["growth_k"]["dtype"] == dname
                                      and pkt.meta["growth_v"]["dtype"] == dname)):
            # the packet's bytes go up as they are
            buf, offs = self._stage.up_bytes([pkt.raw(n) for n in names], self._device)
            dev = []
            for n, off in zip(names, offs):
                dt = torch.float32 if n == "lse" else self._dtype
                nb = pkt.raw(n).size
                dev.append(buf[off:off + nb].view(dt).view(pkt.shape(n)))
        else:
            dev = self._stage.up([pkt.tensor(n).to(torch.float32 if n == "lse" else self._dtype)
                                  for n in names], self._device)
        q, o_acc, lse_acc = dev[0], dev[1], dev[2]
        if consumed:
            self.append_growth(req, layer, dev[3], dev[4])
        # O and LSE in one device buffer, so they come down in one copy
        no = q.numel() * q.element_size()
        lo = (no + 255) & ~255
        res = torch.empty(lo + q.shape[1] * q.shape[0] * 4, dtype=torch.uint8, device=q.device)
        o = res[:no].view(q.dtype).view(q.shape)
        lse = res[lo:].view(torch.float32).view(q.shape[1], q.shape[0])
        self._accumulate_into(q, o_acc, lse_acc, float(pkt.item("scale")), layer, req,
                              pkt.text("chunk"), o, lse)
        self._calls += 1
        (res_h,) = self._stage.down([res])
        if same and not consumed:
            pin = res_h.numpy()
            return replace(pkt, {"o": pin[:no], "lse": pin[lo:lo + q.shape[1] * q.shape[0] * 4]})
        o_h = res_h[:no].view(q.dtype).view(q.shape)
        lse_h = res_h[lo:].view(torch.float32).view(q.shape[1], q.shape[0])
        out = {"chunk": pkt.tensor("chunk"), "layer": pkt.tensor("layer"),
               "q": pkt.tensor("q").to(self._dtype), "o": o_h, "lse": lse_h,
               "scale": pkt.tensor("scale")}
        if "req" in pkt:
            out["req"] = pkt.tensor("req")
        if "growth_k" in pkt and not consumed:
            out["growth_k"] = pkt.tensor("growth_k")
            out["growth_v"] = pkt.tensor("growth_v")
            if "growth_target" in pkt:
                out["growth_target"] = pkt.tensor("growth_target")
        return encode(out)

    # -- relay loop (non-owner nodes) ----------------------------------------
    def start_relay(self, transport) -> None:
        """Background loop: receive a packet, run the hop, forward it."""
        if self._running:
            return
        self._running = True
        self._transport = transport
        threading.Thread(target=self._relay_loop, daemon=True).start()

    def stop_relay(self) -> None:
        self._running = False

    def _relay_loop(self) -> None:
        if not self.wait_ready(timeout_s=3600):
            logger.warning("RingDecodeNode[%d]: chunk store never became ready", self._ring_index)
            return
        torch.cuda.set_device(self._device)
        transport = self._transport
        while self._running:
            try:
                payload = transport.recv_packet(timeout_s=1.0)
            except TimeoutError:
                continue
            except Exception as e:  # noqa: BLE001 -- transport closed
                if self._running:
                    logger.warning("RingDecodeNode[%d]: relay recv error: %s",
                                   self._ring_index, e)
                break
            try:
                transport.send_packet(self.handle_packet(payload))
            except Exception as e:  # noqa: BLE001 -- keep the relay alive
                logger.warning("RingDecodeNode[%d]: relay handle/forward error: %s",
                               self._ring_index, e)


_OWNER_STAGE = threading.local()


def ring_decode_step(transport, q, o_acc, lse_acc, scale, layer, chunk, req="",
                     growth_k=None, growth_v=None, growth_target=-1, timeout_s=600):
    """Owner side (ring_decode.py:314-362): send the accumulator packet into
    the ring and block until it comes back; returns the final (O in q's
    dtype, LSE float32) on q's device."""
    stage = getattr(_OWNER_STAGE, "stage", None)
    if stage is None:
        stage = _OWNER_STAGE.stage = _HostStage()
    transport.send_packet(encode_packet(q, o_acc, lse_acc, scale, layer, chunk, req,
                                        growth_k, growth_v, growth_target, stage=stage))
    pkt = Packet(transport.recv_packet(timeout_s=timeout_s))
    o_h, lse_h = pkt.tensor("o").to(q.dtype), pkt.tensor("lse").to(torch.float32)
    if not q.is_cuda:
        return o_h, lse_h
    o, lse = stage.up([o_h, lse_h], q.device)
    return o, lse
