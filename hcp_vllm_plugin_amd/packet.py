"""The decode ring's packet codec: safetensors read and written directly.

The packet is a safetensors file (ring_decode.py:241-259,336-355): a
little-endian u64 header length N, N bytes of JSON mapping each tensor name to
``{"dtype", "shape", "data_offsets": [begin, end]}`` (offsets relative to the
end of the header; an optional ``"__metadata__"`` entry), then the tensor
bytes.  A hop changes only the accumulator (``o``, ``lse``) and keeps every
other field, so the reply is the received bytes with those two ranges
rewritten -- no re-serialisation.  A packet whose key set changes (growth
consumed by this node) is written by :func:`encode`, which emits the same
format ``safetensors.torch.save`` reads.
"""

from __future__ import annotations

import json
import math
import struct

import numpy as np
import torch

__all__ = ["Packet", "encode", "replace"]

_DTYPES = {
    "BF16": torch.bfloat16, "F16": torch.float16, "F32": torch.float32,
    "F64": torch.float64, "I64": torch.int64, "I32": torch.int32, "I16": torch.int16,
    "I8": torch.int8, "U8": torch.uint8, "BOOL": torch.bool,
}
_NAMES = {v: k for k, v in _DTYPES.items()}
_SIZES = {"BF16": 2, "F16": 2, "F32": 4, "F64": 8, "I64": 8, "I32": 4, "I16": 2, "I8": 1,
          "U8": 1, "BOOL": 1}
_NP_SCALARS = {"F32": np.float32, "F64": np.float64, "I64": np.int64, "I32": np.int32,
               "I16": np.int16, "I8": np.int8, "U8": np.uint8}


class Packet:
    """A parsed packet: tensors are views of one private copy of the bytes."""

    __slots__ = ("buf", "base", "meta")

    def __init__(self, payload: bytes | bytearray | memoryview):
        self.buf = bytearray(payload)
        if len(self.buf) < 8:
            raise ValueError("packet shorter than its header length")
        n = struct.unpack_from("<Q", self.buf, 0)[0]
        if 8 + n > len(self.buf):
            raise ValueError("packet header runs past the payload")
        meta = json.loads(bytes(self.buf[8:8 + n]))
        meta.pop("__metadata__", None)
        self.base = 8 + n
        for name, m in meta.items():
            b, e = m["data_offsets"]
            if m["dtype"] not in _DTYPES or not (0 <= b <= e <= len(self.buf) - self.base):
                raise ValueError(f"packet tensor {name!r}: bad dtype or offsets")
            if e - b != math.prod(m["shape"]) * _SIZES[m["dtype"]]:
                raise ValueError(f"packet tensor {name!r}: {e - b} bytes for shape {m['shape']}")
        self.meta = meta

    def __contains__(self, name: str) -> bool:
        return name in self.meta

    def span(self, name: str) -> tuple[int, int]:
        """Absolute byte range of ``name`` in the packet."""
        b, e = self.meta[name]["data_offsets"]
        return self.base + b, self.base + e

    def dtype(self, name: str) -> torch.dtype:
        return _DTYPES[self.meta[name]["dtype"]]

    def shape(self, name: str) -> list:
        return self.meta[name]["shape"]

    def raw(self, name: str) -> np.ndarray:
        """The tensor's bytes, a uint8 view of the packet."""
        b, e = self.span(name)
        return np.frombuffer(self.buf, dtype=np.uint8, count=e - b, offset=b)

    def tensor(self, name: str) -> torch.Tensor:
        """Host tensor of ``name`` (a view of the packet's bytes when aligned)."""
        m = self.meta[name]
        dt = _DTYPES[m["dtype"]]
        b, e = self.span(name)
        esz = torch.empty((), dtype=dt).element_size()
        if e == b:
            return torch.empty(m["shape"], dtype=dt)
        if b % esz:
            raw = torch.frombuffer(bytearray(self.buf[b:e]), dtype=torch.uint8)
        else:
            raw = torch.frombuffer(self.buf, dtype=torch.uint8, count=e - b, offset=b)
        return raw.view(dt).view(m["shape"])

    def text(self, name: str) -> str:
        b, e = self.span(name)
        return bytes(self.buf[b:e]).decode()

    def item(self, name: str):
        """First element of a numeric tensor as a Python number."""
        m = self.meta[name]
        npt = _NP_SCALARS.get(m["dtype"])
        if npt is None:
            return self.tensor(name).reshape(-1)[0].item()
        b, e = self.span(name)
        if e - b < np.dtype(npt).itemsize:
            raise ValueError(f"packet tensor {name!r} is empty")
        return np.frombuffer(bytes(self.buf[b:b + np.dtype(npt).itemsize]), dtype=npt)[0].item()


def _bytes_of(t: torch.Tensor) -> np.ndarray:
    t = t.detach().contiguous()
    if t.is_cuda:
        raise ValueError("packet tensors must be on the host")
    return t.reshape(-1).view(torch.uint8).numpy() if t.numel() else np.empty(0, np.uint8)


def encode(tensors: dict) -> bytes:
    """Write host tensors (or ``str`` values, stored as uint8 bytes) as a
    safetensors file.  Tensors are laid out by decreasing element size, so each
    starts aligned to its own size."""
    items = []
    for name, t in tensors.items():
        if isinstance(t, str):
            t = torch.frombuffer(bytearray(t.encode()), dtype=torch.uint8) if t else \
                torch.empty(0, dtype=torch.uint8)
        items.append((name, t))
    items.sort(key=lambda kv: (-kv[1].element_size(), kv[0]))
    header, parts, off = {}, [], 0
    for name, t in items:
        data = _bytes_of(t)
        header[name] = {"dtype": _NAMES[t.dtype], "shape": list(t.shape),
                        "data_offsets": [off, off + data.size]}
        parts.append(data)
        off += data.size
    h = json.dumps(header, separators=(",", ":")).encode()
    h += b" " * (-(8 + len(h)) % 8)
    out = bytearray(8 + len(h) + off)
    struct.pack_into("<Q", out, 0, len(h))
    out[8:8 + len(h)] = h
    pos = 8 + len(h)
    view = np.frombuffer(out, dtype=np.uint8)
    for data in parts:
        view[pos:pos + data.size] = data
        pos += data.size
    return bytes(out)


def replace(pkt: Packet, values: dict) -> bytes:
    """The packet's bytes with the named tensors' data replaced.  A value is a
    host tensor of the packet's dtype and shape, or a uint8 array of exactly
    the tensor's byte length."""
    out = bytearray(pkt.buf)
    view = np.frombuffer(out, dtype=np.uint8)
    for name, t in values.items():
        m = pkt.meta[name]
        b, e = pkt.span(name)
        if isinstance(t, np.ndarray):
            if t.dtype != np.uint8 or t.size != e - b:
                raise ValueError(f"packet tensor {name!r}: {t.size} bytes for a {e - b}-byte field")
            view[b:e] = t.reshape(-1)
            continue
        if _DTYPES[m["dtype"]] != t.dtype or list(t.shape) != m["shape"]:
            raise ValueError(f"packet tensor {name!r}: {t.dtype} {tuple(t.shape)} does not "
                             f"match {m['dtype']} {m['shape']}")
        view[b:e] = _bytes_of(t)
    return bytes(out)
