"""Writes the golden fixtures of this directory (run from the repo root:
``python tests/golden/make_golden.py``).

The reference (stark-sim/hcp-vllm-plugin) commits no golden vectors and its
kernel probe draws CUDA-seeded inputs that cannot be regenerated on a CPU
(validate_ring_triton_kernel.py:38,49-51).  These fixtures are therefore
computed here by an independent route -- vectorised float64 numpy with an
explicit max-shifted softmax, not the torch oracle -- from seeded CPU inputs:

* ``micro.npz``: H=4, Hkv=2, D=16, Tq=Tk=8, inputs and outputs stored in
  full, causal at offset 0 and 3 and non-causal.
* ``plumbing_7b_256.npz``: the CPU plumbing case of the reference's fp32
  torch path at the Qwen2.5-7B attention shape (28 query heads, 4 KV heads,
  head_dim 128, scale 1/sqrt(128)): 256 local tokens causal at frame offset 0
  (global positions 256..511 over local keys 256..511) and 256 peer tokens
  (global 0..255) non-causal, q/k/v drawn N(0,1) in fp32 from
  ``torch.Generator().manual_seed(0)`` in the order q, k_local, v_local,
  k_peer, v_peer, rounded to fp16 and upcast.  Stored: SHA-256 of the fp16
  input bytes, both segments' LSE [H, T] in full, and every 32nd token of the
  local, peer and merged outputs.

The merge follows ring_backend.py:409-421 (m = max, w = exp(l - m),
(o1 w1 + o2 w2)/(w1 + w2)).
"""

import hashlib
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
SUB = 32  # token stride of the stored output subsample


def attn64(q, k, v, scale, off):
    """float64 attention with LSE; q [Tq,H,D], k/v [Tk,Hkv,D] numpy."""
    tq, h, d = q.shape
    tk, hkv = k.shape[0], k.shape[1]
    g = h // hkv
    heads = np.arange(h) // g
    kk = k[:, heads]            # [Tk, H, D]
    vv = v[:, heads]
    s = np.einsum("ihd,jhd->hij", q, kk) * scale
    if off is not None:
        vis = np.arange(tk)[None, :] <= off + np.arange(tq)[:, None]
        s = np.where(vis[None], s, -np.inf)
    m = s.max(-1, keepdims=True)
    w = np.exp(s - m)
    den = w.sum(-1)
    out = np.einsum("hij,jhd->ihd", w, vv) / den.T[..., None]
    lse = m[..., 0] + np.log(den)
    return out, lse


def merge64(o1, l1, o2, l2):
    m = np.maximum(l1, l2)
    w1, w2 = np.exp(l1 - m).T[..., None], np.exp(l2 - m).T[..., None]
    return (o1 * w1 + o2 * w2) / (w1 + w2)


def draw(seed, shapes, dtype):
    gen = torch.Generator().manual_seed(seed)
    return [torch.randn(*s, generator=gen).to(dtype) for s in shapes]


def micro():
    q, k, v = draw(11, [(8, 4, 16), (8, 2, 16), (8, 2, 16)], torch.float32)
    q, k, v = (t.double().numpy() for t in (q, k, v))
    res = {"q": q, "k": k, "v": v, "scale": np.float64(0.25)}
    for name, off in (("c0", 0), ("c3", 3), ("nc", None)):
        o, l = attn64(q, k, v, 0.25, off)
        res[f"out_{name}"] = o
        res[f"lse_{name}"] = l
    np.savez(os.path.join(HERE, "micro.npz"), **res)


def plumbing():
    h, hkv, d, n = 28, 4, 128, 256
    ts = draw(0, [(n, h, d), (n, hkv, d), (n, hkv, d), (n, hkv, d), (n, hkv, d)],
              torch.float16)
    sha = hashlib.sha256(b"".join(t.numpy().tobytes() for t in ts)).hexdigest()
    q, kl, vl, kp, vp = (t.double().numpy() for t in ts)
    scale = 1.0 / np.sqrt(d)
    o_l, l_l = attn64(q, kl, vl, scale, 0)
    o_p, l_p = attn64(q, kp, vp, scale, None)
    o_m = merge64(o_l, l_l, o_p, l_p)
    np.savez_compressed(
        os.path.join(HERE, "plumbing_7b_256.npz"),
        input_sha256=np.array(sha), sub=np.int64(SUB),
        lse_local=l_l.astype(np.float32), lse_peer=l_p.astype(np.float32),
        out_local=o_l[::SUB].astype(np.float32), out_peer=o_p[::SUB].astype(np.float32),
        out_merged=o_m[::SUB].astype(np.float32))


if __name__ == "__main__":
    micro()
    plumbing()
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))
