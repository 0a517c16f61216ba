"""End-to-end plumbing check: greedy tokens through the ring backend.

A tiny seeded decoder with random weights (2 layers, Qwen2.5-7B attention
shape: 28 query heads, 4 KV heads, head_dim 128, RoPE) generates greedily
twice from the same prompt:

* ring: the prompt's first P tokens are a peer chunk whose post-RoPE K/V are
  computed separately and staged per layer (stage_peer_kv / map_request_peer,
  ring_backend.py:96-123, the connector's job); the remaining L prompt tokens
  and every generated token go through HcpRingAttentionImpl
  (do_kv_cache_update into a paged [nb, 4, 16, 256] cache with a shuffled
  block table, then forward: local causal + peer + LSE merge for the prefill,
  split-KV decode for each new token) in bf16 on the GPU;
* reference: the same weights, with every attention computed by the oracle
  (fp32 dense causal attention over all keys, the reference's torch path
  ring_backend.py:366-406) on the CPU.

The gate is the reference's engine check (validate_ring_backend.py:194-199):
the same greedy token at every step, the same top-5 set, and max |logit
diff| < 0.1.
"""

import math
import types

import pytest
import torch

from hcp_vllm_plugin_amd import ring_attn_with_lse
from hcp_vllm_plugin_amd import ring_backend as rb
from oracle import ring_oracle as orc

pytestmark = pytest.mark.gpu

H, HKV, D, BS = 28, 4, 128, 16
HID, FF, VOCAB, LAYERS = 512, 1024, 512, 2
P, L, STEPS = 512, 300, 12


class TinyDecoder:
    """Pre-norm decoder: RMSNorm, QKV, RoPE, attention, O proj, SiLU MLP."""

    def __init__(self, seed, device):
        g = torch.Generator().manual_seed(seed)

        def w(*shape):
            return (torch.randn(*shape, generator=g) / math.sqrt(shape[0])).to(device)

        self.emb = torch.randn(VOCAB, HID, generator=g).to(device)
        self.layers = []
        for _ in range(LAYERS):
            self.layers.append(dict(
                wq=w(HID, H * D), wk=w(HID, HKV * D), wv=w(HID, HKV * D),
                wo=w(H * D, HID), w1=w(HID, FF), w2=w(FF, HID)))
        self.lm = w(HID, VOCAB)
        inv = 1.0 / (10000.0 ** (torch.arange(0, D, 2, dtype=torch.float64) / D))
        self.inv_freq = inv.to(device)
        self.device = device

    @staticmethod
    def norm(x):
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)

    def rope(self, x, pos):
        ang = pos.to(torch.float64)[:, None] * self.inv_freq[None, :]
        cos, sin = ang.cos().float()[:, None, :], ang.sin().float()[:, None, :]
        x1, x2 = x[..., : D // 2], x[..., D // 2:]
        return torch.cat([x1 * cos - x2 * sin, x1 * sin + x2 * cos], -1)

    def forward(self, tokens, positions, attn):
        """tokens/positions [T] on the model device; attn(layer_idx, q, k, v)
        -> [T, H, D] fp32.  Returns logits [T, VOCAB] fp32."""
        x = self.emb[tokens]
        t = x.shape[0]
        for i, ly in enumerate(self.layers):
            h = self.norm(x)
            q = self.rope((h @ ly["wq"]).view(t, H, D), positions)
            k = self.rope((h @ ly["wk"]).view(t, HKV, D), positions)
            v = (h @ ly["wv"]).view(t, HKV, D)
            o = attn(i, q, k, v)
            x = x + o.reshape(t, H * D).to(x.device) @ ly["wo"]
            h = self.norm(x)
            x = x + torch.nn.functional.silu(h @ ly["w1"]) @ ly["w2"]
        return self.norm(x) @ self.lm


def layer_name(i):
    return f"model.layers.{i}.self_attn.attn"


def run_reference(model_cpu, prompt):
    """Oracle attention over the full causal context, fp32 on the CPU."""
    kv = [[None, None] for _ in range(LAYERS)]

    def attn(i, q, k, v):
        # K/V rounded to bf16 as the cache stores them; math in fp32
        k = k.to(torch.bfloat16).float()
        v = v.to(torch.bfloat16).float()
        q = q.to(torch.bfloat16).float()
        kv[i][0] = k if kv[i][0] is None else torch.cat([kv[i][0], k])
        kv[i][1] = v if kv[i][1] is None else torch.cat([kv[i][1], v])
        kk, vv = kv[i]
        o, _ = orc.attn_with_lse(q, kk, vv, 1.0 / math.sqrt(D), kk.shape[0] - q.shape[0])
        return o

    toks = list(prompt)
    logits = model_cpu.forward(torch.tensor(toks), torch.arange(len(toks)), attn)
    steps = [logits[-1]]
    for _ in range(STEPS - 1):
        nxt = int(steps[-1].argmax())
        pos = len(toks)
        toks.append(nxt)
        lg = model_cpu.forward(torch.tensor([nxt]), torch.tensor([pos]), attn)
        steps.append(lg[-1])
    return steps


def run_ring(model, prompt, dev):
    rb.clear_peer_kv()
    rb.reset_impl_stats()
    impl = rb.HcpRingAttentionImpl(H, D, 1.0 / math.sqrt(D), HKV)
    total = P + L + STEPS
    nblk = -(-total // BS)
    gen = torch.Generator().manual_seed(123)
    nb = nblk + 8
    bt = torch.randperm(nb, generator=gen)[:nblk].to(torch.int32)[None, :].to(dev)
    caches = [torch.zeros(nb, HKV, BS, 2 * D, dtype=torch.bfloat16, device=dev)
              for _ in range(LAYERS)]
    layers = [types.SimpleNamespace(layer_name=layer_name(i)) for i in range(LAYERS)]

    # peer node: its chunk's K/V (post-RoPE), causal within the chunk
    def peer_attn(i, q, k, v):
        kb, vb = k.to(torch.bfloat16).contiguous(), v.to(torch.bfloat16).contiguous()
        rb.stage_peer_kv("peer0", layer_name(i), kb, vb)
        o, _ = ring_attn_with_lse(q.to(torch.bfloat16).contiguous(), kb, vb,
                                  1.0 / math.sqrt(D), 0)
        return o.float()

    ptoks = torch.tensor(prompt[:P], device=dev)
    model.forward(ptoks, torch.arange(P, device=dev), peer_attn)
    rb.map_request_peer(int(bt[0, 0]), ["peer0"])

    state = {}

    def ring_attn(i, q, k, v):
        t = q.shape[0]
        pos0 = state["pos0"]
        slots = torch.tensor([int(bt[0, p // BS]) * BS + p % BS for p in range(pos0, pos0 + t)],
                             dtype=torch.int64, device=dev)
        kb, vb = k.to(torch.bfloat16), v.to(torch.bfloat16)
        impl.do_kv_cache_update(layers[i], kb, vb, caches[i], slots)
        meta = types.SimpleNamespace(
            num_actual_tokens=t,
            query_start_loc=torch.tensor([0, t], dtype=torch.int32, device=dev),
            seq_lens=torch.tensor([pos0 + t], dtype=torch.int32, device=dev),
            block_table=bt)
        out = torch.empty(t, H, D, dtype=torch.bfloat16, device=dev)
        impl.forward(layers[i], q.to(torch.bfloat16).contiguous(), kb, vb, caches[i], meta, out)
        return out.float()

    toks = list(prompt)
    state["pos0"] = P
    logits = model.forward(torch.tensor(toks[P:], device=dev),
                           torch.arange(P, P + L, device=dev), ring_attn)
    steps = [logits[-1].cpu()]
    for _ in range(STEPS - 1):
        nxt = int(steps[-1].argmax())
        pos = len(toks)
        toks.append(nxt)
        state["pos0"] = pos
        lg = model.forward(torch.tensor([nxt], device=dev), torch.tensor([pos], device=dev),
                           ring_attn)
        steps.append(lg[-1].cpu())
    torch.cuda.synchronize()
    return steps


def test_greedy_tokens_identical(dev):
    gen = torch.Generator().manual_seed(7)
    prompt = torch.randint(0, VOCAB, (P + L,), generator=gen).tolist()
    model = TinyDecoder(seed=2024, device=dev)
    model_cpu = TinyDecoder(seed=2024, device=torch.device("cpu"))
    ring = run_ring(model, prompt, dev)
    assert rb.IMPL_STATS["attn_hip"] > 0 and rb.IMPL_STATS["merge_hip"] > 0
    assert rb.IMPL_STATS["decode_hip"] == LAYERS * (STEPS - 1)
    assert rb.IMPL_STATS["attn_torch"] == 0 and rb.IMPL_STATS["merge_torch"] == 0
    ref = run_reference(model_cpu, prompt)
    worst, margins = 0.0, []
    for s, (a, b) in enumerate(zip(ring, ref)):
        top_a, top_b = a.topk(5).indices, b.topk(5).indices
        srt = b.sort(descending=True).values
        margins.append(float(srt[0] - srt[1]))
        assert int(a.argmax()) == int(b.argmax()), f"step {s}: greedy token differs"
        assert set(top_a.tolist()) == set(top_b.tolist()), f"step {s}: top-5 differs"
        worst = max(worst, float((a - b).abs().max()))
    print(f"max |logit diff| {worst:.4f}; reference top-1 margins min {min(margins):.4f}")
    assert worst < 0.1
