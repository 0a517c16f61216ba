"""GPU: peer-KV ingest into packed device buffers equals safetensors' loader
(bit-exact), and the interleaved hcp-kv-v1 views feed the attention kernel in
place (same result as de-interleaved copies)."""

import os

import pytest
import safetensors.torch as st
import torch

from hcp_vllm_plugin_amd import ring_attn_with_lse
from hcp_vllm_plugin_amd.peer_ingest import PeerIngest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("fmt", ["k_v", "kv"])
def test_ingest_to_device_bit_exact(tmp_path, dev, fmt):
    gen = torch.Generator().manual_seed(3)
    paths = []
    for i, n in enumerate([300, 512, 77]):
        p = os.path.join(tmp_path, f"c{i}.safetensors")
        if fmt == "kv":
            st.save_file({"kv": torch.randn(n, 2, 4, 128, generator=gen).to(torch.bfloat16)}, p)
        else:
            st.save_file({"k": torch.randn(n, 4, 128, generator=gen).to(torch.bfloat16),
                          "v": torch.randn(n, 4, 128, generator=gen).to(torch.bfloat16)}, p)
        paths.append(p)
    ing = PeerIngest(dev, fmt)
    for _ in range(3):  # staging buffers are reused across layers
        got = ing.load(paths)
    got.event.synchronize()
    ref = [st.load_file(p, device=str(dev)) for p in paths]
    if fmt == "kv":
        rk = torch.cat([r["kv"][:, 0] for r in ref])
        rv = torch.cat([r["kv"][:, 1] for r in ref])
    else:
        rk, rv = torch.cat([r["k"] for r in ref]), torch.cat([r["v"] for r in ref])
    assert torch.equal(got.k, rk) and torch.equal(got.v, rv)


def test_interleaved_views_as_peer_segment(tmp_path, dev):
    gen = torch.Generator().manual_seed(4)
    p = os.path.join(tmp_path, "kv.safetensors")
    st.save_file({"kv": torch.randn(1000, 2, 4, 128, generator=gen).to(torch.bfloat16)}, p)
    got = PeerIngest(dev, "kv").load([p])
    q = torch.randn(300, 28, 128, generator=gen).to(torch.bfloat16).to(dev)
    o1, l1 = ring_attn_with_lse(q, got.k, got.v, 128 ** -0.5, None)
    o2, l2 = ring_attn_with_lse(q, got.k.contiguous(), got.v.contiguous(), 128 ** -0.5, None)
    torch.cuda.synchronize()
    assert torch.equal(o1.cpu(), o2.cpu()) and torch.equal(l1.cpu(), l2.cpu())
