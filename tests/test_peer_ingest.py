"""Peer-KV ingest on the CPU: the safetensors header parser and the packed
layouts against safetensors' own loader (bit-exact), for the ring connector's
{"k","v"} files (ring_connector.py:869-915) and hcp-kv-v1 {"kv": [S,2,Hkv,D]}
files (file_connector.py:3-7), several chunks per request (the torch.cat of
ring_backend.py:766-772), truncation to n_tokens, and format errors."""

import os

import pytest
import safetensors.torch as st
import torch

from hcp_vllm_plugin_amd.peer_ingest import PeerIngest, read_header


def _files(tmp_path, fmt, lens, dtype=torch.bfloat16, hkv=4, d=16, seed=0):
    gen = torch.Generator().manual_seed(seed)
    paths = []
    for i, n in enumerate(lens):
        p = os.path.join(tmp_path, f"chunk{i}.safetensors")
        if fmt == "kv":
            st.save_file({"kv": torch.randn(n, 2, hkv, d, generator=gen).to(dtype)}, p,
                         metadata={"format": "hcp-kv-v1"})
        else:
            st.save_file({"k": torch.randn(n, hkv, d, generator=gen).to(dtype),
                          "v": torch.randn(n, hkv, d, generator=gen).to(dtype)}, p)
        paths.append(p)
    return paths


@pytest.mark.parametrize("fmt", ["k_v", "kv"])
def test_header_matches_safetensors(tmp_path, fmt):
    (p,) = _files(tmp_path, fmt, [7])
    hdr = read_header(p)
    with st.safe_open(p, "pt") as f:
        assert sorted(hdr) == sorted(f.keys())
        for name in f.keys():
            t = f.get_tensor(name)
            assert hdr[name].shape == tuple(t.shape) and hdr[name].dtype == t.dtype
            raw = open(p, "rb").read()[hdr[name].begin:hdr[name].end]
            assert raw == t.contiguous().view(torch.uint8).numpy().tobytes()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_k_v_chunks_pack_like_cat(tmp_path, dtype):
    paths = _files(tmp_path, "k_v", [5, 0, 33, 2], dtype)
    got = PeerIngest("cpu", "k_v").load(paths)
    ref = [st.load_file(p) for p in paths]
    assert torch.equal(got.k, torch.cat([r["k"] for r in ref]))
    assert torch.equal(got.v, torch.cat([r["v"] for r in ref]))
    assert got.chunk_starts == [0, 5, 5, 38]
    k1, v1 = got.chunk(2)
    assert torch.equal(k1, ref[2]["k"]) and torch.equal(v1, ref[2]["v"])


def test_kv_format_views_and_truncation(tmp_path):
    paths = _files(tmp_path, "kv", [10, 6])
    got = PeerIngest("cpu", "kv").load(paths, n_tokens=[7, 6])
    ref = [st.load_file(p)["kv"] for p in paths]
    assert torch.equal(got.k, torch.cat([ref[0][:7, 0], ref[1][:, 0]]))
    assert torch.equal(got.v, torch.cat([ref[0][:7, 1], ref[1][:, 1]]))
    # K/V stay interleaved: views with token stride 2 * Hkv * D, no de-interleave
    assert got.k.stride(0) == 2 * 4 * 16 and got.k.stride(-1) == 1
    assert got.v.data_ptr() == got.k.data_ptr() + 4 * 16 * got.k.element_size()


def test_format_errors(tmp_path):
    (p,) = _files(tmp_path, "k_v", [4])
    with pytest.raises(ValueError, match="'kv'"):
        PeerIngest("cpu", "kv").load([p])
    q = os.path.join(tmp_path, "odd.safetensors")
    st.save_file({"k": torch.zeros(4, 4, 16, dtype=torch.float16),
                  "v": torch.zeros(4, 4, 16, dtype=torch.float16)}, q)
    with pytest.raises(ValueError, match="differ"):
        PeerIngest("cpu", "k_v").load([p, q])
    bad = os.path.join(tmp_path, "bad.safetensors")
    open(bad, "wb").write(b"\x01\x02")
    with pytest.raises(ValueError, match="short header"):
        read_header(bad)
    with pytest.raises(ValueError, match="format"):
        PeerIngest("cpu", "kv_v2")
