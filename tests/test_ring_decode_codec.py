"""Decode-ring packet codec and growth assignment (CPU).

The packet is the reference's wire format (ring_decode.py:241-259,
:336-355): a safetensors blob with ``chunk`` / ``layer`` / ``req`` as uint8
bytes, ``q`` / ``o`` in the model dtype, ``lse`` float32 ``[H, T]``,
``scale`` float32 ``[1]`` and, when growth rides along, ``growth_k`` /
``growth_v`` ``[1, Hkv, D]`` with ``growth_target`` int64 ``[1]``.  A packet
made here must parse with plain ``safetensors.torch.load`` to exactly those
keys and dtypes, and a packet laid out by hand that way must decode here.
"""

import safetensors.torch
import torch

from hcp_vllm_plugin_amd.ring_decode import decode_packet, encode_packet, growth_assignee


def _tensors(dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(5)
    q = torch.randn(1, 28, 128, generator=g).to(dtype)
    o = torch.randn(1, 28, 128, generator=g).to(dtype)
    lse = torch.randn(28, 1, generator=g)
    gk = torch.randn(1, 4, 128, generator=g).to(dtype)
    gv = torch.randn(1, 4, 128, generator=g).to(dtype)
    return q, o, lse, gk, gv


def test_packet_keys_and_dtypes_match_the_wire_format():
    q, o, lse, gk, gv = _tensors()
    raw = safetensors.torch.load(encode_packet(q, o, lse, 0.0883883, "model.layers.0.self_attn.attn",
                                               "c0", "12:ab34cd56"))
    assert set(raw) == {"chunk", "layer", "req", "q", "o", "lse", "scale"}
    assert raw["chunk"].dtype == torch.uint8 and bytes(raw["chunk"].tolist()) == b"c0"
    assert bytes(raw["layer"].tolist()) == b"model.layers.0.self_attn.attn"
    assert bytes(raw["req"].tolist()) == b"12:ab34cd56"
    assert raw["scale"].dtype == torch.float32 and raw["scale"].shape == (1,)
    assert raw["lse"].dtype == torch.float32 and raw["lse"].shape == (28, 1)
    assert torch.equal(raw["q"], q) and torch.equal(raw["o"], o) and torch.equal(raw["lse"], lse)

    raw = safetensors.torch.load(encode_packet(q, o, lse, 0.5, "L", "c0", "r", gk, gv, 2))
    assert set(raw) == {"chunk", "layer", "req", "q", "o", "lse", "scale", "growth_k",
                        "growth_v", "growth_target"}
    assert raw["growth_target"].dtype == torch.int64 and raw["growth_target"].tolist() == [2]
    assert torch.equal(raw["growth_k"], gk) and torch.equal(raw["growth_v"], gv)


def test_hand_built_packet_decodes():
    """A packet laid out as ring_decode.py:336-355 writes it."""
    q, o, lse, gk, gv = _tensors(torch.float16)
    d = {
        "chunk": torch.tensor(list(b"chunkA"), dtype=torch.uint8),
        "layer": torch.tensor(list(b"layer7"), dtype=torch.uint8),
        "req": torch.tensor(list(b""), dtype=torch.uint8),
        "q": q, "o": o, "lse": lse,
        "scale": torch.tensor([0.125], dtype=torch.float32),
        "growth_k": gk, "growth_v": gv,
        "growth_target": torch.tensor([3], dtype=torch.int64),
    }
    p = decode_packet(safetensors.torch.save(d))
    assert p["chunk"] == "chunkA" and p["layer"] == "layer7" and p["req"] == ""
    assert p["scale"] == 0.125 and p["growth_target"] == 3
    assert torch.equal(p["q"], q) and torch.equal(p["growth_v"], gv)


def test_packet_without_req_key():
    """Older packets carry no ``req``: it reads as the empty tag."""
    q, o, lse, _, _ = _tensors()
    d = {"chunk": torch.tensor([99], dtype=torch.uint8),
         "layer": torch.tensor([76], dtype=torch.uint8),
         "q": q, "o": o, "lse": lse, "scale": torch.tensor([1.0])}
    p = decode_packet(safetensors.torch.save(d))
    assert p["req"] == "" and p["chunk"] == "c" and p["layer"] == "L"


def test_growth_assignee():
    """ring_decode.py:30-43: rr is p mod N over ring order, owner is N-1."""
    assert [growth_assignee(p, 3) for p in range(7)] == [0, 1, 2, 0, 1, 2, 0]
    assert [growth_assignee(p, 4, "rr") for p in (100, 101, 102, 103)] == [0, 1, 2, 3]
    assert all(growth_assignee(p, 5, "owner") == 4 for p in range(9))


def test_in_place_reply_is_the_packet_with_o_and_lse_rewritten():
    """The hop's reply (packet.replace): every field byte-identical except the
    accumulator, and still a safetensors file plain safetensors reads."""
    from hcp_vllm_plugin_amd.packet import Packet, replace

    q, o, lse, gk, gv = _tensors()
    pkt_bytes = encode_packet(q, o, lse, 0.25, "L3", "c1", "req9", gk, gv, 1)
    pkt = Packet(pkt_bytes)
    o2 = torch.randn(1, 28, 128).to(torch.bfloat16)
    lse2 = torch.randn(28, 1)
    out = replace(pkt, {"o": o2, "lse": lse2})
    assert len(out) == len(pkt_bytes)
    raw = safetensors.torch.load(out)
    ref = safetensors.torch.load(pkt_bytes)
    assert set(raw) == set(ref)
    for k in ref:
        if k not in ("o", "lse"):
            assert torch.equal(raw[k], ref[k]), k
    assert torch.equal(raw["o"], o2) and torch.equal(raw["lse"], lse2)
    # only the two data ranges differ
    diff = [i for i, (a, b) in enumerate(zip(out, pkt_bytes)) if a != b]
    spans = [pkt.span("o"), pkt.span("lse")]
    assert all(any(b <= i < e for b, e in spans) for i in diff)


def test_packet_parser_details():
    from hcp_vllm_plugin_amd.packet import Packet, encode, replace

    q, o, lse, gk, gv = _tensors(torch.float16)
    # a reference packet with metadata and an empty req reads through Packet
    d = {"chunk": torch.tensor(list(b"c"), dtype=torch.uint8),
         "req": torch.zeros(0, dtype=torch.uint8), "q": q, "lse": lse,
         "scale": torch.tensor([0.5]), "growth_target": torch.tensor([7], dtype=torch.int64)}
    pkt = Packet(safetensors.torch.save(d, metadata={"format": "pt"}))
    assert pkt.text("chunk") == "c" and pkt.text("req") == ""
    assert pkt.item("scale") == 0.5 and pkt.item("growth_target") == 7
    assert torch.equal(pkt.tensor("q"), q) and torch.equal(pkt.tensor("lse"), lse)
    # encode lays tensors out aligned to their element size, and strings as uint8
    enc = encode({"req": "", "layer": "L", "q": q, "lse": lse,
                  "t": torch.tensor([3], dtype=torch.int64)})
    p2 = Packet(enc)
    for name in p2.meta:
        b, _ = p2.span(name)
        assert b % p2.tensor(name).element_size() == 0, name
    raw = safetensors.torch.load(enc)
    assert bytes(raw["layer"].tolist()) == b"L" and raw["req"].numel() == 0
    # malformed packets and mismatched replacements are rejected
    for bad in (b"", b"\xff" * 8 + b"{}", enc[:20]):
        try:
            Packet(bad)
        except ValueError:
            pass
        else:
            raise AssertionError(f"accepted {bad[:12]!r}")
    try:
        replace(p2, {"q": q.to(torch.bfloat16)})
    except ValueError:
        pass
    else:
        raise AssertionError("dtype mismatch accepted")
