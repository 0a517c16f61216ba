"""GPU parity of the memory-split decode step (the decode accumulator ring).

* ``RingDecodeNode.accumulate`` / ``handle_packet`` against the oracle's
  ``ring_decode_hop`` (ring_decode.py:187-259) on identical inputs, with the
  growth routing rules (append at the target, forward otherwise).
* The whole protocol through the backend: an owner ``HcpRingAttentionImpl``
  with a registered decode ring (ring_backend.py:175-208, :643-722) and
  in-process ring nodes joined by a chain transport, against the oracle's
  ``DecodeRingSim`` step by step -- which the CPU tests pin to full attention
  over every key.  Also: decode-ring tokens never reach the paged pool, growth
  lands on ``pos mod N``, two requests' growth stays apart, and a prefill
  request in the same batch is unaffected.

Tolerances: out 2e-3 (float16) / 1.5e-2 (bfloat16), LSE 1e-3.
"""

import types

import pytest
import torch

from hcp_vllm_plugin_amd import ring_backend as rb
from hcp_vllm_plugin_amd import ring_decode as rd
from oracle import ring_oracle as orc
from tests._util import LSE_TOL, OUT_TOL, max_err, randn, scale_for

pytestmark = pytest.mark.gpu

H, HKV, D, BS = 28, 4, 128, 16
LAYER = "model.layers.5.self_attn.attn"


@pytest.fixture(autouse=True)
def _clean(monkeypatch):
    rb.clear_peer_kv()
    rb.DECODE_RING_MAP.clear()
    rb.reset_impl_stats()
    rd.RING_NODES.clear()
    rb.WRITE_TRACK["skipped"] = 0
    for k in ("HCP_RING_IMPL", "HCP_RING_MERGE", "HCP_RING_SPLIT_TOKENS", "HCP_RING_ENABLED",
              "HCP_RING_DECODE_RING", "HCP_RING_DECODE_GROWTH"):
        monkeypatch.delenv(k, raising=False)
    yield
    rb.clear_peer_kv()
    rb.DECODE_RING_MAP.clear()
    rd.RING_NODES.clear()


def _node(dev, dtype, idx, chunk_key, k, v):
    n = rd.RingDecodeNode("", [chunk_key], idx, device=str(dev), dtype=dtype, background=False)
    n.add_chunk(chunk_key, LAYER, k.to(dev), v.to(dev))
    n.mark_ready()
    return n


class ChainTransport:
    """In-process ring: the packet visits the nodes in ring order and comes
    back to the owner."""

    def __init__(self, nodes):
        self.nodes = nodes
        self.last = None
        self.sent = 0

    def send_packet(self, payload: bytes) -> None:
        self.sent += 1
        for n in self.nodes:
            payload = n.handle_packet(payload)
        self.last = payload

    def recv_packet(self, timeout_s: float = 1.0) -> bytes:
        p, self.last = self.last, None
        return p


# ---------------------------------------------------------------------------
# one hop
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("tk,ng,tq", [(1, 0, 1), (37, 1, 1), (1000, 5, 1), (4096, 0, 1),
                                      (300, 3, 3)])
def test_accumulate_vs_oracle_hop(dev, dtype, tk, ng, tq):
    gen = torch.Generator().manual_seed(tk + 7 * ng + tq)
    q = randn(gen, (tq, H, D), dtype)
    o_acc = randn(gen, (tq, H, D), dtype)
    lse_acc = torch.randn(H, tq, generator=gen) * 3
    ck, cv = randn(gen, (tk, HKV, D), dtype), randn(gen, (tk, HKV, D), dtype)
    gk, gv = randn(gen, (ng, HKV, D), dtype), randn(gen, (ng, HKV, D), dtype)
    node = _node(dev, dtype, 1, "c0", ck, cv)
    for i in range(ng):  # one token per append, as the ring ships them
        node.append_growth("r", LAYER, gk[i:i + 1].to(dev), gv[i:i + 1].to(dev))
    o, lse = node.accumulate(q.to(dev), o_acc.to(dev), lse_acc.to(dev), scale_for(D), LAYER, "r")
    torch.cuda.synchronize()
    ro, rl = orc.ring_decode_hop(q, o_acc, lse_acc, ck, cv, gk if ng else None,
                                 gv if ng else None, scale_for(D))
    assert o.dtype == dtype and lse.dtype == torch.float32
    assert max_err(o, ro) <= OUT_TOL[dtype]
    assert max_err(lse, rl) <= LSE_TOL


def test_growth_buffer_survives_regrowth(dev):
    """Appends past the initial capacity keep the history (doubling copy)."""
    gen = torch.Generator().manual_seed(3)
    g = rd.GrowthBuffer(HKV, D, torch.bfloat16, dev, capacity=4)
    ks = randn(gen, (37, HKV, D), torch.bfloat16)
    vs = randn(gen, (37, HKV, D), torch.bfloat16)
    for i in range(37):
        g.append(ks[i:i + 1].to(dev), vs[i:i + 1].to(dev))
    assert g.len == 37 and g.k.shape[0] >= 37
    assert torch.equal(g.k[:37].cpu(), ks) and torch.equal(g.v[:37].cpu(), vs)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_handle_packet_growth_routing(dev, dtype):
    """ring_decode.py:202-222, :253-258: growth is appended only at its
    target (a packet without ``growth_target`` targets whoever reads it) and
    forwarded byte-identical otherwise; q / scale / names pass through."""
    gen = torch.Generator().manual_seed(11)
    ck, cv = randn(gen, (200, HKV, D), dtype), randn(gen, (200, HKV, D), dtype)
    node = _node(dev, dtype, 2, "c1", ck, cv)
    q = randn(gen, (1, H, D), dtype)
    o0 = randn(gen, (1, H, D), dtype)
    l0 = torch.randn(H, 1, generator=gen)
    gk, gv = randn(gen, (1, HKV, D), dtype), randn(gen, (1, HKV, D), dtype)
    sc = scale_for(D)

    # addressed elsewhere: forwarded, not kept
    out = rd.decode_packet(node.handle_packet(
        rd.encode_packet(q, o0, l0, sc, LAYER, "c0", "reqA", gk, gv, 1)))
    assert torch.equal(out["growth_k"], gk) and torch.equal(out["growth_v"], gv)
    assert out["growth_target"] == 1 and node.growth_stats() == {}
    assert torch.equal(out["q"], q) and out["chunk"] == "c0" and out["req"] == "reqA"
    assert out["layer"] == LAYER and out["scale"] == torch.tensor([sc]).item()
    ro, rl = orc.ring_decode_hop(q, o0, l0, ck, cv, None, None, sc)
    assert max_err(out["o"], ro) <= OUT_TOL[dtype] and max_err(out["lse"], rl) <= LSE_TOL

    # addressed here: appended before the partial, not forwarded
    out = rd.decode_packet(node.handle_packet(
        rd.encode_packet(q, o0, l0, sc, LAYER, "c0", "reqA", gk, gv, 2)))
    assert "growth_k" not in out and "growth_target" not in out
    assert node.growth_stats() == {"reqA": 1} and node.growth_appends == 1
    ro, rl = orc.ring_decode_hop(q, o0, l0, ck, cv, gk, gv, sc)
    assert max_err(out["o"], ro) <= OUT_TOL[dtype] and max_err(out["lse"], rl) <= LSE_TOL

    # no target key: consumed by the first reader
    d = safetensors_packet(q, o0, l0, sc, gk, gv)
    out = rd.decode_packet(node.handle_packet(d))
    assert "growth_k" not in out and node.growth_stats() == {"reqA": 1, "": 1}
    # another request's growth never enters reqA's partial
    out = rd.decode_packet(node.handle_packet(
        rd.encode_packet(q, o0, l0, sc, LAYER, "c0", "reqA")))
    ro, rl = orc.ring_decode_hop(q, o0, l0, ck, cv, gk, gv, sc)
    assert max_err(out["o"], ro) <= OUT_TOL[dtype] and max_err(out["lse"], rl) <= LSE_TOL
    assert node.calls == 4


def safetensors_packet(q, o, lse, sc, gk, gv):
    import safetensors.torch

    return safetensors.torch.save({
        "chunk": torch.tensor(list(b"c0"), dtype=torch.uint8),
        "layer": torch.tensor(list(LAYER.encode()), dtype=torch.uint8),
        "q": q, "o": o, "lse": lse, "scale": torch.tensor([sc], dtype=torch.float32),
        "growth_k": gk, "growth_v": gv,
    })


# ---------------------------------------------------------------------------
# the whole protocol through the backend
# ---------------------------------------------------------------------------
def _slot(bt_row, pos):
    return int(bt_row[pos // BS]) * BS + pos % BS


class _Req:
    """One decode-ring request: its prefix peers, pool blocks and oracle."""

    def __init__(self, gen, dtype, dev, cache_cpu, layout, blocks, peer_lens, own_len, policy,
                 window=None):
        self.peer_k = [randn(gen, (n, HKV, D), dtype) for n in peer_lens]
        self.peer_v = [randn(gen, (n, HKV, D), dtype) for n in peer_lens]
        self.plen = sum(peer_lens)
        self.own_len = own_len
        self.prompt = self.plen + own_len
        self.bt_row = blocks
        own = orc.gather_paged(cache_cpu.float(), blocks, self.plen, own_len, layout)
        self.sim = orc.DecodeRingSim(list(zip(self.peer_k, self.peer_v)), own, scale_for(D), policy,
                                     window)
        self.steps = 0


def _meta(dev, qsl, seq_lens, bt):
    return types.SimpleNamespace(
        num_actual_tokens=qsl[-1],
        query_start_loc=torch.tensor(qsl, dtype=torch.int32, device=dev),
        seq_lens=torch.tensor(seq_lens, dtype=torch.int32, device=dev),
        block_table=bt.to(dev),
    )


def _setup(dev, dtype, layout, n_req, peer_lens, own_len, policy, seed, monkeypatch,
           extra_blocks=0, window=None):
    gen = torch.Generator().manual_seed(seed)
    if policy != "rr":
        monkeypatch.setenv("HCP_RING_DECODE_GROWTH", policy)
    max_tok = sum(peer_lens) + own_len + 16
    per = -(-max_tok // BS)
    nb = n_req * per + extra_blocks + 2
    shape = (nb, HKV, BS, 2 * D) if layout == "v031" else (nb, 2, BS, HKV, D)
    cache_cpu = randn(gen, shape, dtype)
    perm = torch.randperm(nb, generator=gen).to(torch.int32)
    reqs = []
    for r in range(n_req):
        blocks = perm[r * per:(r + 1) * per].clone()
        reqs.append(_Req(gen, dtype, dev, cache_cpu, layout, blocks, peer_lens, own_len, policy,
                         window))
    # a ring of nodes per request (each node's first chunk key is the one
    # it serves, ring_decode.py:226-228)
    n_peer = len(peer_lens)
    transports = []
    for r, q in enumerate(reqs):
        rnodes = []
        for i in range(n_peer):
            node = rd.RingDecodeNode("", [f"r{r}c{i}"], i + 1, device=str(dev), dtype=dtype,
                                     background=False)
            node.add_chunk(f"r{r}c{i}", LAYER, q.peer_k[i].to(dev), q.peer_v[i].to(dev))
            node.mark_ready()
            rnodes.append(node)
        t = ChainTransport(rnodes)
        transports.append(t)
        rb.register_decode_ring(int(q.bt_row[0]), [(f"r{r}c{i}", f"http://peer{i}")
                                                   for i in range(n_peer)],
                                q.plen, transport=t)
    return gen, cache_cpu, cache_cpu.to(dev), reqs, transports


def _decode_step(dev, dtype, impl, layer, gen, cache, reqs, monkeypatch, prefill=None):
    """One engine step: every request decodes one token (plus an optional
    prefill request in front).  Returns the output rows and oracle rows."""
    rows_q, rows_k, rows_v, seq_lens, bts, slots = [], [], [], [], [], []
    qsl = [0]
    if prefill is not None:
        pq, pk, pv, ptk, pbt = prefill
        rows_q.append(pq)
        rows_k.append(pk)
        rows_v.append(pv)
        seq_lens.append(ptk)
        bts.append(pbt)
        qsl.append(pq.shape[0])
        slots += [_slot(pbt, p) for p in range(ptk - pq.shape[0], ptk)]
    for q in reqs:
        tk = q.prompt + 1 + q.steps
        rows_q.append(randn(gen, (1, H, D), dtype))
        rows_k.append(randn(gen, (1, HKV, D), dtype))
        rows_v.append(randn(gen, (1, HKV, D), dtype))
        seq_lens.append(tk)
        bts.append(q.bt_row)
        qsl.append(qsl[-1] + 1)
        slots.append(_slot(q.bt_row, tk - 1))
    width = max(b.shape[0] for b in bts)
    bt = torch.zeros(len(bts), width, dtype=torch.int32)
    for i, b in enumerate(bts):
        bt[i, :b.shape[0]] = b
    query = torch.cat(rows_q)
    key = torch.cat(rows_k)
    value = torch.cat(rows_v)
    meta = _meta(dev, qsl, seq_lens, bt)
    monkeypatch.setattr(rb, "_forward_attn_metadata", lambda layer: meta)
    slot_dev = torch.tensor(slots, dtype=torch.int64, device=dev)
    kd, vd = key.to(dev), value.to(dev)
    impl.do_kv_cache_update(layer, kd, vd, cache, slot_dev)
    output = torch.full((query.shape[0] + 2, H, D), 7.0, dtype=dtype, device=dev)
    impl.forward(layer, query.to(dev), kd, vd, cache, meta, output)
    torch.cuda.synchronize()
    off = 1 if prefill is not None else 0
    refs = []
    for i, q in enumerate(reqs):
        r = qsl[off + i]
        o_ref, _ = q.sim.step(query[r:r + 1], key[r:r + 1], value[r:r + 1], seq_lens[off + i] - 1)
        refs.append((output[r:r + 1], o_ref))
        q.steps += 1
    assert torch.all(output[qsl[-1]:] == 7.0)
    return output, refs, qsl, query, key, value, seq_lens, bt


@pytest.mark.parametrize("dtype,layout,peer_lens,policy", [
    (torch.float16, "v031", [40, 33], "rr"),
    (torch.float16, "v023", [70], "rr"),
    (torch.bfloat16, "v031", [40, 33, 17], "rr"),
    (torch.float16, "v031", [40, 33], "owner"),
])
def test_backend_decode_ring_matches_protocol(dev, dtype, layout, peer_lens, policy, monkeypatch):
    gen, cache_cpu, cache, reqs, transports = _setup(dev, dtype, layout, 1, peer_lens, 29,
                                                     policy, 17, monkeypatch)
    impl = rb.HcpRingAttentionImpl(H, D, scale_for(D), HKV)
    layer = types.SimpleNamespace(layer_name=LAYER)
    n = len(peer_lens) + 1
    steps = 2 * n + 1
    rb.map_request_peer(int(reqs[0].bt_row[0]), ["staged-prefix"])
    rb.stage_peer_kv("staged-prefix", LAYER, torch.zeros(4, HKV, D, device=dev),
                     torch.zeros(4, HKV, D, device=dev))
    for t in range(steps):
        before = cache.clone()
        _, refs, *_ = _decode_step(dev, dtype, impl, layer, gen, cache, reqs, monkeypatch)
        assert torch.equal(cache, before), "a decode-ring token reached the paged pool"
        for got, want in refs:
            assert max_err(got, want) <= OUT_TOL[dtype], t
    # the staged prefix was released at the transition (ring_backend.py:642)
    assert rb.PEER_REQ_MAP == {} and rb.PEER_KV_STAGING == {}
    assert rb.WRITE_TRACK["skipped"] == steps
    assert rb.IMPL_STATS["ring_decode_steps"] == steps
    assert transports[0].sent == steps
    # growth placement: pos mod N on the peers (the last peer-bound token
    # still pending), the owner's share in its own buffer
    q = reqs[0]
    dr = rb.DECODE_RING_MAP[int(q.bt_row[0])]
    positions = range(q.prompt, q.prompt + steps)
    last = q.prompt + steps - 1

    def assignee(p):
        return n - 1 if policy == "owner" else p % n

    for i, node in enumerate(transports[0].nodes):
        want = sum(1 for p in positions if assignee(p) == i and p != last)
        assert node.growth_stats() == ({dr["req_tag"]: want} if want else {}), i
        assert node.calls == steps
    assert dr["growth"][LAYER].len == sum(1 for p in positions if assignee(p) == n - 1)


def test_backend_decode_ring_two_requests_isolated(dev, monkeypatch):
    """Two ring requests decode in one batch (one split-KV launch for both
    owner partials); each matches its own protocol run."""
    dtype = torch.float16
    gen, cache_cpu, cache, reqs, transports = _setup(dev, dtype, "v031", 2, [50, 21], 35,
                                                     "rr", 23, monkeypatch)
    impl = rb.HcpRingAttentionImpl(H, D, scale_for(D), HKV)
    layer = types.SimpleNamespace(layer_name=LAYER)
    for t in range(5):
        _, refs, *_ = _decode_step(dev, dtype, impl, layer, gen, cache, reqs, monkeypatch)
        for got, want in refs:
            assert max_err(got, want) <= OUT_TOL[dtype], t
    tags = {rb.DECODE_RING_MAP[int(q.bt_row[0])]["req_tag"] for q in reqs}
    assert len(tags) == 2
    assert rb.IMPL_STATS["decode_hip"] == 5  # one launch per step for both rows


def test_backend_decode_ring_next_to_prefill(dev, monkeypatch):
    """A prefill request in the same batch runs the varlen path; the ring
    row takes its own local partial."""
    dtype = torch.float16
    gen, cache_cpu, cache, reqs, transports = _setup(dev, dtype, "v031", 1, [44], 30, "rr", 29,
                                                     monkeypatch, extra_blocks=8)
    impl = rb.HcpRingAttentionImpl(H, D, scale_for(D), HKV)
    layer = types.SimpleNamespace(layer_name=LAYER)
    used = set(reqs[0].bt_row.tolist())
    free = [b for b in range(cache.shape[0]) if b not in used][:8]
    pbt = torch.tensor(free, dtype=torch.int32)
    ptk, ptq = 100, 20
    for t in range(3):
        pre = (randn(gen, (ptq, H, D), dtype), randn(gen, (ptq, HKV, D), dtype),
               randn(gen, (ptq, HKV, D), dtype), ptk, pbt)
        out, refs, qsl, query, key, value, seq_lens, bt = _decode_step(
            dev, dtype, impl, layer, gen, cache, reqs, monkeypatch, prefill=pre)
        for got, want in refs:
            assert max_err(got, want) <= OUT_TOL[dtype], t
        # the prefill rows: written to the pool, then causal attention over it
        c = cache.cpu()
        ref = orc.ring_forward(query[:ptq].float(), c.float(), "v031", [0, ptq], [ptk],
                               bt[:1], scale_for(D), out_dtype=torch.float32)
        assert max_err(out[:ptq], ref[:ptq]) <= OUT_TOL[dtype]
        k_written, _ = orc.gather_paged(c, pbt, ptk - ptq, ptq, "v031")
        assert torch.equal(k_written, key[:ptq])


@pytest.mark.parametrize("window", [1, 7, 40])
def test_backend_decode_ring_sliding_window(dev, window, monkeypatch):
    """The owner's local partial is causal at len - 1 over own chunk + owned
    growth + current token (ring_backend.py:672-679): with a sliding window
    it keeps the last `window` keys of that concatenation; the nodes' partials
    are non-causal and unwindowed."""
    dtype = torch.float16
    gen, cache_cpu, cache, reqs, transports = _setup(dev, dtype, "v031", 1, [40, 33], 29, "rr",
                                                     31, monkeypatch, window=window)
    impl = rb.HcpRingAttentionImpl(H, D, scale_for(D), HKV, sliding_window=window)
    layer = types.SimpleNamespace(layer_name=LAYER)
    for t in range(7):
        _, refs, *_ = _decode_step(dev, dtype, impl, layer, gen, cache, reqs, monkeypatch)
        for got, want in refs:
            assert max_err(got, want) <= OUT_TOL[dtype], t
