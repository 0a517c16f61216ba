"""CPU oracle for the HCP ring-attention hot path (TEST INFRASTRUCTURE ONLY).

This module is the parity checker.  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it.  The product package
(``hcp_vllm_plugin_amd``) never imports or calls anything here, and has no CPU
fallback: when the HIP library is missing it raises.

It restates, in torch float32 on the CPU, with the same operations in the same
order, the reference's plain-PyTorch path of stark-sim/hcp-vllm-plugin:

* ``attn_with_lse``      <- ``_attn_with_lse``   hcp_vllm_plugin/ring_backend.py:366-406
* ``lse_merge``          <- ``_lse_merge``       hcp_vllm_plugin/ring_backend.py:409-421
* ``merge_pair``         <- ``_merge_pair``      hcp_vllm_plugin/ring_decode.py:46-61
* ``merge_attn_states``  <- vLLM ``merge_attn_states`` (external; called at
  ring_backend.py:349-354 with prefix = peer, suffix = local).  Restated from
  vLLM's published formula: max-shifted LSE weights, optional merged LSE out,
  an LSE of +inf read as -inf.
* ``gather_paged``       <- the per-request paged gather ring_backend.py:617-624
  for the vLLM 0.23 layout ``[nb, 2, bs, Hkv, D]`` and the vLLM 0.31 layout
  ``[nb, Hkv, bs, 2*D]`` (file_connector.py:13-16,175-179: K is ``[..., :D]``,
  V is ``[..., D:]``).
* ``kv_cache_update``    <- ``do_kv_cache_update`` ring_backend.py:501-539: slot =
  block * bs + offset, ``key_cache[block_idx, block_off] = key[:n]`` (and V)
  for the 0.23 layout, the same rows of the 0.31 layout's ``[..., :D]`` /
  ``[..., D:]`` halves.  A negative slot (vLLM's padding convention; the
  reference never passes one) is skipped -- parity unpinned for that case.
* ``ring_forward``       <- the segmentation of ``HcpRingAttentionImpl.forward``
  ring_backend.py:576-834 (non-decode-ring branch): vanilla causal when there is
  no peer, ``n_a`` queries inside the peer region, local causal at offset
  ``qpos0 + n_a - peer_end``, peer non-causal, merge, cast to ``output.dtype``.
* ``ring_decode_hop``    <- one node's step ``RingDecodeNode.handle_packet``
  ring_decode.py:187-239: partial over ``cat(chunk snapshot, growth)``
  non-causal, then ``_merge_pair(o_acc, lse_acc, o_loc, lse_loc)``.
* ``DecodeRingSim``      <- the memory-split decode protocol as a whole:
  owner side ring_backend.py:643-722 (own chunk + owned growth + current
  token causal at ``len-1``, growth assignment ``growth_assignee``
  ring_decode.py:30-43, last step's token shipped on this step's packet with
  ``growth_target = assignee + 1``) and every node's hop in ring order,
  ring_decode.py:187-259 (growth appended only at its target, before the
  partial).

Semantics fixed by the reference (ring_triton_attn.py:1-26,64,95-108,137-140):
q ``[Tq, H, D]``, k/v ``[Tk, Hkv, D]``, out ``[Tq, H, D]``, lse ``[H, Tq]`` float32
in natural log; GQA maps query head ``h`` to KV head ``h // (H // Hkv)``; key
``j`` is visible to query ``i`` iff ``j <= causal_offset + i``.

Pinning (tests/test_oracle.py): each function here is checked against things
that do not retype its formula -- float64 brute force with explicit loops,
``torch.nn.functional.scaled_dot_product_attention`` with an explicit mask,
``torch.logsumexp``, closed forms (Tk=1, constant keys), split-merge == full
attention (the reference's own check validate_ring_triton_kernel.py:80-94),
and the committed fixtures under tests/golden/.

Empty segments and rows with no visible key are outside the reference's domain
(it never calls the kernel with Tk=0, ring_backend.py:783).  This build defines
them as out = 0, lse = -inf, and a merge input with lse = -inf carries weight
0.  That convention is parity unpinned against the reference.
"""

from __future__ import annotations

import math

import torch

__all__ = [
    "attn_with_lse",
    "lse_merge",
    "merge_pair",
    "merge_attn_states",
    "gather_paged",
    "kv_cache_update",
    "ring_forward",
    "ring_decode_hop",
    "DecodeRingSim",
    "causal_pairs",
    "attn_flops",
]


def attn_with_lse(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: float,
    q_pos0_in_kv: int | None,
    window: int | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Dense fp32 attention with explicit natural-log LSE.

    Follows ring_backend.py:366-406 op for op: GQA by ``repeat_interleave``
    (:384-387), fp32 scores (:390), ``-inf`` mask for ``j > q0 + i`` and the
    optional window ``j <= qpos - w`` (:391-399), amax / exp / sum (:400-402),
    ``p @ v / denom`` (:403-404), ``lse = m + log(denom)`` (:405).

    Returns (out ``[Tq, H, D]`` fp32, lse ``[H, Tq]`` fp32).
    """
    tq, num_heads, head_dim = q.shape
    tk, num_kv_heads = k.shape[0], k.shape[1]
    if tk == 0:
        return (
            torch.zeros(tq, num_heads, head_dim, dtype=torch.float32),
            torch.full((num_heads, tq), float("-inf"), dtype=torch.float32),
        )
    if num_heads != num_kv_heads:
        rep = num_heads // num_kv_heads
        k = k.repeat_interleave(rep, dim=1)
        v = v.repeat_interleave(rep, dim=1)
    kf = k.float()
    vf = v.float()
    # [H, Tq, Tk]; bmm over heads instead of einsum keeps memory bounded.
    qh = q.float().permute(1, 0, 2)
    kh = kf.permute(1, 2, 0).contiguous()
    scores = torch.bmm(qh, kh) * scale
    if q_pos0_in_kv is not None:
        i = torch.arange(tq)[:, None]
        j = torch.arange(tk)[None, :]
        qpos = q_pos0_in_kv + i
        mask = j <= qpos
        if window is not None:
            mask &= j > qpos - window
        scores = scores.masked_fill(~mask, float("-inf"))
    m = scores.amax(dim=-1)  # [H, Tq]
    # Rows with no visible key: the build's convention (out 0, lse -inf).
    empty = torch.isneginf(m)
    m_safe = torch.where(empty, torch.zeros_like(m), m)
    p = torch.exp(scores - m_safe[..., None])
    denom = p.sum(dim=-1)  # [H, Tq]
    out = torch.bmm(p, vf.permute(1, 0, 2).contiguous()).permute(1, 0, 2)
    denom_safe = torch.where(empty, torch.ones_like(denom), denom)
    out = out / denom_safe.permute(1, 0)[..., None]
    lse = m_safe + torch.log(denom)
    lse = torch.where(empty, torch.full_like(lse, float("-inf")), lse)
    return out.contiguous(), lse


def lse_merge(
    o1: torch.Tensor, lse1: torch.Tensor, o2: torch.Tensor, lse2: torch.Tensor
) -> torch.Tensor:
    """Two-way online-softmax merge (ring_backend.py:409-421), fp32.

    o ``[Tq, H, D]``, lse ``[H, Tq]``.  ``m = max(l1, l2)``, ``w = exp(l - m)``,
    ``(o1 w1 + o2 w2) / (w1 + w2)``.  A pair of -inf inputs gives 0 (build
    convention; the reference divides 0 by 0 there).
    """
    lse1 = lse1.float()
    lse2 = lse2.float()
    m = torch.maximum(lse1, lse2)
    m_safe = torch.where(torch.isneginf(m), torch.zeros_like(m), m)
    w1 = torch.exp(lse1 - m_safe)
    w2 = torch.exp(lse2 - m_safe)
    w1e = w1.permute(1, 0)[..., None]
    w2e = w2.permute(1, 0)[..., None]
    den = w1e + w2e
    den = torch.where(den == 0, torch.ones_like(den), den)
    return (o1.float() * w1e + o2.float() * w2e) / den


def merge_pair(
    o1: torch.Tensor, lse1: torch.Tensor, o2: torch.Tensor, lse2: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor]:
    """Merge with the merged LSE (ring_decode.py:46-61).

    ``lse = m + log(exp(l1 - m) + exp(l2 - m))``, the quantity an accumulator
    ring or a running merge carries forward.
    """
    out = lse_merge(o1, lse1, o2, lse2)
    lse1 = lse1.float()
    lse2 = lse2.float()
    m = torch.maximum(lse1, lse2)
    m_safe = torch.where(torch.isneginf(m), torch.zeros_like(m), m)
    lse = m_safe + torch.log(torch.exp(lse1 - m_safe) + torch.exp(lse2 - m_safe))
    lse = torch.where(torch.isneginf(m), m, lse)
    return out, lse


def merge_attn_states(
    output: torch.Tensor,
    prefix_output: torch.Tensor,
    prefix_lse: torch.Tensor,
    suffix_output: torch.Tensor,
    suffix_lse: torch.Tensor,
    output_lse: torch.Tensor | None = None,
) -> None:
    """vLLM ``merge_attn_states`` semantics, restated (external dependency).

    Writes ``output`` (caller-allocated, any float dtype) and, when given,
    ``output_lse``.  An LSE of +inf is read as -inf (vLLM's published kernel
    does the same for FA2-style empty rows).  Call sites pass prefix = peer,
    suffix = local (ring_backend.py:354).
    """
    p = prefix_lse.float().clone()
    s = suffix_lse.float().clone()
    p[torch.isposinf(p)] = float("-inf")
    s[torch.isposinf(s)] = float("-inf")
    out, lse = merge_pair(prefix_output, p, suffix_output, s)
    output.copy_(out.to(output.dtype))
    if output_lse is not None:
        output_lse.copy_(lse)


def kv_cache_update(
    key: torch.Tensor,
    value: torch.Tensor,
    kv_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    layout: str,
) -> None:
    """Write key/value rows ``[0, n)`` (n = len(slot_mapping)) into ``kv_cache``
    in place at slot = block * bs + offset (ring_backend.py:501-539).

    ``layout="v023"``: ``[nb, 2, bs, Hkv, D]``, key_cache / value_cache =
    ``kv_cache.unbind(1)`` (ring_backend.py:533-538).  ``layout="v031"``:
    ``[nb, Hkv, bs, 2*D]`` with K in ``[..., :D]``, V in ``[..., D:]``
    (file_connector.py:13-16).  Negative slots are skipped.
    """
    n = slot_mapping.shape[0]
    keep = slot_mapping >= 0
    slot = slot_mapping[keep].long()
    k, v = key[:n][keep], value[:n][keep]
    bs = kv_cache.shape[2]
    block_idx = torch.div(slot, bs, rounding_mode="floor")
    block_off = slot % bs
    if layout == "v023":
        key_cache, value_cache = kv_cache.unbind(1)
        key_cache[block_idx, block_off] = k
        value_cache[block_idx, block_off] = v
    elif layout == "v031":
        d = kv_cache.shape[3] // 2
        kv_cache[block_idx, :, block_off, :d] = k
        kv_cache[block_idx, :, block_off, d:] = v
    else:
        raise ValueError(layout)


def gather_paged(
    kv_cache: torch.Tensor,
    block_table_row: torch.Tensor,
    start: int,
    length: int,
    layout: str,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Gather tokens ``[start, start+length)`` of one request from the cache.

    ``layout="v023"``: ``[nb, 2, bs, Hkv, D]`` (ring_backend.py:601,617-624).
    ``layout="v031"``: ``[nb, Hkv, bs, 2*D]`` (file_connector.py:13-16,175-179).
    Returns contiguous k, v ``[length, Hkv, D]``.
    """
    end = start + length
    if layout == "v023":
        bs = kv_cache.shape[2]
        nb = (end + bs - 1) // bs
        blocks = block_table_row[:nb].long()
        k = kv_cache[blocks, 0].reshape(-1, kv_cache.shape[3], kv_cache.shape[4])
        v = kv_cache[blocks, 1].reshape(-1, kv_cache.shape[3], kv_cache.shape[4])
    elif layout == "v031":
        bs = kv_cache.shape[2]
        d = kv_cache.shape[3] // 2
        nb = (end + bs - 1) // bs
        blocks = block_table_row[:nb].long()
        sel = kv_cache[blocks]  # [nb, Hkv, bs, 2D]
        sel = sel.permute(0, 2, 1, 3).reshape(-1, kv_cache.shape[1], 2 * d)
        k, v = sel[..., :d], sel[..., d:]
    else:
        raise ValueError(layout)
    return k[start:end].contiguous(), v[start:end].contiguous()


def ring_forward(
    query: torch.Tensor,
    kv_cache: torch.Tensor,
    layout: str,
    query_start_loc: list[int],
    seq_lens: list[int],
    block_table: torch.Tensor,
    scale: float,
    peers: list[tuple[torch.Tensor, torch.Tensor] | None] | None = None,
    split_tokens: int = 0,
    out_dtype: torch.dtype | None = None,
    window: int | None = None,
) -> torch.Tensor:
    """Restated segmentation of ``HcpRingAttentionImpl.forward``.

    ring_backend.py:576-834, prefill / legacy single-GPU decode branch:

    * per request ``r``: ``qs, qe`` from ``query_start_loc``, ``tk = seq_lens[r]``,
      skip ``tq == 0`` (:611-616);
    * local KV = paged gather of the first ``tk`` tokens (:617-624);
    * ``qpos0 = tk - tq`` (:627);
    * peer = ``peers[r]`` (the staged, concatenated chunks, :738-772) with
      ``peer_end = min(len(peer), tk)`` (:775), else the split env
      ``peer_end = min(split, tk)`` over the local KV (:776-778);
    * ``peer_end == 0``: causal over all local KV at offset ``qpos0`` (:783-789);
    * the first ``n_a = max(0, min(tq, peer_end - qpos0))`` queries: causal over
      all local KV (:811-817);
    * the rest: local causal on ``k_all[peer_end:]`` at offset
      ``qpos0 + n_a - peer_end`` (:820-827), peer non-causal (:828-830),
      merged (:831), cast to the output dtype (:832);
    * ``window`` (``self.sliding_window``) goes to every causal call
      (:786, :815, :826), never to the non-causal peer call (:828-830).
    """
    out_dtype = out_dtype or query.dtype
    output = torch.zeros(query.shape, dtype=out_dtype)
    for r in range(len(seq_lens)):
        qs, qe = query_start_loc[r], query_start_loc[r + 1]
        tq = qe - qs
        tk = seq_lens[r]
        if tq == 0:
            continue
        k_all, v_all = gather_paged(kv_cache, block_table[r], 0, tk, layout)
        q_r = query[qs:qe]
        qpos0 = tk - tq
        staged = peers[r] if peers is not None else None
        if staged is not None:
            k_peer, v_peer = staged
            peer_end = min(k_peer.shape[0], tk)
        elif split_tokens > 0:
            peer_end = min(split_tokens, tk)
            k_peer, v_peer = k_all[:peer_end], v_all[:peer_end]
        else:
            peer_end = 0
            k_peer = v_peer = None
        if peer_end == 0:
            o, _ = attn_with_lse(q_r, k_all, v_all, scale, qpos0, window)
            output[qs:qe] = o.to(out_dtype)
            continue
        n_a = max(0, min(tq, peer_end - qpos0))
        if n_a > 0:
            o_a, _ = attn_with_lse(q_r[:n_a], k_all, v_all, scale, qpos0, window)
            output[qs : qs + n_a] = o_a.to(out_dtype)
        if n_a < tq:
            q_b = q_r[n_a:]
            o_loc, lse_loc = attn_with_lse(
                q_b, k_all[peer_end:], v_all[peer_end:], scale,
                qpos0 + n_a - peer_end, window,
            )
            o_peer, lse_peer = attn_with_lse(q_b, k_peer, v_peer, scale, None)
            o_b = lse_merge(o_loc, lse_loc, o_peer, lse_peer)
            output[qs + n_a : qe] = o_b.to(out_dtype)
    return output


def ring_decode_hop(
    q: torch.Tensor,
    o_acc: torch.Tensor,
    lse_acc: torch.Tensor,
    k_snap: torch.Tensor,
    v_snap: torch.Tensor,
    growth_k: torch.Tensor | None,
    growth_v: torch.Tensor | None,
    scale: float,
) -> tuple[torch.Tensor, torch.Tensor]:
    """One node's accumulator step (ring_decode.py:224-237), fp32.

    ``k = cat(k_snap, growth_k)`` (:229-232), ``(o_loc, lse_loc)`` non-causal
    over it (:234-236), then ``merge_pair(o_acc, lse_acc, o_loc, lse_loc)``
    (:237).
    """
    k, v = k_snap.float(), v_snap.float()
    if growth_k is not None:
        k = torch.cat([k, growth_k.float()], dim=0)
        v = torch.cat([v, growth_v.float()], dim=0)
    o_loc, lse_loc = attn_with_lse(q.float(), k, v, scale, None)
    return merge_pair(o_acc.float(), lse_acc.float(), o_loc, lse_loc)


class DecodeRingSim:
    """The memory-split decode protocol of one request, restated in fp32.

    Ring order: transport index 0 is the owner, 1..N-1 the prefix peers
    (growth index i -> transport i + 1; the owner's growth index is N - 1).
    ``peer_chunks[i]`` is peer i's chunk snapshot ``(k, v)``; ``own_chunk`` the
    owner's own chunk (its pool region ``[plen, plen + own_len)``).
    ``step(q, k_cur, v_cur, pos)`` is one decode step of one layer:

    * owner (ring_backend.py:652-689): ``assignee = growth_assignee(pos)``;
      ``ship`` = the previous step's pending token; local partial over
      ``own chunk + owned growth + current token`` (causal at ``len-1``: every
      key visible, or the last ``window`` of them with a sliding window); the
      current token joins the owned growth or becomes the pending token;
    * the packet visits peers 1..N-1 in order (ring_decode.py:187-259): a node
      appends shipped growth when it is the target, then merges its partial
      over ``snapshot + its growth`` into the accumulator.

    Returns the final (O, LSE) the owner receives, plus the growth held by
    every ring member (``growth_of[i]`` for transport index i).
    """

    def __init__(self, peer_chunks, own_chunk, scale: float, policy: str = "rr",
                 window: int | None = None):
        self.window = window
        self.peer_chunks = [(k.float(), v.float()) for k, v in peer_chunks]
        self.own_k, self.own_v = own_chunk[0].float(), own_chunk[1].float()
        self.scale = scale
        self.policy = policy
        self.n = len(peer_chunks) + 1
        self.growth_of: list[list[tuple[torch.Tensor, torch.Tensor]]] = [
            [] for _ in range(self.n)]
        self.pending = None

    def assignee(self, pos: int) -> int:
        """ring_decode.py:30-43 (growth index)."""
        return self.n - 1 if self.policy == "owner" else pos % self.n

    @staticmethod
    def _cat(base_k, base_v, extra):
        ks = [base_k] + [k for k, _ in extra]
        vs = [base_v] + [v for _, v in extra]
        return torch.cat(ks, 0), torch.cat(vs, 0)

    def step(self, q, k_cur, v_cur, pos: int):
        q, k_cur, v_cur = q.float(), k_cur.float(), v_cur.float()
        a = self.assignee(pos)
        ship, self.pending = self.pending, None
        owner_t = 0
        k_loc, v_loc = self._cat(self.own_k, self.own_v,
                                 self.growth_of[owner_t] + [(k_cur, v_cur)])
        o, lse = attn_with_lse(q, k_loc, v_loc, self.scale, k_loc.shape[0] - 1, self.window)
        if a == self.n - 1:
            self.growth_of[owner_t].append((k_cur, v_cur))
        else:
            self.pending = (a + 1, k_cur, v_cur)
        for t in range(1, self.n):
            if ship is not None and ship[0] == t:
                self.growth_of[t].append((ship[1], ship[2]))
                ship = None
            ck, cv = self.peer_chunks[t - 1]
            gk = gv = None
            if self.growth_of[t]:
                gk = torch.cat([k for k, _ in self.growth_of[t]], 0)
                gv = torch.cat([v for _, v in self.growth_of[t]], 0)
            o, lse = ring_decode_hop(q, o, lse, ck, cv, gk, gv, self.scale)
        return o, lse


def causal_pairs(tq: int, tk: int, offset: int | None) -> int:
    """Visible (query, key) pairs: ``sum_i min(Tk, max(0, o + i + 1))``."""
    if offset is None:
        return tq * tk
    total = 0
    # closed form over the three regimes of o + i + 1
    for i in range(tq):
        total += min(tk, max(0, offset + i + 1))
    return total


def attn_flops(num_heads: int, head_dim: int, pairs: int) -> int:
    """Algorithmic attention FLOPs: ``4 * D * H * pairs`` (QK^T and PV)."""
    return 4 * head_dim * num_heads * pairs


def _selfcheck() -> None:  # pragma: no cover - manual use
    g = torch.Generator().manual_seed(0)
    q = torch.randn(5, 4, 16, generator=g)
    k = torch.randn(7, 2, 16, generator=g)
    v = torch.randn(7, 2, 16, generator=g)
    o, lse = attn_with_lse(q, k, v, 1 / math.sqrt(16), 2)
    print(o.shape, lse.shape)


if __name__ == "__main__":  # pragma: no cover
    _selfcheck()
