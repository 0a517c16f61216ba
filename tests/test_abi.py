"""CPU checks of the C-ABI library (no GPU needed, no kernel launched).

* libhcp_mi355x.so loads and exports every function include/hcp_mi355x.h
  declares, with the declared ABI version.
* The host-side planners (hcp_plan_varlen_tiles, hcp_plan_decode_splits,
  hcp_decode_workspace_bytes) run on the CPU: their output is checked against
  brute-force enumeration of the work they describe.
* Argument validation returns the documented status codes (and text through
  hcp_last_error) before anything reaches the GPU.
"""

import ctypes
import os
import re
import subprocess

import pytest

from hcp_vllm_plugin_amd import _lib
from hcp_vllm_plugin_amd._lib import DecodeSplit, KvSegment, VarlenEntry

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hcp_mi355x.h")


def header_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(hcp_[a-z_0-9]+)\s*\(", src, re.M)


@pytest.fixture(scope="module")
def L():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} not built: run __graft_entry__.build()")
    return _lib.lib()


def test_header_declares_what_the_wrapper_binds():
    assert sorted(header_functions()) == sorted(_lib.EXPORTED_SYMBOLS)


def test_library_exports_every_header_symbol(L):
    names = header_functions()
    assert len(names) >= 10
    for n in names:
        assert hasattr(L, n), n
    # and they are real dynamic exports with C linkage (no C++ mangling)
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH],
                         capture_output=True, text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    for n in names:
        assert n in exported, n


def test_abi_version(L):
    assert L.hcp_abi_version() == _lib.ABI_VERSION


def test_struct_layouts_match_header():
    # hcp_kv_segment: 3 u64 + 5 i64 + 2 i32 = 72 bytes; entry adds 3 i64
    assert ctypes.sizeof(KvSegment) == 72
    assert ctypes.sizeof(VarlenEntry) == 96
    assert ctypes.sizeof(DecodeSplit) == 16
    assert VarlenEntry.kv.offset == 24
    # hcp_paged_cache: 2 u64 + 4 i64 + 2 i32 = 56 bytes
    assert ctypes.sizeof(_lib.PagedCacheDesc) == 56


def _entry(q_start, q_len, off, kv_len, start=0):
    e = VarlenEntry()
    e.q_start, e.q_len, e.causal_offset = q_start, q_len, off
    e.kv.k_addr = e.kv.v_addr = 0x1000
    e.kv.stride_tok, e.kv.stride_head = 512, 128
    e.kv.start, e.kv.len = start, kv_len
    return e


@pytest.mark.parametrize("causal", [0, 1])
def test_plan_varlen_tiles_covers_every_block_longest_first(L, causal):
    specs = [(0, 300, 0, 300), (300, 1, 5, 900), (301, 129, 40, 200), (430, 0, 0, 10),
             (430, 700, -50, 700), (1130, 256, 10000, 64)]
    ents = [_entry(*s) for s in specs]
    arr = (VarlenEntry * len(ents))(*ents)
    bm = L.hcp_varlen_block_m(128, _lib.DTYPE_BF16)
    assert bm > 0
    need = sum(-(-s[1] // bm) for s in specs)
    tiles = (ctypes.c_int32 * (2 * need))()
    n = L.hcp_plan_varlen_tiles(ctypes.addressof(arr), len(ents), causal, bm,
                                ctypes.addressof(tiles), need)
    assert n == need
    got = [(tiles[2 * i], tiles[2 * i + 1]) for i in range(n)]
    want = {(e, b) for e, s in enumerate(specs) for b in range(-(-s[1] // bm))}
    assert set(got) == want and len(got) == len(want)

    def cost(e, b):
        q_start, q_len, off, kv_len = specs[e]
        if not causal:
            return kv_len
        # keys visible to the block's last row, by enumeration
        last = min((b + 1) * bm, q_len + bm) - 1
        return sum(1 for j in range(kv_len) if j <= off + last)

    costs = [cost(e, b) for e, b in got]
    assert costs == sorted(costs, reverse=True)
    # too small a cap is reported, not overrun
    rc = L.hcp_plan_varlen_tiles(ctypes.addressof(arr), len(ents), causal, bm,
                                 ctypes.addressof(tiles), need - 1)
    assert rc == _lib.HCP_EWORKSPACE
    assert b"need" in L.hcp_last_error()


def test_plan_varlen_tiles_rejects_small_paged_blocks(L):
    """Paged prefill reads each wave's 16 rows of a tile from one block."""
    arr = (VarlenEntry * 2)(_entry(0, 100, 0, 300), _entry(100, 50, 0, 200))
    for bs, want in ((8, _lib.HCP_EUNSUPPORTED), (16, None), (32, None)):
        arr[1].kv.block_table = 0x2000
        arr[1].kv.block_size = bs
        arr[1].kv.stride_block = 4 * bs * 256
        tiles = (ctypes.c_int32 * 64)()
        rc = L.hcp_plan_varlen_tiles(arr, 2, 1, 128, tiles, 32)
        if want is None:
            assert rc > 0, (bs, rc)
        else:
            assert rc == want, (bs, rc)
            assert b"block_size >= 16" in L.hcp_last_error()


def test_plan_varlen_tiles_rejects_strides_beyond_32bit_offsets(L):
    """The prefill kernel forms tile offsets in 32 bits: a contiguous token
    stride of 2^24 elements or more, a block stride of 2^31 or more, or a
    block whose rows span over 4 GiB is refused, not mis-addressed."""
    def plan(**kv):
        e = _entry(0, 100, 0, 300)
        for k, v in kv.items():
            setattr(e.kv, k, v)
        arr = (VarlenEntry * 1)(e)
        tiles = (ctypes.c_int32 * 8)()
        return L.hcp_plan_varlen_tiles(arr, 1, 1, 128, tiles, 4)

    assert plan() == 1
    assert plan(stride_tok=1 << 24) == _lib.HCP_EUNSUPPORTED
    paged = dict(block_table=0x2000, block_size=16, stride_block=16 * 1024, stride_tok=256)
    assert plan(**paged) == 1
    assert plan(**{**paged, "stride_block": 1 << 31}) == _lib.HCP_EUNSUPPORTED
    # 256 rows at a 2^23-element (16 MiB) token stride: a block spans 4 GiB + 1 row
    big = {**paged, "block_size": 256, "stride_tok": (1 << 23) + 8, "stride_block": 1 << 30}
    assert plan(**big) == _lib.HCP_EUNSUPPORTED
    assert b"4 GiB" in L.hcp_last_error()


def test_plan_decode_splits_partition_each_segment(L):
    # 3 sequences: (kv lens of its entries)
    seqs = [[4096, 700], [0, 1], [33, 2048, 5]]
    ents, seq_of = [], []
    for s, lens in enumerate(seqs):
        for ln in lens:
            ents.append(_entry(s, 1, 0, ln))
            seq_of.append(s)
    arr = (VarlenEntry * len(ents))(*ents)
    sq = (ctypes.c_int32 * len(ents))(*seq_of)
    split = 256
    cap = sum(-(-e.kv.len // split) for e in ents)
    out = (DecodeSplit * cap)()
    starts = (ctypes.c_int32 * (len(seqs) + 1))()
    n = L.hcp_plan_decode_splits(ctypes.addressof(arr), len(ents), ctypes.addressof(sq),
                                 len(seqs), 0, split, ctypes.addressof(out), cap,
                                 ctypes.addressof(starts))
    assert n == cap
    sp = [(out[i].entry, out[i].key_begin, out[i].key_end) for i in range(n)]
    # every key of every entry in exactly one split, each split <= split_tokens
    for ei, e in enumerate(ents):
        keys = []
        for en, b, k in sp:
            if en == ei:
                assert 0 < k - b <= split
                keys.extend(range(b, k))
        assert keys == list(range(e.kv.len))
    # partial slots of sequence s are exactly the splits of its entries, and
    # the slots are a permutation of 0..n-1
    slots = [out[i].slot for i in range(n)]
    assert sorted(slots) == list(range(n))
    for s in range(len(seqs)):
        mine = sorted(slots[i] for i, (en, _, _) in enumerate(sp) if seq_of[en] == s)
        assert mine == list(range(starts[s], starts[s + 1]))
    assert starts[len(seqs)] == n
    # dispatch order: longest first; equal lengths keep sequence order
    lens = [k - b for _, b, k in sp]
    assert lens == sorted(lens, reverse=True)
    for i in range(n - 1):
        if lens[i] == lens[i + 1]:
            assert slots[i] < slots[i + 1]


def test_plan_decode_splits_causal_limit_and_errors(L):
    ents = [_entry(0, 1, 99, 1000)]
    arr = (VarlenEntry * 1)(*ents)
    sq = (ctypes.c_int32 * 1)(0)
    out = (DecodeSplit * 8)()
    starts = (ctypes.c_int32 * 2)()
    n = L.hcp_plan_decode_splits(ctypes.addressof(arr), 1, ctypes.addressof(sq), 1, 1, 64,
                                 ctypes.addressof(out), 8, ctypes.addressof(starts))
    assert n == 2 and out[1].key_end == 100  # keys j <= 99
    # q_len != 1 is rejected
    ents[0].q_len = 2
    arr = (VarlenEntry * 1)(*ents)
    rc = L.hcp_plan_decode_splits(ctypes.addressof(arr), 1, ctypes.addressof(sq), 1, 0, 64,
                                  ctypes.addressof(out), 8, ctypes.addressof(starts))
    assert rc == _lib.HCP_EINVAL
    assert b"q_len" in L.hcp_last_error()


def test_decode_workspace_bytes(L):
    n, h, d = 37, 28, 128
    b = L.hcp_decode_workspace_bytes(n, h, d)
    o = n * h * d * 4
    assert b >= o + n * h * 4 and b - (o + n * h * 4) < 256
    assert L.hcp_decode_workspace_bytes(0, h, d) == 0


def _fwd(L, **kw):
    a = dict(q=16, k=16, v=16, out=16, lse=16, tq=4, tk=4, h=28, hkv=4, d=128,
             st=8, causal=1, off=0, window=0, dtype=_lib.DTYPE_BF16, scale=0.088)
    a.update(kw)
    s = a["st"]
    return L.hcp_attn_fwd_lse(a["q"], a["k"], a["v"], a["out"], a["lse"], a["tq"], a["tk"],
                              a["h"], a["hkv"], a["d"], s * a["h"], s, s * a["hkv"], s,
                              s * a["hkv"], s, s * a["h"], s, a["tq"], a["scale"],
                              a["causal"], a["off"], a["window"], a["dtype"], None)


def test_argument_validation_status_codes(L):
    assert _fwd(L, h=6, hkv=4) == _lib.HCP_EINVAL
    assert b"multiple" in L.hcp_last_error()
    assert _fwd(L, d=264) == _lib.HCP_EUNSUPPORTED
    assert _fwd(L, dtype=_lib.DTYPE_F32) == _lib.HCP_EUNSUPPORTED
    assert _fwd(L, tq=-1) == _lib.HCP_EINVAL
    assert _fwd(L, scale=float("nan")) == _lib.HCP_EINVAL
    assert _fwd(L, q=None) == _lib.HCP_EINVAL
    assert _fwd(L, q=24) == _lib.HCP_EINVAL          # not 16-byte aligned
    assert _fwd(L, st=12) == _lib.HCP_EINVAL         # stride not a multiple of 8
    assert _fwd(L, tq=0) == _lib.HCP_OK              # nothing to do, nothing launched
    assert _fwd(L, window=-1) == _lib.HCP_EINVAL
    assert b"negative window" in L.hcp_last_error()
    # a K/V token stride the kernel's 32-bit tile offsets cannot step over
    # (2^24 elements or more) is refused, as the varlen planner refuses it
    big = 1 << 24
    rc = L.hcp_attn_fwd_lse(16, 16, 16, 16, 16, 4, 4, 28, 4, 128, 8 * 28, 8, big, 8, big, 8,
                            8 * 28, 8, 4, 0.088, 1, 0, 0, _lib.DTYPE_BF16, None)
    assert rc == _lib.HCP_EUNSUPPORTED and b"2^24" in L.hcp_last_error()
    rc = L.hcp_attn_fwd_lse_merge(16, 16, 16, 16, None, 4, 4, 28, 4, 128, 8 * 28, 8, big, 8,
                                  big, 8, 8 * 28, 8, 4, 0.088, 1, 0, 0, 16, 8 * 28, 8, 16, 4, 1,
                                  _lib.DTYPE_BF16, None)
    assert rc == _lib.HCP_EUNSUPPORTED
    rc = L.hcp_merge_attn_states(16, 8, 8, 7, None, 0, 16, 8, 8, 1, 16, 4, 16, 8, 8, 1, 16, 4,
                                 4, 1, 8, None)
    assert rc == _lib.HCP_EUNSUPPORTED  # out dtype 7
    rc = L.hcp_merge_attn_states(16, 8, 8, 1, None, 0, 16, 8, 8, 1, 16, 4, 16, 8, 8, 1, 16, 4,
                                 4, 1, 12, None)
    assert rc == _lib.HCP_EUNSUPPORTED  # head_dim 12


def _fwd_merge(L, **kw):
    a = dict(q=16, k=16, v=16, out=16, lse=None, tq=4, tk=4, h=28, hkv=4, d=128, st=8,
             causal=1, off=0, window=0, acc=16, acc_lse=16, acc_st=8, prefix=1,
             dtype=_lib.DTYPE_BF16, scale=0.088)
    a.update(kw)
    s, h = a["st"], a["h"]
    return L.hcp_attn_fwd_lse_merge(a["q"], a["k"], a["v"], a["out"], a["lse"], a["tq"], a["tk"],
                                    h, a["hkv"], a["d"], s * h, s, s * a["hkv"], s,
                                    s * a["hkv"], s, s * h, s, a["tq"], a["scale"], a["causal"],
                                    a["off"], a["window"], a["acc"], a["acc_st"] * h,
                                    a["acc_st"], a["acc_lse"], a["tq"], a["prefix"], a["dtype"],
                                    None)


def _varlen_merge(L, **kw):
    a = dict(tiles=16, ntiles=1, acc=16, acc_lse=16, acc_st=8, lse=None)
    a.update(kw)
    return L.hcp_attn_fwd_varlen_merge(16, 8 * 28, 8, 16, 8 * 28, 8, a["lse"], 0, 16, 1,
                                       a["tiles"], a["ntiles"], 28, 4, 128, 0.088, 1, 0, 1,
                                       a["acc"], a["acc_st"] * 28, a["acc_st"], a["acc_lse"],
                                       4, 1, _lib.DTYPE_BF16, None)


def test_attn_merge_status_codes(L):
    """Argument checks of the attention + merge entry points, all returned
    before any launch; without a partial state the plain pass still needs lse."""
    assert _fwd_merge(L, acc=None) == _lib.HCP_EINVAL
    assert b"null merge partial" in L.hcp_last_error()
    assert _fwd_merge(L, acc_lse=None) == _lib.HCP_EINVAL
    assert _fwd_merge(L, acc=24) == _lib.HCP_EINVAL        # not 16-byte aligned
    assert b"aligned" in L.hcp_last_error()
    assert _fwd_merge(L, acc_st=12) == _lib.HCP_EINVAL     # stride not a multiple of 8
    assert _fwd_merge(L, d=264) == _lib.HCP_EUNSUPPORTED
    assert _fwd_merge(L, window=-1) == _lib.HCP_EINVAL
    assert _fwd_merge(L, tq=0) == _lib.HCP_OK               # nothing to do, nothing launched
    assert _fwd(L, lse=None) == _lib.HCP_EINVAL
    assert b"hcp_attn_fwd_lse:" in L.hcp_last_error()
    assert _varlen_merge(L, acc=None) == _lib.HCP_EINVAL
    assert b"hcp_attn_fwd_varlen_merge" in L.hcp_last_error()
    assert _varlen_merge(L, acc=40) == _lib.HCP_EINVAL
    assert _varlen_merge(L, acc_st=4) == _lib.HCP_EINVAL
    assert _varlen_merge(L, ntiles=0) == _lib.HCP_OK


def _dec_acc(L, **kw):
    a = dict(q=16, acc_o=16, acc_lse=16, out=16, h=28, hkv=4, d=128, seqs=1, scale=0.1,
             dtype=_lib.DTYPE_BF16)
    a.update(kw)
    return L.hcp_decode_splitkv_acc(a["q"], 4096, 128, None, 0, None, 0, 16, a["seqs"], None, 0,
                                    a["acc_o"], 4096, 128, a["acc_lse"], 1, a["out"], 4096, 128,
                                    None, 0, a["h"], a["hkv"], a["d"], a["scale"], a["dtype"],
                                    None)


def test_decode_splitkv_acc_status_codes(L):
    """Argument checks of the accumulator decode, all returned before any launch."""
    assert _dec_acc(L, acc_o=None) == _lib.HCP_EINVAL
    assert b"null accumulator" in L.hcp_last_error()
    assert _dec_acc(L, acc_lse=None) == _lib.HCP_EINVAL
    assert _dec_acc(L, acc_o=17) == _lib.HCP_EINVAL       # odd address
    assert _dec_acc(L, d=264) == _lib.HCP_EUNSUPPORTED
    assert _dec_acc(L, h=30) == _lib.HCP_EINVAL           # not a multiple of hkv
    assert _dec_acc(L, scale=0.0) == _lib.HCP_EINVAL
    assert _dec_acc(L, seqs=0) == _lib.HCP_OK              # nothing to do, nothing launched


def test_decode_noalloc_limit_and_status_codes(L):
    """The allocation-free decode's scratch limit is the header's, and plans
    beyond it (and bad arguments) are refused before any HIP call."""
    src = open(HEADER).read()
    m = re.search(r"#define HCP_NOALLOC_SCRATCH_BYTES \((\d+)u << (\d+)\)", src)
    assert m and int(m.group(1)) << int(m.group(2)) == _lib.NOALLOC_SCRATCH_BYTES

    def call(splits=8, seqs=1, h=28, hkv=4, d=128, dtype=_lib.DTYPE_BF16):
        return L.hcp_decode_splitkv_noalloc(16, 128 * h, 128, 16, 1, 16, splits, 16, seqs,
                                            16, 128 * h, 128, None, 0, h, hkv, d, 0.1, dtype,
                                            None)

    # largest split count that fits: partials + LSE, 256-byte aligned
    fit = max(n for n in range(1, 2000)
              if L.hcp_decode_workspace_bytes(n, 28, 128) <= _lib.NOALLOC_SCRATCH_BYTES)
    assert fit == 1161
    assert call(splits=fit + 1) == _lib.HCP_EWORKSPACE
    assert b"fixed scratch" in L.hcp_last_error()
    assert call(d=264) == _lib.HCP_EUNSUPPORTED
    assert call(h=30) == _lib.HCP_EINVAL
    assert call(dtype=_lib.DTYPE_F32) == _lib.HCP_EUNSUPPORTED
    assert call(splits=-1) == _lib.HCP_EINVAL
    assert call(seqs=0) == _lib.HCP_OK  # nothing to do: no device touched


def _cache_desc(bs=16, nb=4):
    c = _lib.PagedCacheDesc()
    c.k_addr, c.v_addr = 0x1000, 0x1100
    c.stride_block, c.stride_head, c.stride_tok = 4 * bs * 256, bs * 256, 256
    c.num_blocks, c.block_size = nb, bs
    return c


def _rc(L, **kw):
    a = dict(key=16, value=16, kst=512, khst=128, slots=16, sdt=_lib.DTYPE_I64, n=4, hkv=4,
             d=128, cache=_cache_desc(), dtype=_lib.DTYPE_BF16)
    a.update(kw)
    c = a["cache"]
    return L.hcp_reshape_and_cache(a["key"], a["kst"], a["khst"], a["value"], a["kst"],
                                   a["khst"], a["slots"], a["sdt"], a["n"], a["hkv"], a["d"],
                                   ctypes.byref(c) if c is not None else None, a["dtype"], None)


def test_reshape_and_cache_status_codes(L):
    """Argument checks of the cache write, all returned before any launch."""
    assert _rc(L, n=0) == _lib.HCP_OK                       # nothing to write
    assert _rc(L, cache=_cache_desc(nb=0)) == _lib.HCP_OK   # empty cache
    assert _rc(L, d=12) == _lib.HCP_EUNSUPPORTED
    assert _rc(L, dtype=_lib.DTYPE_F32) == _lib.HCP_EUNSUPPORTED
    assert _rc(L, sdt=_lib.DTYPE_BF16) == _lib.HCP_EUNSUPPORTED
    assert b"slot dtype" in L.hcp_last_error()
    assert _rc(L, cache=None) == _lib.HCP_EINVAL
    assert _rc(L, cache=_cache_desc(bs=12)) == _lib.HCP_EINVAL
    assert b"power of two" in L.hcp_last_error()
    assert _rc(L, key=None) == _lib.HCP_EINVAL
    assert _rc(L, slots=None) == _lib.HCP_EINVAL
    assert _rc(L, value=24) == _lib.HCP_EINVAL              # not 16-byte aligned
    assert _rc(L, kst=500) == _lib.HCP_EINVAL               # stride not a multiple of 8
    assert _rc(L, n=-1) == _lib.HCP_EINVAL


def test_check_raises_runtime_error_with_library_text(L):
    rc = _fwd(L, d=264)
    with pytest.raises(RuntimeError, match="EUNSUPPORTED.*head_dim 264"):
        _lib.check(rc, "hcp_attn_fwd_lse")


def test_gather_paged_kv_status_codes(L):
    """Argument checks of hcp_gather_paged_kv, all before any device work."""
    g = L.hcp_gather_paged_kv
    # nothing to do: no entries, or no keys
    assert g(0, 0, 0, 0, 4, 128, _lib.DTYPE_BF16, 0, 0, 0) == 0
    assert g(16, 3, 16, 0, 4, 128, _lib.DTYPE_BF16, 16, 16, 0) == 0
    assert g(16, 3, 16, 10, 0, 128, _lib.DTYPE_BF16, 16, 16, 0) == _lib.HCP_EINVAL
    assert g(16, -1, 16, 10, 4, 128, _lib.DTYPE_BF16, 16, 16, 0) == _lib.HCP_EINVAL
    assert g(16, 3, 16, 10, 4, 132, _lib.DTYPE_BF16, 16, 16, 0) == _lib.HCP_EUNSUPPORTED
    assert g(16, 3, 16, 10, 4, 264, _lib.DTYPE_BF16, 16, 16, 0) == _lib.HCP_EUNSUPPORTED
    assert g(16, 3, 16, 10, 4, 128, _lib.DTYPE_F32, 16, 16, 0) == _lib.HCP_EUNSUPPORTED
    assert g(0, 3, 16, 10, 4, 128, _lib.DTYPE_BF16, 16, 16, 0) == _lib.HCP_EINVAL  # null
    assert g(16, 3, 16, 10, 4, 128, _lib.DTYPE_BF16, 8, 16, 0) == _lib.HCP_EINVAL  # align
    assert g(16, 70000, 16, 10, 4, 128, _lib.DTYPE_BF16, 16, 16, 0) == _lib.HCP_EINVAL
    assert "hcp_gather_paged_kv" in L.hcp_last_error().decode()
    # a launch of max_len * heads * head_dim / 8 threads beyond 32 bits is
    # refused on the host (grid.x * 256 must fit 32 bits): 2^28 rows at
    # head_dim 128 is 2^32 threads
    assert g(16, 3, 16, 1 << 26, 4, 128, _lib.DTYPE_BF16, 16, 16, 0) == _lib.HCP_EINVAL
    assert "2^32" in L.hcp_last_error().decode()
