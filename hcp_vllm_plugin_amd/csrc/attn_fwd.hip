// Flash-attention forward with per-row LSE for gfx950 (CDNA4).
//
// Computes, for every query row i of a query range and every query head h,
//   out[i,h,:] = softmax_j(scale * q[i,h,:] . k[j,h/G,:]) @ v[:,h/G,:]
//   lse[h,i]   = log sum_j exp(scale * q . k)       (natural log)
// over the keys j of one KV segment, with optional causal masking
// j <= causal_offset + i.  This is the operation of ring_attn_with_lse /
// _ring_fwd_kernel (hcp_vllm_plugin/ring_triton_attn.py:35-207): online
// softmax in the exp2 domain with the scale pre-multiplied by log2(e)
// (:119-125,186), P rounded to the input dtype before the PV product (:133),
// lse = m * ln2 + ln(l) (:140), GQA head map h / G (:64).
//
// Design (one workgroup = 4 waves = 128 query rows of one head, 32 per wave;
// two workgroups per CU, i.e. two waves per SIMD):
//  * S^T = K Q^T on v_mfma_f32_32x32x16_{bf16,f16}: K (keys x D) is the A
//    operand read from LDS, Q^T the B operand held in registers for the whole
//    kernel.  In the 32x32 accumulator layout a lane owns one column, so each
//    lane owns ONE query row and 16 of its keys per 32-key block: the row max
//    is an in-register max3 chain plus one exchange with lane ^ 32, and the
//    row sum stays a per-lane partial until the epilogue.
//  * O^T = V^T P^T on the same MFMA: P^T comes straight from the S^T
//    registers (the key order inside the k dimension is a free permutation);
//    the V^T A operand is read from a row-major V tile with the gfx950
//    transposing LDS read ds_read_b64_tr_b16: inside each 16-lane block,
//    lane 4e+a reads 4 consecutive d of key kbase+e and every lane receives 4
//    keys of one d column.
//  * Software pipeline over 64-key tiles: iteration n computes S(n+1) on the
//    matrix pipe while the VALU turns S(n) into P(n) and sums it (phase A, at
//    raised wave priority), then O += V(n)^T P(n)^T on the matrix pipe alone
//    (phase B), while the other wave on the SIMD fills the VALU.  Each phase-A
//    MFMA step carries its own share of VALU work, and every MFMA its LDS
//    reads a few MFMAs ahead, written out in order and pinned with scheduling
//    barriers, so the softmax runs under the MFMAs instead of between them.
//  * K and V tiles (64 keys x D, row-major, 16-byte slots XOR-swizzled by
//    2*(row&3) | (row>>2 & 1) so both the K reads and the transposing V reads
//    are bank-conflict free) go HBM/L2 -> LDS with buffer_load ... lds (no
//    register staging, no VALU work), one load instruction every two MFMAs of
//    phase A, K and V alternating.  Two K and two V buffers: iteration n reads
//    K(n+1), V(n) and fills K(n+2), V(n+1) (both buffers free since the last
//    barrier, so all its loads start in phase A and have phase B to land);
//    one barrier per tile.
//  * Lazy rescale without a per-tile max: P = exp2(c S - m_ref) is formed
//    against the current reference (the row max of the row's first tile)
//    together with its f32 row sum.  A lane whose 32 values of the tile sum
//    to at most 2^12 holds no P above 2^12, and the tile goes straight to the
//    PV MFMAs; otherwise (a score far above the reference, rare past a row's
//    first tile) the wave takes the tile's true row max, rescales O and l,
//    and forms P again.  O, l and lse all use the same reference.
//  * Two row sums: l of P in f32 gives the LSE, and lr of P as rounded to
//    the input dtype for the PV product (v_dot2 against (1, 1)) normalises
//    O.  Against a lazy reference a dominant key's P is 2^x with fractional x
//    (the reference kernel's running max gives it exactly 1), whose rounding
//    would shift the output by up to 2^-8 of that key's V; normalising by the
//    sum of the same rounded weights cancels it, keeping the output error at
//    the reference kernel's level.
//  * Causal tiles above a wave's diagonal are skipped; masking runs only on
//    diagonal and ragged tiles.  A ragged last tile is bounded by its buffer
//    descriptor (rows past the segment read as zeros and are masked), so no
//    load leaves the segment and none is predicated.
//  * The local (paged) segment is read in place through the block table
//    (hcp_kv_segment), replacing the per-request gather copy of
//    ring_backend.py:617-624; block ids are fetched ahead of the tile loads.
#include <type_traits>

#include "params.h"

namespace hcp {

#ifndef HCP_KPF
#define HCP_KPF 3  // K fragment reads issued this many MFMAs ahead (phase A)
#endif
#ifndef HCP_VPF
#define HCP_VPF 2  // V fragment reads issued this many MFMAs ahead (phase B)
#endif
#ifndef HCP_FWD_WAVES_PER_EU
#define HCP_FWD_WAVES_PER_EU 2
#endif

constexpr float kSumThresh = 4096.0f;  // a lane's P sum over a tile: P <= 2^12 without a rescale
// word 3 of a raw (stride 0) buffer descriptor on gfx9-family parts:
// DATA_FORMAT = 32 bit, no swizzle, bounds checked against num_records
constexpr int kBufferRsrcWord3 = 0x00020000;

typedef short i16x4 __attribute__((ext_vector_type(4)));

#define HCP_LDS(T) __attribute__((address_space(3))) T

// XOR swizzle of the 16-byte slot index of tile row `row`.  gfx950 LDS has 64
// banks of 4 bytes: a ds_read_b128 serves 16 lanes per cycle (16 consecutive
// K rows, same logical slot -> the swizzle is a bijection on row & 15) and a
// ds_read_b64_tr_b16 serves 32 lanes (4 key rows e = row & 3, 64 bytes each
// -> rows e move to disjoint 64-byte slot groups).  For D = 64 two 128-byte
// rows share the 256-byte bank space, so the row parity takes that role.
template <int D>
__device__ __forceinline__ int tile_swz(int row) {
  if constexpr (D >= 128) return 4 * (row & 3) + ((row >> 2) & 3);
  return 4 * ((row >> 1) & 1) + ((row >> 2) & 3);
}

// The lane's index in its wave, read afresh: an opaque read the compiler
// cannot merge with an earlier one, so a value derived from it is rebuilt
// where it is used instead of being held in a register across the tile loop
// (which needs every register).
__device__ __forceinline__ int lane_id_fresh() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

template <typename V8>
__device__ __forceinline__ V8 lds_read16(const HCP_LDS(char)* p) {
  return __builtin_bit_cast(V8, *reinterpret_cast<const HCP_LDS(u32x4)*>(p));
}

__device__ __forceinline__ i16x4 lds_read_tr(const HCP_LDS(char)* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      reinterpret_cast<HCP_LDS(i16x4)*>(const_cast<HCP_LDS(char)*>(p)));
}

template <int D, typename T, bool CAUSAL, bool PAGED, bool VARLEN, bool PADDED>
__global__ __attribute__((amdgpu_flat_work_group_size(kFwdThreads, kFwdThreads),
                          amdgpu_waves_per_eu(D == 256 ? 1 : HCP_FWD_WAVES_PER_EU,
                                              D == 256 ? 1 : HCP_FWD_WAVES_PER_EU))) void
fa_fwd_kernel(FwdParams p) {
  using E = Elem<T>;
  using V8 = typename E::vec8;
  constexpr int BM = kFwdBM, BN = kFwdBN;
  constexpr int ROWB = D * 2;                     // bytes per tile row
  constexpr int TILEB = BN * ROWB;                // bytes per K (or V) tile
  constexpr int NI = TILEB / (kFwdThreads * 16);  // direct loads per thread per tile
  constexpr int KSTEPS = D / 16;
  constexpr int DBLK = D / 32;
  static_assert(D == 64 || D == 128 || D == 256, "head_dim");
  // D = 256 runs one wave per SIMD (512 registers): the output accumulator
  // (128 registers) lives in AGPRs, fed by the PV product directly
  constexpr bool kAccA = D == 256;

  // Two K tiles and two V tiles.  Iteration n reads K(n+1) and V(n) while the
  // loads of K(n+2) and V(n+1) land in the other buffers.
  __shared__ __attribute__((aligned(1024))) char bufK0[TILEB];
  __shared__ __attribute__((aligned(1024))) char bufK1[TILEB];
  __shared__ __attribute__((aligned(1024))) char bufV0[TILEB];
  __shared__ __attribute__((aligned(1024))) char bufV1[TILEB];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r32 = lane & 31;
  const int g = lane >> 5;

  // ---- work item: (tile, head) ----
  int kvh;
  int64_t item;
  if (!xcd_remap(blockIdx.x, static_cast<int64_t>(p.num_tiles) * p.group,
                 p.num_kv_heads, &kvh, &item))
    return;
  const int tile = static_cast<int>(item / p.group);
  const int head = kvh * p.group + static_cast<int>(item % p.group);

  hcp_varlen_entry e;
  int qb;
  if constexpr (VARLEN) {
    const int ent = p.tiles[2 * tile];
    qb = p.tiles[2 * tile + 1];
    e = p.entries[ent];
  } else {
    e = p.single;
    qb = CAUSAL ? (p.num_tiles - 1 - tile) : tile;  // heaviest first
  }
  // Sliding window (causal only): row i sees keys (off + i - window, off + i].
  // The workgroup's first row has the lowest bound, so the segment is rebased
  // to it: keys below are never loaded, and rows whose bound is higher mask
  // the boundary tiles.
  const int64_t win = CAUSAL ? p.window : 0;
  if (win > 0) {
    int64_t lo = e.causal_offset + static_cast<int64_t>(qb) * BM - win + 1;
    if (lo > 0) {
      if (lo > e.kv.len) lo = e.kv.len;
      e.kv.start += lo;
      e.kv.len -= lo;
      e.causal_offset -= lo;
    }
  }
  // Paged segments are tiled from a 16-key boundary of the request's block
  // frame: a wave's 16 rows of a tile then start on a multiple of 16 and,
  // with block_size >= 16, lie in one block.  The `lead` (< 16) keys in front
  // of the segment load as zeros and are masked for every row; a segment
  // that starts on a block boundary has none.
  int lead = 0;
  if constexpr (PAGED) {
    lead = static_cast<int>(e.kv.start & (kFwdPagedMinBlock - 1));
    e.kv.start -= lead;
    e.kv.len += lead;
    e.causal_offset += lead;
  }
  const int64_t q_len = e.q_len;
  const int kv_len = static_cast<int>(e.kv.len);
  const int64_t off = e.causal_offset;

  // ---- Q^T fragments (B operand): lane owns query row r32 ----
  // A row holds dv <= D valid elements (a multiple of 8; PADDED: fewer than
  // D); the kernel computes in D columns whose tail is zero in Q, K and V
  // and is never stored.
  const int dv = PADDED ? p.head_dim : D;
  const int rowv = dv * 2;  // valid bytes of a row
  const int64_t qi = static_cast<int64_t>(qb) * BM + wave * 32 + r32;
  const bool q_valid = qi < q_len;
  V8 qf[KSTEPS];
  {
    const char* qrow = reinterpret_cast<const char*>(p.q) +
                       ((e.q_start + (q_valid ? qi : 0)) * p.q_stride_tok +
                        static_cast<int64_t>(head) * p.q_stride_head) * 2;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      u32x4 x = q_valid && 16 * s + 8 * g < dv ? ldg16(qrow + (16 * s + 8 * g) * 2)
                                               : u32x4{0, 0, 0, 0};
      qf[s] = as_vec8<V8>(x);
    }
  }

  // ---- key range of the workgroup and of this wave ----
  int64_t n_end = kv_len;
  if (CAUSAL) {
    const int64_t lim = off + static_cast<int64_t>(qb) * BM + BM;
    n_end = n_end < lim ? n_end : lim;
  }
  if (n_end < 0) n_end = 0;
  const int ntiles = static_cast<int>((n_end + BN - 1) / BN);
  const int64_t wave_q0 = static_cast<int64_t>(qb) * BM + wave * 32;
  // tiles this wave computes: all of the workgroup's tiles up to its diagonal;
  // a wave without valid query rows computes none (it still loads and syncs)
  int wtiles = ntiles;
  if (wave_q0 >= q_len) {
    wtiles = 0;
  } else if (CAUSAL) {
    const int64_t wave_last = off + wave_q0 + 31;
    const int64_t wt = wave_last < 0 ? 0 : wave_last / BN + 1;
    wtiles = wt < ntiles ? static_cast<int>(wt) : ntiles;
  }

  // ---- direct tile loads: lane's row / chunk for load instruction i ----
  // instruction i of wave w fills LDS bytes [(w*NI+i)*1024, +1024) of a tile
  // Load instruction i of wave w fills LDS bytes [(w*NI+i)*1024, +1024) of a
  // tile: lane l covers tile row lrow0 + i*RPI, 16-byte chunk lchunk(i).
  // Rows and chunks are recomputed where needed (cheap) instead of being
  // kept in registers for the whole kernel.
  constexpr int RPI = 1024 / ROWB;  // tile rows per load instruction
  const int lrow0 = wave * NI * RPI + (lane * 16) / ROWB;
  auto lrow = [&](int i) __attribute__((always_inline)) { return lrow0 + i * RPI; };
  auto lchunk = [&](int i) __attribute__((always_inline)) {
    return (((lane * 16) % ROWB) / 16) ^ tile_swz<D>(lrow(i));
  };
  const int64_t rowb_g = e.kv.stride_tok * 2;  // bytes between tokens in HBM
  const uint32_t rowb32 = static_cast<uint32_t>(rowb_g);
  const uint32_t tileb32 = static_cast<uint32_t>(BN) * rowb32;  // bytes of a tile's rows
  const char* kseg;
  const char* vseg;
  int bs_shift = 0, bs_mask = 0;
  const int32_t* bt = reinterpret_cast<const int32_t*>(e.kv.block_table);
  int64_t blockb = 0;
  if constexpr (PAGED) {
    kseg = reinterpret_cast<const char*>(e.kv.k_addr) + static_cast<int64_t>(kvh) * e.kv.stride_head * 2;
    vseg = reinterpret_cast<const char*>(e.kv.v_addr) + static_cast<int64_t>(kvh) * e.kv.stride_head * 2;
    bs_shift = 31 - __builtin_clz(e.kv.block_size);
    bs_mask = e.kv.block_size - 1;
    blockb = e.kv.stride_block * 2;
  } else {
    const int64_t base = (e.kv.start * e.kv.stride_tok + static_cast<int64_t>(kvh) * e.kv.stride_head) * 2;
    kseg = reinterpret_cast<const char*>(e.kv.k_addr) + base;
    vseg = reinterpret_cast<const char*>(e.kv.v_addr) + base;
  }
  const uint32_t blockb32 = static_cast<uint32_t>(blockb);  // under 4 GiB (checked on the host)

  // Per-lane 32-bit byte offsets (loop invariant) under a wave-uniform
  // descriptor, the SGPR-base + VGPR-offset form of buffer_load ... lds:
  // contiguous segments rebase a descriptor per tile and offset by the tile
  // row; paged ones rebase it per tile at the wave's first row -- its WROWS
  // rows lie in one block -- and offset by the row inside the wave's share.
  constexpr int WROWS = NI * RPI;  // tile rows each wave loads
  static_assert(!PAGED || WROWS <= kFwdPagedMinBlock, "a wave's rows must fit one block");
  // A chunk past the row's dv elements gets an offset past any num_records:
  // it reads as zeros.
  constexpr uint32_t kOob = 0x80000000u;
  uint32_t goff[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i)
    goff[i] = lchunk(i) * 8 < dv
                  ? static_cast<uint32_t>(PAGED ? lrow(i) - wave * WROWS : lrow(i)) * rowb32 +
                        lchunk(i) * 16u
                  : kOob;

  // paged: block ids of the wave's rows, a window of 64 tiles per VGPR (lane
  // l holds the id of tile base + l, clamped to the last tile and to the
  // segment's last key, so the block-table read stays in the request's row;
  // an id past the cache is clamped to its last block).  One vector load per
  // 64 tiles, issued a window ahead; a tile's id is then a v_readlane into an
  // SGPR, with no memory access in the tile loop.
  auto load_ids = [&](int t0) __attribute__((always_inline)) {
    uint32_t id = 0;
    if constexpr (PAGED) {
      int t = t0 + lane_id_fresh();
      t = t < ntiles ? t : ntiles - 1;
      int key = t * BN + wave * WROWS;
      key = key < kv_len ? key : kv_len - 1;
      const int idx = static_cast<int>((e.kv.start + key) >> bs_shift);
      id = static_cast<uint32_t>(bt[idx]);
      if (e.kv.num_blocks > 0 && id >= static_cast<uint32_t>(e.kv.num_blocks))
        id = static_cast<uint32_t>(e.kv.num_blocks - 1);
    }
    return id;
  };
  uint32_t ids_cur = 0, ids_nxt = 0;  // windows [id_base, +64) and [id_base + 64, +64)
  int id_base = 0;
  auto tile_id = [&](int t) __attribute__((always_inline)) {
    t = t < ntiles ? t : ntiles - 1;
    const int rel = t - id_base;  // 0 .. 127
    const uint32_t a = __builtin_amdgcn_readlane(ids_cur, rel & 63);
    const uint32_t b = __builtin_amdgcn_readlane(ids_nxt, rel & 63);
    return rel < 64 ? a : b;
  };
  // paged: descriptor of the wave's rows of tile t (clamped to the last
  // tile), based at its first row; num_records ends at the segment's last key
  // and at the block's end, so nothing past either is read (those rows read
  // as zeros: unused cache slots may hold NaNs).  The rows start on a
  // multiple of 16 of the block frame (the segment start is aligned down to
  // 16 keys), so with block_size >= 16 all WROWS = 16 of them lie in the block.
  // (32-bit offsets: a block spans under 4 GiB -- hcp_plan_varlen_tiles
  // checks it -- so only the final address add is 64-bit, and the bounds are
  // selects, not branches)
  auto page_rsrc = [&](const char* seg, uint32_t id, int t) __attribute__((always_inline)) {
    t = t < ntiles ? t : ntiles - 1;
    const int r0 = t * BN + wave * WROWS;
    const int in_blk = (static_cast<int>(e.kv.start) + r0) & bs_mask;
    int rows = kv_len - r0;
    rows = rows < WROWS ? rows : WROWS;
    rows = rows < e.kv.block_size - in_blk ? rows : e.kv.block_size - in_blk;
    const uint32_t nrec = rows > 0 ? static_cast<uint32_t>(rows - 1) * rowb32 + rowv : 0u;
    const uint64_t off = static_cast<uint64_t>(id) * blockb32 +
                         static_cast<uint32_t>(in_blk) * rowb32;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(seg + off), 0,
                                             static_cast<int>(nrec), kBufferRsrcWord3);
  };

  // Contiguous prologue loads of one tile of K or V.  Ragged tiles clamp
  // their key rows into the segment (those rows are masked in S, and their
  // finite V values meet P = 0), so no load leaves the segment.
  auto issue = [&](const char* seg, int tile_idx, HCP_LDS(char)* dst) __attribute__((always_inline)) {
    const int n0 = tile_idx * BN;
    const bool ragged = n0 + BN > kv_len;
    // MUBUF form (buffer_load ... lds) over a descriptor rebased per tile:
    // 32-bit offsets never overflow, and unlike the FLAT-encoded
    // global_load_lds it leaves the compiler exact LDS-read wait counts
    const char* base = seg + static_cast<int64_t>(n0) * rowb_g;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(base), 0, 0x7fffffff, kBufferRsrcWord3);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      uint32_t o = goff[i];
      if (ragged && o != kOob) {
        const int key = n0 + lrow(i);
        const int kc = key < kv_len ? key : kv_len - 1;
        o = static_cast<uint32_t>(kc - n0) * rowb32 + lchunk(i) * 16u;
      }
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs, reinterpret_cast<HCP_LDS(void)*>(dst + (wave * NI + i) * 1024), 16,
          static_cast<int>(o), 0, 0, 0);
    }
  };

  // Contiguous segments: a buffer descriptor per (clamped) tile.  Tile
  // indices past the last tile are clamped to it (such loads fill a buffer
  // nobody reads); a ragged last tile gets num_records = its valid bytes, so
  // rows past the segment read as zeros (they are masked in S, and zero V
  // rows meet P = 0) with no per-lane clamping.
  // (a tile's rows span under 2^31 bytes: the token stride is below 2^24
  // elements, checked on the host)
  auto tile_rsrc = [&](const char* seg, int tile_idx) __attribute__((always_inline)) {
    const int t = tile_idx < ntiles ? tile_idx : ntiles - 1;
    const int rows = kv_len - t * BN;
    const uint32_t nrec =
        rows >= BN ? 0x7fffffffu : static_cast<uint32_t>(rows - 1) * rowb32 + rowv;
    return __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(seg + static_cast<uint64_t>(static_cast<uint32_t>(t)) * tileb32), 0,
        static_cast<int>(nrec), kBufferRsrcWord3);
  };
  auto load_at = [&](__amdgpu_buffer_rsrc_t rs, uint32_t o, int i, HCP_LDS(char)* dst)
      __attribute__((always_inline)) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rs, reinterpret_cast<HCP_LDS(void)*>(dst + (wave * NI + i) * 1024), 16,
        static_cast<int>(o), 0, 0, 0);
  };
  auto load_one = [&](__amdgpu_buffer_rsrc_t rs, int i, HCP_LDS(char)* dst)
      __attribute__((always_inline)) { load_at(rs, goff[i], i, dst); };
  // phase A issues one K or V load instruction every kLoadEvery/2 MFMAs
  constexpr int kLoadEvery = 4;

  // ---- LDS read addresses (loop invariant, per lane) ----
  // The swizzle permutes the 16 slots of each 256-byte group of a row only,
  // so a slot 16 or more is the offset of slot - 16 plus 256 bytes: eight K
  // and four V offsets per half cover any D (D = 256 rows have 32 slots).
  // K (A operand of S^T): row 32*blk + r32, 16-byte chunk 2s+g
  // (row + 32 has the same swizzle, so block 1 is an immediate offset)
  // D = 256 non-causal (one wave per SIMD, every register in use): each
  // offset is the first one XOR a constant, formed where it is used -- the
  // row's slot bits (4..8) are disjoint from the row's own offset, so
  // offset(s) = offset(0) ^ 32 s for K and offset(db) = offset(0) ^ 64 db for
  // V -- by an opaque XOR the compiler cannot hoist into a loop-long register.
  // The causal kernels keep the offsets in registers (they fit without
  // spilling there, and the extra XOR per LDS read costs 3% of the step).
  constexpr bool kXorOfs = D == 256 && !CAUSAL;
  auto xor_ofs = [&](int base, int c) __attribute__((always_inline)) {
    if (c == 0) return base;
    int r;
    asm volatile("v_xor_b32 %0, %2, %1" : "=v"(r) : "v"(base), "n"(c));
    return r;
  };
  constexpr int KO = kXorOfs ? 1 : (KSTEPS < 8 ? KSTEPS : 8);
  const int kx = tile_swz<D>(r32);
  int koff[KO];
#pragma unroll
  for (int s = 0; s < KO; ++s) koff[s] = r32 * ROWB + (((2 * s + g) ^ kx) * 16);
  auto kofs = [&](int s) __attribute__((always_inline)) {
    if constexpr (kXorOfs) return xor_ofs(koff[0], 32 * s);
    return koff[s % KO] + 256 * (s / KO);
  };
  // V (transposing read): block beta = lane/16, i = lane%16 = 4*ee + aa reads
  // key 16t + 8h + 4*vg + ee, columns dblk*32 + 16*(beta&1) + 4*aa .. +3; the
  // swizzle of that key does not depend on t, so t is an immediate offset
  const int beta = lane >> 4, ee = (lane & 15) >> 2, aa = lane & 3;
  const int vg = beta >> 1;
  const int vs0 = 2 * (beta & 1) + (aa >> 1);
  constexpr int VO = kXorOfs ? 1 : (DBLK < 4 ? DBLK : 4);
  int voff[VO][2];
#pragma unroll
  for (int db = 0; db < VO; ++db)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int key = 8 * h + 4 * vg + ee;
      voff[db][h] = key * ROWB + (((4 * db + vs0) ^ tile_swz<D>(key)) * 16) + (aa & 1) * 8;
    }
  auto vofs = [&](int db, int h) __attribute__((always_inline)) {
    if constexpr (kXorOfs) return xor_ofs(voff[0][h], 64 * db);
    return voff[db % VO][h] + 256 * (db / VO);
  };

  // ---- online softmax state ----
  // m_ref: exponent reference of the row (log2 units), the row max of the
  // first tile and raised only when a tile's P would exceed 2^12 against it
  // (-inf until the row has seen a key).  O and l are relative to it.
  const float c = p.scale_log2;
  float m_ref = -INFINITY;
  // -m_ref for the exponent's FMA (0 while the row has seen no key), kept
  // with m_ref rather than formed again on every tile
  float m_neg = 0.f;
  float l_run = 0.f;   // sum of P in f32: the LSE
  float lr_run = 0.f;  // sum of P as rounded for the PV product: normalises O
  f32x16 oacc[DBLK];
#pragma unroll
  for (int i = 0; i < DBLK; ++i) oacc[i] = f32x16{};
  // AGPR accumulator (D = 256): 24 wait states, ordered against every read
  // and write of the accumulator (it is an operand), between the products
  // and other instructions that read or write it
  auto acc_fence = [&]() __attribute__((always_inline)) {
    if constexpr (kAccA)
      asm volatile("s_nop 7\n s_nop 7\n s_nop 7"
                   : "+a"(oacc[0]), "+a"(oacc[1]), "+a"(oacc[2]), "+a"(oacc[3]),
                     "+a"(oacc[DBLK > 4 ? 4 : 0]), "+a"(oacc[DBLK > 5 ? 5 : 0]),
                     "+a"(oacc[DBLK > 6 ? 6 : 0]), "+a"(oacc[DBLK > 7 ? 7 : 0]));
  };
  f32x16 SA[2], SB[2];  // scores of two tiles (ping-pong), 2 x 32 keys each
  V8 pf[4];             // P^T of the current tile, 16 keys per fragment

  // S^T = K Q^T of one tile (64 keys) from LDS
  auto qk = [&](const HCP_LDS(char)* Ks, f32x16 (&S)[2]) __attribute__((always_inline)) {
    S[0] = f32x16{};
    S[1] = f32x16{};
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      S[0] = E::mfma32(lds_read16<V8>(Ks + kofs(s)), qf[s], S[0]);
      S[1] = E::mfma32(lds_read16<V8>(Ks + kofs(s) + 32 * ROWB), qf[s], S[1]);
    }
  };

  // causal diagonal / ragged masking of tile n (keys n*BN ..): -inf
  // (and, with a window, tiles below some row's lower bound: the wave's last
  // row has the highest bound off + wave_q0 + 32 - window).  The bounds are
  // taken once, clamped into 32 bits around the segment's key range [0,
  // kv_len): a tile's key offsets n*BN then compare against them directly.
  auto clamp32 = [&](int64_t x) __attribute__((always_inline)) {
    const int64_t lo = -BN, hi = static_cast<int64_t>(kv_len) + BN;
    return static_cast<int>(x < lo ? lo : (x > hi ? hi : x));
  };
  // wave-uniform: a tile at n0 crosses the wave's causal diagonal when
  // n0 > diag_from, lies (partly) below its window when n0 < win_below
  const int diag_from = CAUSAL ? clamp32(off + wave_q0 - BN + 1) : 0;
  const int win_below = win > 0 ? clamp32(off + wave_q0 + 32 - win) : 0;
  auto needs_mask = [&](int n) __attribute__((always_inline)) {
    const int n0 = n * BN;
    return (n0 + BN > kv_len) || (CAUSAL && n0 > diag_from) || (win > 0 && n0 < win_below) ||
           (PAGED && n0 < lead);
  };
  // a wave-uniform bound b relative to a tile, clamped so that b + r32 (the
  // lane's row) stays exact wherever it lies in [-1, BN] and saturates
  // outside it; scalar 64-bit arithmetic, one 32-bit add per lane
  auto rel = [&](int64_t b) __attribute__((always_inline)) {
    const int64_t lo = -BN - 32, hi = BN;
    return static_cast<int>(b < lo ? lo : (b > hi ? hi : b)) + r32;
  };
  auto apply_mask = [&](f32x16 (&S)[2], int n) __attribute__((always_inline)) {
    const int n0 = n * BN;
    const int lim_r = kv_len - 1 - n0;
    // last key the lane's row sees, relative to the tile: off + qi - n0
    int lim_c = BN;
    if (CAUSAL) {
      lim_c = rel(off + wave_q0 - n0);
      lim_c = lim_c < -1 ? -1 : (lim_c > BN ? BN : lim_c);
    }
    const int lim = lim_r < lim_c ? lim_r : lim_c;
    // lowest visible key of the lane's row, relative to the tile (the window's
    // bound off + qi - window + 1, and the paged alignment lead)
    int lo = win > 0 ? rel(off + wave_q0 - win + 1 - n0) : 0;
    if (PAGED && lead - n0 > lo) lo = lead - n0;
    lo = lo < 0 ? 0 : (lo > BN ? BN : lo);
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kk = 32 * h + 8 * (r >> 2) + 4 * g + (r & 3);
        if (kk > lim || kk < lo) S[h][r] = -INFINITY;
      }
  };

  // lane's max over its 32 scores of a tile (raw, unscaled)
  auto tile_max = [&](const f32x16 (&S)[2]) __attribute__((always_inline)) {
    float a[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float a0 = __builtin_fmaxf(__builtin_fmaxf(S[h][0], S[h][1]), S[h][2]);
      float a1 = __builtin_fmaxf(__builtin_fmaxf(S[h][3], S[h][4]), S[h][5]);
      float a2 = __builtin_fmaxf(__builtin_fmaxf(S[h][6], S[h][7]), S[h][8]);
      float a3 = __builtin_fmaxf(__builtin_fmaxf(S[h][9], S[h][10]), S[h][11]);
      float a4 = __builtin_fmaxf(__builtin_fmaxf(S[h][12], S[h][13]), S[h][14]);
      a0 = __builtin_fmaxf(__builtin_fmaxf(a0, a1), a2);
      a3 = __builtin_fmaxf(__builtin_fmaxf(a3, a4), S[h][15]);
      a[h] = __builtin_fmaxf(a0, a3);
    }
    return __builtin_fmaxf(a[0], a[1]);
  };

  // Raise m_ref to the row max of a tile (mh: the lane's raw max; the row
  // pair (lane, lane^32) agrees on it) and rescale O and l, which hold
  // everything up to the previous tile.  Called by the whole wave.
  auto rescale_to = [&](float mh) __attribute__((always_inline)) {
    const float mrow = __builtin_fmaxf(mh, __shfl_xor(mh, 32)) * c;
    const float m_new = __builtin_fmaxf(m_ref, mrow);
    const float alpha = fast_exp2(m_ref - (m_new == -INFINITY ? 0.f : m_new));
    l_run *= alpha;
    lr_run *= alpha;
    // (AGPR accumulator: wait out the last product before the read-back,
    // and let the write-back land before the next product reads it)
    acc_fence();
#pragma unroll
    for (int i = 0; i < DBLK; ++i) oacc[i] *= alpha;
    acc_fence();
    m_ref = m_new;
    m_neg = m_new == -INFINITY ? 0.f : -m_new;
  };

  // One iteration n of the software pipeline, S_cur = scores of tile n
  // (masked, checked against m_ref), S_nxt receives tile n+1:
  //   A: S_nxt = K(n+1) Q^T            on MFMA, interleaved with
  //      P(n) = exp2(c S_cur - m_ref)  on VALU
  //      and l += rowsum P(n)          on VALU
  //   then the (rare) rescale of tile n, the masking of tile n+1, and
  //   B: O += V(n)^T P(n)^T            on MFMA.
  // Each phase is one branch-free basic block (on a wave's last tile, A
  // multiplies a stale LDS tile whose result is discarded); the group
  // barriers ask the scheduler to alternate MFMA, LDS reads and VALU so the
  // matrix pipe stays fed while the softmax runs.  The four tile buffers are
  // distinct __shared__ objects so the compiler can tell the LDS reads from
  // the global->LDS writes in flight and does not wait for the latter.
  // ---- the two phases of one pipeline iteration, in explicit order ----
  // Phase A: S_nxt = K(n+1) Q^T (2*KSTEPS MFMAs, K fragments read from LDS
  // three MFMAs ahead) while P(n) = exp2(c S_cur - m_ref) and its P^T
  // fragments are formed, EA scores per MFMA.
  // V^T fragment j (16 keys x 32 head-dim columns) of tile Vs, transposing reads
  constexpr int VR = HCP_VPF + 1;  // V fragment ring
  auto vread_at = [&](const HCP_LDS(char)* Vs, int j) __attribute__((always_inline)) {
    const int t = j / DBLK, db = j % DBLK;
    const i16x4 lo = lds_read_tr(Vs + vofs(db, 0) + (16 * t) * ROWB);
    const i16x4 hi = lds_read_tr(Vs + vofs(db, 1) + (16 * t) * ROWB);
    u32x4 w;
    w[0] = __builtin_bit_cast(u32x2, lo)[0];
    w[1] = __builtin_bit_cast(u32x2, lo)[1];
    w[2] = __builtin_bit_cast(u32x2, hi)[0];
    w[3] = __builtin_bit_cast(u32x2, hi)[1];
    return w;
  };

  // P for score pair `pair` (scores 2*pair, 2*pair+1 of the lane's 32):
  // exp2(c S - m) packed into its P^T fragment (S is kept) and added to the
  // lane's tile sums (two chains)
  auto exp_pair = [&](int pair, const f32x16 (&Sc)[2], float (&ts)[4])
      __attribute__((always_inline)) {
    const int x = 2 * pair;  // 0..31, even
    const int h = x >> 4, r = x & 15;
    const float p0 = fast_exp2(__builtin_fmaf(Sc[h][r], c, m_neg));
    const float p1 = fast_exp2(__builtin_fmaf(Sc[h][r + 1], c, m_neg));
    // P^T fragment 2h + (r >> 3) holds regs 8t .. 8t+7 of half h
    u32x4 w = __builtin_bit_cast(u32x4, pf[2 * h + (r >> 3)]);
    const uint32_t pw = pack2<T>(p0, p1);
    w[(r & 7) >> 1] = pw;
    pf[2 * h + (r >> 3)] = as_vec8<V8>(w);
    // the tile's sums start at its first pairs (P >= 0: no signed zero to
    // keep, and no accumulator to clear)
    if (pair == 0) {
      ts[0] = p0;
      ts[1] = p1;
    } else {
      ts[0] += p0;
      ts[1] += p1;
    }
    ts[2 + (pair & 1)] = pair < 2 ? sum2_first<T>(pw) : sum2<T>(pw, ts[2 + (pair & 1)]);
  };
  // the rare path of a tile whose P would exceed 2^12 (or a row with no
  // reference yet): rescale to the tile's true row max, form P again
  auto redo_tile = [&](const f32x16 (&Sc)[2], float (&ts)[4]) __attribute__((always_inline)) {
    rescale_to(tile_max(Sc));
#pragma unroll
    for (int pr = 0; pr < 16; ++pr) exp_pair(pr, Sc, ts);
  };
  constexpr int NA = 2 * KSTEPS;  // MFMAs in phase A
  constexpr int EA = 32 / NA;     // scores exponentiated per phase-A MFMA
  constexpr int NB = 4 * DBLK;    // MFMAs in phase B
  auto phase_a = [&](const HCP_LDS(char)* Ks, const f32x16 (&Sc)[2], f32x16 (&Sn)[2],
                     __amdgpu_buffer_rsrc_t rs, HCP_LDS(char)* ldst,
                     __amdgpu_buffer_rsrc_t rs2, HCP_LDS(char)* ldst2, float (&ts)[4])
      __attribute__((always_inline)) {
    // Phase A carries the VALU work; at raised wave priority its instructions
    // issue ahead of the other wave on the SIMD, whose MFMAs (often its phase
    // B) keep the matrix pipe busy meanwhile.  Phase B drops it again.
    __builtin_amdgcn_s_setprio(1);
    constexpr int KR = HCP_KPF + 1;  // K fragment ring
    V8 kf[KR];
#pragma unroll
    for (int j = 0; j < HCP_KPF; ++j)
      kf[j] = lds_read16<V8>(Ks + kofs(j >> 1) + (j & 1) * 32 * ROWB);
#pragma unroll
    for (int st = 0; st < NA; ++st) {
      const int s = st >> 1, blk = st & 1;
      if (st + HCP_KPF < NA) {
        const int j = st + HCP_KPF;
        kf[j % KR] = lds_read16<V8>(Ks + kofs(j >> 1) + (j & 1) * 32 * ROWB);
      }
      Sn[blk] = E::mfma32(kf[st % KR], qf[s], s == 0 ? f32x16{} : Sn[blk]);
      // K(n+2) and V(n+1) tile loads, alternating, one every kLoadEvery/2
      // MFMAs: V's buffer was freed by the previous barrier, and a whole
      // phase B passes before this iteration's barrier waits for the loads
      constexpr int LE = kLoadEvery / 2;
      if (st % LE == 0 && st / LE < 2 * NI) {
        const int i = st / LE;
        if (i % 2 == 0)
          load_one(rs, i / 2, ldst);
        else
          load_one(rs2, i / 2, ldst2);
      }
      // scores st*EA .. st*EA+EA-1 of the current tile (D = 256: one pair
      // every second MFMA)
      if constexpr (EA >= 2) {
#pragma unroll
        for (int q = 0; q < EA; q += 2) exp_pair((st * EA + q) >> 1, Sc, ts);
      } else if (st & 1) {
        exp_pair(st >> 1, Sc, ts);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // P(n) is complete here: keep its computation in this phase (all its uses
    // are in phase B, past the masking branch, where code motion would
    // otherwise move it and serialise it behind the PV MFMAs)
#pragma unroll
    for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(pf[i]));
    asm volatile("" : "+v"(ts[0]), "+v"(ts[1]), "+v"(ts[2]), "+v"(ts[3]));
  };

  // Phase B: O += V(n)^T P(n)^T (NB MFMAs, transposing V reads two MFMAs
  // ahead).
  auto phase_b = [&](const HCP_LDS(char)* Vs) __attribute__((always_inline)) {
    u32x4 vf[VR];
    __builtin_amdgcn_s_setprio(0);
    auto vread = [&](int j) __attribute__((always_inline)) { return vread_at(Vs, j); };
#pragma unroll
    for (int j = 0; j < HCP_VPF; ++j) vf[j] = vread(j);
#pragma unroll
    for (int st = 0; st < NB; ++st) {
      const int t = st / DBLK, db = st % DBLK;
      if (st + HCP_VPF < NB) vf[(st + HCP_VPF) % VR] = vread(st + HCP_VPF);
      if constexpr (kAccA)
        E::mfma32_acc(oacc[db], as_vec8<V8>(vf[st % VR]), pf[t]);
      else
        oacc[db] = E::mfma32(as_vec8<V8>(vf[st % VR]), pf[t], oacc[db]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // One iteration n of the software pipeline (S_cur = scores of tile n,
  // masked; S_nxt receives tile n+1): phase A, then the (rare) rescale of
  // tile n, the masking of tile n+1 when it is a diagonal or ragged tile, and
  // phase B.  On a wave's last tile phase A
  // multiplies a stale LDS tile whose result is discarded.  The four tile
  // buffers are distinct __shared__ objects so the compiler can tell the LDS
  // reads from the global->LDS writes in flight and does not wait for them.
  auto iterate = [&](int n, f32x16 (&Sc)[2], f32x16 (&Sn)[2], HCP_LDS(char)* kload,
                     HCP_LDS(char)* vload, const HCP_LDS(char)* Ks,
                     const HCP_LDS(char)* Vs) __attribute__((always_inline)) {
    // loads for the next iteration: K(n+2) -> kload, V(n+1) -> vload, one
    // load instruction at a time under the MFMAs of phase A (a wave that
    // computes nothing this iteration issues them here).  Tiles past the
    // segment are clamped to its last one: they fill a buffer nobody reads.
    __amdgpu_buffer_rsrc_t rsk, rsv;
    if constexpr (PAGED) {
      if (n + 1 >= id_base + 64) {  // V's tile left the window: slide it
        id_base += 64;
        ids_cur = ids_nxt;
        ids_nxt = load_ids(id_base + 64);
      }
      rsk = page_rsrc(kseg, tile_id(n + 2), n + 2);
      rsv = page_rsrc(vseg, tile_id(n + 1), n + 1);
    } else {
      rsk = tile_rsrc(kseg, n + 2);
      rsv = tile_rsrc(vseg, n + 1);
    }
    if (n < wtiles) {
      float ts[4];  // the tile's P sums (phase A sets all four)
      phase_a(Ks, Sc, Sn, rsk, kload, rsv, vload, ts);
      if (__any(ts[0] + ts[1] > kSumThresh || m_ref == -INFINITY)) redo_tile(Sc, ts);
      l_run += ts[0] + ts[1];
      lr_run += ts[2] + ts[3];
      if (needs_mask(n + 1)) apply_mask(Sn, n + 1);
      phase_b(Vs);
    } else {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        load_one(rsk, i, kload);
        load_one(rsv, i, vload);
      }
    }
    // This iteration's tile loads land in LDS that other waves read next
    // iteration: each wave drains its own DMA, then the barrier publishes it.
    wait_vmcnt<0>();
    __syncthreads();
  };

  HCP_LDS(char)* K0 = (HCP_LDS(char)*)(bufK0);
  HCP_LDS(char)* K1 = (HCP_LDS(char)*)(bufK1);
  HCP_LDS(char)* V0 = (HCP_LDS(char)*)(bufV0);
  HCP_LDS(char)* V1 = (HCP_LDS(char)*)(bufV1);

  // ---- prologue: K(0), K(1), V(0) in flight; S(0) = K(0) Q^T ----
  if (ntiles > 0) {
    if constexpr (PAGED) {
      ids_cur = load_ids(0);
      ids_nxt = load_ids(64);
      const uint32_t id0 = tile_id(0);
      // tile 0: the alignment lead's rows read as zeros (an offset past any
      // num_records), whatever the cache holds there
      const __amdgpu_buffer_rsrc_t rk0 = page_rsrc(kseg, id0, 0), rv0 = page_rsrc(vseg, id0, 0);
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const uint32_t o = lrow(i) < lead ? kOob : goff[i];
        load_at(rk0, o, i, K0);
        load_at(rv0, o, i, V0);
      }
      if (ntiles > 1) {
        const __amdgpu_buffer_rsrc_t rk1 = page_rsrc(kseg, tile_id(1), 1);
#pragma unroll
        for (int i = 0; i < NI; ++i) load_one(rk1, i, K1);
      }
    } else {
      issue(kseg, 0, K0);
      issue(vseg, 0, V0);
      if (ntiles > 1) issue(kseg, 1, K1);
    }
  }
  wait_vmcnt<0>();  // the prologue tiles (and Q) have landed before the barrier
  __syncthreads();
  if (wtiles > 0) {
    qk(K0, SA);
    if (needs_mask(0)) apply_mask(SA, 0);
    rescale_to(tile_max(SA));
  }
  __syncthreads();  // K(0) is read by every wave before K(2) overwrites it

  // iteration n reads K(n+1), V(n) and loads K(n+2), V(n+1); buffers by parity
  int n = 0;
  for (; n + 1 < ntiles; n += 2) {
    iterate(n, SA, SB, K0, V1, K1, V0);
    iterate(n + 1, SB, SA, K1, V0, K0, V1);
  }
  if (n < ntiles) iterate(n, SA, SB, K0, V1, K1, V0);

  // ---- epilogue ----
  // (AGPR accumulator: the last products have landed before it is read)
  acc_fence();
  // (the lane-dependent values of the epilogue are rebuilt from a fresh
  // lane id rather than held across the tile loop)
  const int lane_e = lane_id_fresh();
  const int r32e = lane_e & 31, ge = lane_e >> 5;
  const int64_t qi_e = wave_q0 + r32e;
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float lr_tot = lr_run + __shfl_xor(lr_run, 32);
  // Merge path: this wave's 32 rows of the partial state are fetched whole
  // (coalesced) into the wave's share of the tile buffers, free since the
  // loop's last barrier.  Load instruction i fills bytes [i*1024, +1024) of
  // the share: lane l writes row i*RPL + l/CPR, 16-byte slot l%CPR, which
  // holds the row's chunk (l%CPR) ^ (row & (CPR-1)), so the per-lane 8-byte
  // reads below are at most two-way bank conflicted.  Rows past q_len lie
  // beyond the descriptor's range and read as zeros.
  constexpr int CPR = ROWB / 16;    // 16-byte chunks per row
  constexpr int RPL = 1024 / ROWB;  // rows per load instruction
  static_assert(kFwdThreads / 64 * 32 * ROWB <= 4 * TILEB, "acc staging");
  const int share = wave * 32 * ROWB;
  HCP_LDS(char)* const tbuf[4] = {K0, K1, V0, V1};
  HCP_LDS(char)* const abuf = tbuf[share / TILEB] + share % TILEB;
  if (p.acc_o != nullptr && wave_q0 < q_len) {
    const int64_t sb = p.acc_stride_tok * 2;
    const int rows = q_len - wave_q0 < 32 ? static_cast<int>(q_len - wave_q0) : 32;
    const char* abase = reinterpret_cast<const char*>(p.acc_o) +
                        ((e.q_start + wave_q0) * p.acc_stride_tok +
                         static_cast<int64_t>(head) * p.acc_stride_head) * 2;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(abase), 0, static_cast<int>((rows - 1) * sb) + rowv, kBufferRsrcWord3);
#pragma unroll
    for (int i = 0; i < 32 / RPL; ++i) {
      const int r = i * RPL + lane_e / CPR;
      const int lc = (lane_e % CPR) ^ (r & (CPR - 1));
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs, reinterpret_cast<HCP_LDS(void)*>(abuf + i * 1024), 16,
          lc * 8 < dv ? static_cast<int>(r * sb) + lc * 16 : static_cast<int>(kOob), 0, 0, 0);
    }
  }
  if (qi_e < q_len) {
    const float inv = lr_tot > 0.f ? 1.f / lr_tot : 0.f;
    const int64_t row = e.q_start + qi_e;
    char* orow = reinterpret_cast<char*>(p.out) +
                 (row * p.o_stride_tok + static_cast<int64_t>(head) * p.o_stride_head) * 2;
    float lse_row = l_tot > 0.f ? m_ref * kLn2 + __logf(l_tot) : -INFINITY;
    if (p.acc_o == nullptr) {
#pragma unroll
      for (int db = 0; db < DBLK; ++db) {
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const int d0 = 32 * db + 8 * a + 4 * ge;
          u32x2 w;
          w[0] = pack2<T>(oacc[db][4 * a + 0] * inv, oacc[db][4 * a + 1] * inv);
          w[1] = pack2<T>(oacc[db][4 * a + 2] * inv, oacc[db][4 * a + 3] * inv);
          if (d0 < dv) *reinterpret_cast<u32x2*>(orow + d0 * 2) = w;
        }
      }
    } else {
      // LSE merge with the partial state acc, in merge_kernel's arithmetic:
      // this pass's output enters as stored in the output dtype, a side of
      // weight 0 enters as 0 (acc is then not read), out = fma(prefix, wp,
      // suffix * ws), lse = m + log(e^{lp-m} + e^{ls-m}); an acc LSE of +inf
      // counts as -inf.  The result equals this pass followed by
      // merge_attn_states bit for bit.
      float la = p.acc_lse[static_cast<int64_t>(head) * p.acc_lse_stride_head + row];
      if (la == INFINITY) la = -INFINITY;
      const bool acc_pre = p.acc_prefix != 0;
      const float lp = acc_pre ? la : lse_row, ls = acc_pre ? lse_row : la;
      const float m = __builtin_fmaxf(lp, ls);
      float ps = 0.f, ss = 0.f;
      if (m == -INFINITY) {
        lse_row = -INFINITY;
      } else {
        const float wp = __expf(lp - m), ws = __expf(ls - m);
        const float se = wp + ws;
        ps = wp / se;
        ss = ws / se;
        lse_row = m + __logf(se);
      }
      const float w_acc = acc_pre ? ps : ss, w_own = acc_pre ? ss : ps;
      wait_vmcnt<0>();  // this wave's rows have landed in abuf
#pragma unroll
      for (int db = 0; db < DBLK; ++db) {
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const int d0 = 32 * db + 8 * a + 4 * ge;
          u32x2 own;
          own[0] = pack2<T>(oacc[db][4 * a + 0] * inv, oacc[db][4 * a + 1] * inv);
          own[1] = pack2<T>(oacc[db][4 * a + 2] * inv, oacc[db][4 * a + 3] * inv);
          if (!(w_own > 0.f)) own = u32x2{0, 0};
          const u32x2 oth =
              w_acc > 0.f ? *reinterpret_cast<const HCP_LDS(u32x2)*>(
                                abuf + r32e * ROWB + (((4 * db + a) ^ (r32e & (CPR - 1))) * 16) + 8 * ge)
                          : u32x2{0, 0};
          const u32x2 pre = acc_pre ? oth : own, suf = acc_pre ? own : oth;
          u32x2 w;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const float a0 = E::to_float(static_cast<uint16_t>(pre[h] & 0xffffu));
            const float a1 = E::to_float(static_cast<uint16_t>(pre[h] >> 16));
            const float b0 = E::to_float(static_cast<uint16_t>(suf[h] & 0xffffu));
            const float b1 = E::to_float(static_cast<uint16_t>(suf[h] >> 16));
            w[h] = pack2<T>(__builtin_fmaf(a0, ps, b0 * ss), __builtin_fmaf(a1, ps, b1 * ss));
          }
          if (d0 < dv) *reinterpret_cast<u32x2*>(orow + d0 * 2) = w;
        }
      }
    }
    if (ge == 0 && p.lse != nullptr) p.lse[static_cast<int64_t>(head) * p.lse_stride_head + row] = lse_row;
  }
}

// ---------------------------------------------------------------------------
// Host-side launch helpers (called from abi.hip)
// ---------------------------------------------------------------------------
template <int D, typename T, bool CAUSAL, bool PAGED, bool VARLEN, bool PADDED>
static hipError_t launch_fwd_t(const FwdParams& p, int64_t grid, hipStream_t st) {
  hipLaunchKernelGGL((fa_fwd_kernel<D, T, CAUSAL, PAGED, VARLEN, PADDED>),
                     dim3(static_cast<unsigned>(grid)), dim3(kFwdThreads), 0, st, p);
  return hipGetLastError();
}

template <int D, typename T, bool PADDED>
static hipError_t launch_fwd_p(const FwdParams& p, int64_t grid, bool causal,
                               bool paged, bool varlen, hipStream_t st) {
  if (varlen) {
    if (causal)
      return paged ? launch_fwd_t<D, T, true, true, true, PADDED>(p, grid, st)
                   : launch_fwd_t<D, T, true, false, true, PADDED>(p, grid, st);
    return paged ? launch_fwd_t<D, T, false, true, true, PADDED>(p, grid, st)
                 : launch_fwd_t<D, T, false, false, true, PADDED>(p, grid, st);
  }
  return causal ? launch_fwd_t<D, T, true, false, false, PADDED>(p, grid, st)
                : launch_fwd_t<D, T, false, false, false, PADDED>(p, grid, st);
}

// head_dim == D runs the unpadded instantiations (no per-column checks)
template <int D, typename T>
static hipError_t launch_fwd_d(const FwdParams& p, int64_t grid, bool causal,
                               bool paged, bool varlen, hipStream_t st) {
  return p.head_dim == D ? launch_fwd_p<D, T, false>(p, grid, causal, paged, varlen, st)
                         : launch_fwd_p<D, T, true>(p, grid, causal, paged, varlen, st);
}

hipError_t launch_fwd(const FwdParams& p, int head_dim, int dtype, bool causal,
                      bool paged, bool varlen, hipStream_t st) {
  const int64_t grid =
      xcd_grid_size(static_cast<int64_t>(p.num_tiles) * p.group, p.num_kv_heads);
  if (grid <= 0) return hipSuccess;
  if (head_dim > 128) {  // 136 .. 256: computed in 256 columns, the tail zero
    return dtype == HCP_DTYPE_BF16
               ? launch_fwd_d<256, __bf16>(p, grid, causal, paged, varlen, st)
               : launch_fwd_d<256, _Float16>(p, grid, causal, paged, varlen, st);
  }
  if (head_dim > 64) {  // 72 .. 128: computed in 128 columns, the tail zero
    return dtype == HCP_DTYPE_BF16
               ? launch_fwd_d<128, __bf16>(p, grid, causal, paged, varlen, st)
               : launch_fwd_d<128, _Float16>(p, grid, causal, paged, varlen, st);
  }
  return dtype == HCP_DTYPE_BF16
             ? launch_fwd_d<64, __bf16>(p, grid, causal, paged, varlen, st)
             : launch_fwd_d<64, _Float16>(p, grid, causal, paged, varlen, st);
}

}  // namespace hcp
