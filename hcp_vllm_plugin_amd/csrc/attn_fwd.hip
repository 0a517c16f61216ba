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
// Design (one workgroup = 4 waves = 128 query rows of one head, 32 per wave):
//  * S^T = K Q^T on v_mfma_f32_32x32x16_{bf16,f16}: K (keys x D) is the A
//    operand read from LDS, Q^T the B operand held in registers for the whole
//    kernel.  In the 32x32 accumulator layout a lane owns one column, so each
//    lane owns ONE query row and 16 of its keys per 32-key block: the row max
//    is an in-register max3 tree plus one exchange with lane ^ 32, and the
//    row sum stays a per-lane partial until the epilogue.
//  * O^T = V^T P^T on the same MFMA: P^T comes straight from the S^T
//    registers (the key order inside the k dimension is a free permutation);
//    the V^T A operand is read from a row-major V tile with the gfx950
//    transposing LDS read ds_read_b64_tr_b16: inside each 16-lane block,
//    lane 4e+a reads 4 consecutive d of key kbase+e and every lane receives 4
//    keys of one d column.
//  * K and V tiles (64 keys x D, row-major, 16-byte slots XOR-swizzled by
//    2*(row&3) | (row>>2 & 1) so both the K reads and the transposing V reads
//    are bank-conflict free) are filled by global_load_lds_dwordx4: HBM/L2 ->
//    LDS with no register staging and no VALU work.  Two tile buffers are
//    separate __shared__ objects and the key loop is unrolled by two, so the
//    loads for tile n+1 stay in flight while tile n is computed (one barrier
//    per tile).
//  * Lazy rescale: the running max used as the exponent reference is only
//    raised when some row's tile max exceeds it by more than 2^8; otherwise P
//    values are bounded by 256 and the O rescale (64 multiplies per lane) is
//    skipped.  The result is exact: O, l and lse all use the same reference.
//  * Causal tiles above a wave's diagonal are skipped; masking runs only on
//    diagonal and ragged tiles.  Ragged tiles clamp key rows into the segment
//    (the clamped rows are masked in S, and their finite V values meet P = 0),
//    so no load goes out of bounds and no load is predicated.
//  * The local (paged) segment is read in place through the block table
//    (hcp_kv_segment), replacing the per-request gather copy of
//    ring_backend.py:617-624; block ids are fetched two tiles ahead.
#include "params.h"

namespace hcp {

#ifndef HCP_MFMA_PRIO
#define HCP_MFMA_PRIO 3
#endif

constexpr float kRescaleThresh = 8.0f;  // log2 units: P <= 2^8 between rescales

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
  if constexpr (D == 128) return 4 * (row & 3) + ((row >> 2) & 3);
  return 4 * ((row >> 1) & 1) + ((row >> 2) & 3);
}

__device__ __forceinline__ void lds_load16(const char* g, HCP_LDS(char)* l) {
  __builtin_amdgcn_global_load_lds(
      reinterpret_cast<const __attribute__((address_space(1))) void*>(reinterpret_cast<uintptr_t>(g)),
      reinterpret_cast<HCP_LDS(void)*>(l), 16, 0, 0);
}

template <typename V8>
__device__ __forceinline__ V8 lds_read16(const HCP_LDS(char)* p) {
  return __builtin_bit_cast(V8, *reinterpret_cast<const HCP_LDS(u32x4)*>(p));
}

__device__ __forceinline__ i16x4 lds_read_tr(const HCP_LDS(char)* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      reinterpret_cast<HCP_LDS(i16x4)*>(const_cast<HCP_LDS(char)*>(p)));
}

template <int D, typename T, bool CAUSAL, bool PAGED, bool VARLEN>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256),
                          amdgpu_waves_per_eu(2, 2))) void
fa_fwd_kernel(FwdParams p) {
  using E = Elem<T>;
  using V8 = typename E::vec8;
  constexpr int BM = kFwdBM, BN = kFwdBN;
  constexpr int ROWB = D * 2;                  // bytes per tile row
  constexpr int TILEB = BN * ROWB;             // bytes per K (or V) tile
  constexpr int NI = TILEB / (kFwdThreads * 16);  // direct loads per thread per tile
  constexpr int KSTEPS = D / 16;
  constexpr int DBLK = D / 32;
  static_assert(D == 64 || D == 128, "head_dim");

  __shared__ __attribute__((aligned(1024))) char bufA[2 * TILEB];  // K | V
  __shared__ __attribute__((aligned(1024))) char bufB[2 * TILEB];

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
  const int64_t q_len = e.q_len;
  const int kv_len = static_cast<int>(e.kv.len);
  const int64_t off = e.causal_offset;

  // ---- Q^T fragments (B operand): lane owns query row r32 ----
  const int64_t qi = static_cast<int64_t>(qb) * BM + wave * 32 + r32;
  const bool q_valid = qi < q_len;
  V8 qf[KSTEPS];
  {
    const char* qrow = reinterpret_cast<const char*>(p.q) +
                       ((e.q_start + (q_valid ? qi : 0)) * p.q_stride_tok +
                        static_cast<int64_t>(head) * p.q_stride_head) * 2;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      u32x4 x = q_valid ? ldg16(qrow + (16 * s + 8 * g) * 2) : u32x4{0, 0, 0, 0};
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
  const int64_t wave_last = CAUSAL ? off + wave_q0 + 31 : static_cast<int64_t>(kv_len) - 1;

  // ---- direct tile loads: lane's row / chunk for load instruction i ----
  // instruction i of wave w fills LDS bytes [(w*NI+i)*1024, +1024)
  int lrow[NI];
  int lchunk[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int o = (wave * NI + i) * 1024 + lane * 16;
    lrow[i] = o / ROWB;
    lchunk[i] = ((o % ROWB) / 16) ^ tile_swz<D>(lrow[i]);
  }
  const int64_t rowb_g = e.kv.stride_tok * 2;  // bytes between tokens in HBM
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
  // paged: block ids of the lane's rows for the next tile to be issued
  int bnext[NI];

  auto fetch_blocks = [&](int tile_idx) __attribute__((always_inline)) {
    if constexpr (PAGED) {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        int key = tile_idx * BN + lrow[i];
        key = key < kv_len ? key : kv_len - 1;
        bnext[i] = bt[(e.kv.start + key) >> bs_shift];
      }
    }
  };

  // contiguous: per-lane 32-bit byte offsets inside a tile (loop invariant);
  // the tile base is wave-uniform, so loads use the SGPR-base + VGPR-offset form
  const uint32_t rowb32 = static_cast<uint32_t>(rowb_g);
  uint32_t goff[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) goff[i] = lrow[i] * rowb32 + lchunk[i] * 16u;

  auto issue_tile = [&](int tile_idx, HCP_LDS(char)* dst) __attribute__((always_inline)) {
    const int n0 = tile_idx * BN;
    const bool ragged = n0 + BN > kv_len;
    if constexpr (PAGED) {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        int key = n0 + lrow[i];
        if (ragged) key = key < kv_len ? key : kv_len - 1;
        const int64_t x = e.kv.start + key;
        const int64_t go =
            static_cast<int64_t>(bnext[i]) * blockb + (x & bs_mask) * rowb_g + lchunk[i] * 16;
        HCP_LDS(char)* l = dst + (wave * NI + i) * 1024;
        lds_load16(kseg + go, l);
        lds_load16(vseg + go, l + TILEB);
      }
    } else {
      const char* kt = kseg + static_cast<int64_t>(n0) * rowb_g;
      const char* vt = vseg + static_cast<int64_t>(n0) * rowb_g;
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        uint32_t o = goff[i];
        if (ragged) {
          const int key = n0 + lrow[i];
          const int kc = key < kv_len ? key : kv_len - 1;
          o = static_cast<uint32_t>(kc - n0) * rowb32 + lchunk[i] * 16u;
        }
        HCP_LDS(char)* l = dst + (wave * NI + i) * 1024;
        lds_load16(kt + o, l);
        lds_load16(vt + o, l + TILEB);
      }
    }
  };

  // ---- LDS read addresses (loop invariant, per lane) ----
  // K (A operand of S^T): row 32*blk + r32, 16-byte chunk 2s+g
  // (row + 32 has the same swizzle, so block 1 is an immediate offset)
  const int kx = tile_swz<D>(r32);
  int koff[KSTEPS];
#pragma unroll
  for (int s = 0; s < KSTEPS; ++s) koff[s] = r32 * ROWB + (((2 * s + g) ^ kx) * 16);
  // V (transposing read): block beta = lane/16, i = lane%16 = 4*ee + aa reads
  // key 16t + 8h + 4*vg + ee, columns dblk*32 + 16*(beta&1) + 4*aa .. +3; the
  // swizzle of that key does not depend on t, so t is an immediate offset
  const int beta = lane >> 4, ee = (lane & 15) >> 2, aa = lane & 3;
  const int vg = beta >> 1;
  const int vs0 = 2 * (beta & 1) + (aa >> 1);
  int voff[DBLK][2];
#pragma unroll
  for (int db = 0; db < DBLK; ++db)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int key = 8 * h + 4 * vg + ee;
      voff[db][h] = key * ROWB + (((4 * db + vs0) ^ tile_swz<D>(key)) * 16) + (aa & 1) * 8;
    }

  // ---- online softmax state ----
  const float c = p.scale_log2;
  float m_ref = -INFINITY;
  float l_run = 0.f;
  f32x16 oacc[DBLK];
#pragma unroll
  for (int i = 0; i < DBLK; ++i) oacc[i] = f32x16{};

  // One 32-key half of a tile: mask, lazy-rescale check, exp, P^T fragments.
  // The check needs only this lane's values and a wave vote; the row pair's
  // exact max (lane ^ 32) is formed only on the rare rescale path.
  auto softmax_half = [&](f32x16& sh, int n0, int half, V8* pf) __attribute__((always_inline)) {
    const bool ragged = n0 + BN > kv_len;
    const bool diag = CAUSAL && (n0 + BN - 1 > off + wave_q0);
    if (ragged || diag) {
      const int lim_r = kv_len - 1 - n0;
      const int64_t lim_c64 = CAUSAL ? off + qi - n0 : static_cast<int64_t>(BN);
      const int lim_c = lim_c64 < BN ? static_cast<int>(lim_c64 < -1 ? -1 : lim_c64) : BN;
      const int lim = (lim_r < lim_c ? lim_r : lim_c) - 32 * half;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kk = 8 * (r >> 2) + 4 * g + (r & 3);
        if (kk > lim) sh[r] = -INFINITY;
      }
    }
    float a0 = __builtin_fmaxf(__builtin_fmaxf(sh[0], sh[1]), sh[2]);
    float a1 = __builtin_fmaxf(__builtin_fmaxf(sh[3], sh[4]), sh[5]);
    float a2 = __builtin_fmaxf(__builtin_fmaxf(sh[6], sh[7]), sh[8]);
    float a3 = __builtin_fmaxf(__builtin_fmaxf(sh[9], sh[10]), sh[11]);
    float a4 = __builtin_fmaxf(__builtin_fmaxf(sh[12], sh[13]), sh[14]);
    a0 = __builtin_fmaxf(__builtin_fmaxf(a0, a1), a2);
    a3 = __builtin_fmaxf(__builtin_fmaxf(a3, a4), sh[15]);
    const float mh = __builtin_fmaxf(a0, a3);
    if (__any(mh * c > m_ref + kRescaleThresh)) {
      const float mrow = __builtin_fmaxf(mh, __shfl_xor(mh, 32)) * c;
      const float m_new = __builtin_fmaxf(m_ref, mrow);
      const float alpha = fast_exp2(m_ref - (m_new == -INFINITY ? 0.f : m_new));
      l_run *= alpha;
#pragma unroll
      for (int i = 0; i < DBLK; ++i) oacc[i] *= alpha;
      m_ref = m_new;
    }
    const float m_use = (m_ref == -INFINITY) ? 0.f : m_ref;
#pragma unroll
    for (int r = 0; r < 16; ++r) sh[r] = fast_exp2(__builtin_fmaf(sh[r], c, -m_use));
    float rs = 0.f;
#pragma unroll
    for (int r = 0; r < 16; r += 4) rs += (sh[r] + sh[r + 1]) + (sh[r + 2] + sh[r + 3]);
    l_run += rs;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int b = 8 * t;
      u32x4 w;
      w[0] = pack2<T>(sh[b + 0], sh[b + 1]);
      w[1] = pack2<T>(sh[b + 2], sh[b + 3]);
      w[2] = pack2<T>(sh[b + 4], sh[b + 5]);
      w[3] = pack2<T>(sh[b + 6], sh[b + 7]);
      pf[t] = as_vec8<V8>(w);
    }
  };

  // O^T += V^T P^T for PV steps t (16 keys each) of one half
  auto pv_half = [&](const HCP_LDS(char)* Vs, int half, const V8* pf) __attribute__((always_inline)) {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int t = 2 * half + tt;
#pragma unroll
      for (int db = 0; db < DBLK; ++db) {
        const i16x4 lo = lds_read_tr(Vs + voff[db][0] + (16 * t) * ROWB);
        const i16x4 hi = lds_read_tr(Vs + voff[db][1] + (16 * t) * ROWB);
        u32x4 w;
        w[0] = __builtin_bit_cast(u32x2, lo)[0];
        w[1] = __builtin_bit_cast(u32x2, lo)[1];
        w[2] = __builtin_bit_cast(u32x2, hi)[0];
        w[3] = __builtin_bit_cast(u32x2, hi)[1];
        oacc[db] = E::mfma32(as_vec8<V8>(w), pf[tt], oacc[db]);
      }
    }
  };

  auto qk_block = [&](const HCP_LDS(char)* Ks, int blk) __attribute__((always_inline)) {
    f32x16 sb = f32x16{};
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s)
      sb = E::mfma32(lds_read16<V8>(Ks + koff[s] + blk * 32 * ROWB), qf[s], sb);
    return sb;
  };

  // One tile: QK of both 32-key blocks, then per half softmax and PV.  The
  // wave raises its issue priority while it feeds the matrix pipe, so the
  // other wave on the SIMD fills the gaps with its softmax VALU work.
  auto tile_step = [&](const HCP_LDS(char)* Ks, int n0) __attribute__((always_inline)) {
    if (CAUSAL && n0 > wave_last) return;  // whole tile above this wave's diagonal
    const HCP_LDS(char)* Vs = Ks + TILEB;
    __builtin_amdgcn_s_setprio(HCP_MFMA_PRIO);
    f32x16 s0 = qk_block(Ks, 0);
    f32x16 s1 = qk_block(Ks, 1);
    __builtin_amdgcn_s_setprio(0);
    V8 pf0[2], pf1[2];
    softmax_half(s0, n0, 0, pf0);
    __builtin_amdgcn_s_setprio(HCP_MFMA_PRIO);
    pv_half(Vs, 0, pf0);
    __builtin_amdgcn_s_setprio(0);
    softmax_half(s1, n0, 1, pf1);
    __builtin_amdgcn_s_setprio(HCP_MFMA_PRIO);
    pv_half(Vs, 1, pf1);
    __builtin_amdgcn_s_setprio(0);
  };

  HCP_LDS(char)* A = (HCP_LDS(char)*)(bufA);
  HCP_LDS(char)* B = (HCP_LDS(char)*)(bufB);

  if (ntiles > 0) {
    fetch_blocks(0);
    issue_tile(0, A);
    if (ntiles > 1) fetch_blocks(1);
  }
  __syncthreads();
  for (int it = 0; it < ntiles; it += 2) {
    if (it + 1 < ntiles) {
      issue_tile(it + 1, B);
      if (it + 2 < ntiles) fetch_blocks(it + 2);
    }
    tile_step(A, it * BN);
    __syncthreads();
    if (it + 1 >= ntiles) break;
    if (it + 2 < ntiles) {
      issue_tile(it + 2, A);
      if (it + 3 < ntiles) fetch_blocks(it + 3);
    }
    tile_step(B, (it + 1) * BN);
    __syncthreads();
  }

  // ---- epilogue ----
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  if (q_valid) {
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    const int64_t row = e.q_start + qi;
    char* orow = reinterpret_cast<char*>(p.out) +
                 (row * p.o_stride_tok + static_cast<int64_t>(head) * p.o_stride_head) * 2;
#pragma unroll
    for (int db = 0; db < DBLK; ++db) {
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int d0 = 32 * db + 8 * a + 4 * g;
        u32x2 w;
        w[0] = pack2<T>(oacc[db][4 * a + 0] * inv, oacc[db][4 * a + 1] * inv);
        w[1] = pack2<T>(oacc[db][4 * a + 2] * inv, oacc[db][4 * a + 3] * inv);
        *reinterpret_cast<u32x2*>(orow + d0 * 2) = w;
      }
    }
    if (g == 0) {
      p.lse[static_cast<int64_t>(head) * p.lse_stride_head + row] =
          l_tot > 0.f ? m_ref * kLn2 + __logf(l_tot) : -INFINITY;
    }
  }
}

// ---------------------------------------------------------------------------
// Host-side launch helpers (called from abi.hip)
// ---------------------------------------------------------------------------
template <int D, typename T, bool CAUSAL, bool PAGED, bool VARLEN>
static hipError_t launch_fwd_t(const FwdParams& p, int64_t grid, hipStream_t st) {
  hipLaunchKernelGGL((fa_fwd_kernel<D, T, CAUSAL, PAGED, VARLEN>),
                     dim3(static_cast<unsigned>(grid)), dim3(kFwdThreads), 0, st, p);
  return hipGetLastError();
}

template <int D, typename T>
static hipError_t launch_fwd_d(const FwdParams& p, int64_t grid, bool causal,
                               bool paged, bool varlen, hipStream_t st) {
  if (varlen) {
    if (causal)
      return paged ? launch_fwd_t<D, T, true, true, true>(p, grid, st)
                   : launch_fwd_t<D, T, true, false, true>(p, grid, st);
    return paged ? launch_fwd_t<D, T, false, true, true>(p, grid, st)
                 : launch_fwd_t<D, T, false, false, true>(p, grid, st);
  }
  return causal ? launch_fwd_t<D, T, true, false, false>(p, grid, st)
                : launch_fwd_t<D, T, false, false, false>(p, grid, st);
}

hipError_t launch_fwd(const FwdParams& p, int head_dim, int dtype, bool causal,
                      bool paged, bool varlen, hipStream_t st) {
  const int64_t grid =
      xcd_grid_size(static_cast<int64_t>(p.num_tiles) * p.group, p.num_kv_heads);
  if (grid <= 0) return hipSuccess;
  if (head_dim == 128) {
    return dtype == HCP_DTYPE_BF16
               ? launch_fwd_d<128, __bf16>(p, grid, causal, paged, varlen, st)
               : launch_fwd_d<128, _Float16>(p, grid, causal, paged, varlen, st);
  }
  return dtype == HCP_DTYPE_BF16
             ? launch_fwd_d<64, __bf16>(p, grid, causal, paged, varlen, st)
             : launch_fwd_d<64, _Float16>(p, grid, causal, paged, varlen, st);
}

}  // namespace hcp
