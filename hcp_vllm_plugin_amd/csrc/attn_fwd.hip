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
//    is an in-register max plus one exchange with lane ^ 32, and the row sum
//    stays a per-lane partial until the epilogue.
//  * O^T = V^T P^T on the same MFMA: P^T comes straight from the S^T
//    registers (the key order inside the k dimension is a free permutation,
//    matched by the layout V^T is stored in), V^T is the A operand from LDS.
//  * K (64 keys x D) and V^T (D x 64 keys) tiles are double-buffered in LDS:
//    the global loads of tile n+1 are issued before the MFMAs of tile n and
//    written to the other buffer after them; one barrier per tile.  V is
//    transposed on its way into LDS (each thread owns a 4-d x 8-key or
//    4-d x 4-key sub-block).  Both tiles use an XOR swizzle of 16-byte slots
//    so the MFMA operand reads and the tile writes are bank-conflict free.
//  * Causal tiles above the diagonal of a wave are skipped; masking is only
//    applied on diagonal and ragged tiles.
//  * The local (paged) segment is read in place through the block table
//    (hcp_kv_segment), replacing the per-request gather copy of
//    ring_backend.py:617-624.
#include "params.h"

namespace hcp {



__device__ __forceinline__ int swap_bits23(int x) {
  return (x & ~12) | ((x & 4) << 1) | ((x & 8) >> 1);
}
__device__ __forceinline__ int vt_swz(int d) { return (d + (d >> 3)) & 7; }

template <int D, typename T, bool CAUSAL, bool PAGED, bool VARLEN>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256),
                          amdgpu_waves_per_eu(2, 2))) void
fa_fwd_kernel(FwdParams p) {
  using E = Elem<T>;
  using V8 = typename E::vec8;
  constexpr int BM = kFwdBM, BN = kFwdBN;
  constexpr int KSTEPS = D / 16;     // QK^T k-steps of 16
  constexpr int DBLK = D / 32;       // 32-row blocks of O^T
  constexpr int KSLOTS = D / 8;      // 16-byte slots per K row
  constexpr int KROWS_PER_PASS = kFwdThreads / KSLOTS;
  constexpr int KLOADS = BN / KROWS_PER_PASS;  // 16-byte K loads per thread
  constexpr int VK = D / 16;         // keys per thread in the V^T transpose
  constexpr int DQ = D / 4;          // 4-wide d quads
  static_assert(D == 64 || D == 128, "head_dim");

  __shared__ __attribute__((aligned(16))) uint16_t smem[2][BN * D + D * BN];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
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
    // heaviest (last) query block first for causal
    qb = CAUSAL ? (p.num_tiles - 1 - tile) : tile;
  }
  const int64_t q_len = e.q_len;
  const int64_t kv_len = e.kv.len;
  const int64_t off = e.causal_offset;

  KvAddr kva;
  kva.init(e.kv);

  // ---- Q^T fragments (B operand): lane owns query row r32 ----
  const int64_t qi = static_cast<int64_t>(qb) * BM + wave * 32 + r32;
  const bool q_valid = qi < q_len;
  V8 qf[KSTEPS];
  {
    const char* qrow = reinterpret_cast<const char*>(p.q) +
                       ((e.q_start + (q_valid ? qi : 0)) * p.q_stride_tok +
                        static_cast<int64_t>(head) * p.q_stride_head) *
                           2;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      u32x4 x = q_valid ? ldg16(qrow + (16 * s + 8 * g) * 2) : u32x4{0, 0, 0, 0};
      qf[s] = as_vec8<V8>(x);
    }
  }

  // ---- key range of the workgroup and of this wave ----
  int64_t n_end = kv_len;
  if (CAUSAL) {
    int64_t lim = off + static_cast<int64_t>(qb) * BM + BM;
    n_end = n_end < lim ? n_end : lim;
  }
  if (n_end < 0) n_end = 0;
  const int ntiles = static_cast<int>((n_end + BN - 1) / BN);
  const int64_t wave_q0 = static_cast<int64_t>(qb) * BM + wave * 32;
  const int64_t wave_last = CAUSAL ? off + wave_q0 + 31 : kv_len - 1;

  // ---- tile loader (global -> registers -> LDS) ----
  const int kc = tid % KSLOTS;      // 16-byte chunk of a K row
  const int kr0 = tid / KSLOTS;     // first K row of this thread
  const int vdq = tid % DQ;         // d quad for V
  const int vpg = tid / DQ;         // V^T position group (VK positions)
  u32x4 kreg[KLOADS];
  u32x2 vreg[VK];

  auto load_tile = [&](int64_t n0) {
#pragma unroll
    for (int rr = 0; rr < KLOADS; ++rr) {
      const int64_t key = n0 + kr0 + rr * KROWS_PER_PASS;
      if (key < kv_len) {
        const int64_t o = kva.offset<PAGED>(key, kvh) + kc * 8;
        kreg[rr] = ldg16(kva.k + o * 2);
      } else {
        kreg[rr] = u32x4{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int j = 0; j < VK; ++j) {
      const int64_t key = n0 + swap_bits23(VK * vpg + j);
      if (key < kv_len) {
        const int64_t o = kva.offset<PAGED>(key, kvh) + vdq * 4;
        vreg[j] = ldg8(kva.v + o * 2);
      } else {
        vreg[j] = u32x2{0, 0};
      }
    }
  };

  auto store_tile = [&](int buf) {
    uint16_t* Ks = smem[buf];
    uint16_t* Vt = smem[buf] + BN * D;
#pragma unroll
    for (int rr = 0; rr < KLOADS; ++rr) {
      const int row = kr0 + rr * KROWS_PER_PASS;
      const int slot = row * KSLOTS + (kc ^ (row & 7));
      *reinterpret_cast<u32x4*>(Ks + slot * 8) = kreg[rr];
    }
#pragma unroll
    for (int dd = 0; dd < 4; ++dd) {
      const int d = 4 * vdq + dd;
      const int word = dd >> 1;
      uint32_t packed[VK / 2];
#pragma unroll
      for (int j = 0; j < VK / 2; ++j) {
        uint32_t a = vreg[2 * j][word], b = vreg[2 * j + 1][word];
        packed[j] = (dd & 1) ? ((a >> 16) | (b & 0xffff0000u))
                             : ((a & 0xffffu) | (b << 16));
      }
      if constexpr (VK == 8) {
        const int slot = vpg ^ vt_swz(d);
        *reinterpret_cast<u32x4*>(Vt + d * BN + slot * 8) =
            u32x4{packed[0], packed[1], packed[2], packed[3]};
      } else {
        const int slot = (vpg >> 1) ^ vt_swz(d);
        *reinterpret_cast<u32x2*>(Vt + d * BN + slot * 8 + (vpg & 1) * 4) =
            u32x2{packed[0], packed[1]};
      }
    }
  };

  // ---- online softmax state ----
  const float c = p.scale_log2;
  float m_run = -INFINITY;
  float l_run = 0.f;
  f32x16 oacc[DBLK];
#pragma unroll
  for (int i = 0; i < DBLK; ++i) oacc[i] = f32x16{};

  if (ntiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  for (int it = 0; it < ntiles; ++it) {
    const int64_t n0 = static_cast<int64_t>(it) * BN;
    const bool more = it + 1 < ntiles;
    if (more) load_tile(n0 + BN);
    const uint16_t* Ks = smem[it & 1];
    const uint16_t* Vt = smem[it & 1] + BN * D;

    if (!CAUSAL || n0 <= wave_last) {
      // S^T = K Q^T : two 32-key blocks
      f32x16 s0 = f32x16{}, s1 = f32x16{};
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) {
        const int sl = 2 * s + g;
        const int row0 = r32, row1 = 32 + r32;
        V8 k0 = as_vec8<V8>(*reinterpret_cast<const u32x4*>(
            Ks + (row0 * KSLOTS + (sl ^ (row0 & 7))) * 8));
        V8 k1 = as_vec8<V8>(*reinterpret_cast<const u32x4*>(
            Ks + (row1 * KSLOTS + (sl ^ (row1 & 7))) * 8));
        s0 = E::mfma32(k0, qf[s], s0);
        s1 = E::mfma32(k1, qf[s], s1);
      }
      // masking on ragged / diagonal tiles
      const bool ragged = n0 + BN > kv_len;
      const bool diag = CAUSAL && (n0 + BN - 1 > off + wave_q0);
      if (ragged || diag) {
        const int64_t lim = CAUSAL ? off + qi : kv_len - 1;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kk = 8 * (r >> 2) + 4 * g + (r & 3);
          const int64_t key0 = n0 + kk, key1 = n0 + 32 + kk;
          if (key0 >= kv_len || key0 > lim) s0[r] = -INFINITY;
          if (key1 >= kv_len || key1 > lim) s1[r] = -INFINITY;
        }
      }
      float mx = s0[0];
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, fmaxf(s0[r], s1[r]));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_run, mx * c);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = fast_exp2(m_run - m_use);
      float rs = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s0[r] = fast_exp2(__builtin_fmaf(s0[r], c, -m_use));
        s1[r] = fast_exp2(__builtin_fmaf(s1[r], c, -m_use));
        rs += s0[r] + s1[r];
      }
      l_run = l_run * alpha + rs;
      m_run = m_new;
#pragma unroll
      for (int i = 0; i < DBLK; ++i) oacc[i] *= alpha;

      // P^T fragments: step t uses S^T block t/2, registers 8(t%2)..+7
      V8 pf[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const f32x16& sb = (t < 2) ? s0 : s1;
        const int base = 8 * (t & 1);
        u32x4 w;
        w[0] = pack2<T>(sb[base + 0], sb[base + 1]);
        w[1] = pack2<T>(sb[base + 2], sb[base + 3]);
        w[2] = pack2<T>(sb[base + 4], sb[base + 5]);
        w[3] = pack2<T>(sb[base + 6], sb[base + 7]);
        pf[t] = as_vec8<V8>(w);
      }
      // O^T += V^T P^T
#pragma unroll
      for (int db = 0; db < DBLK; ++db) {
        const int d = 32 * db + r32;
        const int sw = vt_swz(d);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          V8 vf = as_vec8<V8>(*reinterpret_cast<const u32x4*>(
              Vt + d * BN + ((2 * t + g) ^ sw) * 8));
          oacc[db] = E::mfma32(vf, pf[t], oacc[db]);
        }
      }
    }
    if (more) store_tile((it + 1) & 1);
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
          l_tot > 0.f ? m_run * kLn2 + __logf(l_tot) : -INFINITY;
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
