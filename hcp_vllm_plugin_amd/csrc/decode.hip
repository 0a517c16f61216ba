// Split-KV decode for gfx950: one query token per sequence, long KV segments.
//
// The reference decodes with the prefill kernel, grid (H, 1) per request and
// segment (ring_triton_attn.py:179, ring_backend.py:672,820-830): 28
// workgroups on a 256-CU part, 63 of 64 query rows padding, and every query
// head of a GQA group re-reading the same K/V.  Here:
//
//  * kernel 1 (decode_split_kernel): one workgroup per (split, KV head).  A
//    split is a key range of one segment (contiguous peer or paged local; the
//    form is per entry, so one launch serves both).  All G query
//    heads of the KV head are the 16 columns of v_mfma_f32_16x16x32 (G <= 16),
//    so each K/V byte is read from HBM once.  Each of the 4 waves walks its
//    own 32-key chunks straight from global memory into MFMA operands (no LDS,
//    no barrier in the loop); the next chunk's loads are in flight while the
//    current one is computed.
//      S^T = K Q^T   A = K rows (one key per lane row), B = Q^T; k-step s
//                    covers d = 32s .. 32s+31, so each K load instruction
//                    reads one contiguous 64 B piece of 16 key rows
//      O^T = V^T P^T A = V^T, B = P^T taken from the S^T registers.
//    For V^T each lane loads 8 keys x 8 contiguous d (16 B per key, whole
//    256 B rows per load instruction) and transposes the 8x8 block in
//    registers; MFMA number u then covers d = 8*row + u.  The 4 waves'
//    (m, l, O) are combined through LDS and one fp32 partial (O normalised,
//    LSE natural log) per (split, head) goes to the workspace.
//  * kernel 2 (decode_reduce_kernel): per (sequence, head) merges all
//    partials of the sequence -- every split of its local and peer segments --
//    with the LSE merge of ring_decode.py:46-61, writing out in the model
//    dtype and optionally the merged LSE.
#include "params.h"

namespace hcp {

constexpr int kDecThreads = 256;
constexpr int kDecChunk = 32;  // keys per wave step

template <int D, typename T, bool PAGED>
__device__ __forceinline__ void decode_split_body(const DecParams& p, int kvh, int sp,
                                                  const hcp_varlen_entry& e,
                                                  const hcp_decode_split& spl) {
  using E = Elem<T>;
  using V8 = typename E::vec8;
  constexpr int QSTEPS = D / 32;  // 16x16x32 k-steps over d
  constexpr int NU = D / 16;      // PV MFMAs (d = NU*row + u)
  static_assert(D == 64 || D == 128, "head_dim");

  __shared__ float sm_m[4][16];
  __shared__ float sm_l[4][16];
  __shared__ float sm_o[4][16][D];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int c16 = lane & 15;
  const int g4 = lane >> 4;
  const int G = p.group;
  KvAddr kva;
  kva.init(e.kv);
  const int64_t kb = spl.key_begin, ke = spl.key_end;

  // Q^T (B operand): column c16 = query head kvh*G + c16 (zero for c16 >= G)
  V8 qf[QSTEPS];
  {
    const bool hv = c16 < G;
    const char* qrow = reinterpret_cast<const char*>(p.q) +
                       (e.q_start * p.q_stride_tok +
                        static_cast<int64_t>(kvh * G + (hv ? c16 : 0)) * p.q_stride_head) * 2;
#pragma unroll
    for (int s = 0; s < QSTEPS; ++s) {
      u32x4 x = hv ? ldg16(qrow + (32 * s + 8 * g4) * 2) : u32x4{0, 0, 0, 0};
      qf[s] = as_vec8<V8>(x);
    }
  }

  const float c = p.scale_log2;
  float m_run = -INFINITY, l_run = 0.f;
  f32x4 oacc[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) oacc[u] = f32x4{};

  // chunk registers: K rows (2 blocks of 16 keys) and V rows (8 keys)
  u32x4 kreg[2][QSTEPS];
  u32x4 vreg[8];  // D=128: 8 d per key; D=64 uses the low half
  auto load_chunk = [&](int64_t k0) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int64_t key = k0 + 16 * b + c16;
      if (key < ke) {
        const char* src = kva.k + (kva.offset<PAGED>(key, kvh) + 8 * g4) * 2;
#pragma unroll
        for (int s = 0; s < QSTEPS; ++s) kreg[b][s] = ldg16(src + 64 * s);
      } else {
#pragma unroll
        for (int s = 0; s < QSTEPS; ++s) kreg[b][s] = u32x4{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t key = k0 + 16 * (j >> 2) + 4 * g4 + (j & 3);
      if (key < ke) {
        const char* src = kva.v + (kva.offset<PAGED>(key, kvh) + NU * c16) * 2;
        if constexpr (NU == 8) {
          vreg[j] = ldg16(src);
        } else {
          u32x2 x = ldg8(src);
          vreg[j] = u32x4{x[0], x[1], 0, 0};
        }
      } else {
        vreg[j] = u32x4{0, 0, 0, 0};
      }
    }
  };

  const int64_t nchunks = (ke - kb + kDecChunk - 1) / kDecChunk;
  int64_t ci = wave;
  if (ci < nchunks) load_chunk(kb + ci * kDecChunk);
  while (ci < nchunks) {
    const int64_t k0 = kb + ci * kDecChunk;
    // take this chunk's registers, start the next chunk's loads
    u32x4 kc[2][QSTEPS];
    u32x4 vc[8];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int s = 0; s < QSTEPS; ++s) kc[b][s] = kreg[b][s];
#pragma unroll
    for (int j = 0; j < 8; ++j) vc[j] = vreg[j];
    const int64_t cn = ci + 4;
    if (cn < nchunks) load_chunk(kb + cn * kDecChunk);

    f32x4 s0 = f32x4{}, s1 = f32x4{};
#pragma unroll
    for (int s = 0; s < QSTEPS; ++s) {
      s0 = E::mfma16(as_vec8<V8>(kc[0][s]), qf[s], s0);
      s1 = E::mfma16(as_vec8<V8>(kc[1][s]), qf[s], s1);
    }
    if (k0 + kDecChunk > ke) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (k0 + 4 * g4 + r >= ke) s0[r] = -INFINITY;
        if (k0 + 16 + 4 * g4 + r >= ke) s1[r] = -INFINITY;
      }
    }
    float mx = fmaxf(fmaxf(fmaxf(s0[0], s0[1]), fmaxf(s0[2], s0[3])),
                     fmaxf(fmaxf(s1[0], s1[1]), fmaxf(s1[2], s1[3])));
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx * c);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - m_use);
    float rs = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      s0[r] = fast_exp2(__builtin_fmaf(s0[r], c, -m_use));
      s1[r] = fast_exp2(__builtin_fmaf(s1[r], c, -m_use));
      rs += s0[r] + s1[r];
    }
    l_run = l_run * alpha + rs;
    m_run = m_new;
#pragma unroll
    for (int u = 0; u < NU; ++u) oacc[u] *= alpha;

    u32x4 pw;
    pw[0] = pack2<T>(s0[0], s0[1]);
    pw[1] = pack2<T>(s0[2], s0[3]);
    pw[2] = pack2<T>(s1[0], s1[1]);
    pw[3] = pack2<T>(s1[2], s1[3]);
    const V8 pf = as_vec8<V8>(pw);

    // 8 keys x NU d in registers -> NU operands of 8 keys each
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int word = u >> 1;
      u32x4 a;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t x = vc[2 * j][word], y = vc[2 * j + 1][word];
        a[j] = (u & 1) ? ((x >> 16) | (y & 0xffff0000u)) : ((x & 0xffffu) | (y << 16));
      }
      oacc[u] = E::mfma16(as_vec8<V8>(a), pf, oacc[u]);
    }
    ci = cn;
  }

  // ---- combine the 4 waves ----
  float l_tot = l_run + __shfl_xor(l_run, 16);
  l_tot += __shfl_xor(l_tot, 32);
  if (g4 == 0) {
    sm_m[wave][c16] = m_run;
    sm_l[wave][c16] = l_tot;
  }
#pragma unroll
  for (int u = 0; u < NU; ++u)
#pragma unroll
    for (int r = 0; r < 4; ++r) sm_o[wave][c16][NU * (4 * g4 + r) + u] = oacc[u][r];
  __syncthreads();

  for (int idx = tid; idx < G * D; idx += kDecThreads) {
    const int h = idx / D, d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, sm_m[w][h]);
    const float Mu = (M == -INFINITY) ? 0.f : M;
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float sc = fast_exp2(sm_m[w][h] - Mu);
      L += sm_l[w][h] * sc;
      O += sm_o[w][h][d] * sc;
    }
    const int head = kvh * G + h;
    const int64_t slot = static_cast<int64_t>(sp) * p.num_heads + head;
    p.ws_o[slot * D + d] = L > 0.f ? O / L : 0.f;
    if (d == 0) p.ws_lse[slot] = L > 0.f ? M * kLn2 + __logf(L) : -INFINITY;
  }
}

// Paged-ness is a property of each entry (a sequence's peer segment is
// contiguous, its local segment paged), uniform within a workgroup.
template <int D, typename T>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256),
                          amdgpu_waves_per_eu(2, 2))) void
decode_split_kernel(DecParams p) {
  int kvh;
  int64_t item;
  if (!xcd_remap(blockIdx.x, p.num_splits, p.num_kv_heads, &kvh, &item)) return;
  const hcp_decode_split spl = p.splits[item];
  const int sp = spl.slot;  // workspace partial of this split
  const hcp_varlen_entry e = p.entries[spl.entry];
  if (e.kv.block_table != 0)
    decode_split_body<D, T, true>(p, kvh, sp, e, spl);
  else
    decode_split_body<D, T, false>(p, kvh, sp, e, spl);
}

template <int D, typename T>
__global__ __launch_bounds__(D) void decode_reduce_kernel(RedParams p) {
  const int sh = blockIdx.x;
  const int seq = sh / p.num_heads, head = sh % p.num_heads;
  const int d = threadIdx.x;
  const int p0 = p.seq_partial_start[seq], p1 = p.seq_partial_start[seq + 1];
  float M = -INFINITY;
  for (int i = p0; i < p1; ++i)
    M = fmaxf(M, p.ws_lse[static_cast<int64_t>(i) * p.num_heads + head]);
  float o = 0.f, lse = -INFINITY;
  if (M != -INFINITY) {
    float S = 0.f, O = 0.f;
    for (int i = p0; i < p1; ++i) {
      const int64_t slot = static_cast<int64_t>(i) * p.num_heads + head;
      const float w = __expf(p.ws_lse[slot] - M);
      S += w;
      O += w * p.ws_o[slot * D + d];
    }
    o = O / S;
    lse = M + __logf(S);
  }
  uint16_t* orow = reinterpret_cast<uint16_t*>(p.out) + seq * p.o_stride_tok +
                   static_cast<int64_t>(head) * p.o_stride_head;
  orow[d] = Elem<T>::from_float(o);
  if (p.lse != nullptr && d == 0)
    p.lse[static_cast<int64_t>(head) * p.lse_stride_head + seq] = lse;
}

template <int D, typename T>
static hipError_t launch_dec_t(const DecParams& dp, const RedParams& rp, hipStream_t st) {
  const int64_t grid = xcd_grid_size(dp.num_splits, dp.num_kv_heads);
  if (grid > 0) {
    hipLaunchKernelGGL((decode_split_kernel<D, T>), dim3(static_cast<unsigned>(grid)),
                       dim3(kDecThreads), 0, st, dp);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  const int64_t rgrid = static_cast<int64_t>(rp.num_seqs) * rp.num_heads;
  if (rgrid > 0) {
    hipLaunchKernelGGL((decode_reduce_kernel<D, T>), dim3(static_cast<unsigned>(rgrid)),
                       dim3(D), 0, st, rp);
    return hipGetLastError();
  }
  return hipSuccess;
}

hipError_t launch_decode(const DecParams& dp, const RedParams& rp, int head_dim,
                         int dtype, hipStream_t st) {
  if (head_dim == 128)
    return dtype == HCP_DTYPE_BF16 ? launch_dec_t<128, __bf16>(dp, rp, st)
                                   : launch_dec_t<128, _Float16>(dp, rp, st);
  return dtype == HCP_DTYPE_BF16 ? launch_dec_t<64, __bf16>(dp, rp, st)
                                 : launch_dec_t<64, _Float16>(dp, rp, st);
}

}  // namespace hcp
