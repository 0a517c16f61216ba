// Split-KV decode for gfx950: one query token per sequence, long KV segments.
//
// The reference decodes with the prefill kernel, grid (H, 1) per request and
// segment (ring_triton_attn.py:179, ring_backend.py:672,820-830): 28
// workgroups on a 256-CU part, 63 of 64 query rows padding, and every query
// head of a GQA group re-reading the same K/V.  Here:
//
//  * kernel 1 (decode_split_kernel): one workgroup per (split, KV head,
//    head chunk).  A split is a key range of one segment (contiguous peer or
//    paged local; the form is per entry, so one launch serves both).  Up to 16
//    query heads of the KV head are the 16 columns of v_mfma_f32_16x16x32, so
//    with G <= 16 each K/V byte is read from HBM once; a larger group runs in
//    ceil(G / 16) chunks of 16 heads, dispatched next to each other so the
//    chunks after the first mostly read the split's K/V from L2.  Each of the 4 waves walks its
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
// raw buffer descriptor word 3 (32-bit data format, bounds-checked)
constexpr int kBufWord3 = 0x00020000;
// cache policy of the K/V stream: non-temporal (read once per launch)
constexpr int kStreamAux = 2;
#define HCP_LDS_PTR(T) __attribute__((address_space(3))) T*


// LDS of the split kernel, shared by its paged and contiguous instantiations.
// Each wave double-buffers its chunks' K and V rows; D = 256 runs two waves
// per workgroup so the buffers stay within 128 KB.
template <int D>
struct DecShared {
  static constexpr int CHB = kDecChunk * D * 2;  // bytes of a chunk's K (or V) rows
  static constexpr int W = D == 256 ? 2 : 4;     // waves per workgroup
};

template <int D, typename T, bool PAGED>
__device__ __forceinline__ void decode_split_body(const DecParams& p, int kvh_in, int chunk_in,
                                                  int sp,
                                                  const hcp_varlen_entry& e,
                                                  const hcp_decode_split& spl,
                                                  char (*bufE)[2 * DecShared<D>::CHB],
                                                  char (*bufO)[2 * DecShared<D>::CHB],
                                                  float (*sm_m)[16], float (*sm_l)[16]) {
  using E = Elem<T>;
  using V8 = typename E::vec8;
  constexpr int QSTEPS = D / 32;         // 16x16x32 k-steps over d
  constexpr int NU = D / 16;             // PV MFMAs (d = NU*row + u)
  constexpr int ROWB = D * 2;            // bytes of one key row of one head
  constexpr int CPR = ROWB / 16;         // 16-byte slots per row
  constexpr int CHB = kDecChunk * ROWB;  // bytes of the K (or V) rows of a chunk
  constexpr int NLD = CHB / 1024;        // LDS-DMA instructions per K (or V) chunk
  constexpr int KPI = 1024 / ROWB;       // key rows per DMA instruction
  static_assert(D == 64 || D == 128 || D == 256, "head_dim");
  constexpr int W = DecShared<D>::W;  // waves per workgroup

  // Wave-private chunk buffers [K rows | V rows] (bufE / bufO: even / odd
  // chunks of the wave, distinct objects so the compiler can tell reads of
  // one from the DMA writes into the other).  Row r's 16-byte slot c sits at
  // slot c ^ (r % CPR): both operand reads below are then conflict-free.

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int c16 = lane & 15;
  const int g4 = lane >> 4;
  // the KV head and head chunk are workgroup-uniform: keep every address
  // built from them in SGPRs (buffer descriptors from VGPR values become
  // waterfall loops).  This workgroup's query heads: h0 .. h0 + G - 1.
  const int kvh = __builtin_amdgcn_readfirstlane(kvh_in);
  const int chunk = __builtin_amdgcn_readfirstlane(chunk_in);
  const int G = p.group - 16 * chunk < 16 ? p.group - 16 * chunk : 16;
  const int h0 = kvh * p.group + 16 * chunk;
  KvAddr kva;
  kva.init(e.kv);
  const int64_t kb = spl.key_begin, ke = spl.key_end;

  // A row holds dv <= D valid elements (a multiple of 8): the kernel computes
  // in D columns.  Q's tail is zero; a K/V chunk past dv is fetched from the
  // row's first chunk instead (finite values that meet Q's zero columns, or
  // land in output columns that are never stored), so no load leaves the row.
  const int dv = p.head_dim;
  const int cv = dv / 8;  // valid 16-byte chunks of a row
  // Q^T (B operand): column c16 = query head h0 + c16 (zero for c16 >= G);
  // k-step s covers d = 32s .. 32s+31 (lane group g4: 8 of them)
  V8 qf[QSTEPS];
  {
    const bool hv = c16 < G;
    const char* qrow = reinterpret_cast<const char*>(p.q) +
                       (e.q_start * p.q_stride_tok +
                        static_cast<int64_t>(h0 + (hv ? c16 : 0)) * p.q_stride_head) * 2;
#pragma unroll
    for (int s = 0; s < QSTEPS; ++s) {
      u32x4 x = hv && 32 * s + 8 * g4 < dv ? ldg16(qrow + (32 * s + 8 * g4) * 2)
                                           : u32x4{0, 0, 0, 0};
      qf[s] = as_vec8<V8>(x);
    }
  }

  const float c = p.scale_log2;
  float m_run = -INFINITY, l_run = 0.f;
  f32x4 oacc[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) oacc[u] = f32x4{};

  // ---- HBM -> LDS: one chunk (32 keys) of K and V rows ----
  // DMA instruction j writes rows j*KPI .. j*KPI+KPI-1; lane -> (row kr, slot
  // sl), fetching the row's 16-byte piece (sl ^ row % CPR): every
  // instruction reads KPI whole rows (1 KB), streamed past the caches.
  const int kr = lane / CPR, sl = lane % CPR;
  const int64_t rowb_g = kva.stride_tok * 2;
  // (contiguous segments; paged ones are issued by the loop further down)
  auto issue = [&](int64_t k0, HCP_LDS_PTR(char) dst) __attribute__((always_inline)) {
    if constexpr (!PAGED) {
      const int64_t rows = ke - k0;  // >= 1 valid rows in this chunk
      const int nrec = rows >= kDecChunk ? 0x7fffffff
                                         : static_cast<int>((rows - 1) * rowb_g) + 2 * dv;
      const int64_t base = ((kva.start + k0) * kva.stride_tok +
                            static_cast<int64_t>(kvh) * kva.stride_head) * 2;
      const __amdgpu_buffer_rsrc_t rk =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(kva.k + base), 0, nrec, kBufWord3);
      const __amdgpu_buffer_rsrc_t rv =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(kva.v + base), 0, nrec, kBufWord3);
#pragma unroll
      for (int j = 0; j < NLD; ++j) {
        const int row = j * KPI + kr;
        int ch = sl ^ (row % CPR);
        ch = ch < cv ? ch : 0;
        const int off = static_cast<int>(row * rowb_g) + 16 * ch;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rk, reinterpret_cast<HCP_LDS_PTR(void)>(dst + j * 1024), 16, off, 0, 0, kStreamAux);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rv, reinterpret_cast<HCP_LDS_PTR(void)>(dst + CHB + j * 1024), 16, off, 0, 0,
            kStreamAux);
      }
    }
  };

  // ---- one chunk from LDS: S^T = K Q^T, online softmax, O^T += V^T P^T ----
  auto compute = [&](int64_t k0, const HCP_LDS_PTR(char) src) __attribute__((always_inline)) {
    // K rows 16b + c16, d = 32s + 8g4 .. +7: slot (4s + g4) of that row
    f32x4 s0 = f32x4{}, s1 = f32x4{};
#pragma unroll
    for (int s = 0; s < QSTEPS; ++s) {
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const int row = 16 * b + c16;
        const u32x4 kx = *reinterpret_cast<const HCP_LDS_PTR(u32x4)>(
            src + row * ROWB + 16 * ((4 * s + g4) ^ (row % CPR)));
        if (b == 0)
          s0 = E::mfma16(as_vec8<V8>(kx), qf[s], s0);
        else
          s1 = E::mfma16(as_vec8<V8>(kx), qf[s], s1);
      }
    }
    // V rows 16(j>>2) + 4g4 + (j&3), d = NU*c16 .. +NU-1 (NU/2 words)
    constexpr int VW = NU / 2 < 4 ? 4 : NU / 2;
    typedef uint32_t vwords __attribute__((ext_vector_type(VW)));
    vwords vc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int row = 16 * (j >> 2) + 4 * g4 + (j & 3);
      const HCP_LDS_PTR(char) vrow = src + CHB + row * ROWB;
      if constexpr (NU == 16) {
        const u32x4 x0 = *reinterpret_cast<const HCP_LDS_PTR(u32x4)>(
            vrow + 16 * ((2 * c16) ^ (row % CPR)));
        const u32x4 x1 = *reinterpret_cast<const HCP_LDS_PTR(u32x4)>(
            vrow + 16 * ((2 * c16 + 1) ^ (row % CPR)));
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          vc[j][w] = x0[w];
          vc[j][4 + w] = x1[w];
        }
      } else if constexpr (NU == 8) {
        const u32x4 x = *reinterpret_cast<const HCP_LDS_PTR(u32x4)>(vrow + 16 * (c16 ^ (row % CPR)));
#pragma unroll
        for (int w = 0; w < 4; ++w) vc[j][w] = x[w];
      } else {
        const u32x2 x = *reinterpret_cast<const HCP_LDS_PTR(u32x2)>(
            vrow + 16 * ((c16 >> 1) ^ (row % CPR)) + 8 * (c16 & 1));
        vc[j][0] = x[0];
        vc[j][1] = x[1];
        vc[j][2] = 0;
        vc[j][3] = 0;
      }
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
  };

  // ---- the wave's chunks wave, wave+W, ...; next chunk's DMA in flight ----
  const int64_t nchunks = (ke - kb + kDecChunk - 1) / kDecChunk;
  HCP_LDS_PTR(char) be = (HCP_LDS_PTR(char))(bufE[wave]);
  HCP_LDS_PTR(char) bo = (HCP_LDS_PTR(char))(bufO[wave]);
  // The next chunk's DMA is issued unconditionally (past the wave's last
  // chunk it re-reads the split's last chunk into the buffer nobody reads):
  // with no branch around it, the wait before each compute is exactly "the
  // previous chunk's loads", not a conservative wait for all of them.
  const int64_t last = nchunks - 1;
  auto next_k0 = [&](int64_t cn) __attribute__((always_inline)) {
    return kb + (cn < last ? cn : last) * kDecChunk;
  };
  // Before a compute, the wave waits until only the 2*NLD loads it just
  // issued (into the other buffer) are outstanding: its own DMA into the
  // buffer it reads has landed.  Buffers are wave-private, so no barrier.
  int64_t ci = wave;
  // Paged segments: the lane's block ids are fetched one chunk ahead of the
  // chunk's DMA, so looking them up never waits on the DMA in flight.  When
  // the cache spans less than 4 GiB from this head's base the DMA is a
  // bounds-checked buffer load over one descriptor for the whole cache (a
  // block id past the cache reads zeros); otherwise a global load with a
  // 64-bit address (a block id past the cache clamped to its last block).
  if constexpr (PAGED) {
    const int64_t blockb = kva.stride_block * 2;
    const uint64_t span = static_cast<uint64_t>(e.kv.num_blocks) * static_cast<uint64_t>(blockb);
    const bool pbuf = e.kv.num_blocks > 0 && span < (uint64_t{1} << 32);
    if (ci < nchunks) {
      const int64_t hb = static_cast<int64_t>(kvh) * kva.stride_head * 2;
      const int nrec =
          __builtin_amdgcn_readfirstlane(pbuf ? static_cast<int>(static_cast<uint32_t>(span)) : 0);
      // the bases are wave-uniform; say so, or the descriptors land in
      // VGPRs and every buffer load becomes a waterfall loop
      auto uniform_ptr = [](const char* ptr) __attribute__((always_inline)) {
        const uint64_t a = reinterpret_cast<uint64_t>(ptr);
        const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a));
        const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32));
        return reinterpret_cast<char*>((static_cast<uint64_t>(hi) << 32) | lo);
      };
      const __amdgpu_buffer_rsrc_t rk =
          __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(kva.k + hb), 0, nrec, kBufWord3);
      const __amdgpu_buffer_rsrc_t rv =
          __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(kva.v + hb), 0, nrec, kBufWord3);
      const uint32_t id_max = __builtin_amdgcn_readfirstlane(
          e.kv.num_blocks > 0 && e.kv.num_blocks <= 0xffffffffll
              ? static_cast<uint32_t>(e.kv.num_blocks - 1) : 0xffffffffu);
      uint32_t idA[NLD], idB[NLD];
      auto fetch_ids = [&](int64_t k0, uint32_t (&ids)[NLD]) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NLD; ++j) {
          int64_t key = k0 + j * KPI + kr;
          key = key < ke ? key : ke - 1;  // rows past the split: masked
          ids[j] = static_cast<uint32_t>(kva.bt[(kva.start + key) >> kva.bs_shift]);
        }
      };
      // one chunk's DMA; BUF (compile-time) picks the load form
      auto issue_p = [&](auto buf, int64_t k0, const uint32_t (&ids)[NLD], HCP_LDS_PTR(char) dst)
          __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NLD; ++j) {
          const int row = j * KPI + kr;
          int64_t key = k0 + row;
          key = key < ke ? key : ke - 1;
          const int64_t x = kva.start + key;
          int ch = sl ^ (row % CPR);
          ch = ch < cv ? ch : 0;
          const int64_t inb = (x & kva.bs_mask) * rowb_g + 16 * ch;
          if constexpr (decltype(buf)::value) {
            const uint32_t off = ids[j] * static_cast<uint32_t>(blockb) + static_cast<uint32_t>(inb);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rk, reinterpret_cast<HCP_LDS_PTR(void)>(dst + j * 1024), 16,
                static_cast<int>(off), 0, 0, kStreamAux);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rv, reinterpret_cast<HCP_LDS_PTR(void)>(dst + CHB + j * 1024), 16,
                static_cast<int>(off), 0, 0, kStreamAux);
          } else {
            // a block id past the cache is clamped to its last block
            const uint32_t id = ids[j] < id_max ? ids[j] : id_max;
            const int64_t o = static_cast<int64_t>(id) * blockb + hb + inb;
            __builtin_amdgcn_global_load_lds(
                reinterpret_cast<const __attribute__((address_space(1))) void*>(
                    reinterpret_cast<uintptr_t>(kva.k + o)),
                reinterpret_cast<HCP_LDS_PTR(void)>(dst + j * 1024), 16, 0, kStreamAux);
            __builtin_amdgcn_global_load_lds(
                reinterpret_cast<const __attribute__((address_space(1))) void*>(
                    reinterpret_cast<uintptr_t>(kva.v + o)),
                reinterpret_cast<HCP_LDS_PTR(void)>(dst + CHB + j * 1024), 16, 0, kStreamAux);
          }
        }
      };
      // per step: fetch the ids of chunk ci+2W, issue chunk ci+W (its ids
      // fetched a step ago), wait until only those 3*NLD loads are
      // outstanding -- chunk ci has landed -- and compute it
      auto run_loop = [&](auto buf) __attribute__((always_inline)) {
        fetch_ids(kb + ci * kDecChunk, idA);
        fetch_ids(next_k0(ci + W), idB);
        issue_p(buf, kb + ci * kDecChunk, idA, be);
        while (true) {
          fetch_ids(next_k0(ci + 2 * W), idA);
          issue_p(buf, next_k0(ci + W), idB, bo);
          wait_vmcnt<3 * NLD>();
          compute(kb + ci * kDecChunk, be);
          ci += W;
          if (ci >= nchunks) break;
          fetch_ids(next_k0(ci + 2 * W), idB);
          issue_p(buf, next_k0(ci + W), idA, be);
          wait_vmcnt<3 * NLD>();
          compute(kb + ci * kDecChunk, bo);
          ci += W;
          if (ci >= nchunks) break;
        }
      };
      if (pbuf)
        run_loop(std::true_type{});
      else
        run_loop(std::false_type{});
    }
  }
  if (!PAGED && ci < nchunks) {
    issue(kb + ci * kDecChunk, be);
    while (true) {
      issue(next_k0(ci + W), bo);
      wait_vmcnt<2 * NLD>();
      compute(kb + ci * kDecChunk, be);
      ci += W;
      if (ci >= nchunks) break;
      issue(next_k0(ci + W), be);
      wait_vmcnt<2 * NLD>();
      compute(kb + ci * kDecChunk, bo);
      ci += W;
      if (ci >= nchunks) break;
    }
  }

  // ---- combine the W waves (the chunk buffers are reused for O) ----
  // Each wave's last prefetch (issued unconditionally in the loop) may still
  // be writing bufE/bufO, which sm_o overlays: drain it before the barrier.
  wait_vmcnt<0>();
  __syncthreads();
  float (*sm_o)[16][D] = reinterpret_cast<float (*)[16][D]>(&bufE[0][0]);
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

  for (int idx = tid; idx < G * D; idx += 64 * W) {
    const int h = idx / D, d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < W; ++w) M = fmaxf(M, sm_m[w][h]);
    const float Mu = (M == -INFINITY) ? 0.f : M;
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float sc = fast_exp2(sm_m[w][h] - Mu);
      L += sm_l[w][h] * sc;
      O += sm_o[w][h][d] * sc;
    }
    const int head = h0 + h;
    const int64_t slot = static_cast<int64_t>(sp) * p.num_heads + head;
    p.ws_o[slot * D + d] = L > 0.f ? O / L : 0.f;
    if (d == 0) p.ws_lse[slot] = L > 0.f ? M * kLn2 + __logf(L) : -INFINITY;
  }
}

// Paged-ness is a property of each entry (a sequence's peer segment is
// contiguous, its local segment paged), uniform within a workgroup.
template <int D, typename T>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * DecShared<D>::W, 64 * DecShared<D>::W),
                          amdgpu_waves_per_eu(1, 1))) void
decode_split_kernel(DecParams p) {
  constexpr int CHB = DecShared<D>::CHB;
  constexpr int W = DecShared<D>::W;
  __shared__ __attribute__((aligned(1024))) char bufE[W][2 * CHB];
  __shared__ __attribute__((aligned(1024))) char bufO[W][2 * CHB];
  __shared__ float sm_m[W][16];
  __shared__ float sm_l[W][16];
  int kvh;
  int64_t item;
  if (!xcd_remap(blockIdx.x, static_cast<int64_t>(p.num_splits) * p.head_chunks,
                 p.num_kv_heads, &kvh, &item))
    return;
  const int chunk = static_cast<int>(item % p.head_chunks);
  const hcp_decode_split spl = p.splits[item / p.head_chunks];
  const int sp = spl.slot;  // workspace partial of this split
  const hcp_varlen_entry e = p.entries[spl.entry];
  if (e.kv.block_table != 0)
    decode_split_body<D, T, true>(p, kvh, chunk, sp, e, spl, bufE, bufO, sm_m, sm_l);
  else
    decode_split_body<D, T, false>(p, kvh, chunk, sp, e, spl, bufE, bufO, sm_m, sm_l);
}

// Merge every partial of one (sequence, query head) -- and the running
// accumulator, when given -- into the output row and its LSE.  One workgroup
// of D threads per (sequence, head) column group, thread d owns column d;
// with many partials per sequence (1, 2 or 4 groups) the groups take
// interleaved shares of the partials and are summed through LDS.  The max over
// partial LSEs is thread-strided plus a block reduction; the weighted sum
// issues 8 partials' loads before consuming them, so a long sequence (one
// request split over the whole machine) is not a chain of dependent loads.
template <int D, typename T>
__global__ __launch_bounds__(4 * D) void decode_reduce_kernel(RedParams p) {
  constexpr int kMaxWaves = 4 * D / 64;
  __shared__ float sm_max[kMaxWaves];
  __shared__ float sm_s[4];
  __shared__ float sm_o[4][D];
  const int ng = p.groups;  // column groups; group gi takes partials gi, gi + ng, ...
  const int sh = blockIdx.x;
  const int seq = sh / p.num_heads, head = sh % p.num_heads;
  const int tid = threadIdx.x;
  const int d = tid % D, gi = tid / D;
  const int p0 = p.seq_partial_start[seq], p1 = p.seq_partial_start[seq + 1];
  const int n = p1 - p0;
  const int64_t lstep = p.num_heads;
  const float* lcol = p.ws_lse + static_cast<int64_t>(p0) * lstep + head;
  const int64_t ostep = lstep * D;
  const float* ocol = p.ws_o + (static_cast<int64_t>(p0) * lstep + head) * D + d;

  // accumulator first: out / lse may alias acc_o / acc_lse, and every read
  // of them happens before the barriers below, every write after them
  float acc_l = -INFINITY, acc_v = 0.f;
  if (p.acc_lse != nullptr) {
    acc_l = p.acc_lse[static_cast<int64_t>(head) * p.acc_lse_stride_head + seq];
    if (acc_l == INFINITY) acc_l = -INFINITY;  // merge_attn_states reads +inf as empty
    const uint16_t* arow = reinterpret_cast<const uint16_t*>(p.acc_o) +
                           seq * p.acc_stride_tok + static_cast<int64_t>(head) * p.acc_stride_head;
    acc_v = d < p.head_dim ? Elem<T>::to_float(arow[d]) : 0.f;
  }

  // max over the partial LSEs, thread-strided over the whole block
  float m = -INFINITY;
  for (int i = tid; i < n; i += ng * D) m = fmaxf(m, lcol[i * lstep]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  if ((tid & 63) == 0) sm_max[tid >> 6] = m;
  __syncthreads();
  float M = acc_l;
  for (int w = 0; w < ng * D / 64; ++w) M = fmaxf(M, sm_max[w]);

  // this group's share of the weighted sum (S is the same in every column
  // of the group); 8 partials' loads are issued before they are consumed
  float S = 0.f, O = 0.f;
  if (M != -INFINITY) {
    int i = gi;
    for (; i + 7 * ng < n; i += 8 * ng) {
      float l[8], v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        l[j] = lcol[(i + j * ng) * lstep];
        v[j] = ocol[(i + j * ng) * ostep];
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float w = __expf(l[j] - M);
        S += w;
        O += w * v[j];
      }
    }
    for (; i < n; i += ng) {
      const float w = __expf(lcol[i * lstep] - M);
      S += w;
      O += w * ocol[i * ostep];
    }
  }
  if (ng > 1) {
    if (d == 0) sm_s[gi] = S;
    sm_o[gi][d] = O;
    __syncthreads();
    if (gi != 0) return;
    for (int g2 = 1; g2 < ng; ++g2) {
      S += sm_s[g2];
      O += sm_o[g2][d];
    }
  }
  float o = 0.f, lse = -INFINITY;
  if (M != -INFINITY) {
    if (acc_l != -INFINITY) {
      const float w = __expf(acc_l - M);
      S += w;
      O += w * acc_v;
    }
    o = O / S;
    lse = M + __logf(S);
  }
  uint16_t* orow = reinterpret_cast<uint16_t*>(p.out) + seq * p.o_stride_tok +
                   static_cast<int64_t>(head) * p.o_stride_head;
  if (d < p.head_dim) orow[d] = Elem<T>::from_float(o);
  if (p.lse != nullptr && d == 0)
    p.lse[static_cast<int64_t>(head) * p.lse_stride_head + seq] = lse;
}

template <int D, typename T>
static hipError_t launch_dec_t(const DecParams& dp, const RedParams& rp, hipStream_t st) {
  const int64_t grid =
      xcd_grid_size(static_cast<int64_t>(dp.num_splits) * dp.head_chunks, dp.num_kv_heads);
  if (grid > 0) {
    hipLaunchKernelGGL((decode_split_kernel<D, T>), dim3(static_cast<unsigned>(grid)),
                       dim3(64 * DecShared<D>::W), 0, st, dp);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  const int64_t rgrid = static_cast<int64_t>(rp.num_seqs) * rp.num_heads;
  if (rgrid > 0) {
    // more column groups when a sequence has many partials (one long
    // request split over the whole machine): shorter dependent load chains
    RedParams r = rp;
    const int per_seq = rp.num_seqs > 0 ? dp.num_splits / rp.num_seqs : 0;
    r.groups = per_seq >= 48 ? 4 : per_seq >= 24 ? 2 : 1;
    hipLaunchKernelGGL((decode_reduce_kernel<D, T>), dim3(static_cast<unsigned>(rgrid)),
                       dim3(D * r.groups), 0, st, r);
    return hipGetLastError();
  }
  return hipSuccess;
}

hipError_t launch_decode(const DecParams& dp, const RedParams& rp, int head_dim,
                         int dtype, hipStream_t st) {
  if (head_dim > 128)  // 136 .. 256: computed in 256 columns
    return dtype == HCP_DTYPE_BF16 ? launch_dec_t<256, __bf16>(dp, rp, st)
                                   : launch_dec_t<256, _Float16>(dp, rp, st);
  if (head_dim > 64)  // 72 .. 128: computed in 128 columns
    return dtype == HCP_DTYPE_BF16 ? launch_dec_t<128, __bf16>(dp, rp, st)
                                   : launch_dec_t<128, _Float16>(dp, rp, st);
  return dtype == HCP_DTYPE_BF16 ? launch_dec_t<64, __bf16>(dp, rp, st)
                                 : launch_dec_t<64, _Float16>(dp, rp, st);
}

}  // namespace hcp
