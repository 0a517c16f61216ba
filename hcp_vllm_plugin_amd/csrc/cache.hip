// Paged KV-cache write for gfx950: the step right before the attention path.
//
// Writes this step's K/V rows [n, Hkv, D] into the paged cache at
// slot_mapping (slot = block * block_size + offset), the operation of the
// reference's do_kv_cache_update (hcp_vllm_plugin/ring_backend.py:501-539,
// torch advanced-index assignment into [nb, 2, bs, Hkv, D]) and of vLLM's
// reshape_and_cache for the [nb, Hkv, bs, 2*D] layout the local-segment
// reader consumes (file_connector.py:13-16,175-179).  Both layouts are one
// stride triple plus separate K and V base addresses.  A negative slot is a
// padding token and is skipped (vLLM's convention); a slot past the cache is
// skipped as well, so a bad mapping cannot write outside the cache.
//
// HBM-bound copy: each thread moves 16 bytes (8 elements) of one (token,
// head) row of K and of V, so a wave covers whole rows (four 256-byte rows
// at D = 128) on both sides: 2 * n * Hkv * D * 2 bytes read and the same
// written.  Any head_dim that is a multiple of 8.
#include "params.h"

namespace hcp {

template <typename SlotT>
__global__ __launch_bounds__(256) void reshape_and_cache_kernel(CacheParams p) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  // (token, head) row and 16-byte chunk: a shift for a power-of-two chunk
  // count, else a division (workgroup-uniform choice)
  const int64_t row = p.cpr_shift >= 0 ? gid >> p.cpr_shift : gid / p.cpr;
  if (row >= p.num_tokens * p.num_kv_heads) return;
  const int ch = static_cast<int>(gid - row * p.cpr);
  const int64_t t = row / p.num_kv_heads;
  const int h = static_cast<int>(row - t * p.num_kv_heads);
  const int64_t slot = static_cast<int64_t>(reinterpret_cast<const SlotT*>(p.slots)[t]);
  if (slot < 0 || slot >= p.num_slots) return;
  const int64_t blk = slot >> p.bs_shift;
  const int64_t off = slot & p.bs_mask;
  const int64_t dst = (blk * p.stride_block + static_cast<int64_t>(h) * p.stride_head +
                       off * p.stride_tok + ch * 8) * 2;
  const char* k = reinterpret_cast<const char*>(p.key) +
                  (t * p.k_stride_tok + static_cast<int64_t>(h) * p.k_stride_head + ch * 8) * 2;
  const char* v = reinterpret_cast<const char*>(p.value) +
                  (t * p.v_stride_tok + static_cast<int64_t>(h) * p.v_stride_head + ch * 8) * 2;
  const u32x4 kx = ldg16(k);
  const u32x4 vx = ldg16(v);
  *reinterpret_cast<u32x4*>(reinterpret_cast<char*>(p.k_cache) + dst) = kx;
  *reinterpret_cast<u32x4*>(reinterpret_cast<char*>(p.v_cache) + dst) = vx;
}

hipError_t launch_cache_write(const CacheParams& p, bool slots_i64, hipStream_t st) {
  const int64_t threads = p.num_tokens * p.num_kv_heads * p.cpr;
  const int64_t grid = (threads + 255) / 256;
  if (grid <= 0) return hipSuccess;
  if (slots_i64)
    hipLaunchKernelGGL(reshape_and_cache_kernel<int64_t>, dim3(static_cast<unsigned>(grid)),
                       dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL(reshape_and_cache_kernel<int32_t>, dim3(static_cast<unsigned>(grid)),
                       dim3(256), 0, st, p);
  return hipGetLastError();
}

// Paged segment gather: the inverse copy, for prefill over caches whose
// blocks are shorter than the 16 rows a prefill wave loads from one block.
// Entry e's keys [start, start + len) of its request's block frame go to
// rows out_start[e] .. + len of a contiguous [total, Hkv, D] K and V -- the
// reference's per-request gather (ring_backend.py:617-624) for the whole
// batch in one launch, on the device.  Block ids at or past the cache's
// num_blocks (when given) are clamped to its last block, as in the
// attention kernels.  grid.y: entry; grid.x: (token, head, 16-byte chunk).
__global__ __launch_bounds__(256) void gather_segments_kernel(GatherParams p) {
  const hcp_kv_segment s = p.entries[blockIdx.y].kv;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t row = p.cpr_shift >= 0 ? gid >> p.cpr_shift : gid / p.cpr;
  if (row >= s.len * p.num_kv_heads) return;
  // only paged entries with a power-of-two block size are gathered
  if (s.block_table == 0 || s.block_size <= 0 || (s.block_size & (s.block_size - 1))) return;
  const int ch = static_cast<int>(gid - row * p.cpr);
  const int64_t t = row / p.num_kv_heads;
  const int h = static_cast<int>(row - t * p.num_kv_heads);
  const int bs_shift = 31 - __builtin_clz(static_cast<unsigned>(s.block_size));
  const int64_t pos = s.start + t;
  uint32_t blk = static_cast<uint32_t>(reinterpret_cast<const int32_t*>(s.block_table)[pos >> bs_shift]);
  if (s.num_blocks > 0 && blk >= static_cast<uint32_t>(s.num_blocks))
    blk = static_cast<uint32_t>(s.num_blocks - 1);
  const int64_t src = (static_cast<int64_t>(blk) * s.stride_block +
                       static_cast<int64_t>(h) * s.stride_head +
                       (pos & (s.block_size - 1)) * s.stride_tok + ch * 8) * 2;
  const int64_t dst = (((p.out_start[blockIdx.y] + t) * p.num_kv_heads + h) * p.head_dim +
                       ch * 8) * 2;
  const u32x4 kx = ldg16(reinterpret_cast<const char*>(s.k_addr) + src);
  const u32x4 vx = ldg16(reinterpret_cast<const char*>(s.v_addr) + src);
  *reinterpret_cast<u32x4*>(reinterpret_cast<char*>(p.k_out) + dst) = kx;
  *reinterpret_cast<u32x4*>(reinterpret_cast<char*>(p.v_out) + dst) = vx;
}

hipError_t launch_gather(const GatherParams& p, hipStream_t st) {
  const int64_t threads = p.max_len * p.num_kv_heads * p.cpr;
  const int64_t grid = (threads + 255) / 256;
  if (grid <= 0 || p.num_entries <= 0) return hipSuccess;
  hipLaunchKernelGGL(gather_segments_kernel,
                     dim3(static_cast<unsigned>(grid), static_cast<unsigned>(p.num_entries)),
                     dim3(256), 0, st, p);
  return hipGetLastError();
}

}  // namespace hcp
