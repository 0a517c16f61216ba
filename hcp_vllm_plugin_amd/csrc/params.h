// Kernel parameter blocks and launch functions shared between the kernel
// translation units and the extern "C" layer (abi.hip).
#pragma once

#include "common.h"

namespace hcp {

#ifndef HCP_FWD_WAVES
#define HCP_FWD_WAVES 4  // waves per prefill workgroup, 32 query rows each
#endif
constexpr int kFwdThreads = 64 * HCP_FWD_WAVES;
constexpr int kFwdBM = 32 * HCP_FWD_WAVES;  // query rows per prefill workgroup
constexpr int kFwdBN = 64;                  // keys per prefill tile
constexpr int kFwdPagedMinBlock = 16;      // paged prefill: rows a wave reads from one block

// Column width the attention kernels compute a head_dim in: 64, 128 or 256
// (a smaller head_dim, a multiple of 8, is zero-padded to it inside the
// kernels).
__host__ __device__ constexpr int padded_head_dim(int head_dim) {
  return head_dim <= 64 ? 64 : head_dim <= 128 ? 128 : 256;
}

struct FwdParams {
  const void* q;
  int64_t q_stride_tok, q_stride_head;
  void* out;
  int64_t o_stride_tok, o_stride_head;
  float* lse;
  int64_t lse_stride_head;
  const hcp_varlen_entry* entries;  // varlen: device array
  const int32_t* tiles;             // varlen: device (entry, q_block) pairs
  int32_t num_tiles;                // varlen: tiles; else query blocks
  int32_t num_heads, num_kv_heads, group;
  int32_t head_dim;  // valid elements per row (<= the kernel's width; the tail is padding)
  float scale_log2;
  int32_t window;           // causal only: key j visible iff j > qpos - window (0: none)
  hcp_varlen_entry single;  // non-varlen: the one entry
  // Optional partial state merged into the result (acc_o NULL: none).  Its
  // rows are indexed like out's; acc_prefix says which side of the merge it
  // is (1: prefix, this pass the suffix).  lse may then be NULL.
  const void* acc_o;
  int64_t acc_stride_tok, acc_stride_head;
  const float* acc_lse;
  int64_t acc_lse_stride_head;
  int32_t acc_prefix;
};

struct DecParams {
  const void* q;
  int64_t q_stride_tok, q_stride_head;
  const hcp_varlen_entry* entries;
  const hcp_decode_split* splits;
  int32_t num_splits;
  float* ws_o;    // [num_splits, H, D]
  float* ws_lse;  // [num_splits, H]
  int32_t num_heads, num_kv_heads, group;
  int32_t head_chunks;  // ceil(group / 16): workgroups per (split, KV head)
  int32_t head_dim;     // valid elements per row (<= the kernel's width)
  float scale_log2;
};

struct RedParams {
  const float* ws_o;
  const float* ws_lse;
  const int32_t* seq_partial_start;
  int32_t num_seqs;
  void* out;
  int64_t o_stride_tok, o_stride_head;
  float* lse;
  int64_t lse_stride_head;
  int32_t num_heads;
  int32_t head_dim;  // valid elements per row (<= the kernel's width)
  int32_t groups;    // 1, 2 or 4 column groups per (sequence, head), each over a share of the partials
  // optional running accumulator merged in as one more partial (NULL: none)
  const void* acc_o;
  int64_t acc_stride_tok, acc_stride_head;
  const float* acc_lse;
  int64_t acc_lse_stride_head;
};

struct MergeParams {
  void* out;
  int64_t o_stride_tok, o_stride_head;
  float* out_lse;
  int64_t out_lse_stride;
  const void* po;
  int64_t p_stride_tok, p_stride_head;
  const float* plse;
  int64_t p_lse_stride;
  const void* so;
  int64_t s_stride_tok, s_stride_head;
  const float* slse;
  int64_t s_lse_stride;
  int64_t num_tokens;
  int32_t num_heads, head_dim;
  int32_t out_dtype, p_dtype, s_dtype;
};

struct CacheParams {
  const void* key;
  int64_t k_stride_tok, k_stride_head;
  const void* value;
  int64_t v_stride_tok, v_stride_head;
  const void* slots;  // int32 or int64, one per token
  int64_t num_tokens;
  int32_t num_kv_heads;
  int32_t cpr;        // head_dim / 8: 16-byte chunks per row
  int32_t cpr_shift;  // log2(cpr) when cpr is a power of two, else -1
  void* k_cache;
  void* v_cache;
  int64_t stride_block, stride_head, stride_tok;
  int64_t num_slots;  // num_blocks * block_size
  int32_t bs_shift, bs_mask;
};

// Gather of paged KV segments into one contiguous [total, Hkv, D] K and V
// (prefill over caches with blocks shorter than a wave's 16 rows).
struct GatherParams {
  const hcp_varlen_entry* entries;  // device: paged segments
  const int64_t* out_start;         // device: first output token of each entry
  int64_t max_len;                  // longest segment
  int32_t num_entries;
  int32_t num_kv_heads;
  int32_t cpr;        // head_dim / 8: 16-byte chunks per row
  int32_t cpr_shift;  // log2(cpr) when cpr is a power of two, else -1
  int32_t head_dim;
  void* k_out;
  void* v_out;
};

hipError_t launch_fwd(const FwdParams& p, int head_dim, int dtype, bool causal,
                      bool paged, bool varlen, hipStream_t st);
hipError_t launch_decode(const DecParams& dp, const RedParams& rp, int head_dim,
                         int dtype, hipStream_t st);
hipError_t launch_merge(const MergeParams& p, hipStream_t st);
hipError_t launch_cache_write(const CacheParams& p, bool slots_i64, hipStream_t st);
hipError_t launch_gather(const GatherParams& p, hipStream_t st);

}  // namespace hcp
