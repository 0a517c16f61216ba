/*
 * hcp_mi355x.h -- C ABI of libhcp_mi355x.so, the MI355X (gfx950) kernels of the
 * HCP ring-attention hot path.
 *
 * Conventions shared by every entry point
 *   - All tensors are caller-owned device memory passed as raw pointers (or as
 *     64-bit device addresses inside descriptors).  The library never
 *     allocates device memory and keeps no pointer after a call returns; its
 *     only device memory is the fixed scratch array of
 *     hcp_decode_splitkv_noalloc, part of its code object.
 *   - Strides are in ELEMENTS of the tensor's own dtype.  The last dimension
 *     (head_dim) must be contiguous.
 *   - Every launch is asynchronous on `stream` (a hipStream_t, NULL = default
 *     stream).  No entry point synchronizes the device.
 *   - Return value: HCP_OK (0) or a negative hcp_status.  Nothing throws or
 *     aborts across this boundary; hcp_last_error() gives a thread-local text
 *     of the last failure on the calling thread.
 *   - Entry points are stateless and reentrant; they may be called from any
 *     host thread.
 *
 * Reference semantics (stark-sim/hcp-vllm-plugin):
 *   q [Tq, H, D], k/v [Tk, Hkv, D], out [Tq, H, D], lse [H, Tq] float32 natural
 *   log (hcp_vllm_plugin/ring_triton_attn.py:21-25); query head h reads KV head
 *   h / (H / Hkv) (ring_triton_attn.py:64); with causal masking key j is
 *   visible to query i iff j <= causal_offset + i (ring_triton_attn.py:95-108,
 *   ring_backend.py:391-399).  A query row with no visible key, including every
 *   row of an empty segment, gets out = 0 and lse = -inf.
 */
#ifndef HCP_MI355X_H
#define HCP_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HCP_ABI_VERSION 9

typedef enum hcp_status {
  HCP_OK = 0,
  HCP_EINVAL = -1,       /* bad argument: null pointer, negative size, H % Hkv != 0, ... */
  HCP_EUNSUPPORTED = -2, /* valid but not built: head_dim not a multiple of 8 up to 256, dtype, ... */
  HCP_ELAUNCH = -3,      /* the HIP runtime rejected a launch */
  HCP_EWORKSPACE = -4    /* caller workspace smaller than required */
} hcp_status;

typedef enum hcp_dtype {
  HCP_DTYPE_F16 = 0,
  HCP_DTYPE_BF16 = 1,
  HCP_DTYPE_F32 = 2, /* only for merge inputs/outputs */
  HCP_DTYPE_I32 = 3, /* index arrays (slot_mapping) */
  HCP_DTYPE_I64 = 4
} hcp_dtype;

/*
 * A key/value segment.  Contiguous form (block_table == 0): key token t of KV
 * head h is at k_addr + ((start + t) * stride_tok + h * stride_head) elements.
 * Paged form (block_table != 0): token index x = start + t lives in block
 * block_table[x / block_size] at offset x % block_size, i.e. at
 * k_addr + (blk * stride_block + h * stride_head + (x % block_size) * stride_tok).
 * The same strides describe the vLLM 0.31 layout [nb, Hkv, bs, 2*D]
 * (k_addr = cache, v_addr = cache + D, stride_block = Hkv*bs*2D,
 * stride_head = bs*2D, stride_tok = 2D; file_connector.py:13-16,175-179)
 * and the vLLM 0.23 layout [nb, 2, bs, Hkv, D] (v_addr = cache + bs*Hkv*D,
 * stride_block = 2*bs*Hkv*D, stride_head = D, stride_tok = Hkv*D;
 * ring_backend.py:601,617-624).  num_blocks (0: unknown) bounds the block ids
 * the kernels read: a larger id reads the cache's last block (or, for decode
 * over a cache under 4 GiB, zeros) instead of memory outside it.  Paged prefill
 * reads block_size >= 16 in place (hcp_plan_varlen_tiles checks it); smaller
 * blocks are first gathered contiguous with hcp_gather_paged_kv.
 */
typedef struct hcp_kv_segment {
  uint64_t k_addr;
  uint64_t v_addr;
  uint64_t block_table; /* device address of int32 block ids, 0 = contiguous */
  int64_t stride_tok;
  int64_t stride_head;
  int64_t stride_block;
  int64_t start;      /* first token of the segment inside its source */
  int64_t len;        /* number of keys in the segment (0 allowed) */
  int32_t block_size; /* power of two; ignored when contiguous */
  int32_t num_blocks; /* paged: blocks in the cache (ids must be below it), 0 = not given */
} hcp_kv_segment;

/*
 * One query range attending to one KV segment.  Query rows
 * [q_start, q_start + q_len) of q / out / lse.  For causal launches key j of
 * the segment is visible to query i iff j <= causal_offset + i; the offset is
 * the position of query 0 in the segment's own key frame
 * (ring_backend.py:376-377,825).
 */
typedef struct hcp_varlen_entry {
  int64_t q_start;
  int64_t q_len;
  int64_t causal_offset;
  hcp_kv_segment kv;
} hcp_varlen_entry;

/*
 * One decode work split: keys [key_begin, key_end) of entry `entry`.  Its
 * fp32 partial goes to workspace slot `slot`; the slots of sequence s are
 * seq_partial_start[s] .. seq_partial_start[s+1]-1, each used by exactly one
 * split.  Splits run in array order, so the array order is the dispatch
 * order and need not follow the slots.
 */
typedef struct hcp_decode_split {
  int32_t entry;
  int32_t key_begin;
  int32_t key_end;
  int32_t slot;
} hcp_decode_split;

int hcp_abi_version(void);
const char* hcp_last_error(void);

/*
 * Flash-attention forward with per-row LSE on contiguous q/k/v (one request,
 * one segment).  Replaces ring_attn_with_lse -> _ring_fwd_kernel,
 * hcp_vllm_plugin/ring_triton_attn.py:155-207 (and the torch fallback
 * _attn_with_lse, ring_backend.py:366-406).  causal = 0 is the peer
 * (non-causal) pass; causal = 1 with causal_offset is the local pass.
 * window > 0 (causal only, ignored otherwise): sliding window of
 * _attn_with_lse's `window` (ring_backend.py:372,397-398) -- query i at
 * position p = causal_offset + i sees keys j with p - window < j <= p; the
 * reference's Triton path has no window and falls back to torch for it
 * (:315-323).  window = 0: none.
 * dtype: HCP_DTYPE_F16 or HCP_DTYPE_BF16 for q/k/v/out.  head_dim: any
 * multiple of 8 up to 256 (the reference takes any head_dim, padding it to a
 * power of two with masked columns, ring_triton_attn.py:69-78,201; here the
 * kernels compute in 64, 128 or 256 columns whose tail they load as zeros and
 * never store).  The same holds for every attention entry point below.
 */
int hcp_attn_fwd_lse(const void* q, const void* k, const void* v, void* out,
                     float* lse, int64_t tq, int64_t tk, int32_t num_heads,
                     int32_t num_kv_heads, int32_t head_dim,
                     int64_t q_stride_tok, int64_t q_stride_head,
                     int64_t k_stride_tok, int64_t k_stride_head,
                     int64_t v_stride_tok, int64_t v_stride_head,
                     int64_t o_stride_tok, int64_t o_stride_head,
                     int64_t lse_stride_head, float scale, int32_t causal,
                     int64_t causal_offset, int32_t window, int32_t dtype,
                     void* stream);

/*
 * hcp_attn_fwd_lse with the LSE merge of its result and a partial state
 * (acc_out [tq, H, D] in `dtype`, acc_lse [H, tq] f32) done in the same
 * launch: out = merge(prefix, suffix), where the prefix is acc and the
 * suffix this pass if acc_is_prefix != 0, the other way round otherwise;
 * lse (may be NULL) receives the merged LSE.  Replaces one attention pass
 * plus the merge that follows it in HcpRingAttentionImpl.forward -- the
 * local pass with the peer result as the prefix, merge_attn_states(out,
 * o_peer, lse_peer, o_loc, lse_loc) (ring_backend.py:820-831,349-354) -- so
 * the pass's own output never goes through HBM.  The arithmetic is
 * hcp_merge_attn_states' on this pass's output rounded to `dtype`: the
 * result equals hcp_attn_fwd_lse followed by hcp_merge_attn_states bit for
 * bit.  An acc LSE of +inf counts as -inf; a side of weight 0 is not read.
 * out may alias acc_out and lse acc_lse (rows are read before they are
 * written, by the same thread).
 */
int hcp_attn_fwd_lse_merge(const void* q, const void* k, const void* v, void* out,
                           float* lse, int64_t tq, int64_t tk, int32_t num_heads,
                           int32_t num_kv_heads, int32_t head_dim,
                           int64_t q_stride_tok, int64_t q_stride_head,
                           int64_t k_stride_tok, int64_t k_stride_head,
                           int64_t v_stride_tok, int64_t v_stride_head,
                           int64_t o_stride_tok, int64_t o_stride_head,
                           int64_t lse_stride_head, float scale, int32_t causal,
                           int64_t causal_offset, int32_t window,
                           const void* acc_out, int64_t acc_stride_tok,
                           int64_t acc_stride_head, const float* acc_lse,
                           int64_t acc_lse_stride_head, int32_t acc_is_prefix,
                           int32_t dtype, void* stream);

/*
 * Query-block size (rows per tile) used by the varlen prefill kernel for this
 * head_dim / dtype; tiles are (entry, q_block) pairs in these units.
 */
int hcp_varlen_block_m(int32_t head_dim, int32_t dtype);

/*
 * Host-side tile planner for hcp_attn_fwd_varlen.  Reads `num_entries` host
 * entries, writes up to `cap` (entry, q_block) int32 pairs into host memory
 * `tiles_out`, heaviest tile first (longest-processing-time order), and
 * returns the number of tiles (or a negative status; HCP_EWORKSPACE if cap is
 * too small; HCP_EUNSUPPORTED for a paged entry with block_size < 16, since the
 * prefill kernel reads each 16-row share of a 64-key tile from one block, and
 * for strides its 32-bit tile offsets cannot address: a token stride of 2^24
 * elements or more, a block stride of 2^31 elements or more, or block_size *
 * token stride over 4 GiB).  Runs on the CPU only.
 */
int hcp_plan_varlen_tiles(const hcp_varlen_entry* entries, int32_t num_entries,
                          int32_t causal, int32_t block_m, int32_t* tiles_out,
                          int32_t cap);

/*
 * Batched (varlen) flash forward with LSE: one launch covers every entry of a
 * batch.  Replaces the per-request loop of HcpRingAttentionImpl.forward
 * (ring_backend.py:611-832) that gathers the paged local KV (:617-624) and
 * calls ring_attn_with_lse once per request and segment (:820-830).  The
 * paged form reads blocks in place, with no gather copy.  `entries` and
 * `tiles` are DEVICE arrays (tiles from hcp_plan_varlen_tiles).  All entries
 * of one launch share `causal`, `window` (as hcp_attn_fwd_lse, relative to
 * each entry's causal_offset) and the KV form (all paged or all contiguous,
 * `paged`).  out/lse rows are the entries' q rows.
 */
int hcp_attn_fwd_varlen(const void* q, int64_t q_stride_tok,
                        int64_t q_stride_head, void* out, int64_t o_stride_tok,
                        int64_t o_stride_head, float* lse,
                        int64_t lse_stride_head,
                        const hcp_varlen_entry* entries, int32_t num_entries,
                        const int32_t* tiles, int32_t num_tiles,
                        int32_t num_heads, int32_t num_kv_heads,
                        int32_t head_dim, float scale, int32_t causal,
                        int32_t window, int32_t paged, int32_t dtype,
                        void* stream);

/*
 * hcp_attn_fwd_varlen with the merge of hcp_attn_fwd_lse_merge: acc rows are
 * indexed like out's (the entries' q rows).  Replaces the batch's local pass
 * and final merge_attn_states(out, o_peer, lse_peer, o_loc, lse_loc) of
 * HcpRingAttentionImpl.forward (ring_backend.py:820-831) in one launch; rows
 * of the launch get merge(acc, this pass) exactly as the two-step path.
 */
int hcp_attn_fwd_varlen_merge(const void* q, int64_t q_stride_tok,
                              int64_t q_stride_head, void* out,
                              int64_t o_stride_tok, int64_t o_stride_head,
                              float* lse, int64_t lse_stride_head,
                              const hcp_varlen_entry* entries,
                              int32_t num_entries, const int32_t* tiles,
                              int32_t num_tiles, int32_t num_heads,
                              int32_t num_kv_heads, int32_t head_dim,
                              float scale, int32_t causal, int32_t window,
                              int32_t paged, const void* acc_out,
                              int64_t acc_stride_tok, int64_t acc_stride_head,
                              const float* acc_lse, int64_t acc_lse_stride_head,
                              int32_t acc_is_prefix, int32_t dtype,
                              void* stream);

/*
 * Host-side split planner for hcp_decode_splitkv.  Each entry is one query
 * token (q_len == 1) of sequence entry_seq[e]; entries of one sequence must be
 * adjacent.  Splits every entry's visible key range into ceil(len /
 * split_tokens) pieces of nearly equal size (each at most `split_tokens`
 * keys), writing `splits_out` (host) and
 * seq_partial_start[num_seqs + 1] (host): the partial slots of sequence s are
 * [seq_partial_start[s], seq_partial_start[s+1]), numbered in sequence order.
 * The splits are listed longest first (ties in sequence order), so the short
 * ones fill the end of the launch.  Returns the number of splits (or a
 * negative status).  A causal entry sees keys j <= causal_offset.
 */
int hcp_plan_decode_splits(const hcp_varlen_entry* entries,
                           int32_t num_entries, const int32_t* entry_seq,
                           int32_t num_seqs, int32_t causal,
                           int32_t split_tokens, hcp_decode_split* splits_out,
                           int32_t cap, int32_t* seq_partial_start);

/* Bytes of workspace hcp_decode_splitkv needs for `num_splits` partials
 * (kept at the kernel's 64-, 128- or 256-column width). */
size_t hcp_decode_workspace_bytes(int32_t num_splits, int32_t num_heads,
                                  int32_t head_dim);

/*
 * Split-KV decode.  Replaces, for a batch of single-token queries, the
 * per-request local pass, peer pass and merge of HcpRingAttentionImpl.forward
 * (ring_backend.py:611-832 with tq == 1; the local segment of the decode
 * branch :663-679) that launch the flash kernel with grid (H, 1).  Kernel 1
 * computes one fp32 (O, LSE) partial per split and query head, up to 16 query
 * heads of a KV group in one workgroup so K/V are read once (any group size:
 * a larger group runs in chunks of 16 heads, the reference's any-G head map
 * h / G of ring_triton_attn.py:64).  Kernel 2 merges every partial
 * of a sequence -- all splits of its local and peer segments -- into `out`
 * (dtype) and, when `lse` is not NULL, the merged LSE [H, num_seqs]
 * (ring_decode.py:46-61 semantics).  Output row of sequence s is row s.
 * An entry is paged iff its kv.block_table is non-zero, so one launch covers a
 * sequence's contiguous peer segment and its paged local segment.
 * `entries`, `splits`, `seq_partial_start` are DEVICE arrays.
 */
int hcp_decode_splitkv(const void* q, int64_t q_stride_tok,
                       int64_t q_stride_head, const hcp_varlen_entry* entries,
                       int32_t num_entries, const hcp_decode_split* splits,
                       int32_t num_splits, const int32_t* seq_partial_start,
                       int32_t num_seqs, void* workspace,
                       size_t workspace_bytes, void* out, int64_t o_stride_tok,
                       int64_t o_stride_head, float* lse,
                       int64_t lse_stride_head, int32_t num_heads,
                       int32_t num_kv_heads, int32_t head_dim, float scale,
                       int32_t dtype, void* stream);

/*
 * Split-KV decode merged into a running accumulator: the decode ring's step
 * on one node.  Replaces RingDecodeNode.handle_packet's partial over
 * cat(chunk snapshot, growth) and _merge_pair (ring_decode.py:224-237,
 * :46-61): the partials of every segment of sequence s and the accumulator
 * row (acc_o [num_seqs, H, D] in `dtype`, acc_lse [H, num_seqs] float32) are
 * merged in the second kernel -- no separate merge launch -- into `out` and,
 * when `lse` is not NULL, the merged LSE.  An accumulator LSE of -inf (or
 * +inf, read as empty as merge_attn_states does) contributes nothing.
 * `out` may be `acc_o` and `lse` may be `acc_lse` (in-place update).  Other
 * arguments as hcp_decode_splitkv.
 */
int hcp_decode_splitkv_acc(const void* q, int64_t q_stride_tok,
                           int64_t q_stride_head,
                           const hcp_varlen_entry* entries,
                           int32_t num_entries,
                           const hcp_decode_split* splits,
                           int32_t num_splits,
                           const int32_t* seq_partial_start,
                           int32_t num_seqs, void* workspace,
                           size_t workspace_bytes, const void* acc_o,
                           int64_t acc_stride_tok, int64_t acc_stride_head,
                           const float* acc_lse,
                           int64_t acc_lse_stride_head, void* out,
                           int64_t o_stride_tok, int64_t o_stride_head,
                           float* lse, int64_t lse_stride_head,
                           int32_t num_heads, int32_t num_kv_heads,
                           int32_t head_dim, float scale, int32_t dtype,
                           void* stream);

/*
 * Bytes of the library's own decode scratch on each GPU (the fp32 split
 * partials of hcp_decode_splitkv_noalloc): 16 MiB, i.e. up to 1161 splits at
 * 28 query heads and head_dim 128.
 */
#define HCP_NOALLOC_SCRATCH_BYTES (16u << 20)

/*
 * hcp_decode_splitkv without a caller workspace and without any allocation:
 * the split partials go to a fixed device array inside the library
 * (HCP_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends).  No
 * counterpart in the reference: it is for callers that cannot allocate --
 * code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  Arguments as hcp_decode_splitkv minus the workspace; a plan
 * whose hcp_decode_workspace_bytes exceeds HCP_NOALLOC_SCRATCH_BYTES is
 * rejected with HCP_EWORKSPACE before anything is launched.  Every call on a
 * GPU shares that GPU's scratch and leaves its partials there (nothing in it
 * needs to start at zero: each split writes its slot before the reduce reads
 * it), so calls that overlap on one GPU -- on different streams, or from
 * different threads without ordering -- race; calls on one stream do not.
 * The first call on a device (with that device current) resolves the array's
 * address there; later calls reuse it.
 */
int hcp_decode_splitkv_noalloc(const void* q, int64_t q_stride_tok,
                               int64_t q_stride_head,
                               const hcp_varlen_entry* entries,
                               int32_t num_entries,
                               const hcp_decode_split* splits,
                               int32_t num_splits,
                               const int32_t* seq_partial_start,
                               int32_t num_seqs, void* out,
                               int64_t o_stride_tok, int64_t o_stride_head,
                               float* lse, int64_t lse_stride_head,
                               int32_t num_heads, int32_t num_kv_heads,
                               int32_t head_dim, float scale, int32_t dtype,
                               void* stream);

/*
 * LSE merge of two partial attentions over disjoint key sets:
 *   out = (e^{lse_p} o_p + e^{lse_s} o_s) / (e^{lse_p} + e^{lse_s}),
 *   out_lse = log(e^{lse_p} + e^{lse_s})   (when out_lse != NULL).
 * Replaces vLLM merge_attn_states(output, prefix_output, prefix_lse,
 * suffix_output, suffix_lse[, output_lse]) as called at ring_backend.py:349-354
 * and ring_decode.py:55-58, the torch fallback _lse_merge
 * (ring_backend.py:409-421) and the LSE of _merge_pair (ring_decode.py:59-60).
 * o tensors [T, H, D] (any of f16 / bf16 / f32 each), lse [H, T] float32.
 * An input LSE of +inf counts as -inf; two -inf inputs give out = 0,
 * out_lse = -inf.
 */
int hcp_merge_attn_states(void* out, int64_t o_stride_tok,
                          int64_t o_stride_head, int32_t out_dtype,
                          float* out_lse, int64_t out_lse_stride_head,
                          const void* prefix_out, int64_t p_stride_tok,
                          int64_t p_stride_head, int32_t prefix_dtype,
                          const float* prefix_lse, int64_t p_lse_stride_head,
                          const void* suffix_out, int64_t s_stride_tok,
                          int64_t s_stride_head, int32_t suffix_dtype,
                          const float* suffix_lse, int64_t s_lse_stride_head,
                          int64_t num_tokens, int32_t num_heads,
                          int32_t head_dim, void* stream);

/*
 * A paged KV cache: token `off` of block `blk`, KV head `h` lives at
 * k_addr + (blk * stride_block + h * stride_head + off * stride_tok) elements
 * (same for V at v_addr).  vLLM 0.31 [nb, Hkv, bs, 2*D]: v_addr = k_addr + D,
 * stride_block = Hkv*bs*2D, stride_head = bs*2D, stride_tok = 2D
 * (file_connector.py:13-16); vLLM 0.23 [nb, 2, bs, Hkv, D]: v_addr = k_addr +
 * bs*Hkv*D, stride_block = 2*bs*Hkv*D, stride_head = D, stride_tok = Hkv*D
 * (ring_backend.py:601).  block_size is a power of two.
 */
typedef struct hcp_paged_cache {
  uint64_t k_addr;
  uint64_t v_addr;
  int64_t stride_block;
  int64_t stride_head;
  int64_t stride_tok;
  int64_t num_blocks;
  int32_t block_size;
  int32_t reserved;
} hcp_paged_cache;

/*
 * Paged KV-cache write: key/value rows t < num_tokens ([num_tokens, Hkv, D],
 * dtype) go to slot slot_mapping[t] = block * block_size + offset of the
 * cache.  Replaces the torch index assignment of do_kv_cache_update
 * (ring_backend.py:501-539; key_cache[block_idx, block_off] = key[:n]).  A
 * negative slot is a padding token and is skipped (vLLM reshape_and_cache
 * convention; the reference has no padding slots); a slot >= num_blocks *
 * block_size is skipped too.  slot_mapping is a DEVICE array of
 * HCP_DTYPE_I32 or HCP_DTYPE_I64; `cache` is a HOST pointer to the
 * descriptor.  head_dim must be a multiple of 8; rows and the cache must be
 * 16-byte aligned with strides that are multiples of 8 elements.
 */
int hcp_reshape_and_cache(const void* key, int64_t k_stride_tok,
                          int64_t k_stride_head, const void* value,
                          int64_t v_stride_tok, int64_t v_stride_head,
                          const void* slot_mapping, int32_t slot_dtype,
                          int64_t num_tokens, int32_t num_kv_heads,
                          int32_t head_dim, const hcp_paged_cache* cache,
                          int32_t dtype, void* stream);

/*
 * Gather of paged KV segments into contiguous K and V: entry e's keys
 * [kv.start, kv.start + kv.len) of its block frame become rows
 * out_start[e] .. out_start[e] + kv.len - 1 of k_out / v_out, each
 * [total, Hkv, head_dim] contiguous (token stride Hkv * head_dim).  The
 * reference gathers every request's local KV this way before attention
 * (ring_backend.py:617-624); here it serves only paged prefill over caches
 * with block_size < 16, whose blocks are shorter than the rows the prefill
 * kernel reads from one block (hcp_plan_varlen_tiles refuses those), and runs
 * the whole batch in one launch.  `entries` (paged: block_table != 0) and
 * `out_start` (int64) are DEVICE arrays; at most 65535 entries, none longer
 * than max_len; an entry that is not paged or whose block_size is not a
 * power of two is skipped (its rows are left as they were).  Block ids at or past kv.num_blocks (when given) are clamped
 * to the last block.  head_dim a multiple of 8 up to 256; k_out / v_out
 * 16-byte aligned.
 */
int hcp_gather_paged_kv(const hcp_varlen_entry* entries, int32_t num_entries,
                        const int64_t* out_start, int64_t max_len,
                        int32_t num_kv_heads, int32_t head_dim, int32_t dtype,
                        void* k_out, void* v_out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HCP_MI355X_H */
