// extern "C" boundary of libhcp_mi355x.so: argument validation, host-side
// planners and kernel launches.  Declarations and their reference citations
// are in include/hcp_mi355x.h.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <numeric>
#include <vector>

#include "params.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int launch_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return HCP_OK;
  return fail(HCP_ELAUNCH, "%s: HIP launch failed: %s", what, hipGetErrorString(e));
}

bool dtype16(int32_t d) { return d == HCP_DTYPE_F16 || d == HCP_DTYPE_BF16; }

int check_heads(int32_t h, int32_t hkv, int32_t d, int32_t dtype, const char* who) {
  if (h <= 0 || hkv <= 0) return fail(HCP_EINVAL, "%s: num_heads/num_kv_heads must be > 0", who);
  if (h % hkv != 0)
    return fail(HCP_EINVAL, "%s: num_heads (%d) not a multiple of num_kv_heads (%d)", who, h, hkv);
  if (d < 8 || d > 256 || d % 8)
    return fail(HCP_EUNSUPPORTED, "%s: head_dim %d not supported (a multiple of 8 up to 256)",
                who, d);
  if (!dtype16(dtype)) return fail(HCP_EUNSUPPORTED, "%s: dtype %d not supported", who, dtype);
  return HCP_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7) == 0; }

int check_segment(const hcp_kv_segment& s, int32_t hd, const char* who, int idx) {
  if (s.len < 0 || s.start < 0) return fail(HCP_EINVAL, "%s: entry %d: negative kv start/len", who, idx);
  if (s.len > 0 && (s.k_addr == 0 || s.v_addr == 0))
    return fail(HCP_EINVAL, "%s: entry %d: null k/v address", who, idx);
  if ((s.k_addr & 15) || (s.v_addr & 15))
    return fail(HCP_EINVAL, "%s: entry %d: k/v address not 16-byte aligned", who, idx);
  if ((s.stride_tok % 8) || (s.stride_head % 8) || (s.block_table && (s.stride_block % 8)))
    return fail(HCP_EINVAL, "%s: entry %d: kv strides must be multiples of 8 elements", who, idx);
  if (s.block_table) {
    if (s.block_size <= 0 || (s.block_size & (s.block_size - 1)))
      return fail(HCP_EINVAL, "%s: entry %d: block_size %d not a power of two", who, idx,
                  s.block_size);
  }
  (void)hd;
  return HCP_OK;
}

// Optional partial state merged into an attention pass's result.
struct AccArgs {
  const void* o;
  int64_t stride_tok, stride_head;
  const float* lse;
  int64_t lse_stride_head;
  int32_t prefix;
};

int check_acc(const AccArgs& a, const char* who) {
  if (!a.o || !a.lse) return fail(HCP_EINVAL, "%s: null merge partial out/lse", who);
  if (!aligned16(a.o)) return fail(HCP_EINVAL, "%s: merge partial not 16-byte aligned", who);
  if ((a.stride_tok | a.stride_head) % 8)
    return fail(HCP_EINVAL, "%s: merge partial strides must be multiples of 8 elements", who);
  if (a.stride_tok <= 0 || a.stride_tok >= (int64_t{1} << 24))
    return fail(HCP_EUNSUPPORTED, "%s: merge partial token stride must be in (0, 2^24) elements",
                who);
  return HCP_OK;
}

void set_acc(hcp::FwdParams& p, const AccArgs* a) {
  if (!a) return;
  p.acc_o = a->o;
  p.acc_stride_tok = a->stride_tok;
  p.acc_stride_head = a->stride_head;
  p.acc_lse = a->lse;
  p.acc_lse_stride_head = a->lse_stride_head;
  p.acc_prefix = a->prefix != 0;
}

}  // namespace

extern "C" {

int hcp_abi_version(void) { return HCP_ABI_VERSION; }

const char* hcp_last_error(void) { return g_err; }

static int fwd_lse_impl(const char* who, const void* q, const void* k, const void* v, void* out,
                        float* lse, int64_t tq, int64_t tk, int32_t num_heads,
                        int32_t num_kv_heads, int32_t head_dim, int64_t q_stride_tok,
                        int64_t q_stride_head, int64_t k_stride_tok, int64_t k_stride_head,
                        int64_t v_stride_tok, int64_t v_stride_head, int64_t o_stride_tok,
                        int64_t o_stride_head, int64_t lse_stride_head, float scale,
                        int32_t causal, int64_t causal_offset, int32_t window, int32_t dtype,
                        void* stream, const AccArgs* acc) {
  int rc = check_heads(num_heads, num_kv_heads, head_dim, dtype, who);
  if (rc) return rc;
  if (tq < 0 || tk < 0) return fail(HCP_EINVAL, "%s: negative tq/tk", who);
  if (tq == 0) return HCP_OK;
  if (!q || !out || (!lse && !acc)) return fail(HCP_EINVAL, "%s: null q/out/lse", who);
  if (acc && (rc = check_acc(*acc, who))) return rc;
  if (tk > 0 && (!k || !v)) return fail(HCP_EINVAL, "%s: null k/v", who);
  if (!aligned16(q) || !aligned16(out) || (tk > 0 && (!aligned16(k) || !aligned16(v))))
    return fail(HCP_EINVAL, "%s: q/k/v/out must be 16-byte aligned", who);
  if ((q_stride_tok | q_stride_head | k_stride_tok | k_stride_head | v_stride_tok |
       v_stride_head | o_stride_tok | o_stride_head) % 8)
    return fail(HCP_EINVAL, "%s: strides must be multiples of 8 elements", who);
  if (!(scale > 0.f) || !std::isfinite(scale))
    return fail(HCP_EINVAL, "%s: scale must be finite and > 0", who);
  if (tq > (int64_t)INT32_MAX * 64) return fail(HCP_EINVAL, "%s: tq too large", who);
  // the kernel counts a segment's keys (and its tiles' key offsets) in int32
  if (tk > (int64_t)INT32_MAX - 256) return fail(HCP_EUNSUPPORTED, "%s: tk too large", who);
  if (window < 0) return fail(HCP_EINVAL, "%s: negative window", who);

  hcp::FwdParams p{};
  p.q = q;
  p.q_stride_tok = q_stride_tok;
  p.q_stride_head = q_stride_head;
  p.out = out;
  p.o_stride_tok = o_stride_tok;
  p.o_stride_head = o_stride_head;
  p.lse = lse;
  p.lse_stride_head = lse_stride_head;
  p.num_heads = num_heads;
  p.num_kv_heads = num_kv_heads;
  p.group = num_heads / num_kv_heads;
  p.head_dim = head_dim;
  p.scale_log2 = scale * hcp::kLog2e;
  p.num_tiles = static_cast<int32_t>((tq + hcp::kFwdBM - 1) / hcp::kFwdBM);
  p.single.q_start = 0;
  p.single.q_len = tq;
  p.single.causal_offset = causal ? causal_offset : 0;
  p.window = causal ? window : 0;
  p.single.kv.k_addr = reinterpret_cast<uint64_t>(k);
  p.single.kv.v_addr = reinterpret_cast<uint64_t>(v);
  p.single.kv.stride_tok = k_stride_tok;
  p.single.kv.stride_head = k_stride_head;
  p.single.kv.len = tk;
  if (k_stride_tok != v_stride_tok || k_stride_head != v_stride_head)
    return fail(HCP_EUNSUPPORTED, "%s: k and v must share strides", who);
  // the kernel's tile offsets are 32-bit: 64 rows of a tile span under 2^31
  // bytes (a single key row is never stepped over)
  if (tk > 1 && (k_stride_tok <= 0 || k_stride_tok >= (int64_t{1} << 24)))
    return fail(HCP_EUNSUPPORTED, "%s: k/v token stride must be in (0, 2^24) elements", who);
  set_acc(p, acc);
  hipError_t e = hcp::launch_fwd(p, head_dim, dtype, causal != 0, false, false,
                                 static_cast<hipStream_t>(stream));
  return launch_status(e, who);
}

int hcp_attn_fwd_lse(const void* q, const void* k, const void* v, void* out, float* lse,
                     int64_t tq, int64_t tk, int32_t num_heads, int32_t num_kv_heads,
                     int32_t head_dim, int64_t q_stride_tok, int64_t q_stride_head,
                     int64_t k_stride_tok, int64_t k_stride_head, int64_t v_stride_tok,
                     int64_t v_stride_head, int64_t o_stride_tok, int64_t o_stride_head,
                     int64_t lse_stride_head, float scale, int32_t causal,
                     int64_t causal_offset, int32_t window, int32_t dtype, void* stream) {
  return fwd_lse_impl("hcp_attn_fwd_lse", q, k, v, out, lse, tq, tk, num_heads, num_kv_heads,
                      head_dim, q_stride_tok, q_stride_head, k_stride_tok, k_stride_head,
                      v_stride_tok, v_stride_head, o_stride_tok, o_stride_head, lse_stride_head,
                      scale, causal, causal_offset, window, dtype, stream, nullptr);
}

int hcp_attn_fwd_lse_merge(const void* q, const void* k, const void* v, void* out, float* lse,
                           int64_t tq, int64_t tk, int32_t num_heads, int32_t num_kv_heads,
                           int32_t head_dim, int64_t q_stride_tok, int64_t q_stride_head,
                           int64_t k_stride_tok, int64_t k_stride_head, int64_t v_stride_tok,
                           int64_t v_stride_head, int64_t o_stride_tok, int64_t o_stride_head,
                           int64_t lse_stride_head, float scale, int32_t causal,
                           int64_t causal_offset, int32_t window, const void* acc_out,
                           int64_t acc_stride_tok, int64_t acc_stride_head,
                           const float* acc_lse, int64_t acc_lse_stride_head,
                           int32_t acc_is_prefix, int32_t dtype, void* stream) {
  const AccArgs acc{acc_out, acc_stride_tok, acc_stride_head, acc_lse, acc_lse_stride_head,
                    acc_is_prefix};
  return fwd_lse_impl("hcp_attn_fwd_lse_merge", q, k, v, out, lse, tq, tk, num_heads,
                      num_kv_heads, head_dim, q_stride_tok, q_stride_head, k_stride_tok,
                      k_stride_head, v_stride_tok, v_stride_head, o_stride_tok, o_stride_head,
                      lse_stride_head, scale, causal, causal_offset, window, dtype, stream, &acc);
}

int hcp_varlen_block_m(int32_t head_dim, int32_t dtype) {
  (void)head_dim;
  (void)dtype;
  return hcp::kFwdBM;
}

int hcp_plan_varlen_tiles(const hcp_varlen_entry* entries, int32_t num_entries, int32_t causal,
                          int32_t block_m, int32_t* tiles_out, int32_t cap) {
  const char* who = "hcp_plan_varlen_tiles";
  if (num_entries < 0 || block_m <= 0) return fail(HCP_EINVAL, "%s: bad sizes", who);
  if (num_entries > 0 && !entries) return fail(HCP_EINVAL, "%s: null entries", who);
  struct T {
    int64_t cost;
    int32_t e, qb;
  };
  std::vector<T> v;
  for (int32_t i = 0; i < num_entries; ++i) {
    const hcp_varlen_entry& en = entries[i];
    if (en.q_len < 0 || en.kv.len < 0) return fail(HCP_EINVAL, "%s: entry %d negative", who, i);
    // the kernel counts a segment's keys (and its tiles' key offsets) in int32
    if (en.kv.len > (int64_t)INT32_MAX - 256)
      return fail(HCP_EUNSUPPORTED, "%s: entry %d: kv len too large", who, i);
    // the prefill kernel reads a wave's 16 rows of a paged tile from one block
    if (en.kv.block_table && (en.kv.stride_tok <= 0 || en.kv.stride_tok >= (int64_t{1} << 24)))
      return fail(HCP_EUNSUPPORTED, "%s: entry %d: paged token stride must be in (0, 2^24)", who, i);
    if (!en.kv.block_table && en.kv.len > 1 &&
        (en.kv.stride_tok <= 0 || en.kv.stride_tok >= (int64_t{1} << 24)))
      return fail(HCP_EUNSUPPORTED, "%s: entry %d: token stride must be in (0, 2^24)", who, i);
    if (en.kv.block_table && (en.kv.stride_block <= 0 || en.kv.stride_block >= (int64_t{1} << 31)))
      return fail(HCP_EUNSUPPORTED, "%s: entry %d: block stride must be in (0, 2^31) elements",
                  who, i);
    // the kernel's in-block byte offsets are 32-bit
    if (en.kv.block_table &&
        static_cast<int64_t>(en.kv.block_size) * en.kv.stride_tok * 2 > (int64_t{1} << 32))
      return fail(HCP_EUNSUPPORTED, "%s: entry %d: block_size * token stride spans over 4 GiB",
                  who, i);
    if (en.kv.block_table && en.kv.block_size < hcp::kFwdPagedMinBlock)
      return fail(HCP_EUNSUPPORTED, "%s: entry %d: paged prefill needs block_size >= %d, got %d",
                  who, i, hcp::kFwdPagedMinBlock, en.kv.block_size);
    const int64_t nqb = (en.q_len + block_m - 1) / block_m;
    for (int64_t b = 0; b < nqb; ++b) {
      int64_t keys = en.kv.len;
      if (causal) {
        const int64_t lim = en.causal_offset + (b + 1) * block_m;
        keys = std::max<int64_t>(0, std::min(keys, lim));
      }
      v.push_back({keys, i, static_cast<int32_t>(b)});
    }
  }
  if (static_cast<int64_t>(v.size()) > INT32_MAX) return fail(HCP_EINVAL, "%s: too many tiles", who);
  const int32_t n = static_cast<int32_t>(v.size());
  if (n > cap || (n > 0 && !tiles_out))
    return fail(HCP_EWORKSPACE, "%s: need %d tiles, cap %d", who, n, cap);
  // longest processing time first; ties keep (entry, block) order
  std::stable_sort(v.begin(), v.end(), [](const T& a, const T& b) { return a.cost > b.cost; });
  for (int32_t i = 0; i < n; ++i) {
    tiles_out[2 * i] = v[i].e;
    tiles_out[2 * i + 1] = v[i].qb;
  }
  return n;
}

static int fwd_varlen_impl(const char* who, const void* q, int64_t q_stride_tok,
                           int64_t q_stride_head, void* out, int64_t o_stride_tok,
                           int64_t o_stride_head, float* lse, int64_t lse_stride_head,
                           const hcp_varlen_entry* entries, int32_t num_entries,
                           const int32_t* tiles, int32_t num_tiles, int32_t num_heads,
                           int32_t num_kv_heads, int32_t head_dim, float scale, int32_t causal,
                           int32_t window, int32_t paged, int32_t dtype, void* stream,
                           const AccArgs* acc) {
  int rc = check_heads(num_heads, num_kv_heads, head_dim, dtype, who);
  if (rc) return rc;
  if (num_entries < 0 || num_tiles < 0) return fail(HCP_EINVAL, "%s: negative counts", who);
  if (num_tiles == 0) return HCP_OK;
  if (!q || !out || (!lse && !acc) || !entries || !tiles)
    return fail(HCP_EINVAL, "%s: null pointer", who);
  if (acc && (rc = check_acc(*acc, who))) return rc;
  if (!aligned16(q) || !aligned16(out)) return fail(HCP_EINVAL, "%s: q/out not 16-byte aligned", who);
  if ((q_stride_tok | q_stride_head | o_stride_tok | o_stride_head) % 8)
    return fail(HCP_EINVAL, "%s: strides must be multiples of 8 elements", who);
  if (!(scale > 0.f) || !std::isfinite(scale))
    return fail(HCP_EINVAL, "%s: scale must be finite and > 0", who);
  if (window < 0) return fail(HCP_EINVAL, "%s: negative window", who);
  hcp::FwdParams p{};
  p.window = causal ? window : 0;
  p.q = q;
  p.q_stride_tok = q_stride_tok;
  p.q_stride_head = q_stride_head;
  p.out = out;
  p.o_stride_tok = o_stride_tok;
  p.o_stride_head = o_stride_head;
  p.lse = lse;
  p.lse_stride_head = lse_stride_head;
  p.entries = entries;
  p.tiles = tiles;
  p.num_tiles = num_tiles;
  p.num_heads = num_heads;
  p.num_kv_heads = num_kv_heads;
  p.group = num_heads / num_kv_heads;
  p.head_dim = head_dim;
  p.scale_log2 = scale * hcp::kLog2e;
  set_acc(p, acc);
  hipError_t e = hcp::launch_fwd(p, head_dim, dtype, causal != 0, paged != 0, true,
                                 static_cast<hipStream_t>(stream));
  return launch_status(e, who);
}

int hcp_attn_fwd_varlen(const void* q, int64_t q_stride_tok, int64_t q_stride_head, void* out,
                        int64_t o_stride_tok, int64_t o_stride_head, float* lse,
                        int64_t lse_stride_head, const hcp_varlen_entry* entries,
                        int32_t num_entries, const int32_t* tiles, int32_t num_tiles,
                        int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, float scale,
                        int32_t causal, int32_t window, int32_t paged, int32_t dtype,
                        void* stream) {
  return fwd_varlen_impl("hcp_attn_fwd_varlen", q, q_stride_tok, q_stride_head, out,
                         o_stride_tok, o_stride_head, lse, lse_stride_head, entries, num_entries,
                         tiles, num_tiles, num_heads, num_kv_heads, head_dim, scale, causal,
                         window, paged, dtype, stream, nullptr);
}

int hcp_attn_fwd_varlen_merge(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                              void* out, int64_t o_stride_tok, int64_t o_stride_head, float* lse,
                              int64_t lse_stride_head, const hcp_varlen_entry* entries,
                              int32_t num_entries, const int32_t* tiles, int32_t num_tiles,
                              int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                              float scale, int32_t causal, int32_t window, int32_t paged,
                              const void* acc_out, int64_t acc_stride_tok,
                              int64_t acc_stride_head, const float* acc_lse,
                              int64_t acc_lse_stride_head, int32_t acc_is_prefix, int32_t dtype,
                              void* stream) {
  const AccArgs acc{acc_out, acc_stride_tok, acc_stride_head, acc_lse, acc_lse_stride_head,
                    acc_is_prefix};
  return fwd_varlen_impl("hcp_attn_fwd_varlen_merge", q, q_stride_tok, q_stride_head, out,
                         o_stride_tok, o_stride_head, lse, lse_stride_head, entries, num_entries,
                         tiles, num_tiles, num_heads, num_kv_heads, head_dim, scale, causal,
                         window, paged, dtype, stream, &acc);
}

int hcp_plan_decode_splits(const hcp_varlen_entry* entries, int32_t num_entries,
                           const int32_t* entry_seq, int32_t num_seqs, int32_t causal,
                           int32_t split_tokens, hcp_decode_split* splits_out, int32_t cap,
                           int32_t* seq_partial_start) {
  const char* who = "hcp_plan_decode_splits";
  if (num_entries < 0 || num_seqs < 0 || split_tokens <= 0)
    return fail(HCP_EINVAL, "%s: bad sizes", who);
  if ((num_entries > 0 && (!entries || !entry_seq)) || !seq_partial_start)
    return fail(HCP_EINVAL, "%s: null pointer", who);
  int32_t n = 0;
  int32_t cur = 0;
  seq_partial_start[0] = 0;
  for (int32_t i = 0; i < num_entries; ++i) {
    const int32_t s = entry_seq[i];
    if (s < 0 || s >= num_seqs || s < cur)
      return fail(HCP_EINVAL, "%s: entry %d: sequence %d out of order/range", who, i, s);
    if (entries[i].q_len != 1)
      return fail(HCP_EINVAL, "%s: entry %d: q_len must be 1 for decode", who, i);
    if (entries[i].kv.len < 0 || entries[i].kv.len > INT32_MAX)
      return fail(HCP_EINVAL, "%s: entry %d: kv len out of range", who, i);
    while (cur < s) seq_partial_start[++cur] = n;
    int64_t len = entries[i].kv.len;
    if (causal) len = std::max<int64_t>(0, std::min<int64_t>(len, entries[i].causal_offset + 1));
    // ceil(len / split_tokens) pieces of (nearly) equal size
    const int64_t pieces = (len + split_tokens - 1) / split_tokens;
    const int64_t step = pieces > 0 ? (len + pieces - 1) / pieces : 0;
    for (int64_t b = 0; b < len; b += step) {
      if (n >= cap || !splits_out) return fail(HCP_EWORKSPACE, "%s: split cap %d exceeded", who, cap);
      splits_out[n].entry = i;
      splits_out[n].key_begin = static_cast<int32_t>(b);
      splits_out[n].key_end = static_cast<int32_t>(std::min<int64_t>(len, b + step));
      splits_out[n].slot = n;
      ++n;
    }
  }
  while (cur < num_seqs) seq_partial_start[++cur] = n;
  // dispatch order: longest first, so the last workgroups of the launch are
  // the short splits and the machine drains evenly
  std::stable_sort(splits_out, splits_out + n, [](const hcp_decode_split& a,
                                                  const hcp_decode_split& b) {
    return a.key_end - a.key_begin > b.key_end - b.key_begin;
  });
  return n;
}

size_t hcp_decode_workspace_bytes(int32_t num_splits, int32_t num_heads, int32_t head_dim) {
  if (num_splits <= 0 || num_heads <= 0 || head_dim <= 0) return 0;
  head_dim = hcp::padded_head_dim(head_dim);  // partials keep the kernel's width
  const size_t n = static_cast<size_t>(num_splits) * num_heads;
  const size_t o = n * head_dim * sizeof(float);
  const size_t o_al = (o + 255) & ~static_cast<size_t>(255);
  return o_al + n * sizeof(float);
}

static int decode_impl(const char* who, const void* q, int64_t q_stride_tok,
                       int64_t q_stride_head, const hcp_varlen_entry* entries,
                       int32_t num_entries, const hcp_decode_split* splits, int32_t num_splits,
                       const int32_t* seq_partial_start, int32_t num_seqs, void* workspace,
                       size_t workspace_bytes, void* out, int64_t o_stride_tok,
                       int64_t o_stride_head, float* lse, int64_t lse_stride_head,
                       const void* acc_o, int64_t acc_stride_tok, int64_t acc_stride_head,
                       const float* acc_lse, int64_t acc_lse_stride_head, int32_t num_heads,
                       int32_t num_kv_heads, int32_t head_dim, float scale, int32_t dtype,
                       void* stream) {
  int rc = check_heads(num_heads, num_kv_heads, head_dim, dtype, who);
  if (rc) return rc;
  if (num_entries < 0 || num_splits < 0 || num_seqs < 0)
    return fail(HCP_EINVAL, "%s: negative counts", who);
  if (num_seqs == 0) return HCP_OK;
  if (!q || !out || !seq_partial_start || (num_splits > 0 && (!entries || !splits)))
    return fail(HCP_EINVAL, "%s: null pointer", who);
  if (!aligned16(q)) return fail(HCP_EINVAL, "%s: q not 16-byte aligned", who);
  if ((q_stride_tok | q_stride_head) % 8)
    return fail(HCP_EINVAL, "%s: q strides must be multiples of 8 elements", who);
  if (!(scale > 0.f) || !std::isfinite(scale))
    return fail(HCP_EINVAL, "%s: scale must be finite and > 0", who);
  const size_t need = hcp_decode_workspace_bytes(num_splits, num_heads, head_dim);
  if (num_splits > 0 && (!workspace || workspace_bytes < need))
    return fail(HCP_EWORKSPACE, "%s: workspace %zu bytes < %zu needed", who, workspace_bytes, need);
  if (workspace && !aligned16(workspace))
    return fail(HCP_EINVAL, "%s: workspace not 16-byte aligned", who);
  const size_t n = static_cast<size_t>(num_splits) * num_heads;
  const size_t o_al = (n * hcp::padded_head_dim(head_dim) * sizeof(float) + 255) &
                      ~static_cast<size_t>(255);
  hcp::DecParams dp{};
  dp.q = q;
  dp.q_stride_tok = q_stride_tok;
  dp.q_stride_head = q_stride_head;
  dp.entries = entries;
  dp.splits = splits;
  dp.num_splits = num_splits;
  dp.ws_o = static_cast<float*>(workspace);
  dp.ws_lse = reinterpret_cast<float*>(static_cast<char*>(workspace) + o_al);
  dp.num_heads = num_heads;
  dp.num_kv_heads = num_kv_heads;
  dp.group = num_heads / num_kv_heads;
  dp.head_chunks = (dp.group + 15) / 16;
  dp.head_dim = head_dim;
  dp.scale_log2 = scale * hcp::kLog2e;
  hcp::RedParams rp{};
  rp.ws_o = dp.ws_o;
  rp.ws_lse = dp.ws_lse;
  rp.seq_partial_start = seq_partial_start;
  rp.num_seqs = num_seqs;
  rp.out = out;
  rp.o_stride_tok = o_stride_tok;
  rp.o_stride_head = o_stride_head;
  rp.lse = lse;
  rp.lse_stride_head = lse_stride_head;
  rp.num_heads = num_heads;
  rp.head_dim = head_dim;
  rp.acc_o = acc_o;
  rp.acc_stride_tok = acc_stride_tok;
  rp.acc_stride_head = acc_stride_head;
  rp.acc_lse = acc_lse;
  rp.acc_lse_stride_head = acc_lse_stride_head;
  hipError_t e = hcp::launch_decode(dp, rp, head_dim, dtype, static_cast<hipStream_t>(stream));
  return launch_status(e, who);
}

int hcp_decode_splitkv(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                       const hcp_varlen_entry* entries, int32_t num_entries,
                       const hcp_decode_split* splits, int32_t num_splits,
                       const int32_t* seq_partial_start, int32_t num_seqs, void* workspace,
                       size_t workspace_bytes, void* out, int64_t o_stride_tok,
                       int64_t o_stride_head, float* lse, int64_t lse_stride_head,
                       int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, float scale,
                       int32_t dtype, void* stream) {
  return decode_impl("hcp_decode_splitkv", q, q_stride_tok, q_stride_head, entries,
                     num_entries, splits, num_splits, seq_partial_start, num_seqs, workspace,
                     workspace_bytes, out, o_stride_tok, o_stride_head, lse, lse_stride_head,
                     nullptr, 0, 0, nullptr, 0, num_heads, num_kv_heads, head_dim, scale,
                     dtype, stream);
}

int hcp_decode_splitkv_acc(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                           const hcp_varlen_entry* entries, int32_t num_entries,
                           const hcp_decode_split* splits, int32_t num_splits,
                           const int32_t* seq_partial_start, int32_t num_seqs,
                           void* workspace, size_t workspace_bytes, const void* acc_o,
                           int64_t acc_stride_tok, int64_t acc_stride_head,
                           const float* acc_lse, int64_t acc_lse_stride_head, void* out,
                           int64_t o_stride_tok, int64_t o_stride_head, float* lse,
                           int64_t lse_stride_head, int32_t num_heads, int32_t num_kv_heads,
                           int32_t head_dim, float scale, int32_t dtype, void* stream) {
  const char* who = "hcp_decode_splitkv_acc";
  if (!acc_o || !acc_lse) return fail(HCP_EINVAL, "%s: null accumulator", who);
  if (reinterpret_cast<uintptr_t>(acc_o) % 2)
    return fail(HCP_EINVAL, "%s: acc_o not 2-byte aligned", who);
  return decode_impl(who, q, q_stride_tok, q_stride_head, entries, num_entries, splits,
                     num_splits, seq_partial_start, num_seqs, workspace, workspace_bytes, out,
                     o_stride_tok, o_stride_head, lse, lse_stride_head, acc_o, acc_stride_tok,
                     acc_stride_head, acc_lse, acc_lse_stride_head, num_heads, num_kv_heads,
                     head_dim, scale, dtype, stream);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Allocation-free decode: the split partials live in this file-scope device
// array instead of a caller workspace.  In host code `scratch` names a
// host-side stand-in, not device memory: its per-device address comes from
// hipGetSymbolAddress (once per device, with that device current) and only
// that address is ever passed to a kernel.
// ---------------------------------------------------------------------------
static __device__ __align__(256) char scratch[HCP_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (resolved on the first
// call there).
int scratch_on_current_device(void** out, const char* who) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(HCP_ELAUNCH, "%s: hipGetDevice: %s", who, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(HCP_EUNSUPPORTED, "%s: device index %d beyond %d", who, dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(HCP_ELAUNCH, "%s: hipGetSymbolAddress(scratch) on device %d: %s", who, dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return HCP_OK;
}

}  // namespace

extern "C" {

int hcp_decode_splitkv_noalloc(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                               const hcp_varlen_entry* entries, int32_t num_entries,
                               const hcp_decode_split* splits, int32_t num_splits,
                               const int32_t* seq_partial_start, int32_t num_seqs, void* out,
                               int64_t o_stride_tok, int64_t o_stride_head, float* lse,
                               int64_t lse_stride_head, int32_t num_heads, int32_t num_kv_heads,
                               int32_t head_dim, float scale, int32_t dtype, void* stream) {
  const char* who = "hcp_decode_splitkv_noalloc";
  int rc = check_heads(num_heads, num_kv_heads, head_dim, dtype, who);
  if (rc) return rc;
  if (num_splits < 0 || num_seqs < 0) return fail(HCP_EINVAL, "%s: negative counts", who);
  const size_t need = hcp_decode_workspace_bytes(num_splits, num_heads, head_dim);
  if (need > HCP_NOALLOC_SCRATCH_BYTES)
    return fail(HCP_EWORKSPACE,
                "%s: %d splits x %d heads x head_dim %d need %zu bytes of partials; the "
                "library's fixed scratch holds %zu (use hcp_decode_splitkv with a workspace, "
                "or plan fewer splits)",
                who, num_splits, num_heads, head_dim, need,
                static_cast<size_t>(HCP_NOALLOC_SCRATCH_BYTES));
  void* ws = nullptr;
  if (num_splits > 0 && num_seqs > 0 && (rc = scratch_on_current_device(&ws, who))) return rc;
  return decode_impl(who, q, q_stride_tok, q_stride_head, entries, num_entries, splits,
                     num_splits, seq_partial_start, num_seqs, ws, HCP_NOALLOC_SCRATCH_BYTES, out,
                     o_stride_tok, o_stride_head, lse, lse_stride_head, nullptr, 0, 0, nullptr,
                     0, num_heads, num_kv_heads, head_dim, scale, dtype, stream);
}

int hcp_merge_attn_states(void* out, int64_t o_stride_tok, int64_t o_stride_head,
                          int32_t out_dtype, float* out_lse, int64_t out_lse_stride_head,
                          const void* prefix_out, int64_t p_stride_tok, int64_t p_stride_head,
                          int32_t prefix_dtype, const float* prefix_lse,
                          int64_t p_lse_stride_head, const void* suffix_out,
                          int64_t s_stride_tok, int64_t s_stride_head, int32_t suffix_dtype,
                          const float* suffix_lse, int64_t s_lse_stride_head,
                          int64_t num_tokens, int32_t num_heads, int32_t head_dim,
                          void* stream) {
  const char* who = "hcp_merge_attn_states";
  if (num_tokens < 0 || num_heads <= 0 || head_dim <= 0)
    return fail(HCP_EINVAL, "%s: bad sizes", who);
  if (head_dim % 8) return fail(HCP_EUNSUPPORTED, "%s: head_dim must be a multiple of 8", who);
  for (int32_t d : {out_dtype, prefix_dtype, suffix_dtype})
    if (d != HCP_DTYPE_F16 && d != HCP_DTYPE_BF16 && d != HCP_DTYPE_F32)
      return fail(HCP_EUNSUPPORTED, "%s: dtype %d not supported", who, d);
  if (num_tokens == 0) return HCP_OK;
  if (!out || !prefix_out || !suffix_out || !prefix_lse || !suffix_lse)
    return fail(HCP_EINVAL, "%s: null pointer", who);
  if (!aligned16(out) || !aligned16(prefix_out) || !aligned16(suffix_out))
    return fail(HCP_EINVAL, "%s: o tensors must be 16-byte aligned", who);
  if ((o_stride_tok | o_stride_head | p_stride_tok | p_stride_head | s_stride_tok |
       s_stride_head) % 8)
    return fail(HCP_EINVAL, "%s: strides must be multiples of 8 elements", who);
  if (num_tokens * num_heads * (head_dim / 8) > (int64_t)INT32_MAX * 256)
    return fail(HCP_EINVAL, "%s: too large", who);
  hcp::MergeParams p{};
  p.out = out;
  p.o_stride_tok = o_stride_tok;
  p.o_stride_head = o_stride_head;
  p.out_lse = out_lse;
  p.out_lse_stride = out_lse_stride_head;
  p.po = prefix_out;
  p.p_stride_tok = p_stride_tok;
  p.p_stride_head = p_stride_head;
  p.plse = prefix_lse;
  p.p_lse_stride = p_lse_stride_head;
  p.so = suffix_out;
  p.s_stride_tok = s_stride_tok;
  p.s_stride_head = s_stride_head;
  p.slse = suffix_lse;
  p.s_lse_stride = s_lse_stride_head;
  p.num_tokens = num_tokens;
  p.num_heads = num_heads;
  p.head_dim = head_dim;
  p.out_dtype = out_dtype;
  p.p_dtype = prefix_dtype;
  p.s_dtype = suffix_dtype;
  return launch_status(hcp::launch_merge(p, static_cast<hipStream_t>(stream)), who);
}

int hcp_reshape_and_cache(const void* key, int64_t k_stride_tok, int64_t k_stride_head,
                          const void* value, int64_t v_stride_tok, int64_t v_stride_head,
                          const void* slot_mapping, int32_t slot_dtype, int64_t num_tokens,
                          int32_t num_kv_heads, int32_t head_dim, const hcp_paged_cache* cache,
                          int32_t dtype, void* stream) {
  const char* who = "hcp_reshape_and_cache";
  if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0)
    return fail(HCP_EINVAL, "%s: bad sizes", who);
  if (head_dim % 8)
    return fail(HCP_EUNSUPPORTED, "%s: head_dim %d must be a multiple of 8", who, head_dim);
  if (!dtype16(dtype)) return fail(HCP_EUNSUPPORTED, "%s: dtype %d not supported", who, dtype);
  if (slot_dtype != HCP_DTYPE_I32 && slot_dtype != HCP_DTYPE_I64)
    return fail(HCP_EUNSUPPORTED, "%s: slot dtype %d (int32 or int64)", who, slot_dtype);
  if (!cache) return fail(HCP_EINVAL, "%s: null cache descriptor", who);
  const hcp_paged_cache& c = *cache;
  if (c.block_size <= 0 || (c.block_size & (c.block_size - 1)))
    return fail(HCP_EINVAL, "%s: block_size %d not a power of two", who, c.block_size);
  if (c.num_blocks < 0) return fail(HCP_EINVAL, "%s: negative num_blocks", who);
  if (num_tokens == 0 || c.num_blocks == 0) return HCP_OK;
  if (!key || !value || !slot_mapping || !c.k_addr || !c.v_addr)
    return fail(HCP_EINVAL, "%s: null pointer", who);
  if (!aligned16(key) || !aligned16(value) || (c.k_addr & 15) || (c.v_addr & 15))
    return fail(HCP_EINVAL, "%s: key/value/cache must be 16-byte aligned", who);
  if ((k_stride_tok | k_stride_head | v_stride_tok | v_stride_head | c.stride_block |
       c.stride_head | c.stride_tok) % 8)
    return fail(HCP_EINVAL, "%s: strides must be multiples of 8 elements", who);
  if (num_tokens * num_kv_heads > (int64_t)INT32_MAX * 16)
    return fail(HCP_EINVAL, "%s: too many rows", who);
  hcp::CacheParams p{};
  p.key = key;
  p.k_stride_tok = k_stride_tok;
  p.k_stride_head = k_stride_head;
  p.value = value;
  p.v_stride_tok = v_stride_tok;
  p.v_stride_head = v_stride_head;
  p.slots = slot_mapping;
  p.num_tokens = num_tokens;
  p.num_kv_heads = num_kv_heads;
  p.cpr = head_dim / 8;
  p.cpr_shift = (p.cpr & (p.cpr - 1)) ? -1 : 31 - __builtin_clz(static_cast<unsigned>(p.cpr));
  p.k_cache = reinterpret_cast<void*>(c.k_addr);
  p.v_cache = reinterpret_cast<void*>(c.v_addr);
  p.stride_block = c.stride_block;
  p.stride_head = c.stride_head;
  p.stride_tok = c.stride_tok;
  p.num_slots = c.num_blocks * c.block_size;
  p.bs_shift = 31 - __builtin_clz(static_cast<unsigned>(c.block_size));
  p.bs_mask = c.block_size - 1;
  (void)dtype;  // a 16-bit copy: the bytes are moved as they are
  return launch_status(hcp::launch_cache_write(p, slot_dtype == HCP_DTYPE_I64,
                                               static_cast<hipStream_t>(stream)),
                       who);
}

int hcp_gather_paged_kv(const hcp_varlen_entry* entries, int32_t num_entries,
                        const int64_t* out_start, int64_t max_len, int32_t num_kv_heads,
                        int32_t head_dim, int32_t dtype, void* k_out, void* v_out,
                        void* stream) {
  const char* who = "hcp_gather_paged_kv";
  if (num_entries < 0 || max_len < 0 || num_kv_heads <= 0 || head_dim <= 0)
    return fail(HCP_EINVAL, "%s: bad sizes", who);
  if (head_dim % 8 || head_dim > 256)
    return fail(HCP_EUNSUPPORTED, "%s: head_dim %d not supported (a multiple of 8 up to 256)",
                who, head_dim);
  if (!dtype16(dtype)) return fail(HCP_EUNSUPPORTED, "%s: dtype %d not supported", who, dtype);
  if (num_entries > 65535) return fail(HCP_EINVAL, "%s: more than 65535 entries", who);
  if (num_entries == 0 || max_len == 0) return HCP_OK;
  if (!entries || !out_start || !k_out || !v_out) return fail(HCP_EINVAL, "%s: null pointer", who);
  if (!aligned8(entries) || !aligned8(out_start) || !aligned16(k_out) || !aligned16(v_out))
    return fail(HCP_EINVAL, "%s: misaligned pointer", who);
  // one thread per 16-byte piece of a (token, head) row, 256 per workgroup:
  // the launch's grid.x (and grid.x * 256) must stay within 32 bits
  if (max_len * num_kv_heads * (head_dim / 8) > (int64_t{1} << 32) - 256)
    return fail(HCP_EINVAL, "%s: too many rows (max_len * num_kv_heads * head_dim / 8 >= 2^32)",
                who);
  hcp::GatherParams p{};
  p.entries = entries;
  p.out_start = out_start;
  p.max_len = max_len;
  p.num_entries = num_entries;
  p.num_kv_heads = num_kv_heads;
  p.cpr = head_dim / 8;
  p.cpr_shift = (p.cpr & (p.cpr - 1)) ? -1 : 31 - __builtin_clz(static_cast<unsigned>(p.cpr));
  p.head_dim = head_dim;
  p.k_out = k_out;
  p.v_out = v_out;
  (void)dtype;  // a 16-bit copy: the bytes are moved as they are
  return launch_status(hcp::launch_gather(p, static_cast<hipStream_t>(stream)), who);
}

}  // extern "C"
