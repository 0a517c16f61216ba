// LSE merge of two partial attention states (gfx950).
//
// out = (e^{lp} o_p + e^{ls} o_s) / (e^{lp} + e^{ls}), computed max-shifted,
// and optionally out_lse = log(e^{lp} + e^{ls}).  This is the operation of
// vLLM merge_attn_states as the reference calls it (ring_backend.py:349-354:
// prefix = peer, suffix = local; ring_decode.py:55-60 with the merged LSE)
// and of the torch fallback _lse_merge (ring_backend.py:409-421).
//
// HBM-bound elementwise work: each thread owns 8 contiguous head_dim elements
// of one (token, head), so every o load / store is one 16-byte (bf16/f16) or
// 32-byte (f32) access and a wave covers whole 256-byte rows.  The two LSE
// values are read once per (token, head) per thread group; they are tiny next
// to the o traffic (8 bytes per 3*D*2 bytes).
#include "params.h"

namespace hcp {

__device__ __forceinline__ void load8(const void* base, int dtype, float v[8]) {
  if (dtype == HCP_DTYPE_F32) {
    const f32x4* f = reinterpret_cast<const f32x4*>(base);
    f32x4 a = f[0], b = f[1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = a[i];
      v[4 + i] = b[i];
    }
  } else {
    u32x4 w = ldg16(base);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint16_t lo = static_cast<uint16_t>(w[i] & 0xffffu);
      const uint16_t hi = static_cast<uint16_t>(w[i] >> 16);
      if (dtype == HCP_DTYPE_BF16) {
        v[2 * i] = Elem<__bf16>::to_float(lo);
        v[2 * i + 1] = Elem<__bf16>::to_float(hi);
      } else {
        v[2 * i] = Elem<_Float16>::to_float(lo);
        v[2 * i + 1] = Elem<_Float16>::to_float(hi);
      }
    }
  }
}

__device__ __forceinline__ void store8(void* base, int dtype, const float v[8]) {
  if (dtype == HCP_DTYPE_F32) {
    f32x4* f = reinterpret_cast<f32x4*>(base);
    f[0] = f32x4{v[0], v[1], v[2], v[3]};
    f[1] = f32x4{v[4], v[5], v[6], v[7]};
  } else {
    u32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = dtype == HCP_DTYPE_BF16 ? pack2<__bf16>(v[2 * i], v[2 * i + 1])
                                     : pack2<_Float16>(v[2 * i], v[2 * i + 1]);
    *reinterpret_cast<u32x4*>(base) = w;
  }
}

__device__ __forceinline__ int dsize(int dtype) { return dtype == HCP_DTYPE_F32 ? 4 : 2; }

__global__ __launch_bounds__(256) void merge_kernel(MergeParams p) {
  const int chunks = p.head_dim / 8;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t total = p.num_tokens * p.num_heads * chunks;
  if (idx >= total) return;
  const int ch = static_cast<int>(idx % chunks);
  const int64_t th = idx / chunks;
  const int head = static_cast<int>(th % p.num_heads);
  const int64_t tok = th / p.num_heads;

  float lp = p.plse[head * p.p_lse_stride + tok];
  float ls = p.slse[head * p.s_lse_stride + tok];
  if (lp == INFINITY) lp = -INFINITY;
  if (ls == INFINITY) ls = -INFINITY;
  const float m = fmaxf(lp, ls);
  float out[8];
  float lse_out;
  if (m == -INFINITY) {
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = 0.f;
    lse_out = -INFINITY;
  } else {
    const float wp = __expf(lp - m), ws = __expf(ls - m);
    const float se = wp + ws;
    const float ps = wp / se, ss = ws / se;
    // a side with weight 0 (lse -inf, or far below the other) is not read,
    // so an unwritten partial never contributes
    float a[8] = {0, 0, 0, 0, 0, 0, 0, 0}, b[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (ps > 0.f)
      load8(static_cast<const char*>(p.po) +
                (tok * p.p_stride_tok + head * p.p_stride_head + ch * 8) * dsize(p.p_dtype),
            p.p_dtype, a);
    if (ss > 0.f)
      load8(static_cast<const char*>(p.so) +
                (tok * p.s_stride_tok + head * p.s_stride_head + ch * 8) * dsize(p.s_dtype),
            p.s_dtype, b);
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = __builtin_fmaf(a[i], ps, b[i] * ss);
    lse_out = m + __logf(se);
  }
  store8(static_cast<char*>(p.out) +
             (tok * p.o_stride_tok + head * p.o_stride_head + ch * 8) * dsize(p.out_dtype),
         p.out_dtype, out);
  if (p.out_lse != nullptr && ch == 0) p.out_lse[head * p.out_lse_stride + tok] = lse_out;
}

hipError_t launch_merge(const MergeParams& p, hipStream_t st) {
  const int64_t total = p.num_tokens * p.num_heads * (p.head_dim / 8);
  if (total == 0) return hipSuccess;
  const int64_t grid = (total + 255) / 256;
  hipLaunchKernelGGL(merge_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0, st, p);
  return hipGetLastError();
}

}  // namespace hcp
