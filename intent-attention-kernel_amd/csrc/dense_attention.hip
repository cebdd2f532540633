// Dense softmax attention of the reference's dense_attention() in float32, for gfx950.
//
// Reference semantics (src/intent_attention/reference.py:16-45):
//   scores = (q . k^T) * scale
//   causal, no positions:   scores += triu(-inf, diagonal=1)   (query i sees keys j <= i)
//   causal, kv positions:   scores[i, j] = -inf where i < original_kv_positions[j]
//   mask:                   scores += mask                      (an additive mask; bool adds 1.0)
//   out = softmax(scores) . v
// A row whose scores are all -inf is NaN (softmax of -inf everywhere), as in
// torch; an empty key set gives zeros (torch's matmul over an empty dim).
//
// The reference runs these as torch.matmul / softmax in the input dtype. Here
// every product and sum is float32 over float32, float16 or bfloat16 inputs,
// and the output is rounded once to the input dtype.
//
// One workgroup of four waves per (batch, query) row. Wave w takes keys
// 4w .. 4w + 3, then 4w + 16 .. 4w + 19, ...: four consecutive key rows per
// step, whose four wave-wide dot products are reduced together. Lane l holds
// dims l, l + 64, ... of q and of the context, so a key or value row is one
// coalesced load per 64 dims. Each wave keeps a running max, denominator and
// context; the four merge through the LDS at the end.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "iak.h"

namespace iak {

namespace {

constexpr int DENSE_WAVES = 4;
constexpr int KEYS_PER_STEP = 4;

__device__ __forceinline__ float load_elem(const void* p, int64_t i, int dtype) {
  if (dtype == IAK_DTYPE_F32) return reinterpret_cast<const float*>(p)[i];
  if (dtype == IAK_DTYPE_F16) return (float)reinterpret_cast<const _Float16*>(p)[i];
  const uint32_t b = reinterpret_cast<const uint16_t*>(p)[i];
  return __builtin_bit_cast(float, b << 16);
}

__device__ __forceinline__ float load_mask(const void* p, int64_t i, int dtype) {
  if (dtype == IAK_MASK_BOOL) return reinterpret_cast<const uint8_t*>(p)[i] ? 1.f : 0.f;
  return load_elem(p, i, dtype);
}

__device__ __forceinline__ void store_elem(void* p, int64_t i, int dtype, float x) {
  if (dtype == IAK_DTYPE_F32) {
    reinterpret_cast<float*>(p)[i] = x;
  } else if (dtype == IAK_DTYPE_F16) {
    reinterpret_cast<_Float16*>(p)[i] = (_Float16)x;
  } else {
    // bfloat16, round to nearest even (NaN kept quiet)
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    const uint32_t r = (u & 0x7fffffffu) > 0x7f800000u ? (u | 0x00400000u) : u + 0x7fffu + ((u >> 16) & 1u);
    reinterpret_cast<uint16_t*>(p)[i] = (uint16_t)(r >> 16);
  }
}

__device__ __forceinline__ float wave_sum(float v) {
  // butterfly: every lane ends with the same sum (each step adds a pair in both orders)
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// NPL: dims per lane (head_dim and v_dim are at most 64 * NPL)
template <int NPL>
__global__ __launch_bounds__(64 * DENSE_WAVES) void dense_attention_kernel(const iak_dense_attention_args a) {
  __shared__ float part_acc[DENSE_WAVES][64 * NPL];
  __shared__ float part_m[DENSE_WAVES], part_l[DENSE_WAVES];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t row = blockIdx.x;   // b * q_len + i
  const int64_t b = row / a.q_len;
  const int i = (int)(row - b * a.q_len);
  const float NEG_INF = -__builtin_inff();

  float q[NPL], acc[NPL];
  const int64_t qoff = b * a.q_stride_b + (int64_t)i * a.q_stride_t;
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int d = lane + 64 * j;
    q[j] = d < a.head_dim ? load_elem(a.q, qoff + d, a.dtype) : 0.f;
    acc[j] = 0.f;
  }
  const int64_t kb = b * a.k_stride_b, vb = b * a.v_stride_b;
  const int64_t mb = b * a.mask_stride_b + (int64_t)i * a.mask_stride_q;
  float m = NEG_INF, l = 0.f;
  for (int j0 = KEYS_PER_STEP * w; j0 < a.kv_len; j0 += KEYS_PER_STEP * DENSE_WAVES) {
    float s[KEYS_PER_STEP];
#pragma unroll
    for (int u = 0; u < KEYS_PER_STEP; ++u) {
      const int j = j0 + u;
      float t = 0.f;
      if (j < a.kv_len) {   // wave-uniform
        const int64_t ko = kb + (int64_t)j * a.k_stride_t;
#pragma unroll
        for (int jj = 0; jj < NPL; ++jj) {
          const int d = lane + 64 * jj;
          if (d < a.head_dim) t = __builtin_fmaf(q[jj], load_elem(a.k, ko + d, a.dtype), t);
        }
      }
      s[u] = t;
    }
#pragma unroll
    for (int u = 0; u < KEYS_PER_STEP; ++u) s[u] = wave_sum(s[u]);
    float smax = NEG_INF;
#pragma unroll
    for (int u = 0; u < KEYS_PER_STEP; ++u) {
      const int j = j0 + u;
      float x = s[u] * a.sm_scale;
      if (a.causal == IAK_CAUSAL_TRIU) {
        if (j > i) x += NEG_INF;                    // scores + triu(-inf, diagonal=1)
      } else if (a.causal == IAK_CAUSAL_POSITIONS) {
        if ((int64_t)i < a.kv_positions[j < a.kv_len ? j : 0]) x = NEG_INF;   // masked_fill(-inf)
      }
      if (a.mask) x += load_mask(a.mask, mb + (int64_t)(j < a.kv_len ? j : 0) * a.mask_stride_k, a.mask_dtype);
      if (j >= a.kv_len) x = NEG_INF;               // not a key: no mass
      s[u] = x;
      smax = fmaxf(smax, x);
    }
    const float mn = fmaxf(m, smax);
    if (mn > m) {   // wave-uniform
      const float alpha = expf(m - mn);   // 0 while nothing was seen (m = -inf)
      l *= alpha;
#pragma unroll
      for (int j = 0; j < NPL; ++j) acc[j] *= alpha;
      m = mn;
    }
#pragma unroll
    for (int u = 0; u < KEYS_PER_STEP; ++u) {
      const int j = j0 + u;
      if (j >= a.kv_len) break;
      // -inf scores take no mass (also when m is -inf); NaN scores poison l, as in softmax
      const float e = s[u] == NEG_INF ? 0.f : expf(s[u] - m);
      l += e;
      const int64_t vo = vb + (int64_t)j * a.v_stride_t;
#pragma unroll
      for (int jj = 0; jj < NPL; ++jj) {
        const int d = lane + 64 * jj;
        if (d < a.v_dim) acc[jj] = __builtin_fmaf(e, load_elem(a.v, vo + d, a.dtype), acc[jj]);
      }
    }
  }

  if (lane == 0) {
    part_m[w] = m;
    part_l[w] = l;
  }
#pragma unroll
  for (int j = 0; j < NPL; ++j) part_acc[w][lane + 64 * j] = acc[j];
  __syncthreads();
  float M = NEG_INF;
#pragma unroll
  for (int k = 0; k < DENSE_WAVES; ++k) M = fmaxf(M, part_m[k]);
  float wt[DENSE_WAVES], L = 0.f;
#pragma unroll
  for (int k = 0; k < DENSE_WAVES; ++k) {
    wt[k] = part_m[k] == NEG_INF ? 0.f : expf(part_m[k] - M);   // 0 for a wave that saw no mass
    L += wt[k] * part_l[k];
  }
  // all scores -inf: softmax is NaN everywhere; no keys at all: zeros
  const float empty = a.kv_len > 0 ? __builtin_nanf("") : 0.f;
  const int64_t ooff = b * a.out_stride_b + (int64_t)i * a.out_stride_t;
  for (int d = threadIdx.x; d < a.v_dim; d += 64 * DENSE_WAVES) {
    float A = 0.f;
#pragma unroll
    for (int k = 0; k < DENSE_WAVES; ++k) A = __builtin_fmaf(wt[k], part_acc[k][d], A);
    store_elem(a.out, ooff + d, a.dtype, M == NEG_INF ? empty : A / L);
  }
}

}  // namespace

hipError_t launch_dense_attention(const iak_dense_attention_args& a, hipStream_t stream) {
  const dim3 grid((unsigned)((int64_t)a.batch * a.q_len)), block(64 * DENSE_WAVES);
  const int width = a.head_dim > a.v_dim ? a.head_dim : a.v_dim;
  const int npl = (width + 63) / 64;
  if (npl <= 1) hipLaunchKernelGGL(dense_attention_kernel<1>, grid, block, 0, stream, a);
  else if (npl <= 2) hipLaunchKernelGGL(dense_attention_kernel<2>, grid, block, 0, stream, a);
  else if (npl <= 4) hipLaunchKernelGGL(dense_attention_kernel<4>, grid, block, 0, stream, a);
  else if (npl <= 8) hipLaunchKernelGGL(dense_attention_kernel<8>, grid, block, 0, stream, a);
  else hipLaunchKernelGGL(dense_attention_kernel<16>, grid, block, 0, stream, a);
  return hipGetLastError();
}

}  // namespace iak
