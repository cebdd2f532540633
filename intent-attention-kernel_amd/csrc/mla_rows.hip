// Latent context of the reference's MLA decode API in float32, for gfx950.
//
// Reference semantics: the Triton kernel and CPU path of mla_decode_triton
// (src/intent_attention/triton_mla_decode.py:47-107 and _mla_decode_cpu
// :155-186): each (batch, query position) row attends to the latent rows of
// the pages its page table lists -- page p is rows p*page_size ..
// (p+1)*page_size - 1 of C [rows, d_c], the last page of C possibly shorter --
// with scores (q . c) * sm_scale in float32, an online softmax, and context =
// sum(p c) / sum(p); zeros when no row is visited. The projection by W_VO
// that follows is a plain GEMM outside this file.
//
// This is the reference API's arithmetic, not the serving path: the MFMA
// kernel of mla_decode.hip computes over paged f16 / FP8 / INT8 pools with f16
// operands, while this kernel keeps every product and sum in float32 over
// float32, float16 or bfloat16 inputs, any page size and any latent width up
// to 1,024 in one launch.
//
// One workgroup of four waves per row; wave w takes the table's pages w,
// w + 4, ... and keeps its own running max, denominator and context; lane l
// holds dims l, l + 64, ... of q and of the context, so a latent row is read by
// one coalesced load per 64 dims and used for both its score and its
// contribution. A row's score is a wave-wide sum. The four waves' states merge
// through the LDS at the end.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "iak.h"

namespace iak {

namespace {

constexpr int ROW_WAVES = 4;
constexpr int MAX_LATENT = 1024;

__device__ __forceinline__ float load_elem(const void* p, int64_t i, int dtype) {
  if (dtype == IAK_DTYPE_F32) return reinterpret_cast<const float*>(p)[i];
  if (dtype == IAK_DTYPE_F16) return (float)reinterpret_cast<const _Float16*>(p)[i];
  const uint32_t b = reinterpret_cast<const uint16_t*>(p)[i];
  return __builtin_bit_cast(float, b << 16);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// NPL: latent dims per lane (the row's width is at most 64 * NPL)
template <int NPL>
__global__ __launch_bounds__(64 * ROW_WAVES) void mla_rows_kernel(const iak_mla_rows_args a) {
  __shared__ float part_acc[ROW_WAVES][64 * NPL];
  __shared__ float part_m[ROW_WAVES], part_l[ROW_WAVES];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int row = blockIdx.x;   // b * q_len + t
  const int b = row / a.q_len, t = row - b * a.q_len;
  const int dc = a.latent_dim;

  float q[NPL], acc[NPL];
  const int64_t qoff = (int64_t)b * a.q_stride_b + (int64_t)t * a.q_stride_t;
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int d = lane + 64 * j;
    q[j] = d < dc ? load_elem(a.q, qoff + d, a.q_dtype) : 0.f;
    acc[j] = 0.f;
  }
  float m = -__builtin_inff(), l = 0.f;
  for (int i = w; i < a.num_selected; i += ROW_WAVES) {
    const int64_t p = a.page_ids[i];
    const int64_t r0 = p * a.page_size;
    if (p < 0 || r0 >= a.num_rows) continue;   // the host rejects such ids; nothing is read
    const int64_t r1 = r0 + a.page_size < a.num_rows ? r0 + a.page_size : a.num_rows;
    for (int64_t r = r0; r < r1; ++r) {
      float c[NPL];
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < NPL; ++j) {
        const int d = lane + 64 * j;
        c[j] = d < dc ? load_elem(a.latents, r * a.latent_stride + d, a.latent_dtype) : 0.f;
        s = __builtin_fmaf(q[j], c[j], s);
      }
      s = wave_sum(s) * a.sm_scale;
      if (s > m) {   // wave-uniform: every lane holds the same sum
        const float alpha = expf(m - s);   // 0 on the first row (m = -inf)
        l *= alpha;
#pragma unroll
        for (int j = 0; j < NPL; ++j) acc[j] *= alpha;
        m = s;
      }
      const float e = expf(s - m);
      l += e;
#pragma unroll
      for (int j = 0; j < NPL; ++j) acc[j] = __builtin_fmaf(e, c[j], acc[j]);
    }
  }

  if (lane == 0) {
    part_m[w] = m;
    part_l[w] = l;
  }
#pragma unroll
  for (int j = 0; j < NPL; ++j) part_acc[w][lane + 64 * j] = acc[j];
  __syncthreads();
  float M = -__builtin_inff();
#pragma unroll
  for (int k = 0; k < ROW_WAVES; ++k) M = fmaxf(M, part_m[k]);
  float wt[ROW_WAVES], L = 0.f;
#pragma unroll
  for (int k = 0; k < ROW_WAVES; ++k) {
    wt[k] = M > -__builtin_inff() ? expf(part_m[k] - M) : 0.f;   // 0 for a wave that saw no row
    L += wt[k] * part_l[k];
  }
  float* out = a.context + (int64_t)row * dc;
  for (int d = threadIdx.x; d < dc; d += 64 * ROW_WAVES) {
    float A = 0.f;
#pragma unroll
    for (int k = 0; k < ROW_WAVES; ++k) A = __builtin_fmaf(wt[k], part_acc[k][d], A);
    out[d] = L > 0.f ? A / L : 0.f;
  }
}

}  // namespace

hipError_t launch_mla_rows(const iak_mla_rows_args& a, hipStream_t stream) {
  const dim3 grid((unsigned)((int64_t)a.batch * a.q_len)), block(64 * ROW_WAVES);
  const int npl = (a.latent_dim + 63) / 64;
  if (npl <= 1) hipLaunchKernelGGL(mla_rows_kernel<1>, grid, block, 0, stream, a);
  else if (npl <= 2) hipLaunchKernelGGL(mla_rows_kernel<2>, grid, block, 0, stream, a);
  else if (npl <= 4) hipLaunchKernelGGL(mla_rows_kernel<4>, grid, block, 0, stream, a);
  else if (npl <= 9) hipLaunchKernelGGL(mla_rows_kernel<9>, grid, block, 0, stream, a);
  else hipLaunchKernelGGL(mla_rows_kernel<MAX_LATENT / 64>, grid, block, 0, stream, a);
  return hipGetLastError();
}

}  // namespace iak
