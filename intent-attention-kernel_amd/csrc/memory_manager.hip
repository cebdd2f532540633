// KV memory manager kernels for gfx950 (MI355X): FP16 <-> INT8 page
// transcoding with the manager's own arithmetic, and the page warm-up of the
// block prefetcher.
//
// Reference semantics (src/intent_attention/kv_memory_manager.py):
//   demote, write_page's INT8 branch (:233-252):
//       max_abs = |page|.max() (a float16 value; NaN if any element is NaN)
//       scale   = max_abs / 127 if max_abs > 0 else 1.0
//       code    = clamp(round(float16(x / scale)), -128, 127)   (round half to even)
//   promote, _read_page_data's INT8 branch (:286-296):
//       x = float16(float32(code) * scale)
//   set_page_format (:268-284) is a promote or a demote of the page's data.
// The reference divides float16 values by a Python float scale on the CPU:
// float32(x) / float32(scale) rounded once to float16; its float32 scale is the
// correctly rounded quotient max_abs / 127, which is what this file computes
// (IEEE float32 division) and stores. A NaN quotient gives code 0.
//
// One wave per page, four pages per 256-thread workgroup. A lane handles
// 16-byte chunks lane, lane + 64, ... of its page. The demote holds pages of
// up to 4,096 elements in registers and reads them from HBM once (larger
// pages: two passes, the second mostly from the L2). Page data is streamed
// with non-temporal loads (demote) and stores (promote).
//
// Page warm-up (prefetch.py:111-170, launch_prefetch_pages :183-261): the K
// and V rows of the listed pages of every (batch, head) are read with plain
// cached loads, so the next step's decode finds them in the L2 / Infinity
// Cache; the words read are folded into a checksum so the loads stay.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "iak.h"
#include "iak_internal.h"
#include "iak_device.h"

namespace iak {

namespace {

constexpr int TC_WAVES = 4;

typedef uint32_t u2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ int64_t page_slot(const iak_transcode_args& a, int p) {
  return a.pages ? (int64_t)a.pages[p] : (int64_t)p;
}

// Codes of eight float16 values with page scale s: the float32 quotient x / s
// rounded once to float16, then to the nearest integer (ties to even).
// The quotient is Markstein's corrected product with r = 1 / s (IEEE, once per
// page): q0 = x r, e = fma(-q0, s, x), q = fma(e, r, q0); three operations in
// place of a float32 division. For every positive finite float16 absmax m and
// every float16 x with |x| <= m it gives the division's code (checked
// exhaustively on the host, 1,007,713,278 pairs); s = 1 (all-zero and NaN
// pages) makes it exact, and s = inf gives NaN or 0, both code 0, as x / inf.
__device__ __forceinline__ uint2 demote8(const u4 raw, const float s, const float r) {
  const h8 v = __builtin_bit_cast(h8, raw);
  uint32_t w[2] = {0u, 0u};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float x = (float)v[e];
    const float q0 = x * r;
    float q = __builtin_fmaf(__builtin_fmaf(-q0, s, x), r, q0);
    // q is rounded to float32 before float16 (two roundings, as the reference's
    // division); the empty asm keeps the compiler from fusing the fma and the
    // conversion into one mixed-precision fma rounded once to float16
    asm volatile("" : "+v"(q));
    const _Float16 q16 = (_Float16)q;
    float rr = __builtin_rintf((float)q16);
    rr = rr != rr ? 0.f : fminf(fmaxf(rr, -128.f), 127.f);
    w[e >> 2] |= ((uint32_t)(int32_t)rr & 0xFFu) << (8 * (e & 3));
  }
  return uint2{w[0], w[1]};
}

// |x| max of eight float16 values; NaN recorded in `nan` (fmaxf drops it).
__device__ __forceinline__ float absmax8(const u4 raw, float m, bool& nan) {
  const h8 v = __builtin_bit_cast(h8, raw);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float x = fabsf((float)v[e]);
    nan |= x != x;
    m = fmaxf(m, x);
  }
  return m;
}

__device__ __forceinline__ float page_scale(float m, bool nan) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  nan = __builtin_amdgcn_ballot_w64(nan) != 0;
  return (!nan && m > 0.f) ? m / 127.0f : 1.0f;     // IEEE float32 division
}

// Demote with the page held in registers: chunks lane + 64 i, i < MAXC, of
// pages of at most 64 * MAXC 16-byte chunks; every load is issued before the
// absmax reduction, and the page is read from HBM once.
template <int MAXC>
__global__ __launch_bounds__(64 * TC_WAVES) void transcode_demote_kernel(const iak_transcode_args a) {
  const int lane = threadIdx.x & 63;
  const int p = blockIdx.x * TC_WAVES + (threadIdx.x >> 6);
  if (p >= a.num_pages) return;                      // wave-uniform: no barriers below
  const int64_t slot = page_slot(a, p);
  if (slot < 0 || slot >= a.pool_pages) return;
  const int nch = a.page_elems / 8;                  // 8 float16 per 16-byte chunk
  const u4* src = reinterpret_cast<const u4*>(reinterpret_cast<const _Float16*>(a.fp16) + slot * a.page_elems);
  u4 v[MAXC];
#pragma unroll
  for (int i = 0; i < MAXC; ++i)
    v[i] = (lane + 64 * i < nch) ? __builtin_nontemporal_load(src + lane + 64 * i) : u4{0u, 0u, 0u, 0u};
  float m = 0.f;
  bool nan = false;
#pragma unroll
  for (int i = 0; i < MAXC; ++i) m = absmax8(v[i], m, nan);   // zero fill changes no max
  const float s = page_scale(m, nan);
  const float r = 1.0f / s;
  uint2* dst = reinterpret_cast<uint2*>(reinterpret_cast<int8_t*>(a.int8) + slot * a.page_elems);
#pragma unroll
  for (int i = 0; i < MAXC; ++i)
    if (lane + 64 * i < nch) dst[lane + 64 * i] = demote8(v[i], s, r);
  if (lane == 0) a.scales[slot] = s;
}

// Demote of larger pages: two passes over the page (absmax, then codes; the
// second pass mostly hits the L2).
__global__ __launch_bounds__(64 * TC_WAVES) void transcode_demote_2pass_kernel(const iak_transcode_args a) {
  const int lane = threadIdx.x & 63;
  const int p = blockIdx.x * TC_WAVES + (threadIdx.x >> 6);
  if (p >= a.num_pages) return;
  const int64_t slot = page_slot(a, p);
  if (slot < 0 || slot >= a.pool_pages) return;
  const int nch = a.page_elems / 8;
  const u4* src = reinterpret_cast<const u4*>(reinterpret_cast<const _Float16*>(a.fp16) + slot * a.page_elems);
  float m = 0.f;
  bool nan = false;
  for (int c = lane; c < nch; c += 64) m = absmax8(src[c], m, nan);
  const float s = page_scale(m, nan);
  const float r = 1.0f / s;
  uint2* dst = reinterpret_cast<uint2*>(reinterpret_cast<int8_t*>(a.int8) + slot * a.page_elems);
  for (int c = lane; c < nch; c += 64) dst[c] = demote8(src[c], s, r);
  if (lane == 0) a.scales[slot] = s;
}

// Eight float16 values float16(float32(code) * s) of eight codes.
__device__ __forceinline__ u4 promote8(const uint32_t lo, const uint32_t hi, const float s) {
  h8 v;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int code = (int)(int8_t)(((e < 4 ? lo : hi) >> (8 * (e & 3))) & 0xFFu);
    v[e] = (_Float16)((float)code * s);              // float32 product, one rounding to f16
  }
  return __builtin_bit_cast(u4, v);
}

// Promote: chunks of 8 codes (8-byte loads, 16-byte stores, so every store
// instruction of the wave writes 1 KiB contiguously); MAXC chunks per lane with
// every load issued before the first store, larger pages looped; codes read
// and pages written non-temporally.
template <int MAXC>
__global__ __launch_bounds__(64 * TC_WAVES) void transcode_promote_kernel(const iak_transcode_args a) {
  const int lane = threadIdx.x & 63;
  const int p = blockIdx.x * TC_WAVES + (threadIdx.x >> 6);
  if (p >= a.num_pages) return;
  const int64_t slot = page_slot(a, p);
  if (slot < 0 || slot >= a.pool_pages) return;
  const float s = a.scales[slot];
  const int nch = a.page_elems / 8;
  const u2v* src = reinterpret_cast<const u2v*>(reinterpret_cast<const int8_t*>(a.int8) + slot * a.page_elems);
  u4* dst = reinterpret_cast<u4*>(reinterpret_cast<_Float16*>(a.fp16) + slot * a.page_elems);
  for (int c0 = 0; c0 < nch; c0 += 64 * MAXC) {
    u2v x[MAXC];
#pragma unroll
    for (int i = 0; i < MAXC; ++i)
      x[i] = (c0 + lane + 64 * i < nch) ? __builtin_nontemporal_load(src + c0 + lane + 64 * i) : u2v{0u, 0u};
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
      const int c = c0 + lane + 64 * i;
      if (c < nch) __builtin_nontemporal_store(promote8(x[i][0], x[i][1], s), dst + c);
    }
  }
}

// One workgroup per (page list entry, batch, head); rows of the page past
// kv_len are skipped (the reference masks them). The 16-bit element at
// position i of the page (row-major over its rows) enters the checksum as
// value << (16 * (i & 1)), XOR-folded per wave; wave w of workgroup
// (entry, b * heads + h) writes word ((b * heads + h) * num_ids + entry) * 4 + w.
__global__ __launch_bounds__(256) void prefetch_pages_kernel(const iak_prefetch_args a) {
  const int entry = blockIdx.x;
  const int b = blockIdx.y / a.heads, h = blockIdx.y - (blockIdx.y / a.heads) * a.heads;
  const int page = a.page_ids[entry];
  const int64_t t0 = (int64_t)page * a.page_size;
  if (page < 0 || t0 >= a.kv_len) {                 // uniform per workgroup
    if ((threadIdx.x & 63) == 0) a.checksum[((int64_t)blockIdx.y * a.num_ids + entry) * 4 + (threadIdx.x >> 6)] = 0u;
    return;
  }
  const int rows = (int)((t0 + a.page_size <= a.kv_len) ? a.page_size : a.kv_len - t0);
  const int n = rows * a.head_dim;
  uint32_t x = 0u;
  for (int w = 0; w < 2; ++w) {
    const uint16_t* base = reinterpret_cast<const uint16_t*>(w ? a.v : a.k) +
                           (int64_t)b * (w ? a.v_stride_b : a.k_stride_b) +
                           (int64_t)h * (w ? a.v_stride_h : a.k_stride_h);
    const int64_t st = w ? a.v_stride_t : a.k_stride_t;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
      const int r = i / a.head_dim, d = i - r * a.head_dim;
      x ^= (uint32_t)base[(t0 + r) * st + d] << (16 * (i & 1));
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x ^= (uint32_t)__shfl_xor((int)x, off, 64);
  if ((threadIdx.x & 63) == 0)
    a.checksum[((int64_t)blockIdx.y * a.num_ids + entry) * 4 + (threadIdx.x >> 6)] = x;
}

}  // namespace

hipError_t launch_prefetch(const iak_prefetch_args& a, hipStream_t stream) {
  hipLaunchKernelGGL(prefetch_pages_kernel, dim3(a.num_ids, a.batch * a.heads), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_transcode(const iak_transcode_args& a, hipStream_t stream) {
  const int blocks = (a.num_pages + TC_WAVES - 1) / TC_WAVES;
  const int nch = a.page_elems / 8;
  if (a.mode == IAK_TRANSCODE_DEMOTE_INT8) {
    if (nch <= 64 * 4)
      hipLaunchKernelGGL(transcode_demote_kernel<4>, dim3(blocks), dim3(64 * TC_WAVES), 0, stream, a);
    else if (nch <= 64 * 8)
      hipLaunchKernelGGL(transcode_demote_kernel<8>, dim3(blocks), dim3(64 * TC_WAVES), 0, stream, a);
    else
      hipLaunchKernelGGL(transcode_demote_2pass_kernel, dim3(blocks), dim3(64 * TC_WAVES), 0, stream, a);
  } else {
    hipLaunchKernelGGL(transcode_promote_kernel<4>, dim3(blocks), dim3(64 * TC_WAVES), 0, stream, a);
  }
  return hipGetLastError();
}

}  // namespace iak
