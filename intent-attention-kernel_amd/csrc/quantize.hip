// Quantise-on-write for gfx950: float16 K/V pages -> the decode's page pools
// (codes + scales), bit-exact to the reference's arithmetic.
//
// Modes (iak_quantize_args.mode):
//   IAK_QUANT_FAKE_QUANTIZE  fake_quantize_tensor (src/intent_attention/intent_quant.py:221-312)
//       at the page granule (one scale per page; INT4: per page and group of
//       channels): scale = fl16(absmax / 127) (the clamp to 1e-8 is a no-op in
//       float16), q = fl16(x / scale), codes round-half-even(clamp(q, +-maxq))
//       with maxq 127 (INT8) / 7 (INT4); FP8 codes e4m3fn(q) (round to nearest
//       even); INT4_RESIDUAL: base codes with maxq 7, residual r = x - code *
//       scale in float32, s2 = max(fl32(absmax(r) / 127), 1e-8), residual
//       codes round-half-even(clamp(fl32(r / s2), +-7)).
//   IAK_QUANT_FUSED_INT8     fake_int8_pages_from_fp16 of the fused module
//       (fused_selected_quant_decode.py:521-542): float16, scale =
//       fl16(max(absmax, 1e-6) / 127), codes clamp(round(fl16(x / scale)), -128, 127).
//   IAK_QUANT_TRITON_INT8    the variant of triton_intent_quant_attention.py:460-496:
//       float32, scale = max(absmax, 1e-6) / 127, codes clamp(round(x / scale), +-127).
// A quotient 0/0 (an all-zero page) gives integer code 0 and e4m3fn code 0xFF,
// as the reference does on the host.
//
// One wave per page: lane = 4 * token + j holds channels (D/4) j .. (D/4) j + D/4 - 1
// of its token, so the page absmax is a wave reduction and a channel group of
// INT4 is a reduction over the lanes of one j (and its neighbours when a group
// spans more than D/4 channels).

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "iak.h"
#include "iak_internal.h"
#include "iak_device.h"

namespace iak {

__device__ __forceinline__ float wave_max(float v, int lo_bits) {
  // over the lanes that differ in bits 2..5 (the token), then in the low bits
  // 0 .. lo_bits-1 (neighbouring channel blocks of one group)
#pragma unroll
  for (int off = 4; off < 64; off <<= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  if (lo_bits > 0) v = fmaxf(v, __shfl_xor(v, 1, 64));
  if (lo_bits > 1) v = fmaxf(v, __shfl_xor(v, 2, 64));
  return v;
}

__device__ __forceinline__ float f16r(float x) { return (float)(_Float16)x; }   // round to float16

// float16 value -> e4m3fn code, round to nearest even; magnitudes that round
// above 448 are NaN (0x7F | sign); NaN keeps its sign bit.
__device__ __forceinline__ uint32_t e4m3fn_rne(float v) {
  const uint32_t bits = __builtin_bit_cast(uint32_t, v);
  const uint32_t sign = (bits >> 24) & 0x80u;
  const float a = fabsf(v);
  if (a != a) return sign | 0x7Fu;
  uint32_t code;
  if (a < 0.015625f) {                                  // below 2^-6: subnormal, quantum 2^-9
    code = (uint32_t)__builtin_rintf(a * 512.0f);       // 8 rounds up into the smallest normal
  } else {
    const uint32_t ab = __builtin_bit_cast(uint32_t, a);
    // keep 3 mantissa bits with round-half-even, then rebias 127 -> 7
    const uint32_t r = ab + 0x7FFFFu + ((ab >> 20) & 1u);
    code = (r >> 20) - ((127u - 7u) << 3);
    if (code > 0x7Eu) code = 0x7Fu;                     // above 448: NaN
  }
  return sign | code;
}

template <int D>
__global__ __launch_bounds__(256) void quantize_pages_kernel(const iak_quantize_args a) {
  constexpr int PER = D / 4;                  // channels per lane
  const int lane = threadIdx.x & 63;
  const int page = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (page >= a.num_pages) return;
  const int64_t dst = a.dst_pages ? (int64_t)a.dst_pages[page] : page;
  if (dst < 0 || dst >= a.pool_pages) return;
  const int tok = lane >> 2, j = lane & 3;

  // this lane's PER channels of its token
  const _Float16* src = reinterpret_cast<const _Float16*>(a.src) + ((int64_t)page * PS + tok) * D + PER * j;
  float x[PER];
#pragma unroll
  for (int i = 0; i < PER; i += 8) {
    const h8 v = *reinterpret_cast<const h8*>(src + i);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[i + e] = (float)v[e];
  }
  float am = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) am = fmaxf(am, fabsf(x[i]));

  const int prec = a.precision;
  uint8_t* codes = reinterpret_cast<uint8_t*>(a.codes);

  if (prec == IAK_TAG_INT4) {
    // group scale of this lane's channels; lanes per group = group / PER
    const int lpg = a.int4_group / PER;
    const float gam = wave_max(am, lpg >= 4 ? 2 : (lpg >= 2 ? 1 : 0));
    const float s = f16r(gam / 127.0f);
    uint32_t packed[PER / 8];
#pragma unroll
    for (int i = 0; i < PER / 8; ++i) packed[i] = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const float q = f16r(x[i] / s);
      const float r = (q != q) ? 0.f : __builtin_rintf(fminf(fmaxf(q, -7.f), 7.f));
      packed[i / 8] |= (uint32_t)((int)r + 8) << (4 * (i % 8));
    }
    uint32_t* cp = reinterpret_cast<uint32_t*>(codes + dst * PS * (D / 2) + tok * (D / 2) + (PER / 2) * j);
#pragma unroll
    for (int i = 0; i < PER / 8; ++i) cp[i] = packed[i];
    const int ng = D / a.int4_group;
    const int gi = (PER * j) / a.int4_group;
    if (tok == 0 && (PER * j) % a.int4_group == 0) {
      if (a.scale_dtype == IAK_DTYPE_F32) reinterpret_cast<float*>(a.scales)[dst * ng + gi] = s;
      else reinterpret_cast<_Float16*>(a.scales)[dst * ng + gi] = (_Float16)s;
    }
    return;
  }

  const float pam = wave_max(am, 2);
  uint32_t out[PER / 4];
#pragma unroll
  for (int i = 0; i < PER / 4; ++i) out[i] = 0;
  float s = 0.f, s2 = 0.f;

  if (a.mode == IAK_QUANT_FUSED_INT8) {
    s = f16r(f16r(fmaxf(pam, 1e-6f)) / 127.0f);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const float q = f16r(x[i] / s);   // 0/0 when the float16 scale underflows to 0
      const float r = (q != q) ? 0.f : fminf(fmaxf(__builtin_rintf(q), -128.f), 127.f);
      out[i / 4] |= ((uint32_t)(int)r & 0xFFu) << (8 * (i % 4));
    }
  } else if (a.mode == IAK_QUANT_TRITON_INT8) {
    s = fmaxf(pam, 1e-6f) / 127.0f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const float q = x[i] / s;
      const float r = (q != q) ? 0.f : fminf(fmaxf(__builtin_rintf(q), -127.f), 127.f);
      out[i / 4] |= ((uint32_t)(int)r & 0xFFu) << (8 * (i % 4));
    }
  } else if (prec == IAK_TAG_FP8) {
    s = f16r(pam / 127.0f);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      // 0/0 on the host is the negative default NaN -> code 0xFF
      const uint32_t cd = (s == 0.f && x[i] == 0.f) ? 0xFFu : e4m3fn_rne(f16r(x[i] / s));
      out[i / 4] |= cd << (8 * (i % 4));
    }
  } else if (prec == IAK_TAG_INT8) {
    s = f16r(pam / 127.0f);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const float q = f16r(x[i] / s);
      const float r = (q != q) ? 0.f : __builtin_rintf(fminf(fmaxf(q, -127.f), 127.f));
      out[i / 4] |= ((uint32_t)(int)r & 0xFFu) << (8 * (i % 4));
    }
  } else {   // INT4_RESIDUAL
    s = f16r(pam / 127.0f);
    float res[PER];
    int q1[PER];
    float ram = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const float q = f16r(x[i] / s);
      q1[i] = (q != q) ? 0 : (int)__builtin_rintf(fminf(fmaxf(q, -7.f), 7.f));
      res[i] = x[i] - (float)q1[i] * s;                 // float32, as the reference promotes
      ram = fmaxf(ram, fabsf(res[i]));
    }
    s2 = fmaxf(wave_max(ram, 2) / 127.0f, 1e-8f);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const float q = res[i] / s2;
      const int q2 = (q != q) ? 0 : (int)__builtin_rintf(fminf(fmaxf(q, -7.f), 7.f));
      out[i / 4] |= (uint32_t)((q1[i] + 8) | ((q2 + 8) << 4)) << (8 * (i % 4));
    }
  }

  uint32_t* cp = reinterpret_cast<uint32_t*>(codes + dst * PS * D + tok * D + PER * j);
#pragma unroll
  for (int i = 0; i < PER / 4; ++i) cp[i] = out[i];
  if (lane == 0) {
    if (prec == IAK_TAG_INT4_RESIDUAL && a.mode == IAK_QUANT_FAKE_QUANTIZE) {
      reinterpret_cast<float*>(a.scales)[2 * dst] = s;
      reinterpret_cast<float*>(a.scales)[2 * dst + 1] = s2;
    } else if (a.scale_dtype == IAK_DTYPE_F32) {
      reinterpret_cast<float*>(a.scales)[dst] = s;
    } else {
      reinterpret_cast<_Float16*>(a.scales)[dst] = (_Float16)s;
    }
  }
}

hipError_t launch_quantize_pages(const iak_quantize_args& a, hipStream_t stream) {
  const int blocks = (a.num_pages + 3) / 4;
  if (a.head_dim == 128) hipLaunchKernelGGL(quantize_pages_kernel<128>, dim3(blocks), dim3(256), 0, stream, a);
  else hipLaunchKernelGGL(quantize_pages_kernel<64>, dim3(blocks), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace iak
