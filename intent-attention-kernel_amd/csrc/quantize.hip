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
// One wave per page, loaded as whole 1 KB runs: load i of lane l is the 16
// bytes at i * 1024 + 16 * l of the page, i.e. token i * TPL + l / LPT and
// channels 8 * (l % LPT) .. + 7 (TPL tokens per run, LPT lanes per token).
// The page absmax is a wave reduction; an INT4 channel group is a reduction
// over the lanes of one group position across all tokens. Codes go out the same
// way (8, or 4 for INT4, contiguous bytes per lane and token). Pages and codes
// use streaming loads and stores: each instruction covers whole lines and
// nothing is read twice (cfg3 pools 1,816 -> 1,729 us; streaming loads alone
// were slower, streaming stores alone faster).

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "iak.h"
#include "iak_internal.h"
#include "iak_device.h"

namespace iak {

// max over the lanes that differ from this one only in the bits of `mask`
__device__ __forceinline__ float wave_max(float v, int mask) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1)
    if (mask & off) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ __forceinline__ float f16r(float x) { return (float)(_Float16)x; }   // round to float16

// x / s for a float16 numerator and a float16 scale s > 0, from r = 1 / s: the
// product and one FMA correction. Its float16 rounding equals that of the IEEE
// float32 quotient for every finite float16 x and positive finite float16 s
// (checked exhaustively on the host, tests/native/f16_quotient_check.c);
// e == 0 means q0 * s == x exactly, which keeps the sign of a zero quotient.
__device__ __forceinline__ float div_by_scale(float x, float s, float r) {
  const float q0 = __fmul_rn(x, r);
  const float e = __builtin_fmaf(-q0, s, x);
  return e == 0.f ? q0 : __builtin_fmaf(e, r, q0);
}

// the quotients of a lane's values by a float16 scale; s == 0 (an all-zero or
// nearly zero page) keeps the IEEE division and its infinities and NaNs
template <int NL>
__device__ __forceinline__ void scale_quotients(const float (&x)[NL][8], float s, float (&q)[NL][8]) {
  if (s > 0.f) {
    const float r = 1.0f / s;
#pragma unroll
    for (int i = 0; i < NL; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) q[i][e] = div_by_scale(x[i][e], s, r);
  } else {
#pragma unroll
    for (int i = 0; i < NL; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) q[i][e] = x[i][e] / s;
  }
}

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

// KIND: the precision tag for IAK_QUANT_FAKE_QUANTIZE, or KIND_FUSED / KIND_TRITON
constexpr int KIND_FUSED = 16, KIND_TRITON = 17;

template <int D, int KIND>
__global__ __launch_bounds__(256) void quantize_pages_kernel(const iak_quantize_args a) {
  constexpr int NL = PS * D * 2 / 1024;       // 1 KB runs per page: 4 (D = 128) or 2 (D = 64)
  constexpr int LPT = D / 8;                  // lanes per token: 16 or 8
  constexpr int TPL = 64 / LPT;               // tokens per run: 4 or 8
  const int lane = threadIdx.x & 63;
  const int page = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (page >= a.num_pages) return;
  const int64_t dst = a.dst_pages ? (int64_t)a.dst_pages[page] : page;
  if (dst < 0 || dst >= a.pool_pages) return;
  const int c0 = 8 * (lane % LPT);            // first channel of this lane
  const int t0 = lane / LPT;                  // token of run 0; run i holds token t0 + TPL * i

  const _Float16* src = reinterpret_cast<const _Float16*>(a.src) + (int64_t)page * PS * D;
  float x[NL][8];
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const h8 v = ld_nt(reinterpret_cast<const h8*>(src + i * 512 + 8 * lane));
#pragma unroll
    for (int e = 0; e < 8; ++e) x[i][e] = (float)v[e];
  }
  float am = 0.f;
#pragma unroll
  for (int i = 0; i < NL; ++i)
#pragma unroll
    for (int e = 0; e < 8; ++e) am = fmaxf(am, fabsf(x[i][e]));

  uint8_t* codes = reinterpret_cast<uint8_t*>(a.codes);

  if constexpr (KIND == IAK_TAG_INT4) {
    // group = the lanes of one token whose channels share the group, over all tokens
    const int lpg = a.int4_group / 8;         // lanes per group within a token (>= LPT / 4 >= 2)
    const float gam = wave_max(am, (63 & ~(LPT - 1)) | (lpg - 1));
    const float s = f16r(gam / 127.0f);
    float qs[NL][8];
    scale_quotients(x, s, qs);
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      uint32_t packed = 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float q = f16r(qs[i][e]);
        const float r = (q != q) ? 0.f : __builtin_rintf(fminf(fmaxf(q, -7.f), 7.f));
        packed |= (uint32_t)((int)r + 8) << (4 * e);
      }
      st_nt(reinterpret_cast<uint32_t*>(codes + (dst * PS + t0 + TPL * i) * (D / 2) + c0 / 2), packed);
    }
    if (t0 == 0 && c0 % a.int4_group == 0) {
      const int ng = D / a.int4_group, gi = c0 / a.int4_group;
      if (a.scale_dtype == IAK_DTYPE_F32) reinterpret_cast<float*>(a.scales)[dst * ng + gi] = s;
      else reinterpret_cast<_Float16*>(a.scales)[dst * ng + gi] = (_Float16)s;
    }
    return;
  }

  const float pam = wave_max(am, 63);
  uint32_t out[NL][2];
#pragma unroll
  for (int i = 0; i < NL; ++i) out[i][0] = out[i][1] = 0;
  float s = 0.f, s2 = 0.f;

  if constexpr (KIND == KIND_FUSED) {
    s = f16r(f16r(fmaxf(pam, 1e-6f)) / 127.0f);
    float qs[NL][8];
    scale_quotients(x, s, qs);
#pragma unroll
    for (int i = 0; i < NL; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float q = f16r(qs[i][e]);      // 0/0 when the float16 scale underflows to 0
        const float r = (q != q) ? 0.f : fminf(fmaxf(__builtin_rintf(q), -128.f), 127.f);
        out[i][e / 4] |= ((uint32_t)(int)r & 0xFFu) << (8 * (e % 4));
      }
  } else if constexpr (KIND == KIND_TRITON) {
    s = fmaxf(pam, 1e-6f) / 127.0f;
#pragma unroll
    for (int i = 0; i < NL; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float q = x[i][e] / s;
        const float r = (q != q) ? 0.f : fminf(fmaxf(__builtin_rintf(q), -127.f), 127.f);
        out[i][e / 4] |= ((uint32_t)(int)r & 0xFFu) << (8 * (e % 4));
      }
  } else if constexpr (KIND == IAK_TAG_FP8) {
    s = f16r(pam / 127.0f);
    float qs[NL][8];
    scale_quotients(x, s, qs);
    if (s > 0.f) {
      // finite quotients, |q| <= 127 * (1 + 2^-11): the hardware's round-to-
      // nearest-even e4m3fn conversion, two codes per instruction
#pragma unroll
      for (int i = 0; i < NL; ++i)
#pragma unroll
        for (int w = 0; w < 2; ++w) {
          int v = __builtin_amdgcn_cvt_pk_fp8_f32(f16r(qs[i][4 * w]), f16r(qs[i][4 * w + 1]), 0, false);
          v = __builtin_amdgcn_cvt_pk_fp8_f32(f16r(qs[i][4 * w + 2]), f16r(qs[i][4 * w + 3]), v, true);
          out[i][w] = (uint32_t)v;
        }
    } else {
#pragma unroll
      for (int i = 0; i < NL; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          // 0/0 on the host is the negative default NaN -> code 0xFF
          const uint32_t cd = x[i][e] == 0.f ? 0xFFu : e4m3fn_rne(f16r(qs[i][e]));
          out[i][e / 4] |= cd << (8 * (e % 4));
        }
    }
  } else if constexpr (KIND == IAK_TAG_INT8) {
    s = f16r(pam / 127.0f);
    float qs[NL][8];
    scale_quotients(x, s, qs);
#pragma unroll
    for (int i = 0; i < NL; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float q = f16r(qs[i][e]);
        const float r = (q != q) ? 0.f : __builtin_rintf(fminf(fmaxf(q, -127.f), 127.f));
        out[i][e / 4] |= ((uint32_t)(int)r & 0xFFu) << (8 * (e % 4));
      }
  } else {   // INT4_RESIDUAL
    s = f16r(pam / 127.0f);
    float res[NL][8];
    int q1[NL][8];
    float ram = 0.f;
    float qs[NL][8];
    scale_quotients(x, s, qs);
#pragma unroll
    for (int i = 0; i < NL; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float q = f16r(qs[i][e]);
        q1[i][e] = (q != q) ? 0 : (int)__builtin_rintf(fminf(fmaxf(q, -7.f), 7.f));
        res[i][e] = x[i][e] - (float)q1[i][e] * s;      // float32, as the reference promotes
        ram = fmaxf(ram, fabsf(res[i][e]));
      }
    s2 = fmaxf(wave_max(ram, 63) / 127.0f, 1e-8f);
#pragma unroll
    for (int i = 0; i < NL; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float q = res[i][e] / s2;
        const int q2 = (q != q) ? 0 : (int)__builtin_rintf(fminf(fmaxf(q, -7.f), 7.f));
        out[i][e / 4] |= (uint32_t)((q1[i][e] + 8) | ((q2 + 8) << 4)) << (8 * (e % 4));
      }
  }

#pragma unroll
  for (int i = 0; i < NL; ++i) {
    u2 v;
    v[0] = out[i][0];
    v[1] = out[i][1];
    st_nt(reinterpret_cast<u2*>(codes + (dst * PS + t0 + TPL * i) * D + c0), v);
  }
  if (lane == 0) {
    if (KIND == IAK_TAG_INT4_RESIDUAL) {
      reinterpret_cast<float*>(a.scales)[2 * dst] = s;
      reinterpret_cast<float*>(a.scales)[2 * dst + 1] = s2;
    } else if (a.scale_dtype == IAK_DTYPE_F32) {
      reinterpret_cast<float*>(a.scales)[dst] = s;
    } else {
      reinterpret_cast<_Float16*>(a.scales)[dst] = (_Float16)s;
    }
  }
}

template <int D>
static hipError_t launch_d(const iak_quantize_args& a, hipStream_t stream) {
  const dim3 grid((a.num_pages + 3) / 4), block(256);
  if (a.mode == IAK_QUANT_FUSED_INT8)
    hipLaunchKernelGGL((quantize_pages_kernel<D, KIND_FUSED>), grid, block, 0, stream, a);
  else if (a.mode == IAK_QUANT_TRITON_INT8)
    hipLaunchKernelGGL((quantize_pages_kernel<D, KIND_TRITON>), grid, block, 0, stream, a);
  else if (a.precision == IAK_TAG_FP8)
    hipLaunchKernelGGL((quantize_pages_kernel<D, IAK_TAG_FP8>), grid, block, 0, stream, a);
  else if (a.precision == IAK_TAG_INT8)
    hipLaunchKernelGGL((quantize_pages_kernel<D, IAK_TAG_INT8>), grid, block, 0, stream, a);
  else if (a.precision == IAK_TAG_INT4)
    hipLaunchKernelGGL((quantize_pages_kernel<D, IAK_TAG_INT4>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((quantize_pages_kernel<D, IAK_TAG_INT4_RESIDUAL>), grid, block, 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_quantize_pages(const iak_quantize_args& a, hipStream_t stream) {
  return a.head_dim == 128 ? launch_d<128>(a, stream) : launch_d<64>(a, stream);
}

}  // namespace iak
