// Device helpers shared by the libiak kernels (selected-page decode and MLA
// latent decode): packed f16 conversions of quantised codes, lane-swap
// reductions and the split-K log-sum-exp merge.
#ifndef IAK_DEVICE_H
#define IAK_DEVICE_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "iak.h"
#include "iak_internal.h"

namespace iak {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

constexpr int PS = 16;
constexpr float RESCALE_SLACK = 8.0f;      // p <= 2^8 between rescales

// Value exponent. A page's V scale s multiplies the f16 P operand of the value
// product; on its own p * s leaves f16's normal range for small scales (V
// codes of tiny values: p * s in the subnormals) and large ones (overflow).
// Each wave therefore keeps its value accumulator as acc * 2^-E for a
// wave-uniform exponent E that follows the pages' scale exponents: P holds
// p * (s * 2^-E), and E moves (the accumulator rescaled by an exact power of
// two) only when a page's exponent leaves [E - EXP_WINDOW, E + EXP_WINDOW], so
// s * 2^-E stays in [2^-EXP_WINDOW, 2^(EXP_WINDOW + 1)). The result is acc * 2^E.
constexpr int EXP_WINDOW = 4;
constexpr int EXP_LIMIT = 60;              // |E| <= 60: every 2^(E1 - E2) is a finite float

// floor(log2(s)) of a scale, clamped to [-EXP_LIMIT, EXP_LIMIT] (zero and
// subnormal scales give -EXP_LIMIT, inf / NaN give EXP_LIMIT).
__device__ __forceinline__ int scale_exp(float s) {
  const int ef = (int)((__builtin_bit_cast(uint32_t, s) >> 23) & 0xFFu);
  const int e = ef - 127;
  return e < -EXP_LIMIT ? -EXP_LIMIT : (e > EXP_LIMIT ? EXP_LIMIT : e);
}
// 2^e as a float, for |e| <= 126.
__device__ __forceinline__ float pow2f(int e) { return __builtin_bit_cast(float, (uint32_t)(e + 127) << 23); }
constexpr uint32_t MAGIC_I8 = 0x64646464u;  // f16 0x64xx = 1024 + xx
constexpr uint32_t MAGIC_I4 = 0x64006400u;

__device__ __forceinline__ uint32_t bits(h2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }
__device__ __forceinline__ h2 splat2(_Float16 x) { return h2{x, x}; }

__device__ __forceinline__ h8 make_h8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  u4 v = {a, b, c, d};
  return __builtin_bit_cast(h8, v);
}
__device__ __forceinline__ h4 make_h4(uint32_t a, uint32_t b) {
  u2 v = {a, b};
  return __builtin_bit_cast(h4, v);
}

// (lo16(x), lo16(y)) and (hi16(x), hi16(y)) as one dword
__device__ __forceinline__ uint32_t pack_lo(uint32_t x, uint32_t y) {
  return __builtin_amdgcn_perm(y, x, 0x05040100u);
}
__device__ __forceinline__ uint32_t pack_hi(uint32_t x, uint32_t y) {
  return __builtin_amdgcn_perm(y, x, 0x07060302u);
}

// Four signed int8 -> two f16 pairs (b0,b1), (b2,b3), exactly.
__device__ __forceinline__ void i8x4_to_f16(uint32_t x, uint32_t& lo, uint32_t& hi) {
  const uint32_t u = x ^ 0x80808080u;                          // b + 128
  const h2 off = splat2((_Float16)-1152.0f);                   // 1024 + 128
  lo = bits(as_h2(__builtin_amdgcn_perm(MAGIC_I8, u, 0x04010400u)) + off);
  hi = bits(as_h2(__builtin_amdgcn_perm(MAGIC_I8, u, 0x04030402u)) + off);
}

// Four e4m3fn bytes -> two f16 pairs (b0,b1), (b2,b3), exactly.
__device__ __forceinline__ void fp8x4_to_f16(uint32_t x, uint32_t& lo, uint32_t& hi) {
  lo = bits(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x, 1.0f, false));
  hi = bits(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x, 1.0f, true));
}

// (y & mask) | magic as one v_and_or_b32, with `magic` (MAGIC_I4) in a VGPR
// from magic_i4(): gfx950's three-operand VALU encoding takes no literal, and
// the compiler would otherwise split it into v_and_b32 + v_or_b32.
__device__ __forceinline__ uint32_t and_or(uint32_t y, uint32_t mask, uint32_t magic) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(y), "s"(mask), "v"(magic));
  return r;
}
// MAGIC_I4 in a VGPR the compiler cannot rematerialise as a literal
__device__ __forceinline__ uint32_t magic_i4() {
  uint32_t m;
  asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(m));
  return m;
}
// Nibbles at bits 0-3 and 16-19 of y (code + 8) -> f16 pair of codes, exactly.
__device__ __forceinline__ h2 nib_pair(uint32_t y, uint32_t magic) {
  return as_h2(and_or(y, 0x000F000Fu, magic)) + splat2((_Float16)-1032.0f);
}

// INT4_RESIDUAL bytes (low nibble = base code + 8, high nibble = residual code
// + 8) at bytes 0 and 2 of y -> the f16 pair of base codes and the f16 pair of
// 16 x residual codes, both exact integers.
__device__ __forceinline__ h2 i4r_base_pair(uint32_t y, uint32_t magic) { return nib_pair(y, magic); }
__device__ __forceinline__ h2 i4r_resid16_pair(uint32_t y, uint32_t magic) {
  return as_h2(and_or(y, 0x00F000F0u, magic)) + splat2((_Float16)-1152.0f);   // 1024 + 16 * 8
}

// Eight packed INT4 codes (element j = nibble j) -> four f16 pairs, multiplied
// by scale s (`magic` from magic_i4()), in the order the nibble extraction
// yields them: (e0, e4), (e1, e5), (e2, e6), (e3, e7). An MFMA operand built
// from them pairs with a Q operand permuted the same way (q_int4_order).
__device__ __forceinline__ void i4x8_to_f16(uint32_t x, h2 s, uint32_t magic, uint32_t o[4]) {
  o[0] = bits(nib_pair(x, magic) * s);         // (e0, e4)
  o[1] = bits(nib_pair(x >> 4, magic) * s);    // (e1, e5)
  o[2] = bits(nib_pair(x >> 8, magic) * s);    // (e2, e6)
  o[3] = bits(nib_pair(x >> 12, magic) * s);   // (e3, e7)
}
// Eight f16 values in element order -> the order of i4x8_to_f16's output.
__device__ __forceinline__ h8 q_int4_order(h8 v) {
  const u4 d = __builtin_bit_cast(u4, v);
  return make_h8(pack_lo(d[0], d[2]), pack_hi(d[0], d[2]), pack_lo(d[1], d[3]), pack_hi(d[1], d[3]));
}

// Cross-lane reductions over the lanes {l, l^16, l^32, l^48} with the gfx950
// lane-swap instructions (VALU, no LDS round trip): v_permlane32_swap v, t
// with t = v leaves (v[0:32] | v[0:32]) in v and (v[32:64] | v[32:64]) in t,
// so max(v, t) in every lane is the max over lanes l and l^32;
// v_permlane16_swap does the same for l and l^16. Written as one asm block:
// the compiler's own folding drops a float op on the two swap results (it
// treats the second output as an unmodified copy of the input). s_nop 1 is
// the wait the compiler inserts between a VALU write and a lane swap.
__device__ __forceinline__ float xmax16_32(float v) {
  float t;
  asm volatile(
      "v_mov_b32 %1, %0\n\t"
      "s_nop 1\n\t"
      "v_permlane32_swap_b32 %0, %1\n\t"
      "v_max_f32 %0, %0, %1\n\t"
      "v_mov_b32 %1, %0\n\t"
      "s_nop 1\n\t"
      "v_permlane16_swap_b32 %0, %1\n\t"
      "v_max_f32 %0, %0, %1"
      : "+v"(v), "=&v"(t));
  return v;
}
__device__ __forceinline__ float xsum16_32(float v) {
  float t;
  asm volatile(
      "v_mov_b32 %1, %0\n\t"
      "s_nop 1\n\t"
      "v_permlane32_swap_b32 %0, %1\n\t"
      "v_add_f32 %0, %0, %1\n\t"
      "v_mov_b32 %1, %0\n\t"
      "s_nop 1\n\t"
      "v_permlane16_swap_b32 %0, %1\n\t"
      "v_add_f32 %0, %0, %1"
      : "+v"(v), "=&v"(t));
  return v;
}

template <typename T> __device__ __forceinline__ T ld(const T* p) { return *p; }
// Streaming load (the nontemporal hint): for page data read once per launch.
// Each such load instruction should cover whole 128-byte lines; a line read
// in parts by several instructions can be evicted and fetched again between
// them.
template <typename T> __device__ __forceinline__ T ld_nt(const T* p) { return __builtin_nontemporal_load(p); }
// Streaming store: for output written once and not read back by this kernel.
template <typename T> __device__ __forceinline__ void st_nt(T* p, T v) { __builtin_nontemporal_store(v, p); }

__device__ __forceinline__ float load_scale(const void* p, int64_t idx, int dtype) {
  if (dtype == IAK_DTYPE_F32) return reinterpret_cast<const float*>(p)[idx];
  return (float)reinterpret_cast<const _Float16*>(p)[idx];
}

// Index of the lowest set bit of `mask`, which is then cleared.
__device__ __forceinline__ int take(uint64_t& mask) {
  const int idx = __builtin_ctzll(mask);
  mask &= mask - 1;
  return idx;
}

__device__ __forceinline__ float u2f(uint32_t x) { return __builtin_bit_cast(float, x); }
__device__ __forceinline__ uint32_t f2u(float x) { return __builtin_bit_cast(uint32_t, x); }

// --------------------------------------------------------------------------- //
// Cross-split merge. Partial slot of split s of head c in row (b, hk):
// ((b * Hkv + hk) * splits + s) * G + c; acc is float32, or acc / l as float16
// (A16: KArgs::acc16). WPR waves (1, 2 or 4) share one
// (batch, query head): wave part p takes the splits s = p (mod WPR), eight at a
// time with their loads issued together, and keeps a running (max, sum, acc)
// with the online log-sum-exp rule, so it reads every partial once; the parts
// then combine through LDS by the same rule. A 256-thread block holds 4 / WPR
// heads.
// --------------------------------------------------------------------------- //

template <int D, int WPR, bool A16>
__global__ __launch_bounds__(256) void splitk_merge_kernel(const KArgs a) {
  static_assert(WPR == 1 || WPR == 2 || WPR == 4, "1, 2 or 4 waves per head");
  constexpr int PER = D / 64;   // dims per lane
  __shared__ float part_m[4], part_l[4];
  __shared__ float part_o[WPR > 1 ? 4 : 1][WPR > 1 ? D : 1];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int p = w % WPR;                       // this wave's part of its head
  const int bh = blockIdx.x * (4 / WPR) + w / WPR;
  const bool live = bh < a.B * a.Hq;           // uniform per wave; no early return (barriers below)
  const int b = live ? bh / a.Hq : 0, h = live ? bh - b * a.Hq : 0;
  const int hk = h / a.G, c = h - hk * a.G;
  const int S = live ? a.splits : 0;
  const int64_t first = (((int64_t)b * a.Hkv + hk) * a.splits) * a.G + c;   // slot of split 0
  float M = -__builtin_inff(), L = 0.f;
  float o[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) o[j] = 0.f;
  {
    constexpr int U = 8;
    const int n = S > p ? (S - p + WPR - 1) / WPR : 0;   // splits of this part
    for (int i = 0; i < n; i += U) {
      float ms[U], ls[U], av[U][PER];
#pragma unroll
      for (int k = 0; k < U; ++k) {
        const int s = p + WPR * (i + k < n ? i + k : n - 1);
        const int64_t slot = first + (int64_t)s * a.G;
        ms[k] = a.ws_m[slot];
        ls[k] = a.ws_l[slot];
        if constexpr (A16) {
          const _Float16* ap = reinterpret_cast<const _Float16*>(a.ws_acc) + slot * D + PER * lane;
#pragma unroll
          for (int j = 0; j < PER; ++j) av[k][j] = (float)ap[j];
        } else {
          const float* ap = a.ws_acc + slot * D + PER * lane;
#pragma unroll
          for (int j = 0; j < PER; ++j) av[k][j] = ap[j];
        }
      }
#pragma unroll
      for (int k = 0; k < U; ++k) {
        const float mk = ms[k];
        // empty splits (m = -inf) and the clamped reloads past the part's end add nothing
        if (i + k < n && mk > -__builtin_inff()) {
          if (mk > M) {
            const float sc = __builtin_amdgcn_exp2f(M - mk);   // 0 while M is -inf
            L *= sc;
#pragma unroll
            for (int j = 0; j < PER; ++j) o[j] *= sc;
            M = mk;
          }
          const float wgt = __builtin_amdgcn_exp2f(mk - M);
          L += wgt * ls[k];
          const float wa = A16 ? wgt * ls[k] : wgt;   // compact partials hold acc / l
#pragma unroll
          for (int j = 0; j < PER; ++j) o[j] += wa * av[k][j];
        }
      }
    }
  }
  if constexpr (WPR > 1) {
    if (lane == 0) { part_m[w] = M; part_l[w] = L; }
#pragma unroll
    for (int j = 0; j < PER; ++j) part_o[w][PER * lane + j] = o[j];
    __syncthreads();
    if (p != 0) return;
    float Mx = M;
#pragma unroll
    for (int k = 1; k < WPR; ++k) Mx = fmaxf(Mx, part_m[w + k]);
    L = 0.f;
#pragma unroll
    for (int j = 0; j < PER; ++j) o[j] = 0.f;
    if (Mx > -__builtin_inff()) {
#pragma unroll
      for (int k = 0; k < WPR; ++k) {
        const float wk = __builtin_amdgcn_exp2f(part_m[w + k] - Mx);   // 0 for an empty part
        L += wk * part_l[w + k];
#pragma unroll
        for (int j = 0; j < PER; ++j) o[j] += wk * part_o[w + k][PER * lane + j];
      }
    }
  }
  if (!live) return;
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  const int64_t base = (int64_t)b * a.osb + (int64_t)h * a.osh + PER * lane;
  // 16-bit outputs whose rows keep the lane's PER values aligned go out as one
  // store per lane (PER halves packed), the rest element by element
  const int esz = a.out_dtype == IAK_DTYPE_F32 ? 4 : 2;
  const bool packed = esz == 2 && PER % 2 == 0 && a.osb % PER == 0 && a.osh % PER == 0 &&
                      (reinterpret_cast<uintptr_t>(a.out) % (2 * PER)) == 0;
  if (packed) {
    uint32_t wds[PER / 2 > 0 ? PER / 2 : 1];
#pragma unroll
    for (int j = 0; j < PER / 2; ++j) {
      const float v0 = o[2 * j] * inv, v1 = o[2 * j + 1] * inv;
      if (a.out_dtype == IAK_DTYPE_F16) {
        wds[j] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v0) |
                 ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v1) << 16);
      } else {
        wds[j] = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)v0) |
                 ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)v1) << 16);
      }
    }
    uint16_t* op = reinterpret_cast<uint16_t*>(a.out) + base;
    if constexpr (PER == 8) {
      *reinterpret_cast<u4*>(op) = u4{wds[0], wds[1], wds[2], wds[3]};
    } else if constexpr (PER == 4) {
      *reinterpret_cast<u2*>(op) = u2{wds[0], wds[1]};
    } else if constexpr (PER == 2) {
      *reinterpret_cast<uint32_t*>(op) = wds[0];
    } else {
#pragma unroll
      for (int j = 0; j < PER / 2; ++j) reinterpret_cast<uint32_t*>(op)[j] = wds[j];
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const float v = o[j] * inv;
    if (a.out_dtype == IAK_DTYPE_F32) reinterpret_cast<float*>(a.out)[base + j] = v;
    else if (a.out_dtype == IAK_DTYPE_F16) reinterpret_cast<_Float16*>(a.out)[base + j] = (_Float16)v;
    else reinterpret_cast<__bf16*>(a.out)[base + j] = (__bf16)v;
  }
}

// Merge launch: more waves per head when each has many splits to read.
template <int D> hipError_t launch_merge(const KArgs& k, hipStream_t stream) {
  const int heads = k.B * k.Hq;
  const int wpr = k.splits >= 24 ? 4 : (k.splits >= 12 ? 2 : 1);
  const int blocks = (heads * wpr + 3) / 4;
  if (k.acc16) {
    if (wpr == 4) hipLaunchKernelGGL((splitk_merge_kernel<D, 4, true>), dim3(blocks), dim3(256), 0, stream, k);
    else if (wpr == 2) hipLaunchKernelGGL((splitk_merge_kernel<D, 2, true>), dim3(blocks), dim3(256), 0, stream, k);
    else hipLaunchKernelGGL((splitk_merge_kernel<D, 1, true>), dim3(blocks), dim3(256), 0, stream, k);
  } else {
    if (wpr == 4) hipLaunchKernelGGL((splitk_merge_kernel<D, 4, false>), dim3(blocks), dim3(256), 0, stream, k);
    else if (wpr == 2) hipLaunchKernelGGL((splitk_merge_kernel<D, 2, false>), dim3(blocks), dim3(256), 0, stream, k);
    else hipLaunchKernelGGL((splitk_merge_kernel<D, 1, false>), dim3(blocks), dim3(256), 0, stream, k);
  }
  return hipGetLastError();
}

}  // namespace iak

#endif
