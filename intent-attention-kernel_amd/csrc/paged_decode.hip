// Selected-page mixed-precision decode attention for gfx950 (MI355X).
//
// Reference semantics: fused_selected_quant_decode_reference
// (src/intent_attention/fused_selected_quant_decode.py:267-336): for each
// (batch, head) walk the page list, skip SKIP pages (no softmax mass), dequantise
// each page (code * scale), scores q.k / sqrt(D), softmax over every visited
// token, output sum(p v) / sum(p) (0 when nothing was visited).
//
// Work decomposition
//   One wave64 reduces one split: up to `chunk` (<= 64) consecutive entries of
//   one page-table row (batch b, KV head hk). Lane i reads entry i's page id
//   and tag; ballots sort the split's pages into one list per precision so
//   every page loop below runs wave-uniform code. The G = Hq / Hkv query heads
//   of the row share every K/V byte the wave loads (GQA): they are the N
//   columns of the MFMA products. Splits write (m, l, acc) partials; a merge
//   kernel combines them with the log-sum-exp rule. A row that fits one split
//   writes the output directly.
//
// Per page (16 tokens) and wave, lane = c + 16*g (c, g = lane % 16, lane / 16):
//   scores  S^T[16 tok x 16 heads] = K[16 tok x D] . Q^T[D x 16 heads]
//           v_mfma_f32_16x16x32_f16, D/32 k-steps. A operand: lane holds token
//           slot c, dims (D/4)g + 8i .. +7 at step i (K dequantised to f16 in
//           registers); B operand: lane holds head c (zero for c >= G), the
//           same dims. Result: lane holds head c, token slots 4g .. 4g+3.
//           Token slot r is token perm16(r) on FP16 and one-byte pages, whose
//           K reaches this layout through the wave's LDS buffer (the loads
//           themselves cover whole lines), and token r on INT4 pages.
//   softmax exp2 domain; the running max per head is shared by the 4 lane groups
//           (two cross-lane max steps per page) and only moves when a page
//           exceeds it by more than 8 (2^8 head-room in p), so the accumulator
//           rescale is rare.
//   values  O^T[D x 16 heads] += V^T[D x 16 tok] . P^T[16 tok x 16 heads]
//           v_mfma_f32_16x16x16_f16, D/16 row blocks. A operand: lane holds dim
//           (D/16)c + mb of token slots 4g..4g+3; B operand: p of head c, slots
//           4g..4g+3 -- exactly the score result layout, converted to f16.
//           Accumulator: lane holds head c, dims (D/4)g .. (D/4)g + D/4 - 1.
//   Per-page scalar scales fold into the score multiplier (K) and into p (V,
//   relative to the wave's value exponent E: P = p * s * 2^-E, the result is
//   acc * 2^E); INT4 group scales are applied in f16 during dequantisation;
//   INT4_RESIDUAL pages keep their base and residual codes exact and apply the
//   two scales to the f32 products (page_int4r).

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "iak.h"
#include "iak_internal.h"
#include "iak_device.h"

namespace iak {

// --------------------------------------------------------------------------- //
// Raw page data as each lane loads it, per precision and head_dim.
//
// FP16 and one-byte pages are read so that every load instruction covers whole
// 128-byte lines, with the streaming (nontemporal) hint:
//   K  load i of lane l is the 16 bytes at 1024 i + 16 l of the page; the wave
//      rewrites them into the MFMA layout through its LDS buffer (k_through_lds);
//   V  load t of lane (c, g) is token 4t + g, so one instruction reads the four
//      consecutive rows 4t .. 4t+3.
// Lane (c, g) therefore holds K of token perm16(c) and V of tokens perm16(4g + t),
// the same permutation on both sides of the softmax. INT4 pages keep the
// direct layout (token c; tokens 4g + t) and plain loads: their K loads already
// cover the whole page, and streaming loads measured slower on them.
// --------------------------------------------------------------------------- //

template <int D> struct Raw16 {   // FP16: K chunks 64i + lane; V tokens 4t+g dims (D/16)c..
  u4 k[D / 32];                    // D/4 halves = D/32 u4
  uint32_t v[4][D / 32];           // D/16 halves per token = D/32 dwords
};
template <int D> struct Raw8 {    // FP8 / INT8 / INT4_RESIDUAL (one byte per element)
  uint32_t k[D / 16];              // D/4 bytes: chunks 64i + lane
  uint32_t v[4][D / 64 > 0 ? D / 64 : 1];  // D/16 bytes per token 4t+g
};
template <int D> struct Raw4 {    // INT4 (half a byte per element): K token c, V tokens 4g+t
  uint32_t k[D / 32];              // D/8 bytes
  uint32_t v[4];                   // D/32 bytes per token (<= 4)
};

// Token of score row / P slot r of FP16 and one-byte pages: perm16(4g + t) =
// 4t + g.
__device__ __forceinline__ int perm16(int r) { return 4 * (r & 3) + (r >> 2); }

template <int D> __device__ __forceinline__ void load16(Raw16<D>& r, const _Float16* kp, const _Float16* vp,
                                                       int c, int g) {
  const u4* kr = reinterpret_cast<const u4*>(kp) + (c + 16 * g);
#pragma unroll
  for (int i = 0; i < D / 32; ++i) r.k[i] = ld_nt(kr + 64 * i);
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const _Float16* row = vp + (4 * t + g) * D + (D / 16) * c;
    if constexpr (D == 128) {
      u4 x = ld_nt(reinterpret_cast<const u4*>(row));
      r.v[t][0] = x[0]; r.v[t][1] = x[1]; r.v[t][2] = x[2]; r.v[t][3] = x[3];
    } else {
      u2 x = ld_nt(reinterpret_cast<const u2*>(row));
      r.v[t][0] = x[0]; r.v[t][1] = x[1];
    }
  }
}

template <int D> __device__ __forceinline__ void load8(Raw8<D>& r, const uint8_t* kp, const uint8_t* vp,
                                                      int c, int g) {
  const u4* kr = reinterpret_cast<const u4*>(kp) + (c + 16 * g);
#pragma unroll
  for (int i = 0; i < D / 64; ++i) {
    u4 x = ld_nt(kr + 64 * i);
    r.k[4 * i + 0] = x[0]; r.k[4 * i + 1] = x[1]; r.k[4 * i + 2] = x[2]; r.k[4 * i + 3] = x[3];
  }
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint8_t* row = vp + (4 * t + g) * D + (D / 16) * c;
    if constexpr (D == 128) {
      u2 x = ld_nt(reinterpret_cast<const u2*>(row));
      r.v[t][0] = x[0]; r.v[t][1] = x[1];
    } else {
      r.v[t][0] = ld_nt(reinterpret_cast<const uint32_t*>(row));
    }
  }
}

template <int D> __device__ __forceinline__ void load4(Raw4<D>& r, const uint8_t* kp, const uint8_t* vp,
                                                      int c, int g) {
  const uint8_t* krow = kp + c * (D / 2) + (D / 8) * g;
  if constexpr (D == 128) {
    u4 x = ld(reinterpret_cast<const u4*>(krow));
    r.k[0] = x[0]; r.k[1] = x[1]; r.k[2] = x[2]; r.k[3] = x[3];
  } else {
    u2 x = ld(reinterpret_cast<const u2*>(krow));
    r.k[0] = x[0]; r.k[1] = x[1];
  }
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint8_t* row = vp + (4 * g + t) * (D / 2) + (D / 32) * c;
    if constexpr (D == 128) {
      r.v[t] = ld(reinterpret_cast<const uint32_t*>(row));
    } else {
      r.v[t] = ld(reinterpret_cast<const uint16_t*>(row));
    }
  }
}

// --------------------------------------------------------------------------- //
// Wave state and the per-page update shared by all precisions.
// --------------------------------------------------------------------------- //

template <int D, bool QF32> struct Wave {
  h8 qhi[D / 32];
  h8 qlo[QF32 ? D / 32 : 1];
  f4 acc[D / 16];
  float m;   // running max of head c (exp2 domain), equal in the 4 lane groups
  float l;   // partial denominator over this lane's tokens
  int E;     // value exponent (wave-uniform): the value sum is acc * 2^E
  int lim;   // tokens of the current page that exist (< PS on a ragged last page; wave-uniform)
  int g;     // this lane's group (lane / 16)
};

template <int D, bool QF32>
__device__ __forceinline__ f4 scores(const Wave<D, QF32>& w, const h8 (&ka)[D / 32]) {
  f4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < D / 32; ++i) {
    s = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[i], w.qhi[i], s, 0, 0, 0);
    if constexpr (QF32) s = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[i], w.qlo[i], s, 0, 0, 0);
  }
  return s;
}

// Online-softmax update for one page whose raw scores are `s` (lane: head c,
// tokens 4g..4g+3); `smul` = softmax scale * log2(e) * K scale; `vs` = the V
// page scale (1 when V carries its own scale). Returns the page's
// probabilities p (f32, <= 2^8); the V multiplier of the P operand is then
// vs * 2^-E (value_mult), in [2^-EXP_WINDOW, 2^(EXP_WINDOW + 1)).
template <int D, bool QF32>
__device__ __forceinline__ f4 softmax_p(Wave<D, QF32>& w, f4 s, float smul, float vs, bool perm = true) {
  s *= smul;
  if (w.lim < PS) {
    // ragged page: score slot r of lane group g is token perm16(4g + r) = 4r + g
    // (`perm`: FP16 and one-byte pages) or 4g + r (INT4 pages); tokens at or
    // past `lim` are left out (the page's first token always exists)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tok = perm ? 4 * r + w.g : 4 * w.g + r;
      if (tok >= w.lim) s[r] = -__builtin_inff();
    }
  }
  float pm = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
  pm = xmax16_32(pm);
  const bool grow = pm > w.m + RESCALE_SLACK;
  const int e = scale_exp(vs);                    // wave-uniform
  const bool emove = e > w.E + EXP_WINDOW || e < w.E - EXP_WINDOW;
  if (__builtin_amdgcn_ballot_w64(grow) || emove) {   // wave-uniform, rare after the first page
    const float mn = grow ? pm : w.m;
    const float alpha = __builtin_amdgcn_exp2f(w.m - mn);   // 0 on the first page (m = -inf)
    w.l *= alpha;
    const float aacc = emove ? alpha * pow2f(w.E - e) : alpha;
#pragma unroll
    for (int mb = 0; mb < D / 16; ++mb) w.acc[mb] *= aacc;
    w.m = mn;
    if (emove) w.E = e;
  }
  f4 p;
#pragma unroll
  for (int r = 0; r < 4; ++r) p[r] = __builtin_amdgcn_exp2f(s[r] - w.m);
  w.l += (p[0] + p[1]) + (p[2] + p[3]);
  return p;
}

// Probabilities times a V scale, as the f16 B operand of the value product.
__device__ __forceinline__ h4 p_operand(f4 p, float vmul) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  const h2 a = __builtin_convertvector((f2{p[0], p[1]} * vmul), h2);
  const h2 b = __builtin_convertvector((f2{p[2], p[3]} * vmul), h2);
  return make_h4(bits(a), bits(b));
}

// The P multiplier of a V scale `vs` under the wave's value exponent.
template <int D, bool QF32> __device__ __forceinline__ float value_mult(const Wave<D, QF32>& w, float vs) {
  return vs * pow2f(-w.E);
}

template <int D, bool QF32>
__device__ __forceinline__ h4 softmax_step(Wave<D, QF32>& w, f4 s, float smul, float vs, bool perm = true) {
  const f4 p = softmax_p(w, s, smul, vs, perm);
  return p_operand(p, value_mult(w, vs));
}

// V operand of row block mb from four f16-pair rows vt[t][w] = dims (2w, 2w+1)
// of token 4g+t: the dim (D/16)c + mb of tokens 4g .. 4g+3.
template <int D>
__device__ __forceinline__ h4 rows_to_a(const uint32_t (&vt)[4][D / 32], int mb) {
  const int wd = mb >> 1;
  if (mb & 1) return make_h4(pack_hi(vt[0][wd], vt[1][wd]), pack_hi(vt[2][wd], vt[3][wd]));
  return make_h4(pack_lo(vt[0][wd], vt[1][wd]), pack_lo(vt[2][wd], vt[3][wd]));
}

// O^T += V^T P^T, one v_mfma_f32_16x16x16f16 per row block of 16 dims.
template <int D, bool QF32>
__device__ __forceinline__ void pv(Wave<D, QF32>& w, const h4 (&va)[D / 16], h4 pb) {
#pragma unroll
  for (int mb = 0; mb < D / 16; ++mb)
    w.acc[mb] = __builtin_amdgcn_mfma_f32_16x16x16f16(va[mb], pb, w.acc[mb], 0, 0, 0);
}

template <int D, bool QF32>
__device__ __forceinline__ void pv_rows(Wave<D, QF32>& w, const uint32_t (&vt)[4][D / 32], h4 pb) {
  h4 va[D / 16];
#pragma unroll
  for (int mb = 0; mb < D / 16; ++mb) va[mb] = rows_to_a<D>(vt, mb);
  pv(w, va, pb);
}

// --------------------------------------------------------------------------- //
// Per-precision page compute
// --------------------------------------------------------------------------- //

// LDS slot (16-byte units) of chunk `ch` of token row `row` in a wave's K
// transpose buffer of NC chunks per row, XOR-swizzled so that 16 lanes reading
// one chunk of 16 different rows, and 16 lanes writing 256 consecutive bytes,
// each touch every 16-byte bank group once.
template <int NC> __device__ __forceinline__ int kt_slot(int row, int ch) {
  constexpr int RPB = 16 / NC;   // rows per 256 bytes
  return row * NC + (ch ^ ((row / RPB) % NC));
}

// A wave's K page, loaded as 16-byte chunks 64 i + lane (lane = c + 16 g) of
// the page, rewritten through its LDS buffer: afterwards lane (c, g) holds the
// NI chunks NI g .. NI g + NI - 1 of token row perm16(c).
template <int NC, int NI>
__device__ __forceinline__ void k_through_lds(u4 (&k)[NI], u4* kt, int c, int g) {
  const int lane = c + 16 * g;
  // wavefront-scope fences: the buffer's previous reads, these writes and the
  // reads below stay in this order (the lanes exchange data through it)
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int f = 64 * i + lane;
    kt[kt_slot<NC>(f / NC, f % NC)] = k[i];
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  const int row = perm16(c);
#pragma unroll
  for (int i = 0; i < NI; ++i) k[i] = kt[kt_slot<NC>(row, NI * g + i)];
}

template <int D, bool QF32>
__device__ __forceinline__ void page_fp16(Wave<D, QF32>& w, const Raw16<D>& r, float smul, u4* kt, int c, int g) {
  u4 k[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) k[i] = r.k[i];
  k_through_lds<D / 8, D / 32>(k, kt, c, g);
  h8 ka[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) ka[i] = __builtin_bit_cast(h8, k[i]);
  const h4 pb = softmax_step(w, scores(w, ka), smul, 1.0f);
  pv_rows(w, r.v, pb);
}

// The K dwords of a one-byte page in the MFMA layout (lane (c, g): token row
// perm16(c), bytes (D/4) g .. (D/4) g + D/4 - 1).
template <int D> __device__ __forceinline__ void k8_words(const Raw8<D>& r, uint32_t (&kw)[D / 16], u4* kt, int c,
                                                         int g) {
  u4 k[D / 64];
#pragma unroll
  for (int i = 0; i < D / 64; ++i) k[i] = u4{r.k[4 * i], r.k[4 * i + 1], r.k[4 * i + 2], r.k[4 * i + 3]};
  k_through_lds<D / 16, D / 64>(k, kt, c, g);
#pragma unroll
  for (int i = 0; i < D / 64; ++i) {
    kw[4 * i] = k[i][0]; kw[4 * i + 1] = k[i][1]; kw[4 * i + 2] = k[i][2]; kw[4 * i + 3] = k[i][3];
  }
}

// FP8 / INT8 page: codes convert to f16 exactly; the K page scale is in
// `smul`, the V page scale `vs` multiplies p (relative to the value exponent).
template <int D, bool QF32, int TAG>
__device__ __forceinline__ void page_byte(Wave<D, QF32>& w, const Raw8<D>& r, float smul, float vs, u4* kt,
                                          int c, int g) {
  uint32_t kw[D / 16];
  k8_words<D>(r, kw, kt, c, g);
  h8 ka[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) {
    uint32_t o[4];
    if constexpr (TAG == IAK_TAG_FP8) {
      fp8x4_to_f16(kw[2 * i], o[0], o[1]); fp8x4_to_f16(kw[2 * i + 1], o[2], o[3]);
    } else {
      static_assert(TAG == IAK_TAG_INT8, "page_byte handles FP8 and INT8 pages");
      i8x4_to_f16(kw[2 * i], o[0], o[1]); i8x4_to_f16(kw[2 * i + 1], o[2], o[3]);
    }
    ka[i] = make_h8(o[0], o[1], o[2], o[3]);
  }
  const h4 pb = softmax_step(w, scores(w, ka), smul, vs);
  uint32_t vt[4][D / 32];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
#pragma unroll
    for (int j = 0; j < D / 64; ++j) {
      if constexpr (TAG == IAK_TAG_FP8) fp8x4_to_f16(r.v[t][j], vt[t][2 * j], vt[t][2 * j + 1]);
      else i8x4_to_f16(r.v[t][j], vt[t][2 * j], vt[t][2 * j + 1]);
    }
  }
  pv_rows(w, vt, pb);
}

// INT4_RESIDUAL page: every value is base * s0 + resid * s1 with two 4-bit
// codes per byte. Both codes convert to f16 exactly (the residual as 16 x code)
// and the page scales are applied to the f32 products instead of to every
// value:
//   scores  two MFMA chains over the exact codes, s = s0 * (K_base . q) +
//           (s1 / 16) * (K_resid16 . q);
//   values  one v_mfma_f32_16x16x32_f16 per row block whose K dimension
//           stacks the 4 tokens' base codes (k-slots 8g .. 8g+3) and 16 x
//           residual codes (8g+4 .. 8g+7) of the lane's dim, against
//           B = (p * vs0, p * vs1 / 16) of the same tokens.
// `ks0, ks1, vs0, vs1`: K base / residual and V base / residual scales.
template <int D, bool QF32>
__device__ __forceinline__ void page_int4r(Wave<D, QF32>& w, const Raw8<D>& r, float smul, float ks0, float ks1,
                                           float vs0, float vs1, u4* kt, int c, int g) {
  uint32_t kw[D / 16];
  k8_words<D>(r, kw, kt, c, g);
  const uint32_t mg = magic_i4();
  f4 sb = {0.f, 0.f, 0.f, 0.f}, sr = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < D / 32; ++i) {
    // dims 8i .. 8i+7 of the lane's K slice: bytes 0-3 of r.k[2i], then of r.k[2i+1]
    uint32_t b[4], q16[4];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t x = kw[2 * i + h];
      const uint32_t y01 = __builtin_amdgcn_perm(x, x, 0x01010000u);   // bytes 0, 1 -> 0, 2
      const uint32_t y23 = __builtin_amdgcn_perm(x, x, 0x03030202u);   // bytes 2, 3 -> 0, 2
      b[2 * h] = bits(i4r_base_pair(y01, mg));
      b[2 * h + 1] = bits(i4r_base_pair(y23, mg));
      q16[2 * h] = bits(i4r_resid16_pair(y01, mg));
      q16[2 * h + 1] = bits(i4r_resid16_pair(y23, mg));
    }
    const h8 kb = make_h8(b[0], b[1], b[2], b[3]), kr = make_h8(q16[0], q16[1], q16[2], q16[3]);
    sb = __builtin_amdgcn_mfma_f32_16x16x32_f16(kb, w.qhi[i], sb, 0, 0, 0);
    sr = __builtin_amdgcn_mfma_f32_16x16x32_f16(kr, w.qhi[i], sr, 0, 0, 0);
    if constexpr (QF32) {
      sb = __builtin_amdgcn_mfma_f32_16x16x32_f16(kb, w.qlo[i], sb, 0, 0, 0);
      sr = __builtin_amdgcn_mfma_f32_16x16x32_f16(kr, w.qlo[i], sr, 0, 0, 0);
    }
  }
  const float kr16 = ks1 * 0.0625f;
  f4 s;
#pragma unroll
  for (int e = 0; e < 4; ++e) s[e] = sb[e] * ks0 + sr[e] * kr16;
  const f4 p = softmax_p(w, s, smul, vs0);
  const float vm = pow2f(-w.E);
  const h4 pb = p_operand(p, vs0 * vm), pr = p_operand(p, vs1 * 0.0625f * vm);
  const h8 pop = __builtin_shufflevector(pb, pr, 0, 1, 2, 3, 4, 5, 6, 7);
  // V: r.v[t][j] holds dims (D/16)c + 4j .. +3 of token 4g+t
#pragma unroll
  for (int mb = 0; mb < D / 16; ++mb) {
    const int j = mb >> 2, k = mb & 3;
    const uint32_t sel = (uint32_t)k * 0x00000101u + (uint32_t)(4 + k) * 0x01010000u;   // (t_even byte k, t_odd byte k)
    const uint32_t y01 = __builtin_amdgcn_perm(r.v[1][j], r.v[0][j], sel);
    const uint32_t y23 = __builtin_amdgcn_perm(r.v[3][j], r.v[2][j], sel);
    const h8 va = make_h8(bits(i4r_base_pair(y01, mg)), bits(i4r_base_pair(y23, mg)), bits(i4r_resid16_pair(y01, mg)),
                          bits(i4r_resid16_pair(y23, mg)));
    w.acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pop, w.acc[mb], 0, 0, 0);
  }
}

template <int D, bool QF32>
__device__ __forceinline__ void page_int4(Wave<D, QF32>& w, const Raw4<D>& r, float smul, h2 ks, h2 vs) {
  const uint32_t mg = magic_i4();
  h8 ka[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) {
    uint32_t o[4];
    i4x8_to_f16(r.k[i], ks, mg, o);
    ka[i] = make_h8(o[0], o[1], o[2], o[3]);
  }
  const h4 pb = softmax_step(w, scores(w, ka), smul, 1.0f, false);
  // V: tokens (0,1) and (2,3) interleaved per 16 bits, then one nibble per dim
  // gives the (t0, t1) and (t2, t3) halves of the A operand of that dim directly.
  h4 va[D / 16];
  if constexpr (D == 128) {
    const uint32_t y01l = pack_lo(r.v[0], r.v[1]), y01h = pack_hi(r.v[0], r.v[1]);
    const uint32_t y23l = pack_lo(r.v[2], r.v[3]), y23h = pack_hi(r.v[2], r.v[3]);
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const uint32_t y01 = d < 4 ? y01l : y01h, y23 = d < 4 ? y23l : y23h;
      const int sh = 4 * (d & 3);
      va[d] = make_h4(bits(nib_pair(y01 >> sh, mg) * vs), bits(nib_pair(y23 >> sh, mg) * vs));
    }
  } else {   // D == 64: two bytes (4 dims) per token
    const uint32_t y01 = pack_lo(r.v[0], r.v[1]), y23 = pack_lo(r.v[2], r.v[3]);
#pragma unroll
    for (int d = 0; d < 4; ++d)
      va[d] = make_h4(bits(nib_pair(y01 >> (4 * d), mg) * vs), bits(nib_pair(y23 >> (4 * d), mg) * vs));
  }
  pv(w, va, pb);
}

// --------------------------------------------------------------------------- //
// The split kernel
// --------------------------------------------------------------------------- //

struct Split {
  int b, hk, split, n;   // n = pages in this split
};

// Uniform scale slots of the page held by lane `idx` (see load_page_scales).
struct Scales {
  uint32_t s[4];
};
__device__ __forceinline__ Scales read_scales(const uint32_t (&slot)[4], int idx) {
  Scales r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r.s[i] = __builtin_amdgcn_readlane(slot[i], idx);
  return r;
}

// f16 group scale `grp` (0..3) out of two f16x2 dwords, splatted to both halves.
__device__ __forceinline__ h2 group_scale(uint32_t lo, uint32_t hi, int grp) {
  const uint32_t w = (grp & 2) ? hi : lo;
  const uint32_t h = (grp & 1) ? (w >> 16) : (w & 0xFFFFu);
  return as_h2(h | (h << 16));
}

__device__ __forceinline__ uint32_t scale_bits_f32(const void* p, int64_t idx, int dtype) {
  return f2u(load_scale(p, idx, dtype));
}
__device__ __forceinline__ uint32_t scale_bits_f16(const void* p, int64_t idx, int dtype) {
  const _Float16 h = (_Float16)load_scale(p, idx, dtype);
  return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

// Per-lane scale slots of the lane's own page, loaded once per split:
//   FP8 / INT8      s0 = K scale, s1 = V scale (f32 bits)
//   INT4_RESIDUAL   s0, s1 = K base / residual scale, s2, s3 = V base / residual (f32 bits)
//   INT4            s0, s1 = f16 pairs (q0,q1), (q2,q3) of the K scales of the four
//                   quarters of head_dim (quarter q lies in group q * D/4 / int4_group);
//                   s2, s3 = V
// With page descriptors the four slots are words 4-7 of the page's descriptor;
// with entry records, words 4-7 of the record of table entry `ent`.
template <int D>
__device__ __forceinline__ void load_page_scales(const KArgs& a, int pid, int tag, uint32_t (&slot)[4],
                                                 int64_t ent) {
  slot[0] = slot[1] = slot[2] = slot[3] = 0u;
  if (pid < 0) return;
  const int64_t p = pid;
  if (a.recs) {
    const u4 x = *reinterpret_cast<const u4*>(a.recs + 8 * ent + 4);
    slot[0] = x[0]; slot[1] = x[1]; slot[2] = x[2]; slot[3] = x[3];
    return;
  }
  if (a.desc) {
    const u4 x = *reinterpret_cast<const u4*>(a.desc + 8 * p + 4);
    slot[0] = x[0]; slot[1] = x[1]; slot[2] = x[2]; slot[3] = x[3];
    return;
  }
  if (tag == IAK_TAG_FP8) {
    slot[0] = scale_bits_f32(a.k_fp8_scale, p, a.fp8_sd);
    slot[1] = scale_bits_f32(a.v_fp8_scale, p, a.fp8_sd);
  } else if (tag == IAK_TAG_INT8) {
    slot[0] = scale_bits_f32(a.k_int8_scale, p, a.int8_sd);
    slot[1] = scale_bits_f32(a.v_int8_scale, p, a.int8_sd);
  } else if (tag == IAK_TAG_INT4_RESIDUAL) {
    slot[0] = f2u(a.k_int4r_scale[2 * p]);
    slot[1] = f2u(a.k_int4r_scale[2 * p + 1]);
    slot[2] = f2u(a.v_int4r_scale[2 * p]);
    slot[3] = f2u(a.v_int4r_scale[2 * p + 1]);
  } else if (tag == IAK_TAG_INT4) {
    const int ng = D / a.int4_group;   // 1, 2 or 4
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
      const int src = gi * ng / 4;      // the group of quarter gi
      const uint32_t kh = scale_bits_f16(a.k_int4_scale, p * ng + src, a.int4_sd);
      const uint32_t vh = scale_bits_f16(a.v_int4_scale, p * ng + src, a.int4_sd);
      slot[gi >> 1] |= kh << (16 * (gi & 1));
      slot[2 + (gi >> 1)] |= vh << (16 * (gi & 1));
    }
  }
}

template <int D, int QT>
__device__ void write_result(const KArgs& a, const Split& sp, Wave<D, QT != IAK_DTYPE_F16>& w, int c, int g) {
  const float l = xsum16_32(w.l);
  if (c >= a.G) return;
  const int h = sp.hk * a.G + c;
  const float vscale = pow2f(w.E);   // the value sum is acc * 2^E
  if (a.splits == 1) {
    const float inv = l > 0.f ? vscale / l : 0.0f;
    const int64_t base = (int64_t)sp.b * a.osb + (int64_t)h * a.osh + (D / 4) * g;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v[D / 16];
#pragma unroll
      for (int mb = 0; mb < D / 16; ++mb) v[mb] = w.acc[mb][r] * inv;
      const int64_t o = base + (D / 16) * r;
      if (a.out_dtype == IAK_DTYPE_F32) {
        float* op = reinterpret_cast<float*>(a.out) + o;
#pragma unroll
        for (int mb = 0; mb < D / 16; ++mb) op[mb] = v[mb];
      } else if (a.out_dtype == IAK_DTYPE_F16) {
        _Float16* op = reinterpret_cast<_Float16*>(a.out) + o;
#pragma unroll
        for (int mb = 0; mb < D / 16; ++mb) op[mb] = (_Float16)v[mb];
      } else {
        __bf16* op = reinterpret_cast<__bf16*>(a.out) + o;
#pragma unroll
        for (int mb = 0; mb < D / 16; ++mb) op[mb] = (__bf16)v[mb];
      }
    }
    return;
  }
  const int64_t slot = (((int64_t)sp.b * a.Hkv + sp.hk) * a.splits + sp.split) * a.G + c;
  if (g == 0) { a.ws_m[slot] = w.m; a.ws_l[slot] = l; }
  float* op = a.ws_acc + slot * D + (D / 4) * g;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
#pragma unroll
    for (int mb = 0; mb < D / 16; ++mb) op[(D / 16) * r + mb] = w.acc[mb][r] * vscale;
  }
}

// In-kernel merge (KArgs::fused). The workgroup's four waves hold splits
// 4j .. 4j+3 of one row (the plan makes the split count a multiple of four).
// Each wave puts its (m, l, acc * 2^E) per head into the LDS, the workgroup
// combines the four with the log-sum-exp rule into the row's partial j, and
// the workgroup that arrives last at the row's counter merges the row's
// splits / 4 partials into the output, then resets the counter for the next
// call.
// Visibility across the XCDs (each has its own L2): the partials are written
// and read with agent-scope atomic stores and loads, which the L2 writes
// through to memory and re-reads from it (the sc1 scope bit), and the stores
// are acknowledged (s_waitcnt vmcnt(0)) before the barrier that precedes the
// arrival. No agent-scope release fence is used: it writes back the whole L2
// (buffer_wbl2), which took the cfg3 decode from 333 to 645 us; the merging
// workgroup takes an agent-scope acquire (buffer_inv sc1, a cache invalidate)
// after it sees the last arrival. The release side therefore rests on gfx950's
// write-through of sc1 atomic stores, not on the HIP memory model.
// `red`: LDS [4 waves][16 heads][D] floats (the K transpose buffers, done with).
template <int D, int QT>
__device__ void merge_in_kernel(const KArgs& a, const Split& sp, const Wave<D, QT != IAK_DTYPE_F16>& w, int c,
                                int g, float* red, int wv) {
  __shared__ float red_m[IAK_WAVES_PER_BLOCK][16], red_l[IAK_WAVES_PER_BLOCK][16];
  __shared__ int last;
  constexpr int WR = 16 * D;   // floats per wave
  const float l = xsum16_32(w.l);
  // this wave's K transpose reads are done before its region is overwritten
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  if (c < a.G) {
    if (g == 0) { red_m[wv][c] = w.m; red_l[wv][c] = l; }
    const float vscale = pow2f(w.E);   // the value sum is acc * 2^E
    float* mine = red + wv * WR + c * D + (D / 4) * g;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
      for (int mb = 0; mb < D / 16; ++mb) mine[(D / 16) * r + mb] = w.acc[mb][r] * vscale;
    }
  }
  __syncthreads();

  const int t = threadIdx.x;
  const int GD = a.G * D;
  const int nwg = a.splits >> 2, j = sp.split >> 2;
  const int64_t row = (int64_t)sp.b * a.Hkv + sp.hk;
  const int64_t first = row * nwg * a.G;   // partial slot of (row, 0, head 0)
  for (int o = t; o < GD; o += 64 * IAK_WAVES_PER_BLOCK) {
    const int h = o / D;
    float M = -__builtin_inff();
#pragma unroll
    for (int k = 0; k < IAK_WAVES_PER_BLOCK; ++k) M = fmaxf(M, red_m[k][h]);
    float L = 0.f, A = 0.f;
    if (M > -__builtin_inff()) {
#pragma unroll
      for (int k = 0; k < IAK_WAVES_PER_BLOCK; ++k) {
        const float wt = __builtin_amdgcn_exp2f(red_m[k][h] - M);   // 0 for an empty split (m = -inf)
        L += wt * red_l[k][h];
        A += wt * red[k * WR + o];
      }
    }
    const int64_t slot = first + (int64_t)j * a.G + h;
    __hip_atomic_store(a.ws_acc + slot * D + (o - h * D), A, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (o == h * D) {
      __hip_atomic_store(a.ws_m + slot, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(a.ws_l + slot, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  // this workgroup's partial has reached memory before its arrival is counted
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (t == 0) last = atomicAdd(a.counters + row, 1) == nwg - 1;
  __syncthreads();
  if (!last) return;
  // Acquire side of the handoff: drop any stale copy of the partials from this
  // workgroup's caches before reading them (a cache invalidate; the partials
  // themselves are also read with sc1 loads). The release side has no fence:
  // an agent-scope release is a write-back of the whole L2 (it doubled the cfg3
  // step); the partials are written through to memory instead (sc1 atomic
  // stores, acknowledged by the vmcnt wait before the barrier above), which is
  // gfx950's behaviour for agent-scope atomic stores, not a guarantee of the
  // HIP memory model.
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");

  // the row's merge: output (head h, dim d) from the nwg workgroup partials,
  // OU outputs per thread and U partials per batch with every load of a batch
  // issued together, combined with the online log-sum-exp rule
  constexpr int OU = 2, U = 8;
  constexpr int NT = 64 * IAK_WAVES_PER_BLOCK;
  for (int o0 = t; o0 < GD; o0 += NT * OU) {
    float M[OU], L[OU], A[OU];
#pragma unroll
    for (int j = 0; j < OU; ++j) { M[j] = -__builtin_inff(); L[j] = 0.f; A[j] = 0.f; }
    for (int i = 0; i < nwg; i += U) {
      float ms[OU][U], ls[OU][U], av[OU][U];
#pragma unroll
      for (int j = 0; j < OU; ++j) {
        const int o = o0 + NT * j < GD ? o0 + NT * j : o0;   // past the end: a duplicate, not written
        const int h = o / D, d = o - h * D;
#pragma unroll
        for (int k = 0; k < U; ++k) {
          const int64_t sl = first + h + (int64_t)(i + k < nwg ? i + k : nwg - 1) * a.G;
          ms[j][k] = __hip_atomic_load(a.ws_m + sl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          ls[j][k] = __hip_atomic_load(a.ws_l + sl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          av[j][k] = __hip_atomic_load(a.ws_acc + sl * D + d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
#pragma unroll
      for (int j = 0; j < OU; ++j)
#pragma unroll
        for (int k = 0; k < U; ++k) {
          const float mk = ms[j][k];
          if (i + k < nwg && mk > -__builtin_inff()) {   // an empty partial (m = -inf) adds nothing
            if (mk > M[j]) {
              const float sc = __builtin_amdgcn_exp2f(M[j] - mk);   // 0 while M is -inf
              L[j] *= sc;
              A[j] *= sc;
              M[j] = mk;
            }
            const float wt = __builtin_amdgcn_exp2f(mk - M[j]);
            L[j] += wt * ls[j][k];
            A[j] += wt * av[j][k];
          }
        }
    }
#pragma unroll
    for (int j = 0; j < OU; ++j) {
      const int o = o0 + NT * j;
      if (o >= GD) continue;
      const int h = o / D, d = o - h * D;
      const float v = A[j] * (L[j] > 0.f ? 1.0f / L[j] : 0.f);
      const int64_t op = (int64_t)sp.b * a.osb + (int64_t)(sp.hk * a.G + h) * a.osh + d;
      if (a.out_dtype == IAK_DTYPE_F32) reinterpret_cast<float*>(a.out)[op] = v;
      else if (a.out_dtype == IAK_DTYPE_F16) reinterpret_cast<_Float16*>(a.out)[op] = (_Float16)v;
      else reinterpret_cast<__bf16*>(a.out)[op] = (__bf16)v;
    }
  }
  // reset for the next call, written through like the partials (its cache
  // line holds other rows' counters)
  if (t == 0) __hip_atomic_store(a.counters + row, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Q operand of head c (zero for padding columns): dims (D/4)g + 8i .. +7 of step i,
// loaded as 16-byte vectors (the C ABI checks 16-byte alignment of q rows).
template <int D, int QT>
__device__ __forceinline__ void load_q(const KArgs& a, const Split& sp, Wave<D, QT != IAK_DTYPE_F16>& w, int c,
                                       int g) {
  const bool live = c < a.G;
  const int h = sp.hk * a.G + (live ? c : 0);
  const int64_t off = (int64_t)sp.b * a.qsb + (int64_t)h * a.qsh + (D / 4) * g;
#pragma unroll
  for (int i = 0; i < D / 32; ++i) {
    float qv[8];
    if constexpr (QT == IAK_DTYPE_F32) {
      const f4* p = reinterpret_cast<const f4*>(reinterpret_cast<const float*>(a.q) + off + 8 * i);
      const f4 x0 = p[0], x1 = p[1];
#pragma unroll
      for (int e = 0; e < 4; ++e) { qv[e] = x0[e]; qv[4 + e] = x1[e]; }
    } else {
      const u4 x = *reinterpret_cast<const u4*>(reinterpret_cast<const uint16_t*>(a.q) + off + 8 * i);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t lo = x[e] & 0xFFFFu, hi = x[e] >> 16;
        if constexpr (QT == IAK_DTYPE_F16) {
          qv[2 * e] = (float)__builtin_bit_cast(_Float16, (uint16_t)lo);
          qv[2 * e + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)hi);
        } else {   // bf16: the high half of an f32
          qv[2 * e] = u2f(lo << 16);
          qv[2 * e + 1] = u2f(hi << 16);
        }
      }
    }
    h8 vhi, vlo;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = live ? qv[e] : 0.f;
      vhi[e] = (_Float16)v;
      vlo[e] = (_Float16)(v - (float)vhi[e]);
    }
    w.qhi[i] = vhi;
    if constexpr (QT != IAK_DTYPE_F16) w.qlo[i] = vlo;
  }
}

// Read-only target of the ring loads issued past the end of a class: one page
// of any precision (at most PS x 128 x 2 bytes), the same address for every
// wave, so those loads stay in the L2 instead of fetching a streamed page again.
static __device__ __attribute__((aligned(4096))) uint8_t pad_page[PS * 128 * 2];

// Walks the pages of one precision class (lanes set in `mask`) through a ring
// of R register buffers: while one page is computed the next R-1 are in
// flight. Every step issues exactly one page load -- once the class runs out
// of pages the load names page -1, which the load functions point at
// pad_page -- and the loop exits only at its latch, so each buffer stays in
// its registers and the wait before each compute is a fixed vmcnt: loads are
// never drained early.
template <int R, typename Raw, typename LoadF, typename ComputeF>
__device__ __forceinline__ void class_loop(uint64_t mask, int pid, LoadF load, ComputeF compute) {
  if (!mask) return;
  const int n = __builtin_popcountll(mask);
  Raw buf[R];
  int idx[R];
  int last = 0;
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const bool real = mask != 0;
    if (mask) last = take(mask);
    idx[j] = last;
    const int p = __builtin_amdgcn_readlane(pid, last);
    load(buf[j], real ? p : -1);
  }
  // one exit, at the latch: the R steps of the body always issue their loads
  for (int base = 0; base < n; base += R) {
#pragma unroll
    for (int j = 0; j < R; ++j) {
      if (base + j < n) compute(buf[j], idx[j]);
      const bool real = mask != 0;
      if (mask) last = take(mask);
      idx[j] = last;
      const int p = __builtin_amdgcn_readlane(pid, last);
      load(buf[j], real ? p : -1);
    }
  }
}

// Base address of page `p` of a pool with `bytes` per page; pad_page for p < 0.
template <typename T> __device__ __forceinline__ const T* page_at(const void* pool, int p, int bytes) {
  return reinterpret_cast<const T*>(p < 0 ? pad_page : reinterpret_cast<const uint8_t*>(pool) + (int64_t)p * bytes);
}

// Position of work item `item`: split `sp.split` of row `unit` = b * Hkv + hk,
// table entries [start, start + len). The grid holds every row's first-tier
// splits (`chunk` entries) first, then every row's second-tier splits (chunkB
// entries), so the short ones are the last to be dispatched.
__device__ __forceinline__ void locate(const KArgs& a, int item, Split& sp, int& start, int& unit, int& len) {
  // one division whichever tier (two, on branches, cost cfg4's short kernel 0.6 us)
  item = __builtin_amdgcn_readfirstlane(item);
  const int itemsA = a.B * a.Hkv * a.splitsA;
  const bool tail = item >= itemsA;
  const int j = tail ? item - itemsA : item;
  const int per = tail ? a.splits - a.splitsA : a.splitsA;
  len = tail ? a.chunkB : a.chunk;
  unit = j / per;
  const int k = j - unit * per;
  sp.split = (tail ? a.splitsA : 0) + k;
  start = (tail ? a.splitsA * a.chunk : 0) + k * len;
  sp.b = unit / a.Hkv;
  sp.hk = unit - sp.b * a.Hkv;
}

// First metadata stage of an item: lane i loads table entry start + i (bounded
// by the table width, so it needs no count), the row's page count and token
// bound. With entry records the entry's record gives the page id and its
// native tag (`rtag`) in the same load.
__device__ __forceinline__ void load_entry(const KArgs& a, int unit, int start, int len, int lane, int& raw,
                                           int& rtag, int& cnt, int& bnd) {
  raw = -1;
  rtag = IAK_TAG_SKIP;
  if (lane < len && start + lane < a.W) {
    const int64_t e = (int64_t)unit * a.W + start + lane;
    if (a.recs) {
      const u4 r = *reinterpret_cast<const u4*>(a.recs + 8 * e);
      rtag = (int)r[0];
      raw = (int)r[1];
    } else {
      raw = a.table[e];
    }
  }
  cnt = a.counts[unit];
  bnd = a.valid ? a.valid[unit] : 0x7FFFFFFF;
}

// Second stage: drop entries at or past the row's count or wholly past its
// token bound, validate the page id (wrapping negative ids when asked) and load
// its tag through the tag map (caller tags outside [0, 8) take other_tag).
// `lim`: tokens of the lane's entry that exist (PS unless the bound cuts it).
__device__ __forceinline__ void load_tag(const KArgs& a, int raw, int rtag, int cnt, int bnd, int start, int len,
                                         int lane, int& pid, int& tag, int& n, int& lim) {
  cnt = cnt < 0 ? 0 : (cnt > a.W ? a.W : cnt);
  n = cnt - start < len ? cnt - start : len;
  if (n < 0) n = 0;
  pid = -1;
  tag = IAK_TAG_SKIP;
  const int64_t left = (int64_t)bnd - (int64_t)(start + lane) * PS;
  lim = left < 0 ? 0 : (left > PS ? PS : (int)left);
  if (lane < n && lim > 0) {
    int p = raw;
    if (a.neg_wrap && p < 0 && (int64_t)p >= -a.NP) p = (int)((int64_t)p + a.NP);
    if (p >= 0 && (int64_t)p < a.NP) {
      // the caller's tag, or the native tag of the entry's record or of the
      // page's descriptor (the tag map then passes the precisions whose pools
      // are present)
      const int t = a.recs ? rtag : a.desc ? (int)a.desc[8 * (int64_t)p] : a.tags[p];
      tag = (t >= 0 && t < 8) ? (int)((a.tagmap >> (8 * t)) & 0xFFu) : a.other_tag;
      pid = p;
    }
  }
}

// Waves per SIMD the kernel is compiled for: f32 / bf16 queries carry a second
// (low-half) Q operand and get the register budget of two waves per SIMD.
template <int QT> constexpr int waves_per_simd() { return QT == IAK_DTYPE_F16 ? IAK_MIN_WAVES_PER_SIMD : 2; }

// One wave per work item. The dependent metadata loads (table entry and count
// -> tag) are the wave's prologue, the page scales follow the FP16 pages; the
// waves the hardware starts as others finish run their prologue while the rest
// of the CU streams pages.
template <int D, int QT>
__global__ __launch_bounds__(64 * IAK_WAVES_PER_BLOCK, waves_per_simd<QT>())
void paged_decode_kernel(const KArgs a) {
  constexpr bool QF32 = QT != IAK_DTYPE_F16;
  const int lane = threadIdx.x & 63;
  const int c = lane & 15, g = lane >> 4;
  const int item = blockIdx.x * IAK_WAVES_PER_BLOCK + (threadIdx.x >> 6);
  if (item >= a.items) return;   // never taken by an in-kernel-merge grid (whole workgroups)
  // the wave's K transpose buffer: one FP16 page's K (a one-byte page uses
  // half), in dynamic LDS whose per-wave stride also holds the in-kernel merge's
  // 16 x D floats when a.fused
  extern __shared__ u4 decode_lds[];
  const int wv = threadIdx.x >> 6;
  u4* kt = decode_lds + wv * (a.fused ? 4 * D : PS * D / 8);

  Split sp;
  int pid, tag, lim, start, unit;
  uint32_t slot[4];
  {
    int raw, rtag, cnt, bnd, len;
    locate(a, item, sp, start, unit, len);
    load_entry(a, unit, start, len, lane, raw, rtag, cnt, bnd);
    load_tag(a, raw, rtag, cnt, bnd, start, len, lane, pid, tag, sp.n, lim);
  }

  Wave<D, QF32> w;
  w.m = -__builtin_inff();
  w.l = 0.f;
  w.E = 0;
  w.lim = PS;
  w.g = g;
  // tokens of the page of lane idx that exist
  auto page_lim = [&](int idx) { return __builtin_amdgcn_readlane(lim, idx); };
#pragma unroll
  for (int mb = 0; mb < D / 16; ++mb) w.acc[mb] = f4{0.f, 0.f, 0.f, 0.f};
  load_q<D, QT>(a, sp, w, c, g);

  const float smul = a.score_mult;

  // ---- FP16 pages ----
  {
    class_loop<IAK_RING_FP16, Raw16<D>>(
        __builtin_amdgcn_ballot_w64(tag == IAK_TAG_FP16), pid,
        [&](Raw16<D>& r, int p) {
          load16<D>(r, page_at<_Float16>(a.k_fp16, p, PS * D * 2), page_at<_Float16>(a.v_fp16, p, PS * D * 2), c, g);
        },
        [&](const Raw16<D>& r, int idx) {
          w.lim = page_lim(idx);
          page_fp16(w, r, smul, kt, c, g);
        });
  }
  // the scales are first needed by the classes below: loaded here, their round
  // trip overlaps the next class's ring fill instead of preceding the FP16 pages
  load_page_scales<D>(a, pid, tag, slot, (int64_t)unit * a.W + start + lane);

  // ---- one-byte precisions ----
  {
    class_loop<IAK_RING_BYTE, Raw8<D>>(
        __builtin_amdgcn_ballot_w64(tag == IAK_TAG_FP8), pid,
        [&](Raw8<D>& r, int p) {
          load8<D>(r, page_at<uint8_t>(a.k_fp8, p, PS * D), page_at<uint8_t>(a.v_fp8, p, PS * D), c, g);
        },
        [&](const Raw8<D>& r, int idx) {
          const Scales s = read_scales(slot, idx);
          w.lim = page_lim(idx);
          page_byte<D, QF32, IAK_TAG_FP8>(w, r, smul * u2f(s.s[0]), u2f(s.s[1]), kt, c, g);
        });
  }
  {
    class_loop<IAK_RING_BYTE, Raw8<D>>(
        __builtin_amdgcn_ballot_w64(tag == IAK_TAG_INT8), pid,
        [&](Raw8<D>& r, int p) {
          load8<D>(r, page_at<uint8_t>(a.k_int8, p, PS * D), page_at<uint8_t>(a.v_int8, p, PS * D), c, g);
        },
        [&](const Raw8<D>& r, int idx) {
          const Scales s = read_scales(slot, idx);
          w.lim = page_lim(idx);
          page_byte<D, QF32, IAK_TAG_INT8>(w, r, smul * u2f(s.s[0]), u2f(s.s[1]), kt, c, g);
        });
  }
  {
    class_loop<IAK_RING_BYTE, Raw8<D>>(
        __builtin_amdgcn_ballot_w64(tag == IAK_TAG_INT4_RESIDUAL), pid,
        [&](Raw8<D>& r, int p) {
          load8<D>(r, page_at<uint8_t>(a.k_int4r, p, PS * D), page_at<uint8_t>(a.v_int4r, p, PS * D), c, g);
        },
        [&](const Raw8<D>& r, int idx) {
          const Scales s = read_scales(slot, idx);
          w.lim = page_lim(idx);
          page_int4r(w, r, smul, u2f(s.s[0]), u2f(s.s[1]), u2f(s.s[2]), u2f(s.s[3]), kt, c, g);
        });
  }
  // ---- INT4 pages: lane K dims (D/4)g.. lie in group kg, V dims (D/16)c.. in group vg ----
  {
    // the last class: Q takes the element order of the INT4 K operand
    // (i4x8_to_f16), which saves the K pairs' repacking on every page
#pragma unroll
    for (int i = 0; i < D / 32; ++i) {
      w.qhi[i] = q_int4_order(w.qhi[i]);
      if constexpr (QF32) w.qlo[i] = q_int4_order(w.qlo[i]);
    }
    const int kg = g;        // the quarter of head_dim holding the lane's K dims (D/4)g ..
    const int vg = c >> 2;   // and its V dims (D/16)c ..
    class_loop<IAK_RING_INT4, Raw4<D>>(
        __builtin_amdgcn_ballot_w64(tag == IAK_TAG_INT4), pid,
        [&](Raw4<D>& r, int p) {
          load4<D>(r, page_at<uint8_t>(a.k_int4, p, PS * D / 2), page_at<uint8_t>(a.v_int4, p, PS * D / 2), c, g);
        },
        [&](const Raw4<D>& r, int idx) {
          const Scales s = read_scales(slot, idx);
          w.lim = page_lim(idx);
          page_int4(w, r, smul, group_scale(s.s[0], s.s[1], kg), group_scale(s.s[2], s.s[3], vg));
        });
  }

  if (a.fused) {
    merge_in_kernel<D, QT>(a, sp, w, c, g, reinterpret_cast<float*>(decode_lds), wv);
    return;
  }
  write_result<D, QT>(a, sp, w, c, g);
}

// Page descriptors: one thread per page writes the native tag a decode would
// use for it (word 0) and the scale slots it would load (words 4-7).
template <int D>
__global__ __launch_bounds__(256) void pack_descriptors_kernel(const KArgs a, uint32_t* desc) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (p >= a.NP) return;
  const int t = a.tags[p];
  const int tag = (t >= 0 && t < 8) ? (int)((a.tagmap >> (8 * t)) & 0xFFu) : a.other_tag;
  uint32_t slot[4];
  load_page_scales<D>(a, (int)p, tag, slot, 0);
  u4* out = reinterpret_cast<u4*>(desc + 8 * p);
  out[0] = u4{(uint32_t)tag, 0u, 0u, 0u};
  out[1] = u4{slot[0], slot[1], slot[2], slot[3]};
}

hipError_t launch_pack_descriptors(const KArgs& k, void* desc, hipStream_t stream) {
  const int64_t blocks = (k.NP + 255) / 256;
  if (blocks == 0) return hipSuccess;
  if (k.D == 128)
    hipLaunchKernelGGL(pack_descriptors_kernel<128>, dim3((unsigned)blocks), dim3(256), 0, stream, k,
                       static_cast<uint32_t*>(desc));
  else
    hipLaunchKernelGGL(pack_descriptors_kernel<64>, dim3((unsigned)blocks), dim3(256), 0, stream, k,
                       static_cast<uint32_t*>(desc));
  return hipGetLastError();
}

// Entry records: one thread per table entry writes the native tag and the
// resolved page id a decode would use for it (words 0, 1; -1 and SKIP for an
// entry whose id is out of range) and the page's scale slots (words 4-7).
template <int D>
__global__ __launch_bounds__(256) void pack_records_kernel(const KArgs a, uint32_t* recs, int64_t entries) {
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < entries; e += (int64_t)gridDim.x * 256) {
    int p = a.table[e];
    if (a.neg_wrap && p < 0 && (int64_t)p >= -a.NP) p = (int)((int64_t)p + a.NP);
    int tag = IAK_TAG_SKIP;
    if (p >= 0 && (int64_t)p < a.NP) {
      const int t = a.tags[p];
      tag = (t >= 0 && t < 8) ? (int)((a.tagmap >> (8 * t)) & 0xFFu) : a.other_tag;
    } else {
      p = -1;
    }
    uint32_t slot[4];
    load_page_scales<D>(a, p, tag, slot, 0);
    u4* out = reinterpret_cast<u4*>(recs + 8 * e);
    out[0] = u4{(uint32_t)tag, (uint32_t)p, 0u, 0u};
    out[1] = u4{slot[0], slot[1], slot[2], slot[3]};
  }
}

hipError_t launch_pack_records(const KArgs& k, void* recs, hipStream_t stream) {
  const int64_t entries = (int64_t)k.B * k.Hkv * k.W;
  if (entries == 0) return hipSuccess;
  const int64_t want = (entries + 255) / 256;
  const unsigned blocks = (unsigned)(want < 65536 ? want : 65536);
  if (k.D == 128)
    hipLaunchKernelGGL(pack_records_kernel<128>, dim3(blocks), dim3(256), 0, stream, k, static_cast<uint32_t*>(recs),
                       entries);
  else
    hipLaunchKernelGGL(pack_records_kernel<64>, dim3(blocks), dim3(256), 0, stream, k, static_cast<uint32_t*>(recs),
                       entries);
  return hipGetLastError();
}

template <int D, int QT>
hipError_t launch_decode(const KArgs& k, hipStream_t stream, hipEvent_t ev_begin, hipEvent_t ev_end) {
  const int blocks = (k.items + IAK_WAVES_PER_BLOCK - 1) / IAK_WAVES_PER_BLOCK;
  // per-wave LDS: the K transpose buffer (PS x D halves), or 16 x D floats for
  // the in-kernel merge
  const size_t lds = (size_t)IAK_WAVES_PER_BLOCK * (k.fused ? 4 * D : PS * D / 8) * sizeof(u4);
  if (ev_begin) (void)hipEventRecord(ev_begin, stream);
  hipLaunchKernelGGL((paged_decode_kernel<D, QT>), dim3(blocks), dim3(64 * IAK_WAVES_PER_BLOCK), lds,
                     stream, k);
  hipError_t e = hipGetLastError();
  if (ev_end) (void)hipEventRecord(ev_end, stream);
  if (e != hipSuccess || k.splits == 1 || k.fused) return e;
  return launch_merge<D>(k, stream);
}

template <int D>
hipError_t launch_d(const KArgs& k, hipStream_t stream, hipEvent_t eb, hipEvent_t ee) {
  switch (k.q_dtype) {
    case IAK_DTYPE_F32: return launch_decode<D, IAK_DTYPE_F32>(k, stream, eb, ee);
    case IAK_DTYPE_BF16: return launch_decode<D, IAK_DTYPE_BF16>(k, stream, eb, ee);
    default: return launch_decode<D, IAK_DTYPE_F16>(k, stream, eb, ee);
  }
}

hipError_t launch_paged_decode(const KArgs& k, hipStream_t stream, hipEvent_t ev_begin, hipEvent_t ev_end) {
  return k.D == 128 ? launch_d<128>(k, stream, ev_begin, ev_end) : launch_d<64>(k, stream, ev_begin, ev_end);
}

}  // namespace iak
