// MLA latent decode for gfx950 (MI355X): every query head of a sequence
// attends to one shared compressed KV, so the work per sequence is a pair of
// dense products over the selected latent rows -- S = Q C^T and O = P C.
//
// Reference semantics: mla_decode_triton / _mla_decode_cpu
// (src/intent_attention/triton_mla_decode.py:110-186): online softmax over the
// page table's latent pages with s = (q . c) * scale, context = acc / l (zeros
// when no page is visited). The projection by W_VO that the reference applies
// to the context is a plain GEMM and stays outside this kernel.
//
// Work decomposition
//   One workgroup of 4 waves (one per SIMD, up to 512 registers each) reduces
//   one split -- up to 64 consecutive page-table entries of one sequence -- for
//   64 heads. Each latent page is loaded once per workgroup, two pages ahead
//   in registers, and staged in LDS as two f16 tiles: [token][dim] for the
//   score product and [dim][token] (value dims only) for the value product.
//   FP8 / INT8 codes are converted to f16 exactly while staging; the page
//   scale folds into the score multiplier and into P.
//   Scores: wave w owns heads 16w .. 16w+15:
//     S^T[16 tok x 16 heads] = C[16 tok x DQK] . Q^T on v_mfma_f32_16x16x32_f16,
//     the A operand read from the [token][dim] tile, Q resident in registers.
//     Online softmax per head in the exp2 domain (max shared by the four lane
//     groups, lazy rescale with 2^8 head-room as in the paged decode).
//   Values: wave w owns value dims (DV/4)w .. (DV/4)(w+1)-1 for all 64 heads:
//     O[16 heads x 16 dims] += P[16 heads x 16 tok] . C[16 tok x 16 dims] on
//     v_mfma_f32_16x16x16f16; P comes through LDS in the A-operand layout the
//     score result already has, C from the [dim][token] tile.
//   Splits write (m, l, acc) partials merged by splitk_merge_kernel; a sequence
//   that fits one split writes the output directly.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "iak.h"
#include "iak_internal.h"
#include "iak_device.h"

namespace iak {

template <int DQK, int DV> struct Mla {
  static constexpr int WAVES = 4;
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int QB = 1;                 // score head blocks (of 16) per wave
  static constexpr int HEADS = 16 * QB * WAVES;  // heads per workgroup
  static constexpr int HB = HEADS / 16;
  static constexpr int KSTEPS = DQK / 32;      // score k-steps
  static constexpr int DVW = DV / WAVES;       // value dims per wave
  static constexpr int NDB = DVW / 16;         // 16-dim blocks per wave
  static constexpr int T1 = DQK + 8;           // [token][dim] row stride (halves)
  static constexpr int T2 = 20;                // [dim][token] row stride (halves)
  static constexpr int UNITS16 = PS * DQK * 2 / 16;   // 16-byte units of an FP16 page
  static constexpr int UNITS8 = PS * DQK / 16;         // of a one-byte page
  static constexpr int U = (UNITS16 + THREADS - 1) / THREADS;   // loads per thread per page
  static constexpr int TASKS = DQK;            // 4 tokens x 4 dims per staging task
  static_assert(DQK % 32 == 0 && DV % 64 == 0 && DV <= DQK, "unsupported MLA shape");
};

template <int DQK, int DV> struct MlaShared {
  _Float16 t1[2][PS][Mla<DQK, DV>::T1];   // [buffer][token][dim]
  _Float16 t2[2][DV][Mla<DQK, DV>::T2];   // [buffer][value dim][token]
  u4 raw[Mla<DQK, DV>::UNITS8];           // one-byte codes of the page being staged
  u2 pbuf[Mla<DQK, DV>::HB][64];          // P of every head block, A-operand layout
  alignas(16) float alpha[Mla<DQK, DV>::HEADS];   // rescale factor of every head this page
  float lsum[Mla<DQK, DV>::HEADS];        // final denominators
  float mmax[Mla<DQK, DV>::HEADS];        // final maxima
  int grow[Mla<DQK, DV>::WAVES];
};

// Registers of one page being staged by this thread.
template <int DQK, int DV> struct MlaRegs {
  u4 r[Mla<DQK, DV>::U];
};

// Page metadata of one split: lane i holds entry i.
struct MlaPages {
  int pid, tag;
  float scale;
};

// Entries past the row's count, invalid ids, SKIP pages and pages whose first
// token lies at or past the sequence's token bound are left out (pid -1).
__device__ __forceinline__ MlaPages mla_page_meta(const MArgs& a, int b, int start, int lane, int limit) {
  MlaPages m{-1, IAK_TAG_SKIP, 1.0f};
  int raw = -1;
  if (lane < a.chunk && start + lane < a.W) raw = a.table[(int64_t)b * a.W + start + lane];
  int cnt = a.counts[b];
  cnt = cnt < 0 ? 0 : (cnt > a.W ? a.W : cnt);
  int n = cnt - start < a.chunk ? cnt - start : a.chunk;
  if (lane < n && (int64_t)(start + lane) * PS < limit) {
    int p = raw;
    if (a.neg_wrap && p < 0 && (int64_t)p >= -a.NP) p = (int)((int64_t)p + a.NP);
    if (p >= 0 && (int64_t)p < a.NP) {
      int t = IAK_TAG_FP16;
      if (a.tags) {
        const int ct = a.tags[p];
        t = (ct >= 0 && ct < 8) ? (int)((a.tagmap >> (8 * ct)) & 0xFFu) : IAK_TAG_SKIP;
      }
      if (t == IAK_TAG_FP16 || t == IAK_TAG_FP8 || t == IAK_TAG_INT8) {
        m.pid = p;
        m.tag = t;
        if (t == IAK_TAG_FP8) m.scale = load_scale(a.s8f, p, a.sd);
        if (t == IAK_TAG_INT8) m.scale = load_scale(a.s8i, p, a.sd);
      }
    }
  }
  return m;
}

// Global -> registers: the U 16-byte units of page `pid` this thread stages
// (unit tid + THREADS*k; past the page's last unit the last unit is loaded
// again, so every page issues the same loads).
template <int DQK, int DV>
__device__ __forceinline__ void mla_stage_load(MlaRegs<DQK, DV>& rg, const MArgs& a, int pid, int tag, int tid) {
  using C = Mla<DQK, DV>;
  const bool wide = tag == IAK_TAG_FP16;
  const int units = wide ? C::UNITS16 : C::UNITS8;
  const uint8_t* base = wide ? reinterpret_cast<const uint8_t*>(a.c16) + (int64_t)pid * PS * DQK * 2
                             : reinterpret_cast<const uint8_t*>(tag == IAK_TAG_FP8 ? a.c8f : a.c8i) +
                                   (int64_t)pid * PS * DQK;
#pragma unroll
  for (int k = 0; k < C::U; ++k) {
    int u = tid + C::THREADS * k;
    u = u < units ? u : units - 1;
    rg.r[k] = *reinterpret_cast<const u4*>(base + (int64_t)u * 16);
  }
}

// Registers -> LDS: FP16 units straight into the [token][dim] tile, one-byte
// codes into the raw buffer.
template <int DQK, int DV>
__device__ __forceinline__ void mla_stage_store(MlaShared<DQK, DV>& sh, const MlaRegs<DQK, DV>& rg, int buf,
                                                int tag, int tid) {
  using C = Mla<DQK, DV>;
  if (tag == IAK_TAG_FP16) {
#pragma unroll
    for (int k = 0; k < C::U; ++k) {
      const int u = tid + C::THREADS * k;
      if (u < C::UNITS16) {
        const int t = u / (DQK / 8), d = 8 * (u % (DQK / 8));
        *reinterpret_cast<u4*>(&sh.t1[buf][t][d]) = rg.r[k];
      }
    }
  } else {
#pragma unroll
    for (int k = 0; k < C::U; ++k) {
      const int u = tid + C::THREADS * k;
      if (u < C::UNITS8) sh.raw[u] = rg.r[k];
    }
  }
}

// LDS -> tiles: each task takes 4 tokens x 4 dims, converts one-byte codes to
// f16 (exact) into the [token][dim] tile and writes the value dims transposed
// into the [dim][token] tile.
template <int DQK, int DV>
__device__ __forceinline__ void mla_stage_tiles(MlaShared<DQK, DV>& sh, int buf, int tag, int voff, int tid) {
  using C = Mla<DQK, DV>;
  for (int task = tid; task < C::TASKS; task += C::THREADS) {
    const int tg = task / (DQK / 4), d = 4 * (task % (DQK / 4));
    uint32_t lo[4], hi[4];   // token 4tg+t: f16 pairs (d, d+1), (d+2, d+3)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int tok = 4 * tg + t;
      if (tag == IAK_TAG_FP16) {
        const u2 x = *reinterpret_cast<const u2*>(&sh.t1[buf][tok][d]);
        lo[t] = x[0];
        hi[t] = x[1];
      } else {
        const uint32_t x = reinterpret_cast<const uint32_t*>(sh.raw)[(tok * DQK + d) / 4];
        if (tag == IAK_TAG_FP8) fp8x4_to_f16(x, lo[t], hi[t]);
        else i8x4_to_f16(x, lo[t], hi[t]);
        *reinterpret_cast<u2*>(&sh.t1[buf][tok][d]) = u2{lo[t], hi[t]};
      }
    }
    const int vd = d - voff;
    if (vd >= 0 && vd < DV) {
      *reinterpret_cast<u2*>(&sh.t2[buf][vd + 0][4 * tg]) = u2{pack_lo(lo[0], lo[1]), pack_lo(lo[2], lo[3])};
      *reinterpret_cast<u2*>(&sh.t2[buf][vd + 1][4 * tg]) = u2{pack_hi(lo[0], lo[1]), pack_hi(lo[2], lo[3])};
      *reinterpret_cast<u2*>(&sh.t2[buf][vd + 2][4 * tg]) = u2{pack_lo(hi[0], hi[1]), pack_lo(hi[2], hi[3])};
      *reinterpret_cast<u2*>(&sh.t2[buf][vd + 3][4 * tg]) = u2{pack_hi(hi[0], hi[1]), pack_hi(hi[2], hi[3])};
    }
  }
}

template <int DQK, int DV>
__global__ __launch_bounds__(256, 1) void mla_decode_kernel(const MArgs a) {
  using C = Mla<DQK, DV>;
  __shared__ MlaShared<DQK, DV> sh;
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int b = blockIdx.x / a.splits;
  const int split = blockIdx.x - b * a.splits;
  const int hg = blockIdx.y;
  const int start = split * a.chunk;

  // token bound of the sequence (table entry e holds tokens 16e .. 16e+15)
  const int limit = a.valid ? __builtin_amdgcn_readfirstlane(a.valid[b]) : 0x7FFFFFFF;
  const MlaPages meta = mla_page_meta(a, b, start, lane, limit);
  const uint64_t mask = __builtin_amdgcn_ballot_w64(meta.pid >= 0);
  const int np = __builtin_popcountll(mask);

  // Q of the wave's head blocks, rounded to f16: dims 32i + 8g .. +7 of head c
  h8 q[C::QB][C::KSTEPS];
#pragma unroll
  for (int k = 0; k < C::QB; ++k) {
    const int h = hg * C::HEADS + 16 * (C::QB * w + k) + c;
    const bool live = h < a.H;
    const int64_t off = (int64_t)b * a.qsb + (int64_t)(live ? h : 0) * a.qsh + 8 * g;
#pragma unroll
    for (int i = 0; i < C::KSTEPS; ++i) {
      h8 v;
      if (a.q_dtype == IAK_DTYPE_F16) {
        v = *reinterpret_cast<const h8*>(reinterpret_cast<const _Float16*>(a.q) + off + 32 * i);
      } else if (a.q_dtype == IAK_DTYPE_F32) {
        const f4* p = reinterpret_cast<const f4*>(reinterpret_cast<const float*>(a.q) + off + 32 * i);
        const f4 x0 = p[0], x1 = p[1];
#pragma unroll
        for (int e = 0; e < 4; ++e) { v[e] = (_Float16)x0[e]; v[4 + e] = (_Float16)x1[e]; }
      } else {
        const u4 x = *reinterpret_cast<const u4*>(reinterpret_cast<const uint16_t*>(a.q) + off + 32 * i);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[2 * e] = (_Float16)u2f(x[e] << 16);
          v[2 * e + 1] = (_Float16)u2f(x[e] & 0xFFFF0000u);
        }
      }
      if (!live) v = h8{0, 0, 0, 0, 0, 0, 0, 0};
      q[k][i] = v;
    }
  }

  float m[C::QB], l[C::QB];
#pragma unroll
  for (int k = 0; k < C::QB; ++k) { m[k] = -__builtin_inff(); l[k] = 0.f; }
  f4 acc[C::HB][C::NDB];
#pragma unroll
  for (int hb = 0; hb < C::HB; ++hb)
#pragma unroll
    for (int db = 0; db < C::NDB; ++db) acc[hb][db] = f4{0.f, 0.f, 0.f, 0.f};

  if (np > 0) {
    // page cursor: lanes of the pages in table order; past the end the last
    // page is named again (loads stay unconditional, compute is skipped)
    uint64_t rem = mask;
    int last = __builtin_ctzll(mask);
    auto next_page = [&]() {
      if (rem) last = take(rem);
      return last;
    };
    MlaRegs<DQK, DV> regs[2];
    int idx0 = next_page();
    int idx1 = next_page();
    mla_stage_load<DQK, DV>(regs[0], a, __builtin_amdgcn_readlane(meta.pid, idx0),
                            __builtin_amdgcn_readlane(meta.tag, idx0), tid);
    mla_stage_load<DQK, DV>(regs[1], a, __builtin_amdgcn_readlane(meta.pid, idx1),
                            __builtin_amdgcn_readlane(meta.tag, idx1), tid);
    {
      const int tag0 = __builtin_amdgcn_readlane(meta.tag, idx0);
      mla_stage_store<DQK, DV>(sh, regs[0], 0, tag0, tid);
      __syncthreads();
      mla_stage_tiles<DQK, DV>(sh, 0, tag0, a.VOFF, tid);
      __syncthreads();
    }
    int cur = idx0, nxt = idx1;

    // One page: stage page j+1 into the other buffer, then scores and values
    // of page j. `R` is the buffer (and register set) of page j.
    auto step = [&](auto RC, int j) {
      constexpr int R = decltype(RC)::value;
      const int idx2 = next_page();
      mla_stage_load<DQK, DV>(regs[R], a, __builtin_amdgcn_readlane(meta.pid, idx2),
                              __builtin_amdgcn_readlane(meta.tag, idx2), tid);
      const bool have_next = j + 1 < np;
      const int tagn = __builtin_amdgcn_readlane(meta.tag, nxt);
      if (have_next) mla_stage_store<DQK, DV>(sh, regs[1 - R], 1 - R, tagn, tid);
      __syncthreads();
      if (have_next) mla_stage_tiles<DQK, DV>(sh, 1 - R, tagn, a.VOFF, tid);

      if (j >= np) return;
      // ---- scores of page j (buffer R) for the wave's head blocks ----
      const float pscale = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, meta.scale), cur));
      const float smul = a.score_mult * pscale;
      f4 s[C::QB];
#pragma unroll
      for (int k = 0; k < C::QB; ++k) s[k] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < C::KSTEPS; ++i) {
        const h8 av = *reinterpret_cast<const h8*>(&sh.t1[R][c][32 * i + 8 * g]);
#pragma unroll
        for (int k = 0; k < C::QB; ++k) s[k] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, q[k][i], s[k], 0, 0, 0);
      }
      float pm[C::QB];
      bool grow[C::QB];
      bool wgrow = false;
      // tokens at or past the bound (only in the sequence's last visited page)
      const int64_t tok0 = (int64_t)(start + cur) * PS + 4 * g;
      const bool ragged = (int64_t)(start + cur) * PS + PS > limit;
#pragma unroll
      for (int k = 0; k < C::QB; ++k) {
        s[k] *= smul;
        if (ragged) {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (tok0 + r >= limit) s[k][r] = -__builtin_inff();
        }
        pm[k] = xmax16_32(fmaxf(fmaxf(s[k][0], s[k][1]), fmaxf(s[k][2], s[k][3])));
        grow[k] = pm[k] > m[k] + RESCALE_SLACK;
        wgrow = wgrow || grow[k];
      }
      const bool any = __builtin_amdgcn_ballot_w64(wgrow) != 0;
#pragma unroll
      for (int k = 0; k < C::QB; ++k) {
        float al = 1.0f;
        if (any) {
          const float mn = grow[k] ? pm[k] : m[k];
          al = __builtin_amdgcn_exp2f(m[k] - mn);   // 0 on the first page (m = -inf)
          l[k] *= al;
          m[k] = mn;
        }
        const float p0 = __builtin_amdgcn_exp2f(s[k][0] - m[k]);
        const float p1 = __builtin_amdgcn_exp2f(s[k][1] - m[k]);
        const float p2 = __builtin_amdgcn_exp2f(s[k][2] - m[k]);
        const float p3 = __builtin_amdgcn_exp2f(s[k][3] - m[k]);
        l[k] += (p0 + p1) + (p2 + p3);
        typedef float f2 __attribute__((ext_vector_type(2)));
        const h2 x = __builtin_convertvector((f2{p0, p1} * pscale), h2);
        const h2 y = __builtin_convertvector((f2{p2, p3} * pscale), h2);
        sh.pbuf[C::QB * w + k][lane] = u2{bits(x), bits(y)};
        if (g == 0) sh.alpha[16 * (C::QB * w + k) + c] = al;
      }
      if (lane == 0) sh.grow[w] = any ? 1 : 0;
      __syncthreads();

      // ---- values of page j: all the workgroup's heads, the wave's value dims ----
      if (sh.grow[0] | sh.grow[1] | sh.grow[2] | sh.grow[3]) {
#pragma unroll
        for (int hb = 0; hb < C::HB; ++hb) {
          const f4 al = *reinterpret_cast<const f4*>(&sh.alpha[16 * hb + 4 * g]);
#pragma unroll
          for (int db = 0; db < C::NDB; ++db) acc[hb][db] *= al;
        }
      }
      h4 bop[C::NDB];
#pragma unroll
      for (int db = 0; db < C::NDB; ++db)
        bop[db] = *reinterpret_cast<const h4*>(&sh.t2[R][C::DVW * w + 16 * db + c][4 * g]);
#pragma unroll
      for (int hb = 0; hb < C::HB; ++hb) {
        const h4 aop = __builtin_bit_cast(h4, sh.pbuf[hb][lane]);
#pragma unroll
        for (int db = 0; db < C::NDB; ++db)
          acc[hb][db] = __builtin_amdgcn_mfma_f32_16x16x16f16(aop, bop[db], acc[hb][db], 0, 0, 0);
      }
      cur = nxt;
      nxt = idx2;
    };

    // pages in pairs so the buffer and register-set indices are static
    // (both steps of a pair always run -- an exit between them makes the
    // compiler keep two copies of the accumulators -- and a step past the end
    // issues its loads but skips its compute)
    for (int j = 0; j < np; j += 2) {
      step(std::integral_constant<int, 0>{}, j);
      step(std::integral_constant<int, 1>{}, j + 1);
    }
  }

  // ---- denominators and maxima of every head, then the output or the partials ----
#pragma unroll
  for (int k = 0; k < C::QB; ++k) {
    const float ls = xsum16_32(l[k]);
    if (g == 0) {
      sh.lsum[16 * (C::QB * w + k) + c] = ls;
      sh.mmax[16 * (C::QB * w + k) + c] = m[k];
    }
  }
  __syncthreads();
#pragma unroll
  for (int hb = 0; hb < C::HB; ++hb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int hl = 16 * hb + 4 * g + r;
      const int h = hg * C::HEADS + hl;
      if (h >= a.H) continue;
      if (a.splits == 1) {
        const float ls = sh.lsum[hl];
        const float inv = ls > 0.f ? 1.0f / ls : 0.0f;
        const int64_t o = (int64_t)b * a.osb + (int64_t)h * a.osh + C::DVW * w + c;
#pragma unroll
        for (int db = 0; db < C::NDB; ++db) {
          const float v = acc[hb][db][r] * inv;
          if (a.out_dtype == IAK_DTYPE_F32) reinterpret_cast<float*>(a.out)[o + 16 * db] = v;
          else if (a.out_dtype == IAK_DTYPE_F16) reinterpret_cast<_Float16*>(a.out)[o + 16 * db] = (_Float16)v;
          else reinterpret_cast<__bf16*>(a.out)[o + 16 * db] = (__bf16)v;
        }
      } else {
        const int64_t slot = ((int64_t)b * a.splits + split) * a.H + h;
        if (w == 0 && c == 0) {
          a.ws_m[slot] = sh.mmax[hl];
          a.ws_l[slot] = sh.lsum[hl];
        }
        float* op = a.ws_acc + slot * DV + C::DVW * w + c;
#pragma unroll
        for (int db = 0; db < C::NDB; ++db) op[16 * db] = acc[hb][db][r];
      }
    }
  }
}

template <int DQK, int DV>
hipError_t launch_mla(const MArgs& m, hipStream_t stream) {
  hipLaunchKernelGGL((mla_decode_kernel<DQK, DV>), dim3(m.B * m.splits, m.HG), dim3(Mla<DQK, DV>::THREADS), 0,
                     stream, m);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || m.splits == 1) return e;
  // the paged-decode merge over rows (b, 0) of H heads
  KArgs k{};
  k.B = m.B; k.Hq = m.H; k.Hkv = 1; k.G = m.H; k.D = DV; k.splits = m.splits;
  k.out = m.out; k.out_dtype = m.out_dtype; k.osb = m.osb; k.osh = m.osh;
  k.ws_m = m.ws_m; k.ws_l = m.ws_l; k.ws_acc = m.ws_acc;
  const int mblocks = (m.B * m.H + 3) / 4;
  hipLaunchKernelGGL((splitk_merge_kernel<DV>), dim3(mblocks), dim3(256), 0, stream, k);
  return hipGetLastError();
}

hipError_t launch_mla_decode(const MArgs& m, hipStream_t stream) {
  switch (m.DQK * 1000 + m.DV) {
    case 64064: return launch_mla<64, 64>(m, stream);
    case 128128: return launch_mla<128, 128>(m, stream);
    case 256256: return launch_mla<256, 256>(m, stream);
    case 512512: return launch_mla<512, 512>(m, stream);
    case 576512: return launch_mla<576, 512>(m, stream);
    case 576064: return launch_mla<576, 64>(m, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace iak
