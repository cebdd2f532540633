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
//   One workgroup of 8 waves (two per SIMD, up to 256 registers each) reduces
//   one split -- up to 64 consecutive page-table entries of one sequence -- for
//   128 heads, so each latent page is read from HBM once per sequence. Pages
//   stream from HBM straight into an LDS ring (global_load_lds), three pages
//   ahead, and are staged once per workgroup as two f16 tiles: [token][dim]
//   for the score product and [dim][token] (value dims) for the value product.
//   FP8 / INT8 codes are converted to f16 exactly while staging; the page
//   scale folds into the score multiplier and into P.
//   Wave w owns heads 16w .. 16w+15 end to end (its score and value
//   accumulators live in VGPRs: this file is built with MFMA results in VGPRs,
//   so the softmax rescale is plain VALU work):
//     scores  S^T[16 tok x 16 heads] = C[16 tok x DQK] . Q^T on
//             v_mfma_f32_16x16x32_f16, C from the [token][dim] tile, Q
//             resident in registers;
//     softmax online per head in the exp2 domain (max shared by the four lane
//             groups, lazy rescale with 2^8 head-room as in the paged decode),
//             entirely inside the wave;
//     values  O[16 heads x 16 dims] += P[16 heads x 16 tok] . C[16 tok x 16 dims]
//             on v_mfma_f32_16x16x16f16 for all DV dims: the score result's
//             register layout (lane: head column, four consecutive tokens) is
//             exactly the A operand P, so P never leaves the registers; C comes
//             from the [dim][token] tile.
//   Two barriers per page (tile ready; tile buffer free). Splits write (m, l,
//   acc) partials merged by splitk_merge_kernel; a sequence that fits one
//   split writes the output directly.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "iak.h"
#include "iak_internal.h"
#include "iak_device.h"

namespace iak {

template <int DQK, int DV, bool WIDE> struct Mla {
  static constexpr int WAVES = 8;              // two per SIMD
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int HT = 1;                 // 16-head tiles per wave
  static constexpr int HEADS = 16 * HT * WAVES;  // heads per workgroup
  static constexpr int KSTEPS = DQK / 32;      // score k-steps
  static constexpr int NDB = DV / 16;          // 16-dim value blocks (all of them, per wave)
  static constexpr int T1 = DQK + 8;           // [token][dim] row stride (halves)
  static constexpr int T2 = 20;                // [dim][token] row stride (halves)
  static constexpr int PAGE8 = PS * DQK;       // bytes of a one-byte page (a multiple of 1 KB)
  static constexpr int SLOT = WIDE ? 2 * PAGE8 : PAGE8;   // raw ring slot: the widest page
  static constexpr int NDMA = (SLOT / 1024 + WAVES - 1) / WAVES;   // 1 KB copies per wave per page
  static constexpr int RING = WIDE ? 4 : 5;    // raw slots; pages stream RING - 2 steps ahead of staging
  static constexpr int TASKS = DQK;            // 4 tokens x 4 dims per staging task
  static_assert(DQK % 32 == 0 && DV % 16 == 0 && DV <= DQK && PAGE8 % 1024 == 0, "unsupported MLA shape");
};

template <int DQK, int DV, bool WIDE> struct MlaShared {
  using C = Mla<DQK, DV, WIDE>;
  _Float16 t1[2][PS][C::T1];              // [buffer][token][dim]
  _Float16 t2[2][DV][C::T2];              // [buffer][value dim][token]
  alignas(16) uint8_t ring[C::RING][C::SLOT];   // raw pages as copied from HBM
  float lsum[C::HEADS];                   // final denominators
  float mmax[C::HEADS];                   // final maxima
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

// HBM -> LDS ring slot: the page's 1 KB chunks are copied straight into LDS
// (global_load_lds_dwordx4: lane i's 16 bytes land at the slot offset + 16 i),
// chunk w + WAVES*k by wave w. Every wave issues NDMA copies per page -- past
// the page's last chunk the last chunk is copied again -- so the number of
// copies in flight per wave is fixed and each wait is a constant vmcnt. The
// copies bypass the registers; the compiler does not see them, so the waits
// for them are written out (mla_wait_pages) and no compiler-issued load runs
// inside the page loop.
template <int DQK, int DV, bool WIDE>
__device__ __forceinline__ void mla_dma_page(MlaShared<DQK, DV, WIDE>& sh, int slot, const MArgs& a, int pid,
                                             int tag, int w, int lane) {
  using C = Mla<DQK, DV, WIDE>;
  const bool wide = WIDE && tag == IAK_TAG_FP16;
  const int nch = (wide ? 2 * C::PAGE8 : C::PAGE8) / 1024;
  const uint8_t* base = wide ? reinterpret_cast<const uint8_t*>(a.c16) + (int64_t)pid * C::PAGE8 * 2
                             : reinterpret_cast<const uint8_t*>(tag == IAK_TAG_FP8 ? a.c8f : a.c8i) +
                                   (int64_t)pid * C::PAGE8;
  typedef __attribute__((address_space(3))) uint8_t lds_u8;
#pragma unroll
  for (int k = 0; k < C::NDMA; ++k) {
    int ch = w + C::WAVES * k;
    ch = ch < nch ? ch : nch - 1;
    const uint8_t* src = base + (int64_t)ch * 1024 + 16 * lane;
    const uint32_t dst = (uint32_t)(uintptr_t)(lds_u8*)&sh.ring[slot][ch * 1024];
    asm volatile("global_load_lds_dwordx4 %0, off" : : "v"(src), "{m0}"(dst) : "memory");
  }
}

// Wait until at most `pages` pages of this wave's ring copies are in flight.
template <int NDMA, int PAGES> __device__ __forceinline__ void mla_wait_pages() {
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(NDMA * PAGES) : "memory");
}

// LDS -> tiles: each task takes 4 tokens x 4 dims, converts one-byte codes to
// f16 (exact) into the [token][dim] tile and writes the value dims transposed
// into the [dim][token] tile.
template <int DQK, int DV, bool WIDE>
__device__ __forceinline__ void mla_stage_tiles(MlaShared<DQK, DV, WIDE>& sh, int slot, int buf, int tag, int voff,
                                                int tid) {
  using C = Mla<DQK, DV, WIDE>;
  constexpr int NB = DQK / 4;   // 4-dim blocks
  static_assert(NB % 16 == 0, "staging lane map needs a multiple of 16 dim blocks");
  for (int task = tid; task < C::TASKS; task += C::THREADS) {
    // lane map: token group = task % 4, dim block = 16 (task / 64 + tg) +
    // (task / 4) % 16 (mod NB), a bijection onto (tg, block). For DQK = 576 the
    // token groups' rows start on the same LDS bank; the skew of 16 blocks per
    // group spreads the ring reads over all banks, and the [dim][token] writes
    // of a wave cover every bank twice (the minimum for 512 bytes).
    const int tg = task & 3;
    const int blk = (16 * ((task >> 6) + tg) + ((task >> 2) & 15)) % NB;
    const int d = 4 * blk;
    uint32_t lo[4], hi[4];   // token 4tg+t: f16 pairs (d, d+1), (d+2, d+3)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int tok = 4 * tg + t;
      if (WIDE && tag == IAK_TAG_FP16) {
        const u2 x = *reinterpret_cast<const u2*>(&sh.ring[slot][(tok * DQK + d) * 2]);
        lo[t] = x[0];
        hi[t] = x[1];
      } else {
        const uint32_t x = *reinterpret_cast<const uint32_t*>(&sh.ring[slot][tok * DQK + d]);
        if (tag == IAK_TAG_FP8) fp8x4_to_f16(x, lo[t], hi[t]);
        else i8x4_to_f16(x, lo[t], hi[t]);
      }
      *reinterpret_cast<u2*>(&sh.t1[buf][tok][d]) = u2{lo[t], hi[t]};
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

template <int DQK, int DV, bool WIDE>
__global__ __launch_bounds__(512, 1) void mla_decode_kernel(const MArgs a) {
  using C = Mla<DQK, DV, WIDE>;
  __shared__ MlaShared<DQK, DV, WIDE> sh;
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int b = blockIdx.x / a.splits;
  const int split = blockIdx.x - b * a.splits;
  const int hg = blockIdx.y;
  const int start = split * a.chunk;
  const int head0 = hg * C::HEADS + 16 * C::HT * w;   // first head of this wave

  // token bound of the sequence (table entry e holds tokens 16e .. 16e+15)
  const int limit = a.valid ? __builtin_amdgcn_readfirstlane(a.valid[b]) : 0x7FFFFFFF;
  const MlaPages meta = mla_page_meta(a, b, start, lane, limit);
  const uint64_t mask = __builtin_amdgcn_ballot_w64(meta.pid >= 0);
  const int np = __builtin_popcountll(mask);

  // Q of the wave's head tiles, rounded to f16: dims 32i + 8g .. +7 of head c
  h8 q[C::HT][C::KSTEPS];
#pragma unroll
  for (int k = 0; k < C::HT; ++k) {
    const int h = head0 + 16 * k + c;
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

  // per lane: running max and partial denominator of head column c of tile k
  // (the partial covers the lane's four token rows; summed over g at the end)
  float m[C::HT], l[C::HT];
#pragma unroll
  for (int k = 0; k < C::HT; ++k) { m[k] = -__builtin_inff(); l[k] = 0.f; }
  // O tile (k, db): rows = heads 4g .. 4g+3 of tile k, column = value dim 16 db + c
  f4 acc[C::HT][C::NDB];
#pragma unroll
  for (int k = 0; k < C::HT; ++k)
#pragma unroll
    for (int db = 0; db < C::NDB; ++db) acc[k][db] = f4{0.f, 0.f, 0.f, 0.f};

  if (np > 0) {
    // page cursor: lanes of the pages in table order; past the end the last
    // page is named again (loads stay unconditional, compute is skipped)
    uint64_t rem = mask;
    int last = __builtin_ctzll(mask);
    auto next_page = [&]() {
      if (rem) last = take(rem);
      return last;
    };
    auto page_pid = [&](int idx) { return __builtin_amdgcn_readlane(meta.pid, idx); };
    auto page_tag = [&](int idx) { return __builtin_amdgcn_readlane(meta.tag, idx); };
    // pages 0 .. RING-2 start streaming into ring slots 0 .. RING-2; page 0 is
    // staged into tile buffer 0. qi[k] = lane of page j+k.
    int qi[C::RING - 1];
#pragma unroll
    for (int k = 0; k < C::RING - 1; ++k) {
      qi[k] = next_page();
      mla_dma_page<DQK, DV, WIDE>(sh, k, a, page_pid(qi[k]), page_tag(qi[k]), w, lane);
    }
    mla_wait_pages<C::NDMA, C::RING - 2>();
    __syncthreads();
    mla_stage_tiles<DQK, DV, WIDE>(sh, 0, 0, page_tag(qi[0]), a.VOFF, tid);

    // One page per iteration and one barrier: each wave waits for its copies
    // of page j+1, then the barrier makes page j's tiles (staged in the
    // previous iteration) and page j+1's raw bytes visible to every wave and
    // ends every read of the other tile buffer. Then page j+RING-1 starts
    // streaming, page j+1 is staged into the other buffer while the scores of
    // page j run on the matrix cores, and the softmax and values of page j
    // follow. R = j & 1 is the tile buffer of page j; page p streams into ring
    // slot p % RING.
    int slot_new = C::RING - 1, slot_nxt = 1;
    for (int j = 0; j < np; ++j) {
      const int R = j & 1;
      const int cur = qi[0], nxt = qi[1];
      mla_wait_pages<C::NDMA, C::RING - 3>();
      __syncthreads();
      const int inew = next_page();
      mla_dma_page<DQK, DV, WIDE>(sh, slot_new, a, page_pid(inew), page_tag(inew), w, lane);

      // ---- scores of page j (buffer R), issued first so the MFMAs run while
      // the wave stages page j+1 ----
      constexpr int NCH = C::KSTEPS >= 2 ? 2 : 1;    // chains per head tile
      f4 sc[C::HT][NCH];
#pragma unroll
      for (int k = 0; k < C::HT; ++k)
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) sc[k][ch] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < C::KSTEPS; ++i) {
        const h8 av = *reinterpret_cast<const h8*>(&sh.t1[R][c][32 * i + 8 * g]);
#pragma unroll
        for (int k = 0; k < C::HT; ++k)
          sc[k][i % NCH] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, q[k][i], sc[k][i % NCH], 0, 0, 0);
      }

      // ---- stage page j+1 (landed before the barrier) ----
      const bool have_next = j + 1 < np;
      if (have_next) mla_stage_tiles<DQK, DV, WIDE>(sh, slot_nxt, 1 - R, page_tag(nxt), a.VOFF, tid);
#pragma unroll
      for (int k = 0; k < C::RING - 2; ++k) qi[k] = qi[k + 1];
      qi[C::RING - 2] = inew;
      slot_new = slot_new + 1 == C::RING ? 0 : slot_new + 1;
      slot_nxt = slot_nxt + 1 == C::RING ? 0 : slot_nxt + 1;

      const float pscale = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, meta.scale), cur));
      const float smul = a.score_mult * pscale;
      // tokens at or past the bound (only in the sequence's last visited page)
      const int64_t tok0 = (int64_t)(start + cur) * PS + 4 * g;
      const bool ragged = (int64_t)(start + cur) * PS + PS > limit;
      h4 pa[C::HT];        // P of tile k: A operand (row = head c, k = tokens 4g .. 4g+3)
      float al[C::HT];
      bool grow_any = false;
#pragma unroll
      for (int k = 0; k < C::HT; ++k) {
        f4 s = sc[k][0];
#pragma unroll
        for (int ch = 1; ch < NCH; ++ch) s += sc[k][ch];
        s *= smul;
        if (ragged) {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (tok0 + r >= limit) s[r] = -__builtin_inff();
        }
        const float pm = xmax16_32(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])));
        const bool grow = pm > m[k] + RESCALE_SLACK;
        al[k] = 1.0f;
        if (grow) {
          al[k] = __builtin_amdgcn_exp2f(m[k] - pm);   // 0 on the first page (m = -inf)
          m[k] = pm;
        }
        grow_any = grow_any || grow;
        const float p0 = __builtin_amdgcn_exp2f(s[0] - m[k]);
        const float p1 = __builtin_amdgcn_exp2f(s[1] - m[k]);
        const float p2 = __builtin_amdgcn_exp2f(s[2] - m[k]);
        const float p3 = __builtin_amdgcn_exp2f(s[3] - m[k]);
        l[k] = l[k] * al[k] + ((p0 + p1) + (p2 + p3));
        typedef float f2 __attribute__((ext_vector_type(2)));
        const h2 x = __builtin_convertvector((f2{p0, p1} * pscale), h2);
        const h2 y = __builtin_convertvector((f2{p2, p3} * pscale), h2);
        pa[k] = __builtin_bit_cast(h4, u2{bits(x), bits(y)});
      }
      // rescale: the O rows are heads 4g + r, whose factor sits in lane 4g + r
      if (__builtin_amdgcn_ballot_w64(grow_any) != 0) {
#pragma unroll
        for (int k = 0; k < C::HT; ++k) {
          f4 ar;
#pragma unroll
          for (int r = 0; r < 4; ++r) ar[r] = __shfl(al[k], 4 * g + r, 64);
#pragma unroll
          for (int db = 0; db < C::NDB; ++db) acc[k][db] *= ar;
        }
      }

      // ---- values of page j: the wave's heads, every value dim ----
#pragma unroll
      for (int db = 0; db < C::NDB; ++db) {
        const h4 bop = *reinterpret_cast<const h4*>(&sh.t2[R][16 * db + c][4 * g]);
#pragma unroll
        for (int k = 0; k < C::HT; ++k)
          acc[k][db] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa[k], bop, acc[k][db], 0, 0, 0);
      }
    }
    // the copies of the pages past the end land before the LDS is reused or released
    mla_wait_pages<C::NDMA, 0>();
  }

  // ---- denominators and maxima of the wave's heads, then the output or the partials ----
#pragma unroll
  for (int k = 0; k < C::HT; ++k) {
    const float ls = xsum16_32(l[k]);
    if (g == 0) {
      sh.lsum[16 * (C::HT * w + k) + c] = ls;
      sh.mmax[16 * (C::HT * w + k) + c] = m[k];
    }
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < C::HT; ++k) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int hl = 16 * (C::HT * w + k) + 4 * g + r;
      const int h = hg * C::HEADS + hl;
      if (h >= a.H) continue;
      if (a.splits == 1) {
        const float ls = sh.lsum[hl];
        const float inv = ls > 0.f ? 1.0f / ls : 0.0f;
        const int64_t o = (int64_t)b * a.osb + (int64_t)h * a.osh + c;
#pragma unroll
        for (int db = 0; db < C::NDB; ++db) {
          const float v = acc[k][db][r] * inv;
          if (a.out_dtype == IAK_DTYPE_F32) reinterpret_cast<float*>(a.out)[o + 16 * db] = v;
          else if (a.out_dtype == IAK_DTYPE_F16) reinterpret_cast<_Float16*>(a.out)[o + 16 * db] = (_Float16)v;
          else reinterpret_cast<__bf16*>(a.out)[o + 16 * db] = (__bf16)v;
        }
      } else {
        const int64_t slot = ((int64_t)b * a.splits + split) * a.H + h;
        if (c == 0) {
          a.ws_m[slot] = sh.mmax[hl];
          a.ws_l[slot] = sh.lsum[hl];
        }
        float* op = a.ws_acc + slot * DV + c;
#pragma unroll
        for (int db = 0; db < C::NDB; ++db) op[16 * db] = acc[k][db][r];
      }
    }
  }
}

template <int DQK, int DV, bool WIDE>
hipError_t launch_mla_w(const MArgs& m, hipStream_t stream, hipEvent_t ev_begin, hipEvent_t ev_end) {
  if (ev_begin) hipEventRecord(ev_begin, stream);
  hipLaunchKernelGGL((mla_decode_kernel<DQK, DV, WIDE>), dim3(m.B * m.splits, m.HG),
                     dim3(Mla<DQK, DV, WIDE>::THREADS), 0, stream, m);
  hipError_t e = hipGetLastError();
  if (ev_end) hipEventRecord(ev_end, stream);
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

// WIDE: FP16 latent pages are reachable (ring slots sized for two bytes per value)
template <int DQK, int DV>
hipError_t launch_mla(const MArgs& m, hipStream_t stream, hipEvent_t eb, hipEvent_t ee) {
  return m.wide ? launch_mla_w<DQK, DV, true>(m, stream, eb, ee) : launch_mla_w<DQK, DV, false>(m, stream, eb, ee);
}

hipError_t launch_mla_decode(const MArgs& m, hipStream_t stream, hipEvent_t eb, hipEvent_t ee) {
  switch (m.DQK * 1000 + m.DV) {
    case 64064: return launch_mla<64, 64>(m, stream, eb, ee);
    case 128128: return launch_mla<128, 128>(m, stream, eb, ee);
    case 256256: return launch_mla<256, 256>(m, stream, eb, ee);
    case 512512: return launch_mla<512, 512>(m, stream, eb, ee);
    case 576512: return launch_mla<576, 512>(m, stream, eb, ee);
    case 576064: return launch_mla<576, 64>(m, stream, eb, ee);
  }
  return hipErrorInvalidValue;
}

}  // namespace iak
