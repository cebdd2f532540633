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
//   one split -- up to 128 consecutive page-table entries of one sequence -- for
//   128 heads, so each latent page is read from HBM once per sequence. A step
//   is a pair of pages (32 tokens). Pages stream from HBM straight into an LDS
//   ring of page pairs (global_load_lds), SLOTS - 1 steps ahead, and each pair
//   is staged once per workgroup into one f16 tile [token][dim]; FP8 / INT8
//   codes convert to f16 exactly while staging, and the page scale folds into
//   the score multiplier and into P (relative to the wave's value exponent E,
//   as in the paged decode: P = p * s * 2^-E, the value sum is acc * 2^E).
//   Wave w owns heads 16w .. 16w+15 end to end (its score and value
//   accumulators live in VGPRs: this file is built with MFMA results in VGPRs,
//   so the softmax rescale is plain VALU work):
//     scores  S^T[16 tok x 16 heads] = C[16 tok x DQK] . Q^T per page on
//             v_mfma_f32_16x16x32_f16, C from the tile, Q resident in
//             registers;
//     softmax online per head over the pair's 32 tokens in the exp2 domain
//             (max shared by the four lane groups, lazy rescale with 2^8
//             head-room as in the paged decode), entirely inside the wave;
//     values  O[16 heads x 16 dims] += P[16 heads x 32 tok] . C[32 tok x 16 dims]
//             on v_mfma_f32_16x16x32_f16 for all DV dims: the two score
//             results' register layout (lane: head column, four consecutive
//             tokens of each page) is exactly the A operand P, so P never leaves
//             the registers; the C operand comes out of the same [token][dim]
//             tile through the transposing read ds_read_b64_tr_b16.
//   One barrier per pair: pair s+1 is staged into the other tile buffer while
//   pair s is computed. Splits write (m, l, acc) partials merged by
//   splitk_merge_kernel -- acc / l as float16 when every page is quantised and
//   the output is 16-bit (MArgs::acc16), which halves the partial traffic;
//   a sequence that fits one split writes the output directly.

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
  static constexpr int HEADS = 16 * WAVES;     // heads per workgroup (16 per wave)
  static constexpr int KSTEPS = DQK / 32;      // score k-steps
  static constexpr int NDB = DV / 16;          // 16-dim value blocks (all of them, per wave)
  static constexpr int TOK = 2 * PS;           // tokens per step: two pages
  // [token][dim] row stride (halves), = 16 mod 128: the 16-byte score-operand
  // reads of 16 rows and the 8-byte transposing value reads of 16 rows both
  // spread evenly over the 64 LDS banks
  static constexpr int T1 = DQK + ((16 - DQK) % 128 + 128) % 128;
  static constexpr int PAGE8 = PS * DQK;       // bytes of a one-byte page (a multiple of 1 KB)
  static constexpr int SLOT = WIDE ? 2 * PAGE8 : PAGE8;   // raw ring slot: the widest page
  static constexpr int NDMA = (SLOT / 1024 + WAVES - 1) / WAVES;   // 1 KB copies per wave per page
  static constexpr int SLOTS = WIDE ? 2 : 4;   // page pairs in the ring = steps a pair streams in ahead
  static constexpr int CHUNKS = DQK / 8;       // 8-value staging chunks per token
  // operand reads issued ahead of their MFMAs (score k-steps, value blocks):
  // the most the register budget holds without spilling; the MFMAs sit between
  // scheduling barriers so the compiler keeps the reads that far ahead
  static constexpr int PF_SCORE = 2;
  static constexpr int PF_VALUE = 4;
  static_assert(DQK % 32 == 0 && DV % 16 == 0 && DV <= DQK && PAGE8 % 1024 == 0, "unsupported MLA shape");
  static_assert((SLOTS & (SLOTS - 1)) == 0 && SLOTS >= 2, "ring of a power-of-two number of page pairs");
};

template <int DQK, int DV, bool WIDE> struct MlaShared {
  using C = Mla<DQK, DV, WIDE>;
  _Float16 t1[2][C::TOK][C::T1];                    // [buffer][token][dim], f16
  alignas(16) uint8_t ring[C::SLOTS][2][C::SLOT];   // raw page pairs as copied from HBM
  float lsum[C::HEADS];                             // final denominators
  float mmax[C::HEADS];                             // final maxima
};

// Page metadata of one split entry (lane i holds entries i and i + 64).
struct MlaPages {
  int pid, tag;
  float scale;
};

// Entries past the row's count, invalid ids, SKIP pages and pages whose first
// token lies at or past the sequence's token bound are left out (pid -1).
__device__ __forceinline__ MlaPages mla_page_meta(const MArgs& a, int b, int start, int e, int limit) {
  MlaPages m{-1, IAK_TAG_SKIP, 1.0f};
  int raw = -1;
  if (e < a.chunk && start + e < a.W) raw = a.table[(int64_t)b * a.W + start + e];
  int cnt = a.counts[b];
  cnt = cnt < 0 ? 0 : (cnt > a.W ? a.W : cnt);
  int n = cnt - start < a.chunk ? cnt - start : a.chunk;
  if (e < n && (int64_t)(start + e) * PS < limit) {
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
__device__ __forceinline__ void mla_dma_page(uint8_t* slot, const MArgs& a, int pid, int tag, int w, int lane) {
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
    const uint32_t dst = (uint32_t)(uintptr_t)(lds_u8*)(slot + ch * 1024);
    // the copy takes its LDS address from M0, which the compiler writes just
    // before this statement: one wait state between an SALU write of M0 and an
    // LDS DMA that reads it
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(src), "{m0}"(dst) : "memory");
  }
}

// Wait until at most `pages` pages of this wave's ring copies are in flight.
template <int NDMA, int PAGES> __device__ __forceinline__ void mla_wait_pages() {
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(NDMA * PAGES) : "memory");
}

// LDS ring -> [token][dim] f16 tile for a page pair. Sixteen threads share one
// token row (thread t: row t / 16, which is page t / 256, so every wave stages
// one page and its tag is wave-uniform); thread q of a row converts the 8-value
// chunks q, q + 16, ... of it (8 code bytes, or 16 bytes of f16, each). The
// offsets of a thread's chunks differ by constants, and a row's 16 chunks are
// contiguous in the ring and in the tile. FP8 / INT8 codes convert to f16
// exactly.
template <int DQK, int DV, bool WIDE>
__device__ __forceinline__ void mla_stage_pair(MlaShared<DQK, DV, WIDE>& sh, int slot, int buf, int tag0, int tag1,
                                               int tid) {
  using C = Mla<DQK, DV, WIDE>;
  static_assert(C::THREADS == 16 * C::TOK, "16 threads per staged row");
  constexpr int NJ = (C::CHUNKS + 15) / 16;   // chunks per thread (the last one partial)
  const int row = tid >> 4, q = tid & 15;
  const int half = row / PS;
  const int tag = __builtin_amdgcn_readfirstlane(half ? tag1 : tag0);
  const uint8_t* raw = sh.ring[slot][half];
  _Float16* dst = &sh.t1[buf][row][8 * q];
  if (WIDE && tag == IAK_TAG_FP16) {
    const uint8_t* src = raw + (row - PS * half) * DQK * 2 + 16 * q;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      if (q + 16 * j < C::CHUNKS)
        *reinterpret_cast<u4*>(dst + 128 * j) = *reinterpret_cast<const u4*>(src + 256 * j);
    return;
  }
  const uint8_t* src = raw + (row - PS * half) * DQK + 8 * q;
  u2 x[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
    if (q + 16 * j < C::CHUNKS) x[j] = *reinterpret_cast<const u2*>(src + 128 * j);
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    if (q + 16 * j < C::CHUNKS) {
      uint32_t lo0, hi0, lo1, hi1;
      if (tag == IAK_TAG_FP8) { fp8x4_to_f16(x[j][0], lo0, hi0); fp8x4_to_f16(x[j][1], lo1, hi1); }
      else { i8x4_to_f16(x[j][0], lo0, hi0); i8x4_to_f16(x[j][1], lo1, hi1); }
      *reinterpret_cast<u4*>(dst + 128 * j) = u4{lo0, hi0, lo1, hi1};
    }
  }
}

// Four f16 of a value column, transposed out of the [token][dim] tile: lane i of
// each 16-lane group names row `row0 + i / 4`, columns col0 + 4 (i % 4) .. +3;
// lane j receives column col0 + j of rows row0 .. row0 + 3 (ds_read_b64_tr_b16:
// element m of lane j comes from lane 4m + j / 4 of its group, element j % 4).
// `lane_off` is the lane's part of the address, (i / 4) rows + 4 (i % 4)
// columns, computed once per kernel; `off` (row0 rows + col0 columns, and the
// buffer) is uniform, so each read is one add or an immediate offset.
template <int DQK, int DV, bool WIDE>
__device__ __forceinline__ h4 mla_read_column(const MlaShared<DQK, DV, WIDE>& sh, int lane_off, int off) {
  typedef short s4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s4 lds_s4;
  const _Float16* p = &sh.t1[0][0][0] + off + lane_off;
  const s4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(p));
  return __builtin_bit_cast(h4, v);
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
  const int head = hg * C::HEADS + 16 * w + c;   // this lane's score / P head
  // the lane's part of a value-operand read: rows 4g + c / 4, columns 4 (c % 4)
  const int vlane = (4 * g + (c >> 2)) * C::T1 + 4 * (c & 3);

  // token bound of the sequence (table entry e holds tokens 16e .. 16e+15)
  const int limit = a.valid ? __builtin_amdgcn_readfirstlane(a.valid[b]) : 0x7FFFFFFF;
  // entries lane and lane + 64 of the split (up to 128 entries)
  const MlaPages meta = mla_page_meta(a, b, start, lane, limit);
  const MlaPages meta2 = mla_page_meta(a, b, start, lane + 64, limit);
  const uint64_t mask = __builtin_amdgcn_ballot_w64(meta.pid >= 0);
  const uint64_t mask2 = __builtin_amdgcn_ballot_w64(meta2.pid >= 0);
  const int np = __builtin_popcountll(mask) + __builtin_popcountll(mask2);

  // Q of the lane's head, rounded to f16: dims 32i + 8g .. +7 (B operand of the scores)
  h8 q[C::KSTEPS];
  {
    const bool live = head < a.H;
    const int64_t off = (int64_t)b * a.qsb + (int64_t)(live ? head : 0) * a.qsh + 8 * g;
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
      q[i] = v;
    }
  }

  // per lane: running max and partial denominator of head column c (the
  // partial covers the lane's token rows; summed over g at the end)
  float m = -__builtin_inff(), l = 0.f;
  int E = 0;   // value exponent (wave-uniform): the value sum is acc * 2^E
  // O tile db: rows = heads 4g .. 4g+3, column = value dim 16 db + c
  f4 acc[C::NDB];
#pragma unroll
  for (int db = 0; db < C::NDB; ++db) acc[db] = f4{0.f, 0.f, 0.f, 0.f};

  if (np > 0) {
    const int nsteps = (np + 1) >> 1;
    // page cursor: entry indexes (0 .. 127) of the pages in table order; past
    // the end the last page is named again (copies stay unconditional,
    // compute is masked)
    uint64_t rem = mask, rem2 = mask2;
    int last = mask ? __builtin_ctzll(mask) : 64 + __builtin_ctzll(mask2);
    auto next_page = [&]() {
      if (rem) last = take(rem);
      else if (rem2) last = 64 + take(rem2);
      return last;
    };
    // entry idx's field: lane idx of the first or lane idx - 64 of the second half
    auto pick = [&](int v, int v2, int idx) {
      const int x = __builtin_amdgcn_readlane(v, idx & 63), x2 = __builtin_amdgcn_readlane(v2, idx & 63);
      return idx >= 64 ? x2 : x;
    };
    auto page_pid = [&](int idx) { return pick(meta.pid, meta2.pid, idx); };
    auto page_tag = [&](int idx) { return pick(meta.tag, meta2.tag, idx); };
    auto page_scale = [&](int idx) {
      return __builtin_bit_cast(
          float, pick(__builtin_bit_cast(int, meta.scale), __builtin_bit_cast(int, meta2.scale), idx));
    };
    // pq[2k], pq[2k+1]: entry indexes of the pages of step s+k (ring slot (s+k) % SLOTS)
    int pq[2 * C::SLOTS];
#pragma unroll
    for (int k = 0; k < C::SLOTS; ++k)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        pq[2 * k + h] = next_page();
        mla_dma_page<DQK, DV, WIDE>(sh.ring[k][h], a, page_pid(pq[2 * k + h]), page_tag(pq[2 * k + h]), w, lane);
      }
    mla_wait_pages<C::NDMA, 2 * (C::SLOTS - 1)>();
    __syncthreads();
    mla_stage_pair<DQK, DV, WIDE>(sh, 0, 0, page_tag(pq[0]), page_tag(pq[1]), tid);

    // One page pair per iteration and one barrier: each wave waits for its
    // copies of pair s+1, then the barrier makes pair s's tile (staged in the
    // previous iteration) and pair s+1's raw bytes visible to every wave and
    // ends every read of the other tile buffer. Then pair s+SLOTS starts
    // streaming into the ring slot pair s came from, pair s's scores and
    // softmax run, pair s+1 is staged into the other tile buffer, and pair s's
    // values follow. R = s & 1 is pair s's tile buffer.
    for (int st = 0; st < nsteps; ++st) {
      const int R = st & 1;
      const int cur0 = pq[0], cur1 = pq[1], nx0 = pq[2], nx1 = pq[3];
      mla_wait_pages<C::NDMA, 2 * (C::SLOTS - 2)>();
      __syncthreads();
      const int slot = st & (C::SLOTS - 1);
      const int in0 = next_page(), in1 = next_page();
      mla_dma_page<DQK, DV, WIDE>(sh.ring[slot][0], a, page_pid(in0), page_tag(in0), w, lane);
      mla_dma_page<DQK, DV, WIDE>(sh.ring[slot][1], a, page_pid(in1), page_tag(in1), w, lane);

      // Wave priorities by phase: the staging of the next pair and the softmax
      // (VALU and LDS work that the next barrier waits for) issue ahead of the
      // other wave's MFMAs when the two waves of a SIMD are in different
      // phases; the MFMA phases run at the lowest priority.
      // ---- scores of pair s: S^T[16 tok x 16 heads] per page, two chains ----
      __builtin_amdgcn_s_setprio(0);
      f4 s0 = f4{0.f, 0.f, 0.f, 0.f}, s1 = f4{0.f, 0.f, 0.f, 0.f};
      {
        constexpr int PFS = C::PF_SCORE;
        h8 aq0[PFS], aq1[PFS];
#pragma unroll
        for (int d = 0; d < PFS && d < C::KSTEPS; ++d) {
          aq0[d] = *reinterpret_cast<const h8*>(&sh.t1[R][c][32 * d + 8 * g]);
          aq1[d] = *reinterpret_cast<const h8*>(&sh.t1[R][PS + c][32 * d + 8 * g]);
        }
#pragma unroll
        for (int i = 0; i < C::KSTEPS; ++i) {
          const h8 a0 = aq0[i % PFS], a1 = aq1[i % PFS];
          if (i + PFS < C::KSTEPS) {
            aq0[i % PFS] = *reinterpret_cast<const h8*>(&sh.t1[R][c][32 * (i + PFS) + 8 * g]);
            aq1[i % PFS] = *reinterpret_cast<const h8*>(&sh.t1[R][PS + c][32 * (i + PFS) + 8 * g]);
          }
          __builtin_amdgcn_sched_barrier(0);
          s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, q[i], s0, 0, 0, 0);
          s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, q[i], s1, 0, 0, 0);
          __builtin_amdgcn_sched_barrier(0);
        }
      }

#pragma unroll
      for (int k = 0; k < 2 * C::SLOTS - 2; ++k) pq[k] = pq[k + 2];
      pq[2 * C::SLOTS - 2] = in0;
      pq[2 * C::SLOTS - 1] = in1;

      // ---- softmax over the pair's 32 tokens ----
      __builtin_amdgcn_s_setprio(1);
      const float ps0 = page_scale(cur0), ps1 = page_scale(cur1);
      s0 *= a.score_mult * ps0;
      s1 *= a.score_mult * ps1;
      // tokens at or past the bound (the sequence's last visited page), and the
      // second page of a pair past the end
      // second page of a pair past the end; a wave-uniform test skips the
      // masking for the usual pair of two whole pages
      const bool live1 = 2 * st + 1 < np;
      const int64_t end0 = (int64_t)(start + cur0 + 1) * PS, end1 = (int64_t)(start + cur1 + 1) * PS;
      if (!(live1 && end0 <= limit && end1 <= limit)) {
        const int64_t lim0 = (int64_t)limit - (end0 - PS) - 4 * g;
        const int64_t lim1 = live1 ? (int64_t)limit - (end1 - PS) - 4 * g : 0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (r >= lim0) s0[r] = -__builtin_inff();
          if (r >= lim1) s1[r] = -__builtin_inff();
        }
      }
      const float pm = xmax16_32(fmaxf(fmaxf(fmaxf(s0[0], s0[1]), fmaxf(s0[2], s0[3])),
                                       fmaxf(fmaxf(s1[0], s1[1]), fmaxf(s1[2], s1[3]))));
      const bool grow = pm > m + RESCALE_SLACK;
      float al = 1.0f;
      if (grow) {
        al = __builtin_amdgcn_exp2f(m - pm);   // 0 on the first pair (m = -inf)
        m = pm;
      }
      // value exponent: follows the larger page scale of the pair
      const int e = scale_exp(fmaxf(ps0, ps1));
      const bool emove = e > E + EXP_WINDOW || e < E - EXP_WINDOW;
      const float efac = emove ? pow2f(E - e) : 1.0f;
      if (emove) E = e;
      const float vm = pow2f(-E);
      f4 p0, p1;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p0[r] = __builtin_amdgcn_exp2f(s0[r] - m);
        p1[r] = __builtin_amdgcn_exp2f(s1[r] - m);
      }
      l = l * al + (((p0[0] + p0[1]) + (p0[2] + p0[3])) + ((p1[0] + p1[1]) + (p1[2] + p1[3])));
      // P: A operand of the value product (row = head c, k = 8g + m:
      // tokens 4g + m of the first page, then of the second); V scales fold in
      h8 pa;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pa[r] = (_Float16)(p0[r] * (ps0 * vm));
        pa[4 + r] = (_Float16)(p1[r] * (ps1 * vm));
      }
      // ---- stage pair s+1 (landed before the barrier) ----
      __builtin_amdgcn_s_setprio(3);
      if (st + 1 < nsteps)
        mla_stage_pair<DQK, DV, WIDE>(sh, (st + 1) & (C::SLOTS - 1), 1 - R, page_tag(nx0), page_tag(nx1), tid);
      // rescale: the O rows are heads 4g + r, whose factor sits in lane 4g + r
      if (__builtin_amdgcn_ballot_w64(grow) != 0 || emove) {
        f4 ar;
#pragma unroll
        for (int r = 0; r < 4; ++r) ar[r] = __shfl(al, 4 * g + r, 64) * efac;
#pragma unroll
        for (int db = 0; db < C::NDB; ++db) acc[db] *= ar;
      }

      // ---- values of pair s: the wave's heads, every value dim ----
      __builtin_amdgcn_s_setprio(0);
      {
        constexpr int PFV = C::PF_VALUE;
        h8 bq[PFV];
        auto rd = [&](int db) {
          const int off = (R * C::TOK) * C::T1 + a.VOFF + 16 * db;
          const h4 b0 = mla_read_column<DQK, DV, WIDE>(sh, vlane, off);
          const h4 b1 = mla_read_column<DQK, DV, WIDE>(sh, vlane, off + PS * C::T1);
          return __builtin_shufflevector(b0, b1, 0, 1, 2, 3, 4, 5, 6, 7);
        };
#pragma unroll
        for (int d = 0; d < PFV && d < C::NDB; ++d) bq[d] = rd(d);
#pragma unroll
        for (int db = 0; db < C::NDB; ++db) {
          const h8 bop = bq[db % PFV];
          if (db + PFV < C::NDB) bq[db % PFV] = rd(db + PFV);
          __builtin_amdgcn_sched_barrier(0);
          acc[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, bop, acc[db], 0, 0, 0);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    // the copies of the pages past the end land before the LDS is reused or released
    mla_wait_pages<C::NDMA, 0>();
  }

  // ---- denominators and maxima of the wave's heads, then the output or the partials ----
  {
    const float ls = xsum16_32(l);
    if (g == 0) {
      sh.lsum[16 * w + c] = ls;
      sh.mmax[16 * w + c] = m;
    }
  }
  __syncthreads();
  const float vscale = pow2f(E);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int hl = 16 * w + 4 * g + r;
    const int h = hg * C::HEADS + hl;
    if (h >= a.H) continue;
    if (a.splits == 1) {
      const float ls = sh.lsum[hl];
      const float inv = ls > 0.f ? vscale / ls : 0.0f;
      const int64_t o = (int64_t)b * a.osb + (int64_t)h * a.osh + c;
#pragma unroll
      for (int db = 0; db < C::NDB; ++db) {
        const float v = acc[db][r] * inv;
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
      if (a.acc16) {
        const float ls = sh.lsum[hl];
        const float inv = ls > 0.f ? vscale / ls : 0.0f;
        _Float16* op = reinterpret_cast<_Float16*>(a.ws_acc) + slot * DV + c;
#pragma unroll
        for (int db = 0; db < C::NDB; ++db) op[16 * db] = (_Float16)(acc[db][r] * inv);
      } else {
        float* op = a.ws_acc + slot * DV + c;
#pragma unroll
        for (int db = 0; db < C::NDB; ++db) op[16 * db] = acc[db][r] * vscale;
      }
    }
  }
}

template <int DQK, int DV, bool WIDE>
hipError_t launch_mla_w(const MArgs& m, hipStream_t stream, hipEvent_t ev_begin, hipEvent_t ev_end) {
  if (ev_begin) (void)hipEventRecord(ev_begin, stream);
  hipLaunchKernelGGL((mla_decode_kernel<DQK, DV, WIDE>), dim3(m.B * m.splits, m.HG),
                     dim3(Mla<DQK, DV, WIDE>::THREADS), 0, stream, m);
  hipError_t e = hipGetLastError();
  if (ev_end) (void)hipEventRecord(ev_end, stream);
  if (e != hipSuccess || m.splits == 1) return e;
  // the paged-decode merge over rows (b, 0) of H heads
  KArgs k{};
  k.B = m.B; k.Hq = m.H; k.Hkv = 1; k.G = m.H; k.D = DV; k.splits = m.splits;
  k.out = m.out; k.out_dtype = m.out_dtype; k.osb = m.osb; k.osh = m.osh;
  k.ws_m = m.ws_m; k.ws_l = m.ws_l; k.ws_acc = m.ws_acc; k.acc16 = m.acc16;
  return launch_merge<DV>(k, stream);
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
