// Fake-quant reconstruction of selected KV blocks for gfx950: what
// intent_quant_attention_reference (src/intent_attention/intent_quant_attention.py:56-84)
// builds with fake_quantize_tensor (intent_quant.py:221-312) block by block
// and torch.cat, for float32 K and V.
//
// Per block (a token range of K and V) and per channel (absmax over every
// leading row and token of the block, the reference's granule):
//   scale = max(fl32(absmax / 127), 1e-8)            (NaN stays NaN)
//   FP8            e4m3fn(fl32(x / scale)) * scale    (round to nearest even)
//   INT8 / INT4    rne(clamp(fl32(x / scale), +-maxq)) * scale, maxq 127 / 7
//                  (the code through an integer, so a zero code gives +0)
//   INT4_RESIDUAL  base = rne(clamp(x / scale, +-7)) * scale, r = x - base,
//                  s2 = max(fl32(absmax(r) / 127), 1e-8),
//                  base + rne(clamp(fl32(r / s2), +-7)) * s2
//   FP16           float(fl16(x))
//   SKIP           0
// Every division is the IEEE float32 quotient and every product and sum one
// float32 rounding, as torch computes them on float32 tensors; K's channels
// come first, then V's, and block i lands at its output token offset.
//
// A block's rows are its (leading row, token) pairs, leading row by leading
// row. A workgroup takes 64 channels of one block (thread t: channel t % 64)
// and a range of the block's rows, every sixteenth row per thread, so each row
// segment is one coalesced 256-byte load; a thread issues its rows' loads
// eight at a time, all in flight together.
//   One pass (no workspace, or a split of one): the workgroup owns all of the
//   block's rows; the sixteen row phases combine their absmax through the LDS,
//   and a block of at most 512 rows stays in registers between passes (8 or 32
//   per thread; a longer one is read again, from L2).
//   Split (a workspace, fewer than 256 (block, 64 channels) groups, blocks of
//   more than 512 rows): S workgroups per group, each over a contiguous 1/S
//   of the rows, in three launches: each workgroup's channel maxima to the
//   workspace; the INT4_RESIDUAL blocks' residual maxima (their scale is the
//   max of the S partials); then the reconstruction. Max is exact and
//   order-free, so the split gives the one-pass bits.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "iak.h"

// each product and sum rounds on its own, as torch's separate elementwise ops
// do: no fused multiply-adds in this file
#pragma clang fp contract(off)

namespace iak {

namespace {

constexpr int FQ_CHANNELS = 64;
constexpr int FQ_PHASES = 16;
constexpr int FQ_UNROLL = 8;        // loads in flight per thread when streaming
constexpr int FQ_CACHE_SMALL = 8;   // rows per thread held in registers: blocks of <= 128 rows
constexpr int FQ_CACHE_LARGE = 32;  //                                    blocks of <= 512 rows
constexpr int FQ_THREADS = FQ_CHANNELS * FQ_PHASES;
// the split plan: with fewer than FQ_SPLIT_MAX_GROUPS (block, 64 channels)
// groups, blocks of more than FQ_ONE_PASS_ROWS rows are split into ranges of
// about FQ_SPLIT_ROWS rows, up to about FQ_TARGET_WGS workgroups
constexpr int64_t FQ_ONE_PASS_ROWS = (int64_t)FQ_PHASES * FQ_CACHE_LARGE;
constexpr int64_t FQ_SPLIT_ROWS = 256;
constexpr int64_t FQ_SPLIT_MAX_GROUPS = 256;
constexpr int64_t FQ_TARGET_WGS = 1024;
constexpr int FQ_MAX_SPLITS = 256;

enum FqMode { FQ_ONE_PASS = 0, FQ_PARTIAL_MAX = 1, FQ_PARTIAL_RESID = 2, FQ_APPLY = 3 };

// float -> e4m3fn code, round to nearest even (magnitudes that round above 448
// are NaN, NaN keeps its sign bit)
__device__ __forceinline__ uint32_t e4m3fn_code(float v) {
  const uint32_t bits = __builtin_bit_cast(uint32_t, v);
  const uint32_t sign = (bits >> 24) & 0x80u;
  const float a = fabsf(v);
  if (a != a) return sign | 0x7Fu;
  uint32_t code;
  if (a < 0.015625f) {                                  // below 2^-6: subnormal, quantum 2^-9
    code = (uint32_t)__builtin_rintf(a * 512.0f);       // 8 rounds up into the smallest normal
  } else {
    const uint32_t ab = __builtin_bit_cast(uint32_t, a);
    const uint32_t r = ab + 0x7FFFFu + ((ab >> 20) & 1u);   // keep 3 mantissa bits, ties to even
    code = (r >> 20) - ((127u - 7u) << 3);
    if (code > 0x7Eu) code = 0x7Fu;                     // above 448: NaN
  }
  return sign | code;
}

// e4m3fn code -> its float value (exact)
__device__ __forceinline__ float e4m3fn_value(uint32_t code) {
  const uint32_t e = (code >> 3) & 0xFu, m = code & 7u;
  if (e == 0xFu && m == 7u) return __builtin_nanf("");
  const float mag = e == 0 ? (float)m * 0.001953125f                        // m * 2^-9
                           : __builtin_bit_cast(float, ((e + 120u) << 23) | (m << 20));
  return (code & 0x80u) ? -mag : mag;
}

// the reference's scale: max(absmax / 127, 1e-8) in float32, NaN kept (torch's clamp)
__device__ __forceinline__ float block_scale(float absmax) {
  const float s = __fdiv_rn(absmax, 127.0f);
  return s != s ? s : fmaxf(s, 1e-8f);
}

__device__ __forceinline__ float clamp_keep_nan(float x, float lo, float hi) {
  return x != x ? x : fminf(fmaxf(x, lo), hi);
}

// the integer code of q (clamped to +-maxq, ties to even) as a float, through
// an integer as torch's .to(int8).float() goes, so a code of zero is +0; a NaN
// quotient stays NaN (its int8 conversion is undefined in torch)
__device__ __forceinline__ float int_code(float q, float maxq) {
  const float r = __builtin_rintf(clamp_keep_nan(q, -maxq, maxq));
  return r != r ? r : (float)(int)r;
}

// |x| max that propagates NaN (torch.amax)
__device__ __forceinline__ float absmax_step(float m, float x) {
  const float a = fabsf(x);
  return (m != m || a != a) ? __builtin_nanf("") : fmaxf(m, a);
}

// a walk over a thread's rows (every FQ_PHASES-th row of the block, leading
// row by leading row) that keeps the token index and one element offset: each
// step adds FQ_PHASES tokens, and crossing the block's end moves to the next
// leading row (wrap = the leading-row stride minus the block's n tokens)
struct RowCursor {
  int t;
  int64_t off;
};

__device__ __forceinline__ void step(RowCursor& c, int n, int64_t stride_t16, int64_t wrap) {
  c.t += FQ_PHASES;
  c.off += stride_t16;
  while (c.t >= n) { c.t -= n; c.off += wrap; }
}

struct FqBlock {
  int src, n, dst, prec;
  int64_t r_lo, r_hi;     // this workgroup's rows
  int splits;
  float* part_max;        // [num_blocks][splits][k_dim + v_dim] (split launches)
  float* part_resid;      // same shape
};

// CACHE > 0: the workgroup's rows are at most FQ_PHASES * CACHE, read once into
// registers; CACHE 0: streamed FQ_UNROLL rows at a time, once per pass
template <int MODE, int CACHE>
__device__ __forceinline__ void fake_quant_rows(const iak_fake_quant_blocks_args& a, const FqBlock& b,
                                                float (&red)[FQ_PHASES][FQ_CHANNELS]) {
  const int tid = threadIdx.x;
  const int cl = tid % FQ_CHANNELS, ph = tid / FQ_CHANNELS;
  const int c = blockIdx.y * FQ_CHANNELS + cl;
  const int dtot = a.k_dim + a.v_dim;
  const bool live = c < dtot;
  const int n = b.n;
  // this channel's column of K or V (a dead channel past the last reads channel
  // 0 of whichever of K and V has channels; its values are not used)
  const bool isk = live ? c < a.k_dim : a.k_dim > 0;
  const float* base = isk ? a.k : a.v;
  const int64_t sl = isk ? a.k_stride_l : a.v_stride_l, st = isk ? a.k_stride_t : a.v_stride_t;
  const int cc = !live ? 0 : (isk ? c : c - a.k_dim);
  // this thread's first row (r_lo + ph) and its number of rows
  int li0 = (int)(b.r_lo / n), t0 = (int)(b.r_lo % n) + ph;
  while (t0 >= n) { t0 -= n; ++li0; }
  const int64_t first = b.r_lo + ph;
  const int64_t mine = first < b.r_hi ? (b.r_hi - first + FQ_PHASES - 1) / FQ_PHASES : 0;
  const int64_t ost = a.out_stride_t;
  const RowCursor in0{t0, li0 * sl + (int64_t)(b.src + t0) * st + cc};
  const RowCursor out0{t0, li0 * a.out_stride_l + (int64_t)(b.dst + t0) * ost + c};
  const int64_t in_step = FQ_PHASES * st, in_wrap = sl - (int64_t)n * st;
  const int64_t out_step = FQ_PHASES * ost, out_wrap = a.out_stride_l - (int64_t)n * ost;
  // a row past this thread's rows loads the block's first row instead, so
  // every load is in bounds and all of them can be in flight
  const int64_t row0 = (int64_t)b.src * st + cc;
  constexpr int U = CACHE > 0 ? CACHE : FQ_UNROLL;
  float xc[U];
  if constexpr (CACHE > 0) {
    RowCursor ic = in0;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      xc[u] = base[u < mine ? ic.off : row0];
      step(ic, n, in_step, in_wrap);
    }
  }
  // f(x) on each of this thread's values, U loads in flight
  auto each_value = [&](auto&& f) {
    if constexpr (CACHE > 0) {
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (u < mine) f(xc[u]);
    } else {
      RowCursor ic = in0;
      for (int64_t j = 0; j < mine; j += U) {
        float x[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          x[u] = base[j + u < mine ? ic.off : row0];
          step(ic, n, in_step, in_wrap);
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
          if (j + u < mine) f(x[u]);
      }
    }
  };
  // out = g(x) for each of this thread's values
  auto each_store = [&](auto&& g) {
    RowCursor oc = out0;
    if constexpr (CACHE > 0) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (u < mine) a.out[oc.off] = g(xc[u]);
        step(oc, n, out_step, out_wrap);
      }
    } else {
      RowCursor ic = in0;
      for (int64_t j = 0; j < mine; j += U) {
        float x[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          x[u] = base[j + u < mine ? ic.off : row0];
          step(ic, n, in_step, in_wrap);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if (j + u < mine) a.out[oc.off] = g(x[u]);
          step(oc, n, out_step, out_wrap);
        }
      }
    }
  };
  // the sixteen row phases' values of one channel combined through the LDS
  auto channel_absmax = [&](float m) {
    red[ph][cl] = m;
    __syncthreads();
    float r = red[0][cl];
#pragma unroll
    for (int p = 1; p < FQ_PHASES; ++p) r = absmax_step(r, red[p][cl]);
    __syncthreads();   // red[] reusable
    return r;
  };
  const int64_t part_at = ((int64_t)blockIdx.x * b.splits + blockIdx.z) * dtot + c;   // this range's partial
  // the max of the channel's S partial maxima: phase ph reads partials ph,
  // ph + 16, ..., four loads in flight, and the phases combine through the LDS
  auto partials_max = [&](const float* part) {
    const float* p = part + (int64_t)blockIdx.x * b.splits * dtot + (live ? c : 0);
    float m = 0.f;
    for (int j = ph; j < b.splits; j += 4 * FQ_PHASES) {
      float x[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) x[u] = p[(int64_t)(j + u * FQ_PHASES < b.splits ? j + u * FQ_PHASES : ph) * dtot];
#pragma unroll
      for (int u = 0; u < 4; ++u) m = absmax_step(m, x[u]);
    }
    return channel_absmax(m);
  };
  const int prec = b.prec;

  if (MODE == FQ_PARTIAL_RESID && prec != IAK_FQ_INT4_RESIDUAL) return;
  if (prec == IAK_FQ_FP16 || prec == IAK_FQ_SKIP) {
    if (MODE == FQ_PARTIAL_MAX) return;
    if (!live) return;
    each_store([&](float x) { return prec == IAK_FQ_SKIP ? 0.f : (float)(_Float16)x; });
    return;
  }
  // the block's scale: this workgroup's maxima (one pass) or the S partials
  float s;
  if constexpr (MODE == FQ_ONE_PASS || MODE == FQ_PARTIAL_MAX) {
    float m = 0.f;
    each_value([&](float x) { m = absmax_step(m, x); });
    m = channel_absmax(m);
    if constexpr (MODE == FQ_PARTIAL_MAX) {
      if (live && ph == 0) b.part_max[part_at] = m;
      return;
    }
    s = block_scale(m);
  } else {
    s = block_scale(partials_max(b.part_max));
  }
  if (prec != IAK_FQ_INT4_RESIDUAL) {
    if (MODE == FQ_PARTIAL_RESID || !live) return;
    if (prec == IAK_FQ_FP8) {
      each_store([&](float x) { return e4m3fn_value(e4m3fn_code(__fdiv_rn(x, s))) * s; });
    } else {
      const float maxq = prec == IAK_FQ_INT8 ? 127.f : 7.f;
      each_store([&](float x) { return int_code(__fdiv_rn(x, s), maxq) * s; });
    }
    return;
  }
  // INT4_RESIDUAL: the residual's absmax, then base + residual codes
  float s2;
  if constexpr (MODE == FQ_ONE_PASS || MODE == FQ_PARTIAL_RESID) {
    float mr = 0.f;
    each_value([&](float x) { mr = absmax_step(mr, x - int_code(__fdiv_rn(x, s), 7.f) * s); });
    mr = channel_absmax(mr);
    if constexpr (MODE == FQ_PARTIAL_RESID) {
      if (live && ph == 0) b.part_resid[part_at] = mr;
      return;
    }
    s2 = block_scale(mr);
  } else {
    s2 = block_scale(partials_max(b.part_resid));
  }
  if (!live) return;
  each_store([&](float x) {
    const float bq = int_code(__fdiv_rn(x, s), 7.f) * s;
    return bq + int_code(__fdiv_rn(x - bq, s2), 7.f) * s2;
  });
}

// grid (num_blocks, channel groups, splits); one split with MODE FQ_ONE_PASS
template <int MODE>
__global__ __launch_bounds__(FQ_THREADS) void fake_quant_blocks_kernel(const iak_fake_quant_blocks_args a,
                                                                       float* part_max, float* part_resid) {
  __shared__ float red[FQ_PHASES][FQ_CHANNELS];
  const int* meta = a.blocks + 4 * blockIdx.x;
  FqBlock b;
  b.src = meta[0]; b.n = meta[1]; b.dst = meta[2]; b.prec = meta[3];
  if (b.n <= 0) return;
  b.splits = gridDim.z;
  b.part_max = part_max;
  b.part_resid = part_resid;
  const int64_t rows = (int64_t)a.lead * b.n;
  const int64_t chunk = (rows + b.splits - 1) / b.splits;
  b.r_lo = chunk * blockIdx.z;
  b.r_hi = b.r_lo + chunk < rows ? b.r_lo + chunk : rows;
  if (MODE == FQ_ONE_PASS && rows <= FQ_PHASES * FQ_CACHE_SMALL)
    fake_quant_rows<MODE, FQ_CACHE_SMALL>(a, b, red);
  else if (MODE == FQ_ONE_PASS && rows <= FQ_PHASES * FQ_CACHE_LARGE)
    fake_quant_rows<MODE, FQ_CACHE_LARGE>(a, b, red);
  else
    fake_quant_rows<MODE, 0>(a, b, red);
}

int fake_quant_splits(const iak_fake_quant_blocks_args& a) {
  const int64_t rows = (int64_t)a.lead * (a.max_block_tokens > 1 ? a.max_block_tokens : 1);
  const int64_t groups = (int64_t)a.num_blocks * ((a.k_dim + a.v_dim + FQ_CHANNELS - 1) / FQ_CHANNELS);
  if (rows <= FQ_ONE_PASS_ROWS || groups >= FQ_SPLIT_MAX_GROUPS) return 1;
  int64_t s = (rows + FQ_SPLIT_ROWS - 1) / FQ_SPLIT_ROWS;
  const int64_t fill = (FQ_TARGET_WGS + groups - 1) / groups;
  if (s > fill) s = fill;
  if (s > FQ_MAX_SPLITS) s = FQ_MAX_SPLITS;
  return s < 1 ? 1 : (int)s;
}

}  // namespace

size_t fake_quant_blocks_workspace(const iak_fake_quant_blocks_args& a) {
  const int s = fake_quant_splits(a);
  if (s <= 1) return 0;
  return 2 * sizeof(float) * (size_t)a.num_blocks * (size_t)s * (size_t)(a.k_dim + a.v_dim);
}

hipError_t launch_fake_quant_blocks(const iak_fake_quant_blocks_args& a, void* workspace, hipStream_t stream) {
  const int dtot = a.k_dim + a.v_dim;
  const int s = workspace ? fake_quant_splits(a) : 1;
  const unsigned groups = (unsigned)((dtot + FQ_CHANNELS - 1) / FQ_CHANNELS);
  if (s <= 1) {
    hipLaunchKernelGGL(fake_quant_blocks_kernel<FQ_ONE_PASS>, dim3((unsigned)a.num_blocks, groups, 1),
                       dim3(FQ_THREADS), 0, stream, a, nullptr, nullptr);
    return hipGetLastError();
  }
  float* part_max = static_cast<float*>(workspace);
  float* part_resid = part_max + (size_t)a.num_blocks * (size_t)s * (size_t)dtot;
  const dim3 grid((unsigned)a.num_blocks, groups, (unsigned)s);
  hipLaunchKernelGGL(fake_quant_blocks_kernel<FQ_PARTIAL_MAX>, grid, dim3(FQ_THREADS), 0, stream, a, part_max,
                     part_resid);
  hipLaunchKernelGGL(fake_quant_blocks_kernel<FQ_PARTIAL_RESID>, grid, dim3(FQ_THREADS), 0, stream, a, part_max,
                     part_resid);
  hipLaunchKernelGGL(fake_quant_blocks_kernel<FQ_APPLY>, grid, dim3(FQ_THREADS), 0, stream, a, part_max,
                     part_resid);
  return hipGetLastError();
}

}  // namespace iak
