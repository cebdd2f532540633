// Dense softmax attention of the reference's dense_attention() in float32, for gfx950.
//
// Reference semantics (src/intent_attention/reference.py:16-45):
//   scores = (q . k^T) * scale
//   causal, no positions:   scores += triu(-inf, diagonal=1)   (query i sees keys j <= i)
//   causal, kv positions:   scores[i, j] = -inf where i < original_kv_positions[j]
//   mask:                   scores += mask                      (an additive mask; bool adds 1.0)
//   out = softmax(scores) . v
// A row whose scores are all -inf is NaN (softmax of -inf everywhere), as in
// torch; an empty key set gives zeros (torch's matmul over an empty dim).
//
// The reference runs these as torch.matmul / softmax in the input dtype. Here
// every product and sum is float32 over float32, float16 or bfloat16 inputs,
// and the output is rounded once to the input dtype.
//
// Work split. A (batch, query) row's keys go to `splits` workgroups of
// consecutive key ranges (`chunk` keys each); splits > 1 only when the caller
// gives a workspace and there are few rows with 256 keys or more (decode shapes),
// and a second kernel then merges the partials (max, denominator, context)
// by log-sum-exp. A workgroup has WAVES waves (16 when the grid is short, so
// it still has many key rows in flight); wave w takes KEYS consecutive keys
// per step. It loads the K and V rows of all of them first, then reduces the
// KEYS wave-wide dot products together, so one step costs about one memory
// round trip. Lane l holds dims l, l + 64, ... of q and of the context: a key
// or value row is one coalesced load per 64 dims, its row address a scalar.
// Each wave keeps a running max, denominator and context; the waves merge
// through the LDS at the end.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "iak.h"
#include "iak_device.h"

namespace iak {

namespace {

// the split over keys: rows with at least SPLIT_MIN_KEYS keys, ranges of at
// least RANGE_MIN_KEYS keys
#ifndef SPLIT_MIN_KEYS
#define SPLIT_MIN_KEYS 256
#endif
#ifndef RANGE_MIN_KEYS
#define RANGE_MIN_KEYS 64
#endif
// workgroups the split aims at
#ifndef SPLIT_TARGET_WGS
#define SPLIT_TARGET_WGS 256
#endif

// element types: float, _Float16, and bfloat16 held as its 16 bits
struct bf16_bits { uint16_t b; };

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(_Float16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(bf16_bits x) { return __builtin_bit_cast(float, (uint32_t)x.b << 16); }
__device__ __forceinline__ float to_f32(uint8_t x) { return x ? 1.f : 0.f; }   // bool mask: adds 1.0

template <typename T>
__device__ __forceinline__ float load_t(const void* p, int64_t i) {
  return to_f32(reinterpret_cast<const T*>(p)[i]);
}

template <typename T>
__device__ __forceinline__ void store_t(void* p, int64_t i, float x) {
  if constexpr (sizeof(T) == 4) {
    reinterpret_cast<float*>(p)[i] = x;
  } else if constexpr (__is_same(T, _Float16)) {
    reinterpret_cast<_Float16*>(p)[i] = (_Float16)x;
  } else {
    // bfloat16, round to nearest even (NaN kept quiet)
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    const uint32_t r = (u & 0x7fffffffu) > 0x7f800000u ? (u | 0x00400000u) : u + 0x7fffu + ((u >> 16) & 1u);
    reinterpret_cast<uint16_t*>(p)[i] = (uint16_t)(r >> 16);
  }
}

// the mask values of keys j0 .. j0 + KEYS - 1 of one query row (indices
// clamped to the range's last key `last`)
template <typename M, int KEYS>
__device__ __forceinline__ void step_mask(const iak_dense_attention_args& a, int64_t mb, int j0, int last,
                                          float* madd) {
#pragma unroll
  for (int u = 0; u < KEYS; ++u) {
    const int jc = j0 + u < last ? j0 + u : last;
    madd[u] = load_t<M>(a.mask, mb + (int64_t)jc * a.mask_stride_k);
  }
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over the 64 lanes, the same bits in every lane: each step adds two
// values that the partner lane adds in the other order (lane ^ 1 and lane ^ 2
// by quad permutes; then, with a quad's four lanes equal, the quads two and
// one places round the row of 16 by row rotates; then rows through the lane
// swaps), so every lane forms the same sums.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<0xB1>(v);    // quad_perm [1, 0, 3, 2]
  v += dpp<0x4E>(v);    // quad_perm [2, 3, 0, 1]
  v += dpp<0x128>(v);   // row_ror:8
  v += dpp<0x124>(v);   // row_ror:4
  return xsum16_32(v);
}

struct DenseSplit {
  int splits;   // workgroups per row
  int chunk;    // keys per workgroup (the last may have fewer)
  float* ws;    // splits > 1: [rows * splits] max, [rows * splits] denominator, [rows * splits, v_dim] context
};

// T: element type of q, k, v and out; NPL: dims per lane (head_dim and v_dim
// are at most 64 * NPL); KEYS keys per wave and step; WAVES waves per workgroup
template <typename T, int NPL, int KEYS, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void dense_attention_kernel(const iak_dense_attention_args a,
                                                                      const DenseSplit sp) {
  __shared__ float part_acc[WAVES][64 * NPL];
  __shared__ float part_m[WAVES], part_l[WAVES];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t item = blockIdx.x;   // row * splits + split, row = b * q_len + i
  const int64_t row = item / sp.splits;
  const int split = (int)(item - row * sp.splits);
  const int64_t b = row / a.q_len;
  const int i = (int)(row - b * a.q_len);
  const int lo = split * sp.chunk;
  const int hi = a.kv_len - lo < sp.chunk ? a.kv_len : lo + sp.chunk;   // keys lo .. hi - 1
  const float NEG_INF = -__builtin_inff();

  // this lane's dims, clamped into the row (the values past the width are zeroed)
  int dk[NPL], dv[NPL];
  bool okk[NPL], okv[NPL];
  float q[NPL], acc[NPL];
  const T* qrow = reinterpret_cast<const T*>(a.q) + b * a.q_stride_b + (int64_t)i * a.q_stride_t;
#pragma unroll
  for (int jj = 0; jj < NPL; ++jj) {
    const int d = lane + 64 * jj;
    okk[jj] = d < a.head_dim;
    okv[jj] = d < a.v_dim;
    dk[jj] = okk[jj] ? d : a.head_dim - 1;
    dv[jj] = okv[jj] ? d : a.v_dim - 1;
    const float qx = to_f32(qrow[dk[jj]]);
    q[jj] = okk[jj] ? qx : 0.f;
    acc[jj] = 0.f;
  }
  const T* kbase = reinterpret_cast<const T*>(a.k) + b * a.k_stride_b;
  const T* vbase = reinterpret_cast<const T*>(a.v) + b * a.v_stride_b;
  const int64_t mb = b * a.mask_stride_b + (int64_t)i * a.mask_stride_q;
  float m = NEG_INF, l = 0.f;
  // The K and V rows of a step's KEYS keys, loaded unconditionally at clamped
  // indices (a key past the range reads the range's last key; the values are
  // zeroed at use), so no load waits behind a branch. The loop is pipelined:
  // the next step's rows are in flight while this step's are reduced.
  float kn[KEYS][NPL], vn[KEYS][NPL];
  auto load_step = [&](int j0) {
#pragma unroll
    for (int u = 0; u < KEYS; ++u) {
      const int jc = j0 + u < hi ? j0 + u : hi - 1;
      const T* kr = kbase + (int64_t)jc * a.k_stride_t;
      const T* vr = vbase + (int64_t)jc * a.v_stride_t;
#pragma unroll
      for (int jj = 0; jj < NPL; ++jj) {
        kn[u][jj] = to_f32(kr[dk[jj]]);
        vn[u][jj] = to_f32(vr[dv[jj]]);
      }
    }
  };
  if (lo + KEYS * w < hi) load_step(lo + KEYS * w);
  for (int j0 = lo + KEYS * w; j0 < hi; j0 += KEYS * WAVES) {
    float kv[KEYS][NPL], vv[KEYS][NPL];
#pragma unroll
    for (int u = 0; u < KEYS; ++u) {
      const bool key = j0 + u < hi;   // wave-uniform
#pragma unroll
      for (int jj = 0; jj < NPL; ++jj) {
        kv[u][jj] = key && okk[jj] ? kn[u][jj] : 0.f;
        vv[u][jj] = key && okv[jj] ? vn[u][jj] : 0.f;
      }
    }
    // the next step's rows (clamped into the range on the last step)
    load_step(j0 + KEYS * WAVES < hi ? j0 + KEYS * WAVES : j0);
    float s[KEYS];
#pragma unroll
    for (int u = 0; u < KEYS; ++u) {
      float t = 0.f;
#pragma unroll
      for (int jj = 0; jj < NPL; ++jj) t = __builtin_fmaf(q[jj], kv[u][jj], t);
      s[u] = t;
    }
#pragma unroll
    for (int u = 0; u < KEYS; ++u) s[u] = wave_sum(s[u]);
    // the step's mask values and key positions, each set under one uniform branch
    float madd[KEYS];
    bool hidden[KEYS];
#pragma unroll
    for (int u = 0; u < KEYS; ++u) {
      madd[u] = 0.f;
      hidden[u] = false;
    }
    if (a.mask) {
      if (a.mask_dtype == IAK_MASK_BOOL) step_mask<uint8_t, KEYS>(a, mb, j0, hi - 1, madd);
      else if (a.mask_dtype == IAK_DTYPE_F32) step_mask<float, KEYS>(a, mb, j0, hi - 1, madd);
      else if (a.mask_dtype == IAK_DTYPE_F16) step_mask<_Float16, KEYS>(a, mb, j0, hi - 1, madd);
      else step_mask<bf16_bits, KEYS>(a, mb, j0, hi - 1, madd);
    }
    if (a.causal == IAK_CAUSAL_POSITIONS) {
#pragma unroll
      for (int u = 0; u < KEYS; ++u) {
        const int jc = j0 + u < hi ? j0 + u : hi - 1;
        hidden[u] = (int64_t)i < a.kv_positions[jc];   // masked_fill(-inf)
      }
    }
    float smax = NEG_INF;
#pragma unroll
    for (int u = 0; u < KEYS; ++u) {
      const int j = j0 + u;
      float x = s[u] * a.sm_scale;
      if (a.causal == IAK_CAUSAL_TRIU && j > i) x += NEG_INF;   // scores + triu(-inf, diagonal=1)
      if (hidden[u]) x = NEG_INF;
      x += madd[u];
      if (j >= hi) x = NEG_INF;                     // not a key of this range: no mass
      s[u] = x;
      smax = fmaxf(smax, x);
    }
    const float mn = fmaxf(m, smax);
    if (mn > m) {   // wave-uniform
      const float alpha = expf(m - mn);   // 0 while nothing was seen (m = -inf)
      l *= alpha;
#pragma unroll
      for (int jj = 0; jj < NPL; ++jj) acc[jj] *= alpha;
      m = mn;
    }
#pragma unroll
    for (int u = 0; u < KEYS; ++u) {
      // -inf scores (masked keys and the keys past the range) take no mass,
      // also when m is -inf; NaN scores poison l, as in softmax
      const float e = s[u] == NEG_INF ? 0.f : expf(s[u] - m);
      l += e;
#pragma unroll
      for (int jj = 0; jj < NPL; ++jj) acc[jj] = __builtin_fmaf(e, vv[u][jj], acc[jj]);
    }
  }

  if (lane == 0) {
    part_m[w] = m;
    part_l[w] = l;
  }
#pragma unroll
  for (int jj = 0; jj < NPL; ++jj) part_acc[w][lane + 64 * jj] = acc[jj];
  __syncthreads();
  float M = NEG_INF;
#pragma unroll
  for (int k = 0; k < WAVES; ++k) M = fmaxf(M, part_m[k]);
  float wt[WAVES], L = 0.f;
#pragma unroll
  for (int k = 0; k < WAVES; ++k) {
    wt[k] = part_m[k] == NEG_INF ? 0.f : expf(part_m[k] - M);   // 0 for a wave that saw no mass
    L += wt[k] * part_l[k];
  }
  if (sp.splits > 1) {
    // this range's partial: max, denominator and unnormalised context
    const int64_t n = (int64_t)gridDim.x;
    if (threadIdx.x == 0) {
      sp.ws[item] = M;
      sp.ws[n + item] = L;
    }
    float* wacc = sp.ws + 2 * n + item * a.v_dim;
    for (int d = threadIdx.x; d < a.v_dim; d += 64 * WAVES) {
      float A = 0.f;
#pragma unroll
      for (int k = 0; k < WAVES; ++k) A = __builtin_fmaf(wt[k], part_acc[k][d], A);
      wacc[d] = A;
    }
    return;
  }
  // all scores -inf: softmax is NaN everywhere; no keys at all: zeros
  const float empty = a.kv_len > 0 ? __builtin_nanf("") : 0.f;
  const int64_t ooff = b * a.out_stride_b + (int64_t)i * a.out_stride_t;
  for (int d = threadIdx.x; d < a.v_dim; d += 64 * WAVES) {
    float A = 0.f;
#pragma unroll
    for (int k = 0; k < WAVES; ++k) A = __builtin_fmaf(wt[k], part_acc[k][d], A);
    store_t<T>(a.out, ooff + d, M == NEG_INF ? empty : A / L);
  }
}

constexpr int MERGE_THREADS = 256;
constexpr int MAX_SPLITS = 1024;

// block-wide max / sum over MERGE_THREADS threads (the result in every thread)
template <bool MAX>
__device__ __forceinline__ float block_reduce(float v, float* red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float o = __shfl_xor(v, off, 64);
    v = MAX ? fmaxf(v, o) : v + o;
  }
  __syncthreads();   // red[] free from an earlier reduction
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  v = red[0];
#pragma unroll
  for (int k = 1; k < MERGE_THREADS / 64; ++k) v = MAX ? fmaxf(v, red[k]) : v + red[k];
  return v;
}

// One workgroup per row: the log-sum-exp merge of the row's `splits` partials
// (splits <= MAX_SPLITS). The split weights go to the LDS; each context dim is
// then summed over the splits by G thread groups (G = 256 / dims rounded up to
// 64), each over every G-th split, with eight independent loads in flight.
template <typename T>
__global__ __launch_bounds__(MERGE_THREADS) void dense_merge_kernel(const iak_dense_attention_args a,
                                                                    const DenseSplit sp) {
  __shared__ float wt[MAX_SPLITS];
  __shared__ float red[MERGE_THREADS / 64];
  __shared__ float part[MERGE_THREADS];
  const int64_t row = blockIdx.x;
  const int64_t b = row / a.q_len;
  const int i = (int)(row - b * a.q_len);
  const int S = sp.splits;
  const int64_t n = (int64_t)gridDim.x * S;
  const float* wm = sp.ws + row * S;
  const float* wl = sp.ws + n + row * S;
  const float* wacc = sp.ws + 2 * n + row * S * a.v_dim;
  const float NEG_INF = -__builtin_inff();
  float mx = NEG_INF;
  for (int s = threadIdx.x; s < S; s += MERGE_THREADS) mx = fmaxf(mx, wm[s]);
  const float M = block_reduce<true>(mx, red);
  float ls = 0.f;
  for (int s = threadIdx.x; s < S; s += MERGE_THREADS) {
    const float w = wm[s] == NEG_INF ? 0.f : expf(wm[s] - M);   // 0 for a range that saw no mass
    wt[s] = w;
    ls += w * wl[s];
  }
  const float L = block_reduce<false>(ls, red);   // its barriers also publish wt[]
  const int dims = (a.v_dim + 63) & ~63;          // v_dim rounded up to 64
  const int G = dims >= MERGE_THREADS ? 1 : MERGE_THREADS / dims;
  const int g = threadIdx.x / dims, dl = threadIdx.x - g * dims;
  const int64_t ooff = b * a.out_stride_b + (int64_t)i * a.out_stride_t;
  for (int d0 = 0; d0 < a.v_dim; d0 += MERGE_THREADS) {
    const int d = d0 + (G > 1 ? dl : threadIdx.x);
    const int dc = d < a.v_dim ? d : a.v_dim - 1;
    float A = 0.f;
    if (g < G) {
      int s = g;
      for (; s + 7 * G < S; s += 8 * G) {
        float x[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] = wacc[(int64_t)(s + u * G) * a.v_dim + dc];
#pragma unroll
        for (int u = 0; u < 8; ++u) A = __builtin_fmaf(wt[s + u * G], x[u], A);
      }
      for (; s < S; s += G) A = __builtin_fmaf(wt[s], wacc[(int64_t)s * a.v_dim + dc], A);
    }
    if (G > 1) {
      // the G groups' sums of one dim: group 0 adds them in group order
      part[threadIdx.x] = A;
      __syncthreads();
      if (g == 0) {
        for (int k = 1; k < G; ++k) A += part[k * dims + dl];
      }
      __syncthreads();
      if (g != 0) continue;
    }
    // kv_len > 0 here: every score -inf gives NaN
    if (d < a.v_dim) store_t<T>(a.out, ooff + d, M == NEG_INF ? __builtin_nanf("") : A / L);
  }
}

// MAXW: the most waves per workgroup whose registers and LDS fit (16 waves of
// a 1,024-thread workgroup get 128 VGPRs each)
template <typename T, int NPL, int KEYS, int MAXW>
void launch_items(const iak_dense_attention_args& a, const DenseSplit& sp, int64_t items, hipStream_t stream) {
  // waves per workgroup: about 4,096 waves in the grid (16 per CU), between 4 and MAXW
  const int64_t want = (4096 + items - 1) / items;
  const dim3 grid((unsigned)items);
  if (MAXW >= 16 && want >= 16)
    hipLaunchKernelGGL((dense_attention_kernel<T, NPL, KEYS, MAXW >= 16 ? 16 : 4>), grid, dim3(1024), 0, stream,
                       a, sp);
  else if (want >= 8)
    hipLaunchKernelGGL((dense_attention_kernel<T, NPL, KEYS, 8>), grid, dim3(512), 0, stream, a, sp);
  else
    hipLaunchKernelGGL((dense_attention_kernel<T, NPL, KEYS, 4>), grid, dim3(256), 0, stream, a, sp);
}

template <typename T>
void launch_typed(const iak_dense_attention_args& a, const DenseSplit& sp, hipStream_t stream) {
  const int64_t rows = (int64_t)a.batch * a.q_len;
  const int64_t items = rows * sp.splits;
  const int width = a.head_dim > a.v_dim ? a.head_dim : a.v_dim;
  const int npl = (width + 63) / 64;
  // keys per step: 2 * KEYS * NPL registers of K and V in flight per lane
  if (npl <= 1) launch_items<T, 1, 8, 16>(a, sp, items, stream);
  else if (npl <= 2) launch_items<T, 2, 8, 16>(a, sp, items, stream);
  else if (npl <= 4) launch_items<T, 4, 4, 16>(a, sp, items, stream);
  else if (npl <= 8) launch_items<T, 8, 4, 8>(a, sp, items, stream);
  else launch_items<T, 16, 2, 8>(a, sp, items, stream);
  if (sp.splits > 1) hipLaunchKernelGGL(dense_merge_kernel<T>, dim3((unsigned)rows), dim3(256), 0, stream, a, sp);
}

// Splits per row: rows with SPLIT_MIN_KEYS keys or more on a short grid (fewer
// than 512 rows) go over about SPLIT_TARGET_WGS workgroups in ranges of at
// least RANGE_MIN_KEYS keys
// (at most MAX_SPLITS ranges).
DenseSplit split_plan(const iak_dense_attention_args& a) {
  DenseSplit sp{1, a.kv_len, nullptr};
  const int64_t rows = (int64_t)a.batch * a.q_len;
  if (rows <= 0 || rows >= 512 || a.kv_len < SPLIT_MIN_KEYS) return sp;
  int64_t s = (SPLIT_TARGET_WGS + rows - 1) / rows;
  const int64_t by_keys = a.kv_len / RANGE_MIN_KEYS;
  if (s > by_keys) s = by_keys;
  if (s > MAX_SPLITS) s = MAX_SPLITS;   // the merge holds the split weights in the LDS
  if (s <= 1) return sp;
  const int64_t chunk = ((int64_t)a.kv_len + s - 1) / s;
  sp.splits = (int)(((int64_t)a.kv_len + chunk - 1) / chunk);
  sp.chunk = (int)chunk;
  return sp;
}

}  // namespace

size_t dense_attention_workspace(const iak_dense_attention_args& a) {
  const DenseSplit sp = split_plan(a);
  if (sp.splits <= 1) return 0;
  return (size_t)a.batch * a.q_len * sp.splits * (2 + (size_t)a.v_dim) * sizeof(float);
}

hipError_t launch_dense_attention(const iak_dense_attention_args& a, void* workspace, hipStream_t stream) {
  DenseSplit sp = split_plan(a);
  if (!workspace) sp = DenseSplit{1, a.kv_len, nullptr};
  sp.ws = static_cast<float*>(workspace);
  if (a.dtype == IAK_DTYPE_F32) launch_typed<float>(a, sp, stream);
  else if (a.dtype == IAK_DTYPE_F16) launch_typed<_Float16>(a, sp, stream);
  else launch_typed<bf16_bits>(a, sp, stream);
  return hipGetLastError();
}

}  // namespace iak
