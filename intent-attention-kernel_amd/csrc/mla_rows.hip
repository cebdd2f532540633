// Latent context of the reference's MLA decode API in float32, for gfx950.
//
// Reference semantics: the Triton kernel and CPU path of mla_decode_triton
// (src/intent_attention/triton_mla_decode.py:47-107 and _mla_decode_cpu
// :155-186): each (batch, query position) row attends to the latent rows of
// the pages its page table lists -- page p is rows p*page_size ..
// (p+1)*page_size - 1 of C [rows, d_c], the last page of C possibly shorter --
// with scores (q . c) * sm_scale in float32, an online softmax, and context =
// sum(p c) / sum(p); zeros when no row is visited. The projection by W_VO
// that follows is a plain GEMM outside this file.
//
// This is the reference API's arithmetic, not the serving path: the MFMA
// kernel of mla_decode.hip computes over paged f16 / FP8 / INT8 pools with f16
// operands, while this kernel keeps every product and sum in float32 over
// float32, float16 or bfloat16 inputs, any page size and any latent width up
// to 1,024 in one launch.
//
// Keys. The listed pages' rows form one key sequence: key j is row
// page_ids[j / page_size] * page_size + j % page_size of C (the division by a
// multiply-high and one correction, its magic number from the host); a key
// past the end of C (the last page's missing rows) takes no mass. A latent row
// is both the key and the value of its token, so it is loaded once.
//
// Work split. Every query row attends to the same latent rows, so a
// workgroup takes four query rows once there are four (each latent row it
// loads serves all of them). A row group's keys go to `splits` workgroups of
// consecutive key ranges; splits > 1 only when the caller gives a workspace
// and there are fewer than 512 row groups with at least 256 keys, and a
// second kernel merges each row's ranges' (max, denominator, context) by
// log-sum-exp. A workgroup has WAVES waves (16 when the grid is short); wave w
// takes KEYS consecutive keys per step, loads their latent rows first
// (unconditionally, at clamped indices, the values of keys past the range
// zeroed at use) with the next step's rows in flight while this step's dot
// products are reduced (a DPP + lane-swap wave sum with the same bits in every
// lane). Lane l holds dims l, l + 64, ... of q and of the context. Each wave
// keeps a running max, denominator and context per row; the waves merge
// through the LDS.

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

struct bf16_bits { uint16_t b; };

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(_Float16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(bf16_bits x) { return __builtin_bit_cast(float, (uint32_t)x.b << 16); }

__device__ __forceinline__ float load_q(const void* p, int64_t i, int dtype) {
  if (dtype == IAK_DTYPE_F32) return reinterpret_cast<const float*>(p)[i];
  if (dtype == IAK_DTYPE_F16) return (float)reinterpret_cast<const _Float16*>(p)[i];
  return to_f32(reinterpret_cast<const bf16_bits*>(p)[i]);
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over the 64 lanes, the same bits in every lane: each step adds two
// values that the partner lane adds in the other order (lane ^ 1 and lane ^ 2
// by quad permutes; then, with a quad's four lanes equal, the quads two and
// one places round the row of 16 by row rotates; then rows through the lane
// swaps).
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<0xB1>(v);    // quad_perm [1, 0, 3, 2]
  v += dpp<0x4E>(v);    // quad_perm [2, 3, 0, 1]
  v += dpp<0x128>(v);   // row_ror:8
  v += dpp<0x124>(v);   // row_ror:4
  return xsum16_32(v);
}

struct RowSplit {
  int splits;        // workgroups per row group
  int chunk;         // keys per workgroup (the last may have fewer)
  int nkeys;         // num_selected * page_size
  uint32_t magic;    // floor(2^32 / page_size), or 2^32 - 1 for page_size 1
  int rows_per_wg;   // query rows per workgroup (1 or 4)
  float* ws;         // splits > 1: [n] max, [n] denominator, [n, d_c] context, n = rows * splits
};

// The C row of key j: outside [0, num_rows) for a key past the end of C or of
// an invalid page id (the host rejects those; the kernel gives them no mass).
__device__ __forceinline__ int64_t key_row(const iak_mla_rows_args& a, const RowSplit& sp, uint32_t j) {
  uint32_t q = __umulhi(j, sp.magic);   // floor(j / page_size) or one less
  uint32_t r = j - q * (uint32_t)a.page_size;
  if (r >= (uint32_t)a.page_size) {
    ++q;
    r -= (uint32_t)a.page_size;
  }
  return (int64_t)a.page_ids[q] * a.page_size + r;
}

// T: latent element type; NPL: dims per lane (d_c <= 64 * NPL); KEYS keys per
// wave and step; WAVES waves per workgroup; R query rows per workgroup (every
// row attends to the same latent rows, so each loaded row serves all R)
template <typename T, int NPL, int KEYS, int WAVES, int R>
__global__ __launch_bounds__(64 * WAVES) void mla_rows_kernel(const iak_mla_rows_args a, const RowSplit sp) {
  __shared__ float part_acc[WAVES][R][64 * NPL];
  __shared__ float part_m[WAVES][R], part_l[WAVES][R];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t nrows = (int64_t)a.batch * a.q_len;
  const int64_t item = blockIdx.x;   // group * splits + split; rows R * group .. R * group + R - 1
  const int64_t group = item / sp.splits;
  const int split = (int)(item - group * sp.splits);
  const int dc = a.latent_dim;
  const int lo = split * sp.chunk;
  const int hi = sp.nkeys - lo < sp.chunk ? sp.nkeys : lo + sp.chunk;   // keys lo .. hi - 1
  const float NEG_INF = -__builtin_inff();

  int dd[NPL];
  bool ok[NPL];
#pragma unroll
  for (int jj = 0; jj < NPL; ++jj) {
    const int d = lane + 64 * jj;
    ok[jj] = d < dc;
    dd[jj] = ok[jj] ? d : dc - 1;
  }
  float q[R][NPL], acc[R][NPL], m[R], l[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t row = group * R + r;
    const int64_t rowc = row < nrows ? row : nrows - 1;   // a row past the end repeats the last (not written)
    const int64_t b = rowc / a.q_len;
    const int t = (int)(rowc - b * a.q_len);
    const int64_t qoff = b * a.q_stride_b + (int64_t)t * a.q_stride_t;
#pragma unroll
    for (int jj = 0; jj < NPL; ++jj) {
      const float qx = load_q(a.q, qoff + dd[jj], a.q_dtype);
      q[r][jj] = ok[jj] ? qx : 0.f;
      acc[r][jj] = 0.f;
    }
    m[r] = NEG_INF;
    l[r] = 0.f;
  }
  const T* lat = reinterpret_cast<const T*>(a.latents);
  // a step's latent rows, loaded at clamped indices (a key past the range
  // reads the range's last key, a row outside C its first or last row)
  float cn[KEYS][NPL];
  int64_t rows_n[KEYS];
  auto load_step = [&](int j0) {
#pragma unroll
    for (int u = 0; u < KEYS; ++u) {
      const int jc = j0 + u < hi ? j0 + u : hi - 1;
      const int64_t r = key_row(a, sp, (uint32_t)jc);
      rows_n[u] = r;
      const int64_t rc = r < 0 ? 0 : (r < a.num_rows ? r : a.num_rows - 1);
      const T* cr = lat + rc * a.latent_stride;
#pragma unroll
      for (int jj = 0; jj < NPL; ++jj) cn[u][jj] = to_f32(cr[dd[jj]]);
    }
  };
  if (lo + KEYS * w < hi) load_step(lo + KEYS * w);
  for (int j0 = lo + KEYS * w; j0 < hi; j0 += KEYS * WAVES) {
    float cv[KEYS][NPL];
    bool live[KEYS];
#pragma unroll
    for (int u = 0; u < KEYS; ++u) {
      live[u] = j0 + u < hi && rows_n[u] >= 0 && rows_n[u] < a.num_rows;   // wave-uniform
#pragma unroll
      for (int jj = 0; jj < NPL; ++jj) cv[u][jj] = live[u] && ok[jj] ? cn[u][jj] : 0.f;
    }
    // the next step's rows (clamped into the range on the last step)
    load_step(j0 + KEYS * WAVES < hi ? j0 + KEYS * WAVES : j0);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float s[KEYS];
#pragma unroll
      for (int u = 0; u < KEYS; ++u) {
        float x = 0.f;
#pragma unroll
        for (int jj = 0; jj < NPL; ++jj) x = __builtin_fmaf(q[r][jj], cv[u][jj], x);
        s[u] = x;
      }
      float smax = NEG_INF;
#pragma unroll
      for (int u = 0; u < KEYS; ++u) {
        const float x = wave_sum(s[u]) * a.sm_scale;
        s[u] = live[u] ? x : NEG_INF;
        smax = fmaxf(smax, s[u]);
      }
      const float mn = fmaxf(m[r], smax);
      if (mn > m[r]) {   // wave-uniform
        const float alpha = expf(m[r] - mn);   // 0 while nothing was seen (m = -inf)
        l[r] *= alpha;
#pragma unroll
        for (int jj = 0; jj < NPL; ++jj) acc[r][jj] *= alpha;
        m[r] = mn;
      }
#pragma unroll
      for (int u = 0; u < KEYS; ++u) {
        const float e = s[u] == NEG_INF ? 0.f : expf(s[u] - m[r]);   // keys that are not rows take no mass
        l[r] += e;
#pragma unroll
        for (int jj = 0; jj < NPL; ++jj) acc[r][jj] = __builtin_fmaf(e, cv[u][jj], acc[r][jj]);
      }
    }
  }

#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (lane == 0) {
      part_m[w][r] = m[r];
      part_l[w][r] = l[r];
    }
#pragma unroll
    for (int jj = 0; jj < NPL; ++jj) part_acc[w][r][lane + 64 * jj] = acc[r][jj];
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t row = group * R + r;
    if (row >= nrows) break;   // workgroup-uniform
    float M = NEG_INF;
#pragma unroll
    for (int k = 0; k < WAVES; ++k) M = fmaxf(M, part_m[k][r]);
    float wt[WAVES], L = 0.f;
#pragma unroll
    for (int k = 0; k < WAVES; ++k) {
      wt[k] = part_m[k][r] == NEG_INF ? 0.f : expf(part_m[k][r] - M);   // 0 for a wave that saw no row
      L += wt[k] * part_l[k][r];
    }
    if (sp.splits > 1) {
      // this range's partial of the row: max, denominator and unnormalised context
      const int64_t n = nrows * sp.splits;
      const int64_t slot = row * sp.splits + split;
      if (threadIdx.x == 0) {
        sp.ws[slot] = M;
        sp.ws[n + slot] = L;
      }
      float* wacc = sp.ws + 2 * n + slot * dc;
      for (int d = threadIdx.x; d < dc; d += 64 * WAVES) {
        float A = 0.f;
#pragma unroll
        for (int k = 0; k < WAVES; ++k) A = __builtin_fmaf(wt[k], part_acc[k][r][d], A);
        wacc[d] = A;
      }
    } else {
      float* out = a.context + row * dc;
      for (int d = threadIdx.x; d < dc; d += 64 * WAVES) {
        float A = 0.f;
#pragma unroll
        for (int k = 0; k < WAVES; ++k) A = __builtin_fmaf(wt[k], part_acc[k][r][d], A);
        out[d] = L > 0.f ? A / L : 0.f;   // zeros when no row was visited
      }
    }
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
// (splits <= MAX_SPLITS), split weights in the LDS, each context dim summed
// over the splits by G thread groups with eight loads in flight.
__global__ __launch_bounds__(MERGE_THREADS) void mla_rows_merge_kernel(const iak_mla_rows_args a,
                                                                       const RowSplit sp) {
  __shared__ float wt[MAX_SPLITS];
  __shared__ float red[MERGE_THREADS / 64];
  __shared__ float part[MERGE_THREADS];
  const int64_t row = blockIdx.x;
  const int S = sp.splits, dc = a.latent_dim;
  const int64_t n = (int64_t)gridDim.x * S;
  const float* wm = sp.ws + row * S;
  const float* wl = sp.ws + n + row * S;
  const float* wacc = sp.ws + 2 * n + row * S * dc;
  const float NEG_INF = -__builtin_inff();
  float mx = NEG_INF;
  for (int s = threadIdx.x; s < S; s += MERGE_THREADS) mx = fmaxf(mx, wm[s]);
  const float M = block_reduce<true>(mx, red);
  float ls = 0.f;
  for (int s = threadIdx.x; s < S; s += MERGE_THREADS) {
    const float w = wm[s] == NEG_INF ? 0.f : expf(wm[s] - M);   // 0 for a range that visited no row
    wt[s] = w;
    ls += w * wl[s];
  }
  const float L = block_reduce<false>(ls, red);   // its barriers also publish wt[]
  const int dims = (dc + 63) & ~63;
  const int G = dims >= MERGE_THREADS ? 1 : MERGE_THREADS / dims;
  const int g = threadIdx.x / dims, dl = threadIdx.x - g * dims;
  float* out = a.context + row * dc;
  for (int d0 = 0; d0 < dc; d0 += MERGE_THREADS) {
    const int d = d0 + (G > 1 ? dl : threadIdx.x);
    const int dcl = d < dc ? d : dc - 1;
    float A = 0.f;
    if (g < G) {
      int s = g;
      for (; s + 7 * G < S; s += 8 * G) {
        float x[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] = wacc[(int64_t)(s + u * G) * dc + dcl];
#pragma unroll
        for (int u = 0; u < 8; ++u) A = __builtin_fmaf(wt[s + u * G], x[u], A);
      }
      for (; s < S; s += G) A = __builtin_fmaf(wt[s], wacc[(int64_t)s * dc + dcl], A);
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
    if (d < dc) out[d] = L > 0.f ? A / L : 0.f;
  }
}

// MAXW: the most waves per workgroup whose registers and LDS fit
template <typename T, int NPL, int KEYS, int MAXW, int R>
void launch_items(const iak_mla_rows_args& a, const RowSplit& sp, int64_t items, hipStream_t stream) {
  // waves per workgroup: about 4,096 waves in the grid (16 per CU), between 4 and MAXW
  const int64_t want = (4096 + items - 1) / items;
  const dim3 grid((unsigned)items);
  if (MAXW >= 16 && want >= 16)
    hipLaunchKernelGGL((mla_rows_kernel<T, NPL, KEYS, MAXW >= 16 ? 16 : 4, R>), grid, dim3(1024), 0, stream, a, sp);
  else if (want >= 8)
    hipLaunchKernelGGL((mla_rows_kernel<T, NPL, KEYS, 8, R>), grid, dim3(512), 0, stream, a, sp);
  else
    hipLaunchKernelGGL((mla_rows_kernel<T, NPL, KEYS, 4, R>), grid, dim3(256), 0, stream, a, sp);
}

template <typename T, int R>
void launch_rows(const iak_mla_rows_args& a, const RowSplit& sp, hipStream_t stream) {
  const int64_t rows = (int64_t)a.batch * a.q_len;
  const int64_t items = (rows + R - 1) / R * sp.splits;
  const int npl = (a.latent_dim + 63) / 64;
  // per lane: R * NPL query and context values, KEYS * NPL latent values in flight (twice, pipelined)
  if (npl <= 1) launch_items<T, 1, 8, 16, R>(a, sp, items, stream);
  else if (npl <= 2) launch_items<T, 2, 8, 16, R>(a, sp, items, stream);
  else if (npl <= 4) launch_items<T, 4, (R > 1 ? 4 : 8), (R > 1 ? 8 : 16), R>(a, sp, items, stream);
  else if (npl <= 9) launch_items<T, 9, (R > 1 ? 2 : 4), 8, R>(a, sp, items, stream);
  else launch_items<T, 16, 2, (R > 1 ? 4 : 8), R>(a, sp, items, stream);
}

template <typename T>
void launch_typed(const iak_mla_rows_args& a, const RowSplit& sp, hipStream_t stream) {
  const int64_t rows = (int64_t)a.batch * a.q_len;
  if (sp.rows_per_wg == 4) launch_rows<T, 4>(a, sp, stream);
  else launch_rows<T, 1>(a, sp, stream);
  if (sp.splits > 1)
    hipLaunchKernelGGL(mla_rows_merge_kernel, dim3((unsigned)rows), dim3(MERGE_THREADS), 0, stream, a, sp);
}

// Splits per row group: with fewer than 512 groups and SPLIT_MIN_KEYS keys or
// more, a group's keys go over about SPLIT_TARGET_WGS workgroups in ranges of
// at least RANGE_MIN_KEYS keys
// (at most MAX_SPLITS ranges). Four rows per workgroup when that still gives
// 128 workgroups or more, one otherwise (few rows over few keys keep their
// parallelism).
RowSplit plan_for(const iak_mla_rows_args& a, int R) {
  const int64_t nkeys = (int64_t)a.num_selected * a.page_size;
  RowSplit sp{1, (int)nkeys, (int)nkeys, 0u, R, nullptr};
  sp.magic = a.page_size == 1 ? 0xFFFFFFFFu : (uint32_t)((1ull << 32) / (uint64_t)a.page_size);
  const int64_t rows = (int64_t)a.batch * a.q_len;
  const int64_t groups = (rows + R - 1) / R;
  if (rows <= 0 || groups >= 512 || nkeys < SPLIT_MIN_KEYS) return sp;
  int64_t s = (SPLIT_TARGET_WGS + groups - 1) / groups;
  const int64_t by_keys = nkeys / RANGE_MIN_KEYS;
  if (s > by_keys) s = by_keys;
  if (s > MAX_SPLITS) s = MAX_SPLITS;   // the merge holds the split weights in the LDS
  if (s <= 1) return sp;
  const int64_t chunk = (nkeys + s - 1) / s;
  sp.splits = (int)((nkeys + chunk - 1) / chunk);
  sp.chunk = (int)chunk;
  return sp;
}

RowSplit split_plan(const iak_mla_rows_args& a) {
  const int64_t rows = (int64_t)a.batch * a.q_len;
  if (rows >= 4) {
    const RowSplit sp4 = plan_for(a, 4);
    if ((rows + 3) / 4 * sp4.splits >= 128) return sp4;
  }
  return plan_for(a, 1);
}

}  // namespace

size_t mla_rows_workspace(const iak_mla_rows_args& a) {
  const RowSplit sp = split_plan(a);
  if (sp.splits <= 1) return 0;
  return (size_t)a.batch * a.q_len * sp.splits * (2 + (size_t)a.latent_dim) * sizeof(float);
}

hipError_t launch_mla_rows(const iak_mla_rows_args& a, void* workspace, hipStream_t stream) {
  RowSplit sp = split_plan(a);
  if (!workspace) sp.splits = 1, sp.chunk = sp.nkeys;
  sp.ws = static_cast<float*>(workspace);
  if (a.latent_dtype == IAK_DTYPE_F32) launch_typed<float>(a, sp, stream);
  else if (a.latent_dtype == IAK_DTYPE_F16) launch_typed<_Float16>(a, sp, stream);
  else launch_typed<bf16_bits>(a, sp, stream);
  return hipGetLastError();
}

}  // namespace iak
