// Page tables from routed spans for gfx950: the work of
// routing_to_kernel_metadata + metadata_to_kernel_tensors
// (block_router.py:283-296, :383-421; fused_selected_quant_decode.py:344-400)
// on the device, generalised to one span list per group of rows (a GQA
// [B, Hkv, W] table, per-sequence routing) and a logical -> physical block
// table.
//
// One workgroup per row. A row's pages are the concatenation, in span order,
// of each span's page interval [start / ps, (end - 1) / ps]; call the k-th page
// of that concatenation "pair k". Pair k is emitted when its page is seen for
// the first time (the lowest span covering it is its own span) and resident;
// its output position is the number of emitted pairs before it: each thread
// takes PT_PER consecutive pairs (their block-table loads in flight together)
// and one exclusive scan over the threads' counts places them. Spans are
// taken 256 at a time (a scan of their page counts locates each pair), and
// the first-seen test reads an LDS map
// page -> lowest covering span, built with LDS atomicMin over the same pairs
// before they are emitted: a later chunk's spans have larger indices, so the
// map is final for every page of the current chunk. A list whose pages span
// more than PT_OWNER ids tests first-seen against the earlier spans directly.
//
// The precision array is a min-reduction over (row, tag) keys: fill with the
// sentinel, atomicMin(row * 8 + tag) for every emitted page, then map the
// sentinel to the default tag and keys to their tag. Rows that share list and
// block-table row with the previous row produce the same pages and skip it.
//
// All of this is integer work bounded by the pages the lists name; it is
// launch- and latency-bound (a few microseconds), not HBM-bound.

#include <hip/hip_runtime.h>
#include <limits.h>
#include <stdint.h>

#include "iak.h"
#include "iak_internal.h"

namespace iak {

typedef int32_t i4 __attribute__((ext_vector_type(4)));

constexpr int PT_THREADS = 256;
constexpr int PT_OWNER = 16384;   // page ids one list may span for the LDS first-seen map (64 KB)
constexpr int PT_PER = 8;         // consecutive pairs per thread in the emit pass

__device__ __forceinline__ int64_t floor_div(int64_t x, int64_t d) {
  return x >= 0 ? x / d : -((-x + d - 1) / d);
}

// Exclusive prefix of v over the 256 threads; `total` gets the sum. `wsum` is
// 4 entries of LDS; the trailing barrier lets the caller reuse it at once.
__device__ __forceinline__ int64_t block_scan(int64_t v, int64_t& total, int64_t* wsum) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int64_t x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int64_t y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) wsum[w] = x;
  __syncthreads();
  int64_t base = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < PT_THREADS / 64; ++i) {
    const int64_t s = wsum[i];
    base += i < w ? s : 0;
    tot += s;
  }
  __syncthreads();
  total = tot;
  return base + x - v;
}

struct SpanPages {
  int64_t lo, hi;   // clamped page interval; empty when hi < lo
};

// pages of span i (index into the span arrays), clamped to [0, bound)
__device__ __forceinline__ SpanPages span_pages(const iak_page_table_args& a, int64_t i, int64_t bound) {
  const int64_t s = a.span_begin[i], e = a.span_end[i];
  SpanPages p{0, -1};
  if (e > s) {
    p.lo = floor_div(s, a.page_size);
    p.hi = floor_div(e - 1, a.page_size);
    p.lo = p.lo < 0 ? 0 : p.lo;
    p.hi = p.hi > bound - 1 ? bound - 1 : p.hi;
  }
  return p;
}

__global__ __launch_bounds__(PT_THREADS) void page_tables_kernel(const iak_page_table_args a) {
  __shared__ uint32_t owner[PT_OWNER];
  __shared__ int64_t pre[PT_THREADS];     // exclusive page-count prefix of the chunk's spans
  __shared__ int64_t first[PT_THREADS];   // first (clamped) page of each span of the chunk
  __shared__ int32_t tags[PT_THREADS];    // tag of each span of the chunk
  __shared__ int64_t wsum[PT_THREADS / 64];
  __shared__ int64_t rmin[PT_THREADS / 64], rmax[PT_THREADS / 64];

  const int tid = threadIdx.x;
  const int r = blockIdx.x;
  const int list = r / a.rows_per_list, seq = r / a.rows_per_seq;
  const int64_t s0 = a.span_offsets[list];
  const int64_t S = (int64_t)a.span_offsets[list + 1] - s0 > 0 ? (int64_t)a.span_offsets[list + 1] - s0 : 0;
  const int32_t* bt = a.block_table ? a.block_table + (int64_t)seq * a.block_table_width : nullptr;
  const int64_t bound = bt ? a.block_table_width : a.num_pages;   // logical ids that can be resident
  const int W = a.table_width;
  int32_t* table = a.page_table + (int64_t)r * W;
  const bool write_prec = a.page_precision != nullptr &&
      (r == 0 || (r - 1) / a.rows_per_list != list || (r - 1) / a.rows_per_seq != seq);

  // the list's page range decides between the LDS map and the direct test
  bool use_map = false;
  int64_t amin = 0;
  if (a.dedupe) {
    int64_t mn = INT64_MAX, mx = -1;
    for (int64_t i = tid; i < S; i += PT_THREADS) {
      const SpanPages p = span_pages(a, s0 + i, bound);
      if (p.lo <= p.hi) {
        mn = p.lo < mn ? p.lo : mn;
        mx = p.hi > mx ? p.hi : mx;
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const int64_t o = __shfl_xor(mn, off, 64), x = __shfl_xor(mx, off, 64);
      mn = o < mn ? o : mn;
      mx = x > mx ? x : mx;
    }
    if ((tid & 63) == 0) { rmin[tid >> 6] = mn; rmax[tid >> 6] = mx; }
    __syncthreads();
    mn = INT64_MAX;
    mx = -1;
#pragma unroll
    for (int i = 0; i < PT_THREADS / 64; ++i) {
      mn = rmin[i] < mn ? rmin[i] : mn;
      mx = rmax[i] > mx ? rmax[i] : mx;
    }
    use_map = mx < 0 || mx - mn < PT_OWNER;
    amin = mx < 0 ? 0 : mn;
    if (use_map)
      for (int64_t i = tid; i <= mx - amin; i += PT_THREADS) owner[i] = 0xFFFFFFFFu;
    __syncthreads();
  }

  int64_t base = 0;   // pages emitted so far by this row (uniform)
  for (int64_t c0 = 0; c0 < S; c0 += PT_THREADS) {
    const int cn = S - c0 < PT_THREADS ? (int)(S - c0) : PT_THREADS;
    int64_t n = 0, lo = 0;
    int tg = 0;
    if (tid < cn) {
      const SpanPages p = span_pages(a, s0 + c0 + tid, bound);
      lo = p.lo;
      n = p.hi >= p.lo ? p.hi - p.lo + 1 : 0;
      tg = a.span_tag[s0 + c0 + tid] & 7;
    }
    int64_t tot;
    const int64_t ex = block_scan(n, tot, wsum);
    pre[tid] = ex;
    first[tid] = lo;
    tags[tid] = tg;
    __syncthreads();

    // span of pair k: the largest j < cn with pre[j] <= k (never an empty span for k < tot)
    auto locate = [&](int64_t k) {
      int j = 0;
#pragma unroll
      for (int step = PT_THREADS / 2; step > 0; step >>= 1)
        if (j + step < cn && pre[j + step] <= k) j += step;
      return j;
    };
    auto advance = [&](int j, int64_t k) {
      while (j + 1 < cn && pre[j + 1] <= k) ++j;
      return j;
    };

    // pairs in batches of PT_THREADS * PT_PER; thread t takes PT_PER consecutive pairs
    if (use_map) {
      for (int64_t k0 = (int64_t)tid * PT_PER; k0 < tot; k0 += (int64_t)PT_THREADS * PT_PER) {
        int j = locate(k0);
        for (int u = 0; u < PT_PER && k0 + u < tot; ++u) {
          j = advance(j, k0 + u);
          atomicMin(&owner[first[j] + (k0 + u - pre[j]) - amin], (uint32_t)(c0 + j));
        }
      }
      __syncthreads();
    }

    for (int64_t b0 = 0; b0 < tot; b0 += (int64_t)PT_THREADS * PT_PER) {
      const int64_t k0 = b0 + (int64_t)tid * PT_PER;
      int32_t phys[PT_PER];
      int8_t fresh[PT_PER], tagv[PT_PER];
      int j = k0 < tot ? locate(k0) : 0;
#pragma unroll
      for (int u = 0; u < PT_PER; ++u) {      // independent loads, issued back to back
        const int64_t k = k0 + u;
        fresh[u] = 0;
        phys[u] = -1;
        tagv[u] = 0;
        if (k < tot) {
          j = advance(j, k);
          const int64_t i = c0 + j;
          const int64_t pg = first[j] + (k - pre[j]);
          bool f = true;
          if (a.dedupe) {
            if (use_map) {
              f = owner[pg - amin] == (uint32_t)i;
            } else {
              for (int64_t e = 0; e < i && f; ++e) {
                const SpanPages p = span_pages(a, s0 + e, bound);
                f = !(p.lo <= pg && pg <= p.hi);
              }
            }
          }
          fresh[u] = f;
          phys[u] = bt ? bt[pg] : (int32_t)pg;
          tagv[u] = (int8_t)tags[j];
        }
      }
      int64_t mine = 0;
#pragma unroll
      for (int u = 0; u < PT_PER; ++u) mine += (fresh[u] && phys[u] >= 0 && phys[u] < a.num_pages) ? 1 : 0;
      int64_t etot;
      int64_t pos = base + block_scan(mine, etot, wsum);
#pragma unroll
      for (int u = 0; u < PT_PER; ++u) {
        if (fresh[u] && phys[u] >= 0 && phys[u] < a.num_pages) {
          if (pos < W) table[pos] = phys[u];
          if (write_prec) atomicMin(&a.page_precision[phys[u]], r * 8 + tagv[u]);
          ++pos;
        }
      }
      base += etot;
    }
    __syncthreads();   // pre / first / tags are rewritten by the next chunk
  }

  const int64_t cnt = base < W ? base : W;
  if (tid == 0) a.page_counts[r] = (int32_t)cnt;
  for (int64_t e = cnt + tid; e < W; e += PT_THREADS) table[e] = 0;
}

// The precision passes touch every page once: 16-byte accesses over the
// 16-byte-aligned body of the array, single words for the (at most three)
// elements before it and after it.
struct I32Span {
  int32_t* p;
  int64_t n, head, body;   // head: words before the first 16-byte boundary; body: int4 count
};
__device__ __forceinline__ I32Span i32_span(int32_t* p, int64_t n) {
  I32Span s{p, n, 0, 0};
  const int64_t mis = (int64_t)(((16u - ((uint32_t)(uintptr_t)p & 15u)) & 15u) >> 2);
  s.head = mis < n ? mis : n;
  s.body = (n - s.head) >> 2;
  return s;
}

template <typename F> __device__ __forceinline__ void for_each_i32(int32_t* p, int64_t n, F f) {
  const I32Span s = i32_span(p, n);
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  i4* body = reinterpret_cast<i4*>(p + s.head);
  for (int64_t i = t0; i < s.body; i += stride) {
    i4 v = body[i];
    v[0] = f(v[0]); v[1] = f(v[1]); v[2] = f(v[2]); v[3] = f(v[3]);
    body[i] = v;
  }
  // the words outside the body: head and tail, at most 6
  const int64_t tail0 = s.head + 4 * s.body;
  if (t0 < s.head) p[t0] = f(p[t0]);
  if (t0 < n - tail0) p[tail0 + t0] = f(p[tail0 + t0]);
}

__global__ __launch_bounds__(256) void fill_i32_kernel(int32_t* p, int64_t n, int32_t v) {
  for_each_i32(p, n, [v](int32_t) { return v; });
}

__global__ __launch_bounds__(256) void precision_keys_to_tags_kernel(int32_t* p, int64_t n, int32_t dflt) {
  for_each_i32(p, n, [dflt](int32_t x) { return x == INT_MAX ? dflt : (x & 7); });
}

hipError_t launch_page_tables(const iak_page_table_args& a, hipStream_t stream) {
  const int64_t np = a.page_precision ? a.num_pages : 0;
  const int64_t vec = (np + 3) / 4;   // 16-byte groups, one per thread
  const int fill_blocks = (int)((vec + 255) / 256 < 4096 ? (vec + 255) / 256 : 4096);
  if (np > 0) hipLaunchKernelGGL(fill_i32_kernel, dim3(fill_blocks), dim3(256), 0, stream, a.page_precision, np,
                                 (int32_t)INT_MAX);
  if (a.num_rows > 0)
    hipLaunchKernelGGL(page_tables_kernel, dim3(a.num_rows), dim3(PT_THREADS), 0, stream, a);
  if (np > 0) hipLaunchKernelGGL(precision_keys_to_tags_kernel, dim3(fill_blocks), dim3(256), 0, stream,
                                 a.page_precision, np, (int32_t)a.default_tag);
  return hipGetLastError();
}

}  // namespace iak
