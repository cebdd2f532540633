// C ABI of libiak: argument validation, split planning, workspace layout and
// kernel launch for the selected-page decode (declared in include/iak.h).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "iak.h"
#include "iak_internal.h"

namespace {

thread_local char g_err[512] = "";

iak_status fail(iak_status st, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return st;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

const char* tag_name(int t) {
  switch (t) {
    case IAK_TAG_FP16: return "FP16";
    case IAK_TAG_INT8: return "INT8";
    case IAK_TAG_FP8: return "FP8";
    case IAK_TAG_INT4: return "INT4";
    case IAK_TAG_INT4_RESIDUAL: return "INT4_RESIDUAL";
    default: return "SKIP";
  }
}

constexpr size_t WS_ALIGN = 256;
size_t round_up(size_t x) { return (x + WS_ALIGN - 1) / WS_ALIGN * WS_ALIGN; }

struct Plan {
  int G, splits, chunk;
  int splitsA, chunkB;                        // the first tier's splits, the second tier's length
  bool fused;                                 // the decode kernel merges (merge_in_kernel)
  size_t ws_m, ws_l, ws_acc, ws_cnt, total;   // byte offsets / total
};

// `tiers`: two-tier split plans allowed (not for iak_paged_decode_noalloc, whose
// fixed scratch holds one-tier partials)
iak_status validate(const iak_paged_decode_args* a, Plan* plan, bool tiers = true) {
  if (!a) return fail(IAK_EINVAL, "args is NULL");
  if (a->batch < 0 || a->num_q_heads <= 0 || a->num_kv_heads <= 0 || a->table_width < 0 || a->num_pages < 0)
    return fail(IAK_EINVAL, "negative or zero size (batch=%d, num_q_heads=%d, num_kv_heads=%d, table_width=%d, num_pages=%lld)",
                a->batch, a->num_q_heads, a->num_kv_heads, a->table_width, (long long)a->num_pages);
  if (a->num_q_heads % a->num_kv_heads != 0)
    return fail(IAK_EINVAL, "num_q_heads %d is not a multiple of num_kv_heads %d", a->num_q_heads, a->num_kv_heads);
  const int G = a->num_q_heads / a->num_kv_heads;
  if (G > 16) return fail(IAK_ENOTSUP, "GQA group %d > 16 is not supported", G);
  if (a->head_dim != 64 && a->head_dim != 128)
    return fail(IAK_ENOTSUP, "head_dim %d is not supported (64 or 128)", a->head_dim);
  if (a->page_size != 16) return fail(IAK_ENOTSUP, "page_size %d is not supported (16)", a->page_size);
  if (a->num_pages > 0x7FFFFFFFLL) return fail(IAK_EINVAL, "num_pages %lld exceeds int32 page ids", (long long)a->num_pages);
  if (a->q_dtype < 0 || a->q_dtype > 2 || a->out_dtype < 0 || a->out_dtype > 2)
    return fail(IAK_EINVAL, "bad q/out dtype (%d, %d)", a->q_dtype, a->out_dtype);
  if (!std::isfinite(a->sm_scale)) return fail(IAK_EINVAL, "sm_scale is not finite");
  if (a->pages_per_split < 0 || a->pages_per_split > 64)
    return fail(IAK_EINVAL, "pages_per_split %d outside [0, 64]", a->pages_per_split);
  if (a->merge_in_kernel < 0 || a->merge_in_kernel > 2)
    return fail(IAK_EINVAL, "merge_in_kernel %d is not 0, 1 or 2", a->merge_in_kernel);
  if (a->map_other_tags != 0 && a->map_other_tags != 1)
    return fail(IAK_EINVAL, "map_other_tags must be 0 or 1, got %d", a->map_other_tags);
  const long long rows = (long long)a->batch * a->num_kv_heads;
  if (rows > 0) {
    if (!a->q || !a->out) return fail(IAK_EINVAL, "q/out is NULL");
    // q rows are read as 16-byte vectors
    const int qvec = a->q_dtype == IAK_DTYPE_F32 ? 4 : 8;
    if (!aligned16(a->q) || a->q_stride_b % qvec != 0 || a->q_stride_h % qvec != 0)
      return fail(IAK_EINVAL, "q must be 16-byte aligned with strides that are multiples of %d elements", qvec);
    if ((!a->page_table && !a->entry_records) || !a->page_counts)
      return fail(IAK_EINVAL, "page_table/page_counts is NULL");
    if (a->num_pages > 0 && !a->page_tags && !a->page_desc && !a->entry_records)
      return fail(IAK_EINVAL, "page_tags is NULL");
    if (reinterpret_cast<uintptr_t>(a->valid_tokens) & 3u) return fail(IAK_EINVAL, "valid_tokens must be 4-byte aligned");
  }
  if (reinterpret_cast<uintptr_t>(a->page_desc) & 31u) return fail(IAK_EINVAL, "page_desc must be 32-byte aligned");
  if (reinterpret_cast<uintptr_t>(a->entry_records) & 31u)
    return fail(IAK_EINVAL, "entry_records must be 32-byte aligned");
  // every native precision reachable through the tag map needs its pools (with
  // page descriptors or entry records: every native precision whose pools are
  // given, scales coming from the descriptors or records)
  const bool native = a->page_desc || a->entry_records;
  for (int t = 0; t < 8; ++t) {
    int n = a->tag_map[t];
    if (native) {
      n = t;
      const bool given = (t == IAK_TAG_FP16 && a->k_fp16) || (t == IAK_TAG_FP8 && a->k_fp8) ||
                         (t == IAK_TAG_INT8 && a->k_int8) || (t == IAK_TAG_INT4 && a->k_int4) ||
                         (t == IAK_TAG_INT4_RESIDUAL && a->k_int4r);
      if (!given) continue;
    }
    const void *k = nullptr, *v = nullptr, *ks = nullptr, *vs = nullptr;
    int sd = IAK_DTYPE_F32;
    switch (n) {
      case IAK_TAG_FP16: k = a->k_fp16; v = a->v_fp16; ks = vs = k; break;
      case IAK_TAG_FP8: k = a->k_fp8; v = a->v_fp8; ks = a->k_fp8_scale; vs = a->v_fp8_scale; sd = a->fp8_scale_dtype; break;
      case IAK_TAG_INT8: k = a->k_int8; v = a->v_int8; ks = a->k_int8_scale; vs = a->v_int8_scale; sd = a->int8_scale_dtype; break;
      case IAK_TAG_INT4: k = a->k_int4; v = a->v_int4; ks = a->k_int4_scale; vs = a->v_int4_scale; sd = a->int4_scale_dtype; break;
      case IAK_TAG_INT4_RESIDUAL: k = a->k_int4r; v = a->v_int4r; ks = a->k_int4r_scale; vs = a->v_int4r_scale; break;
      default: continue;   // SKIP or unknown: contributes nothing
    }
    if (native) ks = vs = k;   // scales come from the descriptors or records
    if (!k || !v || !ks || !vs)
      return fail(IAK_EINVAL, "tag %d maps to %s but its K/V pool or scales are NULL", t, tag_name(n));
    if (!aligned16(k) || !aligned16(v))
      return fail(IAK_EINVAL, "%s K/V pools must be 16-byte aligned", tag_name(n));
    if (sd != IAK_DTYPE_F16 && sd != IAK_DTYPE_F32)
      return fail(IAK_EINVAL, "%s scale dtype %d must be f16 or f32", tag_name(n), sd);
    if (n == IAK_TAG_INT4) {
      const int grp = a->int4_group, D = a->head_dim;
      if (grp <= 0 || D % grp != 0 || grp % (D / 4) != 0)
        return fail(IAK_ENOTSUP, "int4_group %d must divide head_dim %d and be a multiple of %d", grp, D, D / 4);
    }
  }

  // split plan: one wave per split of up to `chunk` table entries
  const int W = a->table_width;
  int chunk = a->pages_per_split;
  if (chunk == 0) {
    // long splits amortise the per-split prologue and partial traffic, and
    // 64-entry splits keep HBM busy from 2048 waves on. Smaller grids are
    // latency-bound: there the splits shrink until there is one workgroup per
    // CU (the same work on every CU; a grid of 2 or 3 workgroups per CU, or an
    // uneven one, measured slower), but not below ceil(W / 64) entries clamped
    // to [2, 8]: at most ~64 splits per row for the merge to read, and never
    // the single-entry splits whose prologue outweighs their page. Measured
    // (random pages of a 65,536-page pool, best split length in brackets):
    // 8 rows x 64 entries 12.0 -> 10.2 us (2), 32 x 64 13.9 -> 12.2 (2),
    // 8 x 256 14.2 -> 13.4 (4), 16 x 200 14.3 -> 13.3 (4), 64 x 100 15.0 ->
    // 14.4 (7); 2 x 512 and 1 x 1,000 keep 8, their best (1 x 1,000: 17.4 us,
    // against 19.6 at 16 entries and 19.8 at 4)
    chunk = 64;
    if (rows * ((W + 63) / 64) < 2048) {
      const long long want = (long long)IAK_GPU_CUS * IAK_WAVES_PER_BLOCK;   // waves = splits x rows
      const long long splits_per_row = (want + rows - 1) / (rows > 0 ? rows : 1);
      const int least = (W + 63) / 64 < 2 ? 2 : ((W + 63) / 64 > 8 ? 8 : (W + 63) / 64);
      chunk = (int)((W + splits_per_row - 1) / splits_per_row);
      chunk = chunk < least ? least : (chunk > 64 ? 64 : chunk);
    }
    // the same number of splits with even lengths (cfg3: 26 splits of 63
    // entries instead of 25 of 64 and one of 38; kernel 329.1 -> 327.7 us)
    if (W > 0) {
      const int n = (W + chunk - 1) / chunk;
      chunk = (W + n - 1) / n;
    }
  }
  int splits = (W + chunk - 1) / chunk;
  if (splits < 1) splits = 1;
  // Two tiers on grids of more than about 1.5 resident generations of waves
  // (automatic plans): the first three quarters of each row's entries in splits
  // of `chunk` entries, the rest in splits of about IAK_TIER_CHUNK entries
  // (evened over a multiple of four splits) placed after every row's first tier
  // in the grid. Of the waves sharing a CU the oldest are served first (a
  // wave-timeline probe: at cfg3 the older workgroup of a CU takes 95 us per
  // split, the younger 163 us, with the same bytes), so the grid's last
  // workgroups are the slowest; short ones there shorten the tail (cfg3
  // 326.3-327.7 -> 314.1-314.9 us per step with 16 tail splits of 40; tails of
  // 24 / 32 / 44 / 48 entries measured 326.9 / 319.5-320.9 / 318.8 / 322-323).
  // Both tiers hold whole fours of splits, so a workgroup's four waves stay in
  // one tier and one row whichever merge form runs.
  int splitsA = splits, chunkB = chunk;
  if (tiers && a->pages_per_split == 0 && rows * (long long)splits > IAK_TIER_MIN_WAVES) {
    const int sa = (int)((long long)W * 3 / 4 / chunk) / 4 * 4;
    const int tail = W - sa * chunk;
    if (sa >= 4 && tail > 0) {
      const int sb = ((tail + IAK_TIER_CHUNK - 1) / IAK_TIER_CHUNK + 3) / 4 * 4;
      splitsA = sa;
      chunkB = (tail + sb - 1) / sb;
      splits = sa + sb;
    }
  }
  // in-kernel merge: a workgroup's four waves take four splits of one row, so
  // the row's split count becomes a multiple of four (trailing splits may be
  // empty: they read no entry)
  // (automatic: only for grids of many workgroups, where each row's merge
  // overlaps other workgroups' page streaming; its three dependent memory
  // round trips otherwise lengthen the tail: cfg3, 1,792 workgroups, 337.6 ->
  // 333.9 us per step; cfg2, 512, unchanged; cfg4, 256, 42.4 -> 43.0 us)
  // (automatic, small grids: the same when the grid has at most 128
  // workgroups and a row at most 256 partials to merge, where the merge
  // kernel's launch costs more than the last workgroup's merge: 8 rows x 64
  // entries, one query head per KV head, 10.5 -> 8.5 us; four heads 10.9 ->
  // 9.8 us; 8 x 256 entries 13.2 -> 12.6 us; against 1 row x 64 splits x 16
  // heads 17.6 -> 35.2 us and 32 rows x 32 splits 12.0 -> 12.5 us)
  bool fused = a->merge_in_kernel != 0 && splits > 1;
  if (fused && a->merge_in_kernel == 2) {
    const long long wgs = rows * (long long)((splits + 3) / 4);
    fused = wgs >= IAK_MERGE_IN_KERNEL_MIN_WORKGROUPS ||
            (wgs <= IAK_MERGE_IN_KERNEL_SMALL_WORKGROUPS &&
             (long long)((splits + 3) / 4 * 4) * G <= IAK_MERGE_IN_KERNEL_SMALL_PARTIALS);
  }
  if (fused && splitsA == splits) {
    splits = (splits + 3) / 4 * 4;
    splitsA = splits;
  }
  if (rows * (long long)splits > 0x7FFFFFFFLL) return fail(IAK_EINVAL, "too many splits");
  plan->G = G;
  plan->splits = splits;
  plan->chunk = chunk;
  plan->splitsA = splitsA;
  plan->chunkB = chunkB;
  plan->fused = fused;
  // workspace: the split partials (m, l, acc), one per split or, in-kernel,
  // one per workgroup, then the rows' arrival counters; none when one split
  // covers a row
  if (splits == 1) {
    plan->ws_m = plan->ws_l = plan->ws_acc = plan->ws_cnt = plan->total = 0;
  } else {
    const size_t slots = (size_t)rows * (fused ? splits / 4 : splits) * G;
    plan->ws_m = 0;
    plan->ws_l = round_up(slots * sizeof(float));
    plan->ws_acc = plan->ws_l + round_up(slots * sizeof(float));
    plan->ws_cnt = plan->ws_acc + round_up(slots * a->head_dim * sizeof(float));
    plan->total = plan->ws_cnt + (fused ? round_up((size_t)rows * sizeof(int32_t)) : 0);
  }
  return IAK_OK;
}

struct MPlan {
  int splits, chunk, HG;
  size_t ws_m, ws_l, ws_acc, total;
};

bool mla_shape_supported(int dqk, int dv) {
  return (dqk == 64 && dv == 64) || (dqk == 128 && dv == 128) || (dqk == 256 && dv == 256) ||
         (dqk == 512 && dv == 512) || (dqk == 576 && dv == 512) || (dqk == 576 && dv == 64);
}

iak_status validate_mla(const iak_mla_decode_args* a, MPlan* plan) {
  if (!a) return fail(IAK_EINVAL, "args is NULL");
  if (a->batch < 0 || a->num_heads <= 0 || a->table_width < 0 || a->num_pages < 0)
    return fail(IAK_EINVAL, "negative or zero size (batch=%d, num_heads=%d, table_width=%d, num_pages=%lld)",
                a->batch, a->num_heads, a->table_width, (long long)a->num_pages);
  if (!mla_shape_supported(a->qk_dim, a->v_dim))
    return fail(IAK_ENOTSUP, "MLA (qk_dim, v_dim) = (%d, %d) is not supported", a->qk_dim, a->v_dim);
  if (a->v_offset < 0 || a->v_offset % 4 != 0 || a->v_offset + a->v_dim > a->qk_dim)
    return fail(IAK_EINVAL, "v_offset %d must be a multiple of 4 with v_offset + v_dim <= qk_dim", a->v_offset);
  if (a->page_size != 16) return fail(IAK_ENOTSUP, "page_size %d is not supported (16)", a->page_size);
  if (a->num_pages > 0x7FFFFFFFLL) return fail(IAK_EINVAL, "num_pages %lld exceeds int32 page ids", (long long)a->num_pages);
  if (a->q_dtype < 0 || a->q_dtype > 2 || a->out_dtype < 0 || a->out_dtype > 2)
    return fail(IAK_EINVAL, "bad q/out dtype (%d, %d)", a->q_dtype, a->out_dtype);
  if (!std::isfinite(a->sm_scale)) return fail(IAK_EINVAL, "sm_scale is not finite");
  if (a->pages_per_split < 0 || a->pages_per_split > 128)
    return fail(IAK_EINVAL, "pages_per_split %d outside [0, 128]", a->pages_per_split);
  if (a->scale_dtype != IAK_DTYPE_F16 && a->scale_dtype != IAK_DTYPE_F32)
    return fail(IAK_EINVAL, "scale dtype %d must be f16 or f32", a->scale_dtype);
  if (a->batch > 0) {
    if (!a->q || !a->out) return fail(IAK_EINVAL, "q/out is NULL");
    const int qvec = a->q_dtype == IAK_DTYPE_F32 ? 4 : 8;
    if (!aligned16(a->q) || a->q_stride_b % qvec != 0 || a->q_stride_h % qvec != 0)
      return fail(IAK_EINVAL, "q must be 16-byte aligned with strides that are multiples of %d elements", qvec);
    if (!a->page_table || !a->page_counts) return fail(IAK_EINVAL, "page_table/page_counts is NULL");
  }
  // latent pools reachable through the tag map (no tags: every page FP16)
  for (int t = 0; t < 8; ++t) {
    const int n = a->page_tags ? a->tag_map[t] : (t == 0 ? IAK_TAG_FP16 : IAK_TAG_SKIP);
    const void *pool = nullptr, *sc = nullptr;
    switch (n) {
      case IAK_TAG_FP16: pool = a->c_fp16; sc = pool; break;
      case IAK_TAG_FP8: pool = a->c_fp8; sc = a->c_fp8_scale; break;
      case IAK_TAG_INT8: pool = a->c_int8; sc = a->c_int8_scale; break;
      case IAK_TAG_INT4:
      case IAK_TAG_INT4_RESIDUAL:
        return fail(IAK_ENOTSUP, "tag %d maps to %s, which MLA latent pages do not support", t, tag_name(n));
      default: continue;
    }
    if (!pool || !sc) return fail(IAK_EINVAL, "tag %d maps to %s but its latent pool or scales are NULL", t, tag_name(n));
    if (!aligned16(pool)) return fail(IAK_EINVAL, "%s latent pool must be 16-byte aligned", tag_name(n));
  }

  // split plan: one workgroup per (sequence, split, 128 heads); enough
  // workgroups for every CU when the table is long enough
  const int W = a->table_width;
  const int HG = (a->num_heads + 127) / 128;
  int chunk = a->pages_per_split;
  if (chunk == 0) {
    const long long units = (long long)a->batch * HG;
    const long long want = units > 0 ? (256 + units - 1) / units : 1;
    chunk = (int)((W + want - 1) / (want > 0 ? want : 1));
    if (chunk > 128) chunk = 128;
    if (chunk < 1) chunk = 1;
  }
  int splits = (W + chunk - 1) / chunk;
  if (splits < 1) splits = 1;
  if ((long long)a->batch * splits > 0x7FFFFFFFLL || HG > 65535) return fail(IAK_EINVAL, "too many splits");
  plan->splits = splits;
  plan->chunk = chunk;
  plan->HG = HG;
  if (splits == 1) {
    plan->ws_m = plan->ws_l = plan->ws_acc = plan->total = 0;
  } else {
    const size_t slots = (size_t)a->batch * splits * a->num_heads;
    plan->ws_m = 0;
    plan->ws_l = round_up(slots * sizeof(float));
    plan->ws_acc = plan->ws_l + round_up(slots * sizeof(float));
    plan->total = plan->ws_acc + round_up(slots * a->v_dim * sizeof(float));
  }
  return IAK_OK;
}

}  // namespace

// Split-K partials of iak_paged_decode_noalloc: a library-owned device array
// (each GPU holds its own copy). In host code `scratch` names a host-side
// stand-in, not device memory: kernels get the device address that
// hipGetSymbolAddress returns for the current GPU (scratch_address).
static __device__ __align__(256) unsigned char scratch[IAK_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[MAX_DEVICES] = {};

// Device address of `scratch` on GPU `dev`, looked up once per device (with
// that device current) and kept.
iak_status scratch_address(int dev, void** out) {
  if (dev < 0 || dev >= MAX_DEVICES) return fail(IAK_EINVAL, "device %d outside [0, %d)", dev, MAX_DEVICES);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return fail(IAK_EHIP, "hipGetDevice failed: %s", hipGetErrorString(e));
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess)
      return fail(IAK_EHIP, "hipSetDevice(%d) failed: %s", dev, hipGetErrorString(e));
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    if (e != hipSuccess || !p)
      return fail(IAK_EHIP, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return IAK_OK;
}

}  // namespace

namespace iak {
hipError_t launch_mla_rows(const iak_mla_rows_args& a, void* workspace, hipStream_t stream);   // mla_rows.hip
size_t mla_rows_workspace(const iak_mla_rows_args& a);                                      // mla_rows.hip
hipError_t launch_fake_quant_blocks(const iak_fake_quant_blocks_args& a, void* workspace,
                                    hipStream_t stream);                    // fake_quant.hip
size_t fake_quant_blocks_workspace(const iak_fake_quant_blocks_args& a);   // fake_quant.hip
hipError_t launch_dense_attention(const iak_dense_attention_args& a, void* workspace,
                                  hipStream_t stream);                     // dense_attention.hip
size_t dense_attention_workspace(const iak_dense_attention_args& a);     // dense_attention.hip
}

extern "C" {

int iak_abi_version(void) { return IAK_ABI_VERSION; }

const char* iak_status_string(iak_status s) {
  switch (s) {
    case IAK_OK: return "ok";
    case IAK_EINVAL: return "invalid argument";
    case IAK_ENOTSUP: return "unsupported configuration";
    case IAK_EHIP: return "HIP runtime error";
  }
  return "unknown status";
}

const char* iak_last_error(void) { return g_err; }

iak_status iak_paged_decode_workspace(const iak_paged_decode_args* args, size_t* bytes) {
  if (!bytes) return fail(IAK_EINVAL, "bytes is NULL");
  Plan plan;
  const iak_status st = validate(args, &plan);
  if (st != IAK_OK) return st;
  *bytes = plan.total;
  return IAK_OK;
}

iak_status iak_paged_decode_plan(const iak_paged_decode_args* args, iak_paged_decode_plan_info* info) {
  if (!info) return fail(IAK_EINVAL, "info is NULL");
  Plan plan;
  const iak_status st = validate(args, &plan);
  if (st != IAK_OK) return st;
  info->splits = plan.splits;
  info->pages_per_split = plan.chunk;
  info->merge_in_kernel = plan.fused ? 1 : 0;
  info->tail_splits = plan.splits - plan.splitsA;
  info->tail_pages_per_split = plan.splits > plan.splitsA ? plan.chunkB : 0;
  info->workspace_bytes = plan.total;
  return IAK_OK;
}

// Tag translation, pools and scales of a decode (or of a pack). With page
// descriptors or entry records the tag map passes every native precision whose
// pools are given (they hold the native tag) and the scale arrays are not read;
// records also hold resolved page ids (negative_ids is not applied again).
static void fill_metadata(const iak_paged_decode_args* a, iak::KArgs& k) {
  const bool native = a->page_desc || a->entry_records;
  uint64_t map = 0;
  for (int t = 0; t < 8; ++t) {
    int n = native ? t : a->tag_map[t];
    if (n != IAK_TAG_FP16 && n != IAK_TAG_INT8 && n != IAK_TAG_FP8 && n != IAK_TAG_INT4 && n != IAK_TAG_INT4_RESIDUAL)
      n = IAK_TAG_SKIP;
    if (native) {
      const void* pool = n == IAK_TAG_FP16 ? a->k_fp16 : n == IAK_TAG_FP8 ? a->k_fp8 : n == IAK_TAG_INT8 ? a->k_int8
                       : n == IAK_TAG_INT4 ? a->k_int4 : n == IAK_TAG_INT4_RESIDUAL ? a->k_int4r : nullptr;
      if (!pool) n = IAK_TAG_SKIP;
    }
    map |= (uint64_t)n << (8 * t);
  }
  k.tagmap = map;
  k.other_tag = (a->map_other_tags && !native) ? (int)((map >> 56) & 0xFFu) : IAK_TAG_SKIP;
  k.desc = a->entry_records ? nullptr : static_cast<const uint32_t*>(a->page_desc);
  k.recs = static_cast<const uint32_t*>(a->entry_records);
  k.neg_wrap = a->negative_ids != 0 && !a->entry_records;
  k.valid = a->valid_tokens;
  k.k_fp16 = a->k_fp16; k.v_fp16 = a->v_fp16; k.k_fp8 = a->k_fp8; k.v_fp8 = a->v_fp8;
  k.k_int8 = a->k_int8; k.v_int8 = a->v_int8; k.k_int4 = a->k_int4; k.v_int4 = a->v_int4;
  k.k_int4r = a->k_int4r; k.v_int4r = a->v_int4r;
  k.k_fp8_scale = a->k_fp8_scale; k.v_fp8_scale = a->v_fp8_scale; k.fp8_sd = a->fp8_scale_dtype;
  k.k_int8_scale = a->k_int8_scale; k.v_int8_scale = a->v_int8_scale; k.int8_sd = a->int8_scale_dtype;
  k.k_int4_scale = a->k_int4_scale; k.v_int4_scale = a->v_int4_scale; k.int4_sd = a->int4_scale_dtype;
  k.int4_group = a->int4_group > 0 ? a->int4_group : a->head_dim;
  k.k_int4r_scale = a->k_int4r_scale; k.v_int4r_scale = a->v_int4r_scale;
}

iak_status iak_pack_page_descriptors(const iak_paged_decode_args* args, void* page_desc, void* stream) {
  if (!args) return fail(IAK_EINVAL, "args is NULL");
  // the descriptors come from page_tags, the tag map and the scales: validated
  // as for a decode without descriptors and without rows
  iak_paged_decode_args a = *args;
  a.page_desc = nullptr;
  a.entry_records = nullptr;
  a.batch = 0;
  Plan plan;
  const iak_status st = validate(&a, &plan);
  if (st != IAK_OK) return st;
  if (a.num_pages == 0) return IAK_OK;
  if (!a.page_tags) return fail(IAK_EINVAL, "page_tags is NULL");
  if (!page_desc || (reinterpret_cast<uintptr_t>(page_desc) & 31u))
    return fail(IAK_EINVAL, "page_desc must be non-NULL and 32-byte aligned");
  iak::KArgs k;
  std::memset(&k, 0, sizeof(k));
  k.D = a.head_dim;
  k.NP = a.num_pages;
  k.tags = a.page_tags;
  fill_metadata(&a, k);
  const hipError_t e = iak::launch_pack_descriptors(k, page_desc, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(IAK_EHIP, "kernel launch failed: %s", hipGetErrorString(e));
  return IAK_OK;
}

iak_status iak_pack_entry_records(const iak_paged_decode_args* args, void* records, void* stream) {
  if (!args) return fail(IAK_EINVAL, "args is NULL");
  // the records come from the table, the tags, the tag map and the scales:
  // validated as for a decode that reads them
  iak_paged_decode_args a = *args;
  a.page_desc = nullptr;
  a.entry_records = nullptr;
  Plan plan;
  const iak_status st = validate(&a, &plan);
  if (st != IAK_OK) return st;
  const int64_t entries = (int64_t)a.batch * a.num_kv_heads * a.table_width;
  if (entries == 0) return IAK_OK;
  if (!records || (reinterpret_cast<uintptr_t>(records) & 31u))
    return fail(IAK_EINVAL, "records must be non-NULL and 32-byte aligned");
  if (reinterpret_cast<uintptr_t>(a.page_table) & 3u) return fail(IAK_EINVAL, "page_table must be 4-byte aligned");
  iak::KArgs k;
  std::memset(&k, 0, sizeof(k));
  k.B = a.batch; k.Hkv = a.num_kv_heads; k.W = a.table_width; k.D = a.head_dim;
  k.NP = a.num_pages;
  k.table = a.page_table;
  k.tags = a.page_tags;
  fill_metadata(&a, k);
  const hipError_t e = iak::launch_pack_records(k, records, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(IAK_EHIP, "kernel launch failed: %s", hipGetErrorString(e));
  return IAK_OK;
}

static iak_status paged_decode_impl(const iak_paged_decode_args* a, void* workspace, size_t workspace_bytes,
                                    void* stream, void* ev_begin, void* ev_end, bool tiers = true) {
  Plan plan;
  iak_status st = validate(a, &plan, tiers);
  if (st != IAK_OK) return st;
  const long long rows = (long long)a->batch * a->num_kv_heads;
  if (rows == 0) return IAK_OK;
  if (plan.total > 0 && (!workspace || workspace_bytes < plan.total))
    return fail(IAK_EINVAL, "workspace of %zu bytes is smaller than the %zu bytes required", workspace_bytes, plan.total);
  if (plan.total > 0 && !aligned16(workspace)) return fail(IAK_EINVAL, "workspace must be 16-byte aligned");

  iak::KArgs k;
  std::memset(&k, 0, sizeof(k));
  k.B = a->batch; k.Hq = a->num_q_heads; k.Hkv = a->num_kv_heads; k.G = plan.G; k.D = a->head_dim;
  k.W = a->table_width; k.NP = a->num_pages;
  k.splits = plan.splits; k.chunk = plan.chunk; k.splitsA = plan.splitsA; k.chunkB = plan.chunkB;
  k.items = (int)(rows * plan.splits);
  k.q = a->q; k.q_dtype = a->q_dtype; k.q_f32 = a->q_dtype != IAK_DTYPE_F16;
  k.qsb = a->q_stride_b; k.qsh = a->q_stride_h;
  k.out = a->out; k.out_dtype = a->out_dtype; k.osb = a->out_stride_b; k.osh = a->out_stride_h;
  k.table = a->page_table; k.counts = a->page_counts; k.tags = a->page_tags;
  fill_metadata(a, k);
  k.score_mult = a->sm_scale * 1.4426950408889634f;
  if (plan.total > 0) {
    char* ws = static_cast<char*>(workspace);
    k.ws_m = reinterpret_cast<float*>(ws + plan.ws_m);
    k.ws_l = reinterpret_cast<float*>(ws + plan.ws_l);
    k.ws_acc = reinterpret_cast<float*>(ws + plan.ws_acc);
    if (plan.fused) {
      k.fused = 1;
      k.counters = reinterpret_cast<int32_t*>(ws + plan.ws_cnt);
    }
  }
  const hipError_t e = iak::launch_paged_decode(k, static_cast<hipStream_t>(stream),
                                                static_cast<hipEvent_t>(ev_begin), static_cast<hipEvent_t>(ev_end));
  if (e != hipSuccess) return fail(IAK_EHIP, "kernel launch failed: %s", hipGetErrorString(e));
  return IAK_OK;
}

iak_status iak_paged_decode(const iak_paged_decode_args* a, void* workspace, size_t workspace_bytes,
                            void* stream) {
  return paged_decode_impl(a, workspace, workspace_bytes, stream, nullptr, nullptr);
}

iak_status iak_paged_decode_timed(const iak_paged_decode_args* a, void* workspace, size_t workspace_bytes,
                                  void* stream, void* ev_begin, void* ev_end) {
  return paged_decode_impl(a, workspace, workspace_bytes, stream, ev_begin, ev_end);
}

iak_status iak_paged_decode_noalloc(const iak_paged_decode_args* args, void* stream) {
  if (!args) return fail(IAK_EINVAL, "args is NULL");
  // the scratch array holds split partials only: the merge kernel combines them
  iak_paged_decode_args local = *args;
  local.merge_in_kernel = 0;
  const iak_paged_decode_args* a = &local;
  Plan plan;
  const iak_status st = validate(a, &plan, false);
  if (st != IAK_OK) return st;
  if (plan.total > IAK_NOALLOC_SCRATCH_BYTES)
    return fail(IAK_EINVAL,
                "split-K partials of %zu bytes exceed the %zu-byte no-alloc scratch; use iak_paged_decode with a "
                "caller workspace (or fewer splits: pages_per_split)",
                plan.total, (size_t)IAK_NOALLOC_SCRATCH_BYTES);
  if ((long long)a->batch * a->num_kv_heads == 0) return IAK_OK;
  void* ws = nullptr;
  if (plan.total > 0) {
    int dev = -1;
    const hipError_t e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &dev);
    if (e != hipSuccess) return fail(IAK_EHIP, "hipStreamGetDevice failed: %s", hipGetErrorString(e));
    const iak_status s2 = scratch_address(dev, &ws);
    if (s2 != IAK_OK) return s2;
  }
  return paged_decode_impl(a, ws, plan.total, stream, nullptr, nullptr, false);
}

iak_status iak_mla_decode_workspace(const iak_mla_decode_args* args, size_t* bytes) {
  if (!bytes) return fail(IAK_EINVAL, "bytes is NULL");
  MPlan plan;
  const iak_status st = validate_mla(args, &plan);
  if (st != IAK_OK) return st;
  *bytes = plan.total;
  return IAK_OK;
}

static iak_status mla_decode_impl(const iak_mla_decode_args* a, void* workspace, size_t workspace_bytes,
                                  void* stream, void* ev_begin, void* ev_end) {
  MPlan plan;
  iak_status st = validate_mla(a, &plan);
  if (st != IAK_OK) return st;
  if (a->batch == 0) return IAK_OK;
  if (plan.total > 0 && (!workspace || workspace_bytes < plan.total))
    return fail(IAK_EINVAL, "workspace of %zu bytes is smaller than the %zu bytes required", workspace_bytes, plan.total);
  if (plan.total > 0 && !aligned16(workspace)) return fail(IAK_EINVAL, "workspace must be 16-byte aligned");

  iak::MArgs m;
  std::memset(&m, 0, sizeof(m));
  m.B = a->batch; m.H = a->num_heads; m.DQK = a->qk_dim; m.DV = a->v_dim; m.VOFF = a->v_offset;
  m.W = a->table_width; m.NP = a->num_pages;
  m.splits = plan.splits; m.chunk = plan.chunk; m.HG = plan.HG;
  m.q = a->q; m.q_dtype = a->q_dtype; m.qsb = a->q_stride_b; m.qsh = a->q_stride_h;
  m.out = a->out; m.out_dtype = a->out_dtype; m.osb = a->out_stride_b; m.osh = a->out_stride_h;
  m.table = a->page_table; m.counts = a->page_counts; m.tags = a->page_tags;
  uint64_t map = 0;
  for (int t = 0; t < 8; ++t) {
    int n = a->tag_map[t];
    if (n != IAK_TAG_FP16 && n != IAK_TAG_INT8 && n != IAK_TAG_FP8) n = IAK_TAG_SKIP;
    map |= (uint64_t)n << (8 * t);
  }
  m.tagmap = map;
  m.wide = 0;
  for (int t = 0; t < 8; ++t)
    if (((map >> (8 * t)) & 0xFFu) == IAK_TAG_FP16) m.wide = 1;
  if (!a->page_tags) m.wide = 1;
  m.neg_wrap = a->negative_ids != 0;
  m.valid = a->valid_tokens;
  m.c16 = a->c_fp16; m.c8f = a->c_fp8; m.c8i = a->c_int8;
  m.s8f = a->c_fp8_scale; m.s8i = a->c_int8_scale; m.sd = a->scale_dtype;
  m.score_mult = a->sm_scale * 1.4426950408889634f;
  // Compact split partials: each split's context acc / l rounded to float16
  // (relative error <= 2^-11, 1/128 of an e4m3 code's) when every reachable
  // page is FP8 / INT8 and the output itself is 16-bit; FP16 pages or a
  // float32 output keep float32 partials.
  m.acc16 = (!m.wide && a->out_dtype != IAK_DTYPE_F32) ? 1 : 0;
  if (plan.total > 0) {
    char* ws = static_cast<char*>(workspace);
    m.ws_m = reinterpret_cast<float*>(ws + plan.ws_m);
    m.ws_l = reinterpret_cast<float*>(ws + plan.ws_l);
    m.ws_acc = reinterpret_cast<float*>(ws + plan.ws_acc);
  }
  const hipError_t e = iak::launch_mla_decode(m, static_cast<hipStream_t>(stream),
                                              static_cast<hipEvent_t>(ev_begin), static_cast<hipEvent_t>(ev_end));
  if (e != hipSuccess) return fail(IAK_EHIP, "kernel launch failed: %s", hipGetErrorString(e));
  return IAK_OK;
}

iak_status iak_mla_decode(const iak_mla_decode_args* a, void* workspace, size_t workspace_bytes, void* stream) {
  return mla_decode_impl(a, workspace, workspace_bytes, stream, nullptr, nullptr);
}

iak_status iak_mla_decode_timed(const iak_mla_decode_args* a, void* workspace, size_t workspace_bytes,
                                void* stream, void* ev_begin, void* ev_end) {
  return mla_decode_impl(a, workspace, workspace_bytes, stream, ev_begin, ev_end);
}

iak_status iak_timing_event_create(void** event) {
  if (!event) return fail(IAK_EINVAL, "event is NULL");
  hipEvent_t e = nullptr;
  const hipError_t err = hipEventCreateWithFlags(&e, hipEventDisableSystemFence);
  if (err != hipSuccess) return fail(IAK_EHIP, "hipEventCreateWithFlags failed: %s", hipGetErrorString(err));
  *event = e;
  return IAK_OK;
}

iak_status iak_timing_event_record(void* event, void* stream) {
  if (!event) return fail(IAK_EINVAL, "event is NULL");
  const hipError_t err = hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(IAK_EHIP, "hipEventRecord failed: %s", hipGetErrorString(err));
  return IAK_OK;
}

iak_status iak_timing_event_elapsed(void* start, void* end, float* ms) {
  if (!start || !end || !ms) return fail(IAK_EINVAL, "start/end/ms is NULL");
  const hipError_t err = hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(end));
  if (err != hipSuccess) return fail(IAK_EHIP, "hipEventElapsedTime failed: %s", hipGetErrorString(err));
  return IAK_OK;
}

iak_status iak_timing_event_destroy(void* event) {
  if (!event) return IAK_OK;
  const hipError_t err = hipEventDestroy(static_cast<hipEvent_t>(event));
  if (err != hipSuccess) return fail(IAK_EHIP, "hipEventDestroy failed: %s", hipGetErrorString(err));
  return IAK_OK;
}

iak_status iak_quantize_pages(const iak_quantize_args* a, void* stream) {
  if (!a) return fail(IAK_EINVAL, "args is NULL");
  if (a->num_pages < 0 || a->pool_pages < 0) return fail(IAK_EINVAL, "negative page count");
  if (a->head_dim != 64 && a->head_dim != 128)
    return fail(IAK_ENOTSUP, "head_dim %d is not supported (64 or 128)", a->head_dim);
  if (a->page_size != 16) return fail(IAK_ENOTSUP, "page_size %d is not supported (16)", a->page_size);
  const int p = a->precision, m = a->mode;
  if (m == IAK_QUANT_FAKE_QUANTIZE) {
    if (p != IAK_TAG_FP8 && p != IAK_TAG_INT8 && p != IAK_TAG_INT4 && p != IAK_TAG_INT4_RESIDUAL)
      return fail(IAK_EINVAL, "precision %d cannot be quantised (FP8, INT8, INT4 or INT4_RESIDUAL)", p);
  } else if (m == IAK_QUANT_FUSED_INT8 || m == IAK_QUANT_TRITON_INT8) {
    if (p != IAK_TAG_INT8) return fail(IAK_EINVAL, "mode %d writes INT8 pages only", m);
  } else {
    return fail(IAK_EINVAL, "unknown quantisation mode %d", m);
  }
  if (p == IAK_TAG_INT4) {
    const int grp = a->int4_group, D = a->head_dim;
    if (grp <= 0 || D % grp != 0 || grp % (D / 4) != 0)
      return fail(IAK_ENOTSUP, "int4_group %d must divide head_dim %d and be a multiple of %d", grp, D, D / 4);
  }
  if (a->scale_dtype != IAK_DTYPE_F16 && a->scale_dtype != IAK_DTYPE_F32)
    return fail(IAK_EINVAL, "scale dtype %d must be f16 or f32", a->scale_dtype);
  if (a->num_pages == 0) return IAK_OK;
  if (!a->src || !a->codes || !a->scales) return fail(IAK_EINVAL, "src/codes/scales is NULL");
  if (!aligned16(a->src) || !aligned16(a->codes)) return fail(IAK_EINVAL, "src and codes must be 16-byte aligned");
  const hipError_t e = iak::launch_quantize_pages(*a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(IAK_EHIP, "kernel launch failed: %s", hipGetErrorString(e));
  return IAK_OK;
}

iak_status iak_transcode_pages(const iak_transcode_args* a, void* stream) {
  if (!a) return fail(IAK_EINVAL, "args is NULL");
  if (a->num_pages < 0 || a->pool_pages < 0) return fail(IAK_EINVAL, "negative page count");
  if (a->mode != IAK_TRANSCODE_DEMOTE_INT8 && a->mode != IAK_TRANSCODE_PROMOTE_FP16)
    return fail(IAK_EINVAL, "unknown transcode mode %d", a->mode);
  if (a->page_elems <= 0 || a->page_elems % 8 != 0)
    return fail(IAK_ENOTSUP, "page_elems %d must be a positive multiple of 8", a->page_elems);
  if (a->num_pages == 0) return IAK_OK;
  if (!a->fp16 || !a->int8 || !a->scales) return fail(IAK_EINVAL, "fp16/int8/scales is NULL");
  if (!aligned16(a->fp16) || (reinterpret_cast<uintptr_t>(a->int8) & 7u) ||
      (reinterpret_cast<uintptr_t>(a->scales) & 3u) || (reinterpret_cast<uintptr_t>(a->pages) & 3u))
    return fail(IAK_EINVAL, "the fp16 pool must be 16-byte aligned, the int8 pool 8-byte aligned, scales and "
                "pages 4-byte aligned");
  if (!a->pages && a->num_pages > a->pool_pages)
    return fail(IAK_EINVAL, "num_pages %d exceeds pool_pages %lld without a slot list", a->num_pages,
                (long long)a->pool_pages);
  const hipError_t e = iak::launch_transcode(*a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(IAK_EHIP, "kernel launch failed: %s", hipGetErrorString(e));
  return IAK_OK;
}

iak_status iak_prefetch_pages(const iak_prefetch_args* a, void* stream) {
  if (!a) return fail(IAK_EINVAL, "args is NULL");
  if (a->batch < 0 || a->heads < 0 || a->kv_len < 0 || a->num_ids < 0 || a->head_dim <= 0 || a->page_size <= 0)
    return fail(IAK_EINVAL, "negative size or non-positive head_dim / page_size");
  if ((long long)a->batch * a->heads > 65535) return fail(IAK_ENOTSUP, "batch * heads above 65535");
  if (a->num_ids == 0 || a->batch == 0 || a->heads == 0) return IAK_OK;
  if (!a->page_ids || !a->k || !a->v || !a->checksum) return fail(IAK_EINVAL, "page_ids/k/v/checksum is NULL");
  if ((reinterpret_cast<uintptr_t>(a->k) | reinterpret_cast<uintptr_t>(a->v)) & 1u)
    return fail(IAK_EINVAL, "k/v must be 2-byte aligned");
  const hipError_t e = iak::launch_prefetch(*a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(IAK_EHIP, "kernel launch failed: %s", hipGetErrorString(e));
  return IAK_OK;
}

static iak_status validate_mla_rows(const iak_mla_rows_args* a) {
  if (!a) return fail(IAK_EINVAL, "args is NULL");
  if (a->batch < 0 || a->q_len < 0 || a->num_selected < 0 || a->num_rows < 0)
    return fail(IAK_EINVAL, "negative size (batch=%d, q_len=%d, num_selected=%d, num_rows=%lld)", a->batch, a->q_len,
                a->num_selected, (long long)a->num_rows);
  if (a->latent_dim <= 0 || a->latent_dim > 1024)
    return fail(IAK_ENOTSUP, "latent_dim %d is not supported (1 .. 1024)", a->latent_dim);
  if (a->page_size <= 0) return fail(IAK_EINVAL, "page_size must be positive, got %d", a->page_size);
  if ((long long)a->batch * a->q_len > 0x7FFFFFFFLL) return fail(IAK_EINVAL, "batch * q_len too large");
  // the kernel's key indexes (num_selected * page_size keys) run up to 128 past the
  // last key in 32-bit arithmetic
  if ((long long)a->num_selected * a->page_size > 0x7FFFFFFF - 4096)
    return fail(IAK_ENOTSUP, "num_selected * page_size = %lld keys is not supported (at most %d)",
                (long long)a->num_selected * a->page_size, 0x7FFFFFFF - 4096);
  for (int dt : {a->q_dtype, a->latent_dtype})
    if (dt < 0 || dt > 2) return fail(IAK_EINVAL, "unknown dtype %d", dt);
  if ((long long)a->batch * a->q_len == 0) return IAK_OK;
  if (!a->q || !a->context) return fail(IAK_EINVAL, "q/context is NULL");
  if (a->num_selected > 0 && (!a->page_ids || !a->latents)) return fail(IAK_EINVAL, "page_ids/latents is NULL");
  if (a->latent_stride < a->latent_dim && a->num_rows > 1)
    return fail(IAK_EINVAL, "latent_stride %lld is below latent_dim %d", (long long)a->latent_stride, a->latent_dim);
  if (a->num_selected > 0 && a->num_rows <= 0) return fail(IAK_EINVAL, "num_rows is 0 with pages listed");
  return IAK_OK;
}

iak_status iak_mla_decode_rows_workspace(const iak_mla_rows_args* a, size_t* bytes) {
  if (!bytes) return fail(IAK_EINVAL, "bytes is NULL");
  const iak_status st = validate_mla_rows(a);
  if (st != IAK_OK) return st;
  *bytes = (long long)a->batch * a->q_len == 0 ? 0 : iak::mla_rows_workspace(*a);
  return IAK_OK;
}

iak_status iak_mla_decode_rows(const iak_mla_rows_args* a, void* workspace, size_t workspace_bytes, void* stream) {
  const iak_status st = validate_mla_rows(a);
  if (st != IAK_OK) return st;
  if ((long long)a->batch * a->q_len == 0) return IAK_OK;
  if (workspace) {
    const size_t need = iak::mla_rows_workspace(*a);
    if (workspace_bytes < need)
      return fail(IAK_EINVAL, "workspace of %zu bytes is smaller than the %zu bytes required", workspace_bytes, need);
    if (!aligned16(workspace)) return fail(IAK_EINVAL, "workspace must be 16-byte aligned");
  }
  const hipError_t e = iak::launch_mla_rows(*a, workspace, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(IAK_EHIP, "kernel launch failed: %s", hipGetErrorString(e));
  return IAK_OK;
}

static iak_status validate_dense(const iak_dense_attention_args* a) {
  if (!a) return fail(IAK_EINVAL, "args is NULL");
  if (a->batch < 0 || a->q_len < 0 || a->kv_len < 0)
    return fail(IAK_EINVAL, "negative size (batch=%d, q_len=%d, kv_len=%d)", a->batch, a->q_len, a->kv_len);
  if (a->head_dim <= 0 || a->head_dim > 1024 || a->v_dim <= 0 || a->v_dim > 1024)
    return fail(IAK_ENOTSUP, "head_dim %d / v_dim %d is not supported (1 .. 1024)", a->head_dim, a->v_dim);
  if (a->dtype < 0 || a->dtype > 2) return fail(IAK_EINVAL, "unknown dtype %d", a->dtype);
  // the kernel's key indexes run up to 128 past kv_len in 32-bit arithmetic
  if (a->kv_len > 0x7FFFFFFF - 4096)
    return fail(IAK_ENOTSUP, "kv_len %d is not supported (at most %d)", a->kv_len, 0x7FFFFFFF - 4096);
  if (a->mask && (a->mask_dtype < 0 || a->mask_dtype > IAK_MASK_BOOL))
    return fail(IAK_EINVAL, "unknown mask dtype %d", a->mask_dtype);
  if (a->causal < IAK_CAUSAL_NONE || a->causal > IAK_CAUSAL_POSITIONS)
    return fail(IAK_EINVAL, "causal must be 0, 1 or 2, got %d", a->causal);
  if ((long long)a->batch * a->q_len > 0x7FFFFFFFLL) return fail(IAK_EINVAL, "batch * q_len too large");
  if ((long long)a->batch * a->q_len == 0) return IAK_OK;
  if (!a->q || !a->out) return fail(IAK_EINVAL, "q/out is NULL");
  if (a->kv_len > 0 && (!a->k || !a->v)) return fail(IAK_EINVAL, "k/v is NULL");
  if (a->kv_len > 0 && a->causal == IAK_CAUSAL_POSITIONS && !a->kv_positions)
    return fail(IAK_EINVAL, "kv_positions is NULL with causal = IAK_CAUSAL_POSITIONS");
  const long long strides[] = {a->q_stride_b, a->q_stride_t, a->k_stride_b, a->k_stride_t, a->v_stride_b,
                               a->v_stride_t, a->out_stride_b, a->out_stride_t};
  for (long long st : strides)
    if (st < 0) return fail(IAK_EINVAL, "negative stride %lld", st);
  if (a->mask && (a->mask_stride_b < 0 || a->mask_stride_q < 0 || a->mask_stride_k < 0))
    return fail(IAK_EINVAL, "negative mask stride");
  return IAK_OK;
}

iak_status iak_dense_attention_workspace(const iak_dense_attention_args* a, size_t* bytes) {
  if (!bytes) return fail(IAK_EINVAL, "bytes is NULL");
  const iak_status st = validate_dense(a);
  if (st != IAK_OK) return st;
  *bytes = (long long)a->batch * a->q_len == 0 ? 0 : iak::dense_attention_workspace(*a);
  return IAK_OK;
}

iak_status iak_dense_attention(const iak_dense_attention_args* a, void* workspace, size_t workspace_bytes,
                               void* stream) {
  const iak_status st = validate_dense(a);
  if (st != IAK_OK) return st;
  if ((long long)a->batch * a->q_len == 0) return IAK_OK;
  if (workspace) {
    const size_t need = iak::dense_attention_workspace(*a);
    if (workspace_bytes < need)
      return fail(IAK_EINVAL, "workspace of %zu bytes is smaller than the %zu bytes required", workspace_bytes, need);
    if (!aligned16(workspace)) return fail(IAK_EINVAL, "workspace must be 16-byte aligned");
  }
  const hipError_t e = iak::launch_dense_attention(*a, workspace, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(IAK_EHIP, "kernel launch failed: %s", hipGetErrorString(e));
  return IAK_OK;
}

static iak_status validate_fake_quant(const iak_fake_quant_blocks_args* a) {
  if (!a) return fail(IAK_EINVAL, "args is NULL");
  if (a->lead < 0 || a->num_blocks < 0 || a->k_dim < 0 || a->v_dim < 0 || a->max_block_tokens < 0)
    return fail(IAK_EINVAL, "negative size (lead=%d, num_blocks=%d, k_dim=%d, v_dim=%d, max_block_tokens=%d)",
                a->lead, a->num_blocks, a->k_dim, a->v_dim, a->max_block_tokens);
  if ((long long)a->k_dim + a->v_dim > (1LL << 20))
    return fail(IAK_ENOTSUP, "k_dim + v_dim = %lld is not supported (at most 2^20)", (long long)a->k_dim + a->v_dim);
  if (a->num_blocks >= (1 << 22))   // the grid's x extent in work-items stays below 2^32
    return fail(IAK_ENOTSUP, "num_blocks = %d is not supported (below 2^22)", a->num_blocks);
  if (a->lead == 0 || a->num_blocks == 0 || a->k_dim + a->v_dim == 0) return IAK_OK;
  if (!a->blocks || !a->out || (a->k_dim > 0 && !a->k) || (a->v_dim > 0 && !a->v))
    return fail(IAK_EINVAL, "k/v/blocks/out is NULL");
  const long long strides[] = {a->k_stride_l, a->k_stride_t, a->v_stride_l, a->v_stride_t, a->out_stride_l,
                               a->out_stride_t};
  for (long long st : strides)
    if (st < 0) return fail(IAK_EINVAL, "negative stride %lld", st);
  return IAK_OK;
}

iak_status iak_fake_quant_blocks_workspace(const iak_fake_quant_blocks_args* a, size_t* bytes) {
  if (!bytes) return fail(IAK_EINVAL, "bytes is NULL");
  const iak_status st = validate_fake_quant(a);
  if (st != IAK_OK) return st;
  *bytes = (a->lead == 0 || a->num_blocks == 0 || a->k_dim + a->v_dim == 0) ? 0 : iak::fake_quant_blocks_workspace(*a);
  return IAK_OK;
}

iak_status iak_fake_quant_blocks(const iak_fake_quant_blocks_args* a, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  const iak_status st = validate_fake_quant(a);
  if (st != IAK_OK) return st;
  if (a->lead == 0 || a->num_blocks == 0 || a->k_dim + a->v_dim == 0) return IAK_OK;
  if (workspace) {
    const size_t need = iak::fake_quant_blocks_workspace(*a);
    if (workspace_bytes < need)
      return fail(IAK_EINVAL, "workspace of %zu bytes is smaller than the %zu bytes required", workspace_bytes, need);
    if (!aligned16(workspace)) return fail(IAK_EINVAL, "workspace must be 16-byte aligned");
  }
  const hipError_t e = iak::launch_fake_quant_blocks(*a, workspace, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(IAK_EHIP, "kernel launch failed: %s", hipGetErrorString(e));
  return IAK_OK;
}

iak_status iak_build_page_tables(const iak_page_table_args* a, void* stream) {
  if (!a) return fail(IAK_EINVAL, "args is NULL");
  if (a->num_rows < 0 || a->table_width < 0 || a->num_pages < 0)
    return fail(IAK_EINVAL, "negative num_rows / table_width / num_pages");
  if (a->rows_per_seq <= 0 || a->rows_per_list <= 0)
    return fail(IAK_EINVAL, "rows_per_seq and rows_per_list must be positive");
  if (a->page_size <= 0) return fail(IAK_EINVAL, "page_size must be positive, got %d", a->page_size);
  if (a->dedupe != 0 && a->dedupe != 1) return fail(IAK_EINVAL, "dedupe must be 0 or 1");
  if (a->default_tag < IAK_TAG_FP16 || a->default_tag > IAK_TAG_INT4_RESIDUAL)
    return fail(IAK_EINVAL, "default_tag %d is not a page tag", a->default_tag);
  if (a->block_table && a->block_table_width <= 0)
    return fail(IAK_EINVAL, "block_table_width must be positive with a block table");
  if (a->page_precision && a->num_rows >= (1 << 28))
    return fail(IAK_ENOTSUP, "num_rows %d too large for the precision reduction (< 2^28)", a->num_rows);
  if (a->num_rows > 0) {
    if (!a->span_offsets || !a->span_begin || !a->span_end || !a->span_tag)
      return fail(IAK_EINVAL, "span arrays must not be NULL");
    if (!a->page_counts || (a->table_width > 0 && !a->page_table))
      return fail(IAK_EINVAL, "page_table / page_counts is NULL");
  }
  {
    const void* arrays[] = {a->span_offsets, a->span_begin, a->span_end,  a->span_tag,
                            a->block_table,  a->page_table, a->page_counts, a->page_precision};
    for (const void* p : arrays)
      if (reinterpret_cast<uintptr_t>(p) & 3u) return fail(IAK_EINVAL, "int32 arrays must be 4-byte aligned");
  }
  const hipError_t e = iak::launch_page_tables(*a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(IAK_EHIP, "kernel launch failed: %s", hipGetErrorString(e));
  return IAK_OK;
}

}  // extern "C"
