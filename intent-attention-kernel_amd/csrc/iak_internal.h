// Kernel-side argument block of libiak (device pointers and derived sizes),
// built by the C ABI layer (iak_api.hip) from iak_paged_decode_args.
#ifndef IAK_INTERNAL_H
#define IAK_INTERNAL_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "iak.h"

#define IAK_WAVES_PER_BLOCK 4
#define IAK_MIN_WAVES_PER_SIMD 3
// compute units of the MI355X / MI350X (gfx950) the split plan sizes grids for
#define IAK_GPU_CUS 256
// two-tier split plans: from this many waves (about 1.5 resident generations
// of 3 waves per SIMD) the last quarter of each row goes in splits of about
// IAK_TIER_CHUNK entries
#define IAK_TIER_MIN_WAVES (IAK_GPU_CUS * 4 * IAK_MIN_WAVES_PER_SIMD * 3 / 2)
#define IAK_TIER_CHUNK 40
// pages per ring in each precision class loop (one computed, the rest in flight)
#ifndef IAK_RING_FP16
#define IAK_RING_FP16 2
#endif
#ifndef IAK_RING_BYTE
#define IAK_RING_BYTE 3
#endif
#ifndef IAK_RING_INT4
#define IAK_RING_INT4 5
#endif

namespace iak {

struct KArgs {
  int B, Hq, Hkv, G, D, W;
  int64_t NP;
  int splits;   // splits per (batch, kv head) row
  int chunk;    // table entries per split (<= 64)
  int items;    // B * Hkv * splits waves

  const void* q; int q_dtype; int q_f32; int64_t qsb, qsh;
  void* out; int out_dtype; int64_t osb, osh;

  const int32_t* table;
  const int32_t* counts;
  const int32_t* tags;
  uint64_t tagmap;   // byte t = native tag of caller tag t
  int other_tag;     // native tag of caller tags outside [0, 8)
  int neg_wrap;
  const int32_t* valid;   // [B, Hkv] token bound per row, may be null

  const void* k_fp16; const void* v_fp16;
  const void* k_fp8; const void* v_fp8;
  const void* k_int8; const void* v_int8;
  const void* k_int4; const void* v_int4;
  const void* k_int4r; const void* v_int4r;
  const void* k_fp8_scale; const void* v_fp8_scale; int fp8_sd;
  const void* k_int8_scale; const void* v_int8_scale; int int8_sd;
  const void* k_int4_scale; const void* v_int4_scale; int int4_sd; int int4_group;
  const float* k_int4r_scale; const float* v_int4r_scale;

  float score_mult;   // sm_scale * log2(e)

  float* ws_m;        // [B, Hkv, splits, G]
  float* ws_l;        // [B, Hkv, splits, G]
  float* ws_acc;      // [B, Hkv, splits, G, D]
  int acc16;          // ws_acc holds acc / l as float16 (the MLA kernel's compact partials)

  // merge inside the decode kernel: the partials are per workgroup (4 splits),
  // [B, Hkv, splits / 4, G] and [.., D]; counters [B * Hkv] arrivals per row
  int fused;
  int32_t* counters;

  // page descriptors (iak_paged_decode_args.page_desc): [NP] x 32 B as two u4 (tag word, scale slots)
  const uint32_t* desc;
  // entry records (iak_paged_decode_args.entry_records): [B * Hkv * W] x 32 B as two u4
  // ((native tag, page id, 0, 0), scale slots)
  const uint32_t* recs;

  // two-tier plan: splits 0 .. splitsA-1 of a row take `chunk` entries each and
  // come first in the grid (all rows); splits splitsA .. splits-1 take chunkB
  // entries and come last. splitsA == splits: one tier.
  int splitsA, chunkB;
};

// page descriptors from page_tags, the tag map and the scale arrays of `k`
hipError_t launch_pack_descriptors(const KArgs& k, void* desc, hipStream_t stream);
// entry records from the page table, page_tags, the tag map and the scale arrays of `k`
hipError_t launch_pack_records(const KArgs& k, void* recs, hipStream_t stream);

// ev_begin / ev_end (may be null) are recorded on `stream` around the split
// kernel alone, so callers can time it apart from the merge
hipError_t launch_paged_decode(const KArgs& k, hipStream_t stream, hipEvent_t ev_begin = nullptr,
                               hipEvent_t ev_end = nullptr);

// Kernel-side arguments of the MLA latent decode (built from iak_mla_decode_args).
struct MArgs {
  int B, H, DQK, DV, VOFF, W;
  int64_t NP;
  int splits;   // splits per sequence
  int chunk;    // table entries per split (<= 128)
  int HG;       // groups of 128 heads

  const void* q; int q_dtype; int64_t qsb, qsh;
  void* out; int out_dtype; int64_t osb, osh;

  const int32_t* table;
  const int32_t* counts;
  const int32_t* tags;     // may be null: every page FP16
  uint64_t tagmap;
  int neg_wrap;
  const int32_t* valid;    // [B] token bound per sequence, may be null

  const void* c16; const void* c8f; const void* c8i;
  const void* s8f; const void* s8i; int sd;
  int wide;           // FP16 latent pages are reachable

  float score_mult;   // sm_scale * log2(e)

  float* ws_m;        // [B, splits, H]
  float* ws_l;        // [B, splits, H]
  float* ws_acc;      // [B, splits, H, DV]
  int acc16;          // write acc / l as float16 into ws_acc instead of acc as float32
};

hipError_t launch_mla_decode(const MArgs& m, hipStream_t stream, hipEvent_t ev_begin = nullptr,
                             hipEvent_t ev_end = nullptr);

hipError_t launch_quantize_pages(const iak_quantize_args& a, hipStream_t stream);

hipError_t launch_page_tables(const iak_page_table_args& a, hipStream_t stream);

hipError_t launch_transcode(const iak_transcode_args& a, hipStream_t stream);

hipError_t launch_prefetch(const iak_prefetch_args& a, hipStream_t stream);

}  // namespace iak

#endif
