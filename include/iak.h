/*
 * iak.h -- C ABI of the MI355X (gfx950) selected-quant paged decode library
 * (libiak.so). Plain pointers, sizes and status codes; no torch or HIP types.
 *
 * Ownership: the caller owns every buffer (inputs, output, workspace). The
 * library allocates nothing and keeps no state between calls, apart from the
 * static per-GPU scratch of iak_paged_decode_noalloc; calls are asynchronous
 * on the caller's HIP stream and never synchronise the host.
 *
 * Reference interfaces these entry points replace (paths relative to the
 * reference's src/intent_attention/):
 *   iak_paged_decode            fused_selected_quant_decode()          fused_selected_quant_decode.py:408-464
 *                               (its Triton launch _launch_triton_kernel :472-513, kernel :87-255)
 *                               and intent_quant_decode_attention_triton()
 *                                                                      triton_intent_quant_attention.py:342-457
 *   iak_paged_decode_workspace  (no counterpart: sizes the split-K partial buffer the caller allocates)
 *   iak_paged_decode_plan       (no counterpart: the split plan the library chooses for a call)
 *   iak_pack_page_descriptors   (no counterpart: page_precision, page_tags and the per-precision scale
 *                               arrays of fused_selected_quant_decode.py:408-464 packed into one
 *                               32-byte descriptor per page)
 *   iak_pack_entry_records      (no counterpart: the page table's entries with their page's native
 *                               tag and scales (fused_selected_quant_decode.py:344-400 reads them
 *                               entry by entry) packed into one 32-byte record per entry)
 *   iak_paged_decode_timed,     (no counterpart: the same calls with HIP events around the split
 *   iak_mla_decode_timed         kernel, for timing it apart from the merge)
 *   iak_timing_event_*          (no counterpart: fence-free HIP timing events for those calls)
 *   iak_mla_decode              mla_decode_triton() / _mla_decode_cpu()    triton_mla_decode.py:110-186
 *                               (the latent context; mla_sparse_decode_reference mla.py:61-92,
 *                               mla_triton_decode mla.py:95-136)
 *   iak_mla_decode_workspace    (no counterpart: sizes the split-K partial buffer)
 *   iak_mla_decode_rows_workspace (no counterpart: sizes the optional split-over-keys partial buffer)
 *   iak_mla_decode_rows         the latent context of mla_decode_triton() in the reference's float32
 *                               arithmetic: its Triton kernel triton_mla_decode.py:47-107 and
 *                               _mla_decode_cpu :155-186 (also under mla_sparse_decode_reference /
 *                               mla_triton_decode, mla.py:61-136)
 *   iak_quantize_pages          fake_quantize_tensor() intent_quant.py:221-312 at page granules, and
 *                               fake_int8_pages_from_fp16() fused_selected_quant_decode.py:521-542 /
 *                               triton_intent_quant_attention.py:460-496
 *   iak_build_page_tables       routing_to_kernel_metadata() block_router.py:383-421 (page ids: selected_page_ids
 *                               :283-296) followed by metadata_to_kernel_tensors()
 *                               fused_selected_quant_decode.py:344-400 (the loop :394-398)
 *   iak_transcode_pages         KVMemoryManager FP16 <-> INT8 page transcoding: write_page's INT8 branch
 *                               kv_memory_manager.py:233-252, _read_page_data :286-296, set_page_format
 *                               :268-284 (demote_cold_pages :350-362, promote_hot_pages :364-377)
 *   iak_prefetch_pages          launch_prefetch_pages() prefetch.py:183-261 (its Triton kernel :111-170)
 *   iak_dense_attention         dense_attention() reference.py:16-45 (causal, mask, original_kv_positions),
 *                               under semantic_block_attention() reference.py:81-129 and
 *                               intent_quant_attention_reference() intent_quant_attention.py:20-119
 *   iak_dense_attention_workspace (no counterpart: sizes the optional split-over-keys partial buffer)
 *   iak_fake_quant_blocks       the per-block fake_quantize_tensor() reconstructions and their torch.cat
 *                               in intent_quant_attention_reference() intent_quant_attention.py:56-84
 *                               (intent_quant.py:221-312), float32 K and V
 *   iak_fake_quant_blocks_workspace (no counterpart: sizes the optional split of long blocks)
 *   iak_status_string           (no counterpart: the reference raises ValueError/RuntimeError in Python)
 */
#ifndef IAK_H
#define IAK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IAK_ABI_VERSION 11

/* Grid size from which merge_in_kernel = 2 merges inside the decode kernel; it
 * also does so on grids of at most IAK_MERGE_IN_KERNEL_SMALL_WORKGROUPS workgroups
 * whose rows hold at most IAK_MERGE_IN_KERNEL_SMALL_PARTIALS split partials
 * (splits x query heads per KV head), where a second launch costs more than the
 * last workgroup's merge. */
#define IAK_MERGE_IN_KERNEL_MIN_WORKGROUPS 1024
#define IAK_MERGE_IN_KERNEL_SMALL_WORKGROUPS 128
#define IAK_MERGE_IN_KERNEL_SMALL_PARTIALS 256

typedef enum {
  IAK_OK = 0,
  IAK_EINVAL = 1,   /* bad argument (shape, dtype, pointer, size): Python maps it to ValueError */
  IAK_ENOTSUP = 2,  /* valid but unsupported configuration (e.g. head_dim): ValueError          */
  IAK_EHIP = 3      /* HIP runtime error (launch, device): RuntimeError                         */
} iak_status;

/* Native page precision tags: the reference's fused numbering
 * (FusedKVPrecision, fused_selected_quant_decode.py:29-34) with the native
 * precisions appended. */
enum {
  IAK_TAG_FP16 = 0,
  IAK_TAG_INT8 = 1,
  IAK_TAG_SKIP = 2,
  IAK_TAG_FP8 = 3,           /* OCP e4m3fn codes, one scale per page            */
  IAK_TAG_INT4 = 4,          /* two codes per byte, one scale per page x group   */
  IAK_TAG_INT4_RESIDUAL = 5  /* base | residual<<4 per byte, two scales per page */
};

enum { IAK_DTYPE_F16 = 0, IAK_DTYPE_F32 = 1, IAK_DTYPE_BF16 = 2 };

/*
 * Arguments of one decode step. Pools are indexed by physical page id and
 * laid out [num_pages, page_size, head_dim] (contiguous), as the reference's
 * k_pages_fp16 / k_pages_int8 (fused_selected_quant_decode.py:427-433). A page
 * holds one KV head of page_size tokens.
 *
 *   q            [batch, num_q_heads, head_dim], element strides q_stride_b / q_stride_h
 *   out          [batch, num_q_heads, head_dim], element strides out_stride_b / out_stride_h
 *   page_table   [batch, num_kv_heads, table_width] int32 (contiguous); row (b, h) lists the
 *                physical pages attended by KV head h of sequence b; query heads
 *                h*G .. h*G+G-1 (G = num_q_heads / num_kv_heads) share it.
 *   page_counts  [batch, num_kv_heads] int32; entries are clamped to [0, table_width].
 *   page_tags    [num_pages] int32 caller tags, translated by tag_map[tag] to a native tag;
 *                map entries outside the enum contribute nothing.
 *   map_other_tags  0: caller tags outside [0, 8) contribute nothing (the fused
 *                reference's `else: continue`, fused_selected_quant_decode.py:316-317);
 *                1: they take tag_map[7] (the sibling API reads every tag but FP16
 *                and SKIP through its INT8 pool, triton_intent_quant_attention.py:281-307).
 *   negative_ids 0: an id < 0 is an invalid page (contributes nothing);
 *                1: an id in [-num_pages, 0) means id + num_pages (torch indexing).
 *                Ids outside the pool always contribute nothing.
 *
 *   FP16 pages: k_fp16/v_fp16 f16.
 *   FP8 pages:  k_fp8/v_fp8 e4m3fn bytes; k_fp8_scale/v_fp8_scale [num_pages] (scale_dtype).
 *   INT8 pages: k_int8/v_int8 int8; k_int8_scale/v_int8_scale [num_pages] (scale_dtype).
 *   INT4 pages: k_int4/v_int4 [num_pages, page_size, head_dim/2] bytes, element 2j in the
 *               low nibble of byte j, each nibble = code + 8 (codes in [-7, 7]);
 *               k_int4_scale/v_int4_scale [num_pages, head_dim/int4_group] (scale_dtype).
 *   INT4_RESIDUAL pages: k_int4r/v_int4r [num_pages, page_size, head_dim] bytes,
 *               (base code + 8) | (residual code + 8) << 4; k_int4r_scale/v_int4r_scale
 *               [num_pages, 2] f32 (base scale, residual scale).
 *   Dequantised value = code * scale (INT4_RESIDUAL: base*s0 + residual*s1).
 *
 *   sm_scale     softmax scale (the reference uses 1/sqrt(head_dim), :323).
 *   pages_per_split  pages one wave reduces before the cross-split merge; 0 = automatic.
 *   valid_tokens [batch, num_kv_heads] int32 or NULL: token t of table entry e of row
 *                (b, h) exists only if e * page_size + t < valid_tokens[b, h] (a ragged
 *                last page); entries wholly past the bound contribute nothing. The page
 *                memory of tokens past the bound is still read and must hold finite values.
 *   merge_in_kernel  0: a merge kernel combines the split partials after the decode kernel.
 *                1: the decode kernel merges them itself. 2: automatic -- in-kernel for grids
 *                of at least IAK_MERGE_IN_KERNEL_MIN_WORKGROUPS workgroups (where the merges
 *                overlap other workgroups' page streaming) and for the small grids named
 *                beside that constant (one launch instead of two), else the merge kernel. In-kernel,
 *                the four waves of a workgroup
 *                reduce four consecutive splits of one row (the split count is rounded up
 *                to a multiple of four) and combine them in LDS into one partial; the
 *                workgroup that arrives last at the row's arrival counter merges the row's
 *                partials into the output. The counters live at the end of the workspace,
 *                after the partials, so their offset depends on the plan: they must be zero
 *                before a workspace's first use and again whenever a call with another plan
 *                (shape or split count) reuses it; every call leaves its own counters zero
 *                (iak_paged_decode_noalloc ignores this field).
 *   page_desc    NULL, or [num_pages] 32-byte page descriptors (32-byte aligned) written by
 *                iak_pack_page_descriptors: the page's native tag and scales in one line, read
 *                instead of page_tags, tag_map and the scale arrays (which may then be NULL;
 *                a tag whose K/V pools are NULL contributes nothing). Word 0: native tag;
 *                words 1-3: 0; words 4-7: FP8 / INT8 K and V scale (f32), INT4 K group scales
 *                (4 x f16) then V, INT4_RESIDUAL K base, K residual, V base, V residual (f32).
 *                INT4 scales are per quarter of head_dim: quarter q holds the scale of group
 *                q * head_dim / 4 / int4_group.
 *   entry_records NULL, or [batch, num_kv_heads, table_width] 32-byte records (32-byte
 *                aligned) written by iak_pack_entry_records: per table entry the page's native
 *                tag (word 0), its page id (word 1; -1 when the table's id is out of range,
 *                negative ids already wrapped when negative_ids was set at packing), words
 *                2-3: 0, words 4-7 the scales as in page_desc. Read instead of page_table,
 *                page_tags, tag_map, the scale arrays and page_desc (all may then be NULL;
 *                negative_ids is ignored; a tag whose K/V pools are NULL contributes
 *                nothing); page_counts and valid_tokens still apply.
 */
typedef struct {
  int32_t batch, num_q_heads, num_kv_heads, head_dim, page_size, table_width;
  int64_t num_pages;

  const void* q; int32_t q_dtype; int64_t q_stride_b, q_stride_h;
  void* out; int32_t out_dtype; int64_t out_stride_b, out_stride_h;

  const int32_t* page_table;
  const int32_t* page_counts;
  const int32_t* page_tags;
  uint8_t tag_map[8];
  int32_t negative_ids;

  const void* k_fp16; const void* v_fp16;
  const void* k_fp8;  const void* v_fp8;
  const void* k_int8; const void* v_int8;
  const void* k_int4; const void* v_int4;
  const void* k_int4r; const void* v_int4r;

  const void* k_fp8_scale;  const void* v_fp8_scale;  int32_t fp8_scale_dtype;
  const void* k_int8_scale; const void* v_int8_scale; int32_t int8_scale_dtype;
  const void* k_int4_scale; const void* v_int4_scale; int32_t int4_scale_dtype; int32_t int4_group;
  const float* k_int4r_scale; const float* v_int4r_scale;

  float sm_scale;
  int32_t pages_per_split;
  int32_t map_other_tags;
  const int32_t* valid_tokens;
  int32_t merge_in_kernel;
  const void* page_desc;
  const void* entry_records;
} iak_paged_decode_args;

/* ABI version of the loaded library (IAK_ABI_VERSION). */
int iak_abi_version(void);

/* Static description of a status code. */
const char* iak_status_string(iak_status status);

/* Detail of the last non-OK status returned on the calling thread. */
const char* iak_last_error(void);

/* Bytes of device workspace iak_paged_decode needs for these arguments
 * (0 when the whole reduction fits one split). */
iak_status iak_paged_decode_workspace(const iak_paged_decode_args* args, size_t* bytes);

/* The split plan iak_paged_decode uses for these arguments. No counterpart in
 * the reference (its Triton kernel has one program per (batch, head)). */
typedef struct {
  int32_t splits;            /* splits per (batch, kv head) row (1: no merge) */
  int32_t pages_per_split;   /* table entries per split (of the first tier) */
  int32_t merge_in_kernel;   /* 1: the decode kernel merges the splits itself */
  size_t workspace_bytes;    /* = iak_paged_decode_workspace */
  int32_t tail_splits;       /* of `splits`, those of the second tier (0: one tier): the
                                last entries of each row in short splits launched after
                                every row's first tier (automatic plans on large grids) */
  int32_t tail_pages_per_split;   /* table entries per second-tier split (0: one tier) */
} iak_paged_decode_plan_info;
iak_status iak_paged_decode_plan(const iak_paged_decode_args* args, iak_paged_decode_plan_info* info);

/* Page descriptors for `page_desc` (layout above) from the arguments' page_tags,
 * tag_map, map_other_tags and scale arrays, for every one of num_pages pages:
 * the native tag a decode with these arguments would use, and the scales it
 * would load. `page_desc` (32-byte aligned, num_pages x 32 B) is written; the
 * arguments' own page_desc field is ignored. No counterpart in the reference:
 * a layout in which a page's metadata costs one cache line instead of up to
 * three. Async on `stream`. */
iak_status iak_pack_page_descriptors(const iak_paged_decode_args* args, void* page_desc, void* stream);

/* Entry records for `entry_records` (layout above) from the arguments' page_table,
 * negative_ids, page_tags, tag_map, map_other_tags and scale arrays, for all
 * batch x num_kv_heads x table_width entries: the page id, native tag and scales a
 * decode with these arguments would use for each entry. `records` (32-byte aligned,
 * that many x 32 B) is written; the arguments' page_desc and entry_records fields
 * are ignored. No counterpart in the reference: run once per routing decision
 * (after iak_build_page_tables), it turns each split's metadata into one
 * contiguous stream. Async on `stream`. */
iak_status iak_pack_entry_records(const iak_paged_decode_args* args, void* records, void* stream);

/* Selected-page mixed-precision decode attention, split-K over pages with an
 * LSE merge. `workspace` must hold iak_paged_decode_workspace() bytes (may be
 * NULL when that is 0). `stream` is a hipStream_t (NULL = default stream). */
iak_status iak_paged_decode(const iak_paged_decode_args* args, void* workspace,
                            size_t workspace_bytes, void* stream);

/* iak_paged_decode with two hipEvent_t (either may be NULL) recorded on `stream`
 * immediately before and after the split kernel's launch, so a caller can time
 * that kernel apart from the merge. No counterpart in the reference: it is the
 * measurement hook of bench.py's roofline figure. */
iak_status iak_paged_decode_timed(const iak_paged_decode_args* args, void* workspace,
                                  size_t workspace_bytes, void* stream, void* ev_begin, void* ev_end);

/* Maximum split-K partial bytes iak_paged_decode_noalloc serves from its
 * library-owned scratch (what iak_paged_decode_workspace reports for the same
 * arguments). */
#define IAK_NOALLOC_SCRATCH_BYTES (16u << 20)

/* iak_paged_decode without a caller workspace and without any allocation: the
 * split-K partials live in a library-owned device array of
 * IAK_NOALLOC_SCRATCH_BYTES (one per GPU, held until the process ends). It
 * runs the merge kernel on a one-tier split plan (tail_splits = 0), whose
 * partials are at most those of iak_paged_decode_workspace with
 * merge_in_kernel = 0. Arguments whose partials need more return IAK_EINVAL. Every call on a GPU
 * shares that GPU's array, so calls that overlap on one GPU (concurrent
 * streams or threads) race; calls ordered on one stream do not. No
 * counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). */
iak_status iak_paged_decode_noalloc(const iak_paged_decode_args* args, void* stream);

/*
 * MLA latent decode: every query head attends to one shared compressed KV
 * (latent rows of qk_dim values; dims v_offset .. v_offset + v_dim - 1 of a
 * row are also its values). Per sequence b and head h:
 *   s_t = sm_scale * q[b,h,:] . C_t   over the latent rows C_t of the pages
 *         page_table[b, 0 .. page_counts[b]-1] (SKIP pages contribute nothing)
 *   out[b,h,:] = sum_t softmax(s)_t * C_t[v_offset : v_offset + v_dim]   (0 when nothing is visited)
 * Latent pools are [num_pages, page_size, qk_dim]: FP16 values, or FP8-e4m3 / INT8
 * codes with one scale per page (dequantised value = code * scale). Page tags go
 * through tag_map as in iak_paged_decode; INT4 tags are not supported here.
 * Computed with f16 MFMA operands (q rounded to f16) and f32 accumulation.
 * Supported (qk_dim, v_dim): (64,64) (128,128) (256,256) (512,512) (576,512) (576,64).
 */
typedef struct {
  int32_t batch, num_heads, qk_dim, v_dim, v_offset, page_size, table_width;
  int64_t num_pages;

  const void* q; int32_t q_dtype; int64_t q_stride_b, q_stride_h;
  void* out; int32_t out_dtype; int64_t out_stride_b, out_stride_h;

  const int32_t* page_table;   /* [batch, table_width] */
  const int32_t* page_counts;  /* [batch] */
  const int32_t* page_tags;    /* [num_pages]; NULL = every page FP16 */
  uint8_t tag_map[8];
  int32_t negative_ids;
  const int32_t* valid_tokens; /* [batch] or NULL: token t of table entry e exists only if
                                  e * page_size + t < valid_tokens[b] (a ragged last page) */

  const void* c_fp16;          /* [num_pages, page_size, qk_dim] f16 */
  const void* c_fp8;           /* e4m3fn codes */
  const void* c_int8;          /* int8 codes */
  const void* c_fp8_scale; const void* c_int8_scale; int32_t scale_dtype;   /* [num_pages] */

  float sm_scale;
  int32_t pages_per_split;     /* 0 = automatic, else 1 .. 128 */
} iak_mla_decode_args;

/* Bytes of device workspace iak_mla_decode needs (0 when one split covers a sequence). */
iak_status iak_mla_decode_workspace(const iak_mla_decode_args* args, size_t* bytes);

/* MLA latent decode on MFMA, split-K over pages with an LSE merge; async on `stream`. */
iak_status iak_mla_decode(const iak_mla_decode_args* args, void* workspace, size_t workspace_bytes,
                          void* stream);

/* iak_mla_decode with events around the split kernel, as iak_paged_decode_timed
 * (no counterpart in the reference). */
iak_status iak_mla_decode_timed(const iak_mla_decode_args* args, void* workspace, size_t workspace_bytes,
                                void* stream, void* ev_begin, void* ev_end);

/* Timing events for the _timed entry points and for a harness's own brackets (no
 * counterpart in the reference; bench.py's per-launch figures). They are hipEvent_t
 * handles created with hipEventDisableSystemFence: recording one does not write back
 * and invalidate the caches, whose cost a default event adds to the interval it
 * closes after a kernel that wrote many MB (the MLA split kernel's partials). They
 * order nothing for the host: read them with iak_timing_event_elapsed (milliseconds
 * from `start` to `end`) only after a device synchronize. */
iak_status iak_timing_event_create(void** event);
iak_status iak_timing_event_record(void* event, void* stream);
iak_status iak_timing_event_elapsed(void* start, void* end, float* ms);
iak_status iak_timing_event_destroy(void* event);

/*
 * Quantise-on-write: float16 pages [num_pages, page_size, head_dim] -> codes and
 * scales of one pool, page p written to pool page dst_pages[p] (or p when
 * dst_pages is NULL); pages whose destination lies outside [0, pool_pages)
 * are not written. Layouts are those of iak_paged_decode_args.
 *   mode IAK_QUANT_FAKE_QUANTIZE: fake_quantize_tensor (intent_quant.py:221-312) at the
 *        page granule (INT4: page x int4_group channels); precision FP8, INT8, INT4 or
 *        INT4_RESIDUAL; arithmetic in float16 (INT4_RESIDUAL residual in float32).
 *   mode IAK_QUANT_FUSED_INT8:  fake_int8_pages_from_fp16, fused_selected_quant_decode.py:521-542
 *        (float16; clamp(round(x/s), -128, 127)); precision INT8.
 *   mode IAK_QUANT_TRITON_INT8: fake_int8_pages_from_fp16, triton_intent_quant_attention.py:460-496
 *        (float32; clamp(round(x/s), -127, 127)); precision INT8.
 * scale_dtype: F16 or F32 for one scale per page or group; INT4_RESIDUAL writes
 * [pool_pages, 2] f32 (base, residual) pairs.
 */
enum { IAK_QUANT_FAKE_QUANTIZE = 0, IAK_QUANT_FUSED_INT8 = 1, IAK_QUANT_TRITON_INT8 = 2 };

typedef struct {
  int32_t num_pages, page_size, head_dim;
  const void* src;              /* f16 [num_pages, page_size, head_dim] */
  const int32_t* dst_pages;     /* [num_pages] or NULL */
  int64_t pool_pages;
  int32_t precision;            /* IAK_TAG_FP8 / INT8 / INT4 / INT4_RESIDUAL */
  int32_t mode;
  int32_t int4_group;
  void* codes;                  /* pool codes (INT4: head_dim/2 bytes per token) */
  void* scales;                 /* pool scales */
  int32_t scale_dtype;
} iak_quantize_args;

/* Quantise pages into a pool; async on `stream`. */
iak_status iak_quantize_pages(const iak_quantize_args* args, void* stream);

/*
 * Page tables from routed spans (the selected blocks of a routing decision,
 * in routed order), built on the device.
 *
 * Row r (of num_rows = batch * kv_heads; row b * kv_heads + h) reads span list
 * r / rows_per_list and block-table row r / rows_per_seq. Its logical pages
 * are t / page_size for the tokens start <= t < end of each span, span by
 * span, each page once at its first occurrence (dedupe = 1,
 * block_router.py:283-296) or once per span (dedupe = 0). A logical page l
 * maps to block_table[seq * block_table_width + l] (l >= block_table_width or
 * a negative entry: not resident) or to l without a block table; pages whose
 * physical id is outside [0, num_pages) are dropped. Outputs:
 *   page_table [num_rows, table_width]: the first table_width ids, zeros after;
 *   page_counts [num_rows]: min(ids, table_width);
 *   page_precision [num_pages] (optional): the tag of the span that emitted the
 *     page in the lowest row emitting it (the smallest tag if that row emits it
 *     twice), default_tag elsewhere; pages past table_width count.
 * With one list for all rows, no block table and dedupe = 1 the three outputs
 * equal metadata_to_kernel_tensors(routing_to_kernel_metadata(blocks,
 * page_size), num_pages, B, H) whenever every selected page is below
 * num_pages (the reference raises IndexError otherwise).
 * span_offsets has ceil(num_rows / rows_per_list) + 1 entries (CSR into the
 * span arrays); span_tag holds IAK_TAG_* values. Every array is int32 and must
 * be 4-byte aligned (IAK_EINVAL otherwise). Work is proportional to the
 * pages the lists name; a list whose pages span more than 16384 ids tests
 * first occurrence against its earlier spans (quadratic in spans).
 */
typedef struct {
  int32_t num_rows, rows_per_seq, rows_per_list;
  int32_t table_width, page_size, num_pages;
  int32_t dedupe;
  int32_t default_tag;
  int32_t block_table_width;
  const int32_t* span_offsets;
  const int32_t* span_begin;
  const int32_t* span_end;
  const int32_t* span_tag;
  const int32_t* block_table;   /* [num_seqs, block_table_width] or NULL */
  int32_t* page_table;
  int32_t* page_counts;
  int32_t* page_precision;      /* or NULL */
} iak_page_table_args;

/* Build page tables; async on `stream`. */
iak_status iak_build_page_tables(const iak_page_table_args* args, void* stream);

/*
 * KV memory manager page transcoding with the manager's arithmetic
 * (kv_memory_manager.py): pages of page_elems values (page_size x head_dim,
 * a multiple of 8) in two pools indexed by slot, fp16 [pool_pages,
 * page_elems] and int8 [pool_pages, page_elems], with one float32 scale per
 * slot. Page p is slot pages[p] (or p when pages is NULL); slots outside
 * [0, pool_pages) are skipped.
 *   IAK_TRANSCODE_DEMOTE_INT8: fp16 -> int8 codes and scales:
 *       scale = max|x| / 127 (1.0 for an all-zero page or one holding a NaN),
 *       code = clamp(round(float16(x / scale)), -128, 127) (round half to even);
 *   IAK_TRANSCODE_PROMOTE_FP16: int8 codes and scales -> fp16: float16(code * scale).
 * The float32 scale is what the reference's float arithmetic uses of its
 * Python float scale, so both directions are bit-exact to it. The fp16 pool
 * must be 16-byte aligned, the int8 pool 8-byte aligned. A slot listed twice
 * in one call is transcoded twice, concurrently (the result of a race).
 */
enum { IAK_TRANSCODE_DEMOTE_INT8 = 0, IAK_TRANSCODE_PROMOTE_FP16 = 1 };

typedef struct {
  int32_t num_pages;
  int32_t page_elems;
  int32_t mode;
  const int32_t* pages;         /* [num_pages] slots, or NULL */
  int64_t pool_pages;
  void* fp16;                   /* float16 [pool_pages, page_elems] */
  void* int8;                   /* int8 [pool_pages, page_elems] */
  float* scales;                /* float32 [pool_pages] */
} iak_transcode_args;

/* Transcode pages between the FP16 and INT8 pools; async on `stream`. */
iak_status iak_transcode_pages(const iak_transcode_args* args, void* stream);

/*
 * Page warm-up: reads the K and V rows of pages page_ids[0 .. num_ids-1]
 * (pages of page_size tokens; tokens at or past kv_len skipped) of every
 * (batch, head) of k, v [batch, heads, kv_len, head_dim] (16-bit elements,
 * element strides, unit last stride) with cached loads, so a following decode
 * finds them in the L2 / Infinity Cache. Correctness-neutral. The words read
 * are folded into checksum [batch * heads * num_ids * 4] (one per wave:
 * element i of a page enters as value << (16 (i & 1)), XOR-folded).
 */
typedef struct {
  int32_t batch, heads, kv_len, head_dim, page_size, num_ids;
  const int32_t* page_ids;
  const void* k; const void* v;
  int64_t k_stride_b, k_stride_h, k_stride_t;
  int64_t v_stride_b, v_stride_h, v_stride_t;
  uint32_t* checksum;
} iak_prefetch_args;

/* Warm pages into the caches; async on `stream`. */
iak_status iak_prefetch_pages(const iak_prefetch_args* args, void* stream);

/* Latent context of the reference's MLA decode API (mla_decode_triton,
 * triton_mla_decode.py:47-107 / _mla_decode_cpu :155-186), in float32: for each
 * (batch, query position) row, softmax((q . c) * sm_scale) over the latent rows
 * of the listed pages, context = sum(p c) / sum(p), zeros when nothing is
 * visited. Page p is rows p * page_size .. (p + 1) * page_size - 1 of the
 * latents (the last page may be shorter); ids outside [0, ceil(num_rows /
 * page_size)) are rejected by the caller's contract and skipped by the kernel.
 *
 *   q        [batch, q_len, latent_dim] (q_dtype), element strides q_stride_b / q_stride_t
 *   latents  [num_rows, latent_dim] (latent_dtype), element row stride latent_stride
 *   page_ids [num_selected] int32, shared by every row
 *   context  [batch, q_len, latent_dim] float32, contiguous (written)
 *   latent_dim <= 1024; any page_size >= 1; num_selected * page_size <= INT32_MAX - 4096.
 * workspace (may be NULL): with it, a call with fewer than 512 rows and at least
 * 256 listed latent rows splits each row's keys over several workgroups and
 * merges their partials in a second kernel; it must then hold
 * iak_mla_decode_rows_workspace() bytes (16-byte aligned; 0 bytes: not split).
 * Without it every row runs in one workgroup. The results agree to float32
 * rounding of the summation order. Calls that share a workspace on different
 * streams race. */
typedef struct {
  int32_t batch, q_len, latent_dim, page_size, num_selected;
  int64_t num_rows;
  const void* q; int32_t q_dtype; int64_t q_stride_b, q_stride_t;
  const void* latents; int32_t latent_dtype; int64_t latent_stride;
  const int32_t* page_ids;
  float* context;
  float sm_scale;
} iak_mla_rows_args;

/* Bytes of device workspace that lets iak_mla_decode_rows split these rows (0: no split). */
iak_status iak_mla_decode_rows_workspace(const iak_mla_rows_args* args, size_t* bytes);

iak_status iak_mla_decode_rows(const iak_mla_rows_args* args, void* workspace, size_t workspace_bytes,
                               void* stream);

/* Dense softmax attention of the reference's dense_attention() (reference.py:16-45)
 * in float32: for each (batch, query) row i,
 *   s_j = (q_i . k_j) * sm_scale
 *         + (-inf if causal == IAK_CAUSAL_TRIU and j > i)
 *   s_j = -inf if causal == IAK_CAUSAL_POSITIONS and i < kv_positions[j]
 *   s_j += mask[b, i, j]                       (bool masks add 1.0 where true)
 *   out_i = softmax(s) . v
 * NaN when every s_j is -inf (torch's softmax), zeros when kv_len == 0.
 *
 *   q    [batch, q_len, head_dim], k [batch, kv_len, head_dim], v [batch, kv_len, v_dim],
 *   out  [batch, q_len, v_dim]: one dtype (IAK_DTYPE_*), element strides per batch and row,
 *        unit inner stride; a batch stride of 0 broadcasts
 *   mask (may be NULL) element (b, i, j) at b * mask_stride_b + i * mask_stride_q + j * mask_stride_k,
 *        mask_dtype IAK_DTYPE_* or IAK_MASK_BOOL (one byte)
 *   kv_positions [kv_len] int64 (IAK_CAUSAL_POSITIONS only)
 *   head_dim, v_dim <= 1024; kv_len <= INT32_MAX - 4096.
 * workspace (may be NULL): with it, a call with few rows and many keys splits
 * each row's keys over several workgroups and merges their partials in a
 * second kernel; it must then hold iak_dense_attention_workspace() bytes
 * (16-byte aligned; 0 bytes means the shape is not split and the workspace is
 * unused). Without it every row runs in one workgroup. The results agree to
 * float32 rounding of the summation order. Calls that share a workspace on
 * different streams race. */
enum { IAK_MASK_BOOL = 3 };
enum { IAK_CAUSAL_NONE = 0, IAK_CAUSAL_TRIU = 1, IAK_CAUSAL_POSITIONS = 2 };
typedef struct {
  int32_t batch, q_len, kv_len, head_dim, v_dim, dtype;
  const void* q; int64_t q_stride_b, q_stride_t;
  const void* k; int64_t k_stride_b, k_stride_t;
  const void* v; int64_t v_stride_b, v_stride_t;
  void* out; int64_t out_stride_b, out_stride_t;
  const void* mask; int32_t mask_dtype; int64_t mask_stride_b, mask_stride_q, mask_stride_k;
  int32_t causal;
  const int64_t* kv_positions;
  float sm_scale;
} iak_dense_attention_args;

/* Bytes of device workspace that lets iak_dense_attention split these rows (0: no split). */
iak_status iak_dense_attention_workspace(const iak_dense_attention_args* args, size_t* bytes);

iak_status iak_dense_attention(const iak_dense_attention_args* args, void* workspace, size_t workspace_bytes,
                               void* stream);

/* Fake-quant reconstruction of the selected blocks of float32 K and V, as
 * intent_quant_attention_reference() concatenates them (intent_quant_attention.py:56-84,
 * fake_quantize_tensor intent_quant.py:221-312): block i's tokens blocks[i][0] ..
 * blocks[i][0] + blocks[i][1] - 1 of K and V, reconstructed at precision blocks[i][3]
 * (IAK_FQ_*) with one scale per channel (absmax over every leading row and token of
 * the block), land at tokens blocks[i][2] .. of out, K's channels first, then V's.
 *   k [lead, T, k_dim], v [lead, T, v_dim] float32, element strides per leading row and
 *     token, unit channel stride; k_dim + v_dim <= 2^20
 *   blocks [num_blocks][4] int32 on the device (num_blocks < 2^22); the caller keeps the token ranges inside
 *     K, V and out (the kernel does not check them)
 *   out [lead, total, k_dim + v_dim] float32, element strides per leading row and token
 *   max_block_tokens: the longest block's token count, or an upper bound on it (it sizes
 *     the split below; a wrong value changes the speed, never the result)
 * Every division is the IEEE float32 quotient and every code rounds to nearest even,
 * as torch's float32 arithmetic, so the result equals the reference's bit for bit
 * (an integer code of zero gives +0, as .to(int8).float() does).
 * Without a workspace one workgroup takes each (block, 64 channels); with one of the
 * size iak_fake_quant_blocks_workspace() gives (0: no split for these arguments), a
 * block of many rows (leading rows x tokens) is split over several workgroups per
 * channel group, whose per-channel maxima meet in the workspace over three launches. */
enum { IAK_FQ_FP16 = 0, IAK_FQ_FP8 = 1, IAK_FQ_INT8 = 2, IAK_FQ_INT4 = 3, IAK_FQ_INT4_RESIDUAL = 4, IAK_FQ_SKIP = 5 };
typedef struct {
  int32_t lead, num_blocks, k_dim, v_dim;
  const float* k; int64_t k_stride_l, k_stride_t;
  const float* v; int64_t v_stride_l, v_stride_t;
  const int32_t* blocks;
  int32_t max_block_tokens;
  float* out; int64_t out_stride_l, out_stride_t;
} iak_fake_quant_blocks_args;

/* Bytes of device workspace that lets iak_fake_quant_blocks split long blocks (0: no split). */
iak_status iak_fake_quant_blocks_workspace(const iak_fake_quant_blocks_args* args, size_t* bytes);

iak_status iak_fake_quant_blocks(const iak_fake_quant_blocks_args* args, void* workspace, size_t workspace_bytes,
                                 void* stream);

#ifdef __cplusplus
}
#endif

#endif /* IAK_H */
