// Host AddressSanitizer run over libiak's C-ABI argument validation.
//
// Linked with iak_api.hip compiled with host-side ASan (the device code is not
// instrumented) and the library's other objects. Every call here is rejected
// by validation before any launch, or is a pure host query (workspace sizes,
// split plans, status strings), so it needs no GPU: the point is that the
// validation code reads only inside its arguments and its own tables for any
// field values -- random bytes included -- and reports an error instead.
//
// Prints "abi-asan: N calls, M rejected" and exits 0; an ASan report aborts.

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <cstdlib>
#include <random>

#include "iak.h"

namespace {

std::mt19937_64 rng(20261202);

template <typename T> void random_bytes(T& s) {
  unsigned char* p = reinterpret_cast<unsigned char*>(&s);
  for (size_t i = 0; i < sizeof(T); ++i) p[i] = static_cast<unsigned char>(rng());
}

// small or edge values for int fields, so that validation gets past its first checks
int32_t pick_int() {
  static const int32_t v[] = {-1, 0, 1, 2, 3, 4, 7, 8, 15, 16, 17, 31, 32, 48, 63, 64, 100, 128, 255, 256,
                              511, 512, 576, 1024, 1025, 65535, 65536, 0x7FFFFFFF, (int32_t)0x80000000};
  return v[rng() % (sizeof(v) / sizeof(v[0]))];
}

int calls = 0, rejected = 0;
void count(iak_status st) {
  ++calls;
  if (st != IAK_OK) ++rejected;
  (void)iak_last_error();
  (void)iak_status_string(st);
}

void fuzz_paged_decode(int n) {
  for (int i = 0; i < n; ++i) {
    iak_paged_decode_args a;
    random_bytes(a);
    if (rng() % 2) {
      a.batch = pick_int(); a.num_q_heads = pick_int(); a.num_kv_heads = pick_int();
      a.head_dim = pick_int(); a.page_size = pick_int(); a.table_width = pick_int();
      a.num_pages = pick_int(); a.pages_per_split = pick_int();
      a.q_dtype = pick_int() & 3; a.out_dtype = pick_int() & 3;
      a.int4_group = pick_int(); a.merge_in_kernel = pick_int() & 3;
    }
    size_t bytes = 0;
    count(iak_paged_decode_workspace(&a, &bytes));
    iak_paged_decode_plan_info info;
    count(iak_paged_decode_plan(&a, &info));
    // a NULL or misaligned destination is rejected before any launch
    count(iak_pack_page_descriptors(&a, nullptr, nullptr));
    count(iak_pack_page_descriptors(&a, reinterpret_cast<void*>(0x100010), nullptr));
    count(iak_pack_entry_records(&a, nullptr, nullptr));
    count(iak_pack_entry_records(&a, reinterpret_cast<void*>(0x100010), nullptr));
  }
  count(iak_paged_decode_workspace(nullptr, nullptr));
  count(iak_pack_page_descriptors(nullptr, nullptr, nullptr));
  count(iak_pack_entry_records(nullptr, nullptr, nullptr));
  count(iak_paged_decode_plan(nullptr, nullptr));
  // well-formed arguments (fake, aligned device addresses; never launched):
  // the plan and workspace sizes are computed for every shape
  for (int i = 0; i < n; ++i) {
    iak_paged_decode_args a{};
    const int G = 1 + (int)(rng() % 16), Hkv = 1 << (rng() % 4);
    a.batch = (int32_t)(rng() % 65); a.num_kv_heads = Hkv; a.num_q_heads = G * Hkv;
    a.head_dim = rng() % 2 ? 64 : 128; a.page_size = 16; a.table_width = (int32_t)(rng() % 5000);
    a.num_pages = 1 + (int64_t)(rng() % 100000);
    void* const fake = reinterpret_cast<void*>(0x100000);
    a.out = fake;
    a.q = a.k_fp16 = a.v_fp16 = fake;
    a.page_table = a.page_counts = a.page_tags = static_cast<const int32_t*>(fake);
    a.q_stride_b = a.num_q_heads * a.head_dim; a.q_stride_h = a.head_dim;
    a.out_stride_b = a.q_stride_b; a.out_stride_h = a.head_dim;
    for (int t = 0; t < 8; ++t) a.tag_map[t] = t == 0 ? IAK_TAG_FP16 : IAK_TAG_SKIP;
    a.sm_scale = 0.1f;
    a.pages_per_split = (int32_t)(rng() % 65);
    a.merge_in_kernel = (int32_t)(rng() % 3);
    size_t bytes = 0;
    const iak_status s1 = iak_paged_decode_workspace(&a, &bytes);
    iak_paged_decode_plan_info info{};
    const iak_status s2 = iak_paged_decode_plan(&a, &info);
    count(s1);
    count(s2);
    if (s1 != IAK_OK || s2 != IAK_OK || info.workspace_bytes != bytes || info.splits < 1 ||
        (info.merge_in_kernel && info.splits % 4 != 0)) {
      std::printf("abi-asan: inconsistent plan for a well-formed call (B=%d Hkv=%d G=%d W=%d)\n", a.batch, Hkv, G,
                  a.table_width);
      std::exit(1);
    }
  }
}

void fuzz_mla(int n) {
  for (int i = 0; i < n; ++i) {
    iak_mla_decode_args a;
    random_bytes(a);
    if (rng() % 2) {
      a.batch = pick_int(); a.num_heads = pick_int(); a.qk_dim = pick_int(); a.v_dim = pick_int();
      a.v_offset = pick_int(); a.page_size = pick_int(); a.table_width = pick_int(); a.num_pages = pick_int();
      a.q_dtype = pick_int() & 3; a.out_dtype = pick_int() & 3;
    }
    size_t bytes = 0;
    count(iak_mla_decode_workspace(&a, &bytes));
  }
  count(iak_mla_decode_workspace(nullptr, nullptr));
}

// Launching entry points: each case below is invalid (a negative size, a null
// required pointer or an unsupported value), so validation returns first.
void invalid_launches() {
  iak_paged_decode_args d{};
  d.batch = -1;
  count(iak_paged_decode(&d, nullptr, 0, nullptr));
  count(iak_paged_decode_noalloc(&d, nullptr));
  count(iak_paged_decode(nullptr, nullptr, 0, nullptr));
  d.batch = 1; d.num_q_heads = 8; d.num_kv_heads = 2; d.head_dim = 128; d.page_size = 16; d.table_width = 100;
  d.num_pages = 10;   // q, out, tables: null
  count(iak_paged_decode(&d, nullptr, 0, nullptr));

  iak_mla_decode_args m{};
  m.batch = 1; m.num_heads = 128; m.qk_dim = 576; m.v_dim = 512; m.page_size = 16; m.table_width = 4;
  m.num_pages = 4;   // pointers null
  count(iak_mla_decode(&m, nullptr, 0, nullptr));
  m.qk_dim = 100;
  count(iak_mla_decode(&m, nullptr, 0, nullptr));

  iak_quantize_args qa{};
  for (int i = 0; i < 200; ++i) {
    random_bytes(qa);
    qa.num_pages = -1 - (int32_t)(rng() % 5);   // negative: rejected
    count(iak_quantize_pages(&qa, nullptr));
  }
  count(iak_quantize_pages(nullptr, nullptr));

  iak_page_table_args pt;
  for (int i = 0; i < 200; ++i) {
    random_bytes(pt);
    pt.num_rows = 1 + (int32_t)(rng() % 64);
    pt.span_offsets = nullptr;   // required with rows: rejected
    count(iak_build_page_tables(&pt, nullptr));
  }
  count(iak_build_page_tables(nullptr, nullptr));

  iak_transcode_args tc;
  for (int i = 0; i < 200; ++i) {
    random_bytes(tc);
    tc.num_pages = -1;
    count(iak_transcode_pages(&tc, nullptr));
  }
  count(iak_transcode_pages(nullptr, nullptr));

  iak_prefetch_args pf;
  for (int i = 0; i < 200; ++i) {
    random_bytes(pf);
    pf.batch = -1;
    count(iak_prefetch_pages(&pf, nullptr));
  }
  count(iak_prefetch_pages(nullptr, nullptr));

  iak_mla_rows_args r;
  for (int i = 0; i < 200; ++i) {
    random_bytes(r);
    if (rng() % 2) r.latent_dim = 1025 + (int32_t)(rng() % 100);
    else r.page_size = 0;
    if (r.batch > 0 && r.q_len > 0 && r.latent_dim > 0 && r.latent_dim <= 1024 && r.page_size > 0) r.batch = -1;
    count(iak_mla_decode_rows(&r, nullptr, 0, nullptr));
  }
  count(iak_mla_decode_rows(nullptr, nullptr, 0, nullptr));
  // workspace sizes of random shapes (host queries), a split shape with a
  // workspace one byte short, and a key count past the 32-bit limit
  size_t rwb = 0;
  for (int i = 0; i < 2000; ++i) {
    random_bytes(r);
    if (rng() % 2) {
      r.batch = pick_int(); r.q_len = pick_int(); r.latent_dim = pick_int(); r.page_size = pick_int();
      r.num_selected = pick_int(); r.num_rows = pick_int(); r.q_dtype = pick_int() & 3; r.latent_dtype = pick_int() & 3;
    }
    count(iak_mla_decode_rows_workspace(&r, &rwb));
  }
  count(iak_mla_decode_rows_workspace(nullptr, &rwb));
  std::memset(&r, 0, sizeof(r));
  r.batch = 4; r.q_len = 1; r.latent_dim = 576; r.page_size = 64; r.num_selected = 128; r.num_rows = 16384;
  r.latent_stride = 576;
  r.q = r.latents = reinterpret_cast<const void*>(0x1000);
  r.page_ids = reinterpret_cast<const int32_t*>(0x1000);
  r.context = reinterpret_cast<float*>(0x1000);
  count(iak_mla_decode_rows_workspace(&r, nullptr));
  if (iak_mla_decode_rows_workspace(&r, &rwb) != IAK_OK || rwb == 0) {
    std::printf("abi-asan: 4 rows over 8192 latent rows should ask for a split workspace\n");
    std::exit(1);
  }
  if (iak_mla_decode_rows(&r, reinterpret_cast<void*>(0x1000), rwb - 1, nullptr) != IAK_EINVAL) {
    std::printf("abi-asan: a short latent-row workspace was not rejected\n");
    std::exit(1);
  }
  r.page_size = 1 << 20; r.num_selected = 4096;   // 2^32 keys
  if (iak_mla_decode_rows(&r, nullptr, 0, nullptr) != IAK_ENOTSUP) {
    std::printf("abi-asan: num_selected * page_size past INT32_MAX was not rejected\n");
    std::exit(1);
  }

  iak_dense_attention_args da;
  for (int i = 0; i < 300; ++i) {
    random_bytes(da);
    switch (rng() % 4) {   // at least one field invalid, so nothing reaches a launch
      case 0: da.head_dim = 1025 + (int32_t)(rng() % 100); break;
      case 1: da.causal = 3 + (int32_t)(rng() % 50); break;
      case 2: da.dtype = 3 + (int32_t)(rng() % 50); break;
      default: da.q_len = -1 - (int32_t)(rng() % 50); break;
    }
    count(iak_dense_attention(&da, nullptr, 0, nullptr));
  }
  count(iak_dense_attention(nullptr, nullptr, 0, nullptr));

  // workspace sizes of random and of valid shapes (host queries), and a split
  // shape with a workspace one byte short (rejected before the launch)
  size_t wsb = 0;
  for (int i = 0; i < 2000; ++i) {
    random_bytes(da);
    if (rng() % 2) {
      da.batch = pick_int(); da.q_len = pick_int(); da.kv_len = pick_int();
      da.head_dim = pick_int(); da.v_dim = pick_int(); da.dtype = pick_int() & 3;
      da.causal = pick_int() & 3; da.mask = nullptr;
    }
    count(iak_dense_attention_workspace(&da, &wsb));
  }
  count(iak_dense_attention_workspace(nullptr, &wsb));
  std::memset(&da, 0, sizeof(da));
  da.batch = 2; da.q_len = 1; da.kv_len = 8192; da.head_dim = 128; da.v_dim = 128;
  da.q = da.k = da.v = reinterpret_cast<const void*>(0x1000); da.out = reinterpret_cast<void*>(0x1000);
  da.sm_scale = 0.125f;
  count(iak_dense_attention_workspace(&da, nullptr));
  if (iak_dense_attention_workspace(&da, &wsb) != IAK_OK || wsb == 0) {
    std::printf("abi-asan: a 2-row, 8192-key shape should ask for a split workspace\n");
    std::exit(1);
  }
  if (iak_dense_attention(&da, reinterpret_cast<void*>(0x1000), wsb - 1, nullptr) != IAK_EINVAL) {
    std::printf("abi-asan: a short dense workspace was not rejected\n");
    std::exit(1);
  }
  da.kv_len = 0x7FFFFFFF - 64;   // key indexes would pass INT32_MAX: rejected
  if (iak_dense_attention(&da, nullptr, 0, nullptr) != IAK_ENOTSUP) {
    std::printf("abi-asan: a kv_len near INT32_MAX was not rejected\n");
    std::exit(1);
  }
  da.kv_len = 100;
  if (iak_dense_attention_workspace(&da, &wsb) != IAK_OK || wsb != 0) {
    std::printf("abi-asan: a 100-key shape should not be split\n");
    std::exit(1);
  }

  // fake-quant reconstruction: a negative size, a NULL operand, a negative
  // stride or more than 2^20 channels is rejected; empty work returns OK
  // without a launch
  iak_fake_quant_blocks_args fq;
  for (int i = 0; i < 300; ++i) {
    random_bytes(fq);
    switch (rng() % 4) {
      case 0: fq.lead = -1 - (int32_t)(rng() % 50); break;
      case 1: fq.k_dim = (1 << 20) + 1 + (int32_t)(rng() % 50); fq.v_dim = (int32_t)(rng() % 50); break;
      case 2: fq.lead = 1; fq.num_blocks = 1; fq.k_dim = 4; fq.v_dim = 4; fq.blocks = nullptr; break;
      default:
        fq.lead = 1; fq.num_blocks = 1; fq.k_dim = 4; fq.v_dim = 4;
        fq.k = fq.v = reinterpret_cast<const float*>(0x1000); fq.out = reinterpret_cast<float*>(0x1000);
        fq.blocks = reinterpret_cast<const int32_t*>(0x1000); fq.v_stride_t = -1 - (int64_t)(rng() % 50);
        break;
    }
    count(iak_fake_quant_blocks(&fq, nullptr, 0, nullptr));
  }
  count(iak_fake_quant_blocks(nullptr, nullptr, 0, nullptr));
  std::memset(&fq, 0, sizeof(fq));
  fq.lead = 3; fq.k_dim = 64; fq.v_dim = 64;   // no blocks: nothing to launch
  if (iak_fake_quant_blocks(&fq, nullptr, 0, nullptr) != IAK_OK) {
    std::printf("abi-asan: an empty fake-quant call was not accepted\n");
    std::exit(1);
  }
  // workspace sizes of random and of valid arguments (host queries); a long
  // block asks for a split workspace, and one byte short is rejected
  for (int i = 0; i < 2000; ++i) {
    random_bytes(fq);
    if (rng() % 2) {
      fq.lead = pick_int(); fq.num_blocks = pick_int(); fq.k_dim = pick_int() & 0xFFFF;
      fq.v_dim = pick_int() & 0xFFFF; fq.max_block_tokens = pick_int();
      fq.k = fq.v = reinterpret_cast<const float*>(0x1000); fq.out = reinterpret_cast<float*>(0x1000);
      fq.blocks = reinterpret_cast<const int32_t*>(0x1000);
      fq.k_stride_l = fq.k_stride_t = fq.v_stride_l = fq.v_stride_t = fq.out_stride_l = fq.out_stride_t = 1;
    }
    count(iak_fake_quant_blocks_workspace(&fq, &wsb));
  }
  count(iak_fake_quant_blocks_workspace(nullptr, &wsb));
  std::memset(&fq, 0, sizeof(fq));
  fq.lead = 8; fq.num_blocks = 16; fq.k_dim = 64; fq.v_dim = 64; fq.max_block_tokens = 256;
  fq.k = fq.v = reinterpret_cast<const float*>(0x1000); fq.out = reinterpret_cast<float*>(0x1000);
  fq.blocks = reinterpret_cast<const int32_t*>(0x1000);
  count(iak_fake_quant_blocks_workspace(&fq, nullptr));
  if (iak_fake_quant_blocks_workspace(&fq, &wsb) != IAK_OK || wsb == 0) {
    std::printf("abi-asan: 16 blocks of 8 x 256 rows should ask for a split workspace\n");
    std::exit(1);
  }
  if (iak_fake_quant_blocks(&fq, reinterpret_cast<void*>(0x1000), wsb - 1, nullptr) != IAK_EINVAL) {
    std::printf("abi-asan: a short fake-quant workspace was not rejected\n");
    std::exit(1);
  }
  fq.max_block_tokens = 16;
  if (iak_fake_quant_blocks_workspace(&fq, &wsb) != IAK_OK || wsb != 0) {
    std::printf("abi-asan: blocks of 8 x 16 rows should not be split\n");
    std::exit(1);
  }

  // timing events: NULL handles and outputs are rejected before any HIP call
  float ms = 0.f;
  if (iak_timing_event_create(nullptr) != IAK_EINVAL || iak_timing_event_record(nullptr, nullptr) != IAK_EINVAL ||
      iak_timing_event_elapsed(nullptr, nullptr, &ms) != IAK_EINVAL ||
      iak_timing_event_elapsed(reinterpret_cast<void*>(0x1000), reinterpret_cast<void*>(0x1000), nullptr) !=
          IAK_EINVAL ||
      iak_timing_event_destroy(nullptr) != IAK_OK) {
    std::printf("abi-asan: a NULL timing-event argument was not handled\n");
    std::exit(1);
  }
  calls += 5;
  rejected += 4;
}

}  // namespace

int main() {
  for (int s = -3; s < 12; ++s) (void)iak_status_string(static_cast<iak_status>(s));
  if (iak_abi_version() != IAK_ABI_VERSION) {
    std::printf("abi-asan: ABI version %d != %d\n", iak_abi_version(), IAK_ABI_VERSION);
    return 1;
  }
  fuzz_paged_decode(20000);
  fuzz_mla(20000);
  invalid_launches();
  std::printf("abi-asan: %d calls, %d rejected\n", calls, rejected);
  return 0;
}
