"""The C-ABI library: loads, exports every function include/iak.h declares, and
the ctypes mirror of iak_paged_decode_args matches the C layout (checked by
compiling a small offsetof probe of the header with gcc). No GPU calls."""
import ctypes
import os
import re
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "iak.h")


def _declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(iak_[a-z_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    from intent_attention import _native as N
    lib = N.load()
    declared = _declared_functions()
    assert "iak_paged_decode" in declared and len(declared) >= 5
    for name in declared:
        assert hasattr(lib, name), f"libiak.so does not export {name}"
    assert set(N.EXPORTED) <= set(declared)
    assert lib.iak_abi_version() == N.ABI_VERSION
    assert lib.iak_status_string(0) == b"ok"
    # undeclared argtypes would pass a stream handle as a masked C int
    for name in N.EXPORTED:
        assert getattr(lib, name).argtypes is not None, f"{name} has no ctypes argtypes"


@pytest.mark.parametrize("cname,pyname", [("iak_paged_decode_args", "PagedDecodeArgs"),
                                          ("iak_mla_decode_args", "MlaDecodeArgs"),
                                          ("iak_quantize_args", "QuantizeArgs"),
                                          ("iak_transcode_args", "TranscodeArgs"),
                                          ("iak_prefetch_args", "PrefetchArgs"),
                                          ("iak_page_table_args", "PageTableArgs"),
                                          ("iak_paged_decode_plan_info", "PlanInfo"),
                                          ("iak_mla_rows_args", "MlaRowsArgs")])
def test_ctypes_struct_matches_c_layout(cname, pyname):
    from intent_attention import _native as N
    S = getattr(N, pyname)
    fields = [f[0] for f in S._fields_]
    prog = ['#include <stdio.h>', '#include <stddef.h>', '#include "iak.h"', 'int main(void){',
            f'printf("size %zu\\n", sizeof({cname}));']
    prog += [f'printf("{f} %zu\\n", offsetof({cname}, {f}));' for f in fields]
    prog += ["return 0;}"]
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "probe.c")
        open(c, "w").write("\n".join(prog))
        exe = os.path.join(d, "probe")
        subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "include"), c, "-o", exe], check=True)
        got = dict(line.split() for line in subprocess.run([exe], capture_output=True, text=True,
                                                           check=True).stdout.splitlines())
    assert int(got["size"]) == ctypes.sizeof(S)
    for f in fields:
        assert int(got[f]) == getattr(S, f).offset, f


def test_validation_errors_without_gpu():
    """Argument checks run on the host before any launch."""
    from intent_attention import _native as N
    a = N.PagedDecodeArgs()
    a.batch, a.num_q_heads, a.num_kv_heads, a.head_dim, a.page_size = 1, 8, 2, 96, 16
    with pytest.raises(ValueError, match="head_dim 96"):
        N.workspace_bytes(a)
    a.head_dim = 128
    a.num_q_heads = 7
    with pytest.raises(ValueError, match="multiple"):
        N.workspace_bytes(a)
    a.num_q_heads, a.page_size = 8, 32
    with pytest.raises(ValueError, match="page_size 32"):
        N.workspace_bytes(a)
    a.page_size, a.table_width, a.num_pages = 16, 100, 10
    a.q = a.out = a.page_table = a.page_counts = a.page_tags = 16
    for i in range(8):
        a.tag_map[i] = N.TAG_SKIP
    a.tag_map[3] = N.TAG_FP8     # FP8 reachable but no FP8 pool
    with pytest.raises(ValueError, match="FP8"):
        N.workspace_bytes(a)
    a.tag_map[3] = N.TAG_SKIP
    a.sm_scale = 0.1
    n = N.workspace_bytes(a)     # 2 rows x 100 pages: split into several chunks -> workspace
    assert n > 0 and n % 256 == 0


def test_mla_validation_errors_without_gpu():
    from intent_attention import _native as N
    a = N.MlaDecodeArgs()
    a.batch, a.num_heads, a.qk_dim, a.v_dim, a.page_size = 2, 128, 576, 576, 16
    with pytest.raises(ValueError, match="not supported"):
        N.mla_workspace_bytes(a)
    a.v_dim, a.v_offset = 512, 128
    with pytest.raises(ValueError, match="v_offset"):
        N.mla_workspace_bytes(a)
    a.v_offset, a.page_size = 0, 64
    with pytest.raises(ValueError, match="page_size 64"):
        N.mla_workspace_bytes(a)
    a.page_size, a.table_width, a.num_pages = 16, 512, 1024
    a.q = a.out = a.page_table = a.page_counts = a.page_tags = 16
    for i in range(8):
        a.tag_map[i] = N.TAG_SKIP
    a.tag_map[1] = N.TAG_INT4
    with pytest.raises(ValueError, match="INT4"):
        N.mla_workspace_bytes(a)
    a.tag_map[1] = N.TAG_INT8     # INT8 reachable but no latent pool
    with pytest.raises(ValueError, match="INT8"):
        N.mla_workspace_bytes(a)
    a.tag_map[1] = N.TAG_SKIP
    a.sm_scale = 0.04
    n = N.mla_workspace_bytes(a)  # 2 sequences x 512 pages: 64-page splits -> partials
    assert n > 0 and n % 256 == 0


def test_mla_long_split_plan_without_gpu():
    """MLA splits hold up to 128 table entries (a lane takes entries i and
    i + 64): pages_per_split 128 is accepted, 129 is not, and the automatic plan
    of 32 sequences x 1,300 entries (256 workgroups wanted, 8 per sequence)
    takes 11 splits of 128 -- with one entry per lane it would take 21 of 64.
    Read through the workspace size: (2 + v_dim) floats per (sequence, split,
    head), each array rounded up to 256 bytes."""
    from intent_attention import _native as N
    a = N.MlaDecodeArgs()
    a.batch, a.num_heads, a.qk_dim, a.v_dim, a.page_size = 32, 40, 576, 512, 16
    a.table_width, a.num_pages, a.sm_scale = 1300, 4096, 0.04
    a.q = a.out = a.page_table = a.page_counts = a.page_tags = a.c_fp8 = a.c_fp8_scale = 16
    for i in range(8):
        a.tag_map[i] = N.TAG_SKIP
    a.tag_map[0] = N.TAG_FP8

    def ws(splits):
        r = lambda x: (x + 255) // 256 * 256
        slots = a.batch * splits * a.num_heads
        return 2 * r(4 * slots) + r(4 * slots * a.v_dim)

    assert N.mla_workspace_bytes(a) == ws(11)
    a.pages_per_split = 128
    assert N.mla_workspace_bytes(a) == ws(11)
    a.pages_per_split = 64
    assert N.mla_workspace_bytes(a) == ws(21)
    a.pages_per_split = 129
    with pytest.raises(ValueError, match="outside"):
        N.mla_workspace_bytes(a)


def test_quantize_validation_errors_without_gpu():
    from intent_attention import _native as N
    a = N.QuantizeArgs()
    a.num_pages, a.page_size, a.head_dim, a.pool_pages = 4, 16, 96, 4
    with pytest.raises(ValueError, match="head_dim 96"):
        N.quantize_pages(a, 0)
    a.head_dim, a.precision, a.mode = 128, N.TAG_FP16, N.QUANT_FAKE_QUANTIZE
    with pytest.raises(ValueError, match="cannot be quantised"):
        N.quantize_pages(a, 0)
    a.precision, a.mode = N.TAG_FP8, N.QUANT_FUSED_INT8
    with pytest.raises(ValueError, match="INT8 pages only"):
        N.quantize_pages(a, 0)
    a.precision, a.mode, a.int4_group = N.TAG_INT4, N.QUANT_FAKE_QUANTIZE, 48
    with pytest.raises(ValueError, match="int4_group 48"):
        N.quantize_pages(a, 0)
    a.int4_group, a.scale_dtype = 32, N.DTYPE_F16
    with pytest.raises(ValueError, match="NULL"):
        N.quantize_pages(a, 0)


def test_page_table_validation_errors_without_gpu():
    from intent_attention import _native as N
    a = N.PageTableArgs()
    a.num_rows, a.rows_per_seq, a.rows_per_list, a.table_width, a.page_size, a.num_pages = 4, 0, 4, 8, 16, 10
    with pytest.raises(ValueError, match="rows_per_seq"):
        N.build_page_tables(a, 0)
    a.rows_per_seq, a.page_size = 2, 0
    with pytest.raises(ValueError, match="page_size"):
        N.build_page_tables(a, 0)
    a.page_size, a.default_tag = 16, 7
    with pytest.raises(ValueError, match="default_tag"):
        N.build_page_tables(a, 0)
    a.default_tag, a.block_table = 0, 16
    with pytest.raises(ValueError, match="block_table_width"):
        N.build_page_tables(a, 0)
    a.block_table_width = 4
    with pytest.raises(ValueError, match="span arrays"):
        N.build_page_tables(a, 0)
    a.span_offsets = a.span_begin = a.span_end = a.span_tag = 16
    with pytest.raises(ValueError, match="page_table / page_counts"):
        N.build_page_tables(a, 0)
    a.num_rows, a.page_precision = 1 << 28, 16
    with pytest.raises(ValueError, match="2\\^28"):
        N.build_page_tables(a, 0)
    a.num_rows, a.page_table, a.page_counts, a.page_precision = 4, 32, 64, 18   # precision 2 bytes off
    with pytest.raises(ValueError, match="4-byte aligned"):
        N.build_page_tables(a, 0)


def _decode_args(N, B, Hkv, G, W):
    a = N.PagedDecodeArgs()
    a.batch, a.num_q_heads, a.num_kv_heads, a.head_dim, a.page_size = B, Hkv * G, Hkv, 128, 16
    a.table_width, a.num_pages = W, 1 << 20
    a.q = a.out = a.page_table = a.page_counts = a.page_tags = a.k_fp16 = a.v_fp16 = 16
    for i in range(8):
        a.tag_map[i] = N.TAG_FP16 if i == 0 else N.TAG_SKIP
    a.sm_scale = 0.1
    return a


def test_small_grid_plans_without_gpu():
    """Latency-bound grids: the automatic split length falls to one workgroup
    per CU but not below ceil(W / 64) entries clamped to [2, 8], and grids of
    at most IAK_MERGE_IN_KERNEL_SMALL_WORKGROUPS workgroups whose rows hold at
    most IAK_MERGE_IN_KERNEL_SMALL_PARTIALS partials (splits x query heads per
    KV head) merge inside the decode kernel (one launch); others keep the merge
    kernel."""
    from intent_attention import _native as N
    cases = [  # (B, Hkv, G, W) -> (splits, entries per split, in-kernel merge)
        ((1, 8, 1, 64), (32, 2, True)),      # cfg1's grid: 64 workgroups, 32 partials per row
        ((1, 8, 4, 256), (64, 4, True)),     # 128 workgroups, 256 partials per row
        ((4, 8, 4, 64), (32, 2, False)),     # 256 workgroups
        ((1, 1, 16, 1000), (125, 8, False)),  # 2,000 partials per row; the floor of 8 entries
    ]
    for shape, want in cases:
        a = _decode_args(N, *shape)
        a.merge_in_kernel = 2
        p = N.plan_info(a)
        assert (p["splits"], p["pages_per_split"], p["merge_in_kernel"]) == want, (shape, p)
        assert p["tail_splits"] == 0


def test_split_plan_and_merge_form_without_gpu():
    """merge_in_kernel: 0 keeps the split count and the merge kernel; 1 rounds
    the split count up to whole workgroups of four and sizes one partial per
    workgroup plus one counter per row; 2 picks the in-kernel form only for
    grids of IAK_MERGE_IN_KERNEL_MIN_WORKGROUPS workgroups or more. Automatic
    plans of grids above about 1.5 resident generations of waves take two
    tiers: the first three quarters of each row in full splits, whole fours of
    them, the rest in splits of about 40 entries, evened over a multiple of four
    splits, so both merge forms share the split boundaries."""
    from intent_attention import _native as N
    rows_cfg3, rows_cfg4 = (32, 8, 4, 1638), (4, 8, 4, 1229)
    a = _decode_args(N, *rows_cfg3)
    a.pages_per_split = 63                      # an explicit split length: one tier
    p0 = N.plan_info(a)
    assert (p0["splits"], p0["pages_per_split"], p0["merge_in_kernel"], p0["tail_splits"]) == (26, 63, False, 0)
    a.merge_in_kernel = 1
    p1 = N.plan_info(a)
    assert p1["splits"] == 28 and p1["splits"] % 4 == 0 and p1["merge_in_kernel"]
    assert p1["pages_per_split"] * (p1["splits"] - 4) < 1638 <= p1["pages_per_split"] * p1["splits"]
    rows, G, D = 256, 4, 128
    slots = rows * (p1["splits"] // 4) * G
    r256 = lambda x: (x + 255) // 256 * 256  # noqa: E731
    assert p1["workspace_bytes"] == 2 * r256(4 * slots) + r256(4 * slots * D) + r256(4 * rows)
    assert p1["workspace_bytes"] == N.workspace_bytes(a)
    # the automatic plan of the same grid: two tiers, the same for both merge forms
    a.pages_per_split = 0
    tiers = []
    for m in (0, 1, 2):
        a.merge_in_kernel = m
        p = N.plan_info(a)
        first = p["splits"] - p["tail_splits"]
        tb = p["tail_pages_per_split"]
        assert p["pages_per_split"] == 63 and 0 < tb <= 40
        assert first % 4 == 0 and p["tail_splits"] % 4 == 0
        assert first * 63 <= 1638 * 3 // 4 and (first + 4) * 63 > 1638 * 3 // 4
        assert first * 63 + (p["tail_splits"] - 1) * tb < 1638 <= first * 63 + p["tail_splits"] * tb
        assert p["workspace_bytes"] == N.workspace_bytes(a)
        tiers.append((p["splits"], p["tail_splits"], p["merge_in_kernel"]))
    assert tiers == [(32, 16, False), (32, 16, True), (32, 16, True)]
    assert p["tail_pages_per_split"] == 40
    b = _decode_args(N, *rows_cfg4)
    b.merge_in_kernel = 2                       # 32 rows x 8 workgroups: the merge kernel, one tier
    p4 = N.plan_info(b)
    assert not p4["merge_in_kernel"] and p4["splits"] == 32 and p4["tail_splits"] == 0
    b.merge_in_kernel = 3
    with pytest.raises(ValueError, match="merge_in_kernel 3"):
        N.plan_info(b)
    c = _decode_args(N, 1, 2, 4, 40)            # one split per row: no merge, no workspace
    c.merge_in_kernel, c.pages_per_split = 1, 64
    pc = N.plan_info(c)
    assert pc["splits"] == 1 and not pc["merge_in_kernel"] and pc["workspace_bytes"] == 0


def test_mla_rows_validation_errors_without_gpu():
    from intent_attention import _native as N
    a = N.MlaRowsArgs()
    a.batch, a.q_len, a.latent_dim, a.page_size, a.num_selected, a.num_rows = 1, 1, 1025, 16, 1, 64
    with pytest.raises(ValueError, match="latent_dim 1025"):
        N.mla_decode_rows(a, 0)
    a.latent_dim, a.page_size = 576, 0
    with pytest.raises(ValueError, match="page_size"):
        N.mla_decode_rows(a, 0)
    a.page_size, a.q_dtype = 16, 7
    with pytest.raises(ValueError, match="dtype"):
        N.mla_decode_rows(a, 0)
    a.q_dtype = N.DTYPE_F32
    with pytest.raises(ValueError, match="NULL"):
        N.mla_decode_rows(a, 0)
    a.batch = 0                                   # nothing to do: no launch, no error
    N.mla_decode_rows(a, 0)


def test_page_descriptor_validation_without_gpu():
    """page_desc: 32-byte aligned; with it page_tags and the scale arrays may be
    NULL, and only precisions whose K pool is given need their V pool. The pack
    entry point rejects a NULL or misaligned destination and NULL page_tags
    before any launch."""
    from intent_attention import _native as N
    a = _decode_args(N, 2, 2, 4, 100)
    a.num_pages = 64
    a.page_desc = 0x100010                      # 16-byte aligned only
    with pytest.raises(ValueError, match="32-byte aligned"):
        N.workspace_bytes(a)
    a.page_desc = 0x100020
    a.page_tags = None
    assert N.workspace_bytes(a) > 0             # tags come from the descriptors
    a.k_fp8 = 0x200000                          # FP8 K pool without its V pool
    with pytest.raises(ValueError, match="FP8"):
        N.workspace_bytes(a)
    a.v_fp8 = 0x300000                          # scales not needed with descriptors
    assert N.workspace_bytes(a) > 0
    with pytest.raises(ValueError, match="page_tags"):
        N.pack_page_descriptors(a, 0x400000, 0)
    a.page_tags = 16
    with pytest.raises(ValueError, match="page_desc"):
        N.pack_page_descriptors(a, 0, 0)
    with pytest.raises(ValueError, match="page_desc"):
        N.pack_page_descriptors(a, 0x400010, 0)
    # packing reads the tag map and scales: FP8 reachable without its scales
    a.tag_map[3] = N.TAG_FP8
    with pytest.raises(ValueError, match="FP8"):
        N.pack_page_descriptors(a, 0x400000, 0)
    a.num_pages = 0                             # nothing to pack: no launch, no error
    a.tag_map[3] = N.TAG_SKIP
    N.pack_page_descriptors(a, 0, 0)


def test_entry_record_validation_without_gpu():
    """entry_records: 32-byte aligned; with them page_table, page_tags and the
    scale arrays may be NULL (page_counts may not). The pack entry point needs
    the table and tags of a valid decode call and a 32-byte aligned
    destination; it rejects the rest before any launch."""
    from intent_attention import _native as N
    a = _decode_args(N, 2, 2, 4, 100)
    a.num_pages = 64
    a.entry_records = 0x100010
    with pytest.raises(ValueError, match="entry_records must be 32-byte aligned"):
        N.workspace_bytes(a)
    a.entry_records = 0x100020
    a.page_table = a.page_tags = None
    assert N.workspace_bytes(a) > 0
    a.page_counts = None
    with pytest.raises(ValueError, match="page_counts"):
        N.workspace_bytes(a)
    a.page_counts = 16
    with pytest.raises(ValueError, match="page_table"):        # packing needs the table
        N.pack_entry_records(a, 0x400000, 0)
    a.page_table = 16
    with pytest.raises(ValueError, match="page_tags"):
        N.pack_entry_records(a, 0x400000, 0)
    a.page_tags = 16
    with pytest.raises(ValueError, match="records"):
        N.pack_entry_records(a, 0, 0)
    with pytest.raises(ValueError, match="records"):
        N.pack_entry_records(a, 0x400010, 0)
    a.table_width = 0                                          # no entries: no launch, no error
    N.pack_entry_records(a, 0, 0)
