"""ctypes binding of libiak.so, the C ABI declared in include/iak.h.

The library is built in-tree (``make -C intent-attention-kernel_amd/csrc``)
next to this file. Nothing here falls back to another implementation: if the
library is missing or was built for another ABI version, every entry point
raises RuntimeError.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

_HERE = os.path.dirname(os.path.abspath(__file__))
# IAK_LIBRARY selects another build of the same ABI (e.g. a tuning variant)
LIB_PATH = os.environ.get("IAK_LIBRARY") or os.path.join(_HERE, "libiak.so")
ABI_VERSION = 11

IAK_OK, IAK_EINVAL, IAK_ENOTSUP, IAK_EHIP = 0, 1, 2, 3

TAG_FP16, TAG_INT8, TAG_SKIP, TAG_FP8, TAG_INT4, TAG_INT4_RESIDUAL = 0, 1, 2, 3, 4, 5
DTYPE_F16, DTYPE_F32, DTYPE_BF16 = 0, 1, 2
MASK_BOOL = 3
CAUSAL_NONE, CAUSAL_TRIU, CAUSAL_POSITIONS = 0, 1, 2

c_i32, c_i64, c_void_p, c_float = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p, ctypes.c_float


class PagedDecodeArgs(ctypes.Structure):
    """Mirror of ``iak_paged_decode_args`` (include/iak.h)."""

    _fields_ = [
        ("batch", c_i32), ("num_q_heads", c_i32), ("num_kv_heads", c_i32), ("head_dim", c_i32),
        ("page_size", c_i32), ("table_width", c_i32),
        ("num_pages", c_i64),
        ("q", c_void_p), ("q_dtype", c_i32), ("q_stride_b", c_i64), ("q_stride_h", c_i64),
        ("out", c_void_p), ("out_dtype", c_i32), ("out_stride_b", c_i64), ("out_stride_h", c_i64),
        ("page_table", c_void_p), ("page_counts", c_void_p), ("page_tags", c_void_p),
        ("tag_map", ctypes.c_uint8 * 8),
        ("negative_ids", c_i32),
        ("k_fp16", c_void_p), ("v_fp16", c_void_p),
        ("k_fp8", c_void_p), ("v_fp8", c_void_p),
        ("k_int8", c_void_p), ("v_int8", c_void_p),
        ("k_int4", c_void_p), ("v_int4", c_void_p),
        ("k_int4r", c_void_p), ("v_int4r", c_void_p),
        ("k_fp8_scale", c_void_p), ("v_fp8_scale", c_void_p), ("fp8_scale_dtype", c_i32),
        ("k_int8_scale", c_void_p), ("v_int8_scale", c_void_p), ("int8_scale_dtype", c_i32),
        ("k_int4_scale", c_void_p), ("v_int4_scale", c_void_p), ("int4_scale_dtype", c_i32),
        ("int4_group", c_i32),
        ("k_int4r_scale", c_void_p), ("v_int4r_scale", c_void_p),
        ("sm_scale", c_float),
        ("pages_per_split", c_i32),
        ("map_other_tags", c_i32),
        ("valid_tokens", c_void_p),
        ("merge_in_kernel", c_i32),
        ("page_desc", c_void_p),
        ("entry_records", c_void_p),
    ]


class MlaDecodeArgs(ctypes.Structure):
    """Mirror of ``iak_mla_decode_args`` (include/iak.h)."""

    _fields_ = [
        ("batch", c_i32), ("num_heads", c_i32), ("qk_dim", c_i32), ("v_dim", c_i32), ("v_offset", c_i32),
        ("page_size", c_i32), ("table_width", c_i32),
        ("num_pages", c_i64),
        ("q", c_void_p), ("q_dtype", c_i32), ("q_stride_b", c_i64), ("q_stride_h", c_i64),
        ("out", c_void_p), ("out_dtype", c_i32), ("out_stride_b", c_i64), ("out_stride_h", c_i64),
        ("page_table", c_void_p), ("page_counts", c_void_p), ("page_tags", c_void_p),
        ("tag_map", ctypes.c_uint8 * 8),
        ("negative_ids", c_i32),
        ("valid_tokens", c_void_p),
        ("c_fp16", c_void_p), ("c_fp8", c_void_p), ("c_int8", c_void_p),
        ("c_fp8_scale", c_void_p), ("c_int8_scale", c_void_p), ("scale_dtype", c_i32),
        ("sm_scale", c_float),
        ("pages_per_split", c_i32),
    ]


QUANT_FAKE_QUANTIZE, QUANT_FUSED_INT8, QUANT_TRITON_INT8 = 0, 1, 2


class QuantizeArgs(ctypes.Structure):
    """Mirror of ``iak_quantize_args`` (include/iak.h)."""

    _fields_ = [
        ("num_pages", c_i32), ("page_size", c_i32), ("head_dim", c_i32),
        ("src", c_void_p), ("dst_pages", c_void_p), ("pool_pages", c_i64),
        ("precision", c_i32), ("mode", c_i32), ("int4_group", c_i32),
        ("codes", c_void_p), ("scales", c_void_p), ("scale_dtype", c_i32),
    ]


class PageTableArgs(ctypes.Structure):
    """Mirror of ``iak_page_table_args`` (include/iak.h)."""

    _fields_ = [
        ("num_rows", c_i32), ("rows_per_seq", c_i32), ("rows_per_list", c_i32),
        ("table_width", c_i32), ("page_size", c_i32), ("num_pages", c_i32),
        ("dedupe", c_i32), ("default_tag", c_i32), ("block_table_width", c_i32),
        ("span_offsets", c_void_p), ("span_begin", c_void_p), ("span_end", c_void_p), ("span_tag", c_void_p),
        ("block_table", c_void_p),
        ("page_table", c_void_p), ("page_counts", c_void_p), ("page_precision", c_void_p),
    ]


TRANSCODE_DEMOTE_INT8, TRANSCODE_PROMOTE_FP16 = 0, 1


class TranscodeArgs(ctypes.Structure):
    """Mirror of ``iak_transcode_args`` (include/iak.h)."""

    _fields_ = [
        ("num_pages", c_i32), ("page_elems", c_i32), ("mode", c_i32),
        ("pages", c_void_p), ("pool_pages", c_i64),
        ("fp16", c_void_p), ("int8", c_void_p), ("scales", c_void_p),
    ]


class PrefetchArgs(ctypes.Structure):
    """Mirror of ``iak_prefetch_args`` (include/iak.h)."""

    _fields_ = [
        ("batch", c_i32), ("heads", c_i32), ("kv_len", c_i32), ("head_dim", c_i32), ("page_size", c_i32),
        ("num_ids", c_i32),
        ("page_ids", c_void_p), ("k", c_void_p), ("v", c_void_p),
        ("k_stride_b", c_i64), ("k_stride_h", c_i64), ("k_stride_t", c_i64),
        ("v_stride_b", c_i64), ("v_stride_h", c_i64), ("v_stride_t", c_i64),
        ("checksum", c_void_p),
    ]


class MlaRowsArgs(ctypes.Structure):
    """Mirror of ``iak_mla_rows_args`` (include/iak.h)."""

    _fields_ = [
        ("batch", c_i32), ("q_len", c_i32), ("latent_dim", c_i32), ("page_size", c_i32), ("num_selected", c_i32),
        ("num_rows", c_i64),
        ("q", c_void_p), ("q_dtype", c_i32), ("q_stride_b", c_i64), ("q_stride_t", c_i64),
        ("latents", c_void_p), ("latent_dtype", c_i32), ("latent_stride", c_i64),
        ("page_ids", c_void_p),
        ("context", c_void_p),
        ("sm_scale", c_float),
    ]


FQ_FP16, FQ_FP8, FQ_INT8, FQ_INT4, FQ_INT4_RESIDUAL, FQ_SKIP = 0, 1, 2, 3, 4, 5   # IAK_FQ_*


class FakeQuantBlocksArgs(ctypes.Structure):
    """Mirror of ``iak_fake_quant_blocks_args`` (include/iak.h)."""

    _fields_ = [
        ("lead", c_i32), ("num_blocks", c_i32), ("k_dim", c_i32), ("v_dim", c_i32),
        ("k", c_void_p), ("k_stride_l", c_i64), ("k_stride_t", c_i64),
        ("v", c_void_p), ("v_stride_l", c_i64), ("v_stride_t", c_i64),
        ("blocks", c_void_p), ("max_block_tokens", c_i32),
        ("out", c_void_p), ("out_stride_l", c_i64), ("out_stride_t", c_i64),
    ]


class DenseAttentionArgs(ctypes.Structure):
    """Mirror of ``iak_dense_attention_args`` (include/iak.h)."""

    _fields_ = [
        ("batch", c_i32), ("q_len", c_i32), ("kv_len", c_i32), ("head_dim", c_i32), ("v_dim", c_i32),
        ("dtype", c_i32),
        ("q", c_void_p), ("q_stride_b", c_i64), ("q_stride_t", c_i64),
        ("k", c_void_p), ("k_stride_b", c_i64), ("k_stride_t", c_i64),
        ("v", c_void_p), ("v_stride_b", c_i64), ("v_stride_t", c_i64),
        ("out", c_void_p), ("out_stride_b", c_i64), ("out_stride_t", c_i64),
        ("mask", c_void_p), ("mask_dtype", c_i32), ("mask_stride_b", c_i64), ("mask_stride_q", c_i64),
        ("mask_stride_k", c_i64),
        ("causal", c_i32),
        ("kv_positions", c_void_p),
        ("sm_scale", c_float),
    ]


EXPORTED = ("iak_abi_version", "iak_status_string", "iak_last_error",
            "iak_paged_decode_workspace", "iak_paged_decode",
            "iak_mla_decode_workspace", "iak_mla_decode", "iak_quantize_pages",
            "iak_build_page_tables", "iak_paged_decode_timed", "iak_mla_decode_timed",
            "iak_paged_decode_noalloc", "iak_transcode_pages", "iak_prefetch_pages", "iak_paged_decode_plan",
            "iak_mla_decode_rows", "iak_pack_page_descriptors",
            "iak_pack_entry_records", "iak_dense_attention", "iak_dense_attention_workspace",
            "iak_mla_decode_rows_workspace", "iak_fake_quant_blocks",
            "iak_fake_quant_blocks_workspace", "iak_timing_event_create", "iak_timing_event_record",
            "iak_timing_event_elapsed", "iak_timing_event_destroy")
NOALLOC_SCRATCH_BYTES = 16 << 20   # IAK_NOALLOC_SCRATCH_BYTES

_lib: Optional[ctypes.CDLL] = None
_load_error: Optional[str] = None


def load() -> ctypes.CDLL:
    """Load libiak.so once; RuntimeError if it is absent or mismatched."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    if _load_error is not None:
        raise RuntimeError(_load_error)
    if not os.path.exists(LIB_PATH):
        _load_error = (f"libiak.so not found at {LIB_PATH}; build it with "
                       "`make -C intent-attention-kernel_amd/csrc` (or __graft_entry__.build())")
        raise RuntimeError(_load_error)
    try:
        lib = ctypes.CDLL(LIB_PATH)
    except OSError as e:
        _load_error = f"cannot load {LIB_PATH}: {e}"
        raise RuntimeError(_load_error) from e
    lib.iak_abi_version.restype = ctypes.c_int
    lib.iak_abi_version.argtypes = []
    lib.iak_status_string.restype = ctypes.c_char_p
    lib.iak_status_string.argtypes = [ctypes.c_int]
    lib.iak_last_error.restype = ctypes.c_char_p
    lib.iak_last_error.argtypes = []
    lib.iak_paged_decode_workspace.restype = ctypes.c_int
    lib.iak_paged_decode_workspace.argtypes = [ctypes.POINTER(PagedDecodeArgs), ctypes.POINTER(ctypes.c_size_t)]
    lib.iak_paged_decode_plan.restype = ctypes.c_int
    lib.iak_paged_decode_plan.argtypes = [ctypes.POINTER(PagedDecodeArgs), ctypes.POINTER(PlanInfo)]
    lib.iak_paged_decode.restype = ctypes.c_int
    lib.iak_paged_decode.argtypes = [ctypes.POINTER(PagedDecodeArgs), c_void_p, ctypes.c_size_t, c_void_p]
    lib.iak_mla_decode_workspace.restype = ctypes.c_int
    lib.iak_mla_decode_workspace.argtypes = [ctypes.POINTER(MlaDecodeArgs), ctypes.POINTER(ctypes.c_size_t)]
    lib.iak_mla_decode.restype = ctypes.c_int
    lib.iak_mla_decode.argtypes = [ctypes.POINTER(MlaDecodeArgs), c_void_p, ctypes.c_size_t, c_void_p]
    lib.iak_quantize_pages.restype = ctypes.c_int
    lib.iak_quantize_pages.argtypes = [ctypes.POINTER(QuantizeArgs), c_void_p]
    lib.iak_paged_decode_timed.restype = ctypes.c_int
    lib.iak_paged_decode_timed.argtypes = [ctypes.POINTER(PagedDecodeArgs), c_void_p, ctypes.c_size_t, c_void_p,
                                           c_void_p, c_void_p]
    lib.iak_mla_decode_timed.restype = ctypes.c_int
    lib.iak_mla_decode_timed.argtypes = [ctypes.POINTER(MlaDecodeArgs), c_void_p, ctypes.c_size_t, c_void_p,
                                         c_void_p, c_void_p]
    lib.iak_paged_decode_noalloc.restype = ctypes.c_int
    lib.iak_paged_decode_noalloc.argtypes = [ctypes.POINTER(PagedDecodeArgs), c_void_p]
    lib.iak_transcode_pages.restype = ctypes.c_int
    lib.iak_transcode_pages.argtypes = [ctypes.POINTER(TranscodeArgs), c_void_p]
    lib.iak_prefetch_pages.restype = ctypes.c_int
    lib.iak_prefetch_pages.argtypes = [ctypes.POINTER(PrefetchArgs), c_void_p]
    lib.iak_build_page_tables.restype = ctypes.c_int
    lib.iak_mla_decode_rows.restype = ctypes.c_int
    lib.iak_mla_decode_rows.argtypes = [ctypes.POINTER(MlaRowsArgs), c_void_p, ctypes.c_size_t, c_void_p]
    lib.iak_timing_event_create.restype = ctypes.c_int
    lib.iak_timing_event_create.argtypes = [ctypes.POINTER(c_void_p)]
    lib.iak_timing_event_record.restype = ctypes.c_int
    lib.iak_timing_event_record.argtypes = [c_void_p, c_void_p]
    lib.iak_timing_event_elapsed.restype = ctypes.c_int
    lib.iak_timing_event_elapsed.argtypes = [c_void_p, c_void_p, ctypes.POINTER(ctypes.c_float)]
    lib.iak_timing_event_destroy.restype = ctypes.c_int
    lib.iak_timing_event_destroy.argtypes = [c_void_p]
    lib.iak_fake_quant_blocks.restype = ctypes.c_int
    lib.iak_fake_quant_blocks.argtypes = [ctypes.POINTER(FakeQuantBlocksArgs), c_void_p, ctypes.c_size_t, c_void_p]
    lib.iak_fake_quant_blocks_workspace.restype = ctypes.c_int
    lib.iak_fake_quant_blocks_workspace.argtypes = [ctypes.POINTER(FakeQuantBlocksArgs),
                                                    ctypes.POINTER(ctypes.c_size_t)]
    lib.iak_mla_decode_rows_workspace.restype = ctypes.c_int
    lib.iak_mla_decode_rows_workspace.argtypes = [ctypes.POINTER(MlaRowsArgs), ctypes.POINTER(ctypes.c_size_t)]
    lib.iak_build_page_tables.argtypes = [ctypes.POINTER(PageTableArgs), c_void_p]
    lib.iak_pack_page_descriptors.restype = ctypes.c_int
    lib.iak_pack_page_descriptors.argtypes = [ctypes.POINTER(PagedDecodeArgs), c_void_p, c_void_p]
    lib.iak_dense_attention.restype = ctypes.c_int
    lib.iak_dense_attention.argtypes = [ctypes.POINTER(DenseAttentionArgs), c_void_p, ctypes.c_size_t, c_void_p]
    lib.iak_dense_attention_workspace.restype = ctypes.c_int
    lib.iak_dense_attention_workspace.argtypes = [ctypes.POINTER(DenseAttentionArgs), ctypes.POINTER(ctypes.c_size_t)]
    lib.iak_pack_entry_records.restype = ctypes.c_int
    lib.iak_pack_entry_records.argtypes = [ctypes.POINTER(PagedDecodeArgs), c_void_p, c_void_p]
    ver = lib.iak_abi_version()
    if ver != ABI_VERSION:
        _load_error = f"libiak.so ABI version {ver} != expected {ABI_VERSION}; rebuild the library"
        raise RuntimeError(_load_error)
    _lib = lib
    return lib


def check(status: int) -> None:
    """Map a status to the reference's exception types (ValueError / RuntimeError)."""
    if status == IAK_OK:
        return
    lib = load()
    msg = (lib.iak_last_error() or b"").decode(errors="replace")
    what = (lib.iak_status_string(status) or b"").decode()
    if status in (IAK_EINVAL, IAK_ENOTSUP):
        raise ValueError(f"{msg} ({what})")
    raise RuntimeError(f"{msg} ({what})")


class PlanInfo(ctypes.Structure):
    """Mirror of ``iak_paged_decode_plan_info`` (include/iak.h)."""

    _fields_ = [("splits", c_i32), ("pages_per_split", c_i32), ("merge_in_kernel", c_i32),
                ("workspace_bytes", ctypes.c_size_t), ("tail_splits", c_i32), ("tail_pages_per_split", c_i32)]


def plan_info(args: PagedDecodeArgs) -> dict:
    """The split plan the library chooses for ``args``."""
    info = PlanInfo()
    check(load().iak_paged_decode_plan(ctypes.byref(args), ctypes.byref(info)))
    return {"splits": int(info.splits), "pages_per_split": int(info.pages_per_split),
            "merge_in_kernel": bool(info.merge_in_kernel), "workspace_bytes": int(info.workspace_bytes),
            "tail_splits": int(info.tail_splits), "tail_pages_per_split": int(info.tail_pages_per_split)}


def workspace_bytes(args: PagedDecodeArgs) -> int:
    n = ctypes.c_size_t(0)
    check(load().iak_paged_decode_workspace(ctypes.byref(args), ctypes.byref(n)))
    return int(n.value)


def paged_decode(args: PagedDecodeArgs, workspace_ptr: int, workspace_size: int, stream: int,
                 events: Optional[tuple] = None) -> None:
    """``events``: optional (begin, end) hipEvent_t handles recorded around the split kernel."""
    if events is None:
        check(load().iak_paged_decode(ctypes.byref(args), workspace_ptr or None, workspace_size, stream or None))
    else:
        check(load().iak_paged_decode_timed(ctypes.byref(args), workspace_ptr or None, workspace_size,
                                            stream or None, events[0] or None, events[1] or None))


PAGE_DESC_BYTES = 32   # one iak_paged_decode_args.page_desc entry


def pack_page_descriptors(args: PagedDecodeArgs, desc_ptr: int, stream: int) -> None:
    """iak_pack_page_descriptors: ``args.num_pages`` 32-byte descriptors at ``desc_ptr``."""
    check(load().iak_pack_page_descriptors(ctypes.byref(args), desc_ptr or None, stream or None))


ENTRY_RECORD_BYTES = 32   # one iak_paged_decode_args.entry_records entry


def pack_entry_records(args: PagedDecodeArgs, records_ptr: int, stream: int) -> None:
    """iak_pack_entry_records: batch x num_kv_heads x table_width 32-byte records at ``records_ptr``."""
    check(load().iak_pack_entry_records(ctypes.byref(args), records_ptr or None, stream or None))


def paged_decode_noalloc(args: PagedDecodeArgs, stream: int) -> None:
    """iak_paged_decode_noalloc: the split-K partials in the library's own scratch."""
    check(load().iak_paged_decode_noalloc(ctypes.byref(args), stream or None))


def mla_workspace_bytes(args: MlaDecodeArgs) -> int:
    n = ctypes.c_size_t(0)
    check(load().iak_mla_decode_workspace(ctypes.byref(args), ctypes.byref(n)))
    return int(n.value)


def mla_decode(args: MlaDecodeArgs, workspace_ptr: int, workspace_size: int, stream: int,
               events: Optional[tuple] = None) -> None:
    """``events``: optional (begin, end) hipEvent_t handles recorded around the split kernel."""
    if events is None:
        check(load().iak_mla_decode(ctypes.byref(args), workspace_ptr or None, workspace_size, stream or None))
    else:
        check(load().iak_mla_decode_timed(ctypes.byref(args), workspace_ptr or None, workspace_size,
                                          stream or None, events[0] or None, events[1] or None))


def quantize_pages(args: QuantizeArgs, stream: int) -> None:
    check(load().iak_quantize_pages(ctypes.byref(args), stream or None))


def transcode_pages(args: TranscodeArgs, stream: int) -> None:
    check(load().iak_transcode_pages(ctypes.byref(args), stream or None))


def prefetch_pages(args: PrefetchArgs, stream: int) -> None:
    check(load().iak_prefetch_pages(ctypes.byref(args), stream or None))


def mla_decode_rows_workspace(args: MlaRowsArgs) -> int:
    n = ctypes.c_size_t(0)
    check(load().iak_mla_decode_rows_workspace(ctypes.byref(args), ctypes.byref(n)))
    return int(n.value)


def mla_decode_rows(args: MlaRowsArgs, stream: int, workspace: int = 0, workspace_bytes: int = 0) -> None:
    check(load().iak_mla_decode_rows(ctypes.byref(args), workspace or None, workspace_bytes, stream or None))


def build_page_tables(args: PageTableArgs, stream: int) -> None:
    check(load().iak_build_page_tables(ctypes.byref(args), stream or None))


class TimingEvent:
    """A fence-free HIP timing event (``iak_timing_event_create``): ``record``,
    ``elapsed_time`` (ms, read after a device synchronize) and ``cuda_event``
    (the handle the ``_timed`` entry points take), as torch.cuda.Event offers
    them; destroyed with the object."""

    def __init__(self) -> None:
        h = c_void_p()
        check(load().iak_timing_event_create(ctypes.byref(h)))
        self._h = h.value

    @property
    def cuda_event(self) -> int:
        return self._h

    def record(self, stream) -> None:
        check(load().iak_timing_event_record(self._h, getattr(stream, "cuda_stream", stream) or None))

    def elapsed_time(self, end: "TimingEvent") -> float:
        ms = ctypes.c_float(0.0)
        check(load().iak_timing_event_elapsed(self._h, end._h, ctypes.byref(ms)))
        return ms.value

    def __del__(self) -> None:
        h, self._h = getattr(self, "_h", None), None
        if h and _lib is not None:
            _lib.iak_timing_event_destroy(h)


def fake_quant_blocks_workspace(args: FakeQuantBlocksArgs) -> int:
    n = ctypes.c_size_t(0)
    check(load().iak_fake_quant_blocks_workspace(ctypes.byref(args), ctypes.byref(n)))
    return n.value


def fake_quant_blocks(args: FakeQuantBlocksArgs, stream: int, workspace: int = 0, workspace_bytes: int = 0) -> None:
    check(load().iak_fake_quant_blocks(ctypes.byref(args), workspace or None, workspace_bytes, stream or None))


def dense_attention_workspace(args: DenseAttentionArgs) -> int:
    n = ctypes.c_size_t(0)
    check(load().iak_dense_attention_workspace(ctypes.byref(args), ctypes.byref(n)))
    return int(n.value)


def dense_attention(args: DenseAttentionArgs, stream: int, workspace: int = 0, workspace_bytes: int = 0) -> None:
    check(load().iak_dense_attention(ctypes.byref(args), workspace or None, workspace_bytes, stream or None))
