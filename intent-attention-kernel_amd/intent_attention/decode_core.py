"""Device entry point of the selected-page decode: torch tensors -> C ABI.

``paged_decode`` is the one function both reference-shaped APIs
(``fused_selected_quant_decode`` and ``intent_quant_decode_attention_triton``)
call. It checks shapes, fills ``iak_paged_decode_args`` with device pointers,
allocates the split-K workspace from torch's caching allocator and launches
on torch's current HIP stream. It never runs on the CPU: host tensors or a
missing libiak.so raise.
"""
from __future__ import annotations

import math
import threading
import weakref
from collections import OrderedDict
from dataclasses import dataclass, fields
from typing import Dict, Optional, Sequence

import torch

from . import _native as N

PAGE_SIZE = 16
# iak_paged_decode_args.merge_in_kernel for merge_in_kernel=None: automatic (the
# decode kernel merges its split partials itself on grids of many workgroups)
MERGE_IN_KERNEL_AUTO = 2

_DT = {torch.float16: N.DTYPE_F16, torch.float32: N.DTYPE_F32, torch.bfloat16: N.DTYPE_BF16}

# Native tag identity map (IAK_TAG_*); unused slots are SKIP.
NATIVE_TAG_MAP = (N.TAG_FP16, N.TAG_INT8, N.TAG_SKIP, N.TAG_FP8, N.TAG_INT4, N.TAG_INT4_RESIDUAL,
                  N.TAG_SKIP, N.TAG_SKIP)


@dataclass
class PagePools:
    """Per-precision K/V page pools, each indexed by physical page id.

    Shapes (NP pages of PS=16 tokens, head_dim D):
      k_fp16, v_fp16            [NP, 16, D] float16
      k_fp8, v_fp8              [NP, 16, D] uint8 (e4m3fn codes); *_fp8_scale [NP] f16/f32
      k_int8, v_int8            [NP, 16, D] int8;                  *_int8_scale [NP] f16/f32
      k_int4, v_int4            [NP, 16, D/2] uint8 (element 2j low nibble of byte j,
                                nibble = code + 8);                *_int4_scale [NP, D/int4_group]
      k_int4r, v_int4r          [NP, 16, D] uint8 ((base+8) | (residual+8) << 4);
                                *_int4r_scale [NP, 2] float32 (base, residual)
    Absent precisions stay None; pages tagged with them must not be reachable.
    """

    k_fp16: Optional[torch.Tensor] = None
    v_fp16: Optional[torch.Tensor] = None
    k_fp8: Optional[torch.Tensor] = None
    v_fp8: Optional[torch.Tensor] = None
    k_fp8_scale: Optional[torch.Tensor] = None
    v_fp8_scale: Optional[torch.Tensor] = None
    k_int8: Optional[torch.Tensor] = None
    v_int8: Optional[torch.Tensor] = None
    k_int8_scale: Optional[torch.Tensor] = None
    v_int8_scale: Optional[torch.Tensor] = None
    k_int4: Optional[torch.Tensor] = None
    v_int4: Optional[torch.Tensor] = None
    k_int4_scale: Optional[torch.Tensor] = None
    v_int4_scale: Optional[torch.Tensor] = None
    int4_group: int = 32
    k_int4r: Optional[torch.Tensor] = None
    v_int4r: Optional[torch.Tensor] = None
    k_int4r_scale: Optional[torch.Tensor] = None
    v_int4r_scale: Optional[torch.Tensor] = None

    def tensors(self) -> Dict[str, torch.Tensor]:
        return {f.name: getattr(self, f.name) for f in fields(self)
                if isinstance(getattr(self, f.name), torch.Tensor)}

    def has(self, tag: int) -> bool:
        need = {N.TAG_FP16: ("k_fp16", "v_fp16"),
                N.TAG_INT8: ("k_int8", "v_int8", "k_int8_scale", "v_int8_scale"),
                N.TAG_FP8: ("k_fp8", "v_fp8", "k_fp8_scale", "v_fp8_scale"),
                N.TAG_INT4: ("k_int4", "v_int4", "k_int4_scale", "v_int4_scale"),
                N.TAG_INT4_RESIDUAL: ("k_int4r", "v_int4r", "k_int4r_scale", "v_int4r_scale")}.get(tag, ())
        return bool(need) and all(getattr(self, n) is not None for n in need)


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def current_stream_handle(device: torch.device) -> int:
    """The raw hipStream_t of torch's current stream on ``device`` (the cheap lookup
    when this torch build has it)."""
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def require_device(*tensors: torch.Tensor, what: str = "fused selected-quant decode") -> torch.device:
    """All tensors on one ROCm device, or RuntimeError (no host path exists)."""
    devs = {t.device for t in tensors if isinstance(t, torch.Tensor)}
    if not devs or any(d.type != "cuda" for d in devs):
        raise RuntimeError(
            f"{what} runs on the MI355X HIP kernels only: pass tensors on a ROCm device "
            f"(got {sorted(str(d) for d in devs)}); the CPU restatement is test code, not a fallback")
    if len(devs) != 1:
        raise ValueError(f"all tensors must be on one device, got {sorted(str(d) for d in devs)}")
    N.load()
    return devs.pop()


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _check_pool(name: str, t: Optional[torch.Tensor], NP: int, row: Sequence[int], dtypes) -> None:
    if t is None:
        return
    if t.dtype not in dtypes:
        raise ValueError(f"{name} must have dtype in {[str(d) for d in dtypes]}, got {t.dtype}")
    if tuple(t.shape) != (NP, *row):
        raise ValueError(f"{name} must have shape {(NP, *row)}, got {tuple(t.shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _scale_dtype(name: str, *ts: Optional[torch.Tensor]) -> int:
    dts = {t.dtype for t in ts if t is not None}
    if not dts:
        return N.DTYPE_F32
    if len(dts) != 1 or next(iter(dts)) not in (torch.float16, torch.float32):
        raise ValueError(f"{name} scales must both be float16 or both float32, got {dts}")
    return _DT[next(iter(dts))]


def paged_decode(q: torch.Tensor, pools: PagePools, page_table: torch.Tensor, page_counts: torch.Tensor,
                 page_tags: torch.Tensor, *, tag_map: Optional[Sequence[int]] = None,
                 negative_ids: bool = False, sm_scale: Optional[float] = None,
                 out: Optional[torch.Tensor] = None, out_dtype: Optional[torch.dtype] = None,
                 pages_per_split: int = 0, map_other_tags: bool = False,
                 valid_tokens: Optional[torch.Tensor] = None,
                 merge_in_kernel: Optional[bool] = None) -> torch.Tensor:
    """Selected-page decode attention on the GPU.

    q [B, Hq, D] (f16 / f32 / bf16, any strides with unit last stride);
    page_table [B, Hkv, W] int32; page_counts [B, Hkv] int32; page_tags [NP]
    int32 caller tags mapped through ``tag_map`` (8 entries of IAK_TAG_*);
    the default maps each native tag whose pools are present to itself and
    every other tag to SKIP (contributes nothing). Caller tags outside
    [0, 8) contribute nothing, or take ``tag_map[7]`` with
    ``map_other_tags``. Query head h uses row h // (Hq // Hkv).
    ``valid_tokens`` [B, Hkv] int32 (optional): token t of table entry e of a
    row exists only if e * 16 + t < valid_tokens[row] (a ragged last page).
    ``merge_in_kernel``: True: the decode kernel merges the split partials
    itself (one launch); False: a merge kernel after it; None: the library
    chooses (in-kernel on grids of many workgroups).
    Returns out [B, Hq, D].
    """
    plan = make_plan(q, pools, page_table, page_counts, page_tags, tag_map=tag_map, negative_ids=negative_ids,
                     sm_scale=sm_scale, out=out, out_dtype=out_dtype, pages_per_split=pages_per_split,
                     map_other_tags=map_other_tags, valid_tokens=valid_tokens, merge_in_kernel=merge_in_kernel)
    plan.run()
    return plan.out


def make_plan(q: torch.Tensor, pools: PagePools, page_table: torch.Tensor, page_counts: torch.Tensor,
              page_tags: torch.Tensor, *, tag_map: Optional[Sequence[int]] = None,
              negative_ids: bool = False, sm_scale: Optional[float] = None,
              out: Optional[torch.Tensor] = None, out_dtype: Optional[torch.dtype] = None,
              pages_per_split: int = 0, map_other_tags: bool = False,
              valid_tokens: Optional[torch.Tensor] = None,
              merge_in_kernel: Optional[bool] = None,
              page_descriptors: Optional[torch.Tensor] = None,
              entry_records: Optional[torch.Tensor] = None,
              auto_records: bool = True) -> "DecodePlan":
    """Validate the arguments of ``paged_decode`` once; the returned plan
    re-launches the decode on the same tensors with ``run()``.

    ``auto_records`` (default on): when ``run()`` finds the page table, the
    tags and the scale tensors unchanged since the previous run (torch's
    version counters of those tensors), it packs entry records once and reads
    them from then on, until one of those tensors changes; results are
    bit-identical either way. Tensors written other than by torch's in-place
    ops must be marked (``torch.autograd.graph.increment_version``) or the
    plan told (``invalidate_records``): this package's own writers do so.

    ``page_descriptors`` (optional): [num_pages, 8] int32 descriptors from
    ``DecodePlan.pack_descriptors`` (or ``pack_page_descriptors``), read in
    place of ``page_tags``, ``tag_map`` and the scale tensors: one 32-byte
    line of metadata per selected page.
    ``entry_records`` (optional): [B, Hkv, W, 8] int32 records from
    ``DecodePlan.pack_records``, read in place of the page table's entries and
    their pages' tags and scales: one contiguous metadata stream per split."""
    if q.dim() != 3:
        raise ValueError(f"q must have shape [B, H, D], got {tuple(q.shape)}")
    B, Hq, D = q.shape
    if page_table.dim() != 3 or page_table.shape[0] != B:
        raise ValueError(f"page_table must have shape [B, Hkv, W] with B={B}, got {tuple(page_table.shape)}")
    Hkv, W = int(page_table.shape[1]), int(page_table.shape[2])
    if Hkv == 0 or Hq % Hkv != 0:
        raise ValueError(f"query heads {Hq} must be a multiple of page-table heads {Hkv}")
    if tuple(page_counts.shape) != (B, Hkv):
        raise ValueError(f"page_counts must have shape {(B, Hkv)}, got {tuple(page_counts.shape)}")
    if page_tags.dim() != 1:
        raise ValueError(f"page_precision must have shape [num_pages], got {tuple(page_tags.shape)}")
    NP = int(page_tags.shape[0])
    in_ptrs = (page_table.data_ptr(), page_counts.data_ptr(), page_tags.data_ptr(),
               valid_tokens.data_ptr() if valid_tokens is not None else None)
    extra = () if valid_tokens is None else (valid_tokens,)
    dev = require_device(q, page_table, page_counts, page_tags, *extra, *pools.tensors().values())
    if valid_tokens is not None:
        if tuple(valid_tokens.shape) != (B, Hkv) or valid_tokens.dtype != torch.int32:
            raise ValueError(f"valid_tokens must be int32 [{B}, {Hkv}], got {tuple(valid_tokens.shape)} "
                             f"{valid_tokens.dtype}")
        valid_tokens = valid_tokens.contiguous()
    for name, t in (("page_table", page_table), ("page_counts", page_counts), ("page_precision", page_tags)):
        if t.dtype != torch.int32:
            raise ValueError(f"{name} must be int32, got {t.dtype}")
    page_table, page_counts, page_tags = (t.contiguous() for t in (page_table, page_counts, page_tags))
    if q.dtype not in _DT:
        raise ValueError(f"q dtype {q.dtype} not supported")
    qvec = 4 if q.dtype == torch.float32 else 8
    if q.stride(-1) != 1 or q.data_ptr() % 16 or q.stride(0) % qvec or q.stride(1) % qvec:
        # the kernel reads q rows as 16-byte vectors: a fresh (aligned) copy
        q = torch.empty(q.shape, dtype=q.dtype, device=q.device).copy_(q)

    f16, u8, i8 = (torch.float16,), (torch.uint8,), (torch.int8,)
    _check_pool("k_fp16", pools.k_fp16, NP, (PAGE_SIZE, D), f16)
    _check_pool("v_fp16", pools.v_fp16, NP, (PAGE_SIZE, D), f16)
    _check_pool("k_fp8", pools.k_fp8, NP, (PAGE_SIZE, D), u8 + (torch.float8_e4m3fn,))
    _check_pool("v_fp8", pools.v_fp8, NP, (PAGE_SIZE, D), u8 + (torch.float8_e4m3fn,))
    _check_pool("k_int8", pools.k_int8, NP, (PAGE_SIZE, D), i8)
    _check_pool("v_int8", pools.v_int8, NP, (PAGE_SIZE, D), i8)
    _check_pool("k_int4", pools.k_int4, NP, (PAGE_SIZE, D // 2), u8)
    _check_pool("v_int4", pools.v_int4, NP, (PAGE_SIZE, D // 2), u8)
    _check_pool("k_int4r", pools.k_int4r, NP, (PAGE_SIZE, D), u8)
    _check_pool("v_int4r", pools.v_int4r, NP, (PAGE_SIZE, D), u8)
    sc = (torch.float16, torch.float32)
    for n in ("k_fp8_scale", "v_fp8_scale", "k_int8_scale", "v_int8_scale"):
        t = getattr(pools, n)
        if t is not None and (t.dtype not in sc or t.numel() != NP):
            raise ValueError(f"{n} must be [{NP}] float16/float32, got {tuple(t.shape)} {t.dtype}")
    grp = int(pools.int4_group)
    if grp <= 0 or D % grp:
        raise ValueError(f"int4_group must be a positive divisor of head_dim {D}, got {grp}")
    for n in ("k_int4_scale", "v_int4_scale"):
        t = getattr(pools, n)
        if t is not None and (t.dtype not in sc or t.numel() != NP * (D // grp)):
            raise ValueError(f"{n} must be [{NP}, {D // grp}] float16/float32, got {tuple(t.shape)}")
    for n in ("k_int4r_scale", "v_int4r_scale"):
        t = getattr(pools, n)
        if t is not None and (t.dtype != torch.float32 or t.numel() != 2 * NP):
            raise ValueError(f"{n} must be [{NP}, 2] float32, got {tuple(t.shape)} {t.dtype}")
    for n, t in pools.tensors().items():
        if not t.is_contiguous():
            raise ValueError(f"{n} must be contiguous")

    if out is None:
        out = torch.empty((B, Hq, D), dtype=out_dtype or q.dtype, device=dev)
    else:
        if tuple(out.shape) != (B, Hq, D) or out.dtype not in _DT or out.stride(-1) != 1:
            raise ValueError(f"out must be [B, H, D] with unit last stride, got {tuple(out.shape)}")

    a = N.PagedDecodeArgs()
    a.batch, a.num_q_heads, a.num_kv_heads, a.head_dim = B, Hq, Hkv, D
    a.page_size, a.table_width, a.num_pages = PAGE_SIZE, W, NP
    a.q, a.q_dtype, a.q_stride_b, a.q_stride_h = q.data_ptr(), _DT[q.dtype], q.stride(0), q.stride(1)
    a.out, a.out_dtype = out.data_ptr(), _DT[out.dtype]
    a.out_stride_b, a.out_stride_h = out.stride(-3), out.stride(-2)
    a.page_table, a.page_counts, a.page_tags = page_table.data_ptr(), page_counts.data_ptr(), page_tags.data_ptr()
    if tag_map is None:
        tag_map = [t if pools.has(t) else N.TAG_SKIP for t in NATIVE_TAG_MAP]
    tm = list(tag_map) + [N.TAG_SKIP] * (8 - len(tag_map))
    for i in range(8):
        a.tag_map[i] = int(tm[i])
    a.negative_ids = 1 if negative_ids else 0
    for n in ("k_fp16", "v_fp16", "k_fp8", "v_fp8", "k_int8", "v_int8", "k_int4", "v_int4",
              "k_int4r", "v_int4r", "k_fp8_scale", "v_fp8_scale", "k_int8_scale", "v_int8_scale",
              "k_int4_scale", "v_int4_scale", "k_int4r_scale", "v_int4r_scale"):
        setattr(a, n, _ptr(getattr(pools, n)))
    a.fp8_scale_dtype = _scale_dtype("fp8", pools.k_fp8_scale, pools.v_fp8_scale)
    a.int8_scale_dtype = _scale_dtype("int8", pools.k_int8_scale, pools.v_int8_scale)
    a.int4_scale_dtype = _scale_dtype("int4", pools.k_int4_scale, pools.v_int4_scale)
    a.int4_group = grp
    a.sm_scale = (1.0 / math.sqrt(D)) if sm_scale is None else float(sm_scale)
    a.pages_per_split = int(pages_per_split)
    a.map_other_tags = 1 if map_other_tags else 0
    a.valid_tokens = _ptr(valid_tokens)
    a.merge_in_kernel = MERGE_IN_KERNEL_AUTO if merge_in_kernel is None else (1 if merge_in_kernel else 0)

    plan = DecodePlan(a, dev, out, keep=(q, page_table, page_counts, page_tags, valid_tokens, pools))
    plan.reads_in_place = (page_table.data_ptr() == in_ptrs[0] and page_counts.data_ptr() == in_ptrs[1]
                           and page_tags.data_ptr() == in_ptrs[2]
                           and (valid_tokens is None or valid_tokens.data_ptr() == in_ptrs[3]))
    if page_descriptors is not None:
        plan.use_descriptors(page_descriptors)
    if entry_records is not None:
        plan.use_records(entry_records)
    if auto_records and page_descriptors is None and entry_records is None and W > 0:
        scales = [getattr(pools, n) for n in ("k_fp8_scale", "v_fp8_scale", "k_int8_scale", "v_int8_scale",
                                              "k_int4_scale", "v_int4_scale", "k_int4r_scale", "v_int4r_scale")]
        plan._track = tuple(weakref.ref(t) for t in (page_table, page_tags, *scales) if t is not None)
    return plan


def _check_descriptors(desc: torch.Tensor, NP: int, device: torch.device) -> None:
    if desc.dtype != torch.int32 or tuple(desc.shape) != (NP, N.PAGE_DESC_BYTES // 4):
        raise ValueError(f"page descriptors must be int32 [{NP}, {N.PAGE_DESC_BYTES // 4}], "
                         f"got {desc.dtype} {tuple(desc.shape)}")
    if desc.device != device or not desc.is_contiguous() or desc.data_ptr() % 32:
        raise ValueError(f"page descriptors must be a contiguous, 32-byte aligned tensor on {device}")


def pack_page_descriptors(q: torch.Tensor, pools: PagePools, page_tags: torch.Tensor, *,
                          tag_map: Optional[Sequence[int]] = None, map_other_tags: bool = False,
                          out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The page descriptors of ``page_tags`` and ``pools`` (tags translated
    through ``tag_map`` as ``paged_decode`` would), as [num_pages, 8] int32 on
    the GPU, written on the current stream. ``q`` gives head_dim and device
    ([B, Hq, D]; its values are not read)."""
    D = int(q.shape[-1])
    # a one-entry table with no selected pages: the plan carries the tags and pools
    table = torch.zeros((1, 1, 1), dtype=torch.int32, device=q.device)
    counts = torch.zeros((1, 1), dtype=torch.int32, device=q.device)
    plan = make_plan(q[:1, :1], pools, table, counts, page_tags, tag_map=tag_map, map_other_tags=map_other_tags)
    assert plan.args.head_dim == D
    return plan.pack_descriptors(out)


class DecodePlan:
    """Validated launch arguments plus workspace for repeated steps over the
    same tensors (``run`` is one C call on the current stream; the tensors
    are held so their memory stays valid)."""

    def __init__(self, args: N.PagedDecodeArgs, device: torch.device, out: torch.Tensor, keep=()) -> None:
        self.args = args
        self.device = device
        self.out = out
        self._keep = keep
        info = N.plan_info(args)
        self.workspace_bytes = info["workspace_bytes"]
        self.merge_in_kernel = info["merge_in_kernel"]
        # the in-kernel merge's arrival counters (at the end of the workspace)
        # start at zero, and every run leaves them zero
        alloc = torch.zeros if self.merge_in_kernel else torch.empty
        self._ws = alloc(self.workspace_bytes, dtype=torch.uint8, device=device) if self.workspace_bytes else None
        # the zero fill runs on the current stream; a run on another stream waits for it once
        self._filled = None
        if self._ws is not None and self.merge_in_kernel:
            self._filled = torch.cuda.Event()
            self._filled.record(torch.cuda.current_stream(device))
        self._desc: Optional[torch.Tensor] = None
        self._recs: Optional[torch.Tensor] = None
        # automatic entry records: the tensors the records snapshot, the state
        # (their version counters) of the last run, and that of the packed records
        self._track: tuple = ()
        self._last_state: Optional[tuple] = None
        self._auto_recs: Optional[torch.Tensor] = None
        self._auto_state: Optional[tuple] = None
        self._auto_stream: Optional[int] = None   # the stream every automatic pack and read runs on
        self._lock = threading.Lock()             # run_with: one caller at a time re-points the arguments
        self.reads_in_place = False   # table, counts, tags (and token bounds) read where the caller keeps them

    def pack_descriptors(self, out: Optional[torch.Tensor] = None, stream: Optional[int] = None) -> torch.Tensor:
        """Pack this plan's page tags (through its tag map), and the scales each
        page's precision uses, into 32-byte page descriptors ([num_pages, 8]
        int32; ``out`` if given) on ``stream``, and make later runs read them
        instead. The descriptors are a snapshot: pack again after the tags or
        scales change."""
        NP = int(self.args.num_pages)
        if out is None:
            out = torch.empty((NP, N.PAGE_DESC_BYTES // 4), dtype=torch.int32, device=self.device)
        _check_descriptors(out, NP, self.device)
        s = current_stream_handle(self.device) if stream is None else stream
        N.pack_page_descriptors(self.args, out.data_ptr(), s)
        self.use_descriptors(out)
        return out

    def _records_shape(self) -> tuple:
        a = self.args
        return (int(a.batch), int(a.num_kv_heads), int(a.table_width), N.ENTRY_RECORD_BYTES // 4)

    def pack_records(self, out: Optional[torch.Tensor] = None, stream: Optional[int] = None) -> torch.Tensor:
        """Pack this plan's page table entries with their pages' native tags and
        scales into 32-byte entry records ([B, Hkv, W, 8] int32; ``out`` if
        given) on ``stream``, and make later runs read them instead of the
        table, tags and scales. A snapshot: pack again after the table, the
        tags or the scales change (once per routing decision)."""
        shape = self._records_shape()
        if out is None:
            out = torch.empty(shape, dtype=torch.int32, device=self.device)
        self._check_records(out)
        self._track = ()     # records given by the caller: no automatic ones
        self._pack_records_into(out, stream)
        return out

    def _pack_records_into(self, out: torch.Tensor, stream: Optional[int]) -> None:
        s = current_stream_handle(self.device) if stream is None else stream
        saved = (self.args.page_desc, self.args.entry_records)
        N.pack_entry_records(self.args, out.data_ptr(), s)
        self.args.page_desc, self.args.entry_records = saved
        self._set_records(out)

    def _check_records(self, recs: torch.Tensor) -> None:
        shape = self._records_shape()
        if recs.dtype != torch.int32 or tuple(recs.shape) != shape:
            raise ValueError(f"entry records must be int32 {list(shape)}, got {recs.dtype} {tuple(recs.shape)}")
        if recs.device != self.device or not recs.is_contiguous() or recs.data_ptr() % 32:
            raise ValueError(f"entry records must be a contiguous, 32-byte aligned tensor on {self.device}")

    def use_records(self, recs: Optional[torch.Tensor]) -> None:
        """Read ``recs`` (packed for this plan's table, pages and pools) in place
        of the table entries, tags, tag map and scales; None goes back to them.
        Either way the plan stops packing records by itself."""
        self._track = ()
        self._set_records(recs)

    def _set_records(self, recs: Optional[torch.Tensor]) -> None:
        if recs is not None:
            self._check_records(recs)
        self._recs = recs
        self.args.entry_records = recs.data_ptr() if recs is not None else None

    def use_descriptors(self, desc: Optional[torch.Tensor]) -> None:
        """Read ``desc`` (packed for the same pages and pools) in place of the
        tags, tag map and scales; None goes back to them. The plan stops
        packing entry records by itself."""
        if desc is not None:
            _check_descriptors(desc, int(self.args.num_pages), self.device)
        self._track = ()
        if self._auto_state is not None:
            self._set_records(None)
            self._auto_state = None
        self._desc = desc
        self.args.page_desc = desc.data_ptr() if desc is not None else None

    def run(self, stream: Optional[int] = None, events: Optional[tuple] = None) -> None:
        """Launch on ``stream`` (default: torch's current stream). ``events``: an
        optional pair of torch.cuda.Event recorded around the split kernel alone."""
        s = current_stream_handle(self.device) if stream is None else stream
        if self._filled is not None:
            torch.cuda.ExternalStream(s, device=self.device).wait_event(self._filled)
            self._filled = None
        if self._track:
            self._auto_records(s)
        ev = None if events is None else (events[0].cuda_event, events[1].cuda_event)
        N.paged_decode(self.args, self._ws.data_ptr() if self._ws is not None else 0, self.workspace_bytes, s, ev)

    def _auto_records(self, stream: int) -> None:
        """Read packed entry records while the table, tags and scales stay as they
        were: packed (on ``stream``) at the second run that finds them unchanged,
        dropped as soon as one of them changes. The record buffer is the plan's
        for its lifetime and is packed again in place, so every pack and every
        run that reads it stay on one stream: a run on another stream turns the
        automatic records off for this plan."""
        tensors = [r() for r in self._track]
        if any(t is None for t in tensors) or (self._auto_stream is not None and stream != self._auto_stream):
            # a tracked tensor is gone, or the plan moved to another stream
            self._track = ()
            if self._auto_state is not None:
                self._set_records(None)
                self._auto_state = None
            return
        self._auto_stream = stream
        state = tuple(t._version for t in tensors)
        if self._auto_state is not None and state != self._auto_state:
            self._set_records(None)
            self._auto_state = None
        if self._auto_state is None and state == self._last_state:
            if self._auto_recs is None:
                self._auto_recs = torch.empty(self._records_shape(), dtype=torch.int32, device=self.device)
            self._pack_records_into(self._auto_recs, stream)
            self._auto_state = state
        self._last_state = state

    def invalidate_records(self) -> None:
        """Forget the automatically packed entry records (the table, tags or
        scales were written by means torch's version counters do not see)."""
        if self._auto_state is not None:
            self._set_records(None)
        self._auto_state = None
        self._last_state = None

    def run_with(self, q: torch.Tensor, out: torch.Tensor, stream: Optional[int] = None) -> None:
        """Run on ``stream`` (default: torch's current stream) with another query
        and output of the plan's shape and dtypes: q and out [B, Hq, D] or
        [B, Hq, 1, D], out with a unit last stride. A query the kernel cannot
        read in place (misaligned) is copied first."""
        a = self.args
        want = (a.batch, a.num_q_heads, a.head_dim)
        for name, t, dt in (("q", q, a.q_dtype), ("out", out, a.out_dtype)):
            shp = tuple(t.shape)
            if ((shp != want and shp != (want[0], want[1], 1, want[2])) or _DT.get(t.dtype) != dt
                    or t.device != self.device):
                raise ValueError(f"{name} must be {want} (or [B, H, 1, D]) of the plan's dtype and device, "
                                 f"got {t.dtype} {shp}")
        if out.stride(-1) != 1:
            raise ValueError("out must have a unit last stride")
        qvec = 4 if q.dtype == torch.float32 else 8
        if q.stride(-1) != 1 or q.data_ptr() % 16 or q.stride(0) % qvec or q.stride(1) % qvec:
            q = torch.empty(q.shape, dtype=q.dtype, device=q.device).copy_(q)
        with self._lock:   # the argument block is shared: set it and launch as one step
            a.q, a.q_stride_b, a.q_stride_h = q.data_ptr(), q.stride(0), q.stride(1)
            a.out, a.out_stride_b, a.out_stride_h = out.data_ptr(), out.stride(0), out.stride(1)
            self.out = out
            self.run(stream)

    @property
    def reads_records(self) -> bool:
        """True when the next run reads entry records (packed by ``pack_records``
        or automatically)."""
        return self._recs is not None


class PlanCache:
    """Decode plans of repeated calls over the same pool, table and tag tensors,
    for the reference entry points (which validate and allocate on every call).

    A plan is found by the identity of its key tensors (held as weak
    references, so the cache keeps no pool alive) plus the call's other
    settings, the current stream among them (a plan's workspace is reused by
    every run, which is safe only in one stream's order); each hit re-points
    the plan at the call's query and output (``DecodePlan.run_with``). Only
    plans that read the caller's tensors in place are cached: a plan that had
    to copy one (non-contiguous metadata) would not see later writes to it.
    At most ``size`` plans, least recently used first out."""

    def __init__(self, size: int = 8) -> None:
        self.size = size
        self._d: "OrderedDict[tuple, tuple]" = OrderedDict()

    def clear(self) -> None:
        self._d.clear()

    def get(self, tensors: tuple, extra: tuple) -> Optional["DecodePlan"]:
        key = (tuple(map(id, tensors)), extra)
        ent = self._d.get(key)
        if ent is None:
            return None
        refs, plan = ent
        for r, t in zip(refs, tensors):
            if (r() if r is not None else None) is not t:
                del self._d[key]
                return None
        self._d.move_to_end(key)
        return plan

    def put(self, tensors: tuple, extra: tuple, plan: "DecodePlan") -> None:
        if not plan.reads_in_place:
            return
        plan._keep = ()        # the caller's tensors: weak references only
        self._d[(tuple(map(id, tensors)), extra)] = (
            tuple(weakref.ref(t) if t is not None else None for t in tensors), plan)
        while len(self._d) > self.size:
            self._d.popitem(last=False)
