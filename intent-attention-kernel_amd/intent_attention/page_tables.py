"""Kernel page tables from routing decisions, built on the GPU
(``iak_build_page_tables`` in libiak.so).

``routing_to_kernel_tensors(routed_blocks, page_size, num_pages, B, H, config)``
returns what the reference computes in two host steps,
``metadata_to_kernel_tensors(routing_to_kernel_metadata(routed_blocks,
page_size), num_pages, B, H, config)`` (block_router.py:383-421,
fused_selected_quant_decode.py:344-400): ``page_table [B, H, W]`` (the selected
pages in routed order, each page once, truncated to
``config.max_selected_pages`` and zero-filled), ``page_precision [num_pages]``
(the first selecting block's precision, FP16 elsewhere) and
``page_counts [B, H]``, all int32 on the device. Two generalisations the
decode's tables need: ``routed_blocks`` may hold one routing per sequence
(``B`` lists, each broadcast over that sequence's ``H`` KV heads), and
``block_table [B, n_logical]`` maps each sequence's logical pages to physical
pool pages (a negative entry or a page past the row: not resident, dropped).

``build_page_tables`` is the raw builder over span arrays (start, end, tag per
selected block; CSR offsets per list) for callers that keep routing results
on the device.
"""
from __future__ import annotations

from typing import List, Optional, Sequence, Tuple, Union

import numpy as np
import torch

from . import _native as N
from .block_router import RoutedBlock, _SELECTING
from .decode_core import current_stream_handle
from .fused_selected_quant_decode import FusedDecodeConfig, FusedKVPrecision, precision_tag

__all__ = ["build_page_tables", "routing_to_kernel_tensors"]

_I32_MAX = 2 ** 31 - 1


def _i32(x, dev: torch.device, what: str) -> torch.Tensor:
    if isinstance(x, torch.Tensor):
        if x.dtype != torch.int32:
            raise ValueError(f"{what} must be int32, got {x.dtype}")
        t = x.to(dev)
    else:
        a = np.asarray(x, dtype=np.int64).reshape(-1)
        if a.size and (a.min() < -2 ** 31 or a.max() > _I32_MAX):
            raise ValueError(f"{what} does not fit int32")
        t = torch.from_numpy(a.astype(np.int32)).to(dev)
    if t.numel() == 0:                       # a valid pointer for an empty array
        t = torch.zeros(1, dtype=torch.int32, device=dev)
    return t.contiguous()


def build_page_tables(span_offsets, span_begin, span_end, span_tag, *, num_rows: int, table_width: int,
                      page_size: int, num_pages: int, rows_per_seq: int = 1, rows_per_list: Optional[int] = None,
                      block_table: Optional[torch.Tensor] = None, dedupe: bool = True, precision: bool = True,
                      default_tag: int = int(FusedKVPrecision.FP16), device: Optional[torch.device] = None
                      ) -> Tuple[torch.Tensor, Optional[torch.Tensor], torch.Tensor]:
    """(page_table [num_rows, table_width], page_precision [num_pages] or None,
    page_counts [num_rows]) int32 on the device.

    Row ``r`` reads span list ``r // rows_per_list`` (default: one list for all
    rows) and block-table row ``r // rows_per_seq``. ``span_offsets`` has one
    entry per list plus one (CSR into ``span_begin / span_end / span_tag``).
    Host sequences are uploaded; device tensors are used in place.
    """
    if device is None:
        cands = [t for t in (span_offsets, span_begin, span_end, span_tag, block_table)
                 if isinstance(t, torch.Tensor)]
        device = cands[0].device if cands else None
    if device is None or torch.device(device).type != "cuda":
        raise RuntimeError("page tables are built by the MI355X HIP kernel: pass a ROCm device "
                           "(the CPU restatement is test code, not a fallback)")
    dev = torch.device(device)
    N.load()
    rpl = num_rows if rows_per_list is None else rows_per_list
    if num_rows < 0 or table_width < 0 or num_pages < 0 or page_size <= 0 or rows_per_seq <= 0 or rpl < 0:
        raise ValueError("num_rows / table_width / num_pages must be >= 0, page_size and rows_per_* positive")
    rpl = max(rpl, 1)
    n_lists = (num_rows + rpl - 1) // rpl
    n_seqs = (num_rows + rows_per_seq - 1) // rows_per_seq

    off_host = span_offsets.cpu().numpy() if isinstance(span_offsets, torch.Tensor) else np.asarray(span_offsets)
    off_host = off_host.reshape(-1).astype(np.int64)
    n_spans = len(span_begin) if not isinstance(span_begin, torch.Tensor) else span_begin.numel()
    if off_host.size < n_lists + 1:
        raise ValueError(f"span_offsets needs {n_lists + 1} entries for {num_rows} rows, got {off_host.size}")
    if off_host.size and (off_host[0] < 0 or np.any(np.diff(off_host) < 0) or off_host[-1] > n_spans):
        raise ValueError("span_offsets must be non-decreasing, start at >= 0 and end within the span arrays")
    for name, t in (("span_end", span_end), ("span_tag", span_tag)):
        if (t.numel() if isinstance(t, torch.Tensor) else len(t)) != n_spans:
            raise ValueError(f"{name} must have as many entries as span_begin ({n_spans})")

    offs, beg, end, tag = (_i32(x, dev, w) for x, w in ((span_offsets, "span_offsets"), (span_begin, "span_begin"),
                                                        (span_end, "span_end"), (span_tag, "span_tag")))
    bt = None
    if block_table is not None:
        if not isinstance(block_table, torch.Tensor) or block_table.dim() != 2:
            raise ValueError("block_table must be a 2-D int32 tensor [num_seqs, n_logical]")
        if block_table.shape[0] < n_seqs or block_table.shape[1] == 0:
            raise ValueError(f"block_table needs >= {n_seqs} rows and >= 1 column, got {tuple(block_table.shape)}")
        bt = _i32(block_table, dev, "block_table")
    table = torch.empty((num_rows, table_width), dtype=torch.int32, device=dev)
    counts = torch.empty((num_rows,), dtype=torch.int32, device=dev)
    prec = torch.empty((num_pages,), dtype=torch.int32, device=dev) if precision else None
    a = N.PageTableArgs()
    a.num_rows, a.rows_per_seq, a.rows_per_list = num_rows, rows_per_seq, rpl
    a.table_width, a.page_size, a.num_pages = table_width, page_size, num_pages
    a.dedupe, a.default_tag = int(bool(dedupe)), int(default_tag)
    a.block_table_width = int(block_table.shape[1]) if bt is not None else 0
    a.span_offsets, a.span_begin, a.span_end, a.span_tag = (t.data_ptr() for t in (offs, beg, end, tag))
    a.block_table = bt.data_ptr() if bt is not None else None
    a.page_table = table.data_ptr() if table.numel() else None
    a.page_counts = counts.data_ptr() if counts.numel() else None
    a.page_precision = prec.data_ptr() if prec is not None and prec.numel() else None
    N.build_page_tables(a, current_stream_handle(dev))
    return table, prec, counts


def _spans(routed: Sequence[RoutedBlock], native_precisions: bool):
    sel = [b for b in routed if b.decision in _SELECTING]          # block_router.py:276-278
    return ([int(b.start) for b in sel], [int(b.end) for b in sel],
            [precision_tag(b.precision, native_precisions) for b in sel])


def routing_to_kernel_tensors(routed_blocks: Union[List[RoutedBlock], List[List[RoutedBlock]]], page_size: int,
                              num_pages: int, B: int = 1, H: int = 1, config: Optional[FusedDecodeConfig] = None,
                              device: Optional[torch.device] = None, *, native_precisions: bool = False,
                              block_table: Optional[torch.Tensor] = None
                              ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Routing decisions -> (page_table [B, H, W], page_precision [num_pages],
    page_counts [B, H]) int32 on the GPU.

    ``routed_blocks``: one routing (a list of RoutedBlock, broadcast to every
    (b, h) as the reference does) or ``B`` routings (one per sequence).
    Without ``block_table`` a selected page at or past ``num_pages`` raises
    IndexError, as the reference's precision assignment does.
    """
    cfg = config or FusedDecodeConfig()
    per_seq = len(routed_blocks) > 0 and not isinstance(routed_blocks[0], RoutedBlock)
    lists = list(routed_blocks) if per_seq else [routed_blocks]
    if per_seq and len(lists) != B:
        raise ValueError(f"{len(lists)} routings for batch {B}")
    begin, end, tags, offs = [], [], [], [0]
    for lst in lists:
        s, e, t = _spans(lst, native_precisions)
        begin += s
        end += e
        tags += t
        offs.append(len(begin))
    if any(x < 0 for x in begin):
        raise ValueError("selected blocks must start at token >= 0 (BlockLayout.validate)")
    if block_table is None:
        last = max(((e - 1) // page_size for s, e in zip(begin, end) if e > s), default=-1)
        if last >= num_pages:
            raise IndexError(f"selected page {last} is out of bounds for {num_pages} pages")
    dev = torch.device(device) if device is not None else (block_table.device if block_table is not None else None)
    table, prec, counts = build_page_tables(
        offs, begin, end, tags, num_rows=B * H, table_width=cfg.max_selected_pages, page_size=page_size,
        num_pages=num_pages, rows_per_seq=H, rows_per_list=H if per_seq else B * H, block_table=block_table,
        device=dev)
    return table.view(B, H, -1), prec, counts.view(B, H)
