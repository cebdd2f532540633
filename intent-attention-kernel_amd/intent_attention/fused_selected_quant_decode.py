"""Fused selected-quant decode: the reference's operator API on the HIP kernel.

Interface of the reference's fused_selected_quant_decode.py:
``FusedKVPrecision`` (:29-34), ``FusedDecodeConfig`` (:42-49),
``metadata_to_kernel_tensors`` (:344-400), ``fused_selected_quant_decode``
(:408-464) and ``fake_int8_pages_from_fp16`` (:521-542).

``fused_selected_quant_decode`` keeps the reference signature, argument
meaning, output (new [B, H, 1, D] float16 tensor) and ValueError on a
head_dim mismatch. Differences, by design:

* It computes on the MI355X kernel only. Host tensors raise RuntimeError
  instead of running a CPU loop (the CPU restatement lives in the test
  oracle), and so does a missing libiak.so.
* Extensions are keyword-only and default off: GQA (a page table of
  ``[B, Hkv, W]`` rows shared by ``H // Hkv`` query heads) and native page
  pools for FP8 / INT4 / INT4_RESIDUAL (tags 3 / 4 / 5, appended to the
  fused numbering). Without those pools tags other than FP16 / INT8 / SKIP
  contribute nothing, as the reference's ``else: continue`` (:316-317).
* Page counts are clamped to the table width (the Triton kernel's
  ``tl.minimum``, :126; the CPU loop would raise IndexError) and page ids are
  read with torch's indexing rule (an id in [-NP, 0) is id + NP); ids
  outside the pool contribute nothing instead of faulting.
* Repeated calls over the same pool, table, tag and count tensors reuse the
  validated launch plan (``decode_core.PlanCache``: tensors found by
  identity, held weakly); each call still returns a new output. From the
  plan's second run over unchanged tables, tags and scales the decode reads
  packed entry records (bit-identical results; torch's version counters of
  those tensors invalidate them).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from enum import IntEnum
from typing import Dict, Optional, Tuple

import numpy as np
import torch

from . import _native as N
from .decode_core import PagePools, PlanCache, current_stream_handle, make_plan


class FusedKVPrecision(IntEnum):
    """Per-page precision tags (FP16 / INT8 / SKIP as the reference, native tags appended)."""

    FP16 = 0
    INT8 = 1
    SKIP = 2
    FP8 = 3
    INT4 = 4
    INT4_RESIDUAL = 5


@dataclass(frozen=True)
class FusedDecodeConfig:
    page_size: int = 16
    head_dim: int = 64
    max_selected_pages: int = 64
    block_d: int = 64


def is_triton_available() -> bool:
    """This build has no Triton path; kept so reference call sites keep working."""
    return False


def is_cuda_available() -> bool:
    return torch.cuda.is_available()


def is_native_available() -> bool:
    """True when a ROCm device is visible and libiak.so loads."""
    if not torch.cuda.is_available():
        return False
    try:
        N.load()
        return True
    except RuntimeError:
        return False


_NAME_TO_TAG = {"SKIP": FusedKVPrecision.SKIP, "INT8": FusedKVPrecision.INT8}
_NATIVE_NAME_TO_TAG = {"FP8": FusedKVPrecision.FP8, "INT4": FusedKVPrecision.INT4,
                       "INT4_RESIDUAL": FusedKVPrecision.INT4_RESIDUAL}


def precision_tag(name: str, native_precisions: bool = False) -> int:
    """Precision name -> page tag as metadata_to_kernel_tensors maps it
    (fused_selected_quant_decode.py:379-389): "SKIP" -> SKIP, "INT8" / "INT4" /
    "INT4_RESIDUAL" -> INT8, anything else (FP8 included) -> FP16; with
    ``native_precisions`` FP8 / INT4 / INT4_RESIDUAL keep their native tags."""
    name = getattr(name, "value", name)          # KVPrecision members or their names
    tag = _NAME_TO_TAG.get(name, FusedKVPrecision.FP16)
    if name in _NATIVE_NAME_TO_TAG:
        tag = _NATIVE_NAME_TO_TAG[name] if native_precisions else (
            FusedKVPrecision.INT8 if name != "FP8" else FusedKVPrecision.FP16)
    return int(tag)


def metadata_to_kernel_tensors(meta: Dict, num_pages: int, B: int = 1, H: int = 1,
                               config: Optional[FusedDecodeConfig] = None,
                               device: Optional[torch.device] = None, *,
                               native_precisions: bool = False
                               ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Router metadata -> (page_table [B,H,max_sel], page_precision [num_pages], page_counts [B,H]) int32.

    Reference mapping: "SKIP" -> SKIP; "INT8", "INT4", "INT4_RESIDUAL" -> INT8;
    every other name (including "FP8") -> FP16; keys that are not integers are
    ignored; the id list is truncated to max_selected_pages and broadcast to
    every (b, h). ``native_precisions=True`` maps FP8 / INT4 / INT4_RESIDUAL to
    their native tags instead. Built with numpy in O(num_pages + B*H*max_sel).
    """
    cfg = config or FusedDecodeConfig()
    width = cfg.max_selected_pages
    prec = np.full((num_pages,), int(FusedKVPrecision.FP16), dtype=np.int32)
    for key, name in meta.get("block_precision_by_page", {}).items():
        try:
            pid = int(key)
        except ValueError:
            continue
        prec[pid] = precision_tag(name, native_precisions)
    ids = np.asarray(meta.get("selected_page_ids", []), dtype=np.int64)[:width].astype(np.int32)
    table = np.zeros((B, H, width), dtype=np.int32)
    table[:, :, : ids.size] = ids
    counts = np.full((B, H), ids.size, dtype=np.int32)
    dev = device if device is not None else torch.device("cpu")
    return (torch.from_numpy(table).to(dev), torch.from_numpy(prec).to(dev),
            torch.from_numpy(counts).to(dev))


def _tag_map(pools: PagePools) -> Tuple[int, ...]:
    m = [N.TAG_FP16, N.TAG_INT8, N.TAG_SKIP, N.TAG_SKIP, N.TAG_SKIP, N.TAG_SKIP, N.TAG_SKIP, N.TAG_SKIP]
    for tag in (N.TAG_FP8, N.TAG_INT4, N.TAG_INT4_RESIDUAL):
        if pools.has(tag):
            m[tag] = tag
    return tuple(m)


def fused_selected_quant_decode(
    query: torch.Tensor,
    k_pages_fp16: torch.Tensor,
    v_pages_fp16: torch.Tensor,
    k_pages_int8: torch.Tensor,
    v_pages_int8: torch.Tensor,
    k_scales: torch.Tensor,
    v_scales: torch.Tensor,
    page_table: torch.Tensor,
    page_precision: torch.Tensor,
    page_counts: torch.Tensor,
    config: FusedDecodeConfig = FusedDecodeConfig(),
    *,
    native_pools: Optional[PagePools] = None,
    pages_per_split: int = 0,
) -> torch.Tensor:
    """Selected-page decode attention: returns a new [B, H, 1, D] float16 tensor.

    query [B, H, 1, D]; page pools [num_pages, page_size, D]; k/v_scales
    [num_pages] (float16 or float32); page_table [B, H or Hkv, W] int32;
    page_precision [num_pages] int32 (FusedKVPrecision); page_counts
    [B, H or Hkv] int32. ``native_pools`` supplies FP8 / INT4 /
    INT4_RESIDUAL pools (their FP16 / INT8 fields are ignored).
    """
    B, H, _, D = query.shape
    if D != config.head_dim:
        raise ValueError(f"head_dim {D} != config.head_dim {config.head_dim}")
    if query.shape[2] != 1:
        raise ValueError(f"query must have shape [B, H, 1, D] (single-token decode), got {tuple(query.shape)}")
    if config.page_size != k_pages_fp16.shape[1]:
        raise ValueError(f"page_size mismatch: config {config.page_size} vs pages {k_pages_fp16.shape[1]}")
    tensors = (k_pages_fp16, v_pages_fp16, k_pages_int8, v_pages_int8, k_scales, v_scales, page_table,
               page_precision, page_counts)
    if native_pools is not None:
        tensors += tuple(getattr(native_pools, n) for n in _NATIVE_FIELDS)
    stream = current_stream_handle(query.device) if query.is_cuda else None
    extra = (B, H, D, query.dtype, query.device, stream, config,
             pages_per_split, None if native_pools is None else native_pools.int4_group)
    out = torch.empty((B, H, 1, D), dtype=torch.float16, device=query.device)
    plan = _PLANS.get(tensors, extra)
    if plan is not None:
        # the same pools, table, tags and counts as an earlier call: only the query and output are new
        plan.run_with(query, out, stream)
        return out
    pools = PagePools(k_fp16=k_pages_fp16, v_fp16=v_pages_fp16, k_int8=k_pages_int8, v_int8=v_pages_int8,
                      k_int8_scale=k_scales, v_int8_scale=v_scales)
    if native_pools is not None:
        for name in _NATIVE_FIELDS + ("int4_group",):
            setattr(pools, name, getattr(native_pools, name))
    plan = make_plan(query[:, :, 0, :], pools, page_table, page_counts, page_precision,
                     tag_map=_tag_map(pools), negative_ids=True, sm_scale=1.0 / math.sqrt(D),
                     out=out[:, :, 0, :], pages_per_split=pages_per_split)
    plan.run()
    _PLANS.put(tensors, extra, plan)
    return out


_NATIVE_FIELDS = ("k_fp8", "v_fp8", "k_fp8_scale", "v_fp8_scale", "k_int4", "v_int4", "k_int4_scale",
                  "v_int4_scale", "k_int4r", "v_int4r", "k_int4r_scale", "v_int4r_scale")
# validated plans of earlier calls (see decode_core.PlanCache); clear_plan_cache() empties it
_PLANS = PlanCache()


def clear_plan_cache() -> None:
    """Drop the validated plans ``fused_selected_quant_decode`` keeps for repeated calls."""
    _PLANS.clear()


def fused_selected_quant_decode_reference(
    query: torch.Tensor,
    k_pages_fp16: torch.Tensor,
    v_pages_fp16: torch.Tensor,
    k_pages_int8: torch.Tensor,
    v_pages_int8: torch.Tensor,
    k_scales: torch.Tensor,
    v_scales: torch.Tensor,
    page_table: torch.Tensor,
    page_precision: torch.Tensor,
    page_counts: torch.Tensor,
    config: FusedDecodeConfig,
) -> torch.Tensor:
    """The reference's correctness entry point (fused_selected_quant_decode.py:267-336),
    same signature (``config`` required) and result: [B, H, 1, D] float16 of
    the per-(b, h) online-softmax loop over the listed pages. Here it is the
    same computation as ``fused_selected_quant_decode``, on the MI355X kernel:
    device tensors only (host tensors raise RuntimeError; the CPU restatement
    of the loop is test code in ``oracle/``, not a product path)."""
    return fused_selected_quant_decode(query, k_pages_fp16, v_pages_fp16, k_pages_int8, v_pages_int8, k_scales,
                                       v_scales, page_table, page_precision, page_counts, config)


def fake_int8_pages_from_fp16(pages: torch.Tensor, eps: float = 1e-6) -> Tuple[torch.Tensor, torch.Tensor]:
    """[num_pages, page_size, D] float16 -> (int8 codes, float16 scales [num_pages]).

    Per-page absmax in float16 arithmetic, clamp(min=eps), /127, round half
    even, clamp(-128, 127) -- the arithmetic of the reference's function of
    the same name in this module (:521-542); the division is a true division
    on every device.
    """
    if (pages.is_cuda and eps == 1e-6 and pages.dtype == torch.float16 and pages.dim() == 3
            and pages.shape[1] == 16 and pages.shape[2] in (64, 128)):
        from .quantize import fake_int8_pages_device
        return fake_int8_pages_device(pages, "fused")        # the same arithmetic on the HIP quantiser
    n = pages.shape[0]
    flat = pages.view(n, -1)
    absmax = flat.abs().amax(dim=1, keepdim=True).clamp(min=eps)
    scales = absmax / torch.full((1,), 127.0, dtype=absmax.dtype, device=absmax.device)
    q = (flat / scales).round().clamp(-128, 127).to(torch.int8)
    return q.view(pages.shape), scales.squeeze(-1)
