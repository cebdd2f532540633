"""Second decode API of the reference, on the HIP kernel.

Interface of the reference's triton_intent_quant_attention.py:
``TritonKVPrecision`` (:40-48), ``IntentQuantKernelConfig`` (:51-58),
``_validate_decode_inputs`` (:93-123), ``make_page_tables_from_selected_pages``
(:126-203), ``intent_quant_decode_attention_triton`` (:342-457),
``fake_int8_pages_from_fp16`` (:460-496) and ``make_precision_tensor``
(:499-536). Validation order and error messages follow the reference (its
tests match on them). The compute is libiak's paged decode; nothing here
uses Triton (the module that keeps the reference's import path,
``triton_intent_quant_attention``, re-exports these names).

Semantics kept from the reference kernel (:255-335): q [B, H, D] in, output
of q's dtype; tag 0 reads the FP16 pool; every other tag but 5 (SKIP) -- 1-4
(FP8, INT8, INT4, INT4_RESIDUAL), 6, 7, negative or larger tags -- reads the
INT8 pool with the per-page scale (:281-307), except that tags 1, 3 and 4
read their native pools when those are passed; tag 5 or a negative page id
contributes nothing; a row with nothing visited gives 0.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from enum import IntEnum
from typing import Optional, Tuple

import torch

from . import _native as N
from .decode_core import PagePools, PlanCache, current_stream_handle, make_plan


class TritonKVPrecision(IntEnum):
    """Integer precision tags of this API (numbering of the reference)."""

    FP16 = 0
    FP8 = 1
    INT8 = 2
    INT4 = 3
    INT4_RESIDUAL = 4
    SKIP = 5


@dataclass(frozen=True)
class IntentQuantKernelConfig:
    page_size: int = 16
    head_dim: int = 64
    max_selected_pages: int = 64
    block_d: int = 64


def is_triton_available() -> bool:
    return False


def is_cuda_available() -> bool:
    return torch.cuda.is_available()


def _require_device_kernel() -> None:
    if not torch.cuda.is_available():
        raise RuntimeError(
            "CUDA is not available: the IntentQuant decode kernel needs a ROCm (MI355X) device. "
            "CPU reference paths remain available in the test oracle.")
    N.load()


def _validate_decode_inputs(q, page_ids, page_count, page_precision, out) -> None:
    if q.ndim != 3:
        raise ValueError(f"q must have shape [B, H, D], got {tuple(q.shape)}")
    if page_ids.ndim != 3:
        raise ValueError(f"page_ids must have shape [B, H, max_selected_pages], got {tuple(page_ids.shape)}")
    if page_count.ndim != 2:
        raise ValueError(f"page_count must have shape [B, H], got {tuple(page_count.shape)}")
    if page_precision.ndim != 1:
        raise ValueError(f"page_precision must have shape [num_pages], got {tuple(page_precision.shape)}")
    # GQA extension: a page-id row may serve H // Hkv query heads.
    heads_ok = page_ids.shape[1] == q.shape[1] or (page_ids.shape[1] > 0 and q.shape[1] % page_ids.shape[1] == 0)
    if page_ids.shape[0] != q.shape[0] or not heads_ok:
        raise ValueError("page_ids batch/head dimensions must match q")
    if page_count.shape[0] != q.shape[0] or page_count.shape[1] != page_ids.shape[1]:
        raise ValueError("page_count batch/head dimensions must match q")
    if out is not None and out.shape != q.shape:
        raise ValueError(f"out must have shape {tuple(q.shape)}, got {tuple(out.shape)}")


def make_page_tables_from_selected_pages(selected_pages: torch.Tensor, batch: int, heads: int,
                                         max_selected_pages: Optional[int] = None
                                         ) -> Tuple[torch.Tensor, torch.Tensor]:
    """[N] (shared) or [B, H, N] page ids -> (-1 padded [B, H, W] int32, counts [B, H] int32)."""
    if selected_pages.ndim not in (1, 3):
        raise ValueError("selected_pages must have shape [N] or [B, H, N]")
    if selected_pages.ndim == 3 and (selected_pages.shape[0] != batch or selected_pages.shape[1] != heads):
        raise ValueError("selected_pages [B, H, N] must match batch and heads")
    n = selected_pages.shape[-1]
    width = max_selected_pages or n
    if n > width:
        what = "length" if selected_pages.ndim == 1 else "width"
        raise ValueError(f"selected_pages {what} exceeds max_selected_pages")
    dev = selected_pages.device
    ids = torch.full((batch, heads, width), -1, dtype=torch.int32, device=dev)
    src = selected_pages.to(torch.int32)
    ids[:, :, :n] = src.view(1, 1, n) if selected_pages.ndim == 1 else src
    return ids, torch.full((batch, heads), n, dtype=torch.int32, device=dev)


def intent_quant_decode_attention_triton(
    q: torch.Tensor,
    k_pages_fp16: torch.Tensor,
    v_pages_fp16: torch.Tensor,
    k_pages_i8: torch.Tensor,
    v_pages_i8: torch.Tensor,
    k_i8_scales: torch.Tensor,
    v_i8_scales: torch.Tensor,
    page_ids: torch.Tensor,
    page_count: torch.Tensor,
    page_precision: torch.Tensor,
    *,
    config: Optional[IntentQuantKernelConfig] = None,
    out: Optional[torch.Tensor] = None,
    native_pools: Optional[PagePools] = None,
    pages_per_split: int = 0,
) -> torch.Tensor:
    """Single-token decode over selected pages; returns out [B, H, D] (q's dtype)."""
    _require_device_kernel()
    cfg = config or IntentQuantKernelConfig()
    _validate_decode_inputs(q, page_ids, page_count, page_precision, out)
    if not q.is_cuda:
        raise ValueError("q must be a CUDA tensor")
    bsz, heads, dim = q.shape
    if dim != cfg.head_dim:
        raise ValueError(f"q head_dim={dim} does not match config.head_dim={cfg.head_dim}")
    if cfg.block_d < dim:
        raise ValueError("This prototype expects block_d >= head_dim so one program handles the full head.")
    if k_pages_fp16.shape != v_pages_fp16.shape:
        raise ValueError("k_pages_fp16 and v_pages_fp16 must have the same shape")
    if k_pages_i8.shape != v_pages_i8.shape:
        raise ValueError("k_pages_i8 and v_pages_i8 must have the same shape")
    if k_pages_fp16.ndim != 3:
        raise ValueError("page tensors must have shape [num_pages, page_size, D]")
    if k_pages_fp16.shape[1] != cfg.page_size:
        raise ValueError("page_size mismatch")
    if k_pages_fp16.shape[2] != dim:
        raise ValueError("page head_dim mismatch")
    if page_ids.shape[2] != cfg.max_selected_pages:
        raise ValueError("page_ids width must match config.max_selected_pages")
    if out is None:
        out = torch.empty_like(q)
    tensors = (k_pages_fp16, v_pages_fp16, k_pages_i8, v_pages_i8, k_i8_scales, v_i8_scales, page_ids, page_count,
               page_precision)
    if native_pools is not None:
        tensors += tuple(getattr(native_pools, n) for n in _NATIVE_FIELDS)
    stream = current_stream_handle(q.device) if q.is_cuda else None
    extra = (bsz, heads, dim, q.dtype, out.dtype, q.device, stream, cfg,
             pages_per_split, None if native_pools is None else native_pools.int4_group)
    plan = _PLANS.get(tensors, extra)
    if plan is not None:
        # the same pools, ids, counts and tags as an earlier call: only q and out are new
        plan.run_with(q, out, stream)
        return out

    pools = PagePools(k_fp16=k_pages_fp16, v_fp16=v_pages_fp16, k_int8=k_pages_i8, v_int8=v_pages_i8,
                      k_int8_scale=k_i8_scales, v_int8_scale=v_i8_scales)
    # caller tag -> native tag: all but 0 and 5 read INT8 (tags outside [0, 8) take
    # slot 7's) unless a native pool is given for 1, 3 or 4
    tag_map = [N.TAG_FP16, N.TAG_INT8, N.TAG_INT8, N.TAG_INT8, N.TAG_INT8, N.TAG_SKIP, N.TAG_INT8, N.TAG_INT8]
    if native_pools is not None:
        for name in ("k_fp8", "v_fp8", "k_fp8_scale", "v_fp8_scale", "k_int4", "v_int4", "k_int4_scale",
                     "v_int4_scale", "int4_group", "k_int4r", "v_int4r", "k_int4r_scale", "v_int4r_scale"):
            setattr(pools, name, getattr(native_pools, name))
        for caller, native in ((TritonKVPrecision.FP8, N.TAG_FP8), (TritonKVPrecision.INT4, N.TAG_INT4),
                               (TritonKVPrecision.INT4_RESIDUAL, N.TAG_INT4_RESIDUAL)):
            if pools.has(native):
                tag_map[int(caller)] = native
    plan = make_plan(q, pools, page_ids, page_count, page_precision, tag_map=tag_map,
                     negative_ids=False, sm_scale=1.0 / math.sqrt(dim), out=out,
                     pages_per_split=pages_per_split, map_other_tags=True)
    plan.run()
    _PLANS.put(tensors, extra, plan)
    return out


_NATIVE_FIELDS = ("k_fp8", "v_fp8", "k_fp8_scale", "v_fp8_scale", "k_int4", "v_int4", "k_int4_scale",
                  "v_int4_scale", "k_int4r", "v_int4r", "k_int4r_scale", "v_int4r_scale")
# validated plans of earlier calls (decode_core.PlanCache); clear_plan_cache() empties it
_PLANS = PlanCache()


def clear_plan_cache() -> None:
    """Drop the validated plans ``intent_quant_decode_attention_triton`` keeps for repeated calls."""
    _PLANS.clear()


def fake_int8_pages_from_fp16(pages: torch.Tensor, *, eps: float = 1e-6) -> Tuple[torch.Tensor, torch.Tensor]:
    """[num_pages, page_size, D] -> (int8 codes, float32 scales [num_pages]); float32
    arithmetic, clamp_min(eps), /127, round half even, clamp(-127, 127)."""
    if pages.ndim != 3:
        raise ValueError("pages must have shape [num_pages, page_size, D]")
    if (pages.is_cuda and eps == 1e-6 and pages.dtype == torch.float16 and pages.shape[1] == 16
            and pages.shape[2] in (64, 128)):
        from .quantize import fake_int8_pages_device
        return fake_int8_pages_device(pages, "triton")       # the same arithmetic on the HIP quantiser
    n = pages.shape[0]
    flat = pages.float().reshape(n, -1)
    scales = flat.abs().amax(dim=1).clamp_min(eps) / torch.full((1,), 127.0, device=flat.device)
    q = torch.round(flat / scales[:, None]).clamp(-127, 127).to(torch.int8)
    return q.reshape_as(pages), scales.to(torch.float32)


def make_precision_tensor(num_pages: int, fp16_pages: Optional[torch.Tensor] = None,
                          int8_pages: Optional[torch.Tensor] = None, *,
                          device: Optional[torch.device] = None) -> torch.Tensor:
    """int32 [num_pages] tags, INT8 by default, FP16 / INT8 at the given ids."""
    prec = torch.full((num_pages,), int(TritonKVPrecision.INT8), dtype=torch.int32, device=device)
    if fp16_pages is not None:
        prec[fp16_pages.to(device=device, dtype=torch.long)] = int(TritonKVPrecision.FP16)
    if int8_pages is not None:
        prec[int8_pages.to(device=device, dtype=torch.long)] = int(TritonKVPrecision.INT8)
    return prec
