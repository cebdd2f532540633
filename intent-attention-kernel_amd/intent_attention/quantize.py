"""Quantise-on-write of float16 K/V pages into the decode's page pools, on the
MI355X (``iak_quantize_pages``, include/iak.h), bit-exact to the reference's
arithmetic:

* ``quantize_pages(pages, precision)`` -- fake_quantize_tensor
  (intent_quant.py:221-312) at the page granule (INT4: page x ``int4_group``
  channels), returning the pool codes (FP8 e4m3fn bytes, INT8, packed INT4,
  packed INT4_RESIDUAL) and scales;
* ``fake_int8_pages_device(pages, variant)`` -- the two reference functions
  named ``fake_int8_pages_from_fp16`` (fused: float16 arithmetic,
  fused_selected_quant_decode.py:521-542; triton: float32,
  triton_intent_quant_attention.py:460-496).

Codes can be written in place into an existing pool at chosen page ids
(``codes=``, ``scales=``, ``dst_pages=``). Device tensors only.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _native as N
from .decode_core import PAGE_SIZE, current_stream_handle, require_device

_PREC = {"FP8": N.TAG_FP8, "INT8": N.TAG_INT8, "INT4": N.TAG_INT4, "INT4_RESIDUAL": N.TAG_INT4_RESIDUAL}


def _launch(pages: torch.Tensor, tag: int, mode: int, codes: torch.Tensor, scales: torch.Tensor,
            dst_pages: Optional[torch.Tensor], int4_group: int) -> None:
    a = N.QuantizeArgs()
    a.num_pages, a.page_size, a.head_dim = pages.shape[0], pages.shape[1], pages.shape[2]
    a.src = pages.data_ptr()
    a.dst_pages = None if dst_pages is None else dst_pages.data_ptr()
    a.pool_pages = codes.shape[0]
    a.precision, a.mode, a.int4_group = tag, mode, int4_group
    a.codes, a.scales = codes.data_ptr(), scales.data_ptr()
    a.scale_dtype = N.DTYPE_F32 if scales.dtype == torch.float32 else N.DTYPE_F16
    N.quantize_pages(a, current_stream_handle(pages.device))
    # the kernel writes through raw pointers: tell torch's version counters (decode
    # plans that packed these scales into entry records see the change)
    torch.autograd.graph.increment_version([codes, scales])


def _check_pages(pages: torch.Tensor) -> torch.Tensor:
    if pages.dim() != 3 or pages.shape[1] != PAGE_SIZE or pages.dtype != torch.float16:
        raise ValueError(f"pages must be float16 [num_pages, {PAGE_SIZE}, D], got {pages.dtype} "
                         f"{tuple(pages.shape)}")
    return pages.contiguous()


def quantize_pages(pages: torch.Tensor, precision: str, *, int4_group: int = 32,
                   codes: Optional[torch.Tensor] = None, scales: Optional[torch.Tensor] = None,
                   dst_pages: Optional[torch.Tensor] = None,
                   scale_dtype: torch.dtype = torch.float16) -> Tuple[torch.Tensor, torch.Tensor]:
    """Pool codes and scales of ``pages`` [n, 16, D] float16 (see the module docstring).

    Without ``codes``/``scales`` new tensors of n pages are returned: codes
    [n, 16, D] (uint8 FP8 / int8 INT8 / uint8 INT4_RESIDUAL) or [n, 16, D/2]
    uint8 (INT4); scales [n] (FP8, INT8), [n, D/int4_group] (INT4) or [n, 2]
    float32 (INT4_RESIDUAL). With them, page i is written to pool page
    ``dst_pages[i]`` (or i).
    """
    if precision not in _PREC:
        raise ValueError(f"precision must be one of {sorted(_PREC)}, got {precision!r}")
    require_device(pages, *(t for t in (codes, scales, dst_pages) if t is not None), what="page quantiser")
    pages = _check_pages(pages)
    n, ps, D = pages.shape
    tag = _PREC[precision]
    if codes is None:
        width = D // 2 if tag == N.TAG_INT4 else D
        cdt = torch.int8 if tag == N.TAG_INT8 else torch.uint8
        codes = torch.empty((n, ps, width), dtype=cdt, device=pages.device)
    if scales is None:
        if tag == N.TAG_INT4:
            scales = torch.empty((codes.shape[0], D // int4_group), dtype=scale_dtype, device=pages.device)
        elif tag == N.TAG_INT4_RESIDUAL:
            scales = torch.empty((codes.shape[0], 2), dtype=torch.float32, device=pages.device)
        else:
            scales = torch.empty(codes.shape[0], dtype=scale_dtype, device=pages.device)
    pool = codes.shape[0]
    width = D // 2 if tag == N.TAG_INT4 else D
    if tuple(codes.shape) != (pool, ps, width) or not codes.is_contiguous() or codes.element_size() != 1:
        raise ValueError(f"codes must be a contiguous one-byte pool [pool_pages, {ps}, {width}], "
                         f"got {codes.dtype} {tuple(codes.shape)}")
    want = {N.TAG_INT4: (pool, D // int4_group), N.TAG_INT4_RESIDUAL: (pool, 2)}.get(tag, (pool,))
    if tuple(scales.shape) != want or not scales.is_contiguous():
        raise ValueError(f"scales must be contiguous {want}, got {tuple(scales.shape)}")
    if scales.dtype not in (torch.float16, torch.float32):
        raise ValueError(f"scales must be float16 or float32, got {scales.dtype}")
    if tag == N.TAG_INT4_RESIDUAL and scales.dtype != torch.float32:
        raise ValueError("INT4_RESIDUAL scales are float32 [pool_pages, 2]")
    if dst_pages is not None:
        dst_pages = dst_pages.to(torch.int32).contiguous()
        if dst_pages.shape != (n,):
            raise ValueError(f"dst_pages must have shape ({n},)")
    _launch(pages, tag, N.QUANT_FAKE_QUANTIZE, codes, scales, dst_pages, int4_group)
    return codes, scales


def fake_int8_pages_device(pages: torch.Tensor, variant: str) -> Tuple[torch.Tensor, torch.Tensor]:
    """``fake_int8_pages_from_fp16`` of the fused (``variant='fused'``: float16
    scales) or the triton module (``'triton'``: float32 scales) on the GPU."""
    require_device(pages, what="page quantiser")
    pages = _check_pages(pages)
    n = pages.shape[0]
    mode = {"fused": N.QUANT_FUSED_INT8, "triton": N.QUANT_TRITON_INT8}[variant]
    codes = torch.empty(pages.shape, dtype=torch.int8, device=pages.device)
    scales = torch.empty(n, dtype=torch.float16 if variant == "fused" else torch.float32, device=pages.device)
    _launch(pages, N.TAG_INT8, mode, codes, scales, None, 32)
    return codes, scales
