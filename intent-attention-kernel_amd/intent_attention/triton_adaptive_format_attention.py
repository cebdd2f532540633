"""Adaptive-format decode attention on the HIP paged decode.

Interface of the reference's triton_adaptive_format_attention.py:
``AdaptivePageFormat`` (:33-40), ``AdaptiveFormatKernelConfig`` (:43-51),
``is_triton_available`` / ``is_cuda_available`` (:58-68),
``adaptive_format_decode_attention_triton`` (:237-331, its kernel :92-225),
``adaptive_format_decode_attention_reference_dispatch`` (:337-414) and
``make_adaptive_page_tables`` (:420-470).

Semantics kept from the reference's kernel: one output row per (batch, head)
over the ``max_selected_pages`` entries of its page_ids row; an entry with
id < 0 or format SKIP contributes nothing, SPARSE contributes nothing
(interface only, as in the reference), FP16 pages are read as stored, INT8
pages as code * scale with per-page float32 scales, and any other format
value gives page_size zero K/V rows with score 0 (the reference kernel's
masked loads); the softmax scale is 1/sqrt(D); a row with no contribution is
zero; the output has q's dtype.

Differences, by design: the kernel is libiak's paged decode. Pages of 16
tokens with head_dim 64 or 128 are decoded in place; other shapes (and
format values outside 0..3, or INT8 pages without INT8 pools) are staged
first: the contributing pages of each row are gathered into 16-token float16
pages, INT8 pages dequantised to float16(code * scale) by the transcoding
kernel (a float16 rounding the reference's float32 arithmetic does not
make). Page ids at or past the pool size are skipped (the reference reads
out of bounds). ``is_triton_available`` is False: there is no Triton here.
``adaptive_format_decode_attention_reference_dispatch`` runs the same GPU
computation on its own argument conventions (K = V = the K pages, the INT8
K pages and their scales rounded to float16, as the reference's dispatch
passes them); the reference's dispatch returns zeros for every input (its
adaptive_format_attention_reference accumulates only under the
unknown-format branch, adaptive_format_attention.py:98-112).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from enum import IntEnum
from typing import Optional, Tuple

import torch

from . import _native as N
from .decode_core import PAGE_SIZE, PagePools, current_stream_handle, paged_decode


class AdaptivePageFormat(IntEnum):
    FP16 = 0
    INT8 = 1
    SPARSE = 2
    SKIP = 3


@dataclass(frozen=True)
class AdaptiveFormatKernelConfig:
    page_size: int = 16
    head_dim: int = 64
    max_selected_pages: int = 64
    block_d: int = 64
    sparse_max_nnz: int = 256


def is_triton_available() -> bool:
    """Triton is not used: the decode runs on the HIP kernels in libiak.so."""
    return False


def is_cuda_available() -> bool:
    return torch.cuda.is_available()


def _require_device() -> None:
    if not torch.cuda.is_available():
        raise RuntimeError("CUDA is not available: the adaptive-format decode needs a ROCm (MI355X) device. "
                           "CPU reference paths remain available in the test oracle.")
    N.load()


_TAG_MAP = [N.TAG_FP16, N.TAG_INT8, N.TAG_SKIP, N.TAG_SKIP] + [N.TAG_SKIP] * 4


def _promote(codes: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """float16(code * scale) of pages codes [n, E] int8, scales [n] float32."""
    n, E = codes.shape
    out = torch.empty((n, E), dtype=torch.float16, device=codes.device)
    if n == 0:
        return out
    if E % 8:
        raise ValueError(f"page_size * head_dim must be a multiple of 8, got {E}")
    a = N.TranscodeArgs()
    a.num_pages, a.page_elems, a.mode, a.pages, a.pool_pages = n, E, N.TRANSCODE_PROMOTE_FP16, None, n
    a.fp16, a.int8, a.scales = out.data_ptr(), codes.data_ptr(), scales.data_ptr()
    N.transcode_pages(a, current_stream_handle(codes.device))
    return out


def _staged(q, ids, fmts, k16, v16, k8, v8, ks, vs, PS):
    """Gather every row's contributing pages into 16-token float16 pages and
    decode them, the last page of a row bounded by its token count."""
    B, H, D = q.shape
    W = ids.shape[2]
    NP = k16.shape[0]
    dev = q.device
    idc = ids.long().clamp(0, max(NP - 1, 0))
    inb = (ids >= 0) & (ids < NP)
    f = torch.where(inb, fmts.long()[idc], torch.full_like(idc, int(AdaptivePageFormat.SKIP)))
    is16 = inb & (f == 0)
    is8 = inb & (f == 1) & (k8 is not None)
    zero = inb & (((f < 0) | (f > 3)) | ((f == 1) & (k8 is None)))
    take = is16 | is8 | zero
    R = B * H
    kr = torch.zeros((R, W, PS, D), dtype=torch.float16, device=dev)
    vr = torch.zeros_like(kr)
    sel16, sel8 = is16.view(R, W), is8.view(R, W)
    flat = idc.view(R, W)
    if sel16.any():
        p = flat[sel16]
        kr[sel16] = k16[p].to(torch.float16).view(-1, PS, D)
        vr[sel16] = v16[p].to(torch.float16).view(-1, PS, D)
    if sel8.any():
        p = flat[sel8]
        kr[sel8] = _promote(k8[p].reshape(p.numel(), -1).contiguous(), ks.float()[p].contiguous()).view(-1, PS, D)
        vr[sel8] = _promote(v8[p].reshape(p.numel(), -1).contiguous(), vs.float()[p].contiguous()).view(-1, PS, D)
    # compact each row's contributing entries to its front, in table order
    t = take.view(R, W)
    order = torch.argsort((~t).to(torch.int8), dim=1, stable=True)
    kr = torch.gather(kr, 1, order.view(R, W, 1, 1).expand(R, W, PS, D))
    vr = torch.gather(vr, 1, order.view(R, W, 1, 1).expand(R, W, PS, D))
    lens = t.sum(dim=1).to(torch.int32) * PS
    T = W * PS
    P = max(1, (T + PAGE_SIZE - 1) // PAGE_SIZE)
    width = 64 if D <= 64 else 128
    pk = torch.zeros((R, P * PAGE_SIZE, width), dtype=torch.float16, device=dev)
    pv = torch.zeros_like(pk)
    pk[:, :T, :D] = kr.view(R, T, D)
    pv[:, :T, :D] = vr.view(R, T, D)
    qq = torch.zeros((B, H, width), dtype=q.dtype, device=dev)
    qq[..., :D] = q
    table = (torch.arange(R, device=dev, dtype=torch.int32).view(R, 1) * P
             + torch.arange(P, device=dev, dtype=torch.int32).view(1, P)).view(B, H, P)
    counts = ((lens + PAGE_SIZE - 1) // PAGE_SIZE).view(B, H)
    out = paged_decode(qq, PagePools(k_fp16=pk.view(R * P, PAGE_SIZE, width),
                                     v_fp16=pv.view(R * P, PAGE_SIZE, width)),
                       table.contiguous(), counts.contiguous(), torch.zeros(R * P, dtype=torch.int32, device=dev),
                       sm_scale=1.0 / math.sqrt(D), out_dtype=q.dtype, valid_tokens=lens.view(B, H).contiguous())
    return out[..., :D]


def adaptive_format_decode_attention_triton(
    q: torch.Tensor,
    page_ids: torch.Tensor,
    page_formats: torch.Tensor,
    fp16_k_pages: torch.Tensor,
    fp16_v_pages: torch.Tensor,
    int8_k_pages: Optional[torch.Tensor] = None,
    int8_v_pages: Optional[torch.Tensor] = None,
    int8_k_scales: Optional[torch.Tensor] = None,
    int8_v_scales: Optional[torch.Tensor] = None,
    sparse_k_indices: Optional[torch.Tensor] = None,
    sparse_k_values: Optional[torch.Tensor] = None,
    sparse_v_indices: Optional[torch.Tensor] = None,
    sparse_v_values: Optional[torch.Tensor] = None,
    sparse_nnz: Optional[torch.Tensor] = None,
    *,
    config: Optional[AdaptiveFormatKernelConfig] = None,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Adaptive-format decode: q [B, H, D] over page_ids [B, H, max_selected_pages]
    (-1 unused) of pages tagged page_formats [num_pages] -> [B, H, D] in q's dtype."""
    _require_device()
    cfg = config or AdaptiveFormatKernelConfig()
    if not q.is_cuda:
        raise ValueError("q must be a CUDA tensor")
    B, H, D = q.shape
    if cfg.block_d < D:
        raise ValueError("block_d must be >= D")
    if D > 128:
        raise ValueError(f"head_dim {D} exceeds the decode kernel's widest (128)")
    W = cfg.max_selected_pages
    if page_ids.dim() != 3 or tuple(page_ids.shape) != (B, H, W):
        raise ValueError(f"page_ids must be [B, H, max_selected_pages] = {(B, H, W)}, got {tuple(page_ids.shape)}")
    PS = cfg.page_size
    NP = fp16_k_pages.shape[0]
    for name, t in (("fp16_k_pages", fp16_k_pages), ("fp16_v_pages", fp16_v_pages),
                    ("int8_k_pages", int8_k_pages), ("int8_v_pages", int8_v_pages)):
        if t is not None and (t.dim() != 3 or t.shape[0] != NP or tuple(t.shape[1:]) != (PS, D)):
            raise ValueError(f"{name} must be [num_pages, page_size, D] = [{NP}, {PS}, {D}], got {tuple(t.shape)}")
    have8 = int8_k_pages is not None and int8_v_pages is not None
    if have8 and (int8_k_scales is None or int8_v_scales is None):
        int8_k_scales = torch.ones(NP, dtype=torch.float32, device=q.device) if int8_k_scales is None else int8_k_scales
        int8_v_scales = torch.ones(NP, dtype=torch.float32, device=q.device) if int8_v_scales is None else int8_v_scales
    ids = page_ids.to(device=q.device, dtype=torch.int32).contiguous()
    fmts = page_formats.to(device=q.device, dtype=torch.int32).contiguous()
    odd = bool(((fmts < 0) | (fmts > 3)).any()) if fmts.numel() else False
    native = (PS == PAGE_SIZE and D in (64, 128) and not odd and fp16_k_pages.dtype == torch.float16
              and fp16_v_pages.dtype == torch.float16 and (have8 or not bool((fmts == 1).any())))
    if native:
        pools = PagePools(k_fp16=fp16_k_pages.contiguous(), v_fp16=fp16_v_pages.contiguous())
        if have8:
            pools.k_int8, pools.v_int8 = int8_k_pages.contiguous(), int8_v_pages.contiguous()
            pools.k_int8_scale = int8_k_scales.to(torch.float32).contiguous()
            pools.v_int8_scale = int8_v_scales.to(torch.float32).contiguous()
        res = paged_decode(q, pools, ids, torch.full((B, H), W, dtype=torch.int32, device=q.device), fmts,
                           tag_map=_TAG_MAP if have8 else [N.TAG_FP16] + [N.TAG_SKIP] * 7,
                           sm_scale=1.0 / math.sqrt(D), out_dtype=q.dtype)
    else:
        res = _staged(q, ids, fmts, fp16_k_pages, fp16_v_pages, int8_k_pages if have8 else None,
                      int8_v_pages if have8 else None, int8_k_scales, int8_v_scales, PS)
    if out is None:
        return res.contiguous()
    out.copy_(res)
    return out


def adaptive_format_decode_attention_reference_dispatch(
    q: torch.Tensor,
    page_ids: torch.Tensor,
    page_formats: torch.Tensor,
    fp16_k_pages: torch.Tensor,
    fp16_v_pages: torch.Tensor,
    int8_k_pages: Optional[torch.Tensor] = None,
    int8_v_pages: Optional[torch.Tensor] = None,
    int8_k_scales: Optional[torch.Tensor] = None,
    int8_v_scales: Optional[torch.Tensor] = None,
    sparse_k_indices: Optional[torch.Tensor] = None,
    sparse_k_values: Optional[torch.Tensor] = None,
    sparse_v_indices: Optional[torch.Tensor] = None,
    sparse_v_values: Optional[torch.Tensor] = None,
    sparse_nnz: Optional[torch.Tensor] = None,
    *,
    config: Optional[AdaptiveFormatKernelConfig] = None,
) -> torch.Tensor:
    """The adaptive-format decode with the reference dispatch's conventions
    (K = V = fp16_k_pages, INT8 K = V = int8_k_pages with float16 scales),
    on the device; returns [B, H, D] float16."""
    _require_device()
    dev = torch.device("cuda", torch.cuda.current_device())
    t = lambda x: None if x is None else x.to(dev)  # noqa: E731
    k8 = t(int8_k_pages)
    ks = None if int8_k_scales is None or k8 is None else t(int8_k_scales).to(torch.float16).float()
    k16 = t(fp16_k_pages)
    out = adaptive_format_decode_attention_triton(
        t(q), t(page_ids), t(page_formats), k16, k16, k8, k8, ks, ks,
        config=config or AdaptiveFormatKernelConfig(max_selected_pages=page_ids.shape[2]))
    return out.to(torch.float16)


def make_adaptive_page_tables(selected_pages: torch.Tensor, batch: int, heads: int,
                              max_selected_pages: Optional[int] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """page_ids int32 [B, H, width] (-1 padded) and page_counts int32 [B, H] from
    selected_pages [N] (shared) or [B, H, N]."""
    if selected_pages.ndim == 1:
        n = selected_pages.numel()
        src = selected_pages.to(torch.int32).view(1, 1, n)
    elif selected_pages.ndim == 3:
        if selected_pages.shape[0] != batch or selected_pages.shape[1] != heads:
            raise ValueError("selected_pages [B, H, N] must match batch and heads")
        n = selected_pages.shape[2]
        src = selected_pages.to(torch.int32)
    else:
        raise ValueError("selected_pages must have shape [N] or [B, H, N]")
    width = max_selected_pages or n
    if n > width:
        raise ValueError("selected_pages exceeds max_selected_pages")
    page_ids = torch.full((batch, heads, width), -1, dtype=torch.int32, device=selected_pages.device)
    page_ids[:, :, :n] = src
    page_counts = torch.full((batch, heads), n, dtype=torch.int32, device=selected_pages.device)
    return page_ids, page_counts
