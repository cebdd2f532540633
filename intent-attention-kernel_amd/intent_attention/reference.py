"""``dense_attention`` of the reference (reference.py:16-45) on the HIP paged decode.

Softmax attention ``softmax(q k^T / sqrt(D)) v`` over the last two dims, as
the reference computes it with two ``torch.matmul`` calls. Here K and V are
laid out as 16-token float16 pages (zero-padded; the last page of each
sequence bounded by the kernel's token count) and the attention runs on
libiak's selected-page decode kernel: every (leading index, query) pair is a
decode row over all of that index's pages.

Kept from the reference: argument names and defaults, the output (shape and
dtype of ``q``), ``causal=True`` as the upper-triangular mask of
``torch.triu(..., diagonal=1)`` (query i sees keys 0 .. i), and the
RuntimeError of ``torch.matmul`` on mixed dtypes.

Differences, by design:

* device tensors only (host tensors raise RuntimeError; there is no CPU
  path in this package);
* leading dims of q, k and v must be equal (no broadcasting) and
  ``head_dim <= 128`` (padded to 64 or 128 with zeros, which changes no
  score);
* K and V are rounded to float16 pages (the kernel's FP16 pool format):
  float32 inputs differ from the reference's float32 matmuls by that
  rounding (relative 2^-11 per value);
* an additive ``mask`` or ``original_kv_positions`` raise
  NotImplementedError: the paged kernel applies only token bounds.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from .decode_core import PAGE_SIZE, PagePools, paged_decode, require_device
from . import _native as N

_WIDTHS = (64, 128)
_MAX_GROUP = 16          # query rows sharing one page-table row (the kernel's GQA limit)


def _pages_of(x: torch.Tensor, width: int) -> torch.Tensor:
    """[L, T, D] -> float16 pages [L * P, 16, width], zero-padded in tokens and dims."""
    L, T, D = x.shape
    P = max(1, (T + PAGE_SIZE - 1) // PAGE_SIZE)
    pages = torch.zeros((L, P * PAGE_SIZE, width), dtype=torch.float16, device=x.device)
    pages[:, :T, :D] = x
    return pages.view(L * P, PAGE_SIZE, width)


def dense_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False,
                    mask: Optional[torch.Tensor] = None,
                    original_kv_positions: Optional[torch.Tensor] = None) -> torch.Tensor:
    """softmax(q k^T / sqrt(D)) v over [..., T, D] tensors, on the HIP decode kernel."""
    if mask is not None or original_kv_positions is not None:
        raise NotImplementedError("dense_attention on the paged decode kernel supports token bounds only "
                                  "(causal=True); an additive mask or original_kv_positions is not supported")
    dev = require_device(q, k, v, what="dense attention")
    if q.dtype != k.dtype or k.dtype != v.dtype:
        # the reference's torch.matmul refuses mixed dtypes
        raise RuntimeError(f"expected m1 and m2 to have the same dtype, but got: {q.dtype} != "
                           f"{k.dtype if q.dtype != k.dtype else v.dtype}")
    if q.dim() < 2 or k.dim() != q.dim() or v.dim() != q.dim():
        raise ValueError(f"q, k and v must have the same number of dims (>= 2), got {q.dim()}, {k.dim()}, {v.dim()}")
    lead = tuple(q.shape[:-2])
    if tuple(k.shape[:-2]) != lead or tuple(v.shape[:-2]) != lead or k.shape[-2] != v.shape[-2]:
        raise ValueError(f"q, k and v must share their leading dims and k, v their length: "
                         f"{tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    D = q.shape[-1]
    if k.shape[-1] != D or v.shape[-1] != D:
        raise ValueError(f"head dims differ: q {D}, k {k.shape[-1]}, v {v.shape[-1]}")
    if D > _WIDTHS[-1]:
        raise ValueError(f"head_dim {D} exceeds the widest supported ({_WIDTHS[-1]})")
    if q.dtype not in (torch.float16, torch.float32, torch.bfloat16):
        raise ValueError(f"dtype {q.dtype} is not supported")
    width = next(w for w in _WIDTHS if w >= D)
    L = math.prod(lead) if lead else 1
    Tq, Tk = q.shape[-2], k.shape[-2]
    out = torch.zeros(q.shape, dtype=q.dtype, device=dev)
    if L == 0 or Tq == 0:
        return out
    P = max(1, (Tk + PAGE_SIZE - 1) // PAGE_SIZE)
    kp = _pages_of(k.reshape(L, Tk, D), width)
    vp = _pages_of(v.reshape(L, Tk, D), width)
    tags = torch.zeros(L * P, dtype=torch.int32, device=dev)           # every page FP16
    pools = PagePools(k_fp16=kp, v_fp16=vp)
    qq = q.reshape(L, Tq, D)
    if width != D:
        qq = torch.nn.functional.pad(qq, (0, width - D))
    qq = qq.contiguous()
    rows = torch.arange(L, device=dev, dtype=torch.int32)[:, None] * P + torch.arange(P, device=dev,
                                                                                      dtype=torch.int32)
    sm = 1.0 / math.sqrt(D)
    if not causal and Tq <= _MAX_GROUP:
        # one page-table row per leading index, shared by its Tq queries (the GQA group)
        o = paged_decode(qq.view(1, L * Tq, width), pools, rows.view(1, L, P).contiguous(),
                         torch.full((1, L), P, dtype=torch.int32, device=dev), tags, sm_scale=sm,
                         valid_tokens=torch.full((1, L), Tk, dtype=torch.int32, device=dev),
                         tag_map=[N.TAG_FP16] + [N.TAG_SKIP] * 7)
        return o.view(L, Tq, width)[..., :D].reshape(q.shape)
    # one row per (leading index, query): causal rows see keys 0 .. i
    table = rows[:, None, :].expand(L, Tq, P).reshape(1, L * Tq, P).contiguous()
    t = torch.arange(Tq, device=dev, dtype=torch.int32)
    bound = torch.minimum(t + 1, torch.tensor(Tk, dtype=torch.int32, device=dev)) if causal else \
        torch.full((Tq,), Tk, dtype=torch.int32, device=dev)
    o = paged_decode(qq.view(1, L * Tq, width), pools, table,
                     torch.full((1, L * Tq), P, dtype=torch.int32, device=dev), tags, sm_scale=sm,
                     valid_tokens=bound.repeat(L).view(1, L * Tq).contiguous(),
                     tag_map=[N.TAG_FP16] + [N.TAG_SKIP] * 7)
    return o.view(L, Tq, width)[..., :D].reshape(q.shape)
