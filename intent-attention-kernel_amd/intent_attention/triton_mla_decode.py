"""Drop-in for the reference's ``triton_mla_decode`` module on the MI355X
MFMA kernel (``mla_core.mla_paged_decode``).

``mla_decode_triton`` keeps the reference signature and result
(triton_mla_decode.py:110-152): ``q_absorb [batch, q_len, d_c]`` attends to the
latent rows of the pages listed in a 1-D ``page_table`` shared by the batch
(page ``p`` = rows ``p*page_size .. (p+1)*page_size - 1`` of ``C [T, d_c]``),
softmax scale ``1/sqrt(d_c)``, and the context is projected by ``W_VO_fused``;
zeros when the table is empty. The selected rows are gathered in table order
into 16-row pages of float16 (any ``page_size``; the last page of ``C`` may be
shorter, and the gathered rows are bounded by the kernel's token count), ``d_c`` is zero-padded to a supported width
(64, 128, 256, 512 or 576), and the projection is one float32 GEMM. Host
tensors raise RuntimeError: there is no CPU path in this package.
"""
from __future__ import annotations

import math

import torch

from .decode_core import require_device
from .mla_core import LatentPools, mla_paged_decode

_WIDTHS = (64, 128, 256, 512, 576)


def is_triton_available() -> bool:
    """Triton is not used: the decode runs on the HIP kernels in libiak.so."""
    return False


def is_cuda_available() -> bool:
    return torch.cuda.is_available()


def mla_latent_context(q_absorb: torch.Tensor, C: torch.Tensor, page_table: torch.Tensor,
                       page_size: int = 64) -> torch.Tensor:
    """The latent context ``softmax(q C_sel^T / sqrt(d_c)) C_sel`` as float32
    ``[batch, q_len, d_c]`` (the part of ``mla_decode_triton`` before W_VO)."""
    dev = require_device(q_absorb, C, page_table, what="MLA latent decode")
    if q_absorb.dim() != 3 or C.dim() != 2 or C.shape[1] != q_absorb.shape[2]:
        raise ValueError(f"q_absorb must be [batch, q_len, d_c] and C [T, d_c], got {tuple(q_absorb.shape)} "
                         f"and {tuple(C.shape)}")
    batch, q_len, d_c = q_absorb.shape
    if d_c > _WIDTHS[-1]:
        raise ValueError(f"d_c {d_c} exceeds the widest supported latent ({_WIDTHS[-1]})")
    if page_size <= 0:
        raise ValueError(f"page_size must be positive, got {page_size}")
    ids = page_table.reshape(-1).to(device=dev, dtype=torch.int64)
    n_sel = ids.numel()
    if n_sel == 0:
        return torch.zeros(batch, q_len, d_c, dtype=torch.float32, device=dev)
    # page p is rows p*page_size .. (p+1)*page_size - 1 of C, the last page of
    # C possibly shorter (the reference slices C[p*ps:(p+1)*ps])
    n_src = (C.shape[0] + page_size - 1) // page_size
    if int(ids.min()) < 0 or int(ids.max()) >= n_src:
        raise ValueError(f"page ids must lie in [0, {n_src})")
    width = next(w for w in _WIDTHS if w >= d_c)
    rows = (ids[:, None] * page_size + torch.arange(page_size, device=dev)).reshape(-1)
    rows = rows[rows < C.shape[0]]
    T = rows.numel()
    n16 = (T + 15) // 16
    lat = torch.zeros(n16 * 16, width, dtype=torch.float16, device=dev)
    lat[:T, :d_c] = C.index_select(0, rows).to(torch.float16)
    pools = LatentPools(c_fp16=lat.view(n16, 16, width))
    table = torch.arange(n16, dtype=torch.int32, device=dev).expand(batch, n16).contiguous()
    counts = torch.full((batch,), n16, dtype=torch.int32, device=dev)
    valid = torch.full((batch,), T, dtype=torch.int32, device=dev)
    q = torch.zeros(batch, q_len, width, dtype=torch.float16, device=dev)
    q[..., :d_c] = q_absorb.to(torch.float16)
    scale = 1.0 / math.sqrt(d_c)
    v_main = width if width <= 512 else 512
    ctx = mla_paged_decode(q, pools, table, counts, None, v_dim=v_main, sm_scale=scale, valid_tokens=valid,
                           out_dtype=torch.float32)
    if width > 512:
        tail = mla_paged_decode(q, pools, table, counts, None, v_dim=width - 512, v_offset=512, sm_scale=scale,
                                valid_tokens=valid, out_dtype=torch.float32)
        ctx = torch.cat([ctx, tail], dim=-1)
    return ctx[..., :d_c]


def mla_decode_triton(q_absorb: torch.Tensor, C: torch.Tensor, W_VO_fused: torch.Tensor,
                      page_table: torch.Tensor, page_size: int = 64) -> torch.Tensor:
    """MLA decode over page-table-selected latent pages (triton_mla_decode.py:110-152).

    Returns ``[batch, q_len, d_out]`` with the dtype and device of ``q_absorb``;
    zeros when ``page_table`` is empty.
    """
    require_device(q_absorb, C, W_VO_fused, page_table, what="MLA latent decode")
    if W_VO_fused.dim() != 2 or W_VO_fused.shape[0] != q_absorb.shape[2]:
        raise ValueError(f"W_VO_fused must be [d_c, d_out], got {tuple(W_VO_fused.shape)}")
    ctx = mla_latent_context(q_absorb, C, page_table, page_size)
    return (ctx @ W_VO_fused.float()).to(q_absorb.dtype)
