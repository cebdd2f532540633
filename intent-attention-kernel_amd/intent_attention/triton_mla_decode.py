"""Drop-in for the reference's ``triton_mla_decode`` module on the MI355X.

``mla_decode_triton`` keeps the reference signature and result
(triton_mla_decode.py:110-152): ``q_absorb [batch, q_len, d_c]`` attends to the
latent rows of the pages listed in a 1-D ``page_table`` shared by the batch
(page ``p`` = rows ``p*page_size .. (p+1)*page_size - 1`` of ``C [T, d_c]``,
the last page of ``C`` possibly shorter), softmax scale ``1/sqrt(d_c)``, and
the context is projected by ``W_VO_fused``; zeros when the table is empty.

The latent context runs on libiak's ``iak_mla_decode_rows`` in the reference's
arithmetic: float32 products and sums over the inputs as given (float32,
float16 or bfloat16, read in place), any ``page_size``, any ``d_c`` up to 1,024
in one launch. The projection is one float32 GEMM. (The paged serving path,
``mla_core.mla_paged_decode``, is the MFMA kernel over f16 / FP8 / INT8 latent
pools.) Host tensors raise RuntimeError: there is no CPU path in this package.
"""
from __future__ import annotations

import math

import torch

from . import _native as N
from .decode_core import current_stream_handle, require_device

_DT = {torch.float32: N.DTYPE_F32, torch.float16: N.DTYPE_F16, torch.bfloat16: N.DTYPE_BF16}
MAX_LATENT = 1024


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
    if d_c > MAX_LATENT:
        raise ValueError(f"d_c {d_c} exceeds the widest supported latent ({MAX_LATENT})")
    if page_size <= 0:
        raise ValueError(f"page_size must be positive, got {page_size}")
    if q_absorb.dtype not in _DT or C.dtype not in _DT:
        raise ValueError(f"q_absorb and C must be float32, float16 or bfloat16, got {q_absorb.dtype} and {C.dtype}")
    ids = page_table.reshape(-1).to(device=dev, dtype=torch.int32)
    ctx = torch.empty(batch, q_len, d_c, dtype=torch.float32, device=dev)
    if ids.numel() == 0 or batch * q_len == 0:
        return ctx.zero_()
    # page p is rows p*page_size .. (p+1)*page_size - 1 of C, the last page of
    # C possibly shorter (the reference slices C[p*ps:(p+1)*ps])
    n_src = (C.shape[0] + page_size - 1) // page_size
    lo, hi = torch.stack(torch.aminmax(ids)).tolist()          # one device-to-host read
    if lo < 0 or hi >= n_src:
        raise ValueError(f"page ids must lie in [0, {n_src})")
    if q_absorb.stride(2) != 1:
        q_absorb = q_absorb.contiguous()
    if C.stride(1) != 1:
        C = C.contiguous()
    a = N.MlaRowsArgs()
    a.batch, a.q_len, a.latent_dim, a.page_size, a.num_selected = batch, q_len, d_c, int(page_size), ids.numel()
    a.num_rows = C.shape[0]
    a.q, a.q_dtype, a.q_stride_b, a.q_stride_t = q_absorb.data_ptr(), _DT[q_absorb.dtype], q_absorb.stride(0), \
        q_absorb.stride(1)
    a.latents, a.latent_dtype, a.latent_stride = C.data_ptr(), _DT[C.dtype], C.stride(0)
    a.page_ids, a.context, a.sm_scale = ids.data_ptr(), ctx.data_ptr(), 1.0 / math.sqrt(d_c)
    # few rows over many latent rows: a workspace lets the kernel split each
    # row's keys over several workgroups (allocated on this stream, as the rest)
    ws_bytes = N.mla_decode_rows_workspace(a)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
    N.mla_decode_rows(a, current_stream_handle(dev), ws.data_ptr() if ws is not None else 0, ws_bytes)
    return ctx


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
