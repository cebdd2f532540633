"""``dense_attention`` and ``semantic_block_attention`` of the reference
(reference.py:16-129) on libiak's dense attention kernel.

``dense_attention(q, k, v, causal, mask, original_kv_positions)`` is softmax
attention over the last two dims, as the reference computes it with two
``torch.matmul`` calls (reference.py:16-45):

* scores ``(q k^T) / sqrt(D)``;
* ``causal=True`` without positions adds ``triu(-inf, diagonal=1)`` (query i
  sees keys 0 .. i); with ``original_kv_positions`` query i sees key j only
  where ``positions[j] <= i`` (the reference's ``masked_fill``);
  ``original_kv_positions`` without ``causal`` changes nothing;
* an additive ``mask`` broadcast to the scores (a bool mask adds 1.0 where
  true, as ``float + bool`` does in torch);
* a query whose scores are all -inf gives NaN (torch's softmax), an empty key
  set gives zeros.

Leading dims broadcast as in ``torch.matmul``; the output has the shape
``[*lead, Tq, Dv]`` and the dtype of ``q``. The dtype rules of the reference's
two matmuls are kept: ``q`` and ``k`` must share a dtype, and a ``mask`` that
promotes the scores to another dtype than ``v``'s raises the same
RuntimeError the reference's second matmul raises.

The kernel (``iak_dense_attention``) computes every product and sum in
float32 over float32, float16 or bfloat16 inputs and rounds the output once,
where the reference rounds its scores and weights to the input dtype; for
float32 inputs both are float32 arithmetic. head_dim and v_dim are at most
1,024. Device tensors only: host tensors raise RuntimeError. The output
carries no autograd history (inference only).

``semantic_block_attention`` (reference.py:81-129) attends to the layout's
selected tokens through ``dense_attention``, scoring ATTEND blocks that carry
no score first (``_resolve_dynamic_scores`` :52-78 with the cosine probe of
``BlockScorer.score_blocks``, block_scorer.py:17-34).
"""
from __future__ import annotations

import math
from typing import Any, Dict, List, Optional, Tuple, Union

import torch

from . import _native as N
from .block_metadata import BlockLayout, BlockPolicy
from .decode_core import current_stream_handle, require_device

_DTYPES = {torch.float16: N.DTYPE_F16, torch.float32: N.DTYPE_F32, torch.bfloat16: N.DTYPE_BF16}
_MAX_DIM = 1024


def _dtype_name(dt: torch.dtype) -> str:
    """torch's C++ name of a dtype, as its matmul error messages print it."""
    return {torch.float16: "c10::Half", torch.bfloat16: "c10::BFloat16", torch.float32: "float",
            torch.float64: "double"}.get(dt, str(dt))


def _rows(x: torch.Tensor, lead: Tuple[int, ...]) -> torch.Tensor:
    """[*lead', T, D] broadcast to [*lead, T, D] and viewed as [L, T, D] with a unit inner stride
    (a view where the strides allow it, else a copy)."""
    x = x.expand(*lead, x.shape[-2], x.shape[-1])
    x = x.reshape(math.prod(lead), x.shape[-2], x.shape[-1])
    if x.stride(-1) != 1 and x.shape[-1] > 1:
        x = x.contiguous()
    return x


def dense_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False,
                    mask: Optional[torch.Tensor] = None,
                    original_kv_positions: Optional[torch.Tensor] = None) -> torch.Tensor:
    """softmax(q k^T / sqrt(D) [+ causal mask] [+ mask]) v over [..., T, D] tensors, on the HIP kernel."""
    dev = require_device(*(t for t in (q, k, v, mask, original_kv_positions) if t is not None),
                         what="dense attention")
    if q.dim() < 2 or k.dim() < 2 or v.dim() < 2:
        raise RuntimeError("both arguments to matmul need to be at least 2D")
    if q.dtype != k.dtype:
        raise RuntimeError(f"expected m1 and m2 to have the same dtype, but got: {_dtype_name(q.dtype)} != "
                           f"{_dtype_name(k.dtype)}")
    D, Dv = q.shape[-1], v.shape[-1]
    Tq, Tk = q.shape[-2], k.shape[-2]
    if k.shape[-1] != D:
        raise RuntimeError(f"q and k head dims differ: {D} != {k.shape[-1]}")
    if v.shape[-2] != Tk:
        raise RuntimeError(f"k and v lengths differ: {Tk} != {v.shape[-2]}")
    score_dtype = q.dtype if mask is None else torch.promote_types(q.dtype, mask.dtype)
    if score_dtype != v.dtype:
        raise RuntimeError(f"expected m1 and m2 to have the same dtype, but got: {_dtype_name(score_dtype)} != "
                           f"{_dtype_name(v.dtype)}")
    if q.dtype not in _DTYPES:
        raise ValueError(f"dtype {q.dtype} is not supported (float16, float32, bfloat16)")
    if D > _MAX_DIM or Dv > _MAX_DIM:
        raise ValueError(f"head_dim {D} / v_dim {Dv} exceeds the widest supported ({_MAX_DIM})")
    lead = tuple(q.shape[:-2])
    if k.shape[:-2] != lead or v.shape[:-2] != lead:
        lead = tuple(torch.broadcast_shapes(q.shape[:-2], k.shape[:-2], v.shape[:-2]))
    mask_rows = None
    if mask is not None:
        if mask.dtype != torch.bool and mask.dtype not in _DTYPES:
            raise ValueError(f"mask dtype {mask.dtype} is not supported (bool, float16, float32, bfloat16)")
        full = torch.broadcast_shapes(tuple(mask.shape), (*lead, Tq, Tk))
        if tuple(full[-2:]) != (Tq, Tk):
            raise RuntimeError(f"mask of shape {tuple(mask.shape)} does not broadcast to the scores "
                               f"{(*lead, Tq, Tk)}")
        lead = tuple(full[:-2])
        mask_rows = _rows(mask, lead)
    positions = None
    if causal and original_kv_positions is not None:
        if original_kv_positions.dtype.is_floating_point or original_kv_positions.dtype == torch.bool:
            raise ValueError(f"original_kv_positions must be an integer tensor, got {original_kv_positions.dtype}")
        if original_kv_positions.dim() != 1 or original_kv_positions.shape[0] != Tk:
            raise RuntimeError(f"The size of original_kv_positions {tuple(original_kv_positions.shape)} must "
                               f"match the number of keys ({Tk})")
        positions = original_kv_positions.to(torch.int64).contiguous()

    L = math.prod(lead)
    out = torch.empty((*lead, Tq, Dv), dtype=q.dtype, device=dev)
    if L == 0 or Tq == 0:
        return out
    qr, kr, vr = _rows(q, lead), _rows(k, lead), _rows(v, lead)
    o = out.view(L, Tq, Dv)
    a = N.DenseAttentionArgs()
    a.batch, a.q_len, a.kv_len, a.head_dim, a.v_dim, a.dtype = L, Tq, Tk, D, Dv, _DTYPES[q.dtype]
    a.q, a.q_stride_b, a.q_stride_t = qr.data_ptr(), qr.stride(0), qr.stride(1)
    a.k, a.k_stride_b, a.k_stride_t = kr.data_ptr(), kr.stride(0), kr.stride(1)
    a.v, a.v_stride_b, a.v_stride_t = vr.data_ptr(), vr.stride(0), vr.stride(1)
    a.out, a.out_stride_b, a.out_stride_t = o.data_ptr(), o.stride(0), o.stride(1)
    if mask_rows is not None:
        a.mask = mask_rows.data_ptr()
        a.mask_dtype = N.MASK_BOOL if mask.dtype == torch.bool else _DTYPES[mask.dtype]
        a.mask_stride_b, a.mask_stride_q, a.mask_stride_k = (mask_rows.stride(0), mask_rows.stride(1),
                                                             mask_rows.stride(2))
    if causal:
        a.causal = N.CAUSAL_TRIU if positions is None else N.CAUSAL_POSITIONS
        if positions is not None:
            a.kv_positions = positions.data_ptr()
    a.sm_scale = 1.0 / math.sqrt(D)
    # few rows with many keys: a workspace lets the kernel split each row's keys
    # over several workgroups (decode shapes); the operands, any copies made
    # above and the workspace were allocated on this stream, so the caching
    # allocator reuses their memory only after these kernels
    ws_bytes = N.dense_attention_workspace(a)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
    N.dense_attention(a, current_stream_handle(dev), ws.data_ptr() if ws is not None else 0, ws_bytes)
    return out


def _resolve_dynamic_scores(q: torch.Tensor, k: torch.Tensor, layout: BlockLayout) -> Dict[str, float]:
    """Score the ATTEND blocks whose score is None (reference.py:52-78): cosine of the
    query's mean over rows and leading dims with the block's mean key
    (BlockScorer.score_blocks, block_scorer.py:17-34), clamped at 0, written
    into the blocks."""
    targets = [b for b in layout.blocks if b.policy == BlockPolicy.ATTEND and b.score is None]
    if not targets:
        return {}
    qg = q.mean(dim=-2).mean(dim=(0, 1))
    qn = qg / (qg.norm(p=2) + 1e-10)
    reps = [k[..., b.start:b.end, :].mean(dim=-2).mean(dim=(0, 1)) for b in targets]
    sims = [torch.dot(qn, r / (r.norm(p=2) + 1e-10)) for r in reps]
    values = torch.stack(sims).tolist()   # one host copy for all blocks
    dynamic: Dict[str, float] = {}
    for block, s in zip(targets, values):
        block.score = max(0.0, float(s))
        dynamic[block.name] = block.score
    return dynamic


def semantic_block_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, layout: BlockLayout,
                             causal: bool = False, return_debug: bool = False,
                             threshold: float = 0.5) -> Union[torch.Tensor, Tuple[torch.Tensor, Dict[str, Any]]]:
    """Attention of q over the layout's selected tokens (reference.py:81-129); with
    ``causal`` the selected keys keep their original positions."""
    require_device(q, k, v, what="semantic block attention")
    kv_tokens = k.size(-2)
    dynamic = _resolve_dynamic_scores(q, k, layout)
    layout.validate(kv_tokens)
    selected: List[int] = layout.selected_token_indices()
    if not selected:
        out = torch.zeros_like(q)
        if not return_debug:
            return out
        debug: Dict[str, Any] = {"selected_token_count": 0, "selected_block_names": [],
                                 "total_kv_tokens": kv_tokens, "selected_kv_tokens": 0}
        if dynamic:
            debug["dynamic_scores"] = dynamic
        return out, debug
    idx = torch.tensor(selected, dtype=torch.long, device=k.device)
    out = dense_attention(q, k.index_select(-2, idx), v.index_select(-2, idx), causal=causal,
                          original_kv_positions=idx)
    if not return_debug:
        return out
    debug = {"selected_token_count": layout.selected_token_count(),
             "selected_block_names": [b.name for b in layout.selected_blocks()],
             "total_kv_tokens": kv_tokens, "selected_kv_tokens": len(selected)}
    if dynamic:
        debug["dynamic_scores"] = dynamic
    return out, debug
