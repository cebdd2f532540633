"""Device entry point of the MLA latent decode: torch tensors -> C ABI.

``mla_paged_decode`` runs ``iak_mla_decode`` (include/iak.h): every query head
of a sequence attends to the sequence's selected latent pages (one compressed
KV shared by all heads), ``out[b, h] = softmax(sm_scale * q[b, h] . C^T) C[:, v]``
over the latent rows C of the pages ``page_table[b, :page_counts[b]]``. Pages
are FP16, FP8-e4m3 or INT8 (one scale per page). The kernel runs on MFMA with
f16 operands (q is rounded to f16) and f32 accumulation. There is no host path.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, fields
from typing import Dict, Optional, Sequence

import torch

from . import _native as N
from .decode_core import PAGE_SIZE, _DT, _check_pool, _ptr, _scale_dtype, current_stream_handle, require_device

SUPPORTED_SHAPES = ((64, 64), (128, 128), (256, 256), (512, 512), (576, 512), (576, 64))

# native tags a latent page can carry: FP16, INT8, SKIP, FP8
LATENT_TAG_MAP = (N.TAG_FP16, N.TAG_INT8, N.TAG_SKIP, N.TAG_FP8, N.TAG_SKIP, N.TAG_SKIP, N.TAG_SKIP, N.TAG_SKIP)


@dataclass
class LatentPools:
    """Latent page pools indexed by physical page id, [NP, 16, qk_dim]:
    ``c_fp16`` float16 values; ``c_fp8`` e4m3fn codes (uint8 or float8_e4m3fn) and ``c_int8`` int8
    codes, each with one scale per page (``c_fp8_scale`` / ``c_int8_scale``
    [NP], both float16 or both float32). Dequantised value = code * scale."""

    c_fp16: Optional[torch.Tensor] = None
    c_fp8: Optional[torch.Tensor] = None
    c_int8: Optional[torch.Tensor] = None
    c_fp8_scale: Optional[torch.Tensor] = None
    c_int8_scale: Optional[torch.Tensor] = None

    def tensors(self) -> Dict[str, torch.Tensor]:
        return {f.name: getattr(self, f.name) for f in fields(self)
                if isinstance(getattr(self, f.name), torch.Tensor)}

    def has(self, tag: int) -> bool:
        need = {N.TAG_FP16: ("c_fp16",), N.TAG_FP8: ("c_fp8", "c_fp8_scale"),
                N.TAG_INT8: ("c_int8", "c_int8_scale")}.get(tag, ())
        return bool(need) and all(getattr(self, n) is not None for n in need)


class MlaPlan:
    """Validated launch arguments plus workspace (``run`` is one C call on the
    current stream; the tensors are held so their memory stays valid)."""

    def __init__(self, args: N.MlaDecodeArgs, device: torch.device, out: torch.Tensor, keep=()) -> None:
        self.args = args
        self.device = device
        self.out = out
        self._keep = keep
        self.workspace_bytes = N.mla_workspace_bytes(args)
        self._ws = (torch.empty(self.workspace_bytes, dtype=torch.uint8, device=device)
                    if self.workspace_bytes else None)

    def run(self, stream: Optional[int] = None, events: Optional[tuple] = None) -> None:
        """Launch on ``stream`` (default: torch's current stream). ``events``: an
        optional pair of torch.cuda.Event recorded around the split kernel alone."""
        s = current_stream_handle(self.device) if stream is None else stream
        ev = None if events is None else (events[0].cuda_event, events[1].cuda_event)
        N.mla_decode(self.args, self._ws.data_ptr() if self._ws is not None else 0, self.workspace_bytes, s, ev)


def make_mla_plan(q: torch.Tensor, pools: LatentPools, page_table: torch.Tensor, page_counts: torch.Tensor,
                  page_tags: Optional[torch.Tensor] = None, *, v_dim: Optional[int] = None, v_offset: int = 0,
                  sm_scale: Optional[float] = None, tag_map: Optional[Sequence[int]] = None,
                  negative_ids: bool = False, valid_tokens: Optional[torch.Tensor] = None,
                  out: Optional[torch.Tensor] = None, out_dtype: Optional[torch.dtype] = None,
                  pages_per_split: int = 0) -> MlaPlan:
    """Validate the arguments of ``mla_paged_decode`` once, for repeated runs."""
    dev = require_device(q, page_table, page_counts, *pools.tensors().values(), what="MLA latent decode")
    if q.dim() != 3:
        raise ValueError(f"q must have shape [batch, heads, qk_dim], got {tuple(q.shape)}")
    B, H, DQK = q.shape
    if v_dim is None:
        v_dim = DQK if (DQK, DQK) in SUPPORTED_SHAPES else 512
    if (DQK, v_dim) not in SUPPORTED_SHAPES:
        raise ValueError(f"(qk_dim, v_dim) = ({DQK}, {v_dim}) is not one of {SUPPORTED_SHAPES}")
    if q.dtype not in _DT:
        raise ValueError(f"q dtype {q.dtype} is not float16 / float32 / bfloat16")
    qvec = 4 if q.dtype == torch.float32 else 8
    if q.stride(-1) != 1 or q.data_ptr() % 16 or q.stride(0) % qvec or q.stride(1) % qvec:
        # the kernel reads q rows as 16-byte vectors: a fresh (aligned) copy
        q = torch.empty(q.shape, dtype=q.dtype, device=q.device).copy_(q)
    if page_table.dim() != 2 or page_table.shape[0] != B or page_table.dtype != torch.int32:
        raise ValueError(f"page_table must be int32 [batch, W], got {page_table.dtype} {tuple(page_table.shape)}")
    if page_counts.shape != (B,) or page_counts.dtype != torch.int32:
        raise ValueError(f"page_counts must be int32 [batch], got {page_counts.dtype} {tuple(page_counts.shape)}")
    page_table = page_table.contiguous()
    page_counts = page_counts.contiguous()
    present = pools.tensors()
    if not present:
        raise ValueError("no latent pool given")
    NP = next(iter(present.values())).shape[0]
    _check_pool("c_fp16", pools.c_fp16, NP, (PAGE_SIZE, DQK), (torch.float16,))
    _check_pool("c_fp8", pools.c_fp8, NP, (PAGE_SIZE, DQK), (torch.uint8, torch.float8_e4m3fn))
    _check_pool("c_int8", pools.c_int8, NP, (PAGE_SIZE, DQK), (torch.int8,))
    _check_pool("c_fp8_scale", pools.c_fp8_scale, NP, (), (torch.float16, torch.float32))
    _check_pool("c_int8_scale", pools.c_int8_scale, NP, (), (torch.float16, torch.float32))
    if page_tags is not None:
        if page_tags.shape != (NP,) or page_tags.dtype != torch.int32:
            raise ValueError(f"page_tags must be int32 [{NP}], got {page_tags.dtype} {tuple(page_tags.shape)}")
        page_tags = page_tags.contiguous()
    if valid_tokens is not None:
        if valid_tokens.shape != (B,) or valid_tokens.dtype != torch.int32:
            raise ValueError(f"valid_tokens must be int32 [batch], got {valid_tokens.dtype} "
                             f"{tuple(valid_tokens.shape)}")
        valid_tokens = valid_tokens.contiguous()
    if out is None:
        out = torch.empty((B, H, v_dim), dtype=out_dtype or q.dtype, device=dev)
    if out.shape != (B, H, v_dim) or out.dtype not in _DT or out.stride(-1) != 1:
        raise ValueError(f"out must be [batch, heads, v_dim] = {(B, H, v_dim)} with unit inner stride")

    a = N.MlaDecodeArgs()
    a.batch, a.num_heads, a.qk_dim, a.v_dim, a.v_offset = B, H, DQK, v_dim, v_offset
    a.page_size, a.table_width, a.num_pages = PAGE_SIZE, page_table.shape[1], NP
    a.q, a.q_dtype, a.q_stride_b, a.q_stride_h = q.data_ptr(), _DT[q.dtype], q.stride(0), q.stride(1)
    a.out, a.out_dtype, a.out_stride_b, a.out_stride_h = out.data_ptr(), _DT[out.dtype], out.stride(0), out.stride(1)
    a.page_table, a.page_counts, a.page_tags = page_table.data_ptr(), page_counts.data_ptr(), _ptr(page_tags)
    if tag_map is None:
        tag_map = [t if pools.has(t) else N.TAG_SKIP for t in LATENT_TAG_MAP]
    tm = list(tag_map) + [N.TAG_SKIP] * (8 - len(tag_map))
    for i in range(8):
        a.tag_map[i] = int(tm[i])
    a.negative_ids = int(bool(negative_ids))
    a.valid_tokens = _ptr(valid_tokens)
    a.c_fp16, a.c_fp8, a.c_int8 = _ptr(pools.c_fp16), _ptr(pools.c_fp8), _ptr(pools.c_int8)
    a.c_fp8_scale, a.c_int8_scale = _ptr(pools.c_fp8_scale), _ptr(pools.c_int8_scale)
    a.scale_dtype = _scale_dtype("latent", pools.c_fp8_scale, pools.c_int8_scale)
    a.sm_scale = float(1.0 / math.sqrt(DQK) if sm_scale is None else sm_scale)
    a.pages_per_split = int(pages_per_split)
    keep = (q, page_table, page_counts, page_tags, valid_tokens, *present.values())
    return MlaPlan(a, dev, out, keep)


def mla_paged_decode(q: torch.Tensor, pools: LatentPools, page_table: torch.Tensor, page_counts: torch.Tensor,
                     page_tags: Optional[torch.Tensor] = None, **kw) -> torch.Tensor:
    """Latent context ``[batch, heads, v_dim]`` of the MLA decode (see the module
    docstring); keyword arguments as ``make_mla_plan``."""
    plan = make_mla_plan(q, pools, page_table, page_counts, page_tags, **kw)
    plan.run()
    return plan.out
