"""``intent_quant_attention_reference`` of the reference
(intent_quant_attention.py:20-119) with its attention on the HIP dense-attention kernel.

Semantics kept from the reference, step for step:

* ``causal=True`` raises NotImplementedError (:29-35); the layout is
  validated against ``k.size(-2)`` (:37-38); no selected block gives
  ``zeros_like(q)`` (:40-45);
* each selected block (layout order) takes ``quantizer.assign_block_precision``
  and is fake-quantised with ``fake_quantize_tensor`` at the reference's
  granule: one scale per channel over the block's ``[..., T_blk, D]`` slice
  (:56-75). A block whose precision is SKIP contributes zero K/V rows, which
  take softmax mass like any other row;
* the reconstructions are concatenated in block order (torch's type promotion:
  float16 FP16 blocks next to float32 quantised ones give float32) and
  attended densely (:82-85); a query dtype that differs from the
  concatenation's raises the RuntimeError of the reference's matmul;
* ``return_debug`` returns the same dictionary keys and values: byte
  estimates, per-block precision and reconstruction MSE, and the output's
  error against attention over the unquantised selected tokens (:87-118).

``compare_intent_quant_to_fp16_selected`` (:138-165) sets the output against
``semantic_block_attention`` over the same selected tokens and reports the
reference's keys.

The fake quantisation runs as torch ops on the input's device, batched: the
selected blocks of one precision and length are reconstructed together with
one granule per block and channel (the arithmetic of
``intent_quant.fake_quantize_tensor``, element for element; its error
metrics, which this function never reads, are not computed). The attention
is ``reference.dense_attention`` on libiak's dense attention kernel.
Device tensors only: host tensors raise RuntimeError.
"""
from __future__ import annotations

import functools
import math
from collections import OrderedDict
from typing import Any, Dict, List

import numpy as np
import torch

from . import _native as N
from .block_metadata import BlockLayout
from .decode_core import current_stream_handle, require_device
from .intent_quant import IntentQuantizer, KVPrecision, QuantPolicy, _tdiv, compute_quant_error
from .reference import dense_attention, semantic_block_attention


def _empty_debug(layout: BlockLayout, kv_tokens: int) -> Dict[str, Any]:
    """Debug dictionary of a layout that selects nothing (:120-133)."""
    return {
        "selected_block_names": [], "selected_tokens": 0, "precision_by_block": {},
        "estimated_fp16_bytes": 0, "estimated_quant_bytes": 0, "bytes_saved_pct": 0.0,
        "reconstruction_mse_k": {}, "reconstruction_mse_v": {},
        "output_mse_vs_fp16_selected": 0.0, "output_cosine_vs_fp16_selected": 1.0,
        "output_max_abs_error_vs_fp16_selected": 0.0,
    }


def _recon_stack(x: torch.Tensor, precision: KVPrecision, block_dim: int = 0) -> torch.Tensor:
    """Fake-quant reconstruction of n blocks stacked along ``block_dim`` of ``x``
    (``[n, ..., T, D]`` by default, or ``[..., n, T, D]`` with block_dim -3), one
    scale per block and channel (absmax over every dim but the block dim and the
    last): what ``fake_quantize_tensor`` returns for each block on its own
    (intent_quant.py:221-312), computed for all n at once."""
    if precision == KVPrecision.FP16:
        return x.half()
    if precision == KVPrecision.SKIP:
        return torch.zeros_like(x)
    bd = block_dim % x.ndim
    dims = tuple(d for d in range(x.ndim - 1) if d != bd)

    def scale_of(t: torch.Tensor) -> torch.Tensor:
        return _tdiv(t.abs().amax(dim=dims, keepdim=True), 127.0).clamp(min=1e-8)

    scale = scale_of(x)
    if precision == KVPrecision.FP8:
        return (x / scale).to(torch.float8_e4m3fn).float() * scale
    if precision in (KVPrecision.INT8, KVPrecision.INT4):
        qmax = 127 if precision == KVPrecision.INT8 else 7
        return (x / scale).clamp(-qmax, qmax).round().to(torch.int8).float() * scale
    if precision == KVPrecision.INT4_RESIDUAL:
        base = (x / scale).clamp(-7, 7).round().to(torch.int8).float() * scale
        resid = x - base
        rscale = scale_of(resid)
        return base + (resid / rscale).clamp(-7, 7).round().to(torch.int8).float() * rscale
    raise ValueError(f"Unknown precision: {precision}")


def _reconstruct_selected(k: torch.Tensor, v: torch.Tensor, blocks: List, precs: List[KVPrecision]):
    """The reference's ``torch.cat`` of every selected block's fake-quant
    reconstruction (intent_quant_attention.py:56-84), built with one gather
    and one scatter per (precision, length) group: returns (K, V) over the
    selected tokens in block order, the token index and each block's start.
    The scales are per channel (absmax over every dim but the last), so when K
    and V share their leading shape and dtype they go through one chain,
    side by side along the channel dim, and come back as two views of one
    buffer."""
    def out_dtype(x: torch.Tensor) -> torch.dtype:
        # the dtype torch.cat promotes x's reconstructions to: FP16 blocks are
        # float16, SKIP blocks keep x's dtype (zeros_like), the others are
        # codes.float() * scale, i.e. float32 promoted with x's dtype
        return functools.reduce(torch.promote_types, {
            torch.float16 if p == KVPrecision.FP16 else
            (x.dtype if p == KVPrecision.SKIP else torch.promote_types(torch.float32, x.dtype)) for p in precs})
    spans = tuple((b.start, b.end) for b in blocks)
    if _native_blocks_apply(k, v, sum(e - s for s, e in spans), precs):
        return _reconstruct_native(k, v, spans, precs)
    lens = np.array([b.end - b.start for b in blocks], dtype=np.int64)
    first = np.array([b.start for b in blocks], dtype=np.int64)
    starts = np.concatenate(([0], np.cumsum(lens)))
    total = int(starts[-1])
    # token index of every selected position, and each group's positions, uploaded in one copy
    tok_np = np.repeat(first - starts[:-1], lens) + np.arange(total, dtype=np.int64)
    groups: Dict[tuple, List[int]] = {}
    for i, (n, p) in enumerate(zip(lens.tolist(), precs)):
        groups.setdefault((p, n), []).append(i)
    pos_np = [(starts[idx][:, None] + np.arange(n, dtype=np.int64)[None, :]).reshape(-1)
              for (_, n), idx in groups.items()]
    flat = torch.from_numpy(np.concatenate([tok_np] + pos_np))
    if k.is_cuda:
        # staged in pinned memory (torch's caching host allocator keeps the
        # buffer until the copy has run), so the upload does not wait for the
        # work already queued on the stream
        flat = flat.pin_memory().to(k.device, non_blocking=True)
    tok = flat[:total]
    fused = k.shape[:-1] == v.shape[:-1] and k.dtype == v.dtype
    srcs = [torch.cat([k, v], dim=-1)] if fused else [k, v]
    recs = [torch.empty((*x.shape[:-2], total, x.size(-1)), dtype=out_dtype(x), device=k.device) for x in srcs]
    off = total
    for ((prec, n), idx), pn in zip(groups.items(), pos_np):
        pos = flat[off:off + len(pn)]
        off += len(pn)
        src_tok = tok.index_select(0, pos)
        for src, dst in zip(srcs, recs):
            x = src.index_select(-2, src_tok)                       # [..., len(idx) * n, D]
            x = x.reshape(*x.shape[:-2], len(idx), n, x.shape[-1])
            rec = _recon_stack(x, prec, block_dim=-3)
            dst.index_copy_(-2, pos, rec.reshape(*rec.shape[:-3], len(idx) * n, rec.shape[-1]).to(dst.dtype))
    if fused:
        k_rec, v_rec = recs[0][..., :k.size(-1)], recs[0][..., k.size(-1):]
    else:
        k_rec, v_rec = recs
    return k_rec, v_rec, tok, starts.tolist()


# each precision's metadata string (the member's value), looked up once per block
_VALUE = {p: p.value for p in KVPrecision}

_FQ_CODE = {KVPrecision.FP16: N.FQ_FP16, KVPrecision.FP8: N.FQ_FP8, KVPrecision.INT8: N.FQ_INT8,
            KVPrecision.INT4: N.FQ_INT4, KVPrecision.INT4_RESIDUAL: N.FQ_INT4_RESIDUAL,
            KVPrecision.SKIP: N.FQ_SKIP}


def _native_blocks_apply(k: torch.Tensor, v: torch.Tensor, total: int, precs: List[KVPrecision]) -> bool:
    """Whether libiak's fake-quant kernel builds the reconstruction: float32
    device K and V with the same leading shape (K | V share one output
    buffer), at least one block that is not FP16 (so torch.cat's result is
    float32: FP16 blocks alone concatenate to float16), a non-empty leading
    shape and channels in both K and V, all within the kernel's int32 token
    and row indices and its 2^20 channels."""
    if not (k.is_cuda and k.dtype == torch.float32 and v.dtype == torch.float32
            and k.shape[:-1] == v.shape[:-1] and k.dim() >= 2
            and any(p != KVPrecision.FP16 for p in precs)):
        return False
    lead = math.prod(k.shape[:-2])
    return (0 < total and k.size(-2) < 2 ** 31 and 0 < lead < 2 ** 31
            and k.size(-1) > 0 and v.size(-1) > 0 and k.size(-1) + v.size(-1) <= 2 ** 20)


# block tables of recent layouts: (device, stream, spans, precisions) ->
# (token index, kernel block table, block starts, longest block), on the device
_TABLES: "OrderedDict[tuple, tuple]" = OrderedDict()
_TABLES_SIZE = 16


def _block_tables(dev: torch.device, spans: tuple, precs: List[KVPrecision]):
    """The selected tokens' index and ``iak_fake_quant_blocks``' block table
    (source start, length, output start, precision per block) for these spans
    and precisions, uploaded in one pinned copy on the current stream, and kept
    for later calls over the same layout on the same stream (the tables are
    read-only; at most ``_TABLES_SIZE`` layouts, least recently used first
    out)."""
    key = (dev, current_stream_handle(dev), spans, tuple(precs))
    ent = _TABLES.get(key)
    if ent is not None:
        _TABLES.move_to_end(key)
        return ent
    lens = np.array([e - s for s, e in spans], dtype=np.int64)
    first = np.array([s for s, _ in spans], dtype=np.int64)
    starts = np.concatenate(([0], np.cumsum(lens)))
    total = int(starts[-1])
    tok_np = np.repeat(first - starts[:-1], lens) + np.arange(total, dtype=np.int64)
    meta = np.stack([first, lens, starts[:-1],
                     np.array([_FQ_CODE[p] for p in precs], dtype=np.int64)], axis=1).astype(np.int32)
    flat = torch.from_numpy(np.concatenate([tok_np, meta.reshape(-1).view(np.int64)]))
    flat = flat.pin_memory().to(dev, non_blocking=True)
    ent = (flat[:total], flat[total:].view(torch.int32), tuple(starts.tolist()), int(lens.max()))
    _TABLES[key] = ent
    if len(_TABLES) > _TABLES_SIZE:
        _TABLES.popitem(last=False)
    return ent


def _reconstruct_native(k: torch.Tensor, v: torch.Tensor, spans: tuple, precs: List[KVPrecision]):
    """``_reconstruct_selected`` on libiak's ``iak_fake_quant_blocks``: one
    launch writes every block's K | V reconstruction (float32, bit for bit
    the torch chain's) into ``[..., total, Dk + Dv]``, long blocks split over
    several workgroups through a workspace. The block table comes from
    ``_block_tables`` (one upload per layout and stream)."""
    tok, blocks_dev, starts, longest = _block_tables(k.device, spans, precs)
    total = starts[-1]
    dk, dv = k.size(-1), v.size(-1)
    lead_shape = k.shape[:-2]
    k3 = k.reshape(-1, k.size(-2), dk)
    v3 = v.reshape(-1, v.size(-2), dv)
    k3 = k3 if k3.stride(-1) == 1 or dk <= 1 else k3.contiguous()
    v3 = v3 if v3.stride(-1) == 1 or dv <= 1 else v3.contiguous()
    out = torch.empty((k3.size(0), total, dk + dv), dtype=torch.float32, device=k.device)
    a = N.FakeQuantBlocksArgs()
    a.lead, a.num_blocks, a.k_dim, a.v_dim = k3.size(0), len(precs), dk, dv
    a.k, a.k_stride_l, a.k_stride_t = k3.data_ptr(), k3.stride(0), k3.stride(1)
    a.v, a.v_stride_l, a.v_stride_t = v3.data_ptr(), v3.stride(0), v3.stride(1)
    a.blocks, a.max_block_tokens = blocks_dev.data_ptr(), longest
    a.out, a.out_stride_l, a.out_stride_t = out.data_ptr(), out.stride(0), out.stride(1)
    nws = N.fake_quant_blocks_workspace(a)
    ws = torch.empty(nws, dtype=torch.uint8, device=k.device) if nws else None
    N.fake_quant_blocks(a, current_stream_handle(k.device), ws.data_ptr() if ws is not None else 0, nws)
    out = out.reshape(*lead_shape, total, dk + dv)
    return out[..., :dk], out[..., dk:], tok, list(starts)


def intent_quant_attention_reference(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, layout: BlockLayout,
                                     quantizer: IntentQuantizer, causal: bool = False,
                                     return_debug: bool = False) -> Any:
    """Fake-quant -> dequant -> dense attention over the layout's selected blocks."""
    if causal:
        raise NotImplementedError(
            "Causal IntentQuant attention requires explicit query_positions "
            "because selected KV indices are in original context coordinates. "
            "The current CPU reference supports non-causal selected-block "
            "attention only.")
    require_device(q, k, v, what="IntentQuant attention")
    kv_tokens = k.size(-2)
    layout.validate(kv_tokens)
    blocks = layout.selected_blocks()
    if not blocks:
        out = torch.zeros_like(q)
        return (out, _empty_debug(layout, kv_tokens)) if return_debug else out

    head_dim = q.size(-1)
    precision_by_block: Dict[str, str] = {}
    fp16_bytes = 0
    quant_bytes = 0
    # the policy per block (layout order), then one batched reconstruction per
    # (precision, block length) group
    precs: List[KVPrecision] = []
    for i, block in enumerate(blocks):
        n = block.end - block.start
        policy: QuantPolicy = quantizer.assign_block_precision(block)
        name = _VALUE.get(policy.precision)
        precision_by_block[block.name] = name if name is not None else policy.precision.value
        fp16_bytes += 2 * n * head_dim * 2
        quant_bytes += int(round(2 * n * head_dim * policy.estimated_bytes_per_value))
        precs.append(policy.precision)
    k_rec, v_rec, tok, starts = _reconstruct_selected(k, v, blocks, precs)
    k_err: Dict[str, float] = {}
    v_err: Dict[str, float] = {}
    if return_debug:
        for i, block in enumerate(blocks):
            if precs[i] != KVPrecision.SKIP:
                kd = k_rec[..., starts[i]:starts[i + 1], :]
                vd = v_rec[..., starts[i]:starts[i + 1], :]
                if precs[i] == KVPrecision.FP16:
                    kd, vd = kd.half(), vd.half()
                k_err[block.name] = compute_quant_error(k[..., block.start:block.end, :], kd)["mse"]
                v_err[block.name] = compute_quant_error(v[..., block.start:block.end, :], vd)["mse"]

    output = dense_attention(q, k_rec, v_rec, causal=False)
    if not return_debug:
        return output

    sel_k = k.index_select(-2, tok)
    sel_v = v.index_select(-2, tok)
    fp16_out = dense_attention(q, sel_k, sel_v, causal=False)
    err = compute_quant_error(fp16_out, output)
    saved = (1.0 - quant_bytes / max(fp16_bytes, 1)) * 100.0 if fp16_bytes > 0 else 0.0
    debug: Dict[str, Any] = {
        "selected_block_names": [b.name for b in blocks],
        "selected_tokens": layout.selected_token_count(),
        "precision_by_block": precision_by_block,
        "estimated_fp16_bytes": fp16_bytes,
        "estimated_quant_bytes": quant_bytes,
        "bytes_saved_pct": round(saved, 2),
        "reconstruction_mse_k": k_err,
        "reconstruction_mse_v": v_err,
        "output_mse_vs_fp16_selected": err["mse"],
        "output_cosine_vs_fp16_selected": err["cosine_similarity"],
        "output_max_abs_error_vs_fp16_selected": err["max_abs_error"],
    }
    return output, debug


def compare_intent_quant_to_fp16_selected(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, layout: BlockLayout,
                                          quantizer: IntentQuantizer) -> Dict[str, Any]:
    """Error of the fake-quantised attention against unquantised attention over the
    same selected tokens, with the byte estimates and per-block precisions
    (intent_quant_attention.py:138-165)."""
    fp16_out, fp16_debug = semantic_block_attention(q, k, v, layout, causal=False, return_debug=True)
    quant_out, quant_debug = intent_quant_attention_reference(q, k, v, layout, quantizer, causal=False,
                                                              return_debug=True)
    err = compute_quant_error(fp16_out, quant_out)
    return {
        "output_mse": err["mse"],
        "output_cosine_similarity": err["cosine_similarity"],
        "output_max_abs_error": err["max_abs_error"],
        "fp16_selected_tokens": fp16_debug["selected_token_count"],
        "quant_selected_tokens": quant_debug["selected_tokens"],
        "estimated_fp16_bytes": quant_debug["estimated_fp16_bytes"],
        "estimated_quant_bytes": quant_debug["estimated_quant_bytes"],
        "bytes_saved_pct": quant_debug["bytes_saved_pct"],
        "precision_by_block": quant_debug["precision_by_block"],
        "reconstruction_mse_k": quant_debug["reconstruction_mse_k"],
        "reconstruction_mse_v": quant_debug["reconstruction_mse_v"],
    }
