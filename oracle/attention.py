"""Oracle: dense attention and intent_quant_attention_reference.

Restates

  reference.py:16-45                 dense_attention (non-causal path):
                                     softmax(q k^T / sqrt(D)) v
  intent_quant_attention.py:20-119   intent_quant_attention_reference:
                                     per selected block fake-quant -> dequant
                                     -> concatenate -> dense_attention

Reference quirks kept:
* ``causal=True`` raises NotImplementedError mentioning query_positions (:29-35).
* The quantisation granule is the whole block slice ``[..., start:end, :]``,
  i.e. one scale per channel shared across batch and heads
  (intent_quant.py:223 reduces every dim but the last).
* A selected block whose precision is SKIP contributes zero K/V rows, which
  still receive softmax mass exp(0 - max).
* ``torch.cat`` promotes float16 parts next to float32 parts; ``torch.matmul``
  refuses mixed dtypes, so float16 q with any quantised block (or float32 q
  with only FP16 blocks) raises. Restated as a RuntimeError.

The attention is evaluated in float64 (``exact=True``, the default) or in the
dtype torch would use (``exact=False``).

Pinned by: a brute-force softmax on tiny inputs, the reference tests' facts
(empty selection -> zeros, causal raises, semantic == dense over the selected
tokens, test_reference_correctness.py:7-25, test_intent_quant_attention.py)
and golden vectors written by the reference (tests/golden/).
"""
from __future__ import annotations

import math

import numpy as np

from . import quant as Q
from .policy import BlockLayout, IntentQuantizer


def dense_attention(q, k, v, exact: bool = True):
    """reference.py:16-45, causal=False, mask=None."""
    q, k, v = np.asarray(q), np.asarray(k), np.asarray(v)
    if not exact and not (q.dtype == k.dtype == v.dtype):
        raise RuntimeError(
            f"expected m1 and m2 to have the same dtype, but got: {q.dtype} != {k.dtype}")
    dt = np.float64 if exact else q.dtype.type
    scale = 1.0 / math.sqrt(q.shape[-1])
    s = np.matmul(q.astype(dt), np.swapaxes(k.astype(dt), -2, -1)) * dt(scale)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p = p / p.sum(axis=-1, keepdims=True)
    return np.matmul(p, v.astype(dt))


def _promote(parts):
    return np.float32 if any(p.dtype == np.float32 for p in parts) else parts[0].dtype


def intent_quant_attention_reference(q, k, v, layout: BlockLayout, quantizer: IntentQuantizer,
                                     causal: bool = False, exact: bool = True):
    """intent_quant_attention.py:20-86 (output only; debug metrics are not on the path)."""
    if causal:
        raise NotImplementedError(
            "Causal IntentQuant attention requires explicit query_positions "
            "because selected KV indices are in original context coordinates. "
            "The current CPU reference supports non-causal selected-block "
            "attention only.")
    q, k, v = np.asarray(q), np.asarray(k), np.asarray(v)
    layout.validate(k.shape[-2])
    selected = layout.selected_blocks()
    if not selected:
        return np.zeros_like(q)
    k_parts, v_parts = [], []
    for blk in selected:                                            # :56-81
        prec = quantizer.assign_block_precision(blk).precision
        k_parts.append(Q.fake_quantize_tensor(np.ascontiguousarray(k[..., blk.start:blk.end, :]), prec))
        v_parts.append(Q.fake_quantize_tensor(np.ascontiguousarray(v[..., blk.start:blk.end, :]), prec))
    dt = _promote(k_parts)                                          # torch.cat promotion (:83-84)
    K = np.concatenate([p.astype(dt) for p in k_parts], axis=-2)
    V = np.concatenate([p.astype(dt) for p in v_parts], axis=-2)
    if q.dtype != K.dtype:                                          # torch.matmul dtype check
        raise RuntimeError(
            f"expected m1 and m2 to have the same dtype, but got: {q.dtype} != {K.dtype}")
    return dense_attention(q, K, V, exact=exact)
