"""Oracle: dense attention and intent_quant_attention_reference.

Restates

  reference.py:16-45                 dense_attention: softmax(q k^T / sqrt(D)) v,
                                     with causal (triu or original KV
                                     positions) and an additive mask
  reference.py:81-129                semantic_block_attention (selected tokens,
                                     ATTEND blocks scored by block_scorer.py:17-34)
  intent_quant_attention.py:138-165  compare_intent_quant_to_fp16_selected
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
tokens, test_reference_correctness.py:7-25, test_intent_quant_attention.py,
test_causal_attention.py) and golden vectors written by the reference
(tests/golden/). ``dense_attention_masked`` is pinned by an explicit loop
over each query's visible keys (tests/test_oracle_attention.py) and by
identities: positions 0 .. Tk-1 equal the triu mask, a -inf mask entry
equals dropping that key, a per-row constant mask changes nothing.
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


def dense_attention_masked(q, k, v, causal: bool = False, mask=None, original_kv_positions=None):
    """reference.py:16-45 in float64 with every branch: scores (q k^T) / sqrt(D);
    causal without positions adds triu(-inf, 1); causal with positions sets
    scores[i, j] = -inf where i < positions[j] (:31-34); then ``+ mask`` (a bool
    mask adds 1.0); softmax (NaN where every score is -inf); zeros for no keys."""
    q, k, v = (np.asarray(x, dtype=np.float64) for x in (q, k, v))
    Tq, Tk = q.shape[-2], k.shape[-2]
    s = np.matmul(q, np.swapaxes(k, -2, -1)) / math.sqrt(q.shape[-1])
    if causal:
        if original_kv_positions is not None:
            pos = np.asarray(original_kv_positions)
            s = np.where(np.arange(Tq)[:, None] < pos[None, :], -np.inf, s)
        else:
            s = s + np.triu(np.full((Tq, Tk), -np.inf), k=1)
    if mask is not None:
        s = s + np.asarray(mask).astype(np.float64)
    if Tk == 0:
        return np.zeros(s.shape[:-1] + (v.shape[-1],))
    with np.errstate(invalid="ignore"):
        m = s.max(axis=-1, keepdims=True)
        p = np.exp(s - m)
        p = p / p.sum(axis=-1, keepdims=True)
    return np.matmul(p, v)


def dynamic_block_scores(q, k, layout: BlockLayout) -> dict:
    """reference.py:52-78 / block_scorer.py:17-34: the cosine of the query's mean
    (over rows, then the first two dims) with each unscored ATTEND block's mean
    key, clamped at 0 (float64)."""
    q, k = np.asarray(q, np.float64), np.asarray(k, np.float64)
    qg = q.mean(axis=-2).mean(axis=(0, 1))
    qn = qg / (np.linalg.norm(qg) + 1e-10)
    out = {}
    for b in layout.blocks:
        if b.policy == "ATTEND" and b.score is None:
            r = k[..., b.start:b.end, :].mean(axis=-2).mean(axis=(0, 1))
            out[b.name] = max(0.0, float(qn @ (r / (np.linalg.norm(r) + 1e-10))))
    return out


def semantic_block_attention(q, k, v, layout: BlockLayout, causal: bool = False):
    """reference.py:81-129 (output only): attention over the selected tokens, keys at
    their original positions. Unscored ATTEND blocks must be scored by the caller."""
    layout.validate(np.asarray(k).shape[-2])
    idx = np.asarray([t for b in layout.selected_blocks() for t in range(b.start, b.end)],   # block_metadata.py:75-79
                     dtype=np.int64)
    if idx.size == 0:
        return np.zeros(np.asarray(q).shape)
    k, v = np.asarray(k)[..., idx, :], np.asarray(v)[..., idx, :]
    return dense_attention_masked(q, k, v, causal=causal, original_kv_positions=idx)


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
