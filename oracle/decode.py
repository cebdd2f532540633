"""Oracle: fused selected-quant paged decode attention.

Restates ``fused_selected_quant_decode_reference``
(fused_selected_quant_decode.py:267-336), the kernel-semantics spec:

  for each (b, h): for p < page_counts[b, h]:             (:290-299)
      page_id = page_table[b, h, p]; prec = page_precision[page_id]
      SKIP -> continue (no softmax mass)                  (:303-304)
      FP16 -> k, v = pages.float()                        (:306-308)
      INT8 -> k, v = i8.float() * scale.float()           (:309-315)
      other tags -> continue                              (:316-317)
      s = (q . k^T) / sqrt(D); online softmax in fp32     (:323-332)
  out = (acc / max(l, 1e-8)).half()                       (:334)

two ways:

* ``fused_decode_reference_loop`` keeps the loop, the online softmax and the
  float32 arithmetic of the reference (torch-free numpy); it raises
  IndexError where the reference's indexing would (a count above the table
  width). Used for small cases and as the loop-faithful CPU baseline.
* ``paged_decode_oracle`` is the vectorised restatement with this build's
  extension: native tags for FP8 / INT4 (group scales) / INT4_RESIDUAL
  (appended to the fused numbering: FP16 0, INT8 1, SKIP 2, FP8 3, INT4 4,
  INT4_RESIDUAL 5), GQA (a page table per KV head shared by ``Hq // Hkv``
  query heads), and the kernel's guards (counts clamped to the table width,
  page ids outside [0, num_pages) contribute nothing). Dequantisation is the
  reference's (codes times scale, exact in float32); the attention itself is
  evaluated in float64, so it is the exact answer the float32 reference
  approximates. ``dtype=np.float32`` gives the CPU-baseline variant.

Pinned by: the reference tests' facts (all-SKIP -> 0, zero pages -> 0, FP16
path == dense softmax attention over the gathered pages,
test_fused_selected_quant_decode.py:142-224), brute force of the textbook
softmax on tiny inputs, the agreement of the two restatements, and golden
vectors written by the reference's own function (tests/golden/).
``dequant_page`` (the FP8 / INT8 / INT4 / INT4_RESIDUAL reconstruction the
vectorised form and the MLA oracle use) is pinned against the reference's
fake_quantize_tensor reconstructions (golden g1) on packed pool pages and
bit-for-bit against the g1-pinned page-granule reconstruction on seeded pools
of every tag; planted mistakes (tiled group scales, swapped residual scale
slots, swapped nibbles) fail those checks (tests/test_oracle_decode.py).
"""
from __future__ import annotations

import math
from typing import Dict, Optional

import numpy as np

from . import quant as Q

FP16, INT8, SKIP, FP8, INT4, INT4_RESIDUAL = 0, 1, 2, 3, 4, 5
TAG_NAMES = {FP16: "FP16", INT8: "INT8", SKIP: "SKIP", FP8: "FP8", INT4: "INT4",
             INT4_RESIDUAL: "INT4_RESIDUAL"}


def fused_decode_reference_loop(query, k_fp16, v_fp16, k_i8, v_i8, k_scales, v_scales,
                                page_table, page_precision, page_counts, head_dim: int):
    """fused_selected_quant_decode.py:267-336, float32, loop for loop.

    ``query`` [B, H, 1, D]; returns float16 [B, H, 1, D]. ``m_i`` is a Python
    float as in the reference; ``alpha`` is applied to float32 tensors.
    """
    B, H = page_table.shape[:2]
    D = head_dim
    out = np.zeros((B, H, 1, D), dtype=np.float16)
    for b in range(B):
        for h in range(H):
            n = int(page_counts[b, h])
            q = np.asarray(query[b, h, 0, :], np.float32)
            m_i, l_i = -math.inf, np.float32(0.0)
            acc = np.zeros(D, np.float32)
            for p in range(n):
                pid = int(page_table[b, h, p])          # IndexError past the width, as torch
                prec = int(page_precision[pid])
                if prec == SKIP:
                    continue
                if prec == FP16:
                    kb = np.asarray(k_fp16[pid], np.float32)
                    vb = np.asarray(v_fp16[pid], np.float32)
                elif prec == INT8:
                    kb = np.asarray(k_i8[pid], np.float32) * np.float32(k_scales[pid])
                    vb = np.asarray(v_i8[pid], np.float32) * np.float32(v_scales[pid])
                else:
                    continue
                kb, vb = kb.reshape(-1, D), vb.reshape(-1, D)
                s = (q @ kb.T).astype(np.float32) / np.float32(math.sqrt(D))
                m_new = max(m_i, float(s.max()))
                alpha = np.float32(math.exp(m_i - m_new))
                pe = np.exp(s - np.float32(m_new)).astype(np.float32)
                l_i = np.float32(alpha * l_i + pe.sum(dtype=np.float32))
                acc = (alpha * acc + pe @ vb).astype(np.float32)
                m_i = m_new
            out[b, h, 0, :] = (acc / max(float(l_i), 1e-8)).astype(np.float16)
    return out


def dequant_page(pools: Dict, tag: int, pid: int, which: str) -> Optional[np.ndarray]:
    """float64 values of page ``pid`` of K (``which='k'``) or V, as the reference
    reconstructs them (codes times scale, exact in float32); None for SKIP or an
    unknown tag.

    ``pools`` keys: ``{k,v}_fp16`` [NP,PS,D] f16; ``{k,v}_fp8`` [NP,PS,D] u8 codes
    with ``{k,v}_fp8_scale`` [NP]; ``{k,v}_i8`` with ``{k,v}_i8_scale`` [NP];
    ``{k,v}_i4`` [NP,PS,D/2] packed with ``{k,v}_i4_scale`` [NP, D/group];
    ``{k,v}_i4r`` [NP,PS,D] packed with ``{k,v}_i4r_scale`` [NP,2] (base, residual).
    """
    w = which
    f32 = np.float32
    if tag == FP16:
        return np.asarray(pools[f"{w}_fp16"][pid], np.float64)
    if tag == INT8:
        return Q._mul(np.asarray(pools[f"{w}_i8"][pid], np.float64),
                      np.asarray(pools[f"{w}_i8_scale"][pid], f32), f32).astype(np.float64)
    if tag == FP8:
        return Q._mul(Q.e4m3fn_decode(pools[f"{w}_fp8"][pid]),
                      np.asarray(pools[f"{w}_fp8_scale"][pid], f32), f32).astype(np.float64)
    if tag == INT4:
        codes = Q.unpack_int4(pools[f"{w}_i4"][pid])
        sc = np.asarray(pools[f"{w}_i4_scale"][pid], f32).reshape(-1)
        group = codes.shape[-1] // sc.size
        return Q._mul(codes.astype(np.float64), _channel_scales(sc, group)[None, :], f32).astype(np.float64)
    if tag == INT4_RESIDUAL:
        q1, q2 = Q.unpack_int4_residual(pools[f"{w}_i4r"][pid])
        s_base, s_resid = _residual_scales(np.asarray(pools[f"{w}_i4r_scale"][pid], f32).reshape(-1))
        base = Q._mul(q1.astype(np.float64), s_base, f32)
        res = Q._mul(q2.astype(np.float64), s_resid, f32)
        return Q._add(base, res, f32).astype(np.float64)
    return None


def _channel_scales(group_scales: np.ndarray, group: int) -> np.ndarray:
    """Scale of every channel: channels ``g*group .. g*group + group - 1`` share
    group scale g (the group view of intent_quant.py:221-226 reduces over
    ``group`` consecutive channels)."""
    return np.repeat(group_scales, group)


def _residual_scales(pair: np.ndarray):
    """(base scale, residual scale) of an INT4_RESIDUAL page's scale slot pair
    (intent_quant.py:282-307: recon = q1 * s1 + q2 * s2)."""
    return pair[0], pair[1]


def paged_decode_oracle(q, pools: Dict, page_table, page_counts, tags, *,
                        sm_scale: Optional[float] = None, dtype=np.float64,
                        neg_ids_wrap: bool = False, valid_tokens=None):
    """Vectorised selected-page decode with GQA and native precisions.

    ``q`` [B, Hq, D]; ``page_table`` [B, Hkv, W]; ``page_counts`` [B, Hkv];
    ``tags`` [NP] in the native numbering. Returns ``dtype`` [B, Hq, D]. The
    softmax scale defaults to 1/sqrt(D) (reference :323). With
    ``neg_ids_wrap`` a page id in [-NP, 0) means ``id + NP`` (torch indexing
    in the fused reference); otherwise negative ids are invalid (the sibling
    Triton API, triton_intent_quant_attention.py:280). ``valid_tokens``
    [B, Hkv] (this build's extension for a ragged last page): token t of
    table entry e exists only if ``e * PS + t < valid_tokens[b, hk]``.
    Pinned by: brute-force softmax over explicit token lists
    (tests/test_oracle_decode.py).
    """
    q = np.asarray(q)
    B, Hq, D = q.shape
    Hkv, W = page_table.shape[1], page_table.shape[2]
    G = Hq // Hkv
    NP = tags.shape[0]
    scale = (1.0 / math.sqrt(D)) if sm_scale is None else sm_scale
    out = np.zeros((B, Hq, D), dtype=dtype)
    for b in range(B):
        for hk in range(Hkv):
            n = min(int(page_counts[b, hk]), W)
            bound = None if valid_tokens is None else int(valid_tokens[b, hk])
            ks, vs = [], []
            for p in range(n):
                pid = int(page_table[b, hk, p])
                if neg_ids_wrap and -NP <= pid < 0:
                    pid += NP
                if pid < 0 or pid >= NP:
                    continue
                k = dequant_page(pools, int(tags[pid]), pid, "k")
                if k is None:
                    continue
                keep = k.shape[0] if bound is None else max(0, min(k.shape[0], bound - p * k.shape[0]))
                if keep == 0:
                    continue
                ks.append(k[:keep])
                vs.append(dequant_page(pools, int(tags[pid]), pid, "v")[:keep])
            if not ks:
                continue
            K = np.concatenate(ks, 0).astype(dtype)
            V = np.concatenate(vs, 0).astype(dtype)
            qg = q[b, hk * G:(hk + 1) * G, :].astype(dtype)
            s = (qg @ K.T) * dtype(scale)
            s = s - s.max(axis=1, keepdims=True)
            p = np.exp(s)
            out[b, hk * G:(hk + 1) * G, :] = (p @ V) / p.sum(axis=1, keepdims=True)
    return out
