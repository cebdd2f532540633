"""Oracle: MLA latent decode.

Restates ``_mla_decode_cpu`` (triton_mla_decode.py:155-186), the working
semantics of ``mla_decode_triton`` (:110-152):

  for b, for query position qp:
      online softmax over pages of C (page_size rows each) with
      s = (q . c) / sqrt(d_c); context = acc / l (zeros when no page)
      out[b, qp] = context @ W_VO
  output dtype = q_absorb.dtype

and its closed form ``softmax(q C_sel^T / sqrt(d_c)) C_sel @ W_VO``, which is
what ``mla_sparse_decode_reference`` (mla.py:61-92) computes before its
``.half()``. Evaluated in float64.

``mla_paged_decode_oracle`` is the same computation over paged latent pools
with per-sequence page tables, per-page precision tags (FP16 / FP8 / INT8 with
one scale per page, SKIP pages contributing nothing, as in the fused decode,
fused_selected_quant_decode.py:303-304) and an optional per-sequence token
bound -- the form the MLA kernel takes.

Pinned by: the closed form against the loop on tiny inputs, the reference
test facts (empty page table -> zeros, test_triton_mla_decode.py:52-60; CPU
decode == mla_sparse_decode_reference within 1e-2, :83-111) and golden
vectors written by the reference (tests/golden/); the paged form against the
loop on FP16 pools (tests/test_oracle_decode.py).
"""
from __future__ import annotations

import math
from typing import Dict, Optional

import numpy as np

from . import decode as Dm


def mla_decode_cpu_loop(q_absorb, C, W_VO, page_table, page_size: int = 64):
    """triton_mla_decode.py:155-186, loop for loop (float64)."""
    q_absorb = np.asarray(q_absorb, np.float64)
    C = np.asarray(C, np.float64)
    W = np.asarray(W_VO, np.float64)
    batch, q_len, d_c = q_absorb.shape
    out = np.zeros((batch, q_len, W.shape[1]))
    scale = 1.0 / math.sqrt(d_c)
    for b in range(batch):
        for qp in range(q_len):
            q = q_absorb[b, qp]
            acc = np.zeros(d_c)
            m_i, l_i = -math.inf, 0.0
            for i in range(len(page_table)):
                pid = int(page_table[i])
                c_page = C[pid * page_size:(pid + 1) * page_size]
                s = (q[None, :] * c_page).sum(-1) * scale
                m_ij = s.max()
                p = np.exp(s - m_ij)
                l_ij = p.sum()
                m_new = max(m_i, m_ij)
                alpha = math.exp(m_i - m_new)
                beta = math.exp(m_ij - m_new)
                acc = alpha * acc + beta * (p[:, None] * c_page).sum(0)
                l_i = alpha * l_i + beta * l_ij
                m_i = m_new
            ctx = acc / l_i if m_i > -math.inf else np.zeros(d_c)
            out[b, qp] = ctx @ W
    return out


def mla_decode_closed_form(q_absorb, C_sel, W_VO=None, scale=None):
    """softmax(q C^T * scale) C [@ W_VO] in float64; ``q_absorb`` [..., H, d_qk],
    ``C_sel`` [T, d_qk]; with W_VO None the latent context itself is returned
    (the ``W_VO = [I; 0]`` mapping of the MLA config)."""
    q = np.asarray(q_absorb, np.float64)
    C = np.asarray(C_sel, np.float64)
    if C.shape[0] == 0:
        d_out = C.shape[1] if W_VO is None else np.asarray(W_VO).shape[1]
        return np.zeros(q.shape[:-1] + (d_out,))
    sc = (1.0 / math.sqrt(C.shape[1])) if scale is None else scale
    s = q @ C.T * sc
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    ctx = (p @ C) / p.sum(-1, keepdims=True)
    return ctx if W_VO is None else ctx @ np.asarray(W_VO, np.float64)


def mla_paged_decode_oracle(q, pools: Dict, page_table, page_counts, tags=None, *, v_dim: Optional[int] = None,
                            v_offset: int = 0, sm_scale: Optional[float] = None, valid_tokens=None,
                            neg_ids_wrap: bool = False, page_size: int = 16):
    """float64 latent context ``[B, H, v_dim]``.

    ``q`` [B, H, d]; ``pools`` keys ``c_fp16`` [NP, PS, d] f16, ``c_fp8`` u8 codes
    with ``c_fp8_scale`` [NP], ``c_i8`` with ``c_i8_scale`` [NP] (dequantised as
    ``oracle.decode.dequant_page``); ``page_table`` [B, W]; ``page_counts`` [B]
    (clamped to [0, W]); ``tags`` [NP] native tags or None (all FP16). Table
    entry e of sequence b holds tokens ``e*PS .. e*PS+PS-1``; with
    ``valid_tokens`` only tokens below ``valid_tokens[b]`` exist.
    """
    q = np.asarray(q, np.float64)
    B, H, d = q.shape
    v_dim = d if v_dim is None else v_dim
    sc = 1.0 / math.sqrt(d) if sm_scale is None else sm_scale
    table = np.asarray(page_table)
    W = table.shape[1]
    NP = next(iter(v for k, v in pools.items() if not k.endswith("scale"))).shape[0]
    out = np.zeros((B, H, v_dim))
    for b in range(B):
        n = min(max(int(page_counts[b]), 0), W)
        rows = []
        for e in range(n):
            pid = int(table[b, e])
            if neg_ids_wrap and -NP <= pid < 0:
                pid += NP
            if pid < 0 or pid >= NP:
                continue
            tag = Dm.FP16 if tags is None else int(tags[pid])
            if tag not in (Dm.FP16, Dm.FP8, Dm.INT8):
                continue
            page = Dm.dequant_page(pools, tag, pid, "c")
            lim = page_size if valid_tokens is None else int(valid_tokens[b]) - e * page_size
            if lim <= 0:
                continue
            rows.append(page[:min(lim, page_size)])
        if not rows:
            continue
        C = np.concatenate(rows, axis=0)
        s = q[b] @ C.T * sc
        s = s - s.max(-1, keepdims=True)
        p = np.exp(s)
        out[b] = (p @ C[:, v_offset:v_offset + v_dim]) / p.sum(-1, keepdims=True)
    return out
