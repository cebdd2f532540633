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

Pinned by: the closed form against the loop on tiny inputs, the reference
test facts (empty page table -> zeros, test_triton_mla_decode.py:52-60; CPU
decode == mla_sparse_decode_reference within 1e-2, :83-111) and golden
vectors written by the reference (tests/golden/).
"""
from __future__ import annotations

import math

import numpy as np


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
