"""Oracle: the KV memory manager's INT8 page transcoding (test infrastructure).

Restates the arithmetic of kv_memory_manager.py's page store:

  write_page, INT8 format (:233-252 of the reference's kv_memory_manager.py):
      kv_fp16 = kv.to(float16)
      max_abs = kv_fp16.abs().max().item()          a Python float (exact float16 value)
      scale   = max_abs / 127.0 if max_abs > 0 else 1.0     Python float (float64)
      codes   = (kv_fp16 / scale).round().clamp(-128, 127).to(int8)
  _read_page_data, INT8 format (:286-296):
      (codes.to(float32) * scale).to(float16)
  set_page_format (:268-284): read the page in its current format, then write it
      in the new one (FP16 -> INT8 demotes, INT8 -> FP16 promotes).
  step (:481-544): the attention it sets up over the selected pages, i.e.
      adaptive_format_attention_reference (adaptive_format_attention.py:25-112)
      on the tensors of _build_attention_tensors (:444-479) after
      _apply_token_masks (:415-438), with its indentation bug undone (as
      written, the reference adds no page to the softmax and returns zeros):
      per selected page, K = V = its rows (FP16 as stored; INT8 as
      float32(code) * float32(float16(scale)); SPARSE: rows at index
      positions < page_size set to the value, for every sparse slot in order,
      padded slots (index 0, value 0) included; no data: zero rows); masked
      rows of FP16 / INT8 pages zeroed; then softmax(q K^T / sqrt(D)) V over
      all rows, divided by max(l, 1e-8), rounded to float16.

Floating-point model (torch on the CPU, which the manager uses): a float16
tensor divided by a Python scalar is computed as float32(x) / float32(scale),
rounded once to float16 (torch's reduced-float division with a scalar operand
keeps the scalar in the op's float32 math); ``round`` is half to even on that
float16 value; a float32 tensor times a Python scalar is float32(x) *
float32(scale), and ``.to(float16)`` rounds that float32 to nearest even. The
float32 value of the scale is therefore all the arithmetic sees; it equals the
correctly rounded float32 quotient max_abs / 127 (the float64 quotient of a
float16 numerator by 127 never lies on a float32 rounding midpoint: the binary
expansion of 1/127 repeats with period 7). NaN quotients convert to code 0.

Pinned by: golden vectors written by the reference's KVMemoryManager
(tests/golden/g6_kv_transcode.npz: write_page, _read_page_data and both
set_page_format directions on seeded pages of three shapes, including
all-zero, subnormal, tie-heavy and near-65504 pages) and the closed forms in
tests/test_oracle_memory.py. The step's rows and attention have no reference
output to pin against (the reference's step returns zeros): they are pinned
by closed forms there (a zero query averages the rows; one dominant row is
selected; zero rows still take softmax mass; the float16 scale rounding is
visible on a crafted page) and the attention by oracle/attention.py's pins.
"""
from __future__ import annotations

from typing import Tuple

import numpy as np


def scale_of(page_f16: np.ndarray) -> Tuple[float, np.float32]:
    """(the manager's float64 scale, its float32 value) for one float16 page."""
    a = np.abs(np.asarray(page_f16, np.float16).astype(np.float64))
    m = float(a.max()) if a.size else 0.0
    s = m / 127.0 if m > 0 else 1.0
    return s, np.float32(s)


def demote_int8(page_f16: np.ndarray) -> Tuple[np.ndarray, float]:
    """write_page's INT8 branch: (int8 codes of the page's shape, float64 scale)."""
    x = np.asarray(page_f16, np.float16)
    s64, s32 = scale_of(x)
    with np.errstate(all="ignore"):
        q16 = (x.astype(np.float32) / s32).astype(np.float16)        # float32 quotient, one rounding to f16
        r = np.rint(q16.astype(np.float64))                           # half to even
        r = np.where(np.isnan(r), 0.0, np.clip(r, -128, 127))
    return r.astype(np.int8), s64


def promote_fp16(codes: np.ndarray, scale: float) -> np.ndarray:
    """_read_page_data's INT8 branch: (codes.float() * scale).half()."""
    with np.errstate(all="ignore"):
        return (np.asarray(codes, np.int8).astype(np.float32) * np.float32(scale)).astype(np.float16)


def step_rows(pages, page_size: int, head_dim: int, sparse_max_nnz: int = 8) -> np.ndarray:
    """The selected pages' K (= V) rows [n * page_size, head_dim] float64.

    ``pages`` lists, per selected page in table order, a dict with ``format``
    ("FP16", "INT8", "SPARSE"), ``data`` (float16 [page_size, head_dim], the
    page as written; None for a page never written) and optionally ``mask``
    (bool [page_size], applied to FP16 / INT8 pages). INT8 pages are demoted
    here with the manager's arithmetic; SPARSE pages keep the top
    ``sparse_max_nnz`` |values| of the flattened page (ties must not occur).
    """
    rows = np.zeros((len(pages), page_size, head_dim), np.float64)
    for j, pg in enumerate(pages):
        fmt, data = pg["format"], pg.get("data")
        if data is None:
            continue
        x = np.asarray(data, np.float16).reshape(page_size, head_dim)
        if fmt == "FP16":
            rows[j] = x.astype(np.float64)
        elif fmt == "INT8":
            codes, s = demote_int8(x)
            s16 = np.float32(np.float16(s))
            rows[j] = (codes.astype(np.float32) * s16).astype(np.float64)
        elif fmt == "SPARSE":
            flat = x.reshape(-1)
            k = min(sparse_max_nnz, flat.size)
            order = np.argsort(-np.abs(flat.astype(np.float64)), kind="stable")[:k]
            slots = [(int(i), float(flat[i])) for i in order] + [(0, 0.0)] * (sparse_max_nnz - k)
            for r, v in slots:
                if 0 <= r < page_size:
                    rows[j, r, :] = v
        m = pg.get("mask")
        if m is not None and fmt in ("FP16", "INT8"):
            rows[j, ~np.asarray(m, bool)] = 0.0
    return rows.reshape(len(pages) * page_size, head_dim)


def step_attention(query: np.ndarray, rows: np.ndarray) -> np.ndarray:
    """[B, H, D] queries over rows [T, D] (K = V): float64 output [B, H, D]."""
    q = np.asarray(query, np.float64)
    D = q.shape[-1]
    if rows.shape[0] == 0:
        return np.zeros(q.shape, np.float64)
    s = q @ rows.T / np.sqrt(D)
    m = s.max(axis=-1, keepdims=True)
    p = np.exp(s - m)
    return (p @ rows) / np.maximum(p.sum(axis=-1, keepdims=True), 1e-8)
