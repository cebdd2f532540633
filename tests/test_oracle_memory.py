"""Pins the KV memory manager transcoding oracle (oracle/memory.py).

* demote (write_page, INT8) and promote (_read_page_data, INT8) == golden
  vectors written by the reference's KVMemoryManager (g6), bit for bit, and
  both set_page_format directions (INT8 -> FP16 -> INT8);
* closed forms: codes * scale reconstructs within half a code step (plus the
  float16 rounding of the quotient), the absmax element maps to +-127, an
  all-zero page keeps scale 1.0, ties round to even; a planted mistake (the
  exact quotient rounded to an integer without its float16 rounding) fails
  the golden comparison.
"""
import os

import numpy as np
import pytest

from oracle import memory as Mm


@pytest.fixture(scope="module")
def g6(golden_dir):
    return dict(np.load(os.path.join(golden_dir, "g6_kv_transcode.npz")))


@pytest.mark.parametrize("si", [0, 1, 2])
def test_transcode_matches_reference_golden(g6, si):
    x = g6[f"s{si}_x"]
    for p in range(x.shape[0]):
        codes, scale = Mm.demote_int8(x[p])
        assert scale == g6[f"s{si}_scale"][p]
        assert np.array_equal(codes, g6[f"s{si}_codes"][p]), (si, p)
        prom = Mm.promote_fp16(codes, scale)
        assert np.array_equal(prom.view(np.uint16), g6[f"s{si}_promoted"][p].view(np.uint16)), (si, p)
        assert np.array_equal(prom.view(np.uint16), g6[f"s{si}_fp16_back"][p].view(np.uint16))
        codes2, scale2 = Mm.demote_int8(prom)
        assert scale2 == g6[f"s{si}_scale2"][p]
        assert np.array_equal(codes2, g6[f"s{si}_codes2"][p]), (si, p)


def test_closed_forms():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((16, 64)).astype(np.float16)
    codes, s = Mm.demote_int8(x)
    i = np.unravel_index(np.abs(x.astype(np.float64)).argmax(), x.shape)
    assert abs(int(codes[i])) == 127 and np.sign(codes[i]) == np.sign(x[i])
    # half a code step, plus the float16 rounding of the quotient (at most half
    # an ulp of 64..128, 2^-5 of a code step)
    assert np.abs(codes.astype(np.float64) * s - x.astype(np.float64)).max() <= (0.5 + 2 ** -5) * s * (1 + 1e-6)
    z, sz = Mm.demote_int8(np.zeros((4, 8), np.float16))
    assert sz == 1.0 and not z.any()
    # scale 1: a page whose absmax is 127 holds exact ties 0.5, 1.5, 2.5 -> 0, 2, 2
    t = np.zeros((2, 4), np.float16)
    t.flat[:5] = [127, 0.5, 1.5, 2.5, -2.5]
    ct, st = Mm.demote_int8(t)
    assert st == 1.0 and ct.flat[:5].tolist() == [127, 0, 2, 2, -2]


def test_planted_quotient_rounding_mistake_fails(g6):
    """Rounding the exact quotient to an integer directly (skipping the
    float16 rounding of x / scale that the reference's float16 division
    performs) must disagree with the reference somewhere in g6."""
    def wrong(page):
        s64, _ = Mm.scale_of(page)
        q = page.astype(np.float64) / s64
        return np.clip(np.rint(q), -128, 127).astype(np.int8)

    diff = sum(int((wrong(g6[f"s{si}_x"][p]) != g6[f"s{si}_codes"][p]).sum())
               for si in range(3) for p in range(g6[f"s{si}_x"].shape[0]))
    assert diff > 0


def _online_step(q, rows, page_size):
    """The reference's per-page online softmax loop (adaptive_format_attention.py:60-112
    with the update at page level, as its indentation intends), in float64."""
    D = q.shape[-1]
    m, l, acc = -np.inf, 0.0, np.zeros(D)
    for p0 in range(0, rows.shape[0], page_size):
        pk = rows[p0:p0 + page_size]
        s = pk @ q / np.sqrt(D)
        mn = max(m, s.max())
        alpha = np.exp(m - mn) if np.isfinite(m) else 0.0
        p = np.exp(s - mn)
        l = alpha * l + p.sum()
        acc = alpha * acc + p @ pk
        m = mn
    return acc / max(l, 1e-8)


def test_step_attention_closed_forms():
    rng = np.random.default_rng(8)
    PS, D = 4, 16
    pages = [{"format": "FP16", "data": rng.standard_normal((PS, D)).astype(np.float16)},
             {"format": "INT8", "data": rng.standard_normal((PS, D)).astype(np.float16)},
             {"format": "FP16", "data": None}]
    rows = Mm.step_rows(pages, PS, D)
    # the page never written is zero rows, and still takes softmax mass
    assert not rows[2 * PS:].any()
    # a zero query averages every row, the zero rows included
    out0 = Mm.step_attention(np.zeros((1, 1, D)), rows)
    assert np.allclose(out0[0, 0], rows.mean(axis=0), atol=1e-12)
    # the batch softmax equals the reference's per-page online loop
    q = rng.standard_normal((2, 3, D))
    out = Mm.step_attention(q, rows)
    for b in range(2):
        for h in range(3):
            assert np.allclose(out[b, h], _online_step(q[b, h], rows, PS), atol=1e-12)
    # one dominant row is selected
    big = rows[1] * 200.0 / np.linalg.norm(rows[1])
    assert np.allclose(Mm.step_attention(big[None, None], rows)[0, 0], rows[1], atol=1e-6)
    # INT8 rows: codes * float16(scale) within half a code step of the page (plus
    # the float16 rounding of the quotient and of the scale)
    x = pages[1]["data"].astype(np.float64)
    _, s = Mm.demote_int8(pages[1]["data"])
    bound = (0.5 + 2 ** -5) * s + 127 * abs(float(np.float16(s)) - s)
    assert np.abs(rows[PS:2 * PS] - x).max() <= bound * (1 + 1e-6)
    assert Mm.step_attention(np.ones((1, 1, D)), rows[:0]).tolist() == [[[0.0] * D]]


def test_step_rows_sparse_and_mask():
    PS, D = 4, 8
    x = np.zeros((PS, D), np.float16)
    x.flat[[2, 1, 30, 3]] = [9.0, -7.0, 5.0, 0.25]      # flat indices 2, 1, 3 < PS name rows
    rows = Mm.step_rows([{"format": "SPARSE", "data": x}], PS, D, sparse_max_nnz=3)
    # slots by |value|: (2, 9), (1, -7), (30, 5): rows 2 and 1 filled, flat index 30 >= PS dropped
    assert rows[2].tolist() == [9.0] * D and rows[1].tolist() == [-7.0] * D
    assert not rows[0].any() and not rows[3].any()
    # a page smaller than the slot count: padded slots (0, 0.0) zero row 0 last
    y = np.array([[3.0], [-1.0]], np.float16)
    rows = Mm.step_rows([{"format": "SPARSE", "data": y}], 2, 1, sparse_max_nnz=4)
    assert rows[:, 0].tolist() == [0.0, -1.0]
    m = np.array([True, False, True, False])
    z = np.ones((PS, D), np.float16)
    rows = Mm.step_rows([{"format": "FP16", "data": z, "mask": m}], PS, D)
    assert rows[:, 0].tolist() == [1.0, 0.0, 1.0, 0.0]
