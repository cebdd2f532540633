"""Pins oracle/adaptive.py (the adaptive-format decode restatement).

* On FP16 / INT8 / SKIP / SPARSE pages with -1 holes it equals
  oracle.decode.paged_decode_oracle (pinned by golden vectors and brute force)
  with SPARSE mapped to SKIP and the holes removed from the table;
* closed forms: a format outside 0..3 adds page_size zero rows with score 0,
  an all-SKIP row and an all-hole row give zeros;
* a planted mistake (SPARSE pages read as FP16) fails the comparison.
"""
import math

import numpy as np

from oracle import adaptive as Am
from oracle import decode as Dm


def _case(seed, B=2, H=3, D=32, PS=16, NP=12, W=7):
    rng = np.random.default_rng(seed)
    k16 = rng.standard_normal((NP, PS, D)).astype(np.float16)
    v16 = rng.standard_normal((NP, PS, D)).astype(np.float16)
    k8 = rng.integers(-128, 128, (NP, PS, D)).astype(np.int8)
    v8 = rng.integers(-128, 128, (NP, PS, D)).astype(np.int8)
    ks = (rng.random(NP) * 0.02).astype(np.float32)
    vs = (rng.random(NP) * 0.02).astype(np.float32)
    fm = rng.integers(0, 4, NP).astype(np.int32)
    ids = rng.integers(-1, NP, (B, H, W)).astype(np.int32)
    q = rng.standard_normal((B, H, D)).astype(np.float32)
    return q, ids, fm, k16, v16, k8, v8, ks, vs


def _via_paged(q, ids, fm, k16, v16, k8, v8, ks, vs):
    B, H, W = ids.shape
    tags = np.array([{0: Dm.FP16, 1: Dm.INT8}.get(int(f), Dm.SKIP) for f in fm], np.int32)
    pools = {"k_fp16": k16, "v_fp16": v16, "k_i8": k8, "v_i8": v8, "k_i8_scale": ks, "v_i8_scale": vs}
    out = np.zeros(q.shape)
    for b in range(B):
        for h in range(H):
            row = ids[b, h][ids[b, h] >= 0]
            t = row.reshape(1, 1, -1) if row.size else np.zeros((1, 1, 1), np.int32)
            out[b, h] = Dm.paged_decode_oracle(q[b:b + 1, h:h + 1], pools, t, np.array([[row.size]]), tags)[0, 0]
    return out


def test_equals_paged_decode_oracle():
    for seed in range(4):
        args = _case(seed)
        assert np.allclose(Am.adaptive_decode_oracle(*args), _via_paged(*args), atol=1e-12)


def test_planted_sparse_as_fp16_fails():
    q, ids, fm, k16, v16, k8, v8, ks, vs = _case(9)
    fm[:] = 2
    fm[0] = 0
    ids[:, :, 0] = 0
    ids[:, :, 1] = 1
    planted = fm.copy()
    planted[planted == 2] = 0
    good = Am.adaptive_decode_oracle(q, ids, fm, k16, v16, k8, v8, ks, vs)
    assert not np.allclose(good, Am.adaptive_decode_oracle(q, ids, planted, k16, v16, k8, v8, ks, vs), atol=1e-6)


def test_closed_forms():
    q, ids, fm, k16, v16, k8, v8, ks, vs = _case(3, B=1, H=1, W=2)
    PS, D = k16.shape[1], k16.shape[2]
    fm[0], fm[1] = 0, 7
    ids[0, 0] = [0, 1]
    got = Am.adaptive_decode_oracle(q, ids, fm, k16, v16)[0, 0]
    s = k16[0].astype(np.float64) @ q[0, 0].astype(np.float64) / math.sqrt(D)
    m = max(s.max(), 0.0)
    p = np.exp(s - m)
    want = p @ v16[0].astype(np.float64) / (p.sum() + PS * math.exp(-m))
    assert np.allclose(got, want, atol=1e-12)
    fm[:] = 3
    assert not Am.adaptive_decode_oracle(q, ids, fm, k16, v16).any()
    ids[:] = -1
    fm[:] = 0
    assert not Am.adaptive_decode_oracle(q, ids, fm, k16, v16).any()
