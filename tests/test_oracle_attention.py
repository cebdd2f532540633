"""CPU: pins the oracle's masked / causal dense attention and its selected-block
attention (oracle/attention.py) by an explicit loop over each query's
visible keys and by identities the mathematics fixes, with planted mistakes
that must fail the same checks.

The loop spells out the reference's visibility rules (reference.py:28-43)
key by key: without positions query i sees key j when j <= i; with
positions when positions[j] <= i; an additive mask shifts score (i, j).
"""
import math

import numpy as np
import pytest

from oracle import attention as A
from oracle import policy as P


def _loop(q, k, v, causal=False, mask=None, pos=None):
    """Softmax attention of each (lead, query) row written as a loop over keys."""
    q, k, v = (np.asarray(x, np.float64) for x in (q, k, v))
    lead = q.shape[:-2]
    Tq, Tk, D = q.shape[-2], k.shape[-2], q.shape[-1]
    out = np.zeros(lead + (Tq, v.shape[-1]))
    for li in np.ndindex(*lead):
        for i in range(Tq):
            scores = []
            for j in range(Tk):
                s = float(np.dot(q[li][i], k[li][j])) / math.sqrt(D)
                if causal and pos is None and j > i:
                    s = -math.inf
                if causal and pos is not None and not pos[j] <= i:
                    s = -math.inf
                if mask is not None:
                    s += float(np.broadcast_to(mask, lead + (Tq, Tk))[li][i][j])
                scores.append(s)
            if Tk == 0:
                continue
            m = max(scores)
            if m == -math.inf:
                out[li][i] = np.nan
                continue
            w = [math.exp(s - m) if s != -math.inf else 0.0 for s in scores]
            out[li][i] = sum(wj * v[li][j] for j, wj in enumerate(w)) / sum(w)
    return out


def _qkv(seed, lead=(2, 3), Tq=5, Tk=9, D=8, Dv=None):
    r = np.random.default_rng(seed)
    return (r.standard_normal(lead + (Tq, D)), r.standard_normal(lead + (Tk, D)),
            r.standard_normal(lead + (Tk, Dv or D)))


@pytest.mark.parametrize("seed", range(4))
def test_masked_oracle_equals_key_loop(seed):
    q, k, v = _qkv(seed, Dv=6 if seed % 2 else None)
    r = np.random.default_rng(100 + seed)
    Tq, Tk = q.shape[-2], k.shape[-2]
    pos = np.sort(r.choice(20, Tk, replace=False))
    pos[0] = 0                                         # every query sees at least one key
    mask = r.standard_normal((Tq, Tk))
    mask[r.random((Tq, Tk)) < 0.2] = -np.inf
    mask[:, 0] = 0.0
    bmask = r.random((2, 1, Tq, Tk)) < 0.5
    cases = [dict(), dict(causal=True), dict(causal=True, pos=pos), dict(mask=mask),
             dict(causal=True, pos=pos, mask=mask), dict(mask=bmask)]
    for c in cases:
        got = A.dense_attention_masked(q, k, v, causal=c.get("causal", False), mask=c.get("mask"),
                                       original_kv_positions=c.get("pos"))
        ref = _loop(q, k, v, **c)
        np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12, err_msg=str(list(c)))


def test_masked_oracle_identities():
    q, k, v = _qkv(7, Tq=6, Tk=6)
    Tk = k.shape[-2]
    base = A.dense_attention_masked(q, k, v)
    # positions 0 .. Tk-1 are the triu mask
    np.testing.assert_allclose(A.dense_attention_masked(q, k, v, causal=True, original_kv_positions=np.arange(Tk)),
                               A.dense_attention_masked(q, k, v, causal=True), rtol=1e-13, atol=1e-13)
    # positions without causal change nothing
    np.testing.assert_array_equal(A.dense_attention_masked(q, k, v, original_kv_positions=np.arange(Tk)[::-1]), base)
    # a constant per query row shifts every score of that row: no change
    shift = np.random.default_rng(1).standard_normal((6, 1)) * 5
    np.testing.assert_allclose(A.dense_attention_masked(q, k, v, mask=np.broadcast_to(shift, (6, Tk))), base,
                               rtol=1e-12, atol=1e-12)
    # -inf at key 3 for every query = attention without key 3
    mk = np.zeros((6, Tk))
    mk[:, 3] = -np.inf
    keep = [j for j in range(Tk) if j != 3]
    np.testing.assert_allclose(A.dense_attention_masked(q, k, v, mask=mk), A.dense_attention(q, k[..., keep, :],
                               v[..., keep, :]), rtol=1e-12, atol=1e-12)
    # every key masked: NaN (torch's softmax over -inf); no keys: zeros
    assert np.isnan(A.dense_attention_masked(q, k, v, mask=np.full((6, Tk), -np.inf))).all()
    assert (A.dense_attention_masked(q, k[..., :0, :], v[..., :0, :]) == 0).all()
    # with positions all above query 0, query 0 sees nothing
    o = A.dense_attention_masked(q, k, v, causal=True, original_kv_positions=np.arange(Tk) + 1)
    assert np.isnan(o[..., 0, :]).all() and not np.isnan(o[..., 1:, :]).any()


def test_planted_mistakes_fail_the_loop():
    """Mistakes a restatement could make (off-by-one visibility, a mask of the wrong
    sign, positions read as a prefix length) differ from the key loop."""
    q, k, v = _qkv(3, Tq=6, Tk=8)
    pos = np.array([0, 1, 2, 5, 6, 7, 8, 9])
    ref = _loop(q, k, v, causal=True, pos=pos)

    def off_by_one(q, k, v):
        s = np.matmul(q, np.swapaxes(k, -2, -1)) / math.sqrt(q.shape[-1])
        s = np.where(np.arange(6)[:, None] <= pos[None, :], -np.inf, s)
        return A.dense_attention_masked(q, k, v, mask=np.where(np.isinf(s), -np.inf, 0.0)[0, 0])

    bad = off_by_one(q, k, v)
    assert not np.allclose(np.nan_to_num(bad), np.nan_to_num(ref), atol=1e-6)
    mask = np.random.default_rng(5).standard_normal((6, 8))
    assert not np.allclose(A.dense_attention_masked(q, k, v, mask=-mask), _loop(q, k, v, mask=mask), atol=1e-6)
    prefix = A.dense_attention_masked(q, k, v, causal=True)          # positions ignored
    assert not np.allclose(prefix, ref, atol=1e-6)


def test_semantic_block_attention_reference_facts():
    """The reference's test_causal_attention.py facts, on the oracle."""
    q, k, v = _qkv(11, lead=(1, 2), Tq=6, Tk=16)
    B = P.SemanticBlock
    lay = P.BlockLayout([B("first", 0, 4, "ALWAYS"), B("skip", 4, 10, "SKIP"), B("last", 10, 16, "ALWAYS")])
    idx = np.array([0, 1, 2, 3, 10, 11, 12, 13, 14, 15])
    got = A.semantic_block_attention(q, k, v, lay, causal=True)
    np.testing.assert_allclose(got, _loop(q, k[..., idx, :], v[..., idx, :], causal=True, pos=idx), rtol=1e-12)
    full = P.BlockLayout([B("all", 0, 16, "ALWAYS")])
    np.testing.assert_allclose(A.semantic_block_attention(q, k, v, full, causal=True),
                               A.dense_attention_masked(q, k, v, causal=True), rtol=1e-13, atol=1e-13)
    assert (A.semantic_block_attention(q, k, v, P.BlockLayout([B("s", 0, 16, "SKIP")])) == 0).all()


def test_dynamic_block_scores_closed_form():
    """One unscored ATTEND block whose keys are all q's mean direction scores 1;
    the opposite direction scores 0 (clamped); scored blocks are left alone."""
    r = np.random.default_rng(2)
    q = r.standard_normal((1, 2, 4, 8))
    qd = q.mean(axis=-2).mean(axis=(0, 1))
    k = r.standard_normal((1, 2, 24, 8))
    k[..., 0:8, :] = 3 * qd
    k[..., 8:16, :] = -qd
    B = P.SemanticBlock
    lay = P.BlockLayout([B("same", 0, 8, "ATTEND"), B("opp", 8, 16, "ATTEND"), B("scored", 16, 24, "ATTEND", 0.2)])
    s = A.dynamic_block_scores(q, k, lay)
    assert set(s) == {"same", "opp"}
    assert abs(s["same"] - 1.0) < 1e-9 and s["opp"] == 0.0
