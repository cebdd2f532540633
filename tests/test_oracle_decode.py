"""Pins the decode, attention and MLA oracles.

* fused_decode_reference_loop and paged_decode_oracle == the reference's
  fused_selected_quant_decode_reference output (g3), for both scale variants.
* the two restatements agree with each other on mixed FP16/INT8/SKIP inputs,
  and the vectorised one equals a brute-force textbook softmax.
* intent_quant_attention_reference and dense_attention == golden (g4),
  including the cfg1 shape with its alternating FP16/INT8 plan.
* _mla_decode_cpu loop and its closed form == golden (g5).
* reference test facts: all-SKIP -> 0, zero pages -> 0, causal raises.
"""
import math
import os

import numpy as np
import pytest

from oracle import attention as A
from oracle import decode as Dm
from oracle import mla as M
from oracle import policy as P


@pytest.fixture(scope="module")
def g3(golden_dir):
    return dict(np.load(os.path.join(golden_dir, "g3_fused_decode.npz")))


def _pools_from_g3(g, triton_scales=False):
    pre = "t" if triton_scales else ""
    return {"k_fp16": g["k16"], "v_fp16": g["v16"], "k_i8": g[f"{pre}k8"], "v_i8": g[f"{pre}v8"],
            "k_i8_scale": g[f"{pre}ks"], "v_i8_scale": g[f"{pre}vs"]}


@pytest.mark.parametrize("triton_scales", [False, True])
def test_fused_reference_golden(g3, triton_scales):
    pre = "t" if triton_scales else ""
    ref = g3["out_triton_scales" if triton_scales else "out"]
    loop = Dm.fused_decode_reference_loop(
        g3["q"], g3["k16"], g3["v16"], g3[f"{pre}k8"], g3[f"{pre}v8"], g3[f"{pre}ks"], g3[f"{pre}vs"],
        g3["page_table"], g3["page_precision"], g3["page_counts"], 64)
    assert loop.dtype == np.float16
    # same float32 algorithm: at most one float16 ulp from summation order
    assert np.abs(loop.astype(np.float32) - ref.astype(np.float32)).max() <= 2e-3
    vec = Dm.paged_decode_oracle(g3["q"][:, :, 0, :], _pools_from_g3(g3, triton_scales),
                                 g3["page_table"], g3["page_counts"], g3["page_precision"])
    assert np.abs(vec - ref[:, :, 0, :].astype(np.float64)).max() <= 2e-3
    # the exact answer rounded to float16 is within half an ulp + reference rounding
    assert np.abs(vec.astype(np.float16).astype(np.float32) - ref[:, :, 0, :]).max() <= 2e-3


def test_all_skip_and_zero_pages_give_zero(g3):
    pools = _pools_from_g3(g3)
    q = g3["q"][:, :, 0, :]
    skip = np.full(8, Dm.SKIP, np.int32)
    out = Dm.paged_decode_oracle(q, pools, g3["page_table"], g3["page_counts"], skip)
    assert np.abs(out).max() == 0.0
    loop = Dm.fused_decode_reference_loop(g3["q"], g3["k16"], g3["v16"], g3["k8"], g3["v8"], g3["ks"],
                                          g3["vs"], g3["page_table"], skip, g3["page_counts"], 64)
    assert np.abs(loop.astype(np.float32)).max() == 0.0
    zero = np.zeros_like(g3["page_counts"])
    assert np.abs(Dm.paged_decode_oracle(q, pools, g3["page_table"], zero, g3["page_precision"])).max() == 0


def test_count_above_width_raises_in_reference_loop(g3):
    pc = g3["page_counts"].copy()
    pc[0, 0] = g3["page_table"].shape[2] + 1
    with pytest.raises(IndexError):
        Dm.fused_decode_reference_loop(g3["q"], g3["k16"], g3["v16"], g3["k8"], g3["v8"], g3["ks"],
                                       g3["vs"], g3["page_table"], g3["page_precision"], pc, 64)


def test_vectorised_equals_brute_force_softmax():
    rng = np.random.default_rng(7)
    B, Hq, Hkv, D, PS, NP, W = 2, 4, 2, 16, 4, 6, 5
    pools = {"k_fp16": rng.standard_normal((NP, PS, D)).astype(np.float16),
             "v_fp16": rng.standard_normal((NP, PS, D)).astype(np.float16)}
    tags = np.array([0, 0, 2, 0, 0, 0], np.int32)
    table = rng.integers(0, NP, size=(B, Hkv, W)).astype(np.int32)
    counts = np.array([[5, 2], [0, 3]], np.int32)
    q = rng.standard_normal((B, Hq, D)).astype(np.float16)
    out = Dm.paged_decode_oracle(q, pools, table, counts, tags)
    for b in range(B):
        for h in range(Hq):
            hk = h // 2
            toks = [(pid, t) for pid in table[b, hk, :counts[b, hk]] if tags[pid] != 2 for t in range(PS)]
            if not toks:
                assert np.all(out[b, h] == 0)
                continue
            s = [sum(float(q[b, h, d]) * float(pools["k_fp16"][p, t, d]) for d in range(D)) / math.sqrt(D)
                 for p, t in toks]
            mx = max(s)
            w = [math.exp(x - mx) for x in s]
            ref = [sum(wi * float(pools["v_fp16"][p, t, d]) for wi, (p, t) in zip(w, toks)) / sum(w)
                   for d in range(D)]
            assert np.allclose(out[b, h], ref, rtol=0, atol=1e-12)


@pytest.fixture(scope="module")
def g4(golden_dir):
    return dict(np.load(os.path.join(golden_dir, "g4_intent_quant_attention.npz")))


class _Plan:
    def __init__(self, plan):
        self.plan = plan

    def assign_block_precision(self, block):
        return P.QuantPolicy(self.plan[block.name])


def test_intent_quant_attention_cfg1_golden(g4):
    pages = [int(p) for p in g4["cfg1_pages"]]
    k = np.zeros((1, 8, 1024, 64), np.float32)
    v = np.zeros((1, 8, 1024, 64), np.float32)
    tok = np.array([p * 16 + t for p in pages for t in range(16)])
    k[:, :, tok] = g4["cfg1_k_sel"].astype(np.float32)
    v[:, :, tok] = g4["cfg1_v_sel"].astype(np.float32)
    q = g4["cfg1_q"].astype(np.float32)
    blocks, plan = [], {}
    for rank, p in enumerate(pages):
        pol = "ALWAYS" if p < 4 else ("RECENT" if p >= 56 else "ATTEND")
        blocks.append(P.SemanticBlock(f"p{p}", p * 16, p * 16 + 16, pol, 0.9 if pol == "ATTEND" else None))
        plan[f"p{p}"] = "FP16" if rank % 2 == 0 else "INT8"
    out = A.intent_quant_attention_reference(q, k, v, P.BlockLayout(blocks), _Plan(plan))
    assert np.abs(out - g4["cfg1_out"]).max() < 2e-6


def test_intent_quant_attention_mixed_golden(g4):
    q, k, v = g4["mix_q"], g4["mix_k"], g4["mix_v"]
    S = P.SemanticBlock
    layout = P.BlockLayout([S("a", 0, 16, "ALWAYS"), S("b", 16, 40, "ATTEND", 0.5),
                            S("c", 40, 56, "ATTEND", 0.1), S("d", 56, 80, "RECENT"), S("e", 80, 96, "SKIP")])
    plan = {"a": "FP8", "b": "INT4_RESIDUAL", "c": "SKIP", "d": "INT4"}
    out = A.intent_quant_attention_reference(q, k, v, layout, _Plan(plan))
    assert np.abs(out - g4["mix_out"]).max() < 2e-6
    out2 = A.intent_quant_attention_reference(q, k, v, layout, P.IntentQuantizer(memory_pressure=0.5))
    assert np.abs(out2 - g4["mix_out_default"]).max() < 2e-6


def test_intent_quant_attention_reference_facts(g4):
    q, k, v = g4["mix_q"], g4["mix_k"], g4["mix_v"]
    layout = P.BlockLayout([P.SemanticBlock("s", 0, 16, "SKIP")])
    assert np.all(A.intent_quant_attention_reference(q, k, v, layout, P.IntentQuantizer()) == 0)
    with pytest.raises(NotImplementedError, match="query_positions"):
        A.intent_quant_attention_reference(q, k, v, layout, P.IntentQuantizer(), causal=True)
    # float16 q with a quantised block: the reference's matmul refuses mixed dtypes
    lay = P.BlockLayout([P.SemanticBlock("a", 0, 16, "ATTEND", 0.9)])
    with pytest.raises(RuntimeError):
        A.intent_quant_attention_reference(q.astype(np.float16), k.astype(np.float16),
                                           v.astype(np.float16), lay, P.IntentQuantizer())


@pytest.fixture(scope="module")
def g5(golden_dir):
    return dict(np.load(os.path.join(golden_dir, "g5_mla_decode.npz")))


def test_mla_decode_golden(g5):
    ps = int(g5["page_size"])
    out = M.mla_decode_cpu_loop(g5["q_absorb"], g5["C"], g5["W_VO"], g5["page_table"], ps)
    assert np.abs(out - g5["out"]).max() < 1e-4
    Csel = np.concatenate([g5["C"][p * ps:(p + 1) * ps] for p in g5["page_table"]], 0)
    cf = M.mla_decode_closed_form(g5["q_absorb"], Csel, g5["W_VO"])
    assert np.abs(cf - g5["out"]).max() < 1e-4
    empty = M.mla_decode_cpu_loop(g5["q_absorb"], g5["C"], g5["W_VO"], [], ps)
    assert np.all(empty == 0) and np.all(g5["out_empty"] == 0)


def test_mla_paged_oracle_equals_reference_loop():
    """The paged form (per-sequence tables, tags, token bound) reduces to the
    restated reference loop on an FP16 pool with full pages, and a token bound
    equals truncating the gathered rows."""
    rng = np.random.default_rng(7)
    B, H, d, NP = 2, 5, 32, 12
    pool = rng.standard_normal((NP, 16, d)).astype(np.float16)
    q = rng.standard_normal((B, H, d))
    ids = np.array([3, 0, 7, 7, 11], np.int32)
    table = np.stack([ids, ids])
    counts = np.array([5, 5])
    got = M.mla_paged_decode_oracle(q, {"c_fp16": pool}, table, counts)
    ref = M.mla_decode_cpu_loop(q, pool.reshape(-1, d), np.eye(d), ids, page_size=16)
    assert np.abs(got - ref).max() < 1e-12
    # token bound of 70 = 4 full pages + 6 tokens of the fifth
    got = M.mla_paged_decode_oracle(q, {"c_fp16": pool}, table, counts, valid_tokens=np.array([70, 70]))
    rows = np.concatenate([pool[p].astype(np.float64) for p in ids], 0)[:70]
    assert np.abs(got - M.mla_decode_closed_form(q, rows)).max() < 1e-12
    # SKIP pages and a zero count contribute nothing
    tags = np.zeros(NP, np.int32)
    tags[7] = Dm.SKIP
    got = M.mla_paged_decode_oracle(q, {"c_fp16": pool}, table, np.array([5, 0]), tags)
    rows = np.concatenate([pool[p].astype(np.float64) for p in (3, 0, 11)], 0)
    assert np.abs(got[0] - M.mla_decode_closed_form(q[:1], rows)[0]).max() < 1e-12
    assert np.all(got[1] == 0)
