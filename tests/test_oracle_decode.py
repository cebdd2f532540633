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


# --------------------------------------------------------------------------- #
# dequant_page: the native-precision reconstruction every mixed-precision
# parity result rests on (FP8 / INT8 / INT4 group scales / INT4_RESIDUAL)
# --------------------------------------------------------------------------- #

@pytest.fixture(scope="module")
def g1(golden_dir):
    return dict(np.load(os.path.join(golden_dir, "g1_fake_quantize.npz")))


def _same(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return a.shape == b.shape and bool(np.all((a == b) | (np.isnan(a) & np.isnan(b))))


def _one_page_pools(page, prec, group=32):
    """Pools holding ``page`` (float16 [rows, D]) as page 0 of ``prec``, K and V alike,
    in the packed storage dequant_page reads."""
    from oracle import quant as Q
    tag = {"FP8": Dm.FP8, "INT8": Dm.INT8, "INT4": Dm.INT4, "INT4_RESIDUAL": Dm.INT4_RESIDUAL}[prec]
    codes, scales = Q.quantize_page(page, prec, group)
    pools = {}
    for w in ("k", "v"):
        if prec == "FP8":
            pools[f"{w}_fp8"], pools[f"{w}_fp8_scale"] = codes[None], scales.astype(np.float16)
        elif prec == "INT8":
            pools[f"{w}_i8"], pools[f"{w}_i8_scale"] = codes[None], scales.astype(np.float16)
        elif prec == "INT4":
            pools[f"{w}_i4"], pools[f"{w}_i4_scale"] = Q.pack_int4(codes)[None], scales[None].astype(np.float16)
        else:
            (q1, q2), (s1, s2) = codes, scales
            pools[f"{w}_i4r"] = Q.pack_int4_residual(q1, q2)[None]
            pools[f"{w}_i4r_scale"] = np.array([[s1[0], s2[0]]], np.float32)
    return tag, pools


def _golden_page_recon(g1, prec):
    """The reference's fake_quantize_tensor reconstruction of the 48 x 64 page
    (g1 x_f16 as one page): the page view for FP8 / INT8 / INT4_RESIDUAL, the
    32-channel group view for INT4."""
    if prec == "INT4":
        return g1["recon_f16_group_INT4"].reshape(48, 32, 2).transpose(0, 2, 1).reshape(48, 64)
    return g1[f"recon_f16_page_{prec}"].reshape(48, 64)


@pytest.mark.parametrize("prec", ["FP8", "INT8", "INT4", "INT4_RESIDUAL"])
def test_dequant_page_equals_reference_reconstruction(g1, prec):
    """dequant_page on the packed pool page == what the reference's own
    fake_quantize_tensor returned for that page (golden g1), for K and V."""
    page = g1["x_f16"].reshape(48, 64)
    tag, pools = _one_page_pools(page, prec)
    want = _golden_page_recon(g1, prec)
    for w in ("k", "v"):
        assert _same(Dm.dequant_page(pools, tag, 0, w), want), (prec, w)
    assert Dm.dequant_page(pools, Dm.SKIP, 0, "k") is None
    assert Dm.dequant_page({"k_fp16": page[None]}, Dm.FP16, 0, "k").tolist() == page.astype(np.float64).tolist()


def _page_mutation_cases(g1):
    page = g1["x_f16"].reshape(48, 64)
    # a page whose per-group absmax differs by group, so a wrong group map shows
    skew = (page.astype(np.float32) * np.where(np.arange(64) < 32, 1.0, 3.0)).astype(np.float16)
    return page, skew


def test_dequant_page_planted_group_map_mistake_fails(g1, monkeypatch):
    """np.tile instead of np.repeat over the group scales (channel c reads group
    c mod n instead of c // group) is caught by the golden comparison."""
    page, skew = _page_mutation_cases(g1)
    from oracle import quant as Q
    tag, pools = _one_page_pools(skew, "INT4")
    codes, scales = Q.quantize_page(skew, "INT4", 32)
    good = Q.dequantize_page(codes, scales, "INT4", 32)
    assert _same(Dm.dequant_page(pools, tag, 0, "k"), good)
    monkeypatch.setattr(Dm, "_channel_scales", lambda sc, group: np.tile(sc, group))
    assert not _same(Dm.dequant_page(pools, tag, 0, "k"), good)
    tag, pools = _one_page_pools(page, "INT4")
    assert not _same(Dm.dequant_page(pools, tag, 0, "k"), _golden_page_recon(g1, "INT4"))


def test_dequant_page_planted_residual_slot_swap_fails(g1, monkeypatch):
    """Reading the INT4_RESIDUAL (base, residual) scale slots the other way
    round is caught by the golden comparison."""
    page = g1["x_f16"].reshape(48, 64)
    tag, pools = _one_page_pools(page, "INT4_RESIDUAL")
    want = _golden_page_recon(g1, "INT4_RESIDUAL")
    assert _same(Dm.dequant_page(pools, tag, 0, "v"), want)
    monkeypatch.setattr(Dm, "_residual_scales", lambda pair: (pair[1], pair[0]))
    assert not _same(Dm.dequant_page(pools, tag, 0, "v"), want)


def test_dequant_page_planted_nibble_order_mistake_fails(g1, monkeypatch):
    """Unpacking element 2j from the high nibble (and 2j+1 from the low one) is
    caught by the golden comparison, for INT4 and for INT4_RESIDUAL's base /
    residual nibbles."""
    from oracle import quant as Q
    page = g1["x_f16"].reshape(48, 64)
    tag4, pools4 = _one_page_pools(page, "INT4")
    tagr, poolsr = _one_page_pools(page, "INT4_RESIDUAL")
    real4, realr = Q.unpack_int4, Q.unpack_int4_residual

    def swapped4(p):
        c = real4(p)
        out = c.copy()
        out[..., 0::2], out[..., 1::2] = c[..., 1::2], c[..., 0::2]
        return out

    monkeypatch.setattr(Q, "unpack_int4", swapped4)
    monkeypatch.setattr(Q, "unpack_int4_residual", lambda p: realr(p)[::-1])
    assert not _same(Dm.dequant_page(pools4, tag4, 0, "k"), _golden_page_recon(g1, "INT4"))
    assert not _same(Dm.dequant_page(poolsr, tagr, 0, "k"), _golden_page_recon(g1, "INT4_RESIDUAL"))


@pytest.mark.parametrize("D,group", [(64, 32), (64, 64), (128, 32), (128, 64), (128, 128)])
@pytest.mark.parametrize("scale_f32", [False, True])
def test_dequant_page_every_tag_on_built_pools(D, group, scale_f32):
    """Every page of seeded mixed pools (tests/_pools.build_pools: every tag, K
    with 8-sigma outliers, one all-zero and one tiny-valued page per tag,
    float16 or float32 scale storage) reconstructs bit-for-bit as
    quant.dequantize_page(quant.quantize_page(page)), the g1-pinned
    page-granule reconstruction; group scales read per channel c // group."""
    from oracle import quant as Q
    from tests._pools import build_pools
    rng = np.random.default_rng(D * 1000 + group + int(scale_f32))
    names = ["FP16", "FP8", "INT8", "INT4", "INT4_RESIDUAL", "SKIP"]
    tagv = {"FP16": Dm.FP16, "FP8": Dm.FP8, "INT8": Dm.INT8, "INT4": Dm.INT4,
            "INT4_RESIDUAL": Dm.INT4_RESIDUAL, "SKIP": Dm.SKIP}
    tags = np.array([tagv[n] for n in names for _ in range(4)], np.int32)
    NP = tags.size
    pools = build_pools(rng, NP, D, tags, outliers=0.01, int4_group=group, scale_f32=scale_f32)
    # page 1 of each tag all zero, page 2 tiny (float16 subnormal range); every page is
    # re-quantised below from these sources
    src = {"k": pools["k_fp16"].copy(), "v": pools["v_fp16"].copy()}
    for i in range(len(names)):
        for w in ("k", "v"):
            src[w][4 * i + 1] = 0
            src[w][4 * i + 2] = (rng.standard_normal((16, D)) * 1e-5).astype(np.float16)
    for p in range(NP):
        t = int(tags[p])
        for w in ("k", "v"):
            x = src[w][p]
            if t == Dm.FP16:
                pools[f"{w}_fp16"][p] = x
                want = x.astype(np.float64)
            elif t == Dm.SKIP:
                assert Dm.dequant_page(pools, t, p, w) is None
                continue
            else:
                prec = Dm.TAG_NAMES[t]
                codes, scales = Q.quantize_page(x, prec, group)
                sdt = np.float32 if scale_f32 else np.float16
                if t == Dm.FP8:
                    pools[f"{w}_fp8"][p], pools[f"{w}_fp8_scale"][p] = codes, scales[0]
                elif t == Dm.INT8:
                    pools[f"{w}_i8"][p], pools[f"{w}_i8_scale"][p] = codes, scales[0]
                elif t == Dm.INT4:
                    pools[f"{w}_i4"][p] = Q.pack_int4(codes)
                    pools[f"{w}_i4_scale"][p] = scales.astype(sdt)
                else:
                    (q1, q2), (s1, s2) = codes, scales
                    pools[f"{w}_i4r"][p] = Q.pack_int4_residual(q1, q2)
                    pools[f"{w}_i4r_scale"][p] = (s1[0], s2[0])
                want = Q.dequantize_page(codes, scales, prec, group)
            got = Dm.dequant_page(pools, t, p, w)
            assert _same(got, want), (Dm.TAG_NAMES[t], p, w)
            if t in (Dm.INT4,) and p % 4 == 0:
                # closed form: channel c of token r is code[r, c] * scale[c // group]
                codes = Q.unpack_int4(pools[f"{w}_i4"][p]).astype(np.float64)
                sc = np.asarray(pools[f"{w}_i4_scale"][p], np.float32)
                brute = np.array([[np.float32(codes[r, c] * sc[c // group]) for c in range(D)] for r in range(16)])
                assert _same(got, brute)


def test_valid_tokens_bound_equals_brute_force():
    """paged_decode_oracle with a per-row token bound (a ragged last page) ==
    the textbook softmax over the explicit list of (entry, token) pairs the
    bound keeps; a bound at a page boundary equals truncating the count."""
    rng = np.random.default_rng(17)
    B, Hq, Hkv, D, PS, NP, W = 2, 4, 2, 16, 16, 9, 6
    pools = {"k_fp16": rng.standard_normal((NP, PS, D)).astype(np.float16),
             "v_fp16": rng.standard_normal((NP, PS, D)).astype(np.float16)}
    tags = np.array([0, 0, 2, 0, 0, 0, 0, 0, 0], np.int32)
    table = rng.integers(0, NP, size=(B, Hkv, W)).astype(np.int32)
    counts = np.array([[6, 4], [5, 6]], np.int32)
    bound = np.array([[83, 16], [0, 95]], np.int32)
    q = rng.standard_normal((B, Hq, D)).astype(np.float16)
    out = Dm.paged_decode_oracle(q, pools, table, counts, tags, valid_tokens=bound)
    for b in range(B):
        for h in range(Hq):
            hk = h // 2
            toks = [(int(table[b, hk, e]), t) for e in range(counts[b, hk]) for t in range(PS)
                    if tags[table[b, hk, e]] != 2 and e * PS + t < bound[b, hk]]
            if not toks:
                assert np.all(out[b, h] == 0)
                continue
            s = np.array([float(np.dot(q[b, h].astype(np.float64), pools["k_fp16"][p, t].astype(np.float64)))
                          for p, t in toks]) / math.sqrt(D)
            w = np.exp(s - s.max())
            ref = (w[:, None] * np.array([pools["v_fp16"][p, t] for p, t in toks], np.float64)).sum(0) / w.sum()
            assert np.allclose(out[b, h], ref, rtol=0, atol=1e-12)
    full = Dm.paged_decode_oracle(q, pools, table, np.minimum(counts, 1), tags)
    cut = Dm.paged_decode_oracle(q, pools, table, counts, tags, valid_tokens=np.full((B, Hkv), 16))
    assert np.array_equal(full, cut)
