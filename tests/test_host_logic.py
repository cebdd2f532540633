"""Host-side logic of the product package against the oracle and the goldens:
router + metadata (exact, list order included), precision policy (exhaustive
grid), fake-quant and fake_int8 utilities (bit-exact on CPU tensors), and the
device requirement of the decode entry points."""
import itertools
import json
import os

import numpy as np
import pytest
import torch

import intent_attention as ia
import importlib
from intent_attention import intent_quant_decode as iqd
from oracle import policy as P
from oracle import quant as Q

# the package re-exports a function under the submodule's name
fsq_mod = importlib.import_module("intent_attention.fused_selected_quant_decode")


@pytest.fixture(scope="module")
def g2(golden_dir):
    with open(os.path.join(golden_dir, "g2_router_metadata.json")) as f:
        return json.load(f)


def _product_layout(blocks):
    return ia.BlockLayout([ia.SemanticBlock(n, s, e, ia.BlockPolicy(pol), sc) for n, s, e, pol, sc in blocks])


def test_product_router_matches_reference_golden(g2):
    for rec in g2:
        router = ia.BlockRouter(ia.RouterConfig(**rec["config"]))
        routed = router.route_layout(_product_layout(rec["blocks"]), rec["total_tokens"])
        assert [[r.name, r.decision.value, r.precision.value, r.reason] for r in routed] == rec["routed"]
        ps = rec["page_size"]
        assert router.selected_page_ids(routed, ps) == rec["selected_page_ids_router"]
        assert router.prefetch_page_ids(routed, ps) == rec["prefetch_page_ids_router"]
        meta = ia.routing_to_kernel_metadata(routed, ps)
        assert meta == rec["meta"]
        assert list(meta["block_precision_by_page"]) == list(rec["meta"]["block_precision_by_page"])
        num_pages = (rec["total_tokens"] + ps - 1) // ps
        pt, prec, pc = ia.metadata_to_kernel_tensors(meta, num_pages, B=2, H=3,
                                                     config=ia.FusedDecodeConfig(max_selected_pages=40))
        assert pt.dtype == torch.int32 and prec.dtype == torch.int32 and pc.dtype == torch.int32
        assert pt.tolist() == rec["kernel"]["page_table"]
        assert prec.tolist() == rec["kernel"]["page_precision"]
        assert pc.tolist() == rec["kernel"]["page_counts"]
        # the native mapping differs only where the reference folds FP8 / INT4*
        _, prec_n, _ = ia.metadata_to_kernel_tensors(meta, num_pages, native_precisions=True)
        _, prec_o, _ = P.metadata_to_kernel_tensors(meta, num_pages, native_precisions=True)
        assert prec_n.tolist() == prec_o.tolist()


def test_product_router_matches_oracle_on_random_layouts():
    rng = np.random.default_rng(99)
    pols = ["ALWAYS", "ATTEND", "ATTEND", "SKIP", "RECENT", "GLOBAL"]
    for trial in range(60):
        blocks, t = [], 0
        for i in range(int(rng.integers(1, 25))):
            ln = int(rng.integers(1, 200))
            pol = pols[int(rng.integers(0, len(pols)))]
            sc = float(np.round(rng.random(), 1)) if (pol == "ATTEND" or rng.random() < .4) else None
            blocks.append([f"b{i}", t, t + ln, pol, sc])
            t += ln + int(rng.integers(0, 40))
        cfg = dict(top_k_blocks=int(rng.integers(0, 10)), score_threshold=float(rng.random()),
                   memory_pressure=float(np.round(rng.random(), 2)), prefetch_top_k=int(rng.integers(0, 6)))
        ps = int(rng.choice([1, 3, 16, 64]))
        r_o = P.BlockRouter(P.RouterConfig(**cfg))
        ro = r_o.route_layout(P.BlockLayout([P.SemanticBlock(*b) for b in blocks]), t)
        r_p = ia.BlockRouter(ia.RouterConfig(**cfg))
        rp = r_p.route_layout(_product_layout(blocks), t)
        assert [(r.name, r.decision, r.precision, r.reason) for r in ro] == \
            [(r.name, r.decision.value, r.precision.value, r.reason) for r in rp]
        assert P.routing_to_kernel_metadata(ro, ps) == ia.routing_to_kernel_metadata(rp, ps)
        assert r_o.prefetch_page_ids(ro, ps) == r_p.prefetch_page_ids(rp, ps)


def test_precision_policy_matches_oracle_on_grid():
    pols = ["ALWAYS", "GLOBAL", "RECENT", "ATTEND", "SKIP"]
    scores = [None, 0.0, 0.39, 0.4, 0.41, 0.74, 0.75, 0.9, 1.0]
    mps = [0.0, 0.3, 0.31, 0.5, 0.51, 0.6, 0.61, 0.7, 0.71, 0.8, 0.81, 0.9, 0.91, 1.0]
    for pol, sc, mp, pr, pg in itertools.product(pols, scores, mps, (True, False), (True, False)):
        o = P.IntentQuantizer(mp, pr, pg).assign_block_precision(P.SemanticBlock("x", 0, 1, pol, sc))
        p = ia.IntentQuantizer(mp, pr, pg).assign_block_precision(
            ia.SemanticBlock("x", 0, 1, ia.BlockPolicy(pol), sc))
        assert (o.precision, o.reason) == (p.precision.value, p.reason), (pol, sc, mp, pr, pg)


@pytest.fixture(scope="module")
def g1(golden_dir):
    return dict(np.load(os.path.join(golden_dir, "g1_fake_quantize.npz")))


@pytest.mark.parametrize("dt", ["f16", "f32"])
@pytest.mark.parametrize("prec", ["FP8", "INT8", "INT4", "INT4_RESIDUAL"])
def test_product_fake_quantize_matches_golden(g1, dt, prec):
    x = torch.from_numpy(g1[f"x_{dt}"]).reshape(-1, 1)
    recon, meta = ia.fake_quantize_tensor(x, ia.KVPrecision(prec))
    ref = g1[f"recon_{dt}_page_{prec}"]
    r = recon.float().numpy()
    assert np.array_equal(r, ref) or np.array_equal(np.isnan(r), np.isnan(ref)) and \
        np.array_equal(r[~np.isnan(r)], ref[~np.isnan(ref)])
    assert np.array_equal(meta["scale"].float().numpy(), g1[f"scale_{dt}_page_{prec}"])


def test_product_fake_int8_variants_match_golden(golden_dir):
    g3 = dict(np.load(os.path.join(golden_dir, "g3_fused_decode.npz")))
    q, s = fsq_mod.fake_int8_pages_from_fp16(torch.from_numpy(g3["k16"]))
    assert np.array_equal(q.numpy(), g3["k8"]) and np.array_equal(s.numpy(), g3["ks"])
    q, s = iqd.fake_int8_pages_from_fp16(torch.from_numpy(g3["edge_pages"]))
    assert np.array_equal(q.numpy(), g3["edge_tq"]) and np.array_equal(s.numpy(), g3["edge_ts"])
    q, s = ia.fake_int8_pages_from_fp16(torch.from_numpy(g3["v16"]))   # package export = fp32 variant
    assert s.dtype == torch.float32 and np.array_equal(q.numpy(), g3["tv8"])


def test_page_table_and_precision_helpers():
    ids, cnt = ia.make_page_tables_from_selected_pages(torch.tensor([0, 2, 5], dtype=torch.int32), 2, 3, 8)
    o_ids, o_cnt = P.make_page_tables_from_selected_pages(np.array([0, 2, 5]), 2, 3, 8)
    assert ids.tolist() == o_ids.tolist() and cnt.tolist() == o_cnt.tolist()
    with pytest.raises(ValueError, match="exceeds max_selected_pages"):
        ia.make_page_tables_from_selected_pages(torch.arange(10), 1, 1, 5)
    with pytest.raises(ValueError, match="must match batch and heads"):
        ia.make_page_tables_from_selected_pages(torch.arange(6).reshape(1, 3, 2), 2, 3)
    with pytest.raises(ValueError, match="must have shape"):
        ia.make_page_tables_from_selected_pages(torch.arange(24).reshape(2, 3, 2, 2), 2, 3)
    prec = ia.make_precision_tensor(10, fp16_pages=torch.tensor([0, 1, 2]), int8_pages=torch.tensor([3, 4]))
    assert prec.tolist() == P.make_precision_tensor(10, [0, 1, 2], [3, 4]).tolist()
    assert [int(t) for t in ia.TritonKVPrecision] == [0, 1, 2, 3, 4, 5]
    assert [int(t) for t in ia.FusedKVPrecision][:3] == [0, 1, 2]


def test_decode_entry_points_refuse_host_tensors():
    x = torch.zeros(1, 1, 1, 64, dtype=torch.float16)
    p = torch.zeros(2, 16, 64, dtype=torch.float16)
    i8 = torch.zeros(2, 16, 64, dtype=torch.int8)
    s = torch.ones(2, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="ROCm device"):
        ia.fused_selected_quant_decode(x, p, p, i8, i8, s, s, torch.zeros(1, 1, 1, dtype=torch.int32),
                                       torch.zeros(2, dtype=torch.int32), torch.ones(1, 1, dtype=torch.int32),
                                       ia.FusedDecodeConfig())
    with pytest.raises(RuntimeError, match="ROCm device"):
        ia.fused_selected_quant_decode_reference(x, p, p, i8, i8, s, s, torch.zeros(1, 1, 1, dtype=torch.int32),
                                                 torch.zeros(2, dtype=torch.int32), torch.ones(1, 1, dtype=torch.int32),
                                                 ia.FusedDecodeConfig())
    with pytest.raises(ValueError, match="head_dim"):
        ia.fused_selected_quant_decode(x, p, p, i8, i8, s, s, torch.zeros(1, 1, 1, dtype=torch.int32),
                                       torch.zeros(2, dtype=torch.int32), torch.ones(1, 1, dtype=torch.int32),
                                       ia.FusedDecodeConfig(head_dim=128))
    if not torch.cuda.is_available():
        with pytest.raises(RuntimeError, match="CUDA is not available"):
            ia.intent_quant_decode_attention_triton(
                x[:, :, 0], p, p, i8, i8, s, s, torch.zeros(1, 1, 64, dtype=torch.int32),
                torch.ones(1, 1, dtype=torch.int32), torch.zeros(2, dtype=torch.int32))


def test_routed_spans_for_the_device_builder(g2):
    """The span arrays routing_to_kernel_tensors uploads: the selected blocks in
    routed order with the metadata_to_kernel_tensors tag of their precision
    (KVPrecision members and names alike), equal to the oracle's spans."""
    from intent_attention.page_tables import _spans
    from intent_attention.fused_selected_quant_decode import precision_tag
    from oracle import policy as P
    for name in ("FP16", "FP8", "INT8", "INT4", "INT4_RESIDUAL", "SKIP"):
        for native in (False, True):
            assert precision_tag(ia.KVPrecision(name), native) == precision_tag(name, native) == \
                P.reference_tag(name, native)
    for rec in g2:
        router = ia.BlockRouter(ia.RouterConfig(**rec["config"]))
        routed = router.route_layout(_product_layout(rec["blocks"]), rec["total_tokens"])
        o_router = P.BlockRouter(P.RouterConfig(**rec["config"]))
        o_routed = o_router.route_layout(P.BlockLayout([P.SemanticBlock(*b) for b in rec["blocks"]]),
                                         rec["total_tokens"])
        for native in (False, True):
            b, e, t = _spans(routed, native)
            assert list(zip(b, e, t)) == P.routed_spans(o_routed, native)


def test_empty_span_has_no_pages():
    """block_router.py:291-295 walks the tokens: a block with end <= start
    selects no page, also when its start is not page-aligned."""
    blocks = [ia.RoutedBlock("a", 17, 17, ia.BlockPolicy.ALWAYS, None, ia.BlockDecision.SELECT,
                             ia.KVPrecision.FP16, ""),
              ia.RoutedBlock("b", 40, 20, ia.BlockPolicy.ALWAYS, None, ia.BlockDecision.SELECT,
                             ia.KVPrecision.INT8, ""),
              ia.RoutedBlock("c", 33, 34, ia.BlockPolicy.ALWAYS, None, ia.BlockDecision.SELECT,
                             ia.KVPrecision.INT8, "")]
    meta = ia.routing_to_kernel_metadata(blocks, 16)
    assert meta["selected_page_ids"] == [2]
    assert meta["block_precision_by_page"] == {"2": "INT8"}


def test_batched_block_reconstruction_equals_per_block():
    """intent_quant_attention_reference reconstructs the selected blocks of one
    precision and length together; each block's slice is bit-identical to the
    product fake_quantize_tensor on that block alone (the G1-pinned arithmetic),
    for every precision, float16 and float32 inputs, with an outlier channel."""
    import torch
    from intent_attention import KVPrecision, fake_quantize_tensor
    from intent_attention.intent_quant_attention import _recon_stack
    g = torch.Generator().manual_seed(5)
    for dt in (torch.float32, torch.float16):
        blocks = [torch.randn(2, 3, 16, 32, generator=g).to(dt) for _ in range(5)]
        blocks[2][..., 7] *= 40.0
        blocks[4].zero_()
        for prec in KVPrecision:
            got = _recon_stack(torch.stack(blocks), prec)
            for j, b in enumerate(blocks):
                want, _ = fake_quantize_tensor(b, prec)
                assert got[j].dtype == want.dtype
                assert torch.equal(got[j], want) or (torch.isnan(want).any() and
                                                      torch.equal(torch.nan_to_num(got[j]), torch.nan_to_num(want))), (dt, prec, j)


def test_grouped_reconstruction_equals_cat_of_blocks():
    """The selected K/V that intent_quant_attention_reference attends over (one
    gather and one scatter per precision and length group) equals the torch.cat
    of each block's own fake_quantize_tensor in block order, dtype included
    (the reference's loop, intent_quant_attention.py:56-84): mixed precisions,
    ragged block lengths, blocks out of token order, float16 and float32."""
    import torch
    from intent_attention import KVPrecision, fake_quantize_tensor
    from intent_attention.block_metadata import BlockPolicy, SemanticBlock
    from intent_attention.intent_quant_attention import _reconstruct_selected
    g = torch.Generator().manual_seed(11)
    spans = [(40, 56), (0, 16), (16, 20), (60, 76), (20, 24), (80, 83), (24, 40)]
    cases = [
        [KVPrecision.INT4, KVPrecision.FP16, KVPrecision.INT8, KVPrecision.INT4,
         KVPrecision.INT8, KVPrecision.SKIP, KVPrecision.FP8],
        [KVPrecision.FP16] * 7,
        [KVPrecision.SKIP, KVPrecision.INT4, KVPrecision.SKIP, KVPrecision.INT4,
         KVPrecision.SKIP, KVPrecision.INT4, KVPrecision.SKIP],
    ]
    for dt in (torch.float32, torch.float16):
        k = torch.randn(2, 3, 90, 32, generator=g).to(dt)
        v = torch.randn(2, 3, 90, 48, generator=g).to(dt)
        k[..., 5] *= 30.0
        blocks = [SemanticBlock(f"b{i}", s, e, BlockPolicy.ATTEND) for i, (s, e) in enumerate(spans)]
        for precs in cases:
            kr, vr, tok, starts = _reconstruct_selected(k, v, blocks, precs)
            want_k = torch.cat([fake_quantize_tensor(k[..., b.start:b.end, :], p)[0] for b, p in zip(blocks, precs)], dim=-2)
            want_v = torch.cat([fake_quantize_tensor(v[..., b.start:b.end, :], p)[0] for b, p in zip(blocks, precs)], dim=-2)
            assert kr.dtype == want_k.dtype and vr.dtype == want_v.dtype, (dt, precs)
            assert torch.equal(kr, want_k) and torch.equal(vr, want_v), (dt, precs)
            assert tok.tolist() == [t for s, e in spans for t in range(s, e)]
            assert starts[-1] == kr.size(-2)
            # K and V of different dtypes take separate chains: the same results
            v2 = v.double() if dt == torch.float32 else v.float()
            kr2, vr2, _, _ = _reconstruct_selected(k, v2, blocks, precs)
            want_v2 = torch.cat([fake_quantize_tensor(v2[..., b.start:b.end, :], p)[0]
                                 for b, p in zip(blocks, precs)], dim=-2)
            assert torch.equal(kr2.to(want_k.dtype), want_k) and torch.equal(vr2.to(want_v2.dtype), want_v2)


def test_precision_enums_are_singletons_under_identity_hash():
    """The string enums hash by identity (their members are singletons compared by
    identity): dict and set lookups, lookups by value and by name, pickling and
    copying all give the same members, and str() is still the metadata string."""
    import copy
    import pickle
    for enum in (ia.KVPrecision, ia.BlockPolicy):
        members = list(enum)
        table = {m: i for i, m in enumerate(members)}
        assert [table[m] for m in members] == list(range(len(members)))
        for m in members:
            assert enum(m.value) is m and enum[m.name] is m
            assert pickle.loads(pickle.dumps(m)) is m and copy.deepcopy(m) is m
            assert str(m) == m.value and len({m, enum(m.value)}) == 1
    assert ia.QuantPolicy(ia.KVPrecision.INT4_RESIDUAL).estimated_bytes_per_value == 1.0
