"""Pins the router / metadata oracle (oracle/policy.py).

* Every record of tests/golden/g2_router_metadata.json (written by the
  reference's BlockRouter and routing_to_kernel_metadata on 9 layouts x 5
  router configs x 2 page sizes): routed decisions, precisions, reasons,
  selected/prefetch ids, the metadata dict (including key order) and the
  kernel tensors of metadata_to_kernel_tensors.
* The hand-derived answer for the reference tests' basic layout.
* The reference tests' own facts (test_block_router.py,
  test_fused_selected_quant_decode.py:258-286, test_intent_quant.py,
  test_triton_intent_quant_attention.py:28-101).
"""
import json
import os

import numpy as np
import pytest

from oracle import policy as P


@pytest.fixture(scope="module")
def g2(golden_dir):
    with open(os.path.join(golden_dir, "g2_router_metadata.json")) as f:
        return json.load(f)


def _layout(blocks):
    return P.BlockLayout([P.SemanticBlock(n, s, e, pol, sc) for n, s, e, pol, sc in blocks])


def test_router_and_metadata_match_reference_golden(g2):
    assert len(g2) == 90
    for rec in g2:
        layout = _layout(rec["blocks"])
        router = P.BlockRouter(P.RouterConfig(**rec["config"]))
        routed = router.route_layout(layout, rec["total_tokens"])
        assert [[r.name, r.decision, r.precision, r.reason] for r in routed] == rec["routed"]
        ps = rec["page_size"]
        assert router.selected_page_ids(routed, ps) == rec["selected_page_ids_router"]
        assert router.prefetch_page_ids(routed, ps) == rec["prefetch_page_ids_router"]
        meta = P.routing_to_kernel_metadata(routed, ps)
        assert meta == rec["meta"]
        assert list(meta["block_precision_by_page"]) == list(rec["meta"]["block_precision_by_page"])
        num_pages = (rec["total_tokens"] + ps - 1) // ps
        pt, prec, pc = P.metadata_to_kernel_tensors(meta, num_pages, B=2, H=3, max_selected=40)
        assert pt.tolist() == rec["kernel"]["page_table"]
        assert prec.tolist() == rec["kernel"]["page_precision"]
        assert pc.tolist() == rec["kernel"]["page_counts"]


def _basic():
    S = P.SemanticBlock
    return P.BlockLayout([S("system", 0, 64, "ALWAYS"), S("doc_high", 64, 192, "ATTEND", 0.9),
                          S("doc_low", 192, 320, "ATTEND", 0.1), S("recent", 320, 384, "RECENT"),
                          S("unused", 384, 448, "SKIP")])


def test_basic_layout_known_answer():
    router = P.BlockRouter(P.RouterConfig())
    routed = router.route_layout(_basic(), 448)
    assert [(r.name, r.decision, r.precision) for r in routed] == [
        ("system", "PIN_HIGH_PRECISION", "FP16"), ("recent", "SELECT", "FP8"),
        ("doc_high", "QUANTIZE", "INT8"), ("doc_low", "SKIP", "SKIP"), ("unused", "SKIP", "SKIP")]
    meta = P.routing_to_kernel_metadata(routed, 16)
    # routed order, first-seen dedupe, NOT sorted (RECENT pages precede ATTEND pages)
    assert meta["selected_page_ids"] == [0, 1, 2, 3, 20, 21, 22, 23, 4, 5, 6, 7, 8, 9, 10, 11]
    assert meta["block_precision_by_page"] == {
        **{str(i): "FP16" for i in range(4)}, **{str(i): "INT8" for i in range(4, 12)},
        **{str(i): "FP8" for i in range(20, 24)}}
    assert list(meta["block_precision_by_page"]) == [str(i) for i in list(range(12)) + list(range(20, 24))]
    # block_router.py:329-335 unpacks (page, score) pairs as (score, page): the list
    # holds distinct SCORES; every candidate here scores 1.0.
    assert meta["prefetch_page_ids"] == [1.0]
    assert meta["selected_block_names"] == ["system", "recent", "doc_high"]
    assert meta["skipped_block_names"] == ["doc_low", "unused"]
    pt, prec, pc = P.metadata_to_kernel_tensors(meta, 28)
    assert pc.tolist() == [[16]] and pt.shape == (1, 1, 64)
    assert prec.tolist() == [0] * 4 + [1] * 8 + [0] * 16   # FP8 pages 20-23 map to FP16
    _, prec_n, _ = P.metadata_to_kernel_tensors(meta, 28, native_precisions=True)
    assert prec_n.tolist() == [0] * 4 + [1] * 8 + [0] * 8 + [3] * 4 + [0] * 4


def test_metadata_conversion_reference_facts():
    meta = {"selected_page_ids": [0, 3, 5], "block_precision_by_page": {"0": "FP16", "3": "INT8", "5": "SKIP"}}
    pt, prec, pc = P.metadata_to_kernel_tensors(meta, num_pages=8)
    assert pt.shape == (1, 1, 64) and prec.shape == (8,) and pc.shape == (1, 1)
    assert prec[0] == 0 and prec[3] == 1 and prec[5] == 2 and pc[0, 0] == 3
    pt, prec, pc = P.metadata_to_kernel_tensors({"selected_page_ids": [], "block_precision_by_page": {}}, 4)
    assert pt.sum() == 0 and pc.sum() == 0 and (prec == 0).all()
    # non-integer keys are skipped; truncation to max_selected
    meta = {"selected_page_ids": list(range(10)), "block_precision_by_page": {"x": "INT8", "2": "INT4"}}
    pt, prec, pc = P.metadata_to_kernel_tensors(meta, 12, B=2, H=2, max_selected=4)
    assert pc.tolist() == [[4, 4], [4, 4]] and pt[1, 1].tolist() == [0, 1, 2, 3] and prec[2] == 1


def test_policy_table_reference_facts():
    q0, q95 = P.IntentQuantizer(0.0), P.IntentQuantizer(0.95)
    S = P.SemanticBlock
    assert q0.assign_block_precision(S("a", 0, 1, "ALWAYS")).precision == "FP16"
    assert q0.assign_block_precision(S("g", 0, 1, "GLOBAL")).precision == "FP16"
    assert q95.assign_block_precision(S("a", 0, 1, "ALWAYS")).precision == "INT8"
    assert q0.assign_block_precision(S("s", 0, 1, "SKIP")).precision == "SKIP"
    assert q0.assign_block_precision(S("l", 0, 1, "ATTEND", 0.1)).precision == "INT4"
    assert P.IntentQuantizer(0.5).assign_block_precision(S("l", 0, 1, "ATTEND", 0.1)).precision == "SKIP"
    assert q0.assign_block_precision(S("m", 0, 1, "ATTEND", 0.5)).precision == "INT4_RESIDUAL"
    pol = P.QuantPolicy("INT4_RESIDUAL")
    assert pol.estimated_bytes_per_value == 1.0 and pol.requires_scale and pol.uses_residual
    with pytest.raises(ValueError):
        P.IntentQuantizer(1.5)


def test_layout_validation_messages():
    S = P.SemanticBlock
    with pytest.raises(ValueError, match="score is None"):
        P.BlockLayout([S("a", 0, 4, "ATTEND")]).validate(8)
    with pytest.raises(ValueError, match="overlap"):
        P.BlockLayout([S("a", 0, 4, "ALWAYS"), S("b", 3, 6, "ALWAYS")]).validate(8)
    with pytest.raises(ValueError, match="total_tokens"):
        P.BlockLayout([S("a", 0, 9, "ALWAYS")]).validate(8)


def test_page_table_helpers_reference_facts():
    ids, cnt = P.make_page_tables_from_selected_pages(np.array([0, 2, 5]), 2, 3, 8)
    assert ids.shape == (2, 3, 8) and (cnt == 3).all()
    assert (ids[:, :, :3] == [0, 2, 5]).all() and (ids[:, :, 3:] == -1).all()
    with pytest.raises(ValueError, match="exceeds max_selected_pages"):
        P.make_page_tables_from_selected_pages(np.arange(10), 1, 1, 5)
    with pytest.raises(ValueError, match="must match batch and heads"):
        P.make_page_tables_from_selected_pages(np.arange(6).reshape(1, 3, 2), 2, 3)
    prec = P.make_precision_tensor(10, fp16_pages=[0, 1, 2], int8_pages=[3, 4])
    assert prec.tolist() == [0, 0, 0] + [2] * 7
    assert P.TRITON_TAG == {"FP16": 0, "FP8": 1, "INT8": 2, "INT4": 3, "INT4_RESIDUAL": 4, "SKIP": 5}


# --------------------------------------------------------------------------- #
# build_page_tables_oracle: the device page-table builder's semantics
# --------------------------------------------------------------------------- #

def _g2_routed(rec):
    router = P.BlockRouter(P.RouterConfig(**rec["config"]))
    return router.route_layout(_layout(rec["blocks"]), rec["total_tokens"])


def test_page_table_oracle_matches_reference_golden(g2):
    """One list broadcast to B*H rows, identity pages: the reference's kernel
    tensors of every G2 record, in both precision mappings."""
    for rec in g2:
        routed = _g2_routed(rec)
        ps = rec["page_size"]
        num_pages = (rec["total_tokens"] + ps - 1) // ps
        pt, prec, pc = P.build_page_tables_oracle([P.routed_spans(routed)], 6, 40, ps, num_pages)
        assert pt.reshape(2, 3, 40).tolist() == rec["kernel"]["page_table"]
        assert prec.tolist() == rec["kernel"]["page_precision"]
        assert pc.reshape(2, 3).tolist() == rec["kernel"]["page_counts"]
        meta = P.routing_to_kernel_metadata(routed, ps)
        _, prec_n, _ = P.metadata_to_kernel_tensors(meta, num_pages, native_precisions=True)
        _, prec_o, _ = P.build_page_tables_oracle([P.routed_spans(routed, True)], 1, 40, ps, num_pages)
        assert prec_o.tolist() == prec_n.tolist()


def test_page_table_oracle_detects_plausible_mistakes(g2):
    """The golden check above fails for a builder that forgets the
    first-seen dedupe or pages the end token of each span."""
    no_dedupe = off_by_one = 0
    for rec in g2:
        routed = _g2_routed(rec)
        ps = rec["page_size"]
        num_pages = (rec["total_tokens"] + ps - 1) // ps + 1
        spans = P.routed_spans(routed)
        want = rec["kernel"]["page_table"]
        pt, _, _ = P.build_page_tables_oracle([spans], 6, 40, ps, num_pages, dedupe=False)
        no_dedupe += pt.reshape(2, 3, 40).tolist() != want
        pt, _, _ = P.build_page_tables_oracle([[(s, e + 1, t) for s, e, t in spans]], 6, 40, ps, num_pages)
        off_by_one += pt.reshape(2, 3, 40).tolist() != want
    assert no_dedupe > 10 and off_by_one > 10


def _random_routing(rng, n_blocks=25, max_len=300):
    pols = ["ALWAYS", "ATTEND", "ATTEND", "SKIP", "RECENT", "GLOBAL"]
    blocks, t = [], 0
    for i in range(int(rng.integers(1, n_blocks))):
        ln = int(rng.integers(1, max_len))
        pol = pols[int(rng.integers(0, len(pols)))]
        sc = float(np.round(rng.random(), 1)) if (pol == "ATTEND" or rng.random() < .4) else None
        blocks.append(P.SemanticBlock(f"b{i}", t, t + ln, pol, sc))
        t += ln + int(rng.integers(0, 40))
    cfg = P.RouterConfig(top_k_blocks=int(rng.integers(0, 12)), score_threshold=float(rng.random()),
                         memory_pressure=float(np.round(rng.random(), 2)))
    return P.BlockRouter(cfg).route_layout(P.BlockLayout(blocks), t), t


def test_page_table_oracle_matches_reference_composition_on_random_layouts():
    """metadata_to_kernel_tensors(routing_to_kernel_metadata(...)) on random
    layouts, page sizes and widths (truncation included)."""
    rng = np.random.default_rng(7)
    for trial in range(80):
        routed, total = _random_routing(rng)
        ps = int(rng.choice([1, 3, 16, 64]))
        W = int(rng.integers(1, 80))
        num_pages = (total + ps - 1) // ps + int(rng.integers(0, 3))
        meta = P.routing_to_kernel_metadata(routed, ps)
        native = bool(trial % 2)
        pt_r, prec_r, pc_r = P.metadata_to_kernel_tensors(meta, num_pages, B=2, H=2, max_selected=W,
                                                          native_precisions=native)
        pt, prec, pc = P.build_page_tables_oracle([P.routed_spans(routed, native)], 4, W, ps, num_pages)
        assert pt.reshape(2, 2, W).tolist() == pt_r.tolist()
        assert prec.tolist() == prec_r.tolist()
        assert pc.reshape(2, 2).tolist() == pc_r.tolist()


def test_page_table_oracle_block_table_invariants():
    """Identity block table == no block table; a permutation maps every id;
    non-resident entries drop out and the rest keep their order."""
    rng = np.random.default_rng(8)
    for trial in range(30):
        lists, totals = [], []
        for b in range(3):
            routed, total = _random_routing(rng)
            lists.append(P.routed_spans(routed, True))
            totals.append(total)
        ps = 16
        L = max((t + ps - 1) // ps for t in totals)
        W = int(rng.integers(4, 60))
        R, H = 6, 2
        base = P.build_page_tables_oracle(lists, R, W, ps, L, rows_per_seq=H, rows_per_list=H)
        ident = np.tile(np.arange(L, dtype=np.int32), (3, 1))
        got = P.build_page_tables_oracle(lists, R, W, ps, L, rows_per_seq=H, rows_per_list=H, block_table=ident)
        for x, y in zip(base, got):
            assert np.array_equal(x, y)
        # per-sequence permutations into a pool of 3 * L pages
        perm = np.stack([rng.permutation(L).astype(np.int32) + s * L for s in range(3)])
        pt, prec, pc = P.build_page_tables_oracle(lists, R, W, ps, 3 * L, rows_per_seq=H, rows_per_list=H,
                                                  block_table=perm)
        assert np.array_equal(pc, base[2])
        for r in range(R):
            n = pc[r]
            assert np.array_equal(pt[r, :n], perm[r // H][base[0][r, :n]])
        # holes: entries set to -1 vanish, order kept, precision of dropped pages untouched
        holes = ident.copy()
        holes[rng.random(holes.shape) < 0.3] = -1
        pt_h, _, pc_h = P.build_page_tables_oracle(lists, R, 4096, ps, L, rows_per_seq=H, rows_per_list=H,
                                                   block_table=holes)
        full, _, pcf = P.build_page_tables_oracle(lists, R, 4096, ps, L, rows_per_seq=H, rows_per_list=H)
        for r in range(R):
            keep = [p for p in full[r, :pcf[r]] if holes[r // H][p] >= 0]
            assert pt_h[r, :pc_h[r]].tolist() == keep
