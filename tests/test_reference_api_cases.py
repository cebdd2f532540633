"""The reference's own unit-test cases for this path's Python API, restated
against this package (CPU unless marked gpu): tests/test_triton_intent_quant_attention.py,
test_intent_quant.py, test_block_router.py, test_block_metadata.py, test_mla.py,
the metadata conversion cases of test_fused_selected_quant_decode.py and the
BlockPrefetcher cases of test_prefetch.py. Each case asserts what the
reference's test asserts, so a caller of the reference finds the same behaviour
(names, defaults, return shapes and dtypes, error types and messages). Where
this package deliberately differs the case says so: kernel entry points refuse
host tensors (RuntimeError) instead of running a CPU loop, and their device
results are checked on the GPU. test_triton_kernel.py and the prefetch tests
built on semantic_block_attention_triton cover triton_kernel.py, which is out
of this path's scope."""
import math
import sys

import pytest
import torch

from intent_attention.block_metadata import SELECTED_POLICIES, BlockLayout, BlockPolicy as BP, SemanticBlock as S
from intent_attention.block_router import (BlockDecision, BlockRouter, RoutedBlock, RouterConfig, compute_block_scores,
                                           routing_to_kernel_metadata)
from intent_attention.fused_selected_quant_decode import FusedDecodeConfig, FusedKVPrecision, metadata_to_kernel_tensors
from intent_attention.intent_quant import (_BYTES_PER_VALUE, IntentQuantizer, KVPrecision, QuantPolicy,
                                           compute_quant_error, fake_quantize_tensor)
from intent_attention.mla import MLABlockTable, MLAConfig, absorb_weights, mla_sparse_decode_reference
from intent_attention.prefetch import BlockPrefetcher
from intent_attention.triton_intent_quant_attention import (IntentQuantKernelConfig, TritonKVPrecision,
                                                            fake_int8_pages_from_fp16,
                                                            intent_quant_decode_attention_triton,
                                                            is_cuda_available, is_triton_available,
                                                            make_page_tables_from_selected_pages,
                                                            make_precision_tensor)


def _say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


# --------------------------------------------------------------------------- #
# triton_intent_quant_attention.py: helpers, enums, configs, errors
# --------------------------------------------------------------------------- #

def test_sibling_api_probes_enums_and_config():
    assert isinstance(is_triton_available(), bool) and isinstance(is_cuda_available(), bool)
    assert [int(TritonKVPrecision[n]) for n in ("FP16", "FP8", "INT8", "INT4", "INT4_RESIDUAL", "SKIP")] == \
        [0, 1, 2, 3, 4, 5]
    cfg = IntentQuantKernelConfig()
    assert (cfg.page_size, cfg.head_dim, cfg.max_selected_pages, cfg.block_d) == (16, 64, 64, 64)


def test_page_tables_from_selected_pages():
    ids, counts = make_page_tables_from_selected_pages(torch.tensor([0, 2, 5], dtype=torch.int32), batch=2, heads=3,
                                                       max_selected_pages=8)
    assert ids.shape == (2, 3, 8) and counts.shape == (2, 3) and bool((counts == 3).all())
    assert ids[:, :, :3].eq(torch.tensor([0, 2, 5], dtype=torch.int32)).all() and ids[:, :, 3:].eq(-1).all()
    per_row = torch.arange(12, dtype=torch.int32).reshape(2, 3, 2)
    ids, counts = make_page_tables_from_selected_pages(per_row, batch=2, heads=3, max_selected_pages=4)
    assert ids.shape == (2, 3, 4) and bool((counts == 2).all())
    assert torch.equal(ids[:, :, :2], per_row) and ids[:, :, 2:].eq(-1).all()
    bad = [((torch.arange(10, dtype=torch.int32),), dict(batch=1, heads=1, max_selected_pages=5),
            "exceeds max_selected_pages"),
           ((torch.arange(24, dtype=torch.int32).reshape(2, 3, 2, 2),), dict(batch=2, heads=3), "must have shape"),
           ((torch.arange(6, dtype=torch.int32).reshape(1, 3, 2),), dict(batch=2, heads=3),
            "must match batch and heads")]
    for args, kw, msg in bad:
        with pytest.raises(ValueError, match=msg):
            make_page_tables_from_selected_pages(*args, **kw)


def test_precision_tensor_and_fake_int8_pages():
    prec = make_precision_tensor(10)
    assert prec.shape == (10,) and prec.dtype == torch.int32 and prec.eq(int(TritonKVPrecision.INT8)).all()
    prec = make_precision_tensor(10, fp16_pages=torch.tensor([0, 1, 2]), int8_pages=torch.tensor([3, 4]))
    assert prec[:3].eq(int(TritonKVPrecision.FP16)).all() and prec[3:].eq(int(TritonKVPrecision.INT8)).all()
    codes, scales = fake_int8_pages_from_fp16(torch.randn(4, 16, 32))
    assert codes.shape == (4, 16, 32) and codes.dtype == torch.int8
    assert scales.shape == (4,) and scales.dtype == torch.float32


def test_fused_metadata_to_kernel_tensors():
    """test_fused_selected_quant_decode.py:258-291: ids [0, 3, 5] with FP16 /
    INT8 / SKIP give a [1, 1, 64] table, [8] tags and one count of 3; an empty
    selection gives zeros and FP16 everywhere."""
    meta = {"selected_page_ids": [0, 3, 5], "block_precision_by_page": {"0": "FP16", "3": "INT8", "5": "SKIP"}}
    pt, prec, pc = metadata_to_kernel_tensors(meta, num_pages=8)
    assert pt.shape == (1, 1, 64) and prec.shape == (8,) and pc.shape == (1, 1)
    assert all(t.dtype == torch.int32 for t in (pt, prec, pc))
    assert (prec[0], prec[3], prec[5]) == (FusedKVPrecision.FP16, FusedKVPrecision.INT8, FusedKVPrecision.SKIP)
    assert pc[0, 0].item() == 3 and pt[0, 0, :3].tolist() == [0, 3, 5] and pt[0, 0, 3:].eq(0).all()
    pt, prec, pc = metadata_to_kernel_tensors({"selected_page_ids": [], "block_precision_by_page": {}}, num_pages=4)
    assert pt.sum().item() == 0 and pc.sum().item() == 0 and bool((prec == FusedKVPrecision.FP16).all())
    assert FusedDecodeConfig().max_selected_pages == pt.shape[-1]


def test_sibling_decode_refuses_host_tensors():
    """The reference raises "Triton is not installed|CUDA is not available"
    without a GPU; this package raises the latter for host tensors."""
    B, H, D = 2, 4, 64
    args = (torch.randn(B, H, D), torch.randn(20, 16, D), torch.randn(20, 16, D),
            torch.randint(-127, 127, (20, 16, D), dtype=torch.int8),
            torch.randint(-127, 127, (20, 16, D), dtype=torch.int8), torch.randn(20), torch.randn(20),
            torch.randint(0, 10, (B, H, 8), dtype=torch.int32), torch.full((B, H), 3, dtype=torch.int32),
            torch.zeros(20, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="Triton is not installed|CUDA is not available"):
        intent_quant_decode_attention_triton(*args)


@pytest.mark.gpu
def test_sibling_decode_smoke_on_device():
    """The reference's GPU smoke case (one head, four FP16 pages): shape, dtype
    and finite values, plus the value against float64 attention over the
    four pages."""
    _say("sibling decode smoke")
    dev = torch.device("cuda:0")
    B, H, D, NP, PS = 1, 1, 64, 4, 16
    g = torch.Generator().manual_seed(4)
    q = torch.randn(B, H, D, generator=g).half().to(dev)
    k16, v16 = (torch.randn(NP, PS, D, generator=g).half().to(dev) for _ in range(2))
    k8, v8 = (torch.randint(-127, 127, (NP, PS, D), generator=g, dtype=torch.int8).to(dev) for _ in range(2))
    ks, vs = (torch.rand(NP, generator=g).to(dev) for _ in range(2))
    sel = torch.arange(NP, device=dev)
    ids, counts = make_page_tables_from_selected_pages(sel, B, H, max_selected_pages=NP)
    prec = make_precision_tensor(NP, fp16_pages=sel, device=dev)
    cfg = IntentQuantKernelConfig(page_size=PS, head_dim=D, max_selected_pages=NP, block_d=64)
    out = intent_quant_decode_attention_triton(q, k16, v16, k8, v8, ks, vs, ids, counts, prec, config=cfg)
    torch.cuda.synchronize()
    assert out.shape == (B, H, D) and out.dtype == q.dtype and torch.isfinite(out).all()
    kk, vv, qq = k16.double().reshape(-1, D).cpu(), v16.double().reshape(-1, D).cpu(), q.double().reshape(D).cpu()
    want = torch.softmax(kk @ qq / math.sqrt(D), 0) @ vv
    assert float((out.double().reshape(D).cpu() - want).abs().max()) <= 2e-3


# --------------------------------------------------------------------------- #
# intent_quant.py: the precision policy, byte estimates, fake quantisation
# --------------------------------------------------------------------------- #

def _assign(pressure, policy, score=None):
    return IntentQuantizer(memory_pressure=pressure).assign_block_precision(S("b", 0, 128, policy, score)).precision


def test_policy_cases():
    P = KVPrecision
    for policy in (BP.ALWAYS, BP.GLOBAL):
        assert _assign(0.0, policy) == P.FP16
        assert _assign(0.95, policy) in (P.FP16, P.FP8, P.INT8)
    assert _assign(0.0, BP.SKIP) == P.SKIP
    assert _assign(0.0, BP.ATTEND, 0.1) in (P.INT4, P.INT4_RESIDUAL, P.SKIP)
    assert _assign(0.0, BP.ATTEND, 0.9) in (P.FP16, P.FP8, P.INT8)
    lo, hi = IntentQuantizer(memory_pressure=0.0), IntentQuantizer(memory_pressure=0.9)
    for blk in (S("doc", 0, 128, BP.ATTEND, 0.8), S("rec", 128, 256, BP.RECENT)):
        assert hi.assign_block_precision(blk).estimated_bytes_per_value <= \
            lo.assign_block_precision(blk).estimated_bytes_per_value
    for bad in (-0.1, 1.5):
        with pytest.raises(ValueError):
            IntentQuantizer(memory_pressure=bad)


def test_layout_estimates_and_tables():
    q5 = IntentQuantizer(memory_pressure=0.5)
    lay = BlockLayout([S("sys", 0, 128, BP.ALWAYS), S("doc1", 128, 640, BP.ATTEND, 0.9),
                       S("doc2", 640, 1152, BP.ATTEND, 0.3), S("recent", 1152, 1280, BP.RECENT),
                       S("skip", 1280, 1408, BP.SKIP)])
    est = q5.estimate_layout_bytes(lay, heads=32, head_dim=128)
    assert est["bytes_saved"] > 0 and est["bytes_saved_pct"] > 0.0 and est["total_tokens"] == 1408
    lay = BlockLayout([S("sys", 0, 64, BP.ALWAYS), S("doc", 64, 192, BP.ATTEND, 0.9),
                       S("ldoc", 192, 320, BP.ATTEND, 0.2), S("recent", 320, 384, BP.RECENT),
                       S("skip", 384, 448, BP.SKIP)])
    dist = q5.estimate_layout_bytes(lay, heads=1, head_dim=64)["precision_distribution"]
    assert isinstance(dist, dict) and sum(dist.values()) == 448
    rows = IntentQuantizer(memory_pressure=0.3).summary_table(
        BlockLayout([S("sys", 0, 64, BP.ALWAYS), S("doc", 64, 192, BP.ATTEND, 0.8), S("skip", 192, 256, BP.SKIP)]),
        heads=8, head_dim=64)
    assert [r["block"] for r in rows] == ["sys", "doc", "skip"]
    assert all({"precision", "dense_fp16_bytes", "quant_bytes"} <= set(r) for r in rows)
    pol = IntentQuantizer().assign_layout_precision(
        BlockLayout([S("a", 0, 64, BP.ALWAYS), S("b", 64, 128, BP.RECENT), S("c", 128, 192, BP.SKIP)]))
    assert set(pol) == {"a", "b", "c"}


def test_quant_policy_fields():
    p = QuantPolicy(KVPrecision.INT4_RESIDUAL, "test")
    assert (p.estimated_bytes_per_value, p.requires_scale, p.uses_residual) == (1.0, True, True)
    p = QuantPolicy(KVPrecision.SKIP)
    assert (p.estimated_bytes_per_value, p.requires_scale, p.uses_residual) == (0.0, False, False)


def test_fake_quantize_shapes_metadata_and_errors():
    x = torch.randn(2, 4, 128, 64)
    for prec in (KVPrecision.FP16, KVPrecision.FP8, KVPrecision.INT8, KVPrecision.INT4):
        recon, meta = fake_quantize_tensor(x, prec)
        assert recon.shape == x.shape and isinstance(meta, dict)
    x = torch.randn(1, 2, 16, 32)
    for prec in (KVPrecision.FP8, KVPrecision.INT8, KVPrecision.INT4, KVPrecision.INT4_RESIDUAL):
        _, meta = fake_quantize_tensor(x, prec)
        assert all(isinstance(meta[k], float) for k in ("mse", "max_abs_error", "cosine_similarity"))
    recon, meta = fake_quantize_tensor(torch.randn(1, 2, 8, 32), KVPrecision.FP16)
    assert recon.shape == (1, 2, 8, 32) and meta["precision"] == "fp16"
    recon, _ = fake_quantize_tensor(torch.randn(1, 2, 8, 32), KVPrecision.SKIP)
    assert bool((recon == 0.0).all())
    orig = torch.randn(2, 4, 16, 64)
    err = compute_quant_error(orig, orig + torch.randn_like(orig) * 0.01)
    assert {"mse", "max_abs_error", "cosine_similarity"} <= set(err)


# --------------------------------------------------------------------------- #
# block_router.py
# --------------------------------------------------------------------------- #

def _router(**kw):
    return BlockRouter(RouterConfig(**kw))


def _five_blocks():
    return BlockLayout([S("system", 0, 64, BP.ALWAYS), S("doc_high", 64, 192, BP.ATTEND, 0.9),
                        S("doc_low", 192, 320, BP.ATTEND, 0.1), S("recent", 320, 384, BP.RECENT),
                        S("unused", 384, 448, BP.SKIP)])


def test_router_decisions():
    one = lambda policy, **kw: _router(**kw).route_layout(BlockLayout([S("x", 0, 64, policy)]), total_tokens=64)[0]  # noqa: E731
    assert one(BP.ALWAYS).decision == BlockDecision.PIN_HIGH_PRECISION
    assert one(BP.GLOBAL).decision == BlockDecision.PIN_HIGH_PRECISION
    assert one(BP.RECENT).decision == BlockDecision.SELECT
    r = _router(score_threshold=0.5).route_layout(BlockLayout([S("important", 0, 64, BP.ATTEND, 0.9)]), 64)
    assert r[0].decision in (BlockDecision.SELECT, BlockDecision.QUANTIZE)
    r = _router(score_threshold=0.5).route_layout(BlockLayout([S("marked_skip", 0, 32, BP.SKIP, 0.8)]), 32)
    assert r[0].decision == BlockDecision.SELECT
    rt = _router(score_threshold=0.5, top_k_blocks=1)
    r = rt.route_layout(BlockLayout([S("good", 0, 32, BP.ATTEND, 0.9), S("bad", 32, 64, BP.ATTEND, 0.1)]), 64)
    d = {b.name: b.decision for b in r}
    assert d["good"] != BlockDecision.SKIP and d["bad"] == BlockDecision.SKIP
    assert [b.name for b in rt.skipped_blocks(r)] == ["bad"]
    rt = _router(top_k_blocks=2)
    r = rt.route_layout(BlockLayout([S(n, 16 * i, 16 * i + 16, BP.ATTEND, 0.9 - 0.1 * i)
                                     for i, n in enumerate("abcd")]), 64)
    assert len(rt.selected_blocks(r)) <= 2


def test_router_pages_tokens_and_precisions():
    rt = _router()
    for lay, total in ((BlockLayout([S("a", 0, 48, BP.ALWAYS), S("b", 48, 96, BP.ATTEND, 0.9)]), 96),
                       (BlockLayout([S("a", 0, 32, BP.ALWAYS), S("b", 32, 64, BP.ATTEND, 0.9)]), 64)):
        pids = rt.selected_page_ids(rt.route_layout(lay, total), page_size=16)
        assert pids == sorted(pids) and len(pids) == len(set(pids))
    idx = rt.selected_token_indices(rt.route_layout(BlockLayout([S("a", 0, 16, BP.ALWAYS),
                                                                 S("b", 32, 48, BP.ATTEND, 0.9)]), 48))
    assert idx == sorted(idx) and 16 not in idx
    lay = BlockLayout([S("always", 0, 32, BP.ALWAYS), S("doc", 32, 64, BP.ATTEND, 0.5)])
    bpe = {p: {b.name: _BYTES_PER_VALUE.get(b.precision, 2.0)
               for b in _router(memory_pressure=p).route_layout(lay, 64)} for p in (0.1, 0.9)}
    assert bpe[0.9]["doc"] <= bpe[0.1]["doc"]
    rt = _router(prefetch_top_k=2)
    pf = rt.prefetch_page_ids(rt.route_layout(BlockLayout([S("a", 0, 32, BP.ALWAYS), S("b", 32, 64, BP.ATTEND, 0.2)]),
                                              64), page_size=16)
    assert isinstance(pf, list) and len(pf) <= 2


def test_router_metadata_summary_and_scores():
    rt = _router()
    routed = rt.route_layout(_five_blocks(), total_tokens=448)
    assert len(routed) == 5 and all(isinstance(b, RoutedBlock) for b in routed)
    meta = routing_to_kernel_metadata(routed, page_size=16)
    assert {"selected_page_ids", "prefetch_page_ids", "block_precision_by_page", "selected_block_names",
            "skipped_block_names", "reasons_by_block"} <= set(meta)
    assert meta["selected_page_ids"] and len(meta["selected_block_names"]) >= 3
    s = rt.routing_summary(routed)
    assert s["selected_tokens"] > 0 and s["skipped_tokens"] >= 0 and s["total_blocks"] == 5
    assert s["precision_distribution"] and s["bytes_saved_pct"] >= 0.0
    scores = compute_block_scores(torch.randn(64), {"a": torch.randn(64), "b": torch.randn(64)})
    assert set(scores) == {"a", "b"} and all(0.0 <= v <= 1.0 for v in scores.values())


# --------------------------------------------------------------------------- #
# block_metadata.py
# --------------------------------------------------------------------------- #

def test_layout_validation_and_selection():
    lay = BlockLayout([S("a", 0, 10, BP.ALWAYS)])
    lay.validate(10)
    assert lay.selected_token_count() == 10
    BlockLayout([]).validate(100)
    bad = [([S("", 0, 10, BP.ALWAYS)], 10, "empty name"), ([S("a", -1, 10, BP.ALWAYS)], 10, "start.*< 0"),
           ([S("a", 5, 5, BP.ALWAYS)], 10, "end.*<= start"), ([S("a", 10, 5, BP.ALWAYS)], 10, "end.*<= start"),
           ([S("a", 0, 11, BP.ALWAYS)], 10, "end.*> total_tokens"),
           ([S("b", 10, 20, BP.SKIP), S("a", 0, 10, BP.ALWAYS)], 20, "not sorted"),
           ([S("a", 0, 10, BP.ALWAYS), S("b", 5, 15, BP.SKIP)], 15, "overlap"),
           ([S("a", 0, 10, BP.ATTEND, None)], 10, "score is None")]
    for blocks, total, msg in bad:
        with pytest.raises(ValueError, match=msg):
            BlockLayout(blocks).validate(total)
    lay = BlockLayout([S("a", 0, 10, BP.ALWAYS), S("b", 10, 20, BP.SKIP), S("c", 20, 30, BP.ATTEND, 0.8)])
    assert [b.name for b in lay.selected_blocks()] == ["a", "c"]
    assert set(SELECTED_POLICIES) == set(BP) - {BP.SKIP}


# --------------------------------------------------------------------------- #
# mla.py
# --------------------------------------------------------------------------- #

def test_mla_config_table_and_weights():
    cfg = MLAConfig(d_model=4096, d_c=512, n_heads=32, d_head=128)
    assert (cfg.d_model, cfg.d_c) == (4096, 512)
    table = MLABlockTable(cfg)
    assert table.get_latent(99) is None
    table.append(0, torch.randn(64, 512))
    assert table.get_latent(0).shape == (64, 512) and table.memory_bytes() == 64 * 512 * 2
    table = MLABlockTable(MLAConfig(d_model=4096, d_c=512, n_heads=32, d_head=128, d_rope=64))
    table.append(0, torch.randn(64, 512), rope_page=torch.randn(64, 64))
    assert table.get_rope(0).shape == (64, 64)
    w_qk, w_vo = absorb_weights(torch.randn(4096, 512), torch.randn(4096, 512), torch.randn(4096, 512),
                                torch.randn(512, 4096))
    assert w_qk.shape == (4096, 512) and w_vo.shape == (4096, 4096)


def test_mla_sparse_decode_refuses_host_tensors():
    """The reference runs mla_sparse_decode_reference on the CPU; here it runs
    on the kernels and host tensors raise (its device result is checked in
    test_mla_sparse_decode_returns_tuple_on_device)."""
    cfg = MLAConfig(d_model=4096, d_c=512, n_heads=32, d_head=128)
    table = MLABlockTable(cfg)
    table.append(0, torch.randn(64, 512))
    lay = BlockLayout([S("b0", 0, 64, BP.ATTEND, 0.9)])
    with pytest.raises(RuntimeError):
        mla_sparse_decode_reference(torch.randn(2, 32, 8, 128), table, torch.randn(4096, 512), torch.randn(512, 4096),
                                    lay, threshold=0.5, return_debug=True)


@pytest.mark.gpu
def test_mla_sparse_decode_returns_tuple_on_device():
    _say("mla_sparse_decode_reference tuple")
    dev = torch.device("cuda:0")
    cfg = MLAConfig(d_model=4096, d_c=512, n_heads=32, d_head=128)
    table = MLABlockTable(cfg)
    table.append(0, torch.randn(64, 512).to(dev))
    lay = BlockLayout([S("b0", 0, 64, BP.ATTEND, 0.9)])
    out, dbg = mla_sparse_decode_reference(torch.randn(2, 32, 8, 128, device=dev), table,
                                           torch.randn(4096, 512, device=dev), torch.randn(512, 4096, device=dev),
                                           lay, threshold=0.5, return_debug=True)
    torch.cuda.synchronize()
    assert out.shape == (2, 8, 4096) and dbg is not None and "selected_latent_tokens" in dbg


# --------------------------------------------------------------------------- #
# prefetch.py: BlockPrefetcher
# --------------------------------------------------------------------------- #

def test_block_prefetcher_cases():
    def pf(*steps):
        p = BlockPrefetcher(history_size=4, min_frequency=3)
        for s in steps:
            p.record(list(s))
        return p
    assert pf().predict_next([1, 2, 3]) == []
    assert pf([1]).predict_next([1]) == []
    assert pf([10, 20], [10, 20], [10, 20]).predict_next([10, 20]) == [10, 20]
    assert pf([1, 2], [1, 3], [1, 4]).predict_next([1, 5]) == [1]
    assert pf([3, 1, 2], [3, 1, 2], [3, 1, 2]).predict_next([3, 1, 2]) == [1, 2, 3]
    assert pf([99], [99], [99]).predict_next([99]) == [99]
    p = pf([1], [1], [1])
    p.reset()
    assert p.predict_next([1]) == []

