"""intent_quant_attention_reference, compare_intent_quant_to_fp16_selected,
semantic_block_attention and dense_attention of the product
(intent_attention.intent_quant_attention / intent_attention.reference), with
the attention on the HIP dense attention kernel.

GPU: the reference's own outputs (golden g4: the cfg1 shape with its
alternating FP16 / INT8 plan, and a plan with every precision including a
SKIP-precision block, plus the default policy) within the quantised-page bar
1e-2; the debug dictionary's keys and values; dense_attention against a
float64 softmax over shapes, dtypes, causal masks and ragged lengths, against
the float64 oracle with additive float / bool / -inf masks, original KV
positions (sorted and not), broadcast leading dims and all-masked rows; the
reference's test_causal_attention.py cases and its compare-function test on
device tensors; the reference's error behaviour. CPU: the errors raised
before any device work (causal, host tensors).
"""
import math
import os
import sys

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import policy as P


def _say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def g4(golden_dir):
    return dict(np.load(os.path.join(golden_dir, "g4_intent_quant_attention.npz")))


class _Plan:
    """Duck-typed quantizer with a fixed precision per block (product types)."""

    def __init__(self, plan):
        self.plan = plan

    def assign_block_precision(self, block):
        from intent_attention import KVPrecision, QuantPolicy
        return QuantPolicy(KVPrecision(self.plan[block.name]))


def _cfg1_inputs(g4):
    from intent_attention import BlockLayout, BlockPolicy, SemanticBlock
    pages = [int(p) for p in g4["cfg1_pages"]]
    k = np.zeros((1, 8, 1024, 64), np.float32)
    v = np.zeros((1, 8, 1024, 64), np.float32)
    tok = np.array([p * 16 + t for p in pages for t in range(16)])
    k[:, :, tok] = g4["cfg1_k_sel"].astype(np.float32)
    v[:, :, tok] = g4["cfg1_v_sel"].astype(np.float32)
    blocks, plan = [], {}
    for rank, p in enumerate(pages):
        pol = BlockPolicy.ALWAYS if p < 4 else (BlockPolicy.RECENT if p >= 56 else BlockPolicy.ATTEND)
        blocks.append(SemanticBlock(f"p{p}", p * 16, p * 16 + 16, pol, 0.9 if pol == BlockPolicy.ATTEND else None))
        plan[f"p{p}"] = "FP16" if rank % 2 == 0 else "INT8"
    return g4["cfg1_q"].astype(np.float32), k, v, BlockLayout(blocks), plan


def _mix_layout():
    from intent_attention import BlockLayout, BlockPolicy as BP, SemanticBlock as S
    return BlockLayout([S("a", 0, 16, BP.ALWAYS), S("b", 16, 40, BP.ATTEND, 0.5), S("c", 40, 56, BP.ATTEND, 0.1),
                        S("d", 56, 80, BP.RECENT), S("e", 80, 96, BP.SKIP)])


def test_errors_before_device_work():
    from intent_attention import dense_attention, intent_quant_attention_reference, IntentQuantizer
    q = torch.zeros(1, 2, 1, 64)
    lay = _mix_layout()
    with pytest.raises(NotImplementedError, match="query_positions"):
        intent_quant_attention_reference(q, q, q, lay, IntentQuantizer(), causal=True)
    with pytest.raises(RuntimeError, match="HIP kernels only"):
        intent_quant_attention_reference(q, torch.zeros(1, 2, 96, 64), torch.zeros(1, 2, 96, 64), lay,
                                         IntentQuantizer())
    with pytest.raises(RuntimeError, match="HIP kernels only"):
        dense_attention(q, q, q)
    with pytest.raises(RuntimeError, match="HIP kernels only"):
        dense_attention(q, q, q, mask=torch.zeros(1, 1))


@pytest.mark.gpu
def test_cfg1_golden(g4):
    from intent_attention import intent_quant_attention_reference
    _say("intent_quant_attention_reference cfg1 vs golden")
    dev = torch.device("cuda:0")
    q, k, v, layout, plan = _cfg1_inputs(g4)
    t = lambda x: torch.from_numpy(x).to(dev)  # noqa: E731
    out = intent_quant_attention_reference(t(q), t(k), t(v), layout, _Plan(plan))
    torch.cuda.synchronize()
    assert out.shape == q.shape and out.dtype == torch.float32
    ref = g4["cfg1_out"]
    err = float(np.abs(out.cpu().numpy() - ref).max())
    rel = err / float(np.abs(ref).max())
    _say(f"  cfg1 max abs err {err:.2e} (relative {rel:.2e})")
    assert err <= 1e-2


@pytest.mark.gpu
def test_mixed_plan_and_default_policy_golden(g4):
    from intent_attention import IntentQuantizer, intent_quant_attention_reference
    _say("intent_quant_attention_reference mixed plan vs golden")
    dev = torch.device("cuda:0")
    q, k, v = (torch.from_numpy(g4[n]).to(dev) for n in ("mix_q", "mix_k", "mix_v"))
    lay = _mix_layout()
    plan = {"a": "FP8", "b": "INT4_RESIDUAL", "c": "SKIP", "d": "INT4"}
    out = intent_quant_attention_reference(q, k, v, lay, _Plan(plan))
    out2 = intent_quant_attention_reference(q, k, v, lay, IntentQuantizer(memory_pressure=0.5))
    torch.cuda.synchronize()
    e1 = float(np.abs(out.cpu().numpy() - g4["mix_out"]).max())
    e2 = float(np.abs(out2.cpu().numpy() - g4["mix_out_default"]).max())
    _say(f"  mixed plan max abs err {e1:.2e}, default policy {e2:.2e}")
    assert e1 <= 1e-2 and e2 <= 1e-2


@pytest.mark.gpu
def test_debug_dictionary(g4):
    from intent_attention import intent_quant_attention_reference
    from intent_attention.intent_quant_attention import _empty_debug
    _say("intent_quant_attention_reference return_debug")
    dev = torch.device("cuda:0")
    q, k, v = (torch.from_numpy(g4[n]).to(dev) for n in ("mix_q", "mix_k", "mix_v"))
    lay = _mix_layout()
    plan = {"a": "FP8", "b": "INT4_RESIDUAL", "c": "SKIP", "d": "INT4"}
    out, dbg = intent_quant_attention_reference(q, k, v, lay, _Plan(plan), return_debug=True)
    assert set(dbg) == set(_empty_debug(lay, 96))
    assert dbg["selected_block_names"] == ["a", "b", "c", "d"]
    assert dbg["selected_tokens"] == 80
    assert dbg["precision_by_block"] == plan
    assert dbg["estimated_fp16_bytes"] == 2 * 80 * 32 * 2
    assert dbg["estimated_quant_bytes"] == int(round(2 * 32 * (16 * 1.0 + 24 * 1.0 + 16 * 0.0 + 24 * 0.5)))
    assert set(dbg["reconstruction_mse_k"]) == {"a", "b", "d"}
    # the unquantised-selection output the debug compares against: float64 dense attention
    sel = np.concatenate([np.arange(0, 80)])
    dense = A.dense_attention(g4["mix_q"], g4["mix_k"][:, :, sel], g4["mix_v"][:, :, sel])
    o = out.cpu().numpy().astype(np.float64)
    mse = float(((dense - o) ** 2).mean())
    assert abs(dbg["output_mse_vs_fp16_selected"] - mse) <= 0.05 * mse + 1e-6
    assert 0.0 < dbg["output_cosine_vs_fp16_selected"] <= 1.0 + 1e-6
    empty = P.BlockLayout([])
    from intent_attention import BlockLayout
    z, dz = intent_quant_attention_reference(q, k, v, BlockLayout([]), _Plan({}), return_debug=True)
    assert torch.count_nonzero(z) == 0 and dz == _empty_debug(empty, 96)


DENSE = [
    # lead, Tq, Tk, D, dtype, causal
    ((1, 8), 1, 1024, 64, "float32", False),
    ((2, 4), 8, 300, 64, "float16", False),
    ((3,), 16, 77, 128, "bfloat16", False),
    ((2, 2), 40, 129, 100, "float32", False),
    ((1, 3), 24, 24, 64, "float16", True),
    ((2,), 5, 50, 32, "float32", True),
    ((1, 1), 3, 0, 64, "float32", False),
    ((2,), 4, 200, 576, "float16", True),        # DeepSeek's latent + RoPE width
    ((1,), 3, 70, 1024, "bfloat16", False),      # the widest head the kernel takes
    ((3,), 2, 33, 1, "float32", False),
    # grids of many rows take fewer waves per row (16 up to 256 rows, 8 up to 512, then 4);
    # few rows with 512 keys or more split each row's keys over workgroups
    ((2, 3), 2, 3000, 128, "bfloat16", True),     # 12 rows x 11 key ranges, most of them fully masked
    ((1, 2), 3, 5000, 1024, "float16", False),    # 6 rows of the widest head over 19 ranges
    ((4, 8), 64, 96, 64, "float16", True),        # 2,048 rows: 4 waves per row
    ((2, 4), 48, 130, 128, "float32", False),     # 384 rows: 8 waves per row
    ((2,), 300, 40, 1024, "float32", False),      # 600 rows of the widest head: 4 waves per row
]


@pytest.mark.gpu
@pytest.mark.parametrize("lead,Tq,Tk,D,dt,causal", DENSE)
def test_dense_attention_against_float64(lead, Tq, Tk, D, dt, causal):
    from intent_attention import dense_attention
    _say("dense_attention", f"lead={lead} Tq={Tq} Tk={Tk} D={D} dtype={dt} causal={causal}")
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(Tq * 1000 + Tk + D)
    q = torch.randn(*lead, Tq, D, generator=g).to(getattr(torch, dt))
    k = torch.randn(*lead, Tk, D, generator=g).to(getattr(torch, dt))
    v = torch.randn(*lead, Tk, D, generator=g).to(getattr(torch, dt))
    out = dense_attention(q.to(dev), k.to(dev), v.to(dev), causal=causal)
    torch.cuda.synchronize()
    assert out.shape == q.shape and out.dtype == q.dtype
    qd, kd, vd = (x.double() for x in (q, k, v))
    s = qd @ kd.transpose(-2, -1) / math.sqrt(D)
    if causal:
        s = s + torch.triu(torch.full((Tq, Tk), float("-inf"), dtype=torch.float64), diagonal=1)
    ref = (torch.softmax(s, dim=-1) @ vd) if Tk else torch.zeros_like(qd)
    err = float((out.cpu().double() - ref).abs().max())
    # float32 arithmetic (2e-5), then one rounding of the output to its dtype: half an ulp
    # of the largest output, 2^-11 relative for float16 and 2^-8 for bfloat16
    half_ulp = {"float32": 0.0, "float16": 2.0 ** -11, "bfloat16": 2.0 ** -8}[dt]
    tol = 2e-5 + half_ulp * float(ref.abs().max()) if Tk else 0.0
    _say(f"  max abs err {err:.2e}")
    assert err <= tol


@pytest.mark.gpu
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_dense_attention_split_matches_single_pass(dt, monkeypatch):
    """The split-over-keys path and the one-workgroup-per-row path (no
    workspace) agree to float32 summation order, also with a mask and causal
    key positions."""
    from intent_attention import dense_attention
    from intent_attention import _native as N
    dev = torch.device("cuda:0")
    _say("dense_attention split vs single pass", dt)
    q, k, v, g = _dense_case(8, (2, 4), 3, 4097, 96, 80, dt, dev)
    mask = torch.randn(3, 4097, generator=g).to(dt).to(dev)
    pos = torch.randperm(4097, generator=g).to(dev)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    assert N.dense_attention_workspace(_probe_args(qd, kd, vd)) > 0
    for kw in (dict(), dict(mask=mask, causal=True, original_kv_positions=pos)):
        split = dense_attention(qd, kd, vd, **kw)
        with monkeypatch.context() as mp:
            mp.setattr(N, "dense_attention_workspace", lambda a: 0)
            single = dense_attention(qd, kd, vd, **kw)
        torch.cuda.synchronize()
        err = float((split.float() - single.float()).abs().max())
        _say(f"  {sorted(kw)}: max |split - single| {err:.2e}")
        assert torch.isnan(split).sum() == torch.isnan(single).sum() == 0
        assert err <= (1e-5 if dt == torch.float32 else 8e-3)


def _probe_args(q, k, v):
    """DenseAttentionArgs of the leading-dims-flattened shapes, for the workspace query."""
    from intent_attention import _native as N
    a = N.DenseAttentionArgs()
    L = math.prod(q.shape[:-2])
    a.batch, a.q_len, a.kv_len, a.head_dim, a.v_dim, a.dtype = L, q.shape[-2], k.shape[-2], q.shape[-1], v.shape[-1], 0
    a.q, a.k, a.v, a.out = q.data_ptr(), k.data_ptr(), v.data_ptr(), q.data_ptr()
    return a


@pytest.mark.gpu
def test_dense_attention_dtype_mismatch_raises():
    from intent_attention import dense_attention
    dev = torch.device("cuda:0")
    q = torch.zeros(1, 2, 1, 64, device=dev)
    with pytest.raises(RuntimeError, match="same dtype"):
        dense_attention(q.half(), q, q)
    with pytest.raises(RuntimeError, match="same dtype"):
        # float16 scores + a float32 mask promote to float32, which the second matmul refuses
        dense_attention(q.half(), q.half(), q.half(), mask=torch.zeros(1, 1, device=dev))


_TOL = {torch.float32: 2e-5, torch.float16: 1e-3, torch.bfloat16: 8e-3}


def _dense_case(seed, lead, Tq, Tk, D, Dv, dt, dev):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(*lead, Tq, D, generator=g).to(dt)
    k = torch.randn(*lead, Tk, D, generator=g).to(dt)
    v = torch.randn(*lead, Tk, Dv, generator=g).to(dt)
    return q, k, v, g


def _cmp(out, ref, dt, what):
    o = out.cpu().double().numpy()
    nan_ok = np.array_equal(np.isnan(o), np.isnan(ref))
    err = float(np.nanmax(np.abs(o - ref))) if np.isfinite(ref).any() else 0.0
    _say(f"  {what}: max abs err {err:.2e}, NaN pattern equal {nan_ok}")
    assert nan_ok and err <= _TOL[dt]


@pytest.mark.gpu
@pytest.mark.parametrize("Tq,Tk", [(12, 70), (2, 3000)])
@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.bfloat16])
def test_dense_attention_masks_and_positions(dt, Tq, Tk):
    """Additive masks (float with -inf entries, bool, per-batch), original KV positions
    (sorted and unsorted, with and without a mask), v_dim != head_dim and broadcast
    leading dims, against the float64 oracle; 3,000 keys over 12 rows take the
    split-over-keys path (partials merged by a second kernel)."""
    from intent_attention import dense_attention
    dev = torch.device("cuda:0")
    _say("dense_attention masks / positions", dt, f"Tq={Tq} Tk={Tk}")
    q, k, v, g = _dense_case(5, (2, 3), Tq, Tk, 64, 48, dt, dev)
    t = lambda x: x.to(dev)  # noqa: E731
    fmask = torch.randn(Tq, Tk, generator=g)
    fmask[torch.rand(Tq, Tk, generator=g) < 0.3] = float("-inf")
    fmask[:, 5] = 0.0
    bmask = torch.rand(2, 1, Tq, Tk, generator=g) < 0.5
    lmask = torch.randn(2, 3, Tq, Tk, generator=g)
    pos_sorted = torch.sort(torch.randperm(max(200, 3 * Tk), generator=g)[:Tk]).values
    pos_sorted[0] = 0
    pos_perm = pos_sorted[torch.randperm(Tk, generator=g)]
    qn, kn, vn = (x.double().numpy() for x in (q, k, v))
    cases = [
        ("float mask [Tq, Tk] with -inf", dict(mask=fmask.to(dt)), dict(mask=fmask.to(dt).double().numpy())),
        ("bool mask [2, 1, Tq, Tk]", dict(mask=bmask), dict(mask=bmask.numpy())),
        ("mask per (b, h)", dict(mask=lmask.to(dt)), dict(mask=lmask.to(dt).double().numpy())),
        ("causal, sorted positions", dict(causal=True, original_kv_positions=pos_sorted),
         dict(causal=True, original_kv_positions=pos_sorted.numpy())),
        ("causal, unsorted positions", dict(causal=True, original_kv_positions=pos_perm),
         dict(causal=True, original_kv_positions=pos_perm.numpy())),
        ("causal, positions and mask", dict(causal=True, original_kv_positions=pos_perm, mask=fmask.to(dt)),
         dict(causal=True, original_kv_positions=pos_perm.numpy(), mask=fmask.to(dt).double().numpy())),
        ("positions without causal", dict(original_kv_positions=pos_perm), dict()),
    ]
    for what, kw, okw in cases:
        kw = {n: (t(x) if isinstance(x, torch.Tensor) else x) for n, x in kw.items()}
        out = dense_attention(t(q), t(k), t(v), **kw)
        torch.cuda.synchronize()
        assert out.shape == (2, 3, Tq, 48) and out.dtype == dt
        _cmp(out, A.dense_attention_masked(qn, kn, vn, **okw), dt, what)
    # k / v shared by every batch entry (leading dims broadcast as in torch.matmul)
    out = dense_attention(t(q), t(k[:1]), t(v[:1]), mask=t(fmask.to(dt)))
    _cmp(out, A.dense_attention_masked(qn, kn[:1], vn[:1], mask=fmask.to(dt).double().numpy()), dt, "broadcast k / v")
    # every key of query 0 masked: NaN, as torch's softmax gives; the other rows finite
    allm = torch.zeros(Tq, Tk)
    allm[0] = float("-inf")
    out = dense_attention(t(q), t(k), t(v), mask=t(allm.to(dt)))
    torch.cuda.synchronize()
    assert torch.isnan(out[..., 0, :]).all() and not torch.isnan(out[..., 1:, :]).any()
    _cmp(out, A.dense_attention_masked(qn, kn, vn, mask=allm.to(dt).double().numpy()), dt, "all-masked row")


@pytest.mark.gpu
def test_reference_causal_attention_cases():
    """The reference's tests/test_causal_attention.py cases on device tensors: the
    relations it asserts (semantic == dense with original positions, 1e-5) plus
    each output against the float64 oracle."""
    from intent_attention import BlockLayout, BlockPolicy, SemanticBlock, dense_attention, semantic_block_attention
    dev = torch.device("cuda:0")
    _say("reference test_causal_attention cases")
    g = torch.Generator().manual_seed(0)
    r = lambda *s: torch.randn(*s, generator=g).to(dev)  # noqa: E731
    S, BP = SemanticBlock, BlockPolicy

    def check(out, ref_np, what):
        err = float(np.abs(out.cpu().double().numpy() - ref_np).max())
        _say(f"  {what}: max abs err vs float64 {err:.2e}")
        assert not torch.isnan(out).any() and err <= 2e-5

    def npy(*xs):
        return [x.cpu().double().numpy() for x in xs]

    # identical layout: causal selected == dense causal
    q, k, v = r(2, 4, 8, 64), r(2, 4, 32, 64), r(2, 4, 32, 64)
    d = dense_attention(q, k, v, causal=True)
    sel, dbg = semantic_block_attention(q, k, v, BlockLayout([S("all", 0, 32, BP.ALWAYS)]), causal=True,
                                        return_debug=True)
    assert torch.allclose(d, sel, atol=1e-5)
    check(d, A.dense_attention_masked(*npy(q, k, v), causal=True), "identical layout")
    # prevents future attention, skip middle, non-contiguous masking: semantic == dense with positions
    for Tk, blocks, idx in (
            (12, [S("b", 0, 10, BP.ALWAYS)], list(range(10))),
            (16, [S("first", 0, 4, BP.ALWAYS), S("skip", 4, 10, BP.SKIP), S("last", 10, 16, BP.ALWAYS)],
             [0, 1, 2, 3, 10, 11, 12, 13, 14, 15]),
            (12, [S("early", 0, 3, BP.ALWAYS), S("late", 8, 12, BP.ALWAYS)], [0, 1, 2, 8, 9, 10, 11])):
        q, k, v = r(1, 1, 6, 8), r(1, 1, Tk, 8), r(1, 1, Tk, 8)
        out, _ = semantic_block_attention(q, k, v, BlockLayout(blocks), causal=True, return_debug=True)
        ix = torch.tensor(idx, device=dev)
        od = dense_attention(q, k.index_select(-2, ix), v.index_select(-2, ix), causal=True, original_kv_positions=ix)
        assert torch.allclose(out, od, atol=1e-5)
        qn, kn, vn = npy(q, k, v)
        check(out, A.dense_attention_masked(qn, kn[..., idx, :], vn[..., idx, :], causal=True,
                                            original_kv_positions=np.array(idx)), f"positions {idx}")
    # every query has visible keys
    q, k, v = r(1, 1, 4, 8), r(1, 1, 8, 8), r(1, 1, 8, 8)
    out, _ = semantic_block_attention(q, k, v, BlockLayout([S("early", 0, 3, BP.ALWAYS), S("late", 3, 8, BP.ALWAYS)]),
                                      causal=True, return_debug=True)
    assert not torch.isnan(out).any()
    # decode step: one query at position 0
    q, k, v = r(1, 1, 1, 8), r(1, 1, 16, 8), r(1, 1, 16, 8)
    out, _ = semantic_block_attention(q, k, v, BlockLayout([S("b", 0, 16, BP.ALWAYS)]), causal=True,
                                      return_debug=True)
    assert torch.allclose(out, dense_attention(q, k, v, causal=True), atol=1e-5)
    check(out, A.dense_attention_masked(*npy(q, k, v), causal=True), "decode step")
    # all blocks selected (ATTEND with a score)
    q, k, v = r(2, 4, 16, 64), r(2, 4, 64, 64), r(2, 4, 64, 64)
    lay = BlockLayout([S("a", 0, 32, BP.ALWAYS), S("b", 32, 64, BP.ATTEND, score=0.9)])
    o_sel, _ = semantic_block_attention(q, k, v, lay, causal=True, return_debug=True, threshold=0.5)
    assert torch.allclose(dense_attention(q, k, v, causal=True), o_sel, atol=1e-5)
    # debug metadata
    q, k, v = r(1, 1, 4, 8), r(1, 1, 16, 8), r(1, 1, 16, 8)
    _, dbg = semantic_block_attention(q, k, v, BlockLayout([S("test", 0, 16, BP.ALWAYS)]), causal=True,
                                      return_debug=True)
    assert dbg == {"selected_token_count": 16, "selected_block_names": ["test"], "total_kv_tokens": 16,
                   "selected_kv_tokens": 16}


@pytest.mark.gpu
def test_reference_correctness_cases():
    """The reference's tests/test_reference_correctness.py cases on device
    tensors: semantic_block_attention equals dense attention over the selected
    tokens (SKIP left out), a layout that selects nothing gives zeros and an
    empty debug record, the five policies together select ALWAYS + ATTEND +
    RECENT + GLOBAL, causal attention is finite, never looks ahead (the
    reference's triu construction, here in float64), and a single ALWAYS block
    under the causal mask equals dense causal attention."""
    from intent_attention import BlockLayout, BlockPolicy, SemanticBlock, dense_attention, semantic_block_attention
    dev = torch.device("cuda:0")
    _say("reference test_reference_correctness cases")
    g = torch.Generator().manual_seed(1)
    r = lambda *s: torch.randn(*s, generator=g).to(dev)  # noqa: E731
    S, BP = SemanticBlock, BlockPolicy

    q, k, v = r(2, 4, 16, 64), r(2, 4, 128, 64), r(2, 4, 128, 64)
    out, dbg = semantic_block_attention(q, k, v, BlockLayout([S("a", 0, 64, BP.ALWAYS), S("b", 64, 128, BP.SKIP)]),
                                        return_debug=True)
    want = dense_attention(q, k[:, :, :64], v[:, :, :64])
    assert torch.allclose(out, want) and dbg["selected_token_count"] == 64 and out.shape == (2, 4, 16, 64)

    q, k, v = r(1, 1, 8, 32), r(1, 1, 16, 32), r(1, 1, 16, 32)
    skip = BlockLayout([S("a", 0, 16, BP.SKIP)])
    assert torch.equal(semantic_block_attention(q, k, v, skip), torch.zeros_like(q))
    out, dbg = semantic_block_attention(q, k, v, skip, return_debug=True)
    assert torch.equal(out, torch.zeros_like(q))
    assert dbg["selected_token_count"] == 0 and dbg["selected_block_names"] == []

    q, k, v = r(1, 2, 8, 32), r(1, 2, 128, 32), r(1, 2, 128, 32)
    lay = BlockLayout([S("always", 0, 32, BP.ALWAYS), S("attend", 32, 64, BP.ATTEND, score=0.9),
                       S("skip", 64, 96, BP.SKIP), S("recent", 96, 112, BP.RECENT),
                       S("global", 112, 128, BP.GLOBAL)])
    out, dbg = semantic_block_attention(q, k, v, lay, return_debug=True)
    assert out.shape == (1, 2, 8, 32) and dbg["selected_token_count"] == 96 and dbg["total_kv_tokens"] == 128
    sel = torch.cat([torch.arange(0, 64), torch.arange(96, 128)]).to(dev)
    assert torch.allclose(out, dense_attention(q, k.index_select(-2, sel), v.index_select(-2, sel)))

    q, k, v = r(1, 2, 8, 32), r(1, 2, 16, 32), r(1, 2, 16, 32)
    out = dense_attention(q, k, v, causal=True)
    assert out.shape == (1, 2, 8, 32) and torch.isfinite(out).all()

    q = r(1, 1, 4, 8)
    k = torch.eye(4, 8).unsqueeze(0).unsqueeze(0).to(dev)
    v = torch.ones(1, 1, 4, 8, device=dev)
    out = dense_attention(q, k, v, causal=True)
    qd, kd, vd = q.double().cpu(), k.double().cpu(), v.double().cpu()
    manual = torch.matmul(torch.softmax(torch.matmul(qd, kd.transpose(-2, -1)) / (8 ** 0.5)
                                        + torch.triu(torch.full((4, 4), float("-inf"), dtype=torch.float64), diagonal=1),
                                        dim=-1), vd)
    assert torch.allclose(out.cpu().double(), manual, atol=1e-5)

    q, k, v = r(1, 2, 8, 32), r(1, 2, 16, 32), r(1, 2, 16, 32)
    out_sel, _ = semantic_block_attention(q, k, v, BlockLayout([S("a", 0, 16, BP.ALWAYS)]), causal=True,
                                          return_debug=True)
    assert torch.allclose(out_sel, dense_attention(q, k, v, causal=True), atol=1e-5)


@pytest.mark.gpu
def test_reference_intent_quant_attention_and_router_cases():
    """The reference's tests/test_intent_quant_attention.py and
    tests/test_end_to_end_router.py cases on device tensors (float32, so the
    reconstruction runs on the fake-quant kernel), each output also against the
    oracle's intent_quant_attention_reference (2e-5): output shape, the debug
    keys and counts, finite error metrics, non-negative byte savings, an ALWAYS
    block at least as precise as a low-score ATTEND block, zeros when nothing
    is selected, and the router -> kernel metadata -> attention chain."""
    from intent_attention import (BlockLayout, BlockPolicy as BP, BlockRouter, IntentQuantizer, RouterConfig,
                                  SemanticBlock as S, intent_quant_attention_reference, routing_to_kernel_metadata,
                                  semantic_block_attention)
    dev = torch.device("cuda:0")
    _say("reference test_intent_quant_attention / test_end_to_end_router cases")
    g = torch.Generator().manual_seed(12)

    def qkv(kv_len=64, q_len=8, heads=2, d=32):
        return tuple(torch.randn(1, heads, n, d, generator=g) for n in (q_len, kv_len, kv_len))

    def oracle(q, k, v, lay, pressure):
        olay = P.BlockLayout([P.SemanticBlock(b.name, b.start, b.end, b.policy.value, b.score) for b in lay.blocks])
        return A.intent_quant_attention_reference(q.numpy(), k.numpy(), v.numpy(), olay,
                                                  P.IntentQuantizer(memory_pressure=pressure))

    basic = BlockLayout([S("always", 0, 16, BP.ALWAYS), S("attend_high", 16, 32, BP.ATTEND, score=0.9),
                         S("attend_low", 32, 48, BP.ATTEND, score=0.3), S("skip", 48, 64, BP.SKIP)])
    for pressure in (0.3, 0.5, 0.8):
        q, k, v = qkv()
        out, dbg = intent_quant_attention_reference(q.to(dev), k.to(dev), v.to(dev), basic,
                                                    IntentQuantizer(memory_pressure=pressure), return_debug=True)
        assert out.shape == q.shape and torch.isfinite(out).all()
        assert {"precision_by_block", "bytes_saved_pct", "reconstruction_mse_k", "reconstruction_mse_v",
                "output_mse_vs_fp16_selected"} <= set(dbg)
        assert len(dbg["selected_block_names"]) == 3 and dbg["selected_tokens"] == 48
        assert dbg["output_mse_vs_fp16_selected"] >= 0.0 and -1.0 <= dbg["output_cosine_vs_fp16_selected"] <= 1.0
        assert dbg["bytes_saved_pct"] >= 0.0
        err = float(np.abs(out.cpu().numpy() - oracle(q, k, v, basic, pressure)).max())
        assert err <= 2e-5, (pressure, err)

    lay = BlockLayout([S("always", 0, 16, BP.ALWAYS), S("low_score", 16, 32, BP.ATTEND, score=0.1),
                       S("skip_me", 32, 48, BP.SKIP)])
    q, k, v = qkv(kv_len=48)
    _, dbg = intent_quant_attention_reference(q.to(dev), k.to(dev), v.to(dev), lay,
                                              IntentQuantizer(memory_pressure=0.7), return_debug=True)
    order = {"fp16": 0, "fp8": 1, "int8": 2, "int4_residual": 3, "int4": 4, "skip": 5}
    assert order.get(dbg["precision_by_block"]["always"], 99) <= order.get(dbg["precision_by_block"]["low_score"], 99)

    q, k, v = qkv(kv_len=16)
    out = intent_quant_attention_reference(q.to(dev), k.to(dev), v.to(dev), BlockLayout([S("skip", 0, 16, BP.SKIP)]),
                                           IntentQuantizer())
    assert torch.equal(out, torch.zeros_like(out))

    routed_layout = BlockLayout([S("system", 0, 64, BP.ALWAYS), S("doc_high", 64, 192, BP.ATTEND, score=0.85),
                                 S("doc_low", 192, 320, BP.ATTEND, score=0.15), S("recent", 320, 384, BP.RECENT),
                                 S("unused", 384, 448, BP.SKIP)])
    config = RouterConfig(memory_pressure=0.5)
    routed = BlockRouter(config).route_layout(routed_layout, 448)
    meta = routing_to_kernel_metadata(routed, page_size=16)
    assert meta["selected_page_ids"] and all(isinstance(p, int) for p in meta["selected_page_ids"])
    q, k, v = qkv(kv_len=448, q_len=4)
    out, dbg = semantic_block_attention(q.to(dev), k.to(dev), v.to(dev), routed_layout, return_debug=True)
    assert tuple(out.shape) == (1, 2, 4, 32) and dbg["selected_token_count"] > 0
    assert set(meta["selected_block_names"]) <= {b.name for b in routed_layout.selected_blocks()}
    out, dbg = intent_quant_attention_reference(q.to(dev), k.to(dev), v.to(dev), routed_layout,
                                                IntentQuantizer(memory_pressure=config.memory_pressure),
                                                return_debug=True)
    assert tuple(out.shape) == (1, 2, 4, 32)
    for name, prec in dbg["precision_by_block"].items():
        if name in meta["selected_block_names"]:
            assert prec.lower() in ("fp16", "fp8", "int8", "int4", "int4_residual")
    err = float(np.abs(out.cpu().numpy() - oracle(q, k, v, routed_layout, 0.5)).max())
    assert err <= 2e-5, err


@pytest.mark.gpu
def test_semantic_block_attention_dynamic_scores():
    """ATTEND blocks without a score are scored by the cosine probe before
    validation (reference.py:52-78), the scores land in the blocks and the debug
    dictionary, and the output is attention over the selected tokens."""
    from intent_attention import BlockLayout, BlockPolicy as BP, SemanticBlock as S, semantic_block_attention
    dev = torch.device("cuda:0")
    _say("semantic_block_attention dynamic scores")
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(1, 2, 4, 32, generator=g) for _ in range(3))
    k = torch.cat([k, torch.randn(1, 2, 44, 32, generator=g)], dim=-2)
    v = torch.cat([v, torch.randn(1, 2, 44, 32, generator=g)], dim=-2)
    mk = lambda: BlockLayout([S("sys", 0, 8, BP.ALWAYS), S("d1", 8, 24, BP.ATTEND), S("d2", 24, 40, BP.ATTEND),  # noqa
                              S("d3", 40, 48, BP.ATTEND, 0.7)])
    lay = mk()
    out, dbg = semantic_block_attention(q.to(dev), k.to(dev), v.to(dev), lay, return_debug=True)
    torch.cuda.synchronize()
    ref_scores = A.dynamic_block_scores(q.numpy(), k.numpy(), mk())
    assert set(dbg["dynamic_scores"]) == {"d1", "d2"}
    for n, s in ref_scores.items():
        assert abs(dbg["dynamic_scores"][n] - s) <= 1e-5
        assert lay.blocks[[b.name for b in lay.blocks].index(n)].score == dbg["dynamic_scores"][n]
    ref = A.dense_attention_masked(q.double().numpy(), k.double().numpy(), v.double().numpy())
    err = float(np.abs(out.cpu().double().numpy() - ref).max())
    _say(f"  scores {dbg['dynamic_scores']}, max abs err {err:.2e}")
    assert err <= 2e-5


@pytest.mark.gpu
def test_compare_function_returns_expected_keys():
    """The reference's test_compare_function_returns_expected_keys on device tensors,
    plus the values against the float64 oracle: the quantised output (through the
    golden-pinned fake quantisation) against attention over the selected tokens."""
    from intent_attention import (BlockLayout, BlockPolicy as BP, IntentQuantizer, SemanticBlock as S,
                                  compare_intent_quant_to_fp16_selected)
    dev = torch.device("cuda:0")
    _say("compare_intent_quant_to_fp16_selected")
    g = torch.Generator().manual_seed(9)
    q, k, v = (torch.randn(1, 2, 8 if i == 0 else 64, 32, generator=g) for i in range(3))
    lay = BlockLayout([S("always", 0, 16, BP.ALWAYS), S("attend_high", 16, 32, BP.ATTEND, score=0.9),
                       S("attend_low", 32, 48, BP.ATTEND, score=0.3), S("skip", 48, 64, BP.SKIP)])
    res = compare_intent_quant_to_fp16_selected(q.to(dev), k.to(dev), v.to(dev), lay,
                                                IntentQuantizer(memory_pressure=0.4))
    assert {"output_mse", "output_cosine_similarity", "bytes_saved_pct", "precision_by_block"} <= set(res)
    assert res["bytes_saved_pct"] >= 0.0
    assert res["fp16_selected_tokens"] == res["quant_selected_tokens"] == 48
    assert set(res) == {"output_mse", "output_cosine_similarity", "output_max_abs_error", "fp16_selected_tokens",
                        "quant_selected_tokens", "estimated_fp16_bytes", "estimated_quant_bytes", "bytes_saved_pct",
                        "precision_by_block", "reconstruction_mse_k", "reconstruction_mse_v"}
    olay = P.BlockLayout([P.SemanticBlock(b.name, b.start, b.end, b.policy.value, b.score) for b in lay.blocks])
    oq = P.IntentQuantizer(memory_pressure=0.4)
    assert res["precision_by_block"] == {b.name: oq.assign_block_precision(b).precision
                                         for b in olay.selected_blocks()}
    qn, kn, vn = (x.numpy() for x in (q, k, v))
    fp16 = A.semantic_block_attention(qn, kn, vn, olay)
    quant = A.intent_quant_attention_reference(qn, kn, vn, olay, oq)
    d = fp16 - quant
    mse, mx = float((d ** 2).mean()), float(np.abs(d).max())
    _say(f"  output_mse {res['output_mse']:.3e} (oracle {mse:.3e}), max abs {res['output_max_abs_error']:.3e} "
         f"(oracle {mx:.3e}), bytes saved {res['bytes_saved_pct']} %")
    assert abs(res["output_mse"] - mse) <= 0.02 * mse + 1e-9
    assert abs(res["output_max_abs_error"] - mx) <= 0.02 * mx + 1e-6
    assert 0.0 < res["output_cosine_similarity"] <= 1.0 + 1e-6


@pytest.mark.gpu
def test_dense_attention_fuzz():
    """Seeded random shapes around the kernel's thresholds (split over keys from
    256 keys on fewer than 512 rows, 4 / 8 / 16 waves per workgroup, head
    widths 1 .. 1,024, v_dim != head_dim), every dtype, with and without masks,
    triu or KV-position causality and broadcast leading dims, against the
    float64 oracle."""
    from intent_attention import dense_attention
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(2026)
    dts = [torch.float32, torch.float16, torch.bfloat16]
    for case in range(24):
        dt = dts[case % 3]
        lead = tuple(int(x) for x in rng.integers(1, 4, size=int(rng.integers(1, 3))))
        Tq = int(rng.choice([1, 1, 2, 5, 33]))
        Tk = int(rng.choice([1, 17, 300, 1023, 1024, 1500, 4100]))
        D = int(rng.choice([1, 32, 64, 96, 128, 200, 576]))
        Dv = int(rng.choice([D, 48, 128]))
        q, k, v, g = _dense_case(100 + case, lead, Tq, Tk, D, Dv, dt, dev)
        kw, okw = {}, {}
        mode = case % 4
        if mode == 1:
            m = torch.randn(Tq, Tk, generator=g)
            m[torch.rand(Tq, Tk, generator=g) < 0.2] = float("-inf")
            m[:, 0] = 0.0
            kw["mask"], okw["mask"] = m.to(dt), m.to(dt).double().numpy()
        elif mode == 2:
            kw["causal"] = okw["causal"] = True
        elif mode == 3:
            pos = torch.randperm(max(Tk, 2 * Tq), generator=g)[:Tk]
            pos[int(rng.integers(0, Tk))] = 0   # a key every query sees
            kw["causal"] = okw["causal"] = True
            kw["original_kv_positions"], okw["original_kv_positions"] = pos, pos.numpy()
        shared_kv = bool(rng.integers(0, 2)) and len(lead) == 2
        kk, vv = (k[:, :1], v[:, :1]) if shared_kv else (k, v)
        _say(f"  fuzz {case}: lead={lead} Tq={Tq} Tk={Tk} D={D} Dv={Dv} {dt} mode={mode} shared_kv={shared_kv}")
        t = lambda x: x.to(dev) if isinstance(x, torch.Tensor) else x  # noqa: E731
        out = dense_attention(t(q), t(kk), t(vv), **{n: t(x) for n, x in kw.items()})
        torch.cuda.synchronize()
        assert out.shape == (*lead, Tq, Dv) and out.dtype == dt
        ref = A.dense_attention_masked(q.double().numpy(), kk.double().numpy(), vv.double().numpy(), **okw)
        o = out.cpu().double().numpy()
        assert np.array_equal(np.isnan(o), np.isnan(ref)) and not np.isnan(ref).any()
        err = float(np.abs(o - ref).max())
        # float32 arithmetic, then one rounding of the output to its dtype (half an ulp
        # of the largest output: 2^-11 relative for float16, 2^-8 for bfloat16)
        half_ulp = {torch.float32: 0.0, torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}[dt]
        tol = 2e-5 + half_ulp * float(np.abs(ref).max())
        _say(f"    max abs err {err:.2e} (bar {tol:.2e})")
        assert err <= tol, (case, err, tol)
