"""intent_quant_attention_reference and dense_attention of the product
(intent_attention.intent_quant_attention / intent_attention.reference), with
the attention on the HIP paged decode.

GPU: the reference's own outputs (golden g4: the cfg1 shape with its
alternating FP16 / INT8 plan, and a plan with every precision including a
SKIP-precision block, plus the default policy) within the quantised-page bar
1e-2; the debug dictionary's keys and values; dense_attention against a
float64 softmax over shapes, dtypes, causal masks and ragged lengths, and
the reference's error behaviour. CPU: the errors raised before any device
work (causal, host tensors, additive masks).
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
    with pytest.raises(NotImplementedError, match="mask"):
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
    # float16 pages: K/V rounded to float16 (float32 / bfloat16 inputs), the output to its dtype
    tol = {"float32": 2e-3, "float16": 2e-3, "bfloat16": 1e-2}[dt]
    _say(f"  max abs err {err:.2e}")
    assert err <= tol


@pytest.mark.gpu
def test_dense_attention_dtype_mismatch_raises():
    from intent_attention import dense_attention
    dev = torch.device("cuda:0")
    q = torch.zeros(1, 2, 1, 64, device=dev)
    with pytest.raises(RuntimeError, match="same dtype"):
        dense_attention(q.half(), q, q)
