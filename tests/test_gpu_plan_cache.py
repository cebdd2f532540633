"""GPU: validated plans reused across calls, and entry records packed
automatically on a plan's repeated runs.

* ``DecodePlan`` (auto_records on): the second run over an unchanged table,
  tags and scales packs entry records and reads them; outputs stay
  bit-identical to a plan that never does; an in-place write to the table
  (torch op), to the tags, or to the scales through the quantiser (raw
  pointer writes that bump torch's version counters) drops the records and
  the next runs match the oracle on the new state.
* ``fused_selected_quant_decode`` / ``intent_quant_decode_attention_triton``:
  repeated calls over the same pools, table, tags and counts reuse one plan,
  return a new output each call, follow new query values and in-place table
  edits, and do not keep the pools alive.
"""
import gc
import sys
import weakref

import numpy as np
import pytest

from oracle import decode as Dm
from tests._pools import build_pools, to_device_pools

pytestmark = pytest.mark.gpu
TOL_QUANT = 1e-2


def _say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def dev():
    import torch
    return torch.device("cuda:0")


def _case(seed, B=2, Hq=8, Hkv=2, D=128, NP=120, W=90):
    rng = np.random.default_rng(seed)
    mix = {Dm.FP16: .25, Dm.FP8: .2, Dm.INT8: .2, Dm.INT4: .15, Dm.INT4_RESIDUAL: .15, Dm.SKIP: .05}
    tags = rng.choice(list(mix), size=NP, p=np.array(list(mix.values())) / sum(mix.values())).astype(np.int32)
    pools = build_pools(rng, NP, D, tags, outliers=0.01)
    table = rng.integers(0, NP, size=(B, Hkv, W)).astype(np.int32)
    counts = rng.integers(W // 2, W + 1, size=(B, Hkv)).astype(np.int32)
    q = rng.standard_normal((B, Hq, D)).astype(np.float16)
    return q, pools, table, counts, tags


def test_auto_records_follow_the_state(dev):
    import torch
    from intent_attention.decode_core import make_plan
    from intent_attention.quantize import quantize_pages
    _say("automatic entry records")
    q, pools, table, counts, tags = _case(301)
    t = lambda x: torch.from_numpy(x).to(dev)  # noqa: E731
    dp = to_device_pools(pools, dev)
    tq, tt, tc, tg = t(q), t(table), t(counts), t(tags)
    plain = make_plan(tq, dp, tt, tc, tg, out_dtype=torch.float32, auto_records=False)
    auto = make_plan(tq, dp, tt, tc, tg, out_dtype=torch.float32, pages_per_split=16)
    ref_plan = make_plan(tq, dp, tt, tc, tg, out_dtype=torch.float32, pages_per_split=16, auto_records=False)
    plain.run()
    ref_plan.run()
    auto.run()
    assert not auto.reads_records
    auto.run()                        # second run on the same state: records packed and read
    torch.cuda.synchronize()
    assert auto.reads_records and not plain.reads_records
    assert torch.equal(auto.out, ref_plan.out)
    oracle = Dm.paged_decode_oracle(q.astype(np.float32), pools, table, counts, tags)
    assert float(np.abs(auto.out.cpu().numpy() - oracle).max()) <= TOL_QUANT

    # an in-place table edit (torch op): records dropped, new state decoded
    perm = np.random.default_rng(5).permutation(table.shape[-1])
    table2 = np.ascontiguousarray(table[..., perm][..., ::-1])
    tt.copy_(t(table2))
    auto.out.fill_(float("nan"))
    auto.run()
    torch.cuda.synchronize()
    assert not auto.reads_records
    oracle2 = Dm.paged_decode_oracle(q.astype(np.float32), pools, table2, counts, tags)
    assert float(np.abs(auto.out.cpu().numpy() - oracle2).max()) <= TOL_QUANT
    auto.run()
    ref_plan.run()
    torch.cuda.synchronize()
    assert auto.reads_records and torch.equal(auto.out, ref_plan.out)

    # tags edited in place: an INT8 page becomes SKIP
    i8 = int(np.flatnonzero(tags == Dm.INT8)[0])
    tags2 = tags.copy()
    tags2[i8] = Dm.SKIP
    tg[i8] = Dm.SKIP
    auto.run()
    torch.cuda.synchronize()
    oracle3 = Dm.paged_decode_oracle(q.astype(np.float32), pools, table2, counts, tags2)
    assert float(np.abs(auto.out.cpu().numpy() - oracle3).max()) <= TOL_QUANT

    # scales rewritten by the quantiser (raw pointers; it bumps the version counters):
    # every INT8 page's K re-quantised from 4x its values
    auto.run()
    torch.cuda.synchronize()
    assert auto.reads_records
    ids = np.flatnonzero(tags2 == Dm.INT8)
    src = (torch.from_numpy(pools["k_fp16"][ids].astype(np.float32) * 4).half()).to(dev)
    quantize_pages(src, "INT8", codes=dp.k_int8, scales=dp.k_int8_scale, dst_pages=t(ids.astype(np.int32)))
    auto.run()
    torch.cuda.synchronize()
    pools4 = dict(pools)
    pools4["k_i8"] = dp.k_int8.cpu().numpy()
    pools4["k_i8_scale"] = dp.k_int8_scale.cpu().numpy()
    oracle4 = Dm.paged_decode_oracle(q.astype(np.float32), pools4, table2, counts, tags2)
    err = float(np.abs(auto.out.cpu().numpy() - oracle4).max())
    moved = float(np.abs(oracle4 - oracle3).max())
    _say(f"  after re-quantisation: max abs err {err:.2e} (the change moved outputs by {moved:.2e})")
    assert err <= TOL_QUANT and moved > 10 * TOL_QUANT


@pytest.mark.parametrize("api", ["fused", "sibling"])
def test_reference_api_reuses_plans(dev, api):
    import torch
    from intent_attention import fused_selected_quant_decode, intent_quant_decode_attention_triton
    import importlib
    # the package exports a function of the same name as the module: import the module itself
    fmod = importlib.import_module("intent_attention.fused_selected_quant_decode")
    smod = importlib.import_module("intent_attention.intent_quant_decode")
    from intent_attention import FusedDecodeConfig, IntentQuantKernelConfig
    _say("plan cache", api)
    rng = np.random.default_rng(17)
    B, H, D, NP, W = 2, 4, 64, 48, 20
    tags = rng.choice([Dm.FP16, Dm.INT8], size=NP).astype(np.int32)
    pools = build_pools(rng, NP, D, tags)
    table = rng.integers(0, NP, size=(B, H, W)).astype(np.int32)
    counts = np.full((B, H), W, np.int32)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)  # noqa: E731
    k16, v16, k8, v8 = t(pools["k_fp16"]), t(pools["v_fp16"]), t(pools["k_i8"]), t(pools["v_i8"])
    ks, vs = t(pools["k_i8_scale"]), t(pools["v_i8_scale"])
    tt, tc = t(table), t(counts)
    mod = fmod if api == "fused" else smod
    mod.clear_plan_cache()
    if api == "fused":
        tg = t(tags)
        cfg = FusedDecodeConfig(head_dim=D, max_selected_pages=W)

        def call(q):
            return fused_selected_quant_decode(q[:, :, None, :], k16, v16, k8, v8, ks, vs, tt, tg, tc, cfg)[:, :, 0]
    else:
        # sibling numbering: FP16 0, INT8 2
        tg = t(np.where(tags == Dm.FP16, 0, 2).astype(np.int32))
        cfg = IntentQuantKernelConfig(head_dim=D, max_selected_pages=W)

        def call(q):
            return intent_quant_decode_attention_triton(q, k16, v16, k8, v8, ks, vs, tt, tc, tg, config=cfg)

    outs = []
    for step in range(4):
        q = rng.standard_normal((B, H, D)).astype(np.float16)
        o = call(t(q))
        outs.append(o)
        torch.cuda.synchronize()
        ref = Dm.paged_decode_oracle(q.astype(np.float32), pools, table, counts, tags)
        err = float(np.abs(o.float().cpu().numpy() - ref).max())
        assert err <= TOL_QUANT, (step, err)
        assert len(mod._PLANS._d) == 1
    assert len({o.data_ptr() for o in outs}) == len(outs)      # a new output every call
    # an in-place table edit is seen by the cached plan (its records are dropped)
    table2 = np.ascontiguousarray(table[..., ::-1])
    tt.copy_(t(table2))
    q = rng.standard_normal((B, H, D)).astype(np.float16)
    o = call(t(q))
    torch.cuda.synchronize()
    ref = Dm.paged_decode_oracle(q.astype(np.float32), pools, table2, counts, tags)
    assert float(np.abs(o.float().cpu().numpy() - ref).max()) <= TOL_QUANT
    assert len(mod._PLANS._d) == 1
    # the cache holds no pool alive
    probe = weakref.ref(k16)
    del k16, v16, k8, v8, ks, vs, call
    gc.collect()
    assert probe() is None
    mod.clear_plan_cache()


def test_streams_keep_plans_apart(dev):
    """A plan's automatic records stay on the stream that packed them: a run on
    another stream turns them off (still correct); the reference entry point
    keeps one plan per stream, since a plan's workspace is reused by every run."""
    import importlib
    import torch
    from intent_attention import FusedDecodeConfig, fused_selected_quant_decode
    from intent_attention.decode_core import make_plan
    fmod = importlib.import_module("intent_attention.fused_selected_quant_decode")
    _say("plans and streams")
    q, pools, table, counts, tags = _case(303)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)  # noqa: E731
    dp = to_device_pools(pools, dev)
    tq, tt, tc, tg = t(q), t(table), t(counts), t(tags)
    plan = make_plan(tq, dp, tt, tc, tg, out_dtype=torch.float32, pages_per_split=16)
    plan.run()
    plan.run()
    torch.cuda.synchronize()
    assert plan.reads_records
    want = plan.out.clone()
    from intent_attention.decode_core import current_stream_handle
    side = torch.cuda.Stream(device=dev)
    assert current_stream_handle(dev) == torch.cuda.current_stream(dev).cuda_stream
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        assert current_stream_handle(dev) == side.cuda_stream
        plan.out.fill_(float("nan"))
        plan.run()
    torch.cuda.synchronize()
    assert not plan.reads_records and torch.equal(plan.out, want)

    fmod.clear_plan_cache()
    rng = np.random.default_rng(9)
    B, H, D, NP, W = 1, 2, 64, 24, 12
    ftags = rng.choice([Dm.FP16, Dm.INT8], size=NP).astype(np.int32)
    fp = build_pools(rng, NP, D, ftags)
    args = [t(fp["k_fp16"]), t(fp["v_fp16"]), t(fp["k_i8"]), t(fp["v_i8"]), t(fp["k_i8_scale"]),
            t(fp["v_i8_scale"]), t(rng.integers(0, NP, size=(B, H, W)).astype(np.int32)), t(ftags),
            t(np.full((B, H), W, np.int32))]
    cfg = FusedDecodeConfig(head_dim=D, max_selected_pages=W)
    qq = t(rng.standard_normal((B, H, 1, D)).astype(np.float16))
    a = fused_selected_quant_decode(qq, *args, cfg)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        b = fused_selected_quant_decode(qq, *args, cfg)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and len(fmod._PLANS._d) == 2
    fmod.clear_plan_cache()


@pytest.mark.parametrize("merge", [False, True])
def test_plan_replays_in_a_hip_graph(dev, merge):
    """A plan's step captured in a HIP graph (torch.cuda.CUDAGraph) for a
    launch-bound serving loop: the capture holds the split kernel and the
    merge (kernel, or in-kernel with its self-resetting arrival counters) and
    no allocation, memset or host synchronisation. Each replay, after an
    in-place update of the query and with eager work and synchronisations
    between replays, matches an eager plan over the same tensors bit for bit
    and the oracle within the quantised bar."""
    import torch
    from intent_attention.decode_core import make_plan
    _say("plan in a HIP graph, merge in kernel:", merge)
    q, pools, table, counts, tags = _case(307)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)  # noqa: E731
    dp = to_device_pools(pools, dev)
    tq, tt, tc, tg = t(q), t(table), t(counts), t(tags)
    kw = dict(out_dtype=torch.float32, pages_per_split=16, merge_in_kernel=merge, auto_records=False)
    plan = make_plan(tq, dp, tt, tc, tg, **kw)
    eager = make_plan(tq, dp, tt, tc, tg, **kw)
    plan.run()                        # first run outside the capture (workspace fill waited on)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan.run()
    rng = np.random.default_rng(11)
    for i in range(4):
        qn = rng.standard_normal(q.shape).astype(np.float16)
        tq.copy_(t(qn))
        plan.out.fill_(float("nan"))
        graph.replay()
        eager.run()
        torch.cuda.synchronize()
        assert torch.equal(plan.out, eager.out), i
        ref = Dm.paged_decode_oracle(qn.astype(np.float32), pools, table, counts, tags)
        err = float(np.abs(plan.out.cpu().numpy() - ref).max())
        _say(f"  replay {i}: bit-identical to eager, max abs err vs oracle {err:.2e}")
        assert err <= TOL_QUANT
    del graph
