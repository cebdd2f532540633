"""The decode kernel's in-kernel merge (iak_paged_decode_args.merge_in_kernel = 1)
against the merge-kernel form of the same call and against the oracle.

In-kernel, a workgroup's four waves reduce four consecutive splits of one row
and combine them in LDS; the workgroup that arrives last at the row's counter
merges the row. Checked here: every GQA width and head_dim, query and output
dtypes, split counts that are not multiples of four (empty trailing splits),
rows with no pages, token bounds, more than eight workgroups per row; the
result is deterministic from run to run (the merge order is fixed, whichever
workgroup merges); the arrival counters are left zero after every call; stale
partials in the workspace do not leak into the next call; three HIP graph
replays equal the eager call."""
import sys

import numpy as np
import pytest

from oracle import decode as Dm
from tests._pools import random_case, to_device_pools

pytestmark = pytest.mark.gpu

TOL_QUANT = 1e-2
MIX = {"FP16": .25, "FP8": .2, "INT8": .2, "INT4": .15, "INT4_RESIDUAL": .15, "SKIP": .05}


def _say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def dev():
    import torch
    return torch.device("cuda:0")


def _plans(dev, seed, B, Hq, Hkv, D, NP, W, pps, q_dtype=None, out_dtype=None, valid=None, zero_rows=()):
    import torch
    from intent_attention.decode_core import make_plan
    q, pools, table, counts, tags = random_case(seed, B, Hq, Hkv, D, NP, W, MIX, outliers=0.01)
    for r in zero_rows:
        counts.flat[r] = 0
    t = lambda x: torch.from_numpy(x).to(dev)  # noqa: E731
    qd = t(q) if q_dtype is None else t(q).to(q_dtype)
    dp = to_device_pools(pools, dev)
    vt = None if valid is None else t(valid)
    kw = dict(out_dtype=out_dtype or torch.float32, pages_per_split=pps, valid_tokens=vt)
    fused = make_plan(qd, dp, t(table), t(counts), t(tags), merge_in_kernel=True, **kw)
    split = make_plan(qd, dp, t(table), t(counts), t(tags), merge_in_kernel=False, **kw)
    ref = Dm.paged_decode_oracle(qd.float().cpu().numpy(), pools, table, counts, tags, valid_tokens=valid)
    return fused, split, ref


def _counters(plan):
    """The arrival-counter region at the end of the workspace, as int32."""
    rows = plan.args.batch * plan.args.num_kv_heads
    tail = (rows * 4 + 255) // 256 * 256
    return plan._ws[-tail:].view(dtype=__import__("torch").int32)


CASES = [
    # seed, B, Hq, Hkv, D, NP, W, pages_per_split
    (101, 2, 8, 2, 128, 96, 70, 16),     # 5 splits -> 8 (3 empty), 2 workgroups per row
    (102, 3, 4, 4, 64, 64, 45, 8),       # G = 1, 6 splits -> 8
    (103, 2, 32, 2, 128, 128, 120, 8),   # G = 16, 15 splits -> 16
    (104, 1, 8, 1, 64, 80, 33, 16),      # 3 splits -> 4
    (105, 2, 16, 2, 128, 256, 600, 8),   # 75 splits -> 76: 19 workgroups per row (> 8 per load round)
    (106, 4, 32, 8, 128, 200, 150, 0),   # automatic plan
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"seed{c[0]}")
def test_in_kernel_merge_matches_merge_kernel_and_oracle(dev, case):
    import torch
    seed, B, Hq, Hkv, D, NP, W, pps = case
    _say("in-kernel merge", f"seed={seed} B={B} Hq={Hq} Hkv={Hkv} D={D} W={W} pages_per_split={pps}")
    fused, split, ref = _plans(dev, seed, B, Hq, Hkv, D, NP, W, pps, zero_rows=(B * Hkv - 1,))
    split.run()
    fused.run()
    torch.cuda.synchronize()
    a, b = fused.out.cpu().numpy(), split.out.cpu().numpy()
    scale = max(float(np.abs(b).max()), 1e-30)
    d_split = float(np.abs(a - b).max())
    err = float(np.abs(a - ref).max())
    _say(f"  vs merge kernel {d_split:.2e} (max |out| {scale:.2e}); vs oracle {err:.2e}")
    assert d_split <= 1e-5 * scale
    assert err <= TOL_QUANT
    assert np.all(a[-1, -(Hq // Hkv):] == 0.0)           # the empty row
    assert int(_counters(fused).abs().sum()) == 0          # counters left zero
    first = fused.out.clone()
    for _ in range(2):
        fused.out.fill_(float("nan"))
        fused.run()
        torch.cuda.synchronize()
        assert torch.equal(fused.out, first)               # deterministic, counters reset
    assert int(_counters(fused).abs().sum()) == 0


@pytest.mark.parametrize("q_dtype,out_dtype", [("float32", "float16"), ("bfloat16", "bfloat16"),
                                               ("float16", "float16")])
def test_in_kernel_merge_dtypes_and_token_bounds(dev, q_dtype, out_dtype):
    import torch
    qd, od = getattr(torch, q_dtype), getattr(torch, out_dtype)
    _say("in-kernel merge dtypes", q_dtype, out_dtype)
    B, Hq, Hkv, D, NP, W = 2, 8, 2, 128, 96, 80
    valid = np.array([[16 * 80, 16 * 37 + 5], [16 * 12 + 1, 0]], np.int32)
    fused, split, ref = _plans(dev, 111, B, Hq, Hkv, D, NP, W, 8, q_dtype=qd, out_dtype=od, valid=valid)
    split.run()
    fused.run()
    torch.cuda.synchronize()
    a, b = fused.out.float().cpu().numpy(), split.out.float().cpu().numpy()
    ulp = 1e-2 if od == torch.bfloat16 else 1e-3              # one output rounding apart
    assert np.abs(a - b).max() <= ulp * max(float(np.abs(b).max()), 1e-30)
    assert np.abs(a - ref).max() <= TOL_QUANT + (2e-2 if od == torch.bfloat16 else 0.0)


def test_stale_partials_do_not_leak(dev):
    """Garbage in the partial region (counters kept zero) changes nothing:
    every partial a merge reads is written in the same call."""
    import torch
    _say("in-kernel merge stale partials")
    fused, _, ref = _plans(dev, 121, 2, 8, 2, 128, 96, 70, 8)
    fused.run()
    torch.cuda.synchronize()
    want = fused.out.clone()
    cnt = _counters(fused)
    body = fused._ws[: fused._ws.numel() - cnt.numel() * 4]
    body.view(torch.float32).fill_(float("nan"))
    fused.run()
    torch.cuda.synchronize()
    assert torch.equal(fused.out, want)


def test_graph_replays_equal_eager(dev):
    import torch
    _say("in-kernel merge graph replays")
    fused, _, _ = _plans(dev, 131, 2, 16, 4, 128, 128, 90, 8)
    fused.run()
    torch.cuda.synchronize()
    want = fused.out.clone()
    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            fused.run()
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize()
    for i in range(3):
        fused.out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(fused.out, want), i
        assert int(_counters(fused).abs().sum()) == 0


def test_first_run_on_another_stream(dev):
    """The plan zero-fills its counters on the current stream; a first run on
    another stream waits for that fill."""
    import torch
    _say("in-kernel merge on a side stream")
    fused, _, ref = _plans(dev, 141, 2, 8, 2, 128, 96, 70, 8)
    side = torch.cuda.Stream(dev)
    fused.run(stream=side.cuda_stream)
    side.synchronize()
    got = fused.out.clone()
    assert np.abs(got.cpu().numpy() - ref).max() <= TOL_QUANT
    fused.run()
    torch.cuda.synchronize()
    assert torch.equal(got, fused.out)


def test_long_rows(dev):
    """Rows of 8,192 selected pages (131,072 tokens; entries may repeat a page):
    128 splits per row, 32 workgroup partials per row in-kernel; both merge
    forms against the oracle, with a peaked softmax (query scale 4)."""
    import torch
    from intent_attention import _native as N
    from intent_attention.decode_core import make_plan
    B, Hq, Hkv, D, NP, W = 1, 16, 2, 128, 2048, 8192
    q, pools, table, counts, tags = random_case(151, B, Hq, Hkv, D, NP, W, {"FP16": .5, "INT8": .3, "FP8": .2},
                                                q_scale=4.0)
    counts[:] = [[W, W - 777]]
    ref = Dm.paged_decode_oracle(q, pools, table, counts, tags, dtype=np.float32)
    t = lambda x: torch.from_numpy(x).to(dev)  # noqa: E731
    dp = to_device_pools(pools, dev)
    for merge in (True, False):
        _say("long rows", f"merge_in_kernel={merge}")
        plan = make_plan(t(q), dp, t(table), t(counts), t(tags), out_dtype=torch.float32, merge_in_kernel=merge)
        info = N.plan_info(plan.args)
        assert info["splits"] >= 128 and info["merge_in_kernel"] == merge
        plan.run()
        torch.cuda.synchronize()
        got = plan.out.cpu().numpy()
        err = float(np.abs(got - ref).max())
        rel = err / float(np.abs(ref).max())
        _say(f"  splits {info['splits']}, max abs err {err:.2e}, relative {rel:.2e}")
        assert err <= TOL_QUANT and rel <= 1e-2


def test_two_tier_plan(dev):
    """A grid large enough for the automatic two-tier plan (64 rows of 4,800
    entries: 5,120 waves): both merge forms against the oracle on two
    sequences, and against a one-tier plan of the same split length."""
    import torch
    from intent_attention import _native as N
    from intent_attention.decode_core import make_plan
    B, Hq, Hkv, D, NP, W = 8, 32, 8, 128, 2048, 4800
    q, pools, table, counts, tags = random_case(161, B, Hq, Hkv, D, NP, W, {"FP16": .3, "INT8": .3, "FP8": .2,
                                                                          "INT4": .2}, q_scale=4.0)
    counts[:] = W
    counts[3, 5] = W - 1111
    t = lambda x: torch.from_numpy(x).to(dev)  # noqa: E731
    dp = to_device_pools(pools, dev)
    sel = [0, 3]
    ref = Dm.paged_decode_oracle(q[sel], pools, table[sel], counts[sel], tags, dtype=np.float32)
    outs = {}
    for merge in (True, False):
        plan = make_plan(t(q), dp, t(table), t(counts), t(tags), out_dtype=torch.float32, merge_in_kernel=merge)
        info = N.plan_info(plan.args)
        _say("two-tier plan", f"merge_in_kernel={merge}", info)
        assert info["tail_splits"] > 0 and info["merge_in_kernel"] == merge
        plan.run()
        torch.cuda.synchronize()
        got = plan.out.cpu().numpy()
        err = float(np.abs(got[sel] - ref).max())
        rel = err / float(np.abs(ref).max())
        _say(f"  vs oracle: max abs err {err:.2e}, relative {rel:.2e}")
        assert err <= TOL_QUANT and rel <= 1e-2
        outs[merge] = got
    one = make_plan(t(q), dp, t(table), t(counts), t(tags), out_dtype=torch.float32, merge_in_kernel=False,
                    pages_per_split=info["pages_per_split"])
    assert N.plan_info(one.args)["tail_splits"] == 0
    one.run()
    torch.cuda.synchronize()
    base = one.out.cpu().numpy()
    scale = float(np.abs(base).max())
    for merge, got in outs.items():
        d = float(np.abs(got - base).max())
        _say(f"  merge_in_kernel={merge} vs one tier: {d:.2e} (max |out| {scale:.2e})")
        assert d <= 1e-3 * scale
    assert float(np.abs(outs[True] - outs[False]).max()) <= 1e-5 * scale


@pytest.mark.parametrize("out_name", ["float16", "bfloat16"])
@pytest.mark.parametrize("D", [64, 128])
def test_merge_kernel_packed_and_element_stores_agree(dev, out_name, D):
    """The merge kernel writes a 16-bit output row as one packed store per lane
    when the output keeps the lane's values aligned, else element by element.
    The same call into an aligned output and into a view one element off (so
    every row is misaligned) gives bit-identical values."""
    import torch
    from intent_attention.decode_core import make_plan
    od = getattr(torch, out_name)
    _say("merge stores", f"D={D} out={out_name}")
    B, Hq, Hkv = 2, 8, 2
    q, pools, table, counts, tags = random_case(740 + D, B, Hq, Hkv, D, 300, 90, MIX, outliers=0.01)
    t = lambda x: torch.from_numpy(x).to(dev)  # noqa: E731
    dp = to_device_pools(pools, dev)
    big = torch.full((B * Hq * D + 1,), float("nan"), dtype=od, device=dev)
    views = {"aligned": big[:B * Hq * D].view(B, Hq, D), "offset": big[1:].view(B, Hq, D)}
    got = {}
    for name, out in views.items():
        plan = make_plan(t(q), dp, t(table), t(counts), t(tags), out=out, merge_in_kernel=False, pages_per_split=8)
        assert plan.args.out % 4 == (0 if name == "aligned" else 2)
        plan.run()
        torch.cuda.synchronize()
        got[name] = out.float().cpu().numpy().copy()
    assert np.isfinite(got["aligned"]).all()
    assert np.array_equal(got["aligned"], got["offset"])


@pytest.mark.parametrize("out_name", ["float16", "bfloat16"])
def test_mla_merge_packed_and_element_stores_agree(dev, out_name):
    """As above for the MLA decode's merge (512 value dims, eight per lane)."""
    import torch
    sys.path.insert(0, __import__("os").path.dirname(__file__))
    from test_gpu_mla import _latent_case, _device_pools
    from intent_attention.mla_core import make_mla_plan
    od = getattr(torch, out_name)
    _say("mla merge stores", f"out={out_name}")
    q, pools, table, counts, tags = _latent_case(77, 2, 20, 576, 200, 140, {"FP8": .45, "INT8": .45, "SKIP": .1})
    B, H = 2, 20
    big = torch.full((B * H * 512 + 8,), float("nan"), dtype=od, device=dev)
    views = {"aligned": big[:B * H * 512].view(B, H, 512), "offset": big[1:1 + B * H * 512].view(B, H, 512)}
    got = {}
    for name, out in views.items():
        plan = make_mla_plan(torch.from_numpy(q).to(dev), _device_pools(pools, dev), torch.from_numpy(table).to(dev),
                             torch.from_numpy(counts).to(dev), torch.from_numpy(tags).to(dev), v_dim=512, out=out,
                             pages_per_split=16)
        plan.run()
        torch.cuda.synchronize()
        got[name] = out.float().cpu().numpy().copy()
    assert np.isfinite(got["aligned"]).all()
    assert np.array_equal(got["aligned"], got["offset"])
