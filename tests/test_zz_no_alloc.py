"""iak_paged_decode_noalloc (no caller workspace, no allocation: the split-K
partials in the library's own per-GPU scratch) against iak_paged_decode with
a caller workspace and the merge kernel (merge_in_kernel = 0, the form the
no-alloc entry point always takes), through the C ABI: two calls in a row, the
second with a smaller input, each bit-identical to the workspace entry point
(the same kernels and split plan) and within the quantised-page bar of the oracle; a
call whose partials exceed the scratch is rejected before any launch; and the
call captured in a HIP graph (after one eager call), replayed three times with
the query and the page table changed in between, each replay bit-identical to
iak_paged_decode on the same inputs."""
import sys

import numpy as np
import pytest

from oracle import decode as Dm
from tests._pools import random_case, to_device_pools

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


def _case(dev, seed, B, Hq, Hkv, W, NP, pps, with_tensors=False):
    import torch
    from intent_attention.decode_core import make_plan
    mix = {"FP16": .25, "FP8": .2, "INT8": .2, "INT4": .2, "INT4_RESIDUAL": .15}
    q, pools, table, counts, tags = random_case(seed, B, Hq, Hkv, 128, NP, W, mix, outliers=0.01)
    t = lambda x: torch.from_numpy(x).to(dev)  # noqa: E731
    tq, tt = t(q), t(table)
    plan = make_plan(tq, to_device_pools(pools, dev), tt, t(counts), t(tags), out_dtype=torch.float32,
                     pages_per_split=pps, merge_in_kernel=False, auto_records=False)
    if with_tensors:
        return plan, (q, pools, table, counts, tags), (tq, tt)
    return plan, (q, pools, table, counts, tags)


def test_noalloc_matches_workspace_entry_point():
    import torch
    from intent_attention import _native as N
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev).cuda_stream
    for seed, B, Hq, Hkv, W, NP, pps in ((61, 4, 16, 4, 300, 160, 0), (62, 2, 8, 2, 90, 64, 16)):
        _say("noalloc", f"seed={seed} B={B} Hq={Hq} Hkv={Hkv} W={W} pages_per_split={pps}")
        plan, host = _case(dev, seed, B, Hq, Hkv, W, NP, pps)
        assert 0 < plan.workspace_bytes <= N.NOALLOC_SCRATCH_BYTES
        plan.run()
        torch.cuda.synchronize()
        want = plan.out.clone()
        plan.out.fill_(float("nan"))
        torch.cuda.synchronize()
        N.paged_decode_noalloc(plan.args, stream)
        torch.cuda.synchronize()
        assert torch.equal(plan.out, want)
        ref = Dm.paged_decode_oracle(host[0], host[1], host[2], host[3], host[4])
        err = float(np.abs(plan.out.cpu().numpy() - ref).max())
        _say(f"  bit-identical to iak_paged_decode; max abs err vs oracle {err:.2e}")
        assert err <= 1e-2


def test_noalloc_rejects_partials_above_the_scratch():
    import torch
    from intent_attention import _native as N
    from intent_attention.decode_core import PagePools, make_plan
    dev = torch.device("cuda:0")
    _say("noalloc size limit")
    B, Hq, Hkv, D, W, NP = 64, 32, 8, 128, 1024, 64
    pools = PagePools(k_fp16=torch.zeros(NP, 16, D, dtype=torch.float16, device=dev),
                      v_fp16=torch.zeros(NP, 16, D, dtype=torch.float16, device=dev))
    plan = make_plan(torch.zeros(B, Hq, D, dtype=torch.float16, device=dev), pools,
                     torch.zeros(B, Hkv, W, dtype=torch.int32, device=dev),
                     torch.full((B, Hkv), W, dtype=torch.int32, device=dev),
                     torch.zeros(NP, dtype=torch.int32, device=dev), pages_per_split=64, merge_in_kernel=False)
    assert plan.workspace_bytes > N.NOALLOC_SCRATCH_BYTES
    with pytest.raises(ValueError, match="no-alloc scratch"):
        N.paged_decode_noalloc(plan.args, torch.cuda.current_stream(dev).cuda_stream)


def test_noalloc_under_graph_capture():
    import torch
    from intent_attention import _native as N
    dev = torch.device("cuda:0")
    _say("noalloc graph capture: seed=63 B=3 Hq=16 Hkv=4 W=120")
    plan, host, (tq, tt) = _case(dev, 63, 3, 16, 4, 120, 96, 16, with_tensors=True)
    assert 0 < plan.workspace_bytes <= N.NOALLOC_SCRATCH_BYTES
    # eager call first: the scratch address of this GPU is looked up outside the capture
    N.paged_decode_noalloc(plan.args, torch.cuda.current_stream(dev).cuda_stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        N.paged_decode_noalloc(plan.args, torch.cuda.current_stream(dev).cuda_stream)
    torch.cuda.synchronize()
    rng = np.random.default_rng(7)
    for rep in range(3):
        if rep == 1:       # new query values in place
            tq.copy_(torch.from_numpy(rng.standard_normal(tuple(tq.shape)).astype(np.float16)).to(dev))
        if rep == 2:       # a new page table in place
            tt.copy_(torch.from_numpy(rng.integers(0, 96, size=tuple(tt.shape)).astype(np.int32)).to(dev))
        plan.out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = plan.out.clone()
        plan.out.fill_(float("nan"))
        plan.run()          # iak_paged_decode with the caller's workspace, eager
        torch.cuda.synchronize()
        same = torch.equal(got, plan.out)
        _say(f"  replay {rep}: bit-identical to iak_paged_decode {same}")
        assert same and not torch.isnan(got).any()
    ref = Dm.paged_decode_oracle(tq.cpu().numpy(), host[1], tt.cpu().numpy(), host[3], host[4])
    assert float(np.abs(got.cpu().numpy() - ref).max()) <= 1e-2
    del g
