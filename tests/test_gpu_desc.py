"""Page descriptors (iak_paged_decode_args.page_desc, iak_pack_page_descriptors)
and entry records (entry_records, iak_pack_entry_records) on the GPU.

A descriptor holds a page's native tag and the scales its precision uses in
one 32-byte line; an entry record holds the same for one page-table entry,
with the resolved page id. Checked here: the packed words equal a host
restatement of the tag translation, id resolution and scale slots (tag map,
map_other_tags, out-of-range tags and ids, negative ids, f16 and f32 scales,
INT4 groups of D/4, D/2 and D); a decode that reads descriptors or records is
bit-identical to the same decode on page_table, page_tags, tag_map and the
scale arrays, in both merge forms, with token bounds and negative page ids; a
precision with no pools in the decode contributes nothing; the result also
matches the oracle."""
import sys

import numpy as np
import pytest

from oracle import decode as Dm
from tests._pools import build_pools, to_device_pools

pytestmark = pytest.mark.gpu

TOL_QUANT = 1e-2
NATIVE = (Dm.FP16, Dm.INT8, Dm.FP8, Dm.INT4, Dm.INT4_RESIDUAL)


def _say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def dev():
    import torch
    return torch.device("cuda:0")


def _f32_bits(x) -> int:
    return int(np.float32(x).view(np.uint32))


def _f16_bits(x) -> int:
    return int(np.float16(np.float32(x)).view(np.uint16))


def expected_descriptors(caller_tags, tag_map, map_other_tags, pools, D, group):
    """Host restatement: word 0 the native tag a decode uses for the page, words
    4-7 the scale slots of that precision, everything else zero."""
    NP = len(caller_tags)
    out = np.zeros((NP, 8), np.uint32)
    tm = [int(t) if int(t) in NATIVE else Dm.SKIP for t in tag_map]
    for p, c in enumerate(caller_tags):
        c = int(c)
        t = tm[c] if 0 <= c < 8 else (tm[7] if map_other_tags else Dm.SKIP)
        out[p, 0] = t
        out[p, 4:8] = scale_slots(t, p, pools, D, group)
    return out


def scale_slots(t, p, pools, D, group):
    """Words 4-7 of page p's descriptor for native tag t."""
    out = np.zeros(4, np.uint32)
    if t == Dm.FP8:
        out[0], out[1] = _f32_bits(pools["k_fp8_scale"][p]), _f32_bits(pools["v_fp8_scale"][p])
    elif t == Dm.INT8:
        out[0], out[1] = _f32_bits(pools["k_i8_scale"][p]), _f32_bits(pools["v_i8_scale"][p])
    elif t == Dm.INT4_RESIDUAL:
        kr, vr = pools["k_i4r_scale"][p], pools["v_i4r_scale"][p]
        out[:] = [_f32_bits(kr[0]), _f32_bits(kr[1]), _f32_bits(vr[0]), _f32_bits(vr[1])]
    elif t == Dm.INT4:
        # one f16 scale per quarter of head_dim: the group holding dims q * D/4 ..
        for w, base in (("k", 0), ("v", 2)):
            s = pools[f"{w}_i4_scale"][p]
            h = [_f16_bits(s[(q * (D // 4)) // group]) for q in range(4)]
            out[base] = h[0] | (h[1] << 16)
            out[base + 1] = h[2] | (h[3] << 16)
    return out


def expected_records(table, caller_tags, tag_map, map_other_tags, negative_ids, pools, D, group):
    """Host restatement of the entry records of every table entry."""
    NP = len(caller_tags)
    per_page = expected_descriptors(caller_tags, tag_map, map_other_tags, pools, D, group)
    flat = table.reshape(-1)
    out = np.zeros((flat.size, 8), np.uint32)
    for e, raw in enumerate(flat):
        p = int(raw)
        if negative_ids and -NP <= p < 0:
            p += NP
        if 0 <= p < NP:
            out[e] = per_page[p]
            out[e, 1] = p
        else:
            out[e, 0], out[e, 1] = Dm.SKIP, 0xFFFFFFFF
    return out.reshape(*table.shape, 8)


def _case(seed, B, Hq, Hkv, D, NP, W, *, group=32, scale_f32=False, mix=None):
    rng = np.random.default_rng(seed)
    mix = mix or {Dm.FP16: .2, Dm.FP8: .2, Dm.INT8: .2, Dm.INT4: .15, Dm.INT4_RESIDUAL: .15, Dm.SKIP: .1}
    names = list(mix)
    probs = np.array([mix[n] for n in names])
    tags = rng.choice(names, size=NP, p=probs / probs.sum()).astype(np.int32)
    pools = build_pools(rng, NP, D, tags, outliers=0.01, int4_group=group, scale_f32=scale_f32)
    table = rng.integers(0, NP, size=(B, Hkv, W)).astype(np.int32)
    counts = rng.integers(0, W + 1, size=(B, Hkv)).astype(np.int32)
    counts.flat[0] = W
    q = rng.standard_normal((B, Hq, D)).astype(np.float16)
    return q, pools, table, counts, tags


CASES = [
    # seed, B, Hq, Hkv, D, NP, W, int4 group, f32 scales, pages_per_split
    (201, 2, 8, 2, 128, 96, 70, 32, False, 8),
    (202, 3, 4, 4, 64, 64, 45, 64, True, 16),
    (203, 2, 32, 2, 128, 128, 120, 64, False, 0),
    (204, 1, 16, 1, 128, 80, 33, 128, True, 8),
    (205, 4, 32, 8, 128, 300, 200, 32, False, 0),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"seed{c[0]}")
@pytest.mark.parametrize("merge", [False, True], ids=["merge-kernel", "in-kernel"])
def test_descriptor_decode_bit_identical(dev, case, merge):
    import torch
    from intent_attention.decode_core import make_plan
    seed, B, Hq, Hkv, D, NP, W, group, f32, pps = case
    _say("descriptors", f"seed={seed} B={B} Hq={Hq} Hkv={Hkv} D={D} group={group} f32={f32} merge={merge}")
    q, pools, table, counts, tags = _case(seed, B, Hq, Hkv, D, NP, W, group=group, scale_f32=f32)
    t = lambda x: torch.from_numpy(x).to(dev)  # noqa: E731
    dp = to_device_pools(pools, dev, int4_group=group)
    kw = dict(out_dtype=torch.float32, pages_per_split=pps, merge_in_kernel=merge)
    base = make_plan(t(q), dp, t(table), t(counts), t(tags), **kw)
    desc_plan = make_plan(t(q), dp, t(table), t(counts), t(tags), **kw)
    desc = desc_plan.pack_descriptors()
    torch.cuda.synchronize()
    want = expected_descriptors(tags, list(range(8)), False, pools, D, group)
    want[:, 0] = [x if pools_has(dp, x) else Dm.SKIP for x in want[:, 0]]
    got = desc.cpu().numpy().view(np.uint32)
    assert np.array_equal(got, want)
    base.run()
    desc_plan.run()
    torch.cuda.synchronize()
    assert torch.equal(desc_plan.out, base.out)
    ref = Dm.paged_decode_oracle(q.astype(np.float32), pools, table, counts, tags)
    assert float(np.abs(desc_plan.out.cpu().numpy() - ref).max()) <= TOL_QUANT
    # entry records (the plan reads them in place of the descriptors too)
    recs = desc_plan.pack_records()
    torch.cuda.synchronize()
    want_r = expected_records(table, tags, list(range(8)), False, False, pools, D, group)
    assert np.array_equal(recs.cpu().numpy().view(np.uint32), want_r)
    desc_plan.out.fill_(float("nan"))
    desc_plan.run()
    torch.cuda.synchronize()
    assert torch.equal(desc_plan.out, base.out)
    desc_plan.use_records(None)
    # back to the tag and scale arrays
    desc_plan.use_descriptors(None)
    desc_plan.out.fill_(float("nan"))
    desc_plan.run()
    torch.cuda.synchronize()
    assert torch.equal(desc_plan.out, base.out)


def pools_has(dp, tag):
    return dp.has(int(tag))


def test_descriptors_follow_tag_map_and_other_tags(dev):
    """Caller tags through a permuting tag map, with tags outside [0, 8) taking
    tag_map[7]; negative page ids wrap; token bounds cut rows."""
    import torch
    from intent_attention.decode_core import make_plan
    B, Hq, Hkv, D, NP, W = 2, 16, 4, 128, 160, 90
    q, pools, table, counts, native = _case(211, B, Hq, Hkv, D, NP, W)
    # caller tag c maps to tag_map[c]; invert for the pages' native tags
    tag_map = [Dm.INT8, Dm.FP16, Dm.FP8, Dm.SKIP, Dm.INT4_RESIDUAL, Dm.INT4, 9, Dm.FP16]
    inv = {Dm.INT8: [0], Dm.FP16: [1, 7, 12, -3], Dm.FP8: [2], Dm.SKIP: [3, 6],
           Dm.INT4_RESIDUAL: [4], Dm.INT4: [5]}
    rng = np.random.default_rng(5)
    caller = np.array([rng.choice(inv[int(n)]) for n in native], np.int32)
    neg = table.copy()
    flip = rng.random(neg.shape) < 0.3
    neg[flip] -= NP                              # the same pages as negative ids
    valid = np.minimum(counts * 16, rng.integers(0, W * 16 + 1, size=counts.shape)).astype(np.int32)
    t = lambda x: torch.from_numpy(x).to(dev)  # noqa: E731
    dp = to_device_pools(pools, dev)
    kw = dict(tag_map=tag_map, map_other_tags=True, negative_ids=True, valid_tokens=t(valid),
              out_dtype=torch.float32, pages_per_split=8)
    base = make_plan(t(q), dp, t(neg), t(counts), t(caller), **kw)
    dplan = make_plan(t(q), dp, t(neg), t(counts), t(caller), **kw)
    desc = dplan.pack_descriptors()
    torch.cuda.synchronize()
    want = expected_descriptors(caller, tag_map, True, pools, D, 32)
    assert np.array_equal(desc.cpu().numpy().view(np.uint32), want)
    assert np.array_equal(want[:, 0], native.astype(np.uint32))
    base.run()
    dplan.run()
    torch.cuda.synchronize()
    assert torch.equal(dplan.out, base.out)
    ref = Dm.paged_decode_oracle(q.astype(np.float32), pools, table, counts, native, valid_tokens=valid)
    assert float(np.abs(dplan.out.cpu().numpy() - ref).max()) <= TOL_QUANT
    # entry records: negative ids resolved at packing, out-of-range ids past the counts
    neg2 = neg.copy()
    for r in range(B * Hkv):
        b, h = divmod(r, Hkv)
        neg2[b, h, counts[b, h]:] = rng.choice([NP, NP + 5, -NP - 1, 2 ** 31 - 1], size=W - counts[b, h])
    rplan = make_plan(t(q), dp, t(neg2), t(counts), t(caller), **kw)
    recs = rplan.pack_records()
    torch.cuda.synchronize()
    want_r = expected_records(neg2, caller, tag_map, True, True, pools, D, 32)
    assert np.array_equal(recs.cpu().numpy().view(np.uint32), want_r)
    rplan.run()
    torch.cuda.synchronize()
    assert torch.equal(rplan.out, base.out)


def test_descriptor_precision_without_pools_is_skipped(dev):
    """Descriptors packed with every pool, read by a decode that has no INT4
    pools: INT4 pages contribute nothing, as with INT4 mapped to SKIP."""
    import dataclasses

    import torch
    from intent_attention.decode_core import make_plan, pack_page_descriptors
    B, Hq, Hkv, D, NP, W = 2, 8, 2, 128, 96, 60
    q, pools, table, counts, tags = _case(221, B, Hq, Hkv, D, NP, W)
    t = lambda x: torch.from_numpy(x).to(dev)  # noqa: E731
    full = to_device_pools(pools, dev)
    desc = pack_page_descriptors(t(q), full, t(tags))
    no_int4 = dataclasses.replace(full, k_int4=None, v_int4=None, k_int4_scale=None, v_int4_scale=None)
    tm = [Dm.FP16, Dm.INT8, Dm.SKIP, Dm.FP8, Dm.SKIP, Dm.INT4_RESIDUAL, Dm.SKIP, Dm.SKIP]
    want = make_plan(t(q), full, t(table), t(counts), t(tags), tag_map=tm, out_dtype=torch.float32)
    got = make_plan(t(q), no_int4, t(table), t(counts), t(tags), out_dtype=torch.float32, page_descriptors=desc)
    want.run()
    got.run()
    torch.cuda.synchronize()
    assert torch.equal(got.out, want.out)
    # the same with entry records packed on the full pools
    rfull = make_plan(t(q), full, t(table), t(counts), t(tags), out_dtype=torch.float32)
    recs = rfull.pack_records()
    got_r = make_plan(t(q), no_int4, t(table), t(counts), t(tags), out_dtype=torch.float32, entry_records=recs)
    got_r.run()
    torch.cuda.synchronize()
    assert torch.equal(got_r.out, want.out)
    tags_skip = np.where(tags == Dm.INT4, Dm.SKIP, tags).astype(np.int32)
    ref = Dm.paged_decode_oracle(q.astype(np.float32), pools, table, counts, tags_skip)
    assert float(np.abs(got.out.cpu().numpy() - ref).max()) <= TOL_QUANT


def test_records_plan_graph_replays(dev):
    """A plan reading entry records, captured in a HIP graph (in-kernel merge):
    three replays, with eager work between them, equal the eager call."""
    import torch
    from intent_attention.decode_core import make_plan
    q, pools, table, counts, tags = _case(231, 2, 16, 4, 128, 128, 90)
    t = lambda x: torch.from_numpy(x).to(dev)  # noqa: E731
    dp = to_device_pools(pools, dev)
    plan = make_plan(t(q), dp, t(table), t(counts), t(tags), out_dtype=torch.float32, pages_per_split=8,
                     merge_in_kernel=True)
    plan.pack_records()
    plan.run()
    torch.cuda.synchronize()
    want = plan.out.clone()
    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            plan.run()
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize()
    for i in range(3):
        plan.out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(plan.out, want), i
