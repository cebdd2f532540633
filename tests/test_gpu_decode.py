"""GPU parity of the HIP selected-page decode against the CPU oracle.

Every case calls libiak through the C ABI (``intent_attention.paged_decode``
and the two reference-shaped APIs) and compares with
``oracle.decode.paged_decode_oracle`` (float64 attention over the
reference's dequantised values) on the same seeded inputs:
max-abs <= 2e-3 when only FP16 pages are visited, <= 1e-2 with quantised pages.
The fused API is also checked against the reference's own output
(tests/golden/g3_fused_decode.npz).
"""
import os
import sys

import numpy as np
import pytest

from oracle import decode as Dm
from tests._pools import random_case, to_device_pools

pytestmark = pytest.mark.gpu

TOL_FP16 = 2e-3
TOL_QUANT = 1e-2


def _say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def dev():
    import torch
    return torch.device("cuda:0")


def _run(dev, q, pools_np, table, counts, tags, **kw):
    import torch
    from intent_attention import paged_decode
    pools = to_device_pools(pools_np, dev)
    qt = torch.from_numpy(q).to(dev)
    out = paged_decode(qt, pools, torch.from_numpy(table).to(dev), torch.from_numpy(counts).to(dev),
                       torch.from_numpy(tags).to(dev), **kw)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


CASES = [
    # name, seed, B, Hq, Hkv, D, NP, W, mix
    ("fp16_gqa4_d128", 11, 2, 8, 2, 128, 48, 40, {"FP16": 1}),
    ("fp16_mha_d64", 12, 2, 4, 4, 64, 32, 20, {"FP16": 1}),
    ("int8_gqa4_d128", 13, 2, 8, 2, 128, 48, 40, {"INT8": 1}),
    ("fp8_gqa4_d128", 14, 2, 8, 2, 128, 48, 40, {"FP8": 1}),
    ("int4_gqa4_d128", 15, 2, 8, 2, 128, 48, 40, {"INT4": 1}),
    ("int4r_gqa4_d128", 16, 2, 8, 2, 128, 48, 40, {"INT4_RESIDUAL": 1}),
    ("mixed_gqa4_d128", 17, 3, 8, 2, 128, 96, 70,
     {"FP16": .25, "FP8": .2, "INT8": .25, "INT4": .15, "INT4_RESIDUAL": .1, "SKIP": .05}),
    ("mixed_mha_d64", 18, 2, 4, 4, 64, 64, 50,
     {"FP16": .3, "FP8": .2, "INT8": .2, "INT4": .2, "INT4_RESIDUAL": .1}),
    ("mixed_gqa8_d128", 19, 2, 16, 2, 128, 64, 33, {"FP16": .5, "INT8": .3, "INT4": .2}),
    ("mixed_gqa16_d64", 20, 1, 16, 1, 64, 64, 64, {"FP16": .4, "FP8": .3, "INT4": .3}),
]


@pytest.mark.parametrize("name,seed,B,Hq,Hkv,D,NP,W,mix", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("pps", [0, 16, 64])
def test_paged_decode_matches_oracle(dev, name, seed, B, Hq, Hkv, D, NP, W, mix, pps):
    _say(name, f"seed={seed} B={B} Hq={Hq} Hkv={Hkv} D={D} NP={NP} W={W} pages_per_split={pps}")
    q, pools, table, counts, tags = random_case(seed, B, Hq, Hkv, D, NP, W, mix, outliers=0.01)
    got = _run(dev, q, pools, table, counts, tags, pages_per_split=pps)
    ref = Dm.paged_decode_oracle(q, pools, table, counts, tags)
    tol = TOL_FP16 if set(mix) == {"FP16"} else TOL_QUANT
    err = np.abs(got - ref).max()
    assert err <= tol, f"{name}: max abs err {err:.3e} > {tol}"
    # rows that visit no page are exactly zero
    for b in range(B):
        for hk in range(Hkv):
            if counts[b, hk] == 0:
                G = Hq // Hkv
                assert np.all(got[b, hk * G:(hk + 1) * G] == 0)


@pytest.mark.parametrize("pps", [0, 4, 7])
def test_class_ring_boundaries(dev, pps):
    """Rows in which every precision class has 0 .. 7 pages (around each class
    loop's ring depth of 2, 3 or 5), shuffled together: the ring loads past a
    class's end read a shared pad page and must contribute nothing."""
    from tests._pools import build_pools
    _say("ring boundaries", f"pages_per_split={pps}")
    rng = np.random.default_rng(4242 + pps)
    names = ["FP16", "FP8", "INT8", "INT4", "INT4_RESIDUAL"]
    per = 8                                     # physical pages per class
    tags = np.repeat(np.array([Dm.FP16, Dm.FP8, Dm.INT8, Dm.INT4, Dm.INT4_RESIDUAL], np.int32), per)
    NP, D, B, Hq, Hkv = len(tags), 128, 2, 8, 4
    pools = build_pools(rng, NP, D, tags, outliers=0.01)
    rows = []
    for r in range(B * Hkv):
        ids = [k * per + int(x) for k in range(len(names)) for x in rng.integers(0, per, size=(r + 3 * k) % 8)]
        rng.shuffle(ids)
        rows.append(ids)
    W = max(len(x) for x in rows)
    table = np.zeros((B, Hkv, W), np.int32)
    counts = np.zeros((B, Hkv), np.int32)
    for r, ids in enumerate(rows):
        table.flat[r * W: r * W + len(ids)] = ids
        counts.flat[r] = len(ids)
    q = rng.standard_normal((B, Hq, D)).astype(np.float16)
    got = _run(dev, q, pools, table, counts, tags, pages_per_split=pps)
    ref = Dm.paged_decode_oracle(q, pools, table, counts, tags)
    err = float(np.abs(got - ref).max())
    assert err <= TOL_QUANT, f"max abs err {err:.3e}"


@pytest.mark.parametrize("W", [448, 1000])
def test_many_rows(dev, W):
    """256 (batch, kv head) rows with ragged counts: the automatic plan (64-entry
    splits, partials merged per row) against the oracle on rows sampled from
    the batch and, for the whole output, against a uniform 16-entry plan."""
    _say("many rows", f"W={W}")
    B, Hq, Hkv, D = 32, 32, 8, 128
    q, pools, table, counts, tags = random_case(
        51 + W, B, Hq, Hkv, D, 2048, W,
        {"FP16": .25, "FP8": .25, "INT8": .3, "INT4": .15, "INT4_RESIDUAL": .05}, outliers=0.01,
        q_scale=1 / np.sqrt(D))
    counts[1] = W                    # full rows next to the random counts
    got = _run(dev, q, pools, table, counts, tags)
    uni = _run(dev, q, pools, table, counts, tags, pages_per_split=16)
    assert np.abs(got - uni).max() <= 1e-3
    for b in (0, 1, 17, 31):
        ref = Dm.paged_decode_oracle(q[b:b + 1], pools, table[b:b + 1], counts[b:b + 1], tags)
        err = np.abs(got[b:b + 1] - ref).max()
        assert err <= TOL_QUANT, f"batch {b}: max abs err {err:.3e}"


@pytest.mark.parametrize("qdt,odt", [("f32", "f32"), ("f16", "f32"), ("f32", "f16"), ("bf16", "bf16")])
def test_q_and_out_dtypes(dev, qdt, odt):
    import torch
    _say("dtypes", qdt, odt)
    q, pools, table, counts, tags = random_case(31, 2, 8, 2, 128, 40, 30,
                                                {"FP16": .5, "INT8": .3, "FP8": .2})
    q32 = np.random.default_rng(5).standard_normal(q.shape).astype(np.float32)
    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
    qt = torch.from_numpy(q32).to(tdt[qdt])
    qref = qt.float().numpy()
    from intent_attention import paged_decode
    out = paged_decode(qt.to(dev), to_device_pools(pools, dev), torch.from_numpy(table).to(dev),
                       torch.from_numpy(counts).to(dev), torch.from_numpy(tags).to(dev), out_dtype=tdt[odt])
    assert out.dtype == tdt[odt]
    ref = Dm.paged_decode_oracle(qref, pools, table, counts, tags)
    tol = TOL_QUANT + (1e-2 if odt == "bf16" else 0)
    assert np.abs(out.float().cpu().numpy() - ref).max() <= tol


@pytest.mark.parametrize("pps", [0, 16])
def test_large_value_magnitudes(dev, pps):
    """V values N(0, 9000^2) (|v| up to ~4e4, inside float16): p (up to 2^8
    between lazy rescales) times such a V page scale (~300) would overflow
    float16; the kernel's value exponent keeps the P operand in range. The
    output matches the oracle to the same relative bar as unit-scale values,
    with no inf or nan; K stays unit-scale, with outliers to move the running
    max."""
    vs = 9000.0
    _say("large V magnitudes", f"v_scale={vs} pages_per_split={pps}")
    q, pools, table, counts, tags = random_case(
        61, 2, 8, 2, 128, 64, 48, {"FP16": .2, "FP8": .2, "INT8": .3, "INT4_RESIDUAL": .3},
        outliers=0.02, v_scale=vs)
    got = _run(dev, q, pools, table, counts, tags, pages_per_split=pps)
    assert np.all(np.isfinite(got))
    ref = Dm.paged_decode_oracle(q, pools, table, counts, tags)
    err = np.abs(got - ref).max() / vs
    assert err <= TOL_QUANT, f"max abs err / v_scale {err:.3e}"


SMALL_V_MIXES = {"fp8": {"FP8": 1}, "int8": {"INT8": 1}, "int4r": {"INT4_RESIDUAL": 1},
                 "mixed": {"FP16": .2, "FP8": .2, "INT8": .2, "INT4": .2, "INT4_RESIDUAL": .2}}


def _row_rel_err(got, ref):
    """Worst over (batch, head) rows of max|got - ref| / max|ref| in the row."""
    d = np.abs(got - ref).max(axis=-1)
    m = np.abs(ref).max(axis=-1)
    live = m > 0
    assert np.all(d[~live] == 0)
    return float((d[live] / m[live]).max())


@pytest.mark.parametrize("vs", [1e-3, 3e-4])
@pytest.mark.parametrize("mix", list(SMALL_V_MIXES))
@pytest.mark.parametrize("pps", [0, 7])
def test_small_value_magnitudes(dev, vs, mix, pps):
    """V values N(0, vs^2): the V page scales (absmax / 127, ~1e-5) would put
    p * scale in the float16 subnormals; the kernel's value exponent keeps the
    P operand normal. Relative bar 2e-3 per row (the output is ~vs)."""
    _say("small V magnitudes", f"v_scale={vs} mix={mix} pages_per_split={pps}")
    q, pools, table, counts, tags = random_case(
        81 + pps, 2, 8, 2, 128, 64, 48, SMALL_V_MIXES[mix], outliers=0.01, v_scale=vs)
    got = _run(dev, q, pools, table, counts, tags, pages_per_split=pps, out_dtype=__import__("torch").float32)
    ref = Dm.paged_decode_oracle(q, pools, table, counts, tags)
    err = _row_rel_err(got, ref)
    _say(f"  worst row relative error {err:.2e}")
    assert err <= 2e-3, f"relative err {err:.3e}"


@pytest.mark.parametrize("pps", [0, 5])
def test_value_scales_spanning_binades(dev, pps):
    """Every page's V drawn at its own magnitude, 10^U(-4, 2.5) (binades -14 ..
    8), so a split's value exponent moves up and down between pages; every
    precision. Relative bar 2e-3 per row."""
    from tests._pools import build_pools
    _say("V scales spanning binades", f"pages_per_split={pps}")
    rng = np.random.default_rng(91 + pps)
    NP, D, B, Hq, Hkv, W = 80, 128, 2, 8, 2, 60
    names = [Dm.FP16, Dm.FP8, Dm.INT8, Dm.INT4, Dm.INT4_RESIDUAL]
    tags = np.array([names[i % 5] for i in range(NP)], np.int32)
    pools = build_pools(rng, NP, D, tags, outliers=0.01, v_scale=10.0 ** rng.uniform(-4, 2.5, NP))
    table = rng.integers(0, NP, size=(B, Hkv, W)).astype(np.int32)
    counts = np.full((B, Hkv), W, np.int32)
    q = rng.standard_normal((B, Hq, D)).astype(np.float16)
    got = _run(dev, q, pools, table, counts, tags, pages_per_split=pps, out_dtype=__import__("torch").float32)
    ref = Dm.paged_decode_oracle(q, pools, table, counts, tags)
    assert np.all(np.isfinite(got))
    err = _row_rel_err(got, ref)
    _say(f"  worst row relative error {err:.2e}")
    assert err <= 2e-3, f"relative err {err:.3e}"


@pytest.mark.parametrize("mix", ["FP16", "FP8", "INT8", "INT4", "INT4_RESIDUAL", "all"])
@pytest.mark.parametrize("pps", [0, 5])
def test_valid_tokens_ragged_rows(dev, mix, pps):
    """A per-row token bound: tokens of table entry e at or past
    valid_tokens - 16 e are left out (a ragged last page), entries wholly past
    it contribute nothing; every precision class (INT4 pages hold tokens in
    direct order in the score layout, the others permuted), bounds 0 ..
    16 * count + 5."""
    import torch
    from intent_attention import paged_decode
    _say("valid_tokens", f"mix={mix} pages_per_split={pps}")
    m = ({"FP16": .2, "FP8": .2, "INT8": .2, "INT4": .2, "INT4_RESIDUAL": .2} if mix == "all" else {mix: 1})
    B, Hq, Hkv, D, NP, W = 3, 8, 4, 128, 40, 23
    q, pools, table, counts, tags = random_case(300 + pps + len(mix), B, Hq, Hkv, D, NP, W, m, outliers=0.01)
    rng = np.random.default_rng(5 + pps)
    bound = (rng.integers(0, 16 * counts + 6)).astype(np.int32)
    bound.flat[1] = 0
    bound.flat[2] = 16 * int(counts.flat[2])          # exactly at a page boundary
    bound.flat[3] = 16 * int(counts.flat[3]) - 15     # one token of the last page
    got = _run(dev, q, pools, table, counts, tags, pages_per_split=pps, out_dtype=torch.float32,
               valid_tokens=torch.from_numpy(bound).to(dev))
    ref = Dm.paged_decode_oracle(q, pools, table, counts, tags, valid_tokens=bound)
    err = float(np.abs(got - ref).max())
    assert err <= (TOL_FP16 if mix == "FP16" else TOL_QUANT), f"max abs err {err:.3e}"
    G = Hq // Hkv
    assert np.all(got.reshape(B, Hkv, G, D)[np.unravel_index(1, (B, Hkv))] == 0)


def test_misaligned_query_view(dev):
    """A query view 2 bytes past an aligned address (the kernel reads 16-byte
    query vectors) is copied to an aligned buffer by the host layer; the
    result equals the aligned query's."""
    import torch
    from intent_attention import paged_decode
    _say("misaligned q view")
    q, pools, table, counts, tags = random_case(71, 2, 8, 2, 128, 40, 30, {"FP16": .5, "INT8": .5})
    dp = to_device_pools(pools, dev)
    tt, ct, gt = (torch.from_numpy(x).to(dev) for x in (table, counts, tags))
    base = torch.from_numpy(q).to(dev)
    buf = torch.zeros(q.size + 8, dtype=torch.float16, device=dev)
    view = buf[1:1 + q.size].view(q.shape)
    view.copy_(base)
    assert view.data_ptr() % 16 != 0
    want = paged_decode(base, dp, tt, ct, gt)
    got = paged_decode(view, dp, tt, ct, gt)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_invalid_ids_and_clamped_counts(dev):
    import torch
    _say("invalid ids / clamped counts")
    q, pools, table, counts, tags = random_case(41, 2, 4, 2, 64, 32, 12, {"FP16": .6, "INT8": .4})
    table[0, 0, 3] = -1        # negative: invalid in this mode
    table[0, 1, 5] = 32        # past the pool: invalid
    table[1, 0, 0] = -33       # below -NP: invalid even with wrap
    counts[1, 1] = 99          # clamped to the width
    got = _run(dev, q, pools, table, counts, tags)
    ref = Dm.paged_decode_oracle(q, pools, table, counts, tags)
    assert np.abs(got - ref).max() <= TOL_QUANT
    table[0, 0, 4] = -2        # wraps to page 30 with negative_ids
    got = _run(dev, q, pools, table, counts, tags, negative_ids=True)
    ref = Dm.paged_decode_oracle(q, pools, table, counts, tags, neg_ids_wrap=True)
    assert np.abs(got - ref).max() <= TOL_QUANT


def test_selection_is_exact(dev):
    """q = 0 gives a uniform softmax, so the output is the mean of the visited
    pages' V rows; with V[page p] = e_p the visited multiset is recovered."""
    import torch
    _say("selection exactness probe")
    D, NP, W = 64, 64, 40
    rng = np.random.default_rng(3)
    tags = np.zeros(NP, np.int32)
    tags[rng.choice(NP, 10, replace=False)] = Dm.SKIP
    pools = {"k_fp16": rng.standard_normal((NP, 16, D)).astype(np.float16),
             "v_fp16": np.zeros((NP, 16, D), np.float16)}
    for p in range(NP):
        pools["v_fp16"][p, :, p] = 1.0
    from intent_attention import PagePools, paged_decode
    pp = PagePools(k_fp16=torch.from_numpy(pools["k_fp16"]).to(dev), v_fp16=torch.from_numpy(pools["v_fp16"]).to(dev))
    table = rng.integers(0, NP, size=(3, 2, W)).astype(np.int32)
    counts = np.array([[40, 17], [1, 0], [33, 40]], np.int32)
    q = np.zeros((3, 2, D), np.float16)
    out = paged_decode(torch.from_numpy(q).to(dev), pp, torch.from_numpy(table).to(dev),
                       torch.from_numpy(counts).to(dev), torch.from_numpy(tags).to(dev),
                       out_dtype=torch.float32).cpu().numpy()
    for b in range(3):
        for h in range(2):
            vis = [p for p in table[b, h, :counts[b, h]] if tags[p] != Dm.SKIP]
            exp = np.zeros(D)
            for p in vis:
                exp[p] += 1.0 / len(vis)
            assert np.abs(out[b, h] - exp).max() < 1e-3, (b, h)


@pytest.fixture(scope="module")
def g3(golden_dir):
    return dict(np.load(os.path.join(golden_dir, "g3_fused_decode.npz")))


@pytest.mark.parametrize("variant", ["fused_fp16_scales", "triton_fp32_scales"])
def test_fused_api_matches_reference_golden(dev, g3, variant):
    """fused_selected_quant_decode on the GPU vs the reference's own CPU output."""
    import torch
    from intent_attention import FusedDecodeConfig, fused_selected_quant_decode
    _say("fused API vs golden", variant)
    pre = "t" if variant.startswith("triton") else ""
    t = lambda k: torch.from_numpy(g3[k]).to(dev)  # noqa: E731
    cfg = FusedDecodeConfig(page_size=16, head_dim=64, max_selected_pages=g3["page_table"].shape[2])
    out = fused_selected_quant_decode(t("q"), t("k16"), t("v16"), t(f"{pre}k8"), t(f"{pre}v8"), t(f"{pre}ks"),
                                      t(f"{pre}vs"), t("page_table"), t("page_precision"), t("page_counts"), cfg)
    assert out.shape == (2, 4, 1, 64) and out.dtype == torch.float16 and out.is_cuda
    ref = g3["out_triton_scales" if pre else "out"].astype(np.float32)
    assert np.abs(out.float().cpu().numpy() - ref).max() <= TOL_FP16
    # the reference's correctness entry point, same arguments, same device result
    from intent_attention import fused_selected_quant_decode_reference
    out_r = fused_selected_quant_decode_reference(t("q"), t("k16"), t("v16"), t(f"{pre}k8"), t(f"{pre}v8"),
                                                  t(f"{pre}ks"), t(f"{pre}vs"), t("page_table"), t("page_precision"),
                                                  t("page_counts"), cfg)
    assert torch.equal(out_r, out)


def test_fused_api_reference_test_facts(dev):
    """test_fused_selected_quant_decode.py facts on the GPU: all-SKIP -> 0, zero pages -> 0,
    FP16 path == dense attention over the gathered pages."""
    import torch
    from intent_attention import FusedDecodeConfig, FusedKVPrecision, fake_int8_pages_from_fp16
    from intent_attention import fused_selected_quant_decode
    from intent_attention.fused_selected_quant_decode import fake_int8_pages_from_fp16 as fused_fake_int8
    _say("fused API reference facts")
    g = torch.Generator().manual_seed(0)
    B, H, D, PS, NP, W = 2, 4, 64, 16, 8, 4
    k16 = torch.randn(NP, PS, D, generator=g).half()
    v16 = torch.randn(NP, PS, D, generator=g).half()
    k8, ks = fused_fake_int8(k16)
    v8, vs = fused_fake_int8(v16)
    q = torch.randn(B, H, 1, D, generator=g).half()
    pt = torch.arange(W, dtype=torch.int32).repeat(B, H, 1)
    pc = torch.full((B, H), W, dtype=torch.int32)
    prec = torch.full((NP,), int(FusedKVPrecision.FP16), dtype=torch.int32)
    cfg = FusedDecodeConfig(page_size=PS, head_dim=D, max_selected_pages=W)
    args = [x.to(dev) for x in (q, k16, v16, k8, v8, ks, vs, pt, prec, pc)]
    out = fused_selected_quant_decode(*args, cfg).float().cpu()
    kk = k16[:W].reshape(-1, D).float()
    vv = v16[:W].reshape(-1, D).float()
    dense = torch.softmax(q[:, :, 0].float() @ kk.T / D ** 0.5, -1) @ vv
    assert (out[:, :, 0] - dense).abs().max() < 1e-2
    skip = torch.full((NP,), int(FusedKVPrecision.SKIP), dtype=torch.int32).to(dev)
    assert fused_selected_quant_decode(*args[:8], skip, args[9], cfg).abs().max().item() < 1e-6
    zero = torch.zeros(B, H, dtype=torch.int32).to(dev)
    assert fused_selected_quant_decode(*args[:9], zero, cfg).abs().max().item() < 1e-6
    with pytest.raises(ValueError, match="head_dim"):
        fused_selected_quant_decode(*args, FusedDecodeConfig(head_dim=128))
    del fake_int8_pages_from_fp16


def test_fused_api_reference_precision_cases(dev):
    """The per-precision and per-count cases of test_fused_selected_quant_decode.py
    (:158-255) on the GPU, each compared with the oracle's restatement of the
    reference loop (fused_selected_quant_decode.py:267-336): all INT8; FP16 and
    INT8 halves; FP16 with page 1 INT8 and page 2 SKIP; one page per row; and
    counts of 1, 2 and 3 across the rows. The reference's tests assert only the
    shape; these also hold the values to the loop."""
    import torch
    from intent_attention import FusedDecodeConfig, FusedKVPrecision
    from intent_attention.fused_selected_quant_decode import (fake_int8_pages_from_fp16,
                                                              fused_selected_quant_decode_reference)
    g = torch.Generator().manual_seed(1)
    B, H, D, PS, NP, W = 2, 4, 64, 16, 8, 4
    k16 = torch.randn(NP, PS, D, generator=g).half()
    v16 = torch.randn(NP, PS, D, generator=g).half()
    k8, ks = fake_int8_pages_from_fp16(k16)
    v8, vs = fake_int8_pages_from_fp16(v16)
    q = torch.randn(B, H, 1, D, generator=g).half()
    pt = torch.arange(W, dtype=torch.int32).repeat(B, H, 1)
    full = torch.full((B, H), W, dtype=torch.int32)
    cfg = FusedDecodeConfig(page_size=PS, head_dim=D, max_selected_pages=W)
    fp16, int8, skip = int(FusedKVPrecision.FP16), int(FusedKVPrecision.INT8), int(FusedKVPrecision.SKIP)

    def prec(*pairs, default=fp16):
        p = torch.full((NP,), default, dtype=torch.int32)
        for idx, tag in pairs:
            p[idx] = tag
        return p

    uneven = torch.full((B, H), 2, dtype=torch.int32)
    uneven[0, 0], uneven[B - 1, H - 1] = 1, 3
    cases = {"int8": (prec(default=int8), full),
             "mixed": (prec((slice(NP // 2, None), int8)), full),
             "mixed_with_skip": (prec((1, int8), (2, skip)), full),
             "single_page": (prec(), torch.ones(B, H, dtype=torch.int32)),
             "uneven_counts": (prec((1, int8)), uneven)}
    for name, (p, pc) in cases.items():
        _say("fused reference case", name)
        args = [x.to(dev) for x in (q, k16, v16, k8, v8, ks, vs, pt, p, pc)]
        out = fused_selected_quant_decode_reference(*args, cfg)
        assert out.shape == (B, H, 1, D) and out.dtype == torch.float16 and out.is_cuda
        ref = Dm.fused_decode_reference_loop(q.numpy(), k16.numpy(), v16.numpy(), k8.numpy(), v8.numpy(),
                                             ks.float().numpy(), vs.float().numpy(), pt.numpy(), p.numpy(),
                                             pc.numpy(), D)
        err = np.abs(out.float().cpu().numpy() - ref.astype(np.float32)).max()
        tol = TOL_FP16 if bool((p[:W] == fp16).all()) else TOL_QUANT
        assert err <= tol, (name, err)


def test_sibling_api_triton_numbering(dev):
    """intent_quant_decode_attention_triton: tag 0 FP16; 5 or an id < 0 invalid;
    every other tag -- 1-4, 6, 7, negative, 8 and above -- reads the INT8 pool
    (triton_intent_quant_attention.py:281-307)."""
    import torch
    from intent_attention import (IntentQuantKernelConfig, TritonKVPrecision, intent_quant_decode_attention_triton,
                                  make_page_tables_from_selected_pages)
    _say("sibling API")
    rng = np.random.default_rng(9)
    B, H, D, NP = 2, 4, 64, 12
    q, pools, table, counts, tags = random_case(51, B, H, H, D, NP, 8, {"FP16": .5, "INT8": .5}, scale_f32=True)
    ttags = np.where(tags == Dm.FP16, 0, rng.choice([1, 2, 3, 4, 6, 7, -3, 9, 1 << 20], size=NP)).astype(np.int32)
    ttags[0] = int(TritonKVPrecision.SKIP)
    sel = torch.tensor([0, 3, 5, 7, 2, 11, 1, 4, 6, 8], dtype=torch.int32)
    quant_sel = [p for p in sel.tolist()[1:] if tags[p] != Dm.FP16]
    assert len(quant_sel) >= 3
    for p, t in zip(quant_sel, (6, -3, 1 << 20, 7, 9)):
        ttags[p] = t                           # tags outside the numbering on selected pages
    ids, cnt = make_page_tables_from_selected_pages(sel, B, H, max_selected_pages=12)
    cfg = IntentQuantKernelConfig(page_size=16, head_dim=D, max_selected_pages=12)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)  # noqa: E731
    out = intent_quant_decode_attention_triton(
        t(q), t(pools["k_fp16"]), t(pools["v_fp16"]), t(pools["k_i8"]), t(pools["v_i8"]),
        t(pools["k_i8_scale"]), t(pools["v_i8_scale"]), ids.to(dev), cnt.to(dev), t(ttags), config=cfg)
    assert out.dtype == torch.float16 and out.shape == (B, H, D)
    native = np.where(ttags == 0, Dm.FP16, np.where(ttags == 5, Dm.SKIP, Dm.INT8)).astype(np.int32)
    ref = Dm.paged_decode_oracle(q, pools, ids.numpy(), cnt.numpy(), native)
    assert np.abs(out.float().cpu().numpy() - ref).max() <= TOL_QUANT
