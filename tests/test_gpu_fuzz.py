"""Seeded randomized GPU parity sweeps: shapes, GQA groups, precision mixes,
split lengths, query / output dtypes, ragged counts, invalid ids and token
bounds drawn at random (fixed seeds, so every run checks the same cases)
against the CPU oracle. Each case is small enough for the oracle to finish in
well under a second. Bars as in the targeted tests: max-abs <= 2e-3 when only
FP16 pages are visited, <= 1e-2 with quantised pages, plus the rounding of a
float16 / bfloat16 output (2^-11 / 2^-8 of the output's magnitude); page
tables exact."""
import sys

import numpy as np
import pytest

from oracle import decode as Dm
from oracle import mla as M
from oracle import policy as P
from tests._pools import random_case, to_device_pools

pytestmark = pytest.mark.gpu

PRECISIONS = ["FP16", "FP8", "INT8", "INT4", "INT4_RESIDUAL", "SKIP"]


def _say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def dev():
    import torch
    return torch.device("cuda:0")


def _decode_case(seed):
    rng = np.random.default_rng(1000 + seed)
    D = int(rng.choice([64, 128]))
    Hkv = int(rng.integers(1, 5))
    G = int(rng.choice([1, 2, 3, 4, 5, 8, 16]))
    B = int(rng.integers(1, 4))
    NP = int(rng.integers(8, 120))
    W = int(rng.integers(1, 150))
    names = list(rng.choice(PRECISIONS, size=int(rng.integers(1, 5)), replace=False))
    mix = {n: float(rng.random() + 0.1) for n in names}
    pps = int(rng.choice([0, 1, 3, 16, 37, 64]))
    qdt = str(rng.choice(["f16", "f32", "bf16"]))
    odt = str(rng.choice(["f16", "f32", "bf16"]))
    q_scale = float(rng.choice([1.0, 1 / np.sqrt(D), 3.0]))
    neg = bool(rng.random() < 0.3)
    return dict(seed=seed, B=B, Hq=G * Hkv, Hkv=Hkv, D=D, NP=NP, W=W, mix=mix, pps=pps, qdt=qdt, odt=odt,
                q_scale=q_scale, neg=neg)


@pytest.mark.parametrize("seed", range(96))
def test_decode_random_configs(dev, seed):
    import torch
    from intent_attention import paged_decode
    c = _decode_case(seed)
    _say("fuzz decode", c)
    q, pools, table, counts, tags = random_case(2000 + seed, c["B"], c["Hq"], c["Hkv"], c["D"], c["NP"], c["W"],
                                                c["mix"], outliers=0.01, q_scale=c["q_scale"])
    rng = np.random.default_rng(3000 + seed)
    # invalid ids (negative, past the pool) and counts past the width
    bad = rng.random(table.shape) < 0.05
    table[bad] = rng.choice([-1, -c["NP"], c["NP"], c["NP"] + 7, -c["NP"] - 1], size=int(bad.sum()))
    if rng.random() < 0.5:
        counts.flat[-1] = c["W"] + 5
    tdt = {"f16": torch.float16, "f32": torch.float32, "bf16": torch.bfloat16}
    qt = torch.from_numpy(q.astype(np.float32)).to(tdt[c["qdt"]])
    qref = qt.float().numpy()
    out = paged_decode(qt.to(dev), to_device_pools(pools, dev), torch.from_numpy(table).to(dev),
                       torch.from_numpy(counts).to(dev), torch.from_numpy(tags).to(dev),
                       negative_ids=c["neg"], out_dtype=tdt[c["odt"]], pages_per_split=c["pps"])
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    ref = Dm.paged_decode_oracle(qref, pools, table, counts, tags, neg_ids_wrap=c["neg"])
    quant = any(n not in ("FP16", "SKIP") for n in c["mix"])
    # the bar of the precisions visited, plus the rounding of the output dtype
    amax = max(1.0, float(np.abs(ref).max()))
    tol = (1e-2 if quant else 2e-3) + {"f32": 0.0, "f16": 2.0 ** -11, "bf16": 2.0 ** -8}[c["odt"]] * amax
    assert np.all(np.isfinite(got))
    err = float(np.abs(got - ref).max())
    assert err <= tol, f"case {c}: max abs err {err:.3e} > {tol:.3e}"


def _latent_case(rng, B, H, DQK, NP, W, mix):
    code = {"FP16": Dm.FP16, "FP8": Dm.FP8, "INT8": Dm.INT8, "SKIP": Dm.SKIP}
    names = list(mix)
    probs = np.array([mix[n] for n in names], float)
    tags = np.array([code[n] for n in rng.choice(names, size=NP, p=probs / probs.sum())], np.int32)
    lat = rng.standard_normal((NP, 16, DQK)).astype(np.float16)
    sdt = np.float16 if rng.random() < 0.5 else np.float32
    pools = {"c_fp16": lat, "c_fp8": np.zeros((NP, 16, DQK), np.uint8), "c_fp8_scale": np.zeros(NP, sdt),
             "c_i8": np.zeros((NP, 16, DQK), np.int8), "c_i8_scale": np.zeros(NP, sdt)}
    from oracle import quant as Q
    for p in range(NP):
        if tags[p] == Dm.FP8:
            cc, s = Q.quantize_page(lat[p], "FP8")
            pools["c_fp8"][p], pools["c_fp8_scale"][p] = cc, s[0]
        elif tags[p] == Dm.INT8:
            cc, s = Q.quantize_page(lat[p], "INT8")
            pools["c_i8"][p], pools["c_i8_scale"][p] = cc, s[0]
    table = rng.integers(0, NP, size=(B, W)).astype(np.int32)
    counts = rng.integers(0, W + 1, size=B).astype(np.int32)
    q = rng.standard_normal((B, H, DQK)).astype(np.float16)
    return q, pools, table, counts, tags


MLA_SHAPES = [(64, 64, 0), (128, 128, 0), (256, 256, 0), (512, 512, 0), (576, 512, 0), (576, 64, 512)]


@pytest.mark.parametrize("seed", range(40))
def test_mla_random_configs(dev, seed):
    import torch
    from intent_attention import LatentPools, mla_paged_decode
    rng = np.random.default_rng(5000 + seed)
    dqk, dv, voff = MLA_SHAPES[int(rng.integers(0, len(MLA_SHAPES)))]
    B, H = int(rng.integers(1, 4)), int(rng.choice([1, 16, 70, 128, 130, 256]))
    NP, W = int(rng.integers(4, 60)), int(rng.integers(1, 200))
    names = list(rng.choice(["FP16", "FP8", "INT8", "SKIP"], size=int(rng.integers(1, 4)), replace=False))
    mix = {n: float(rng.random() + 0.1) for n in names}
    pps = int(rng.choice([0, 1, 5, 16, 64, 100, 128]))   # past 64: two entries per lane
    c = dict(seed=seed, dqk=dqk, dv=dv, voff=voff, B=B, H=H, NP=NP, W=W, mix=mix, pps=pps)
    _say("fuzz mla", c)
    q, pools, table, counts, tags = _latent_case(rng, B, H, dqk, NP, W, mix)
    valid = np.maximum(counts * 16 - rng.integers(0, 16, size=B), 0).astype(np.int32)
    t = {k: torch.from_numpy(v).to(dev) for k, v in pools.items()}
    lp = LatentPools(c_fp16=t["c_fp16"], c_fp8=t["c_fp8"], c_fp8_scale=t["c_fp8_scale"], c_int8=t["c_i8"],
                     c_int8_scale=t["c_i8_scale"])
    got = mla_paged_decode(torch.from_numpy(q).to(dev), lp, torch.from_numpy(table).to(dev),
                           torch.from_numpy(counts).to(dev), torch.from_numpy(tags).to(dev), v_dim=dv,
                           v_offset=voff, valid_tokens=torch.from_numpy(valid).to(dev), pages_per_split=pps,
                           out_dtype=torch.float32)
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    ref = M.mla_paged_decode_oracle(q, pools, table, counts, tags, v_dim=dv, v_offset=voff, valid_tokens=valid)
    assert np.all(np.isfinite(got))
    quant = any(n in ("FP8", "INT8") for n in mix)
    err = float(np.abs(got - ref).max())
    assert err <= (1e-2 if quant else 2e-3), f"case {c}: max abs err {err:.3e}"


@pytest.mark.parametrize("seed", range(48))
def test_page_tables_random_configs(dev, seed):
    import torch
    from intent_attention import build_page_tables
    rng = np.random.default_rng(7000 + seed)
    ps = int(rng.choice([1, 4, 16, 64]))
    n_seq = int(rng.integers(1, 5))
    rows_per_seq = int(rng.integers(1, 5))
    per_seq_lists = bool(rng.random() < 0.6)
    R = n_seq * rows_per_seq
    rows_per_list = rows_per_seq if per_seq_lists else R
    n_lists = (R + rows_per_list - 1) // rows_per_list
    L = int(rng.integers(1, 400))              # logical pages per sequence
    lists = []
    for _ in range(n_lists):
        n = int(rng.integers(0, 80))
        s = rng.integers(-20, L * ps, size=n)
        e = s + rng.integers(-5, 40 * ps, size=n)
        tg = rng.integers(0, 6, size=n)
        lists.append([(int(a), int(b), int(cc)) for a, b, cc in zip(s, e, tg)])
    use_bt = bool(rng.random() < 0.7)
    NP = int(rng.integers(1, 3 * L + 2))
    bt = None
    if use_bt:
        bt = rng.integers(-1, NP, size=(n_seq, L)).astype(np.int32)
    W = int(rng.integers(0, 300))
    dedupe = bool(rng.random() < 0.8)
    c = dict(seed=seed, ps=ps, n_seq=n_seq, rows_per_seq=rows_per_seq, per_seq_lists=per_seq_lists, L=L, NP=NP,
             W=W, use_bt=use_bt, dedupe=dedupe)
    _say("fuzz page tables", c)
    offs, b, e, t = [0], [], [], []
    for lst in lists:
        for s_, e_, t_ in lst:
            b.append(s_)
            e.append(e_)
            t.append(t_)
        offs.append(len(b))
    btt = None if bt is None else torch.from_numpy(bt).to(dev)
    pt, prec, pc = build_page_tables(offs, b, e, t, num_rows=R, table_width=W, page_size=ps, num_pages=NP,
                                     rows_per_seq=rows_per_seq, rows_per_list=rows_per_list, block_table=btt,
                                     dedupe=dedupe, device=dev)
    torch.cuda.synchronize()
    want = P.build_page_tables_oracle(lists, R, W, ps, NP, rows_per_seq=rows_per_seq, rows_per_list=rows_per_list,
                                      block_table=bt, dedupe=dedupe)
    assert np.array_equal(pc.cpu().numpy(), want[2]), c
    assert np.array_equal(pt.cpu().numpy(), want[0]), c
    assert np.array_equal(prec.cpu().numpy(), want[1]), c
