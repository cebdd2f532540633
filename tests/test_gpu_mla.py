"""GPU parity of the MLA latent decode (iak_mla_decode through the C ABI)
against the CPU oracle, plus the reference-shaped APIs against the
reference's golden output (tests/golden/g5_mla_decode.npz).

Bars: max-abs <= 2e-3 with FP16 latent pages only, <= 1e-2 with FP8 / INT8
pages (the values are averages of N(0, 1) latents). The kernel computes with
f16 MFMA operands: float32 inputs of the reference-shaped API are rounded to
f16 first, which moves the golden output by up to 2.3e-3 at its magnitudes
(|out| <= 10); that test allows 1e-2.
"""
import sys

import numpy as np
import pytest

from oracle import decode as Dm
from oracle import mla as M
from oracle import quant as Q

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def dev():
    import torch
    return torch.device("cuda:0")


def _latent_case(seed, B, H, DQK, NP, W, mix, scale_f32=False, lat_scale=1.0, q_scale=1.0):
    rng = np.random.default_rng(seed)
    names = list(mix)
    probs = np.array([mix[n] for n in names], float)
    code = {"FP16": Dm.FP16, "FP8": Dm.FP8, "INT8": Dm.INT8, "SKIP": Dm.SKIP}
    tags = np.array([code[n] for n in rng.choice(names, size=NP, p=probs / probs.sum())], np.int32)
    lat = (rng.standard_normal((NP, 16, DQK)) * lat_scale).astype(np.float16)
    sdt = np.float32 if scale_f32 else np.float16
    pools = {"c_fp16": lat, "c_fp8": np.zeros((NP, 16, DQK), np.uint8), "c_fp8_scale": np.zeros(NP, sdt),
             "c_i8": np.zeros((NP, 16, DQK), np.int8), "c_i8_scale": np.zeros(NP, sdt)}
    for p in range(NP):
        if tags[p] == Dm.FP8:
            c, s = Q.quantize_page(lat[p], "FP8")
            pools["c_fp8"][p], pools["c_fp8_scale"][p] = c, s[0]
        elif tags[p] == Dm.INT8:
            c, s = Q.quantize_page(lat[p], "INT8")
            pools["c_i8"][p], pools["c_i8_scale"][p] = c, s[0]
    table = rng.integers(0, NP, size=(B, W)).astype(np.int32)
    counts = rng.integers(1, W + 1, size=B).astype(np.int32)
    counts[0] = W
    q = (rng.standard_normal((B, H, DQK)) * q_scale).astype(np.float16)
    return q, pools, table, counts, tags


def _device_pools(pools, dev):
    import torch
    from intent_attention import LatentPools
    t = {k: torch.from_numpy(v).to(dev) for k, v in pools.items()}
    return LatentPools(c_fp16=t["c_fp16"], c_fp8=t["c_fp8"], c_fp8_scale=t["c_fp8_scale"], c_int8=t["c_i8"],
                       c_int8_scale=t["c_i8_scale"])


SHAPES = [(64, 64, 0), (128, 128, 0), (256, 256, 0), (512, 512, 0), (576, 512, 0), (576, 64, 512)]


@pytest.mark.parametrize("dqk,dv,voff", SHAPES, ids=[f"{a}x{b}+{c}" for a, b, c in SHAPES])
@pytest.mark.parametrize("pps", [0, 16])
def test_mla_matches_oracle(dev, dqk, dv, voff, pps):
    import torch
    from intent_attention import mla_paged_decode
    _say("mla", f"qk={dqk} v={dv} voff={voff} pages_per_split={pps}")
    mix = {"FP16": .4, "FP8": .25, "INT8": .25, "SKIP": .1}
    q, pools, table, counts, tags = _latent_case(100 + dqk + dv + pps, 3, 70, dqk, 40, 37, mix)
    valid = (counts * 16).astype(np.int32)
    valid[1] = max(1, valid[1] - 7)            # ragged last page of sequence 1
    got = mla_paged_decode(torch.from_numpy(q).to(dev), _device_pools(pools, dev), torch.from_numpy(table).to(dev),
                           torch.from_numpy(counts).to(dev), torch.from_numpy(tags).to(dev), v_dim=dv,
                           v_offset=voff, valid_tokens=torch.from_numpy(valid).to(dev), pages_per_split=pps,
                           out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = M.mla_paged_decode_oracle(q, pools, table, counts, tags, v_dim=dv, v_offset=voff, valid_tokens=valid)
    err = np.abs(got.cpu().numpy() - ref).max()
    assert err <= 1e-2, f"max abs err {err:.3e}"


@pytest.mark.parametrize("pps", [128, 100, 65, 0])
@pytest.mark.parametrize("wide", [False, True])
def test_mla_long_splits(dev, pps, wide):
    """Splits of more than 64 table entries (a lane holds entries i and i + 64
    of its split): 150-entry tables in splits of 128 / 100 / 65 entries, one
    sequence whose count ends inside the second half of its first split, one
    with a ragged token bound there, and the automatic plan on a table wide
    enough (32 sequences x 1,300 entries: 11 splits of 128) for it to take
    more than 64 per split.
    FP8 / INT8 pages only and with FP16 pages as well (the two ring widths)."""
    import torch
    from intent_attention import mla_paged_decode
    W = 1300 if pps == 0 else 150
    _say("mla long splits", f"pages_per_split={pps} W={W} fp16={wide}")
    mix = {"FP16": .3, "FP8": .3, "INT8": .3, "SKIP": .1} if wide else {"FP8": .45, "INT8": .45, "SKIP": .1}
    q, pools, table, counts, tags = _latent_case(3000 + pps + wide, 3 if pps else 32, 40, 576, 700, W, mix)
    counts[0] = W
    if pps:
        counts[1] = 97                          # ends in the second half of split 0
    valid = (counts * 16).astype(np.int32)
    valid[-1] = 16 * 80 + 5                     # token bound inside entry 80
    got = mla_paged_decode(torch.from_numpy(q).to(dev), _device_pools(pools, dev), torch.from_numpy(table).to(dev),
                           torch.from_numpy(counts).to(dev), torch.from_numpy(tags).to(dev), v_dim=512,
                           valid_tokens=torch.from_numpy(valid).to(dev), pages_per_split=pps,
                           out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = M.mla_paged_decode_oracle(q, pools, table, counts, tags, v_dim=512, valid_tokens=valid)
    err = np.abs(got.cpu().numpy() - ref).max()
    _say(f"  max abs err {err:.2e}")
    assert err <= 1e-2, f"max abs err {err:.3e}"


@pytest.mark.parametrize("lat_scale", [1e-3, 3e-4, 300.0])
@pytest.mark.parametrize("pps", [0, 9])
def test_mla_small_and_large_latent_magnitudes(dev, lat_scale, pps):
    """Latents N(0, lat_scale^2) on FP8 / INT8 pages: page scales of ~1e-5
    (small) would put p * scale in the float16 subnormals and ~10 (large)
    times p up to 2^8 near its top; the value exponent keeps P normal.
    Relative bar 2e-3 per (sequence, head)."""
    import torch
    from intent_attention import mla_paged_decode
    _say("mla latent magnitudes", f"lat_scale={lat_scale} pages_per_split={pps}")
    mix = {"FP8": .45, "INT8": .45, "SKIP": .1}
    q, pools, table, counts, tags = _latent_case(910 + pps, 3, 70, 576, 40, 37, mix, lat_scale=lat_scale,
                                                 q_scale=1.0 / lat_scale)
    got = mla_paged_decode(torch.from_numpy(q.astype(np.float32)).to(dev), _device_pools(pools, dev),
                           torch.from_numpy(table).to(dev), torch.from_numpy(counts).to(dev),
                           torch.from_numpy(tags).to(dev), v_dim=512, pages_per_split=pps,
                           out_dtype=torch.float32)
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    ref = M.mla_paged_decode_oracle(q.astype(np.float32), pools, table, counts, tags, v_dim=512)
    assert np.all(np.isfinite(got))
    d = np.abs(got - ref).max(axis=-1)
    m = np.abs(ref).max(axis=-1)
    err = float((d / m).max())
    _say(f"  worst relative error {err:.2e}")
    assert err <= 2e-3, f"relative err {err:.3e}"


@pytest.mark.parametrize("dqk,dv,voff", SHAPES, ids=[f"{a}x{b}+{c}" for a, b, c in SHAPES])
@pytest.mark.parametrize("out_name", ["float16", "bfloat16"])
@pytest.mark.parametrize("pps", [0, 5])
def test_mla_quantised_pools_16bit_out(dev, dqk, dv, voff, out_name, pps):
    """FP8 / INT8 latent pools without an FP16 pool and a 16-bit output: the
    split partials are float16 acc / l. Checked against the oracle (1e-2) and
    against the same call with a float32 output, whose partials are float32 acc:
    the two differ by the partials' and the output's rounding only."""
    import torch
    from intent_attention import LatentPools, mla_paged_decode
    _say("mla 16-bit out", f"qk={dqk} v={dv} voff={voff} out={out_name} pages_per_split={pps}")
    mix = {"FP8": .45, "INT8": .45, "SKIP": .1}
    q, pools, table, counts, tags = _latent_case(700 + dqk + dv + pps, 3, 70, dqk, 40, 37, mix)
    valid = (counts * 16).astype(np.int32)
    valid[2] = max(1, valid[2] - 5)
    t = {k: torch.from_numpy(v).to(dev) for k, v in pools.items()}
    lp = LatentPools(c_fp8=t["c_fp8"], c_fp8_scale=t["c_fp8_scale"], c_int8=t["c_i8"], c_int8_scale=t["c_i8_scale"])
    args = (torch.from_numpy(q).to(dev), lp, torch.from_numpy(table).to(dev), torch.from_numpy(counts).to(dev),
            torch.from_numpy(tags).to(dev))
    kw = dict(v_dim=dv, v_offset=voff, valid_tokens=torch.from_numpy(valid).to(dev), pages_per_split=pps)
    got = mla_paged_decode(*args, out_dtype=getattr(torch, out_name), **kw)
    full = mla_paged_decode(*args, out_dtype=torch.float32, **kw)
    torch.cuda.synchronize()
    assert got.dtype == getattr(torch, out_name)
    got, full = got.float().cpu().numpy(), full.cpu().numpy()
    ref = M.mla_paged_decode_oracle(q, pools, table, counts, tags, v_dim=dv, v_offset=voff, valid_tokens=valid)
    assert np.all(np.isfinite(got))
    err = float(np.abs(got - ref).max())
    assert err <= 1e-2, f"max abs err {err:.3e}"
    # one float16 rounding of each partial (half an ulp, <= 2^-11 of a value that
    # is a convex combination of dequantised latents) plus the output's own rounding
    half_ulp_out = 2.0 ** -8 if out_name == "bfloat16" else 2.0 ** -11
    lat_max = 1.1 * float(np.abs(pools["c_fp16"].astype(np.float32)).max())
    bound = 2.0 ** -11 * lat_max + half_ulp_out * float(np.abs(full).max()) + 1e-6
    dif = float(np.abs(got - full).max())
    assert dif <= bound, f"16-bit vs float32 output differ by {dif:.3e} > {bound:.3e}"


def test_mla_fp16_pages_and_f32_scales(dev):
    import torch
    from intent_attention import mla_paged_decode
    _say("mla fp16-only / f32 scales")
    q, pools, table, counts, tags = _latent_case(5, 2, 128, 576, 64, 80, {"FP16": 1.0}, scale_f32=True)
    got = mla_paged_decode(torch.from_numpy(q).to(dev), _device_pools(pools, dev), torch.from_numpy(table).to(dev),
                           torch.from_numpy(counts).to(dev), torch.from_numpy(tags).to(dev), v_dim=512,
                           out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = M.mla_paged_decode_oracle(q, pools, table, counts, tags, v_dim=512)
    assert np.abs(got.cpu().numpy() - ref).max() <= 2e-3
    # the same pages through the quantised pools: codes exact in f16, scales folded in
    q, pools, table, counts, tags = _latent_case(6, 2, 128, 576, 64, 80, {"FP8": .5, "INT8": .5}, scale_f32=True)
    got = mla_paged_decode(torch.from_numpy(q).to(dev), _device_pools(pools, dev), torch.from_numpy(table).to(dev),
                           torch.from_numpy(counts).to(dev), torch.from_numpy(tags).to(dev), v_dim=512,
                           out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = M.mla_paged_decode_oracle(q, pools, table, counts, tags, v_dim=512)
    assert np.abs(got.cpu().numpy() - ref).max() <= 1e-2


def test_mla_large_latent_magnitudes(dev):
    """Latent values N(0, 9000^2) (|c| up to ~4e4, inside float16) with queries
    scaled by 1/9000: p (up to 2^8 between lazy rescales) times such an INT8
    page scale (~300) would overflow float16; the kernel's value exponent keeps
    the P operand in range. Same relative bar as unit-scale latents, no inf or
    nan."""
    import torch
    from intent_attention import mla_paged_decode
    ls = 9000.0
    _say("mla large latent magnitudes", f"lat_scale={ls}")
    q, pools, table, counts, tags = _latent_case(7, 2, 128, 576, 64, 80, {"FP16": .2, "FP8": .3, "INT8": .5},
                                                 lat_scale=ls, q_scale=1.0 / ls)
    got = mla_paged_decode(torch.from_numpy(q).to(dev), _device_pools(pools, dev), torch.from_numpy(table).to(dev),
                           torch.from_numpy(counts).to(dev), torch.from_numpy(tags).to(dev), v_dim=512,
                           out_dtype=torch.float32)
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    assert np.all(np.isfinite(got))
    ref = M.mla_paged_decode_oracle(q, pools, table, counts, tags, v_dim=512)
    err = np.abs(got - ref).max() / ls
    assert err <= 1e-2, f"max abs err / lat_scale {err:.3e}"


def test_mla_misaligned_query_and_fp8_dtype(dev):
    """A query view 2 bytes past an aligned address, and the FP8 latent pool
    given as torch.float8_e4m3fn instead of uint8 codes: same result."""
    import torch
    from intent_attention import mla_paged_decode, LatentPools
    _say("mla misaligned q / float8 pool dtype")
    q, pools, table, counts, tags = _latent_case(8, 2, 128, 576, 32, 20, {"FP8": .5, "INT8": .5})
    dp = _device_pools(pools, dev)
    tt, ct, gt = (torch.from_numpy(x).to(dev) for x in (table, counts, tags))
    base = torch.from_numpy(q).to(dev)
    want = mla_paged_decode(base, dp, tt, ct, gt, v_dim=512, out_dtype=torch.float32)
    buf = torch.zeros(q.size + 8, dtype=torch.float16, device=dev)
    view = buf[1:1 + q.size].view(q.shape)
    view.copy_(base)
    assert view.data_ptr() % 16 != 0
    dp8 = LatentPools(c_fp16=dp.c_fp16, c_fp8=dp.c_fp8.view(torch.float8_e4m3fn), c_fp8_scale=dp.c_fp8_scale,
                      c_int8=dp.c_int8, c_int8_scale=dp.c_int8_scale)
    got = mla_paged_decode(view, dp8, tt, ct, gt, v_dim=512, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_mla_empty_rows_are_zero(dev):
    import torch
    from intent_attention import mla_paged_decode
    _say("mla empty rows")
    q, pools, table, counts, tags = _latent_case(9, 3, 16, 64, 8, 5, {"FP16": .5, "SKIP": .5})
    counts[:] = [0, 5, 2]
    tags[table[2, :2]] = Dm.SKIP               # sequence 2 visits only SKIP pages
    got = mla_paged_decode(torch.from_numpy(q).to(dev), _device_pools(pools, dev), torch.from_numpy(table).to(dev),
                           torch.from_numpy(counts).to(dev), torch.from_numpy(tags).to(dev),
                           out_dtype=torch.float32).cpu().numpy()
    assert np.all(got[0] == 0) and np.all(got[2] == 0)
    ref = M.mla_paged_decode_oracle(q, pools, table, counts, tags)
    assert np.abs(got - ref).max() <= 2e-3


def test_mla_decode_triton_matches_reference_golden(dev):
    import torch
    from intent_attention import mla_decode_triton
    _say("mla_decode_triton vs golden G5")
    import os
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "g5_mla_decode.npz"))
    t = {k: torch.from_numpy(g[k]).to(dev) for k in ("q_absorb", "C", "W_VO", "page_table")}
    out = mla_decode_triton(t["q_absorb"], t["C"], t["W_VO"], t["page_table"], page_size=int(g["page_size"]))
    assert out.dtype == torch.float32 and tuple(out.shape) == g["out"].shape
    err = float(np.abs(out.cpu().numpy() - g["out"]).max())
    _say(f"  max abs err vs the reference's output {err:.2e} (max |out| {np.abs(g['out']).max():.2f})")
    assert err <= 2e-3 and err <= 1e-5 * float(np.abs(g["out"]).max())   # float32 arithmetic, as the reference
    empty = mla_decode_triton(t["q_absorb"], t["C"], t["W_VO"], t["page_table"][:0], page_size=int(g["page_size"]))
    assert torch.all(empty == 0)


@pytest.mark.parametrize("page_size", [8, 16, 32, 64])
def test_mla_decode_triton_page_sizes(dev, page_size):
    """Reference test shapes (test_triton_mla_decode.py:39-50) against the
    restated CPU loop (float64) on float32 inputs."""
    import torch
    from intent_attention import mla_decode_triton
    _say("mla_decode_triton page_size", page_size)
    rng = np.random.default_rng(page_size)
    qa = rng.standard_normal((2, 3, 64)).astype(np.float32)
    C = rng.standard_normal((6 * page_size, 64)).astype(np.float32)
    W = rng.standard_normal((64, 128)).astype(np.float32)
    pt = np.array([4, 0, 5, 2], np.int32)
    out = mla_decode_triton(torch.from_numpy(qa).to(dev), torch.from_numpy(C).to(dev), torch.from_numpy(W).to(dev),
                            torch.from_numpy(pt).to(dev), page_size=page_size)
    ref = M.mla_decode_cpu_loop(qa, C, W, pt, page_size)
    assert np.abs(out.cpu().numpy() - ref).max() <= 2e-5 * max(1.0, float(np.abs(ref).max()))


@pytest.mark.parametrize("d_c,page_size,dtype", [(576, 64, "float32"), (576, 16, "bfloat16"), (1024, 7, "float32"),
                                                 (100, 5, "float16"), (512, 1, "float32"), (33, 3, "float32")])
def test_mla_decode_triton_widths_and_dtypes(dev, d_c, page_size, dtype):
    """Every latent width up to 1,024 in one call of the float32 row kernel
    (DeepSeek's d_c = 576 included), float16 / bfloat16 inputs read as given,
    a ragged last page of C, repeated and out-of-order page ids, strided q;
    against the reference loop (float64) on the same input values."""
    import torch
    from intent_attention import mla_decode_triton
    _say("mla_decode_triton", f"d_c={d_c} page_size={page_size} {dtype}")
    rng = np.random.default_rng(d_c + page_size)
    dt = getattr(torch, dtype)
    T = 9 * page_size - (page_size // 2)                       # the last page is shorter
    qa = torch.from_numpy(rng.standard_normal((3, 2, 2 * d_c)).astype(np.float32)).to(dev).to(dt)[..., ::2]
    C = torch.from_numpy(rng.standard_normal((T, d_c)).astype(np.float32)).to(dev).to(dt)
    W = torch.from_numpy((rng.standard_normal((d_c, 40)) / np.sqrt(d_c)).astype(np.float32)).to(dev)
    pt = torch.tensor([8, 0, 3, 3, 5, 1], dtype=torch.int32, device=dev)
    out = mla_decode_triton(qa, C, W, pt, page_size=page_size)
    assert out.dtype == dt and tuple(out.shape) == (3, 2, 40)
    ref = M.mla_decode_cpu_loop(qa.float().cpu().numpy(), C.float().cpu().numpy(), W.cpu().numpy(), pt.cpu().numpy(),
                                page_size)
    got = out.float().cpu().numpy()
    out_ulp = {"float32": 0.0, "float16": 2.0 ** -11, "bfloat16": 2.0 ** -8}[dtype]   # one output rounding
    bar = (2e-5 + out_ulp) * max(1.0, float(np.abs(ref).max()))
    err = float(np.abs(got - ref).max())
    _say(f"  max abs err {err:.2e} (bar {bar:.2e})")
    assert err <= bar
    with pytest.raises(ValueError, match="page ids"):
        mla_decode_triton(qa, C, W, torch.tensor([9], dtype=torch.int32, device=dev), page_size=page_size)


def test_mla_block_table_api(dev):
    """mla_triton_decode / mla_sparse_decode_reference through MLABlockTable and
    a BlockLayout, against the closed form (reference test_vs_reference shape
    with unit-scale weights)."""
    import torch
    from intent_attention import (BlockLayout, BlockPolicy, MLABlockTable, MLAConfig, SemanticBlock,
                                  mla_sparse_decode_reference, mla_triton_decode)
    _say("mla block-table API")
    rng = np.random.default_rng(11)
    d_model, d_c, n_heads, d_head, ps = 96, 64, 4, 16, 16
    cfg = MLAConfig(d_model, d_c, n_heads, d_head)
    table = MLABlockTable(cfg, page_size=ps)
    lat = [rng.standard_normal((ps, d_c)).astype(np.float16).astype(np.float32) for _ in range(4)]
    for bid in range(4):
        table.append(bid, torch.from_numpy(lat[bid]).to(dev))
    W_QK = (rng.standard_normal((n_heads * d_head, d_c)) / 8).astype(np.float32)
    W_VO = rng.standard_normal((d_c, d_model)).astype(np.float32)
    q = rng.standard_normal((2, n_heads, 3, d_head)).astype(np.float32)
    blocks = [SemanticBlock(f"b{i}", i * ps, (i + 1) * ps, BlockPolicy.ATTEND, score=s)
              for i, s in enumerate((0.9, 0.2, 0.7, 0.6))]
    layout = BlockLayout(blocks)
    tq, tqk, tvo = (torch.from_numpy(x).to(dev) for x in (q, W_QK, W_VO))
    out_t, dbg = mla_triton_decode(tq, table, tqk, tvo, layout, threshold=0.5, return_debug=True)
    out_r, _ = mla_sparse_decode_reference(tq, table, tqk, tvo, layout, threshold=0.5)
    qa = np.transpose(q, (0, 2, 1, 3)).reshape(2, 3, n_heads * d_head).astype(np.float64) @ W_QK
    Csel = np.concatenate([lat[i] for i in (0, 2, 3)], 0)
    ref = M.mla_decode_closed_form(qa, Csel, W_VO)
    assert dbg["selected_latent_tokens"] == 3 * ps and dbg["selected_block_names"] == ["b0", "b2", "b3"]
    assert out_t.dtype == torch.float32 and out_r.dtype == torch.float16
    big = max(1.0, float(np.abs(ref).max()))
    assert np.abs(out_t.cpu().numpy() - ref).max() <= 2e-5 * big                    # float32 throughout
    assert np.abs(out_r.float().cpu().numpy() - ref).max() <= (2e-5 + 2.0 ** -11) * big   # + the f16 output


@pytest.mark.parametrize("d_c,page_size,dtype,npages", [(576, 64, "float16", 40), (512, 16, "bfloat16", 100),
                                                        (1024, 7, "float32", 200), (33, 1, "float32", 1500),
                                                        (256, 32, "float32", 300)])
def test_mla_decode_triton_split_over_keys(dev, d_c, page_size, dtype, npages):
    """Rows with 256 listed latent rows or more on a short grid take the
    split-over-keys path (partials merged by a second kernel): the ragged last
    page of C listed, repeated and out-of-order ids, against the reference loop
    (float64) on the same input values."""
    import torch
    from intent_attention import mla_decode_triton
    from intent_attention import _native as N
    _say("mla_decode_triton split", f"d_c={d_c} page_size={page_size} {dtype} pages={npages}")
    rng = np.random.default_rng(d_c * 7 + page_size)
    dt = getattr(torch, dtype)
    n_src = npages // 2 + 3
    T = n_src * page_size - (page_size // 2)                    # the last page is shorter
    qa = torch.from_numpy(rng.standard_normal((2, 2, d_c)).astype(np.float32)).to(dev).to(dt)
    C = torch.from_numpy(rng.standard_normal((T, d_c)).astype(np.float32)).to(dev).to(dt)
    W = torch.from_numpy((rng.standard_normal((d_c, 24)) / np.sqrt(d_c)).astype(np.float32)).to(dev)
    ids = rng.integers(0, n_src, size=npages).astype(np.int32)
    ids[npages // 3] = n_src - 1                                 # the short page
    pt = torch.from_numpy(ids).to(dev)
    a = N.MlaRowsArgs()
    a.batch, a.q_len, a.latent_dim, a.page_size, a.num_selected, a.num_rows = 2, 2, d_c, page_size, npages, T
    a.q, a.latents, a.page_ids, a.context, a.latent_stride = 16, 16, 16, 16, d_c
    assert N.mla_decode_rows_workspace(a) > 0                   # the shape is split
    out = mla_decode_triton(qa, C, W, pt, page_size=page_size)
    ref = M.mla_decode_cpu_loop(qa.float().cpu().numpy(), C.float().cpu().numpy(), W.cpu().numpy(), ids, page_size)
    got = out.float().cpu().numpy()
    out_ulp = {"float32": 0.0, "float16": 2.0 ** -11, "bfloat16": 2.0 ** -8}[dtype]
    bar = (2e-5 + out_ulp) * max(1.0, float(np.abs(ref).max()))
    err = float(np.abs(got - ref).max())
    _say(f"  max abs err {err:.2e} (bar {bar:.2e})")
    assert err <= bar


def test_mla_rows_split_matches_single_pass(dev, monkeypatch):
    """The split-over-keys path and the one-workgroup-per-row path (no
    workspace) of the float32 latent context agree to float32 summation order."""
    import torch
    from intent_attention import _native as N
    from intent_attention.triton_mla_decode import mla_latent_context
    _say("mla rows split vs single pass")
    rng = np.random.default_rng(4)
    qa = torch.from_numpy(rng.standard_normal((3, 1, 576)).astype(np.float32)).to(dev)
    C = torch.from_numpy(rng.standard_normal((64 * 200, 576)).astype(np.float32)).to(dev)
    pt = torch.from_numpy(rng.permutation(200)[:150].astype(np.int32)).to(dev)
    split = mla_latent_context(qa, C, pt, 64)
    with monkeypatch.context() as mp:
        mp.setattr(N, "mla_decode_rows_workspace", lambda a: 0)
        single = mla_latent_context(qa, C, pt, 64)
    torch.cuda.synchronize()
    err = float((split - single).abs().max())
    _say(f"  max |split - single| {err:.2e}")
    assert err <= 1e-5 * max(1.0, float(single.abs().max()))


@pytest.mark.parametrize("q_dt,c_dt,npages", [("float16", "bfloat16", 40), ("bfloat16", "float32", 3),
                                              ("float32", "float16", 30)])
def test_mla_latent_context_mixed_dtypes(dev, q_dt, c_dt, npages):
    """The float32 latent context reads the query and the latents each in its
    own dtype (the query's read once per row, the latents' per key), split and
    one-pass shapes, against the float64 loop on the same values."""
    import torch
    from intent_attention.triton_mla_decode import mla_latent_context
    _say("mla latent context, q", q_dt, "C", c_dt, "pages", npages)
    rng = np.random.default_rng(npages)
    d_c, ps = 576, 64
    qa = torch.from_numpy(rng.standard_normal((2, 2, d_c)).astype(np.float32)).to(dev).to(getattr(torch, q_dt))
    C = torch.from_numpy(rng.standard_normal((64 * ps, d_c)).astype(np.float32)).to(dev).to(getattr(torch, c_dt))
    ids = rng.integers(0, 64, size=npages).astype(np.int32)
    ctx = mla_latent_context(qa, C, torch.from_numpy(ids).to(dev), ps)
    eye = np.eye(d_c, dtype=np.float32)   # the loop's projection by the identity gives the context itself
    ref = M.mla_decode_cpu_loop(qa.float().cpu().numpy(), C.float().cpu().numpy(), eye, ids, ps)
    err = float(np.abs(ctx.cpu().numpy() - ref).max())
    _say(f"  max abs err {err:.2e}")
    assert ctx.dtype == torch.float32 and err <= 2e-5 * max(1.0, float(np.abs(ref).max()))
