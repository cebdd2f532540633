"""Pins the quantisation oracle (oracle/quant.py).

* e4m3fn encoder == torch's own float8_e4m3fn cast on every float16 value
  (the library the reference calls, intent_quant.py:243).
* fake_quantize_tensor reconstructions and scales == golden vectors written by
  the reference (tests/golden/g1_fake_quantize.npz), float16 and float32.
* both fake_int8_pages_from_fp16 variants == golden vectors (g3).
* closed forms: codes*scale reconstructs exactly, ties go to even, INT4
  saturates at 7/127 of the absmax, clamps, packing round trips.
"""
import os

import numpy as np
import pytest
import torch

from oracle import quant as Q


def _same(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return a.shape == b.shape and bool(np.all((a == b) | (np.isnan(a) & np.isnan(b))))


def test_e4m3_encoder_matches_torch_on_all_fp16():
    bits = np.arange(65536, dtype=np.uint16)
    x16 = bits.view(np.float16)
    ref = torch.from_numpy(x16.astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    mine = Q.e4m3fn_encode(x16.astype(np.float64))
    nan_ref = (ref & 0x7F) == 0x7F
    nan_mine = (mine & 0x7F) == 0x7F
    assert np.array_equal(nan_ref, nan_mine)
    assert np.array_equal(ref[~nan_ref], mine[~nan_mine])


def test_e4m3_decode_roundtrip_and_values():
    codes = np.arange(256, dtype=np.uint8)
    vals = Q.e4m3fn_decode(codes)
    tv = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    assert _same(vals, tv)
    finite = ~np.isnan(vals)
    assert np.array_equal(Q.e4m3fn_encode(vals[finite]), codes[finite])
    assert vals[finite].max() == 448.0 and Q.e4m3fn_decode(np.uint8(1)) == 2.0 ** -9


def test_e4m3_ties_round_to_even():
    # 1.0625 is halfway between 1.0 (mantissa 000) and 1.125 (001): even -> 1.0
    assert Q.e4m3fn_decode(Q.e4m3fn_encode(1.0625)) == 1.0
    # 1.1875 is halfway between 1.125 (001) and 1.25 (010): even -> 1.25
    assert Q.e4m3fn_decode(Q.e4m3fn_encode(1.1875)) == 1.25
    # 464 is halfway between 448 and the NaN slot: stays 448; above it is NaN
    assert Q.e4m3fn_decode(Q.e4m3fn_encode(464.0)) == 448.0
    assert np.isnan(Q.e4m3fn_decode(Q.e4m3fn_encode(465.0)))


@pytest.fixture(scope="module")
def g1(golden_dir):
    return dict(np.load(os.path.join(golden_dir, "g1_fake_quantize.npz")))


VIEWS = {
    "page": lambda x: x.reshape(-1, 1),
    "group": lambda x: x.reshape(x.shape[0] * 16, 2, 32).transpose(0, 2, 1).reshape(-1, 2),
    "chan": lambda x: x.reshape(1, 3, 16, 64),
}


@pytest.mark.parametrize("dt", ["f16", "f32"])
@pytest.mark.parametrize("view", list(VIEWS))
@pytest.mark.parametrize("prec", ["FP8", "INT8", "INT4", "INT4_RESIDUAL"])
def test_fake_quantize_matches_reference_golden(g1, dt, view, prec):
    x = g1[f"x_{dt}"]
    xv = np.ascontiguousarray(VIEWS[view](x))
    r = Q.fake_quantize_codes(xv, prec)
    key = f"{dt}_{view}_{prec}"
    assert _same(r["recon"].astype(np.float32), g1[f"recon_{key}"]), key
    assert _same(r["scale"].astype(np.float32), g1[f"scale_{key}"]), key
    if prec == "INT4_RESIDUAL":
        assert _same(r["scale2"], g1[f"rscale_{key}"]), key


@pytest.mark.parametrize("dt", ["f16", "f32"])
@pytest.mark.parametrize("prec", ["FP8", "INT8", "INT4", "INT4_RESIDUAL"])
def test_all_zero_block_matches_reference(g1, dt, prec):
    z = np.zeros((16 * 64, 1), np.float16 if dt == "f16" else np.float32)
    assert _same(Q.fake_quantize_codes(z, prec)["recon"], g1[f"zero_recon_{dt}_{prec}"])


def test_codes_times_scale_is_the_reconstruction(g1):
    x = g1["x_f16"].reshape(-1, 64)
    for prec in ("FP8", "INT8", "INT4"):
        r = Q.fake_quantize_codes(x.reshape(-1, 1), prec)
        vals = Q.e4m3fn_decode(r["codes"]) if prec == "FP8" else r["codes"].astype(np.float64)
        assert np.array_equal(vals * np.float64(r["scale"][0, 0]), r["recon"].astype(np.float64))


def test_int4_saturates_at_seven_127ths():
    # fake_quantize_tensor divides by 127 for INT4 too (intent_quant.py:224, :263-264),
    # so every value above 7/127 of the absmax clamps to code 7.
    x = np.linspace(-1, 1, 255).astype(np.float32).reshape(-1, 1)
    r = Q.fake_quantize_codes(x, "INT4")
    s = r["scale"][0, 0]
    assert s == np.float32(1.0) / np.float32(127.0)
    big = np.abs(x[:, 0]) > 7.5 * s
    assert np.all(np.abs(r["codes"][big, 0]) == 7)
    assert r["codes"].min() == -7 and r["codes"].max() == 7


def test_int8_ties_to_even():
    x = np.array([[127.0], [0.5], [1.5], [2.5], [-0.5], [-2.5]], np.float32)
    r = Q.fake_quantize_codes(x, "INT8")   # scale = 1 exactly
    assert r["scale"][0, 0] == 1.0
    assert r["codes"][:, 0].tolist() == [127, 0, 2, 2, 0, -2]


@pytest.fixture(scope="module")
def g3(golden_dir):
    return dict(np.load(os.path.join(golden_dir, "g3_fused_decode.npz")))


def test_fake_int8_pages_fused_variant_matches_reference(g3):
    for pages, q, s in ((g3["k16"], g3["k8"], g3["ks"]), (g3["v16"], g3["v8"], g3["vs"]),
                        (g3["edge_pages"], g3["edge_q"], g3["edge_s"])):
        mq, ms = Q.fake_int8_pages_fused(pages)
        assert ms.dtype == np.float16 and np.array_equal(mq, q)
        assert _same(ms, s)


def test_fake_int8_pages_triton_variant_matches_reference(g3):
    for pages, q, s in ((g3["k16"], g3["tk8"], g3["tks"]), (g3["v16"], g3["tv8"], g3["tvs"]),
                        (g3["edge_pages"], g3["edge_tq"], g3["edge_ts"])):
        mq, ms = Q.fake_int8_pages_triton(pages)
        assert ms.dtype == np.float32 and np.array_equal(mq, q)
        assert _same(ms, s)


def test_page_granule_quantiser_is_fake_quantize_on_the_page_view(g1):
    x = g1["x_f16"]                      # [3, 16, 64]; treat the 48 rows as one "page"
    page = x.reshape(48, 64)
    for prec, view in (("FP8", "page"), ("INT8", "page"), ("INT4", "group"), ("INT4_RESIDUAL", "page")):
        codes, scales = Q.quantize_page(page, prec)
        recon = Q.dequantize_page(codes, scales, prec)
        ref = g1[f"recon_f16_{view}_{prec}"]
        if view == "page":
            ref = ref.reshape(48, 64)
        else:
            ref = ref.reshape(48, 32, 2).transpose(0, 2, 1).reshape(48, 64)
        assert _same(recon, ref), prec


def test_int4_packing_roundtrip():
    rng = np.random.default_rng(0)
    c = rng.integers(-7, 8, size=(5, 16, 128)).astype(np.int8)
    p = Q.pack_int4(c)
    assert p.shape == (5, 16, 64) and np.array_equal(Q.unpack_int4(p), c)
    assert int(p[0, 0, 0]) == (int(c[0, 0, 0]) + 8) | ((int(c[0, 0, 1]) + 8) << 4)
    c2 = rng.integers(-7, 8, size=(5, 16, 128)).astype(np.int8)
    r = Q.pack_int4_residual(c, c2)
    a, b = Q.unpack_int4_residual(r)
    assert np.array_equal(a, c) and np.array_equal(b, c2)
