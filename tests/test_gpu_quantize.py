"""GPU parity of the page quantiser (iak_quantize_pages through the C ABI):
codes and scales bit-exact against the oracle's restatement of the
reference's arithmetic (oracle.quant), for every precision and both
fake_int8_pages_from_fp16 variants, including the e4m3fn encoder over every
float16 value in [-127, 127] and the all-zero page."""
import sys

import numpy as np
import pytest

from oracle import quant as Q

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def dev():
    import torch
    return torch.device("cuda:0")


def _pages(seed, n, D):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, 16, D)).astype(np.float16)
    m = rng.random(x.shape) < 0.01                       # outliers
    x = np.where(m, (8 * np.sign(x.astype(np.float32))).astype(np.float16), x)
    x[1] = 0                                             # all-zero page
    x[2] *= np.float16(1e-5)                             # tiny page: scale underflows toward 0
    x[3, :, : D // 2] = 0                                # half-zero page (zero INT4 groups)
    return x


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("prec", ["FP8", "INT8", "INT4_RESIDUAL"])
def test_page_granule_codes_are_bit_exact(dev, D, prec):
    import torch
    from intent_attention import quantize_pages
    _say("quantise", prec, D)
    x = _pages(3 + D, 12, D)
    codes, scales = quantize_pages(torch.from_numpy(x).to(dev), prec)
    codes, scales = codes.cpu().numpy(), scales.cpu().numpy()
    for p in range(x.shape[0]):
        c, s = Q.quantize_page(x[p], prec)
        if prec == "INT4_RESIDUAL":
            (q1, q2), (s1, s2) = c, s
            assert np.array_equal(codes[p], Q.pack_int4_residual(q1, q2)), p
            assert scales[p, 0] == np.float32(s1[0]) and scales[p, 1] == s2[0], p
        else:
            want = c.view(np.uint8) if prec == "FP8" else c
            assert np.array_equal(codes[p].view(np.uint8), want.view(np.uint8)), p
            assert scales[p].tobytes() == np.asarray(s[0], np.float16).tobytes(), p


@pytest.mark.parametrize("D,group", [(128, 32), (128, 64), (128, 128), (64, 32), (64, 64)])
def test_int4_group_codes_are_bit_exact(dev, D, group):
    import torch
    from intent_attention import quantize_pages
    _say("quantise INT4", D, group)
    x = _pages(5 + group, 10, D)
    codes, scales = quantize_pages(torch.from_numpy(x).to(dev), "INT4", int4_group=group,
                                   scale_dtype=torch.float32)
    codes, scales = codes.cpu().numpy(), scales.cpu().numpy()
    for p in range(x.shape[0]):
        c, s = Q.quantize_page(x[p], "INT4", group)
        assert np.array_equal(codes[p], Q.pack_int4(c)), p
        assert np.array_equal(scales[p], s.astype(np.float32)), p


def test_e4m3fn_encoder_over_all_float16(dev):
    """absmax 127 gives scale 1, so the codes are e4m3fn of the values themselves."""
    import torch
    from intent_attention import quantize_pages
    _say("e4m3fn exhaustive")
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    v = allh[np.isfinite(allh) & (np.abs(allh.astype(np.float32)) <= 127)]
    per = 16 * 128 - 1
    n = -(-v.size // per)
    x = np.zeros((n, 16 * 128), np.float16)
    x[:, 0] = 127
    flat = np.concatenate([v, np.zeros(n * per - v.size, np.float16)])
    x[:, 1:] = flat.reshape(n, per)
    codes, scales = quantize_pages(torch.from_numpy(x.reshape(n, 16, 128)).to(dev), "FP8")
    assert np.all(scales.cpu().numpy() == 1)
    got = codes.cpu().numpy().reshape(n, -1)[:, 1:].reshape(-1)[: v.size]
    assert np.array_equal(got, Q.e4m3fn_encode(v.astype(np.float64)))


@pytest.mark.parametrize("variant", ["fused", "triton"])
def test_fake_int8_variants_are_bit_exact(dev, variant):
    import torch
    from intent_attention import fake_int8_pages_device
    _say("fake_int8", variant)
    x = _pages(11, 9, 128)
    codes, scales = fake_int8_pages_device(torch.from_numpy(x).to(dev), variant)
    ref = Q.fake_int8_pages_fused(x) if variant == "fused" else Q.fake_int8_pages_triton(x)
    assert np.array_equal(codes.cpu().numpy(), ref[0])
    assert scales.cpu().numpy().tobytes() == ref[1].astype(scales.cpu().numpy().dtype).tobytes()


def test_scatter_into_pool(dev):
    """Pages written at chosen pool ids; ids outside the pool are skipped."""
    import torch
    from intent_attention import quantize_pages
    _say("quantise scatter")
    x = _pages(13, 4, 128)
    codes = torch.full((10, 16, 128), 7, dtype=torch.int8, device=dev)
    scales = torch.full((10,), 3.0, dtype=torch.float16, device=dev)
    dst = torch.tensor([8, 0, 11, 5], dtype=torch.int32, device=dev)
    quantize_pages(torch.from_numpy(x).to(dev), "INT8", codes=codes, scales=scales, dst_pages=dst)
    c, s = codes.cpu().numpy(), scales.cpu().numpy()
    for i, d in enumerate((8, 0, None, 5)):
        if d is None:
            continue
        rc, rs = Q.quantize_page(x[i], "INT8")
        assert np.array_equal(c[d], rc) and s[d] == rs[0]
    untouched = [k for k in range(10) if k not in (8, 0, 5)]
    assert np.all(c[untouched] == 7) and np.all(s[untouched] == 3.0)
