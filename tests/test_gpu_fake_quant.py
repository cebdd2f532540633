"""GPU parity of the selected-block reconstruction that
intent_quant_attention_reference attends over (its per-block
fake_quantize_tensor and torch.cat, intent_quant_attention.py:56-84), built
for float32 K and V by libiak's iak_fake_quant_blocks through the C ABI: bit
for bit the oracle's restatement of fake_quantize_tensor (oracle.quant, pinned
against the reference's golden g1) applied block by block, for every
precision, ragged blocks out of token order, zero, tiny and outlier channels,
magnitudes down to e4m3fn's subnormal codes, a channel count that leaves part
of a 64-channel group idle, strided K and V, and NaN / inf inputs."""
import sys

import numpy as np
import pytest

from oracle import quant as Q

pytestmark = pytest.mark.gpu

PRECS = ["FP16", "FP8", "INT8", "INT4", "INT4_RESIDUAL", "SKIP"]


def _say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def dev():
    import torch
    return torch.device("cuda:0")


def _blocks(spans):
    from intent_attention.block_metadata import BlockPolicy, SemanticBlock
    return [SemanticBlock(f"b{i}", s, e, BlockPolicy.ATTEND, score=1.0) for i, (s, e) in enumerate(spans)]


def _oracle_cat(x: np.ndarray, spans, precs):
    """The reference's loop on the oracle: each block's reconstruction, in
    block order, as float32 (torch.cat's promotion for float32 inputs)."""
    return np.concatenate([Q.fake_quantize_tensor(np.ascontiguousarray(x[..., s:e, :]), p).astype(np.float32)
                           for (s, e), p in zip(spans, precs)], axis=-2)


def _bits_equal(got: np.ndarray, want: np.ndarray) -> bool:
    return got.shape == want.shape and np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _run(dev, k_np, v_np, spans, precs, k_dev=None, v_dev=None):
    import torch
    from intent_attention import KVPrecision
    from intent_attention.intent_quant_attention import _native_blocks_apply, _reconstruct_selected
    k = torch.from_numpy(k_np).to(dev) if k_dev is None else k_dev
    v = torch.from_numpy(v_np).to(dev) if v_dev is None else v_dev
    total = sum(e - s for s, e in spans)
    kprecs = [KVPrecision(p) for p in precs]
    assert _native_blocks_apply(k, v, total, kprecs)      # the case runs on the kernel
    kr, vr, tok, starts = _reconstruct_selected(k, v, _blocks(spans), kprecs)
    torch.cuda.synchronize()
    assert kr.dtype == torch.float32 and vr.dtype == torch.float32
    assert tok.tolist() == [t for s, e in spans for t in range(s, e)]
    assert starts == list(np.concatenate(([0], np.cumsum([e - s for s, e in spans]))))
    return kr.cpu().numpy(), vr.cpu().numpy()


def _kv(seed, lead, T, dk, dv):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((*lead, T, dk)).astype(np.float32)
    v = rng.standard_normal((*lead, T, dv)).astype(np.float32)
    k[..., 5] *= 30.0                                    # outlier channel
    k[..., 1] = 0.0                                      # zero channel: scale floor 1e-8, codes 0
    v[..., 2] *= np.float32(1e-12)                       # tiny channel: absmax / 127 below 1e-8
    m = rng.random(v.shape) < 0.01                       # scattered outliers
    v = np.where(m, v * 50.0, v).astype(np.float32)
    return k, v


# blocks out of token order, ragged lengths (1 .. 33 tokens)
SPANS = [(40, 56), (0, 16), (16, 20), (60, 93), (20, 24), (93, 94), (24, 40), (100, 117)]


@pytest.mark.parametrize("dk,dv", [(32, 48), (64, 64), (128, 128)])
def test_mixed_blocks_bit_exact(dev, dk, dv):
    _say("fake-quant blocks mixed", dk, dv)
    k, v = _kv(7 + dk, (2, 3), 120, dk, dv)
    for r, precs in enumerate([
            ["INT4", "FP16", "INT8", "INT4_RESIDUAL", "INT8", "SKIP", "FP8", "INT4"],
            ["FP8"] * 8, ["INT4_RESIDUAL"] * 8, ["FP16"] * 7 + ["SKIP"], ["SKIP"] * 8,
            ["SKIP", "INT4", "SKIP", "INT4", "SKIP", "INT4", "SKIP", "FP8"]]):
        kr, vr = _run(dev, k, v, SPANS, precs)
        assert _bits_equal(kr, _oracle_cat(k, SPANS, precs)), (dk, dv, r, precs)
        assert _bits_equal(vr, _oracle_cat(v, SPANS, precs)), (dk, dv, r, precs)


def test_fp16_blocks_alone_stay_float16(dev):
    """Only FP16 blocks: torch.cat of float16 reconstructions is float16, so
    the reconstruction is float16 (torch's own chain, not the float32 kernel)."""
    import torch
    from intent_attention import KVPrecision
    from intent_attention.intent_quant_attention import _native_blocks_apply, _reconstruct_selected
    _say("fake-quant blocks all FP16")
    k, v = _kv(2, (2,), 120, 64, 32)
    kd, vd = torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev)
    precs = [KVPrecision.FP16] * len(SPANS)
    assert not _native_blocks_apply(kd, vd, 100, precs)
    kr, vr, _, _ = _reconstruct_selected(kd, vd, _blocks(SPANS), precs)
    assert kr.dtype == torch.float16 and vr.dtype == torch.float16
    assert np.array_equal(kr.cpu().numpy(), _oracle_cat(k, SPANS, ["FP16"] * len(SPANS)).astype(np.float16))


@pytest.mark.parametrize("prec", PRECS)
def test_each_precision_long_blocks_2d(dev, prec):
    """K and V as [T, D] (one leading row), blocks of up to 700 tokens, values
    over eight decades (e4m3fn subnormal and zero codes), odd channel counts."""
    _say("fake-quant blocks long", prec)
    rng = np.random.default_rng(PRECS.index(prec))
    T = 1500
    mag = 10.0 ** rng.uniform(-8, 0, size=(T, 80))
    k = (np.sign(rng.standard_normal((T, 80))) * mag).astype(np.float32)
    v = rng.standard_normal((T, 72)).astype(np.float32)
    spans = [(800, 1500), (0, 3), (3, 400), (400, 800)]
    precs = [prec] * len(spans) if prec != "FP16" else ["FP16"] * 3 + ["INT8"]
    kr, vr = _run(dev, k, v, spans, precs)
    assert _bits_equal(kr, _oracle_cat(k, spans, precs)), prec
    assert _bits_equal(vr, _oracle_cat(v, spans, precs)), prec


def test_strided_inputs(dev):
    """K a channel slice of a wider tensor (token stride above its width), V a
    view with permuted leading dims (reshaped to a copy): the same bits as
    contiguous inputs."""
    import torch
    _say("fake-quant blocks strided")
    rng = np.random.default_rng(5)
    wide = rng.standard_normal((2, 4, 128, 96)).astype(np.float32)
    vt = rng.standard_normal((4, 2, 128, 64)).astype(np.float32)
    k_np = np.ascontiguousarray(wide[..., 16:80])
    v_np = np.ascontiguousarray(vt.transpose(1, 0, 2, 3))
    k_dev = torch.from_numpy(wide).to(dev)[..., 16:80]
    v_dev = torch.from_numpy(vt).to(dev).permute(1, 0, 2, 3)
    spans = [(64, 128), (0, 7), (7, 64)]
    precs = ["INT4_RESIDUAL", "FP8", "INT8"]
    kr, vr = _run(dev, k_np, v_np, spans, precs, k_dev=k_dev, v_dev=v_dev)
    assert _bits_equal(kr, _oracle_cat(k_np, spans, precs))
    assert _bits_equal(vr, _oracle_cat(v_np, spans, precs))


def test_nan_and_inf_propagate(dev):
    """A NaN or inf in a block's channel makes that channel's scale NaN or inf,
    so every quantised value of the channel in that block is NaN (torch.amax
    propagates NaN; x / inf is 0 or NaN and 0 * inf is NaN); FP16 rounds the
    values themselves and SKIP writes zeros; other channels and blocks are
    untouched."""
    _say("fake-quant blocks nan/inf")
    k, v = _kv(3, (1, 2), 64, 64, 64)
    k[0, 1, 10, 7] = np.nan
    v[0, 0, 40, 9] = np.inf
    spans = [(0, 32), (32, 64)]
    for precs in (["INT8", "FP8"], ["INT4_RESIDUAL", "INT4"], ["FP16", "SKIP"]):
        kr, vr = _run(dev, k, v, spans, precs)
        for got, x, blk, ch in ((kr, k, 0, 7), (vr, v, 1, 9)):
            s, e = spans[blk]
            p = precs[blk]
            col = got[..., s:e, ch]
            if p == "FP16":
                assert _bits_equal(col, x[..., s:e, ch].astype(np.float16).astype(np.float32))
            elif p == "SKIP":
                assert not col.any()
            else:
                assert np.isnan(col).all(), (p, ch)
            # everything else matches the oracle bit for bit
            keep = np.ones(got.shape, bool)
            keep[..., s:e, ch] = False
            assert _bits_equal(got[keep], _oracle_cat(x, spans, precs)[keep]), precs


def test_attention_output_unchanged_by_kernel_path(dev):
    """intent_quant_attention_reference on float32 device tensors (the kernel
    path) gives the output of attention over the oracle's reconstruction."""
    import torch
    from oracle import attention as A
    from intent_attention import BlockLayout, KVPrecision, QuantPolicy, intent_quant_attention_reference
    _say("fake-quant blocks through intent_quant_attention_reference")
    k, v = _kv(21, (1, 4), 120, 64, 64)
    q = np.random.default_rng(22).standard_normal((1, 4, 3, 64)).astype(np.float32)
    precs = ["INT4", "FP16", "INT8", "INT4_RESIDUAL", "INT8", "SKIP", "FP8", "INT4"]
    spans = sorted(SPANS)                                  # a layout lists its blocks in token order
    blocks = _blocks(spans)

    class _Plan:
        def assign_block_precision(self, block):
            p = KVPrecision(precs[int(block.name[1:])])
            return QuantPolicy(precision=p, reason="test")

    out = intent_quant_attention_reference(torch.from_numpy(q).to(dev), torch.from_numpy(k).to(dev),
                                           torch.from_numpy(v).to(dev), BlockLayout(blocks), _Plan())
    want = A.dense_attention(q, _oracle_cat(k, spans, precs), _oracle_cat(v, spans, precs))
    err = float(np.abs(out.cpu().numpy() - want).max())
    assert err <= 2e-5, err


def test_split_equals_one_pass_through_the_c_abi(dev):
    """iak_fake_quant_blocks with its split workspace (long blocks over several
    workgroups, three launches) and without one (a workgroup per block and 64
    channels): the same bits, and the oracle's. Blocks of 1 .. 1,100 tokens
    over 6 leading rows, so some split ranges are empty; every precision."""
    import torch
    from intent_attention import _native as N
    _say("fake-quant blocks split vs one pass (C ABI)")
    rng = np.random.default_rng(17)
    lead, T, dk, dv = 6, 2400, 96, 64
    k = rng.standard_normal((lead, T, dk)).astype(np.float32)
    v = rng.standard_normal((lead, T, dv)).astype(np.float32)
    k[..., 3] *= 40.0
    v[..., 7] = 0.0
    spans = [(1200, 2300), (0, 1), (1, 3), (3, 515), (515, 1200), (2300, 2400)]
    codes = [N.FQ_INT4_RESIDUAL, N.FQ_FP8, N.FQ_INT8, N.FQ_INT4, N.FQ_FP16, N.FQ_SKIP]
    names = ["INT4_RESIDUAL", "FP8", "INT8", "INT4", "FP16", "SKIP"]
    lens = [e - s for s, e in spans]
    dst = np.concatenate(([0], np.cumsum(lens)))
    meta = np.array([[s, n, d, c] for (s, _), n, d, c in zip(spans, lens, dst[:-1], codes)], dtype=np.int32)
    kd, vd = torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev)
    blocks = torch.from_numpy(meta).to(dev)
    total = int(dst[-1])

    def run(split):
        out = torch.full((lead, total, dk + dv), float("nan"), device=dev)
        a = N.FakeQuantBlocksArgs()
        a.lead, a.num_blocks, a.k_dim, a.v_dim = lead, len(spans), dk, dv
        a.k, a.k_stride_l, a.k_stride_t = kd.data_ptr(), kd.stride(0), kd.stride(1)
        a.v, a.v_stride_l, a.v_stride_t = vd.data_ptr(), vd.stride(0), vd.stride(1)
        a.blocks, a.max_block_tokens = blocks.data_ptr(), max(lens)
        a.out, a.out_stride_l, a.out_stride_t = out.data_ptr(), out.stride(0), out.stride(1)
        nws = N.fake_quant_blocks_workspace(a)
        assert nws > 0                                   # these blocks are long enough to split
        ws = torch.empty(nws, dtype=torch.uint8, device=dev)
        if split:
            N.fake_quant_blocks(a, torch.cuda.current_stream(dev).cuda_stream, ws.data_ptr(), nws)
        else:
            N.fake_quant_blocks(a, torch.cuda.current_stream(dev).cuda_stream)
        torch.cuda.synchronize()
        return out.cpu().numpy()

    one, split = run(False), run(True)
    assert _bits_equal(split, one)
    assert _bits_equal(one[..., :dk], _oracle_cat(k, spans, names))
    assert _bits_equal(one[..., dk:], _oracle_cat(v, spans, names))


def test_fuzz_bit_exact(dev):
    """24 seeded cases: leading shapes of 1-3 dims, 1-40 leading rows, K and V
    widths from 1 to 200 channels, 1-12 blocks of 1-300 tokens in shuffled
    order with random precisions, magnitudes spread over a few decades and a
    token stride wider than the rows; each against the oracle bit for bit
    (one pass or split, as the workspace rule picks)."""
    import torch
    rng = np.random.default_rng(2026)
    for case in range(24):
        nlead = int(rng.integers(1, 4))
        lead = tuple(int(x) for x in rng.integers(1, 5, size=nlead))
        if case % 6 == 5:
            lead = (int(rng.integers(20, 41)),)
        dk, dv = int(rng.integers(1, 201)), int(rng.integers(1, 201))
        nb = int(rng.integers(1, 13))
        lens = [int(x) for x in rng.integers(1, 301 if case % 4 == 0 else 40, size=nb)]
        gaps = [int(x) for x in rng.integers(0, 5, size=nb)]
        spans, t = [], 0
        for n, gp in zip(lens, gaps):
            spans.append((t + gp, t + gp + n))
            t += gp + n
        T = t + int(rng.integers(0, 8))
        order = rng.permutation(nb)
        spans = [spans[i] for i in order]
        precs = [str(p) for p in rng.choice(PRECS, size=nb)]
        if all(p == "FP16" for p in precs):
            precs[0] = "INT8"
        scale = (10.0 ** rng.uniform(-3, 2, size=(dk,))).astype(np.float32)
        k = (rng.standard_normal((*lead, T, dk)) * scale).astype(np.float32)
        v = (rng.standard_normal((*lead, T, dv)) * 10.0 ** rng.uniform(-2, 1)).astype(np.float32)
        _say("fake-quant fuzz", case, lead, T, dk, dv, nb, precs)
        wide = torch.zeros((*lead, T, dk + 3), device=dev)
        wide[..., 1:dk + 1] = torch.from_numpy(k).to(dev)
        k_dev = wide[..., 1:dk + 1]                          # token stride dk + 3
        kr, vr = _run(dev, k, v, spans, precs, k_dev=k_dev)
        assert _bits_equal(kr, _oracle_cat(k, spans, precs)), (case, lead, dk, dv, spans, precs)
        assert _bits_equal(vr, _oracle_cat(v, spans, precs)), (case, lead, dk, dv, spans, precs)


def test_block_table_cache(dev):
    """The kernel path keeps each layout's device block table (per device,
    stream, spans and precisions): a repeated call reuses it and gives the same
    bits, a changed precision or another stream builds a new one, and at most
    _TABLES_SIZE layouts stay cached."""
    import torch
    from intent_attention import KVPrecision
    from intent_attention import intent_quant_attention as IQ
    _say("fake-quant block-table cache")
    k, v = _kv(31, (1, 4), 120, 64, 64)
    kd, vd = torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev)
    precs = [KVPrecision(p) for p in ["INT8", "FP8", "INT4", "INT4_RESIDUAL", "FP16", "SKIP", "INT8", "FP8"]]
    IQ._TABLES.clear()
    kr1, vr1, tok1, _ = IQ._reconstruct_selected(kd, vd, _blocks(SPANS), precs)
    kr2, vr2, tok2, _ = IQ._reconstruct_selected(kd, vd, _blocks(SPANS), precs)
    torch.cuda.synchronize()
    assert len(IQ._TABLES) == 1 and tok1 is tok2                 # one upload, reused
    assert torch.equal(kr1.view(torch.int32), kr2.view(torch.int32))
    assert torch.equal(vr1.view(torch.int32), vr2.view(torch.int32))
    precs2 = list(precs)
    precs2[0] = KVPrecision.INT4
    kr3, _, _, _ = IQ._reconstruct_selected(kd, vd, _blocks(SPANS), precs2)
    assert len(IQ._TABLES) == 2
    names = [p.value for p in precs2]
    assert _bits_equal(kr3.cpu().numpy(), _oracle_cat(k, SPANS, names))
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        kr4, _, _, _ = IQ._reconstruct_selected(kd, vd, _blocks(SPANS), precs)
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    assert len(IQ._TABLES) == 3                                   # per stream
    assert torch.equal(kr4.view(torch.int32), kr1.view(torch.int32))
    for i in range(IQ._TABLES_SIZE + 4):                          # distinct layouts: the LRU bound
        IQ._reconstruct_selected(kd, vd, _blocks([(i, i + 3), (50, 60)]), [KVPrecision.INT8, KVPrecision.FP8])
    torch.cuda.synchronize()
    assert len(IQ._TABLES) == IQ._TABLES_SIZE
    IQ._TABLES.clear()
