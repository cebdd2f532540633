"""Adaptive-format decode (adaptive_format_decode_attention_triton) on the GPU
against oracle/adaptive.py: pages decoded in place (16-token pages, head_dim
64 / 128) and staged (other page shapes, format values outside 0..3, INT8
pages without INT8 pools), with -1 holes, SKIP and SPARSE pages, out-of-pool
ids, float16 / float32 queries; the reference tests' cases (shapes, zero
selected pages -> zeros); the reference dispatch's conventions."""
import sys

import numpy as np
import pytest

from oracle import adaptive as Am

pytestmark = pytest.mark.gpu

# the decode kernel's P operand is float16 (relative 2^-11); staged INT8 pages
# are rounded to float16 once more; outputs compared relative to max |ref|
TOL = 4e-3


def _say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


def _case(seed, B, H, D, PS, NP, W, odd=False):
    rng = np.random.default_rng(seed)
    k16 = rng.standard_normal((NP, PS, D)).astype(np.float16)
    v16 = rng.standard_normal((NP, PS, D)).astype(np.float16)
    k8 = rng.integers(-127, 128, (NP, PS, D)).astype(np.int8)
    v8 = rng.integers(-127, 128, (NP, PS, D)).astype(np.int8)
    ks = (rng.random(NP) * 0.02 + 0.001).astype(np.float32)
    vs = (rng.random(NP) * 0.02 + 0.001).astype(np.float32)
    fm = rng.integers(0, 4, NP).astype(np.int32)
    if odd:
        fm[rng.permutation(NP)[:2]] = [5, -2]
    ids = rng.integers(-1, NP + 2, (B, H, W)).astype(np.int32)     # holes and ids past the pool
    q = rng.standard_normal((B, H, D)).astype(np.float32)
    return q, ids, fm, k16, v16, k8, v8, ks, vs


def _run(args, qdtype, with_int8=True):
    import torch
    from intent_attention.triton_adaptive_format_attention import (AdaptiveFormatKernelConfig,
                                                                   adaptive_format_decode_attention_triton)
    q, ids, fm, k16, v16, k8, v8, ks, vs = args
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()  # noqa: E731
    cfg = AdaptiveFormatKernelConfig(page_size=k16.shape[1], head_dim=q.shape[2], max_selected_pages=ids.shape[2],
                                     block_d=max(64, q.shape[2]))
    kw = dict(int8_k_pages=t(k8), int8_v_pages=t(v8), int8_k_scales=t(ks), int8_v_scales=t(vs)) if with_int8 else {}
    out = adaptive_format_decode_attention_triton(t(q).to(qdtype), t(ids), t(fm), t(k16), t(v16), config=cfg, **kw)
    assert out.dtype == qdtype and out.shape == q.shape
    return out.float().cpu().numpy()


@pytest.mark.parametrize("B,H,D,PS,NP,W,odd", [
    (2, 4, 64, 16, 40, 24, False),      # in place
    (1, 8, 128, 16, 64, 48, False),     # in place
    (2, 2, 32, 8, 12, 6, False),        # staged: page shape
    (1, 3, 16, 4, 10, 5, False),        # staged: page shape
    (2, 3, 64, 16, 20, 9, True),        # staged: format values outside 0..3
    (1, 2, 48, 8, 9, 7, True),
])
def test_adaptive_vs_oracle(B, H, D, PS, NP, W, odd):
    import torch
    args = _case(B * 100 + D + PS, B, H, D, PS, NP, W, odd)
    q = args[0]
    for qdtype in (torch.float32, torch.float16):
        _say("adaptive", f"B={B} H={H} D={D} PS={PS} NP={NP} W={W} odd={odd} q={qdtype}")
        qq = q if qdtype == torch.float32 else q.astype(np.float16).astype(np.float32)
        ref = Am.adaptive_decode_oracle(qq, *args[1:])
        got = _run(args, qdtype)
        err = np.abs(got - ref).max()
        assert err <= TOL * max(1.0, np.abs(ref).max()), err


@pytest.mark.parametrize("PS,D", [(16, 64), (4, 16)])
def test_int8_pages_without_int8_pools_are_zero_rows(PS, D):
    import torch
    args = _case(7 + PS, 1, 2, D, PS, 8, 6)
    q, ids, fm, k16, v16 = args[:5]
    _say("adaptive no-int8", f"PS={PS} D={D}")
    ref = Am.adaptive_decode_oracle(q, ids, np.where(fm == 1, 9, fm), k16, v16)
    got = _run(args, torch.float32, with_int8=False)
    assert np.abs(got - ref).max() <= TOL * max(1.0, np.abs(ref).max())


def test_reference_cases_and_empty_rows():
    import torch
    from intent_attention.triton_adaptive_format_attention import (
        AdaptiveFormatKernelConfig, AdaptivePageFormat, adaptive_format_decode_attention_reference_dispatch,
        adaptive_format_decode_attention_triton, make_adaptive_page_tables)
    rng = np.random.default_rng(1)
    B, H, D, PS, NP, MAX_SEL = 1, 2, 32, 8, 4, 2
    fp16_kv = torch.from_numpy(rng.standard_normal((NP, PS, D)).astype(np.float16)).cuda()
    int8_kv = (fp16_kv * 10).to(torch.int8)
    int8_scales = torch.full((NP,), 0.1, dtype=torch.float32, device="cuda")
    q = torch.from_numpy(rng.standard_normal((B, H, D)).astype(np.float16)).cuda()
    page_ids = torch.zeros(B, H, MAX_SEL, dtype=torch.int32, device="cuda")
    page_ids[0, 0, 1] = 1
    fm = torch.tensor([0, 1, 3, 3], dtype=torch.int32, device="cuda")
    cfg = AdaptiveFormatKernelConfig(page_size=PS, head_dim=D, max_selected_pages=MAX_SEL)
    out = adaptive_format_decode_attention_triton(q, page_ids, fm, fp16_kv, fp16_kv, int8_k_pages=int8_kv,
                                                  int8_v_pages=int8_kv, int8_k_scales=int8_scales,
                                                  int8_v_scales=int8_scales, config=cfg)
    assert out.shape == (B, H, D) and torch.isfinite(out).all()
    ref = Am.adaptive_decode_oracle(q.float().cpu().numpy(), page_ids.cpu().numpy(), fm.cpu().numpy(),
                                    fp16_kv.cpu().numpy(), fp16_kv.cpu().numpy(), int8_kv.cpu().numpy(),
                                    int8_kv.cpu().numpy(), int8_scales.cpu().numpy(), int8_scales.cpu().numpy())
    assert np.abs(out.float().cpu().numpy() - ref).max() <= TOL * max(1.0, np.abs(ref).max())
    # every entry a hole, or every page SKIP / SPARSE: zeros
    for ids, f in ((torch.full_like(page_ids, -1), fm), (page_ids, torch.tensor([3, 2, 3, 2], device="cuda"))):
        z = adaptive_format_decode_attention_triton(q, ids, f, fp16_kv, fp16_kv, config=cfg)
        assert not z.any()
    # the dispatch: K = V = the K pages, INT8 scales rounded to float16
    s16 = int8_scales.half().float().cpu().numpy()
    d = adaptive_format_decode_attention_reference_dispatch(q.cpu(), page_ids.cpu(), fm.cpu(), fp16_kv.cpu(),
                                                            fp16_kv.cpu(), int8_k_pages=int8_kv.cpu(),
                                                            int8_k_scales=int8_scales.cpu(), config=cfg)
    refd = Am.adaptive_decode_oracle(q.float().cpu().numpy(), page_ids.cpu().numpy(), fm.cpu().numpy(),
                                     fp16_kv.cpu().numpy(), fp16_kv.cpu().numpy(), int8_kv.cpu().numpy(),
                                     int8_kv.cpu().numpy(), s16, s16)
    assert d.dtype == torch.float16 and np.abs(d.float().cpu().numpy() - refd).max() <= TOL * max(1, np.abs(refd).max())
    ids2, counts = make_adaptive_page_tables(torch.tensor([3, 1, 2], dtype=torch.int32), batch=2, heads=2,
                                             max_selected_pages=4)
    assert ids2.tolist() == [[[3, 1, 2, -1]] * 2] * 2 and counts.tolist() == [[3, 3], [3, 3]]
    assert int(AdaptivePageFormat.SPARSE) == 2
