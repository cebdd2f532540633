"""KV memory manager on the GPU: the transcoding kernels (iak_transcode_pages),
the manager built on them, and the page warm-up (iak_prefetch_pages).

* demote / promote through the C ABI == the reference's own outputs (g6
  golden vectors: write_page INT8 codes and scale, _read_page_data, both
  set_page_format directions), bit for bit, and == the oracle on random and
  special pages (NaN, inf, subnormal, all-zero, exact ties) with a slot list
  holding out-of-range slots that must leave the pools untouched;
* KVMemoryManager: the reference's test cases on device pools, with data
  checked bit-exactly against the oracle, and step() against the oracle's
  attention over the reconstructed rows, on both decode routes (pools in the
  kernel layout, and staged rows for other page shapes, SPARSE pages and
  partial-page masks);
* warm-up: the per-wave checksums == a CPU fold of the same rows (ragged last
  page, pages past kv_len and negative ids skipped, strided views), and a
  decode after a warm-up is bit-identical to one without.
"""
import os
import sys

import numpy as np
import pytest

from oracle import memory as Mm

pytestmark = pytest.mark.gpu

# float16 step outputs vs the float64 oracle: the decode kernel's P operand is
# float16 (relative 2^-11) and the output is rounded to float16
STEP_TOL = 4e-3


def _say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


def _dev():
    import torch
    return torch.device("cuda:0")


def _transcode(mode, fp16, int8, scales, pages=None):
    import torch
    from intent_attention import _native as N
    a = N.TranscodeArgs()
    n = fp16.shape[0] if pages is None else pages.numel()
    a.num_pages, a.page_elems, a.mode = n, fp16[0].numel(), mode
    a.pages = 0 if pages is None else pages.data_ptr()
    a.pool_pages = fp16.shape[0]
    a.fp16, a.int8, a.scales = fp16.data_ptr(), int8.data_ptr(), scales.data_ptr()
    N.transcode_pages(a, torch.cuda.current_stream(fp16.device).cuda_stream)
    torch.cuda.synchronize()


def _u16(x):
    return np.ascontiguousarray(x).view(np.uint16)


def _same_f16(a, b):
    """Bit-equal float16 arrays, any NaN matching any NaN (the sign of a
    default NaN differs between the GPU and the host's float unit)."""
    a, b = np.asarray(a, np.float16), np.asarray(b, np.float16)
    na, nb = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(na, nb) and np.array_equal(_u16(a)[~na], _u16(b)[~nb]))


@pytest.fixture(scope="module")
def g6(golden_dir):
    return dict(np.load(os.path.join(golden_dir, "g6_kv_transcode.npz")))


@pytest.mark.parametrize("si", [0, 1, 2])
def test_transcode_kernels_match_reference_golden(g6, si):
    import torch
    from intent_attention import _native as N
    dev = _dev()
    x = g6[f"s{si}_x"]
    n = x.shape[0]
    _say("transcode golden", f"set={si} shape={x.shape}")
    fp16 = torch.from_numpy(x.reshape(n, -1).copy()).to(dev)
    int8 = torch.zeros(fp16.shape, dtype=torch.int8, device=dev)
    scales = torch.zeros(n, dtype=torch.float32, device=dev)
    _transcode(N.TRANSCODE_DEMOTE_INT8, fp16, int8, scales)
    assert np.array_equal(int8.cpu().numpy().reshape(x.shape), g6[f"s{si}_codes"])
    assert np.array_equal(scales.cpu().numpy(), g6[f"s{si}_scale"].astype(np.float32))
    back = torch.empty_like(fp16)
    _transcode(N.TRANSCODE_PROMOTE_FP16, back, int8, scales)
    got = back.cpu().numpy().reshape(x.shape)
    assert np.array_equal(_u16(got), _u16(g6[f"s{si}_promoted"]))
    assert np.array_equal(_u16(got), _u16(g6[f"s{si}_fp16_back"]))
    _transcode(N.TRANSCODE_DEMOTE_INT8, back, int8, scales)
    assert np.array_equal(int8.cpu().numpy().reshape(x.shape), g6[f"s{si}_codes2"])
    assert np.array_equal(scales.cpu().numpy(), g6[f"s{si}_scale2"].astype(np.float32))


def _special_pages(rng, n, elems):
    x = (rng.standard_normal((n, elems)) * rng.choice([1e-3, 1.0, 30.0], size=(n, 1))).astype(np.float16)
    x[0] = 0
    x[1, 5] = np.nan
    x[2, 3] = np.inf
    x[3] *= np.float16(1e-4)                     # subnormal codes after scaling
    x[4] = np.round(rng.standard_normal(elems) * 4) / 4
    x[4, 0] = 127.0                              # scale 1: exact ties at .5 steps
    x[5, 0] = 65504.0
    x[6] = -x[6]
    return x


# 8 .. 2048: register demote (4 chunks per lane); 4096: 8 chunks per lane;
# 8200: two-pass demote; 4096 and 8200: promote over several 256-chunk rounds
@pytest.mark.parametrize("elems", [8, 1024, 2048, 16 * 48 + 8, 4096, 8200])
def test_transcode_slot_lists_vs_oracle(elems):
    import torch
    from intent_attention import _native as N
    dev = _dev()
    rng = np.random.default_rng(elems)
    NPOOL = 40
    x = _special_pages(rng, NPOOL, elems)
    slots = rng.permutation(NPOOL)[:25].astype(np.int32)
    listed = np.concatenate([slots, np.array([-1, NPOOL, NPOOL + 7, -100], np.int32)])
    rng.shuffle(listed)
    _say("transcode slots", f"elems={elems} slots={len(listed)}")
    fp16 = torch.from_numpy(x.copy()).to(dev)
    int8 = torch.full((NPOOL, elems), 0x5A, dtype=torch.int8, device=dev)
    scales = torch.full((NPOOL,), 7.0, dtype=torch.float32, device=dev)
    ids = torch.from_numpy(listed).to(dev)
    _transcode(N.TRANSCODE_DEMOTE_INT8, fp16, int8, scales, ids)
    codes, sc = int8.cpu().numpy(), scales.cpu().numpy()
    want_codes, want_sc = {}, {}
    for p in range(NPOOL):
        if p in set(slots.tolist()):
            c, s = Mm.demote_int8(x[p])
            want_codes[p], want_sc[p] = c, np.float32(s)
            assert np.array_equal(codes[p], c), p
            assert sc[p] == np.float32(s) or (np.isnan(sc[p]) and np.isnan(np.float32(s))), p
        else:
            assert (codes[p] == 0x5A).all() and sc[p] == 7.0, p
    # promote the listed slots into a pool of sentinels
    out = torch.full((NPOOL, elems), -3.0, dtype=torch.float16, device=dev)
    _transcode(N.TRANSCODE_PROMOTE_FP16, out, int8, scales, ids)
    got = out.cpu().numpy()
    for p in range(NPOOL):
        if p in want_codes:
            want = Mm.promote_fp16(want_codes[p], float(want_sc[p]))
            assert _same_f16(got[p], want), p
        else:
            assert (got[p] == -3.0).all(), p


def test_transcode_rejects_bad_arguments():
    import torch
    from intent_attention import _native as N
    dev = _dev()
    fp16 = torch.zeros((4, 12), dtype=torch.float16, device=dev)      # 12 elements: not a multiple of 8
    int8 = torch.zeros((4, 12), dtype=torch.int8, device=dev)
    scales = torch.zeros(4, dtype=torch.float32, device=dev)
    with pytest.raises(ValueError, match="multiple of 8"):
        _transcode(N.TRANSCODE_DEMOTE_INT8, fp16, int8, scales)
    a = N.TranscodeArgs()
    a.num_pages, a.page_elems, a.mode, a.pool_pages = 1, 8, 5, 1
    a.fp16, a.int8, a.scales = fp16.data_ptr(), int8.data_ptr(), scales.data_ptr()
    with pytest.raises(ValueError, match="mode"):
        N.transcode_pages(a, 0)


# ----------------------------------------------------------------- manager


def _mgr(num_pages=8, page_size=4, head_dim=16, **kw):
    from intent_attention.kv_memory_manager import KVMemoryManager
    return KVMemoryManager(num_pages=num_pages, page_size=page_size, head_dim=head_dim, device="cuda:0", **kw)


def _rand_page(rng, ps, d, scale=1.0):
    return (rng.standard_normal((ps, d)) * scale).astype(np.float16)


def _t(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(_dev())


def test_manager_write_read_and_transitions():
    from intent_attention.kv_memory_manager import PageStorageFormat as F
    rng = np.random.default_rng(11)
    m = _mgr()
    m.policy.attend_low_format = F.INT8
    assert m.allocate_pages("a", "ALWAYS", 2) == [0, 1]
    assert m.allocate_pages("b", "ATTEND", 1, score=0.1) == [2]
    assert m.allocate_pages("s", "SKIP", 1) == [3]
    pages = [_rand_page(rng, 4, 16) for _ in range(4)]
    pages[1].flat[[3, 17, 40, 55, 60]] = [9.0, -8.5, 8.0, 7.5, -7.0]     # distinct top-5 |values|
    for pid in range(4):
        m.write_page(pid, _t(pages[pid]))
    assert np.array_equal(_u16(m.pages[0].kv_fp16.cpu().numpy()), _u16(pages[0]))
    st = m.pages[2]
    codes, s = Mm.demote_int8(pages[2])
    assert st.format == F.INT8 and st.kv_fp16 is None
    assert np.array_equal(st.kv_int8.cpu().numpy(), codes) and st.kv_int8_scale == s      # float64, as written
    assert np.array_equal(_u16(m._read_page_data(2).cpu().numpy()), _u16(Mm.promote_fp16(codes, s)))
    assert m.pages[3].kv_fp16 is None and m.pages[3].kv_int8 is None          # SKIP writes nothing
    # FP16 -> INT8 -> FP16 through set_page_format: oracle demote then promote
    m.set_page_format(0, F.INT8)
    c0, s0 = Mm.demote_int8(pages[0])
    assert m.pages[0].kv_fp16 is None and np.array_equal(m.pages[0].kv_int8.cpu().numpy(), c0)
    m.set_page_format(0, F.FP16)
    assert m.pages[0].kv_int8 is None
    assert np.array_equal(_u16(m.pages[0].kv_fp16.cpu().numpy()), _u16(Mm.promote_fp16(c0, s0)))
    # SPARSE keeps the top-k flat values; back to FP16 scatters them
    m.sparse_max_nnz = 5
    m.set_page_format(1, F.SPARSE)
    assert m.pages[1].sp_nnz == 5
    m.set_page_format(1, F.FP16)
    flat = pages[1].reshape(-1)
    top = np.argsort(-np.abs(flat.astype(np.float64)), kind="stable")[:5]
    want = np.zeros_like(flat)
    want[top] = flat[top]
    assert np.array_equal(_u16(m.pages[1].kv_fp16.cpu().numpy().reshape(-1)), _u16(want))


def test_manager_demote_promote_cycle_and_selection():
    from intent_attention.kv_memory_manager import PageStorageFormat as F
    rng = np.random.default_rng(12)
    m = _mgr()
    m.allocate_pages("keep", "ALWAYS", 3)
    m.allocate_pages("skip", "SKIP", 2)
    pages = [_rand_page(rng, 4, 16, 10.0) for _ in range(3)]
    for pid in range(3):
        m.write_page(pid, _t(pages[pid]))
        m.pages[pid].last_access_step = 0
    selected, fmts, ids, masks = m.select_pages()
    assert selected == [0, 1, 2] and masks is None
    assert ids.tolist() == [[[0, 1, 2]]] and fmts.tolist() == [0, 0, 0, 3, 3]
    m.step_count = 15
    assert m.demote_cold_pages() == [0, 1, 2]
    for pid in range(3):
        c, s = Mm.demote_int8(pages[pid])
        assert m.pages[pid].format == F.INT8 and np.array_equal(m.pages[pid].kv_int8.cpu().numpy(), c)
        m.pages[pid].access_count = 10 if pid != 1 else 0
    assert m.promote_hot_pages() == [0, 2]
    for pid in (0, 2):
        c, s = Mm.demote_int8(pages[pid])
        assert np.array_equal(_u16(m.pages[pid].kv_fp16.cpu().numpy()), _u16(Mm.promote_fp16(c, s)))
    assert m.pages[1].format == F.INT8
    # a page whose format is set by hand, without data: promoted to an empty FP16 page
    m.pages[1].kv_int8 = None
    m.pages[1].access_count = 10
    assert m.promote_hot_pages() == [1]
    assert m.pages[1].format == F.FP16 and m.pages[1].kv_fp16 is None


def _oracle_pages(m, pages_np, selected, masks=None):
    """The oracle's per-page description of the manager's selected pages."""
    out = []
    for pid in selected:
        st = m.pages[pid]
        has = {0: st.kv_fp16 is not None, 1: st.kv_int8 is not None, 2: st.sp_k_values is not None}
        d = {"format": st.format.name, "data": pages_np[pid] if has.get(int(st.format), False) else None}
        if masks and pid in masks:
            d["mask"] = masks[pid].cpu().numpy()
        out.append(d)
    return out


@pytest.mark.parametrize("ps,d", [(4, 16), (16, 64), (16, 128), (8, 48)])
def test_manager_step_vs_oracle(ps, d):
    import torch
    from intent_attention.kv_memory_manager import PageStorageFormat as F
    rng = np.random.default_rng(ps * 1000 + d)
    _say("manager step", f"page_size={ps} head_dim={d}")
    m = _mgr(num_pages=12, page_size=ps, head_dim=d)
    m.allocate_pages("sys", "ALWAYS", 3)
    m.allocate_pages("low", "ATTEND", 4, score=0.1)       # INT8
    m.allocate_pages("skip", "SKIP", 2)
    m.allocate_pages("late", "RECENT", 2)                 # second page never written
    pages = {pid: _rand_page(rng, ps, d, 2.0) for pid in range(11)}
    for pid in range(10):
        m.write_page(pid, _t(pages[pid]))
    q = rng.standard_normal((2, 3, d)).astype(np.float32)
    for step in range(3):
        out = m.step(_t(q).half() if step == 1 else _t(q))
        selected, _, _, _ = m.select_pages()
        assert selected == [0, 1, 2, 3, 4, 5, 6, 9, 10]
        qq = q.astype(np.float16).astype(np.float64) if step == 1 else q
        ref = Mm.step_attention(qq, Mm.step_rows(_oracle_pages(m, pages, selected), ps, d))
        assert out.dtype == torch.float16 and out.shape == (2, 3, d)
        err = np.abs(out.float().cpu().numpy() - ref).max()
        assert err <= STEP_TOL * max(1.0, np.abs(ref).max()), (step, err)
        assert m.pages[0].access_count == step + 1 and m.pages[0].last_access_step == step + 1
        if step == 0:
            m.set_page_format(1, F.INT8)                  # mixed formats in one block
    # a SPARSE page goes through the staged rows (page 0: FP16, distinct top |values|)
    pages[0] = pages[0].copy()
    pages[0].flat[[0, 5, 17, 3, 40, 2, 60, 1]] = [9.0, -8.5, 8.0, 7.5, -7.0, 6.5, 6.0, -5.5]
    m.write_page(0, _t(pages[0]))
    m.set_page_format(0, F.SPARSE)
    out = m.step(_t(q))
    ref = Mm.step_attention(q, Mm.step_rows(_oracle_pages(m, pages, m.select_pages()[0]), ps, d))
    assert np.abs(out.float().cpu().numpy() - ref).max() <= STEP_TOL * max(1.0, np.abs(ref).max())


@pytest.mark.parametrize("ps,d", [(4, 16), (16, 64)])
def test_manager_step_with_partial_page_masks(ps, d):
    from intent_attention.block_metadata import BlockLayout, BlockPolicy, SemanticBlock
    rng = np.random.default_rng(77 + ps)
    m = _mgr(num_pages=8, page_size=ps, head_dim=d)
    m.register_layout(BlockLayout([SemanticBlock("a", 0, ps + ps // 2, BlockPolicy.ALWAYS),
                                   SemanticBlock("b", 2 * ps + 1, 3 * ps + 3, BlockPolicy.ATTEND, score=0.1)]))
    selected, _, _, masks = m.select_pages()
    # a: pages 0 (full) and 1 (first half); b: page 2 (ps tokens from an unaligned
    # start: not partial) and page 3 (two tokens at offsets 1, 2)
    assert masks is not None and set(masks) == {1, 3}
    assert masks[3].tolist() == [i in (1, 2) for i in range(ps)]
    pages = {pid: _rand_page(rng, ps, d) for pid in m.pages}
    for pid in m.pages:
        m.write_page(pid, _t(pages[pid]))
    q = rng.standard_normal((1, 2, d)).astype(np.float32)
    for use in (False, True):
        out = m.step(_t(q), mask=use)
        ref = Mm.step_attention(q, Mm.step_rows(_oracle_pages(m, pages, selected, masks if use else None), ps, d))
        assert np.abs(out.float().cpu().numpy() - ref).max() <= STEP_TOL * max(1.0, np.abs(ref).max()), use


def test_manager_empty_warmup_and_all_flags():
    import torch
    from intent_attention.kv_memory_manager import PageStorageFormat as F
    rng = np.random.default_rng(5)
    out = _mgr(num_pages=4).step(torch.randn(1, 1, 16, device=_dev(), dtype=torch.float16))
    assert out.shape == (1, 1, 16) and not out.any()
    m = _mgr()
    m.allocate_pages("block", "ALWAYS", 4)
    pages = {pid: _rand_page(rng, 4, 16) for pid in range(4)}
    for pid in range(4):
        m.write_page(pid, _t(pages[pid]))
    m.set_page_format(0, F.INT8)
    m.set_page_format(1, F.INT8)
    m._prefetch_predictions = [0, 1, 3]
    assert m._prefetch_warmup() == [0, 1]
    assert m.pages[0].format == F.FP16 and m.pages[1].format == F.FP16
    q = torch.randn(1, 1, 16, device=_dev(), dtype=torch.float16)
    for _ in range(4):
        out = m.step(q, demote=True, promote=True, warmup=True, adapt=True, mask=True)
        assert out.shape == (1, 1, 16) and torch.isfinite(out).all()
    assert m.predict_prefetch() == [0, 1, 2, 3]
    summ = m.page_summary()
    assert summ["num_pages"] == 4 and summ["step"] == 4 and summ["total_accesses"] == 16


def test_manager_adapt_policy():
    rng = np.random.default_rng(6)
    m = _mgr(num_pages=4, adapt_policy_every=1)
    m.allocate_pages("block", "ALWAYS", 2)
    for pid in range(2):
        m.write_page(pid, _t(_rand_page(rng, 4, 16)))
    old = m.policy.demote_cold_after_steps
    m._demote_history.extend([True, True, False])
    m._adapt_policy()
    assert m.policy.demote_cold_after_steps == old + 1          # hit rate 2/3 > 0.3; no cold pages
    m2 = _mgr(num_pages=4, adapt_policy_every=1)
    m2.allocate_pages("block", "ALWAYS", 2)
    m2.step_count = 20
    m2._adapt_policy()
    assert m2.policy.demote_cold_after_steps == old - 1         # every FP16 page cold


# ----------------------------------------------------------------- warm-up


def _checksums_cpu(k, v, page_ids, page_size):
    """The warm-up's per-wave fold, on the host: [B * H * n_ids * 4] uint32."""
    B, H, T, D = k.shape
    out = np.zeros((B * H, len(page_ids), 4), np.uint32)
    for e, p in enumerate(page_ids):
        t0 = p * page_size
        if p < 0 or t0 >= T:
            continue
        rows = min(page_size, T - t0)
        i = np.arange(rows * D)
        wave = (i % 256) // 64
        for x in (k, v):
            blk = np.ascontiguousarray(x[:, :, t0:t0 + rows, :]).view(np.uint16).reshape(B * H, -1).astype(np.uint32)
            words = blk << (16 * (i & 1)).astype(np.uint32)
            for w in range(4):
                out[:, e, w] ^= np.bitwise_xor.reduce(words[:, wave == w], axis=1) if (wave == w).any() else 0
    return out.reshape(-1)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_prefetch_checksums(dtype):
    import torch
    from intent_attention.prefetch import get_prefetch_stream, launch_prefetch_pages
    rng = np.random.default_rng(9)
    B, H, T, D, PS = 2, 3, 100, 64, 16
    kb = torch.from_numpy(rng.standard_normal((B, H, T, 2 * D)).astype(np.float32)).to(getattr(torch, dtype))
    vb = torch.from_numpy(rng.standard_normal((B, H, T, D)).astype(np.float32)).to(getattr(torch, dtype))
    kd, v = kb.to(_dev())[..., D:], vb.to(_dev())                # k: a strided view ([..., D:] of 2D columns)
    ids = [0, 3, 6, 99, -1, 2, 6]
    _say("prefetch", dtype, f"ids={ids}")
    s = get_prefetch_stream()
    got = launch_prefetch_pages(kd, v, torch.tensor(ids, device=_dev()), stream=s, page_size=PS)
    torch.cuda.synchronize()
    want = _checksums_cpu(kb[..., D:].view(torch.int16).numpy(), vb.view(torch.int16).numpy(), ids, PS)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want)


def test_prefetch_leaves_decode_unchanged():
    import torch
    from intent_attention.kv_memory_manager import PageStorageFormat as F
    from intent_attention.prefetch import launch_prefetch_pages
    rng = np.random.default_rng(10)
    m = _mgr(num_pages=16, page_size=16, head_dim=64)
    m.allocate_pages("a", "ALWAYS", 6)
    for pid in range(6):
        m.write_page(pid, _t(_rand_page(rng, 16, 64)))
    m.set_page_format(2, F.INT8)
    q = _t(rng.standard_normal((1, 4, 64)).astype(np.float32))
    a = m.step(q)
    pool = m._fp16_pool.view(1, 1, -1, 64)
    launch_prefetch_pages(pool, pool, torch.arange(6, device=_dev()), page_size=16)
    b = m.step(q)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
