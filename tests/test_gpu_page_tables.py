"""GPU page-table builder (iak_build_page_tables through the C ABI) against the
reference's kernel tensors (golden G2) and the CPU oracle
(oracle.policy.build_page_tables_oracle). Integer work: every comparison is
exact."""
import json
import os
import sys

import numpy as np
import pytest

from oracle import policy as P

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def dev():
    import torch
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def g2(golden_dir):
    with open(os.path.join(golden_dir, "g2_router_metadata.json")) as f:
        return json.load(f)


def _np(t):
    return None if t is None else t.cpu().numpy()


def test_routing_to_kernel_tensors_matches_reference_golden(dev, g2):
    import intent_attention as ia
    _say("page tables: G2 records")
    for rec in g2:
        layout = ia.BlockLayout([ia.SemanticBlock(n, s, e, ia.BlockPolicy(pol), sc)
                                 for n, s, e, pol, sc in rec["blocks"]])
        routed = ia.BlockRouter(ia.RouterConfig(**rec["config"])).route_layout(layout, rec["total_tokens"])
        ps = rec["page_size"]
        num_pages = (rec["total_tokens"] + ps - 1) // ps
        pt, prec, pc = ia.routing_to_kernel_tensors(routed, ps, num_pages, B=2, H=3,
                                                    config=ia.FusedDecodeConfig(max_selected_pages=40), device=dev)
        assert pt.device.type == "cuda" and pt.dtype == prec.dtype == pc.dtype
        assert pt.tolist() == rec["kernel"]["page_table"]
        assert prec.tolist() == rec["kernel"]["page_precision"]
        assert pc.tolist() == rec["kernel"]["page_counts"]
        _, prec_n, _ = ia.routing_to_kernel_tensors(routed, ps, num_pages, native_precisions=True, device=dev)
        meta = ia.routing_to_kernel_metadata(routed, ps)
        _, prec_h, _ = ia.metadata_to_kernel_tensors(meta, num_pages, native_precisions=True)
        assert prec_n.tolist() == prec_h.tolist()


def _random_spans(rng, n_spans, max_tok, max_len, tags=(0, 1, 2, 3, 4, 5)):
    s = rng.integers(0, max_tok, size=n_spans)
    e = s + rng.integers(-3, max_len, size=n_spans)          # some empty / inverted spans
    t = rng.choice(tags, size=n_spans)
    return [(int(a), int(b), int(c)) for a, b, c in zip(s, e, t)]


def _flatten(lists):
    offs, b, e, t = [0], [], [], []
    for lst in lists:
        for s_, e_, t_ in lst:
            b.append(s_)
            e.append(e_)
            t.append(t_)
        offs.append(len(b))
    return offs, b, e, t


def _check(dev, lists, R, W, ps, NP, rows_per_seq=1, rows_per_list=None, block_table=None, dedupe=True):
    import torch
    from intent_attention import build_page_tables
    offs, b, e, t = _flatten(lists)
    bt = None if block_table is None else torch.from_numpy(np.ascontiguousarray(block_table, np.int32)).to(dev)
    pt, prec, pc = build_page_tables(offs, b, e, t, num_rows=R, table_width=W, page_size=ps, num_pages=NP,
                                     rows_per_seq=rows_per_seq, rows_per_list=rows_per_list, block_table=bt,
                                     dedupe=dedupe, device=dev)
    torch.cuda.synchronize()
    want = P.build_page_tables_oracle(lists, R, W, ps, NP, rows_per_seq=rows_per_seq, rows_per_list=rows_per_list,
                                      block_table=block_table, dedupe=dedupe)
    assert np.array_equal(_np(pc), want[2])
    assert np.array_equal(_np(pt), want[0])
    assert np.array_equal(_np(prec), want[1])


@pytest.mark.parametrize("dedupe", [True, False])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_per_sequence_lists_with_block_table(dev, seed, dedupe):
    """B sequences x Hkv rows, one routing per sequence, block tables with holes
    into a shared pool, truncation and overlapping spans."""
    _say("page tables: per-sequence lists, block table", seed, dedupe)
    rng = np.random.default_rng(seed)
    B, H, ps, L = 5, 4, 16, 300
    lists = [_random_spans(rng, int(rng.integers(0, 40)), L * ps, 200) for _ in range(B)]
    NP = B * L
    bt = np.stack([rng.permutation(NP)[:L] for _ in range(B)]).astype(np.int32)
    bt[rng.random(bt.shape) < 0.15] = -1
    for W in (1, 37, 400):
        _check(dev, lists, B * H, W, ps, NP, rows_per_seq=H, rows_per_list=H, block_table=bt, dedupe=dedupe)


def test_shared_pages_precision_lowest_row_wins(dev):
    """Sequences that select the same physical page with different tags."""
    _say("page tables: precision conflicts")
    lists = [[(0, 64, 1), (32, 96, 3)], [(0, 128, 0)], [(16, 48, 5), (200, 260, 4)]]
    bt = np.array([[7, 3, 9, 1, 2, 5, 6, 4, 8, 0, 10, 11, 12, 13, 14, 15, 16]] * 3, np.int32)
    bt[1, :4] = [3, 7, 1, 9]
    _check(dev, lists, 6, 8, 16, 17, rows_per_seq=2, rows_per_list=2, block_table=bt)


def test_many_spans_and_wide_lists(dev):
    """More than 256 spans in a list (chunked scan), a list whose pages span more
    than the LDS map (direct first-seen test) and per-row lists."""
    _say("page tables: 700 spans, wide range, per-row lists")
    rng = np.random.default_rng(5)
    many = _random_spans(rng, 700, 4000 * 16, 300)
    _check(dev, [many], 3, 2000, 16, 4000)
    wide = [(0, 40, 1), (16 * 20000, 16 * 20000 + 50, 3), (8, 64, 0), (16 * 19999, 16 * 20001, 5), (-20, 5, 2)]
    _check(dev, [wide], 2, 16, 16, 30000)
    wide_many = _random_spans(rng, 300, 16 * 40000, 64)
    _check(dev, [wide_many], 1, 512, 16, 40000)
    rows = [_random_spans(rng, int(rng.integers(0, 30)), 3000, 300) for _ in range(8)]
    _check(dev, rows, 8, 64, 7, 500, rows_per_seq=8, rows_per_list=1)


@pytest.mark.parametrize("lead", [0, 1, 2, 3])
def test_precision_array_unaligned_and_odd_length(dev, lead):
    """The precision passes use 16-byte accesses on the 16-byte-aligned body of
    the array and single words around it: an array starting `lead` words past a
    16-byte boundary with 1003 pages is written exactly and its neighbours are
    left alone (through the C ABI, which takes any 4-byte-aligned pointer)."""
    import torch
    from intent_attention import _native as N
    _say("page tables: precision array offset", lead)
    rng = np.random.default_rng(9 + lead)
    R, W, ps, NP = 3, 500, 16, 1003
    lists = [_random_spans(rng, 40, NP * ps, 200)]
    want = P.build_page_tables_oracle(lists, R, W, ps, NP)
    offs, b, e, t = _flatten(lists)
    i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=dev)  # noqa: E731
    spans = [i32(x) for x in (offs, b, e, t)]
    table = torch.empty((R, W), dtype=torch.int32, device=dev)
    counts = torch.empty(R, dtype=torch.int32, device=dev)
    buf = torch.full((NP + 8,), -77, dtype=torch.int32, device=dev)
    prec = buf[lead:lead + NP]
    a = N.PageTableArgs()
    a.num_rows, a.rows_per_seq, a.rows_per_list = R, 1, R
    a.table_width, a.page_size, a.num_pages, a.dedupe, a.default_tag = W, ps, NP, 1, 0
    a.span_offsets, a.span_begin, a.span_end, a.span_tag = (x.data_ptr() for x in spans)
    a.page_table, a.page_counts, a.page_precision = table.data_ptr(), counts.data_ptr(), prec.data_ptr()
    N.build_page_tables(a, torch.cuda.current_stream(dev).cuda_stream)
    torch.cuda.synchronize()
    got = buf.cpu().numpy()
    assert np.array_equal(got[lead:lead + NP], want[1])
    assert np.all(got[:lead] == -77) and np.all(got[lead + NP:] == -77)
    assert np.array_equal(_np(table), want[0]) and np.array_equal(_np(counts), want[2])


def test_empty_inputs(dev):
    import torch
    from intent_attention import build_page_tables
    _say("page tables: empty inputs")
    _check(dev, [[]], 4, 8, 16, 10)
    _check(dev, [[(5, 5, 1), (9, 3, 1)]], 2, 8, 16, 10)        # empty and inverted spans
    _check(dev, [[(0, 100, 1)]], 2, 0, 16, 10)                 # width 0: counts 0, precision still set
    pt, prec, pc = build_page_tables([0], [], [], [], num_rows=0, table_width=4, page_size=16, num_pages=5,
                                     device=dev)
    assert pt.shape == (0, 4) and pc.shape == (0,) and prec.tolist() == [0] * 5
    pt, prec, pc = build_page_tables([0, 1], [0], [32], [1], num_rows=3, table_width=4, page_size=16,
                                     num_pages=0, device=dev)
    assert pc.tolist() == [0, 0, 0] and pt.tolist() == [[0] * 4] * 3 and prec.numel() == 0
    torch.cuda.synchronize()


def test_device_routing_feeds_the_decode(dev):
    """Per-sequence routings through routing_to_kernel_tensors, then the decode
    on those tables equals the decode on host-built tables."""
    import torch
    import intent_attention as ia
    from intent_attention.decode_core import PagePools, paged_decode
    _say("page tables -> paged decode")
    rng = np.random.default_rng(3)
    B, Hkv, G, D, T = 3, 2, 4, 128, 1024
    routings = []
    for b in range(B):
        blocks, t = [], 0
        while t < T - 16:
            ln = int(rng.integers(8, 120))
            pol = ["ALWAYS", "ATTEND", "SKIP", "RECENT"][int(rng.integers(0, 4))]
            sc = float(np.round(rng.random(), 1)) if pol == "ATTEND" else None
            blocks.append(ia.SemanticBlock(f"s{b}b{len(blocks)}", t, min(t + ln, T), ia.BlockPolicy(pol), sc))
            t += ln
        routings.append(ia.BlockRouter(ia.RouterConfig(memory_pressure=0.2))
                        .route_layout(ia.BlockLayout(blocks), T))
    L = T // 16
    NP = B * L
    bt = torch.from_numpy(np.stack([rng.permutation(NP)[:L] for _ in range(B)]).astype(np.int32)).to(dev)
    cfg = ia.FusedDecodeConfig(max_selected_pages=L)
    pt, prec, pc = ia.routing_to_kernel_tensors(routings, 16, NP, B=B, H=Hkv, config=cfg, block_table=bt)
    # host construction of the same tables
    want = P.build_page_tables_oracle([P.routed_spans(r_) for r_ in _to_oracle(routings)], B * Hkv, L, 16, NP,
                                      rows_per_seq=Hkv, rows_per_list=Hkv, block_table=bt.cpu().numpy())
    assert np.array_equal(_np(pt).reshape(B * Hkv, L), want[0]) and np.array_equal(_np(prec), want[1])
    k = torch.randn(NP, 16, D, device=dev).half()
    v = torch.randn(NP, 16, D, device=dev).half()
    pools = PagePools(k_fp16=k, v_fp16=v)
    q = torch.randn(B, Hkv * G, D, device=dev).half()
    out_dev = paged_decode(q, pools, pt, pc, prec, out_dtype=torch.float32)
    out_host = paged_decode(q, pools, torch.from_numpy(want[0].reshape(B, Hkv, L)).to(dev),
                            torch.from_numpy(want[2].reshape(B, Hkv)).to(dev), torch.from_numpy(want[1]).to(dev),
                            out_dtype=torch.float32)
    assert torch.equal(out_dev, out_host)


def _to_oracle(routings):
    return [[P.RoutedBlock(r.name, r.start, r.end, r.policy.value, r.score, r.decision.value, r.precision.value,
                           r.reason) for r in rs] for rs in routings]


def test_side_stream_and_graph_replays(dev):
    """The builder on a non-default stream and captured in a HIP graph: every
    replay (outputs clobbered by eager work in between) equals the eager result."""
    import torch
    from intent_attention import _native as N
    _say("page tables: side stream + graph replays")
    rng = np.random.default_rng(12)
    lists = [_random_spans(rng, 40, 200 * 16, 300) for _ in range(4)]
    R, W, NP = 8, 64, 4 * 200
    offs, b, e, t = (torch.tensor(x, dtype=torch.int32, device=dev) for x in _flatten(lists))
    bt = torch.from_numpy(np.stack([rng.permutation(NP)[:200] for _ in range(4)]).astype(np.int32)).to(dev)
    table = torch.empty((R, W), dtype=torch.int32, device=dev)
    counts = torch.empty(R, dtype=torch.int32, device=dev)
    prec = torch.empty(NP, dtype=torch.int32, device=dev)
    a = N.PageTableArgs()
    a.num_rows, a.rows_per_seq, a.rows_per_list, a.table_width, a.page_size, a.num_pages = R, 2, 2, W, 16, NP
    a.dedupe, a.default_tag, a.block_table_width = 1, 0, 200
    a.span_offsets, a.span_begin, a.span_end, a.span_tag = offs.data_ptr(), b.data_ptr(), e.data_ptr(), t.data_ptr()
    a.block_table, a.page_table, a.page_counts, a.page_precision = (bt.data_ptr(), table.data_ptr(),
                                                                    counts.data_ptr(), prec.data_ptr())
    want = P.build_page_tables_oracle(lists, R, W, 16, NP, rows_per_seq=2, rows_per_list=2,
                                      block_table=bt.cpu().numpy())
    side = torch.cuda.Stream(dev)
    with torch.cuda.stream(side):
        N.build_page_tables(a, side.cuda_stream)
    side.synchronize()
    assert np.array_equal(_np(table), want[0]) and np.array_equal(_np(counts), want[2])
    assert np.array_equal(_np(prec), want[1])
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        N.build_page_tables(a, torch.cuda.current_stream(dev).cuda_stream)
    for rep in range(3):
        table.fill_(-7)
        counts.fill_(-7)
        prec.fill_(-7)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(_np(table), want[0]), rep
        assert np.array_equal(_np(counts), want[2]), rep
        assert np.array_equal(_np(prec), want[1]), rep
