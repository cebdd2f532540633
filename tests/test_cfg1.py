"""cfg1 end to end through the product API.

B=1, 8 query / 8 KV heads, head_dim 64, 1024 tokens in 64 pages; the router
selects 32 pages (0-3 ALWAYS, 56-63 RECENT, 20 random ATTEND pages) and a
duck-typed plan alternates FP16 / INT8 by ascending page id; INT8 pages carry
per-page, per-head absmax scales. The path is the reference's:
BlockRouter.route_layout -> routing_to_kernel_metadata ->
metadata_to_kernel_tensors -> fused_selected_quant_decode
(examples/end_to_end_router_demo.py:48-119 for the first three steps).

CPU: the routing metadata equals the oracle's restatement of the router
(golden-pinned, tests/test_oracle_policy.py), the selection and precision
plan are the configuration's. GPU: the HIP decode equals the loop
restatement of fused_selected_quant_decode_reference (quantised pages: 1e-2)
and stays within quantisation noise of float16-value dense attention over
the selected tokens (the configuration's own comparison).
"""
import math
import sys

import numpy as np
import pytest
import torch

import bench
from oracle import decode as Dm
from oracle import policy as P


def _say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


def test_cfg1_routing_matches_oracle_and_config():
    wl = bench.build_cfg1(torch.device("cpu"))
    c = bench.CFG1
    pages = wl["pages"]
    assert len(pages) == 32 and pages[:4] == [0, 1, 2, 3] and pages[-8:] == list(range(56, 64))
    assert all(4 <= p < 56 for p in pages[4:24]) and pages == sorted(set(pages))
    # routed order: pinned blocks in layout order (ALWAYS, then RECENT), then the ATTEND blocks
    meta = wl["meta"]
    assert meta["selected_page_ids"] == pages[:4] + pages[-8:] + pages[4:24]
    # the oracle's restatement of the router gives the same metadata
    oblocks = [P.SemanticBlock(b.name, b.start, b.end, b.policy.value, b.score) for b in wl["layout_blocks"]]

    class Plan:
        def assign_block_precision(self, block):
            return P.QuantPolicy(wl["plan"][block.name].value)

    routed = P.BlockRouter(P.RouterConfig(top_k_blocks=c["attend"]), quantizer=Plan()).route_layout(
        P.BlockLayout(oblocks), c["T"])
    ometa = P.routing_to_kernel_metadata(routed, 16)
    for key in ("selected_page_ids", "block_precision_by_page", "selected_block_names", "skipped_block_names"):
        assert ometa[key] == meta[key], key
    # kernel tensors: per-head physical pages h*64 + p, alternating precisions by rank
    table, prec, counts = wl["table"].numpy(), wl["prec"].numpy(), wl["counts"].numpy()
    assert counts.tolist() == [[32] * 8]
    for h in range(8):
        assert table[0, h].tolist() == [h * 64 + p for p in meta["selected_page_ids"]]
    for rank, p in enumerate(pages):
        for h in range(8):
            assert prec[h * 64 + p] == (0 if rank % 2 == 0 else 1)
    # INT8 pages: per-page (one KV head per physical page) absmax / 127 in float16
    k16 = wl["k16"].numpy()
    amax = np.abs(k16.reshape(k16.shape[0], -1)).max(axis=1).astype(np.float16)
    assert np.array_equal(wl["ks"].numpy(), (amax.astype(np.float64) / 127).astype(np.float16))


@pytest.mark.gpu
def test_cfg1_fused_decode_on_gpu():
    from intent_attention import fused_selected_quant_decode
    _say("cfg1 end to end: router -> metadata -> fused_selected_quant_decode")
    dev = torch.device("cuda:0")
    wl = bench.build_cfg1(dev)
    out = fused_selected_quant_decode(*bench.cfg1_args(wl))
    torch.cuda.synchronize()
    assert out.shape == (1, 8, 1, 64) and out.dtype == torch.float16
    got = out.float().cpu().numpy()
    h = {k: wl[k].cpu().numpy() for k in ("q", "k16", "v16", "k8", "v8", "ks", "vs", "table", "prec", "counts")}
    loop = Dm.fused_decode_reference_loop(h["q"], h["k16"], h["v16"], h["k8"], h["v8"], h["ks"], h["vs"],
                                          h["table"], h["prec"], h["counts"], 64)
    err = float(np.abs(got - loop.astype(np.float32)).max())
    exact = Dm.paged_decode_oracle(h["q"][:, :, 0, :], {"k_fp16": h["k16"], "v_fp16": h["v16"], "k_i8": h["k8"],
                                                         "v_i8": h["v8"], "k_i8_scale": h["ks"],
                                                         "v_i8_scale": h["vs"]},
                                   h["table"], h["counts"], h["prec"])
    err_exact = float(np.abs(got[:, :, 0, :] - exact).max())
    # the configuration's comparison: float16-value dense attention over the selected tokens
    dense = np.zeros((8, 64))
    for hh in range(8):
        ids = h["table"][0, hh]
        K = h["k16"][ids].reshape(-1, 64).astype(np.float64)
        V = h["v16"][ids].reshape(-1, 64).astype(np.float64)
        s = K @ h["q"][0, hh, 0].astype(np.float64) / math.sqrt(64)
        w = np.exp(s - s.max())
        dense[hh] = w @ V / w.sum()
    d = got[0, :, 0, :] - dense
    cos = float((got[0, :, 0, :] * dense).sum() / math.sqrt((got ** 2).sum() * (dense ** 2).sum()))
    _say(f"cfg1: max abs vs loop restatement {err:.2e}, vs exact oracle {err_exact:.2e}; vs float16 dense "
         f"attention max abs {np.abs(d).max():.2e}, cosine {cos:.6f}")
    assert err <= 1e-2 and err_exact <= 1e-2
    assert np.abs(d).max() <= 2e-2 and cos >= 0.999
