"""Write the golden vectors in tests/golden/*.npz by running the reference.

Run in the build container only (the reference tree does not exist on the GPU
box):

    PYTHONPATH=/root/reference/src python tests/golden/make_golden.py

It imports the reference package read-only and calls, on small seeded
inputs, exactly the functions whose results nothing else pins: the
float16/float32 arithmetic of ``fake_quantize_tensor`` (G1), router metadata
on odd layouts (G2), ``fused_selected_quant_decode_reference`` and both
``fake_int8_pages_from_fp16`` variants (G3), ``intent_quant_attention_reference``
(G4), ``_mla_decode_cpu`` (G5) and the KV memory manager's INT8 page
transcoding (G6). The fixtures hold inputs and outputs only.
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))

from intent_attention import block_metadata as bm                                  # noqa: E402
from intent_attention import block_router as br                                    # noqa: E402
import importlib                                                                   # noqa: E402

fsq = importlib.import_module("intent_attention.fused_selected_quant_decode")        # the package re-exports a function of the same name
from intent_attention import intent_quant as iq                                    # noqa: E402
from intent_attention import intent_quant_attention as iqa                         # noqa: E402
from intent_attention import triton_intent_quant_attention as tiq                  # noqa: E402
from intent_attention import triton_mla_decode as tmd                              # noqa: E402
from intent_attention import kv_memory_manager as kvm                              # noqa: E402


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def _save(name: str, **arrays) -> None:
    path = os.path.join(HERE, name)
    np.savez_compressed(path, **arrays)
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


# --------------------------------------------------------------------------- #
# G1: fake_quantize_tensor
# --------------------------------------------------------------------------- #

def g1() -> None:
    g = torch.Generator().manual_seed(1001)
    out = {}
    base = torch.randn(3, 16, 64, generator=g)
    base[0, 3, 5] = 8.0                     # an outlier
    base[1] = torch.round(base[1] * 4) / 4  # many exact quarters -> ties after scaling
    base[2, :, 7] = 0.0                     # a zero channel
    cases = {
        "page": lambda x: x.reshape(-1, 1),                                          # per page
        "group": lambda x: x.view(x.shape[0] * 16, 2, 32).permute(0, 2, 1).reshape(-1, 2),  # per 32-group
        "chan": lambda x: x.reshape(1, 3, 16, 64),                                   # per channel
    }
    for dt_name, dt in (("f16", torch.float16), ("f32", torch.float32)):
        x = base.to(dt)
        out[f"x_{dt_name}"] = _np(x)
        for view_name, view in cases.items():
            xv = view(x).contiguous()
            for prec in (iq.KVPrecision.FP8, iq.KVPrecision.INT8, iq.KVPrecision.INT4,
                         iq.KVPrecision.INT4_RESIDUAL):
                recon, meta = iq.fake_quantize_tensor(xv, prec)
                key = f"{dt_name}_{view_name}_{prec.value}"
                out[f"recon_{key}"] = _np(recon.float() if recon.dtype == torch.float16 else recon)
                out[f"scale_{key}"] = _np(meta["scale"].float())
                if "residual_scale" in meta:
                    out[f"rscale_{key}"] = _np(meta["residual_scale"].float())
    # all-zero page in both dtypes (0/0 paths)
    for dt_name, dt in (("f16", torch.float16), ("f32", torch.float32)):
        z = torch.zeros(16, 64, dtype=dt).reshape(-1, 1)
        for prec in (iq.KVPrecision.FP8, iq.KVPrecision.INT8, iq.KVPrecision.INT4,
                     iq.KVPrecision.INT4_RESIDUAL):
            recon, meta = iq.fake_quantize_tensor(z, prec)
            out[f"zero_recon_{dt_name}_{prec.value}"] = _np(recon.float())
    _save("g1_fake_quantize.npz", **out)


# --------------------------------------------------------------------------- #
# G2: router -> routing_to_kernel_metadata
# --------------------------------------------------------------------------- #

def _layouts():
    P = bm.BlockPolicy
    S = bm.SemanticBlock
    yield "basic", 448, bm.BlockLayout([
        S("system", 0, 64, P.ALWAYS), S("doc_high", 64, 192, P.ATTEND, score=0.9),
        S("doc_low", 192, 320, P.ATTEND, score=0.1), S("recent", 320, 384, P.RECENT),
        S("unused", 384, 448, P.SKIP)])
    yield "e2e", 448, bm.BlockLayout([
        S("system", 0, 64, P.ALWAYS), S("doc_high", 64, 192, P.ATTEND, score=0.85),
        S("doc_low", 192, 320, P.ATTEND, score=0.15), S("recent", 320, 384, P.RECENT),
        S("unused", 384, 448, P.SKIP)])
    # odd boundaries, ties, skip blocks with scores, global, gaps
    yield "odd", 1000, bm.BlockLayout([
        S("g", 3, 40, P.GLOBAL), S("a1", 40, 77, P.ATTEND, score=0.5),
        S("a2", 77, 100, P.ATTEND, score=0.5), S("s1", 120, 150, P.SKIP, score=0.6),
        S("a3", 150, 151, P.ATTEND, score=0.95), S("s2", 151, 200, P.SKIP, score=0.1),
        S("a4", 210, 333, P.ATTEND, score=0.2), S("r", 900, 1000, P.RECENT)])
    rng = np.random.default_rng(2024)
    for n in range(6):
        blocks, t = [], int(rng.integers(0, 20))
        pols = [P.ALWAYS, P.ATTEND, P.ATTEND, P.ATTEND, P.SKIP, P.RECENT, P.GLOBAL]
        for i in range(int(rng.integers(5, 30))):
            ln = int(rng.integers(1, 90))
            pol = pols[int(rng.integers(0, len(pols)))]
            score = None
            if pol == P.ATTEND or rng.random() < 0.3:
                score = float(np.round(rng.random(), 2))
            blocks.append(S(f"b{i}", t, t + ln, pol, score=score))
            t += ln + int(rng.integers(0, 30))
        yield f"rand{n}", t + 5, bm.BlockLayout(blocks)


def g2() -> None:
    records = []
    configs = [dict(), dict(score_threshold=0.3), dict(top_k_blocks=2, memory_pressure=0.9),
               dict(top_k_blocks=100, memory_pressure=0.2), dict(memory_pressure=0.65, prefetch_top_k=8)]
    for name, total, layout in _layouts():
        for ci, cfg in enumerate(configs):
            for ps in (16, 7):
                router = br.BlockRouter(br.RouterConfig(**cfg))
                routed = router.route_layout(layout, total)
                meta = br.routing_to_kernel_metadata(routed, page_size=ps)
                num_pages = (total + ps - 1) // ps
                pt, prec, pc = fsq.metadata_to_kernel_tensors(
                    meta, num_pages=num_pages, B=2, H=3,
                    config=fsq.FusedDecodeConfig(max_selected_pages=40))
                records.append({
                    "layout": name, "total_tokens": total, "config": cfg, "page_size": ps,
                    "blocks": [[b.name, b.start, b.end, b.policy.value, b.score] for b in layout.blocks],
                    "routed": [[r.name, r.decision.value, r.precision.value, r.reason] for r in routed],
                    "meta": meta,
                    "selected_page_ids_router": router.selected_page_ids(routed, ps),
                    "prefetch_page_ids_router": router.prefetch_page_ids(routed, ps),
                    "kernel": {"page_table": _np(pt).tolist(), "page_precision": _np(prec).tolist(),
                               "page_counts": _np(pc).tolist()},
                })
    path = os.path.join(HERE, "g2_router_metadata.json")
    with open(path, "w") as f:
        json.dump(records, f, default=float)  # insertion order kept: dict order is part of the result
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


# --------------------------------------------------------------------------- #
# G3: fused_selected_quant_decode_reference + fake_int8_pages_from_fp16
# --------------------------------------------------------------------------- #

def g3() -> None:
    g = torch.Generator().manual_seed(3003)
    B, H, D, PS, NP, W = 2, 4, 64, 16, 8, 6
    k16 = torch.randn(NP, PS, D, generator=g).half()
    v16 = torch.randn(NP, PS, D, generator=g).half()
    q = torch.randn(B, H, 1, D, generator=g).half()
    k8, ks = fsq.fake_int8_pages_from_fp16(k16)
    v8, vs = fsq.fake_int8_pages_from_fp16(v16)
    tk8, tks = tiq.fake_int8_pages_from_fp16(k16)
    tv8, tvs = tiq.fake_int8_pages_from_fp16(v16)
    pt = torch.randint(0, NP, (B, H, W), generator=g, dtype=torch.int32)
    pc = torch.randint(0, W + 1, (B, H), generator=g, dtype=torch.int32)
    pc[0, 0] = W
    prec = torch.tensor([0, 1, 2, 0, 1, 1, 0, 2], dtype=torch.int32)
    cfg = fsq.FusedDecodeConfig(page_size=PS, head_dim=D, max_selected_pages=W)
    out = fsq.fused_selected_quant_decode_reference(q, k16, v16, k8, v8, ks, vs, pt, prec, pc, cfg)
    out_t = fsq.fused_selected_quant_decode_reference(q, k16, v16, tk8, tv8, tks, tvs, pt, prec, pc, cfg)
    # fake_int8 on an all-zero page and on a page of exact ties
    z = torch.zeros(2, PS, D).half()
    z[1] = (torch.arange(PS * D).reshape(PS, D) % 9 - 4).half() * 0.5
    zq, zs = fsq.fake_int8_pages_from_fp16(z)
    tzq, tzs = tiq.fake_int8_pages_from_fp16(z)
    _save("g3_fused_decode.npz", q=_np(q), k16=_np(k16), v16=_np(v16), k8=_np(k8), v8=_np(v8),
          ks=_np(ks), vs=_np(vs), tk8=_np(tk8), tv8=_np(tv8), tks=_np(tks), tvs=_np(tvs),
          page_table=_np(pt), page_counts=_np(pc), page_precision=_np(prec),
          out=_np(out), out_triton_scales=_np(out_t),
          edge_pages=_np(z), edge_q=_np(zq), edge_s=_np(zs), edge_tq=_np(tzq), edge_ts=_np(tzs))


# --------------------------------------------------------------------------- #
# G4: intent_quant_attention_reference
# --------------------------------------------------------------------------- #

class _PlanQuantizer:
    """Duck-typed quantizer: a fixed precision per block name."""

    def __init__(self, plan):
        self.plan = plan

    def assign_block_precision(self, block):
        return iq.QuantPolicy(self.plan[block.name])


def g4() -> None:
    g = torch.Generator().manual_seed(4004)
    P, S = bm.BlockPolicy, bm.SemanticBlock
    out = {}
    # cfg1 shape: B1, H8, D64, 1024 tokens = 64 pages; selection per the config
    B, H, D, T = 1, 8, 64, 1024
    q = torch.randn(B, H, 1, D, generator=g).half().float()
    k = torch.randn(B, H, T, D, generator=g).half().float()
    v = torch.randn(B, H, T, D, generator=g).half().float()
    mid = torch.randperm(52, generator=g)[:20].sort().values + 4
    pages = list(range(4)) + [int(p) for p in mid] + list(range(56, 64))
    blocks, plan = [], {}
    for rank, p in enumerate(pages):
        pol = P.ALWAYS if p < 4 else (P.RECENT if p >= 56 else P.ATTEND)
        name = f"p{p}"
        blocks.append(S(name, p * 16, p * 16 + 16, pol, score=0.9 if pol == P.ATTEND else None))
        plan[name] = iq.KVPrecision.FP16 if rank % 2 == 0 else iq.KVPrecision.INT8
    layout = bm.BlockLayout(blocks)
    res = iqa.intent_quant_attention_reference(q, k, v, layout, _PlanQuantizer(plan))
    # only the selected pages' tokens are stored (the rest cannot affect the output)
    tok = torch.tensor([p * 16 + t for p in pages for t in range(16)])
    out.update(cfg1_q=_np(q.half()), cfg1_k_sel=_np(k[:, :, tok].half()),  # exact: fp16 values
               cfg1_v_sel=_np(v[:, :, tok].half()), cfg1_pages=np.array(pages),
               cfg1_out=_np(res))
    # mixed plan with every precision, fp32 inputs, default-policy quantizer too
    B, H, D, T = 1, 2, 32, 96
    q = torch.randn(B, H, 3, D, generator=g)
    k = torch.randn(B, H, T, D, generator=g)
    v = torch.randn(B, H, T, D, generator=g)
    layout = bm.BlockLayout([S("a", 0, 16, P.ALWAYS), S("b", 16, 40, P.ATTEND, score=0.5),
                             S("c", 40, 56, P.ATTEND, score=0.1), S("d", 56, 80, P.RECENT),
                             S("e", 80, 96, P.SKIP)])
    plan = {"a": iq.KVPrecision.FP8, "b": iq.KVPrecision.INT4_RESIDUAL, "c": iq.KVPrecision.SKIP,
            "d": iq.KVPrecision.INT4}
    res = iqa.intent_quant_attention_reference(q, k, v, layout, _PlanQuantizer(plan))
    res2 = iqa.intent_quant_attention_reference(q, k, v, layout, iq.IntentQuantizer(memory_pressure=0.5))
    out.update(mix_q=_np(q), mix_k=_np(k), mix_v=_np(v), mix_out=_np(res), mix_out_default=_np(res2))
    _save("g4_intent_quant_attention.npz", **out)


# --------------------------------------------------------------------------- #
# G5: _mla_decode_cpu
# --------------------------------------------------------------------------- #

def g5() -> None:
    g = torch.Generator().manual_seed(5005)
    batch, q_len, d_c, d_out, ps = 2, 3, 48, 40, 8
    qa = torch.randn(batch, q_len, d_c, generator=g)
    C = torch.randn(6 * ps, d_c, generator=g)
    W = torch.randn(d_c, d_out, generator=g)
    pt = torch.tensor([4, 0, 5, 2], dtype=torch.int32)
    out = tmd._mla_decode_cpu(qa, C, W, pt, page_size=ps)
    out_empty = tmd._mla_decode_cpu(qa, C, W, torch.tensor([], dtype=torch.int32), page_size=ps)
    _save("g5_mla_decode.npz", q_absorb=_np(qa), C=_np(C), W_VO=_np(W), page_table=_np(pt),
          page_size=np.array(ps), out=_np(out), out_empty=_np(out_empty))


# --------------------------------------------------------------------------- #
# G6: KVMemoryManager INT8 transcoding (write_page, _read_page_data, set_page_format)
# --------------------------------------------------------------------------- #

def g6() -> None:
    g = torch.Generator().manual_seed(6006)
    out = {}
    for si, (ps, d) in enumerate(((16, 64), (16, 128), (8, 48))):
        n = 7
        pages = torch.randn(n, ps, d, generator=g)
        pages[1] *= 1e-3                           # small values
        pages[2, 0, 0] = 60000.0                   # near the top of float16
        pages[3] = 0.0                             # all zero: scale 1.0
        pages[4] = torch.round(pages[4] * 8) / 8   # exact eighths: ties after scaling
        pages[5] *= 3e-6                           # float16 subnormals
        pages[6] = torch.round(pages[6] * 127) / 127 * 3.0
        x16 = pages.half()
        mgr = kvm.KVMemoryManager(num_pages=n, page_size=ps, head_dim=d)
        ids = mgr.allocate_pages("blk", "ATTEND", n, score=0.1)   # attend_low_format: INT8
        codes, scales, promoted, codes2, scales2, fp16_back = [], [], [], [], [], []
        for i, pid in enumerate(ids):
            mgr.write_page(pid, x16[i])                              # demote (write as INT8)
            st = mgr.pages[pid]
            codes.append(_np(st.kv_int8.clone()))
            scales.append(st.kv_int8_scale)
            promoted.append(_np(mgr._read_page_data(pid)))          # promote arithmetic
            mgr.set_page_format(pid, kvm.PageStorageFormat.FP16)     # INT8 -> FP16 transcode
            fp16_back.append(_np(mgr.pages[pid].kv_fp16.clone()))
            mgr.set_page_format(pid, kvm.PageStorageFormat.INT8)     # FP16 -> INT8 transcode
            codes2.append(_np(mgr.pages[pid].kv_int8.clone()))
            scales2.append(mgr.pages[pid].kv_int8_scale)
        out.update({f"s{si}_x": _np(x16), f"s{si}_codes": np.stack(codes), f"s{si}_scale": np.array(scales),
                    f"s{si}_promoted": np.stack(promoted), f"s{si}_fp16_back": np.stack(fp16_back),
                    f"s{si}_codes2": np.stack(codes2), f"s{si}_scale2": np.array(scales2)})
    _save("g6_kv_transcode.npz", **out)


if __name__ == "__main__":
    torch.set_num_threads(1)
    which = sys.argv[1:] or ["g1", "g2", "g3", "g4", "g5", "g6"]
    for w in which:
        globals()[w]()
