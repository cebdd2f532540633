"""Test helper: seeded mixed-precision page pools built with the oracle.

Pages are float16 N(0, 1) (K optionally with 8-sigma outliers); each page gets
one precision; codes and scales come from the oracle's page-granule quantiser
(the reference's fake_quantize_tensor arithmetic), so the GPU kernel is fed
exactly the codes the reference would produce.
"""
from __future__ import annotations

import numpy as np

from oracle import decode as Dm
from oracle import quant as Q

TAGS = {"FP16": Dm.FP16, "INT8": Dm.INT8, "SKIP": Dm.SKIP, "FP8": Dm.FP8, "INT4": Dm.INT4,
        "INT4_RESIDUAL": Dm.INT4_RESIDUAL}


def build_pools(rng: np.random.Generator, num_pages: int, D: int, tags: np.ndarray, *,
                outliers: float = 0.0, int4_group: int = 32, scale_f32: bool = False, v_scale: float = 1.0):
    """numpy pools dict in the layout ``oracle.decode.dequant_page`` reads
    (V values N(0, v_scale^2), rounded to float16; ``v_scale`` may be one
    value per page)."""
    PS = 16
    k = rng.standard_normal((num_pages, PS, D)).astype(np.float16)
    vsc = np.asarray(v_scale, np.float64).reshape(-1, 1, 1) if np.ndim(v_scale) else v_scale
    v = (rng.standard_normal((num_pages, PS, D)) * vsc).astype(np.float16)
    if outliers > 0:
        m = rng.random(k.shape) < outliers
        k = np.where(m, (8.0 * np.sign(k.astype(np.float32))).astype(np.float16), k)
    pools = {"k_fp16": k, "v_fp16": v}
    sdt = np.float32 if scale_f32 else np.float16
    for w, src in (("k", k), ("v", v)):
        fp8 = np.zeros((num_pages, PS, D), np.uint8)
        fp8s = np.zeros(num_pages, sdt)
        i8 = np.zeros((num_pages, PS, D), np.int8)
        i8s = np.zeros(num_pages, sdt)
        i4 = np.full((num_pages, PS, D // 2), 0x88, np.uint8)
        i4s = np.zeros((num_pages, D // int4_group), sdt)
        i4r = np.full((num_pages, PS, D), 0x88, np.uint8)
        i4rs = np.zeros((num_pages, 2), np.float32)
        for p in range(num_pages):
            t = int(tags[p])
            if t == Dm.FP8:
                c, s = Q.quantize_page(src[p], "FP8")
                fp8[p], fp8s[p] = c, s[0]
            elif t == Dm.INT8:
                c, s = Q.quantize_page(src[p], "INT8")
                i8[p], i8s[p] = c, s[0]
            elif t == Dm.INT4:
                c, s = Q.quantize_page(src[p], "INT4", int4_group)
                i4[p], i4s[p] = Q.pack_int4(c), s
            elif t == Dm.INT4_RESIDUAL:
                (q1, q2), (s1, s2) = Q.quantize_page(src[p], "INT4_RESIDUAL")
                i4r[p] = Q.pack_int4_residual(q1, q2)
                i4rs[p] = (s1[0], s2[0])
        pools.update({f"{w}_fp8": fp8, f"{w}_fp8_scale": fp8s, f"{w}_i8": i8, f"{w}_i8_scale": i8s,
                      f"{w}_i4": i4, f"{w}_i4_scale": i4s, f"{w}_i4r": i4r, f"{w}_i4r_scale": i4rs})
    return pools


def to_device_pools(pools, device, int4_group: int = 32):
    """numpy pools -> intent_attention.PagePools on ``device``."""
    import torch
    from intent_attention import PagePools

    def t(x):
        return torch.from_numpy(np.ascontiguousarray(x)).to(device)

    return PagePools(
        k_fp16=t(pools["k_fp16"]), v_fp16=t(pools["v_fp16"]),
        k_fp8=t(pools["k_fp8"]), v_fp8=t(pools["v_fp8"]),
        k_fp8_scale=t(pools["k_fp8_scale"]), v_fp8_scale=t(pools["v_fp8_scale"]),
        k_int8=t(pools["k_i8"]), v_int8=t(pools["v_i8"]),
        k_int8_scale=t(pools["k_i8_scale"]), v_int8_scale=t(pools["v_i8_scale"]),
        k_int4=t(pools["k_i4"]), v_int4=t(pools["v_i4"]),
        k_int4_scale=t(pools["k_i4_scale"]), v_int4_scale=t(pools["v_i4_scale"]), int4_group=int4_group,
        k_int4r=t(pools["k_i4r"]), v_int4r=t(pools["v_i4r"]),
        k_int4r_scale=t(pools["k_i4r_scale"]), v_int4r_scale=t(pools["v_i4r_scale"]))


def random_case(seed: int, B: int, Hq: int, Hkv: int, D: int, NP: int, W: int, mix=None, *,
                outliers: float = 0.0, q_scale: float = 1.0, scale_f32: bool = False, v_scale: float = 1.0):
    """(q, pools, table, counts, tags) with a seeded mixed-precision setup."""
    rng = np.random.default_rng(seed)
    names = list(mix or {"FP16": 1.0})
    probs = np.array([mix[n] for n in names] if mix else [1.0])
    tags = np.array([TAGS[n] for n in rng.choice(names, size=NP, p=probs / probs.sum())], np.int32)
    pools = build_pools(rng, NP, D, tags, outliers=outliers, scale_f32=scale_f32, v_scale=v_scale)
    table = rng.integers(0, NP, size=(B, Hkv, W)).astype(np.int32)
    counts = rng.integers(0, W + 1, size=(B, Hkv)).astype(np.int32)
    counts.flat[0] = W
    q = (rng.standard_normal((B, Hq, D)) * q_scale).astype(np.float16)
    return q, pools, table, counts, tags
