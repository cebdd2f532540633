"""CPU-baseline jobs timed by bench.py (test infrastructure: the oracle on the host).

Each job builds synthetic host inputs of one benchmark configuration and runs
the oracle on as many units of it as fit in a time budget, with one BLAS
thread. The inputs are random codes of the configuration's precision mix and
shapes: the oracle's work does not depend on the values, only on shapes and
precisions, so the host does not copy the GPU's pools. bench.py runs one job
in its own process (the 1-thread figure) and one job per core in spawned
processes (the all-core figure: independent units decoded concurrently).

Jobs return ``(units, seconds)``. Units: one (batch, KV head) row of a decode
configuration, one MLA sequence of cfg5, one page of the quantise-on-write
leg, one step of cfg1, one page demoted and promoted for the transcoding leg.
"""
from __future__ import annotations

import time
from typing import Dict, Tuple

import numpy as np

from . import decode as Dm
from . import quant as Q

FP16, INT8, SKIP, FP8, INT4, INT4_RESIDUAL = Dm.FP16, Dm.INT8, Dm.SKIP, Dm.FP8, Dm.INT4, Dm.INT4_RESIDUAL

# per (batch, KV head) row: query heads G, head_dim D, selected pages W, precision mix
DECODE_ROWS = {
    "cfg2": dict(G=4, D=128, W=1024, mix={FP16: 1.0}),
    "cfg3": dict(G=4, D=128, W=1638, mix={FP16: .25, FP8: .25, INT8: .30, INT4: .20}),
    "cfg4": dict(G=4, D=128, W=1228, mix={FP16: .10, INT8: .30, INT4_RESIDUAL: .60}),
}


def _limit_threads():
    from threadpoolctl import threadpool_limits
    return threadpool_limits(limits=1)


def _fp8_codes(rng, shape):
    """Random finite e4m3fn codes (never the NaN codes 0x7F / 0xFF)."""
    return (rng.integers(0, 0x7F, size=shape) | (rng.integers(0, 2, size=shape) << 7)).astype(np.uint8)


def _nibble_bytes(rng, shape):
    """Random bytes whose two nibbles are codes + 8 in [1, 15]."""
    return (rng.integers(1, 16, size=shape) | (rng.integers(1, 16, size=shape) << 4)).astype(np.uint8)


def synthetic_row(name: str, seed: int):
    """(q [1, G, D], pools, table [1, 1, W], counts [1, 1], tags [W]) of one row."""
    c = DECODE_ROWS[name]
    G, D, W = c["G"], c["D"], c["W"]
    rng = np.random.default_rng(seed)
    names = list(c["mix"])
    p = np.array([c["mix"][t] for t in names])
    tags = np.array(names, np.int32)[rng.choice(len(names), size=W, p=p / p.sum())]
    pools: Dict[str, np.ndarray] = {}
    for w in ("k", "v"):
        pools[f"{w}_fp16"] = rng.standard_normal((W, 16, D)).astype(np.float16)
        pools[f"{w}_fp8"] = _fp8_codes(rng, (W, 16, D))
        pools[f"{w}_fp8_scale"] = np.full(W, 0.03, np.float16)
        pools[f"{w}_i8"] = rng.integers(-127, 128, size=(W, 16, D)).astype(np.int8)
        pools[f"{w}_i8_scale"] = np.full(W, 0.03, np.float16)
        pools[f"{w}_i4"] = _nibble_bytes(rng, (W, 16, D // 2))
        pools[f"{w}_i4_scale"] = np.full((W, D // 32), 0.03, np.float16)
        pools[f"{w}_i4r"] = _nibble_bytes(rng, (W, 16, D))
        pools[f"{w}_i4r_scale"] = np.tile(np.array([[0.03, 0.002]], np.float32), (W, 1))
    q = (rng.standard_normal((1, G, D)) / np.sqrt(D)).astype(np.float16)
    table = np.arange(W, dtype=np.int32).reshape(1, 1, W)
    counts = np.array([[W]], np.int32)
    return q, pools, table, counts, tags


def decode_job(name: str, seed: int, budget_s: float) -> Tuple[int, float]:
    """Rows of a decode configuration through paged_decode_oracle (float32)."""
    q, pools, table, counts, tags = synthetic_row(name, seed)
    done, t0 = 0, time.perf_counter()
    with _limit_threads():
        while done == 0 or time.perf_counter() - t0 < budget_s:
            Dm.paged_decode_oracle(q, pools, table, counts, tags, dtype=np.float32)
            done += 1
    return done, time.perf_counter() - t0


def mla_job(seed: int, budget_s: float, H: int = 128, DQK: int = 576, DV: int = 512,
            W: int = 512) -> Tuple[int, float]:
    """cfg5 sequences (128 heads over 512 latent pages, FP8 / INT8) through
    mla_paged_decode_oracle."""
    from .mla import mla_paged_decode_oracle
    rng = np.random.default_rng(seed)
    tags = np.where(rng.random(W) < 0.5, FP8, INT8).astype(np.int32)
    pools = {"c_fp8": _fp8_codes(rng, (W, 16, DQK)), "c_fp8_scale": np.full(W, 0.03, np.float16),
             "c_i8": rng.integers(-127, 128, size=(W, 16, DQK)).astype(np.int8),
             "c_i8_scale": np.full(W, 0.03, np.float16)}
    q = rng.standard_normal((1, H, DQK)).astype(np.float16)
    table = np.arange(W, dtype=np.int32).reshape(1, W)
    done, t0 = 0, time.perf_counter()
    with _limit_threads():
        while done == 0 or time.perf_counter() - t0 < budget_s:
            mla_paged_decode_oracle(q, pools, table, np.array([W]), tags, v_dim=DV)
            done += 1
    return done, time.perf_counter() - t0


QUANT_MIX = (("FP8", .25), ("INT8", .30), ("INT4", .20))


def quantize_job(seed: int, budget_s: float, D: int = 128) -> Tuple[int, float]:
    """Pages of the quantise-on-write leg through quant.quantize_page, round
    robin over K and V of the three precisions (weighted like the cfg3 pools)."""
    rng = np.random.default_rng(seed)
    pages = rng.standard_normal((64, 16, D)).astype(np.float16)
    order = [n for n, f in QUANT_MIX for _ in range(int(round(f * 20)))]
    done, t0 = 0, time.perf_counter()
    with _limit_threads():
        while done == 0 or time.perf_counter() - t0 < budget_s:
            Q.quantize_page(pages[done % 64], order[done % len(order)], 32)
            done += 1
    return done, time.perf_counter() - t0


def transcode_job(seed: int, budget_s: float, D: int = 128) -> Tuple[int, float]:
    """Pages of the KV memory manager's transcoding leg: one unit is a 16 x D
    float16 page demoted to INT8 (memory.demote_int8) and promoted back
    (memory.promote_fp16)."""
    from . import memory as M
    rng = np.random.default_rng(seed)
    pages = rng.standard_normal((64, 16, D)).astype(np.float16)
    done, t0 = 0, time.perf_counter()
    with _limit_threads():
        while done == 0 or time.perf_counter() - t0 < budget_s:
            codes, s = M.demote_int8(pages[done % 64])
            M.promote_fp16(codes, s)
            done += 1
    return done, time.perf_counter() - t0


def _cfg1_pages(rng):
    return sorted([0, 1, 2, 3] + [int(p) for p in rng.permutation(52)[:20] + 4] + list(range(56, 64)))


def cfg1_step(seed: int, which: str = "loop"):
    """A no-argument callable running one cfg1 step (B1, 8 heads, D64, 32 of 64
    pages alternating FP16 / INT8 by ascending page id) on synthetic inputs:
    ``loop``: fused_decode_reference_loop, the reference's per-(b, h, page)
    loop; ``vector``: paged_decode_oracle in float32; ``iqa``:
    intent_quant_attention_reference's restatement (per step, every selected
    16-token block fake-quantised with per-channel scales and dequantised,
    then dense attention on float32-carried float16 inputs)."""
    rng = np.random.default_rng(seed)
    H, D, P = 8, 64, 64
    pages = _cfg1_pages(rng)
    if which == "iqa":
        from . import attention as A
        from . import policy as Pol
        q = rng.standard_normal((1, H, 1, D)).astype(np.float16).astype(np.float32)
        k = rng.standard_normal((1, H, P * 16, D)).astype(np.float16).astype(np.float32)
        v = rng.standard_normal((1, H, P * 16, D)).astype(np.float16).astype(np.float32)
        blocks, plan = [], {}
        for r, p in enumerate(pages):
            pol = "ALWAYS" if p < 4 else ("RECENT" if p >= 56 else "ATTEND")
            blocks.append(Pol.SemanticBlock(f"p{p}", p * 16, p * 16 + 16, pol, 0.9 if pol == "ATTEND" else None))
            plan[f"p{p}"] = "FP16" if r % 2 == 0 else "INT8"

        class Plan:
            def assign_block_precision(self, block):
                return Pol.QuantPolicy(plan[block.name])

        layout, quantizer = Pol.BlockLayout(blocks), Plan()
        return lambda: A.intent_quant_attention_reference(q, k, v, layout, quantizer, exact=False)
    k = rng.standard_normal((H * P, 16, D)).astype(np.float16)
    v = rng.standard_normal((H * P, 16, D)).astype(np.float16)
    k8, ks = Q.fake_int8_pages_fused(k)
    v8, vs = Q.fake_int8_pages_fused(v)
    table = np.array([[[h * P + p for p in pages] for h in range(H)]], np.int32)
    prec = np.zeros(H * P, np.int32)
    for r, p in enumerate(pages):
        prec[[h * P + p for h in range(H)]] = 0 if r % 2 == 0 else 1
    counts = np.full((1, H), len(pages), np.int32)
    q = rng.standard_normal((1, H, 1, D)).astype(np.float16)
    if which == "loop":
        return lambda: Dm.fused_decode_reference_loop(q, k, v, k8, v8, ks, vs, table, prec, counts, D)
    pools = {"k_fp16": k, "v_fp16": v, "k_i8": k8, "v_i8": v8, "k_i8_scale": ks, "v_i8_scale": vs}
    return lambda: Dm.paged_decode_oracle(q[:, :, 0, :], pools, table, counts, prec, dtype=np.float32)


def cfg1_job(which: str, seed: int, budget_s: float) -> Tuple[int, float]:
    """cfg1 steps of one path (see cfg1_step) within the budget."""
    step = cfg1_step(seed, which)
    done, t0 = 0, time.perf_counter()
    with _limit_threads():
        while done == 0 or time.perf_counter() - t0 < budget_s:
            step()
            done += 1
    return done, time.perf_counter() - t0


def tables_job(spec_path: str, seed: int, budget_s: float) -> Tuple[int, float]:
    """Full page-table builds of the cfg3-tables leg through
    policy.build_page_tables_oracle (the routing -> kernel-tensor loops);
    ``spec_path``: an .npz bench.py writes with the routed spans and block
    table of its workload."""
    import json

    from . import policy as P
    z = np.load(spec_path, allow_pickle=False)
    lists = [[tuple(s) for s in row] for row in json.loads(str(z["lists"]))]
    R, W, PS, NP, Hkv = (int(z[k]) for k in ("R", "W", "PS", "NP", "Hkv"))
    bt = z["block_table"]
    done, t0 = 0, time.perf_counter()
    while done == 0 or time.perf_counter() - t0 < budget_s:
        P.build_page_tables_oracle(lists, R, W, PS, NP, rows_per_seq=1, rows_per_list=Hkv, block_table=bt)
        done += 1
    return done, time.perf_counter() - t0


JOBS = {"decode": decode_job, "mla": mla_job, "quantize": quantize_job, "cfg1": cfg1_job, "tables": tables_job,
        "transcode": transcode_job}


def _run(args):
    job, extra, seed, budget = args
    return JOBS[job](*extra, seed, budget)


def main(argv=None) -> None:
    """``python -m oracle.baseline JOB [ARG ...] --workers N --budget S``: the
    job once in this process (one thread), then N copies at once in forked
    worker processes (this process never touches a GPU); prints one JSON line
    with units and seconds of both."""
    import argparse
    import json
    import multiprocessing as mp
    ap = argparse.ArgumentParser()
    ap.add_argument("job", choices=sorted(JOBS))
    ap.add_argument("extra", nargs="*")
    ap.add_argument("--workers", type=int, default=1)
    ap.add_argument("--budget", type=float, default=8.0)
    a = ap.parse_args(argv)
    n1, s1 = _run((a.job, a.extra, 0, a.budget))
    res = {"job": a.job, "threads_1": {"units": n1, "seconds": s1, "units_per_s": n1 / s1}}
    if a.workers > 1:
        with mp.get_context("fork").Pool(a.workers) as pool:
            t0 = time.perf_counter()
            outs = pool.map(_run, [(a.job, a.extra, i + 1, a.budget) for i in range(a.workers)])
            wall = time.perf_counter() - t0
        units = sum(n for n, _ in outs)
        span = max(s for _, s in outs)
        res["threads_all"] = {"workers": a.workers, "units": units, "seconds": span, "wall_s": wall,
                              "units_per_s": units / span}
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()


def cfg1_protocol(seed: int = 0, warmup: int = 3, iters: int = 100) -> Dict[str, Dict[str, float]]:
    """cfg1 CPU paths timed per iteration (3 warm-up, 100 timed, one thread):
    the loop-faithful restatement of fused_selected_quant_decode_reference, the
    intent_quant_attention_reference-shaped path (per-step fake quant ->
    dequant -> dense) and the vectorised oracle; median / p10 / p90 in us."""
    out = {}
    with _limit_threads():
        for name, which in (("loop_faithful", "loop"), ("iqa_reference", "iqa"), ("vectorised", "vector")):
            step = cfg1_step(seed, which)
            ts = []
            for i in range(warmup + iters):
                t0 = time.perf_counter()
                step()
                if i >= warmup:
                    ts.append((time.perf_counter() - t0) * 1e6)
            ts.sort()
            out[name] = {"median_us": ts[len(ts) // 2], "p10_us": ts[len(ts) // 10],
                         "p90_us": ts[(9 * len(ts)) // 10], "iters": iters}
    return out
