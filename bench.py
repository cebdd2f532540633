"""Decode-step benchmark of the MI355X selected-quant paged decode.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config cfg3]

Workload (default ``cfg3``, the configuration the headline metric is quoted
on): Llama-3-8B GQA decode, batch 32, 32 query / 8 KV heads, head_dim 128,
65536-token context per sequence in 16-token pages (4096 pages per sequence
and KV head, 1,048,576 physical pages), 40 % of pages selected uniformly at
random (1638 per sequence and KV head), physical page table a random
permutation. Per-page precision at random: 25 % FP16, 25 % FP8-e4m3, 30 %
INT8, 20 % INT4 (two codes per byte, one scale per page, KV head and
32-channel group). K/V float16 N(0, 1) with 1 % of K elements set to 8*sign;
Q N(0, 1)/sqrt(128). Codes and scales are the reference's fake-quant
arithmetic (absmax/127 in float16, round half even), computed on the GPU with
torch ops; tests check them bit-exact against the oracle.

A step is one decode of the whole batch (split kernel + merge kernel) with
every input already in HBM; the 2 GB the step reads exceed the 256 MB
Infinity Cache, so consecutive steps do not hit in it (cfg4, whose step reads
178 MB, rotates four page tables with disjoint selections; cfg5 four page
sets). Timing: HIP events on
the stream the kernels run on, around the K back-to-back timed steps. A second
pass of K steps records events around each step (the p10/p50/p90 spread) and,
through iak_paged_decode_timed, around the split kernel alone: its average
duration is the denominator of ``roofline.achieved`` (the split kernel's
algorithmic bytes, all but the output the merge writes). ``value`` is the
achieved algorithmic bandwidth of the whole step (bytes the step must read and
write / step time). The CPU baseline times the test oracle (numpy, one thread)
on a bounded sample of rows of the same workload.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "intent-attention-kernel_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402
import torch  # noqa: E402

METRIC = ("decode-attn µs/step + achieved HBM GB/s (% of peak), Llama-3-8B GQA, 64k ctx, mixed")
HBM_PEAK_GBPS = 8000.0
PS = 16

TAG_FP16, TAG_INT8, TAG_SKIP, TAG_FP8, TAG_INT4, TAG_INT4R = 0, 1, 2, 3, 4, 5

CONFIGS = {
    # name: B, Hq, Hkv, D, tokens, selected fraction or count, precision mix, outlier frac, q scale
    "cfg2": dict(B=16, Hq=32, Hkv=8, D=128, T=32768, sel="cfg2", mix={TAG_FP16: 1.0}, outliers=0.0,
                 q_scale=1 / math.sqrt(128)),
    "cfg3": dict(B=32, Hq=32, Hkv=8, D=128, T=65536, sel=0.40,
                 mix={TAG_FP16: .25, TAG_FP8: .25, TAG_INT8: .30, TAG_INT4: .20}, outliers=0.01,
                 q_scale=1 / math.sqrt(128)),
    # a cfg4 step reads 178 MB, which the 256 MB Infinity Cache could hold from one
    # step to the next: four page tables with disjoint selections per (batch, KV
    # head) rotate, so a step's pages were last read three steps (> 500 MB) before
    "cfg4": dict(B=4, Hq=32, Hkv=8, D=128, T=131072, sel=0.15,
                 mix={TAG_FP16: .10, TAG_INT8: .30, TAG_INT4R: .60}, outliers=0.0, q_scale=1.0, sets=4),
    # small all-precision case for tests and smoke runs
    "tiny": dict(B=2, Hq=8, Hkv=2, D=128, T=2048, sel=0.40,
                 mix={TAG_FP16: .2, TAG_FP8: .2, TAG_INT8: .2, TAG_INT4: .2, TAG_INT4R: .2}, outliers=0.01,
                 q_scale=1 / math.sqrt(128)),
}


# cfg1 (the reference's CPU-runnable case): batch 1,
# 8 query / 8 KV heads, head_dim 64, 1024 tokens = 64 pages of 16; the router
# selects 32 pages (0-3 ALWAYS, 56-63 RECENT, 20 drawn from 4-55 as ATTEND);
# selected pages alternate FP16 / INT8 by ascending page id (even rank FP16),
# INT8 with per-page, per-head absmax scales.
CFG1 = dict(B=1, H=8, D=64, T=1024, pages=64, always=4, recent=8, attend=20)


class _PagePlan:
    """Duck-typed quantizer: a fixed precision per block name (the
    alternating plan cfg1 states; the router only calls
    assign_block_precision)."""

    def __init__(self, plan):
        self.plan = plan

    def assign_block_precision(self, block):
        from intent_attention import QuantPolicy
        return QuantPolicy(self.plan[block.name])


def build_cfg1(device: torch.device, seed: int = 1):
    """cfg1 through the reference's routing path on the product API:
    BlockLayout (one block per page) -> BlockRouter.route_layout ->
    routing_to_kernel_metadata -> metadata_to_kernel_tensors, then the pools
    the fused entry point reads. Physical pages are head-major: page (h, p) is
    h * 64 + p, so the broadcast logical table is offset by h * 64 per head."""
    from intent_attention import (BlockLayout, BlockPolicy, BlockRouter, FusedDecodeConfig, KVPrecision,
                                  RouterConfig, SemanticBlock, metadata_to_kernel_tensors,
                                  routing_to_kernel_metadata)
    # the fused module's variant (float16 arithmetic and scales), fused_selected_quant_decode.py:521-542
    from intent_attention.fused_selected_quant_decode import fake_int8_pages_from_fp16
    c = CFG1
    B, H, D, P = c["B"], c["H"], c["D"], c["pages"]
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, 1, D, generator=g).half()
    k = torch.randn(H * P, PS, D, generator=g).half()
    v = torch.randn(H * P, PS, D, generator=g).half()
    mid = (torch.randperm(P - c["always"] - c["recent"], generator=g)[:c["attend"]] + c["always"]).sort().values
    pages = list(range(c["always"])) + [int(p) for p in mid] + list(range(P - c["recent"], P))
    rank = {p: i for i, p in enumerate(pages)}
    blocks, plan = [], {}
    for p in range(P):
        if p < c["always"]:
            pol = BlockPolicy.ALWAYS
        elif p >= P - c["recent"]:
            pol = BlockPolicy.RECENT
        elif p in rank:
            pol = BlockPolicy.ATTEND
        else:
            pol = BlockPolicy.SKIP
        blocks.append(SemanticBlock(f"p{p}", p * PS, (p + 1) * PS, pol, 0.9 if pol == BlockPolicy.ATTEND else None))
        plan[f"p{p}"] = (KVPrecision.SKIP if p not in rank else
                         (KVPrecision.FP16 if rank[p] % 2 == 0 else KVPrecision.INT8))
    router = BlockRouter(RouterConfig(top_k_blocks=c["attend"]), quantizer=_PagePlan(plan))
    routed = router.route_layout(BlockLayout(blocks), c["T"])
    meta = routing_to_kernel_metadata(routed, PS)
    cfg = FusedDecodeConfig(page_size=PS, head_dim=D, max_selected_pages=len(pages))
    table, prec, counts = metadata_to_kernel_tensors(meta, P, B, H, cfg, device=device)
    table = (table + (torch.arange(H, device=device, dtype=torch.int32) * P)[None, :, None]).contiguous()
    prec = prec.repeat(H).contiguous()
    k, v, q = k.to(device), v.to(device), q.to(device)
    k8, ks = fake_int8_pages_from_fp16(k)
    v8, vs = fake_int8_pages_from_fp16(v)
    return dict(name="cfg1", cfg=cfg, q=q, k16=k, v16=v, k8=k8, v8=v8, ks=ks, vs=vs, table=table, prec=prec,
                counts=counts, pages=pages, meta=meta, plan=plan, layout_blocks=blocks)


def cfg1_args(wl):
    """Positional arguments of fused_selected_quant_decode for a cfg1 workload."""
    return (wl["q"], wl["k16"], wl["v16"], wl["k8"], wl["v8"], wl["ks"], wl["vs"], wl["table"], wl["prec"],
            wl["counts"], wl["cfg"])


# --------------------------------------------------------------------------- #
# Quantisation of synthetic pages (reference arithmetic, torch ops on device)
# --------------------------------------------------------------------------- #

def _div127(x: torch.Tensor) -> torch.Tensor:
    # a tensor divisor keeps a true division on GPU tensors
    return x / torch.full((1,), 127.0, dtype=x.dtype, device=x.device)


def quantize_pages(x: torch.Tensor, tag: int, group: int = 32):
    """x [n, 16, D] float16 -> (codes, scales) in the kernel's storage format.

    FP8 / INT8 / INT4_RESIDUAL: one scale per page; INT4: one per ``group``
    channels. float16 arithmetic as fake_quantize_tensor on float16 input.
    """
    n, ps, D = x.shape
    if tag in (TAG_FP8, TAG_INT8, TAG_INT4R):
        flat = x.reshape(n, -1)
        scale = _div127(flat.abs().amax(dim=1, keepdim=True)).clamp(min=1e-8)
        y = flat / scale
        if tag == TAG_FP8:
            codes = y.to(torch.float8_e4m3fn).view(torch.uint8)
            return codes.reshape(n, ps, D), scale.reshape(n)
        if tag == TAG_INT8:
            return y.clamp(-127, 127).round().to(torch.int8).reshape(n, ps, D), scale.reshape(n)
        q1 = y.clamp(-7, 7).round()
        base = q1.float() * scale.float()
        resid = flat.float() - base
        s2 = (resid.abs().amax(dim=1, keepdim=True) / torch.full((1,), 127.0, device=x.device)).clamp(min=1e-8)
        q2 = (resid / s2).clamp(-7, 7).round()
        packed = ((q1.to(torch.int16) + 8) | ((q2.to(torch.int16) + 8) << 4)).to(torch.uint8)
        return packed.reshape(n, ps, D), torch.stack([scale.float().reshape(n), s2.reshape(n)], dim=1)
    if tag == TAG_INT4:
        g = x.reshape(n, ps, D // group, group)
        scale = _div127(g.abs().amax(dim=(1, 3), keepdim=True)).clamp(min=1e-8)
        codes = (g / scale).clamp(-7, 7).round().to(torch.int16).reshape(n, ps, D) + 8
        packed = (codes[..., 0::2] | (codes[..., 1::2] << 4)).to(torch.uint8)
        return packed, scale.reshape(n, D // group)
    raise ValueError(tag)


# --------------------------------------------------------------------------- #
# Workload
# --------------------------------------------------------------------------- #

def build_workload(name: str, device: torch.device, seed: int = 1234, chunk_pages: int = 65536):
    from intent_attention import PagePools
    cfg = CONFIGS[name]
    B, Hq, Hkv, D, T = cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["D"], cfg["T"]
    P = T // PS
    NP = B * Hkv * P
    g = torch.Generator(device=device).manual_seed(seed)
    gc = torch.Generator().manual_seed(seed)

    # per-physical-page precision
    tags_list = list(cfg["mix"])
    probs = torch.tensor([cfg["mix"][t] for t in tags_list])
    tag_idx = torch.multinomial(probs, NP, replacement=True, generator=gc)
    tags = torch.tensor(tags_list, dtype=torch.int32)[tag_idx].to(device)

    # page table: random physical permutation; selection per (b, kv head)
    perm = torch.randperm(NP, generator=gc).to(torch.int32).reshape(B * Hkv, P)
    if cfg["sel"] == "cfg2":      # first 64 ALWAYS, last 256 RECENT, 704 random from the middle
        mid = torch.stack([torch.randperm(P - 320, generator=gc)[:704] + 64 for _ in range(B * Hkv)])
        logical = torch.cat([torch.arange(64).expand(B * Hkv, 64), mid.sort(dim=1).values,
                             torch.arange(P - 256, P).expand(B * Hkv, 256)], dim=1)
        logicals = [logical]
    else:
        # `sets` page tables whose selections are disjoint per (batch, KV head)
        nsel = int(cfg["sel"] * P)
        sets = cfg.get("sets", 1)
        assert sets * nsel <= P, "disjoint page sets need sets * selected <= pages"
        orders = [torch.randperm(P, generator=gc) for _ in range(B * Hkv)]
        logicals = [torch.stack([o[k * nsel:(k + 1) * nsel].sort().values for o in orders]) for k in range(sets)]
    tables = [torch.gather(perm, 1, lg).reshape(B, Hkv, -1).contiguous().to(device) for lg in logicals]
    table = tables[0]
    W = table.shape[2]
    counts = torch.full((B, Hkv), W, dtype=torch.int32, device=device)

    pools = PagePools(int4_group=32)
    pools.k_fp16 = torch.empty((NP, PS, D), dtype=torch.float16, device=device)
    pools.v_fp16 = torch.empty((NP, PS, D), dtype=torch.float16, device=device)
    present = set(cfg["mix"])
    if TAG_FP8 in present:
        pools.k_fp8 = torch.zeros((NP, PS, D), dtype=torch.uint8, device=device)
        pools.v_fp8 = torch.zeros_like(pools.k_fp8)
        pools.k_fp8_scale = torch.zeros(NP, dtype=torch.float16, device=device)
        pools.v_fp8_scale = torch.zeros_like(pools.k_fp8_scale)
    if TAG_INT8 in present:
        pools.k_int8 = torch.zeros((NP, PS, D), dtype=torch.int8, device=device)
        pools.v_int8 = torch.zeros_like(pools.k_int8)
        pools.k_int8_scale = torch.zeros(NP, dtype=torch.float16, device=device)
        pools.v_int8_scale = torch.zeros_like(pools.k_int8_scale)
    if TAG_INT4 in present:
        pools.k_int4 = torch.full((NP, PS, D // 2), 0x88, dtype=torch.uint8, device=device)
        pools.v_int4 = torch.full_like(pools.k_int4, 0x88)
        pools.k_int4_scale = torch.zeros((NP, D // 32), dtype=torch.float16, device=device)
        pools.v_int4_scale = torch.zeros_like(pools.k_int4_scale)
    if TAG_INT4R in present:
        pools.k_int4r = torch.full((NP, PS, D), 0x88, dtype=torch.uint8, device=device)
        pools.v_int4r = torch.full_like(pools.k_int4r, 0x88)
        pools.k_int4r_scale = torch.zeros((NP, 2), dtype=torch.float32, device=device)
        pools.v_int4r_scale = torch.zeros_like(pools.k_int4r_scale)

    dest = {TAG_FP8: ("fp8", "fp8_scale"), TAG_INT8: ("int8", "int8_scale"), TAG_INT4: ("int4", "int4_scale"),
            TAG_INT4R: ("int4r", "int4r_scale")}
    for lo in range(0, NP, chunk_pages):
        hi = min(NP, lo + chunk_pages)
        for w in ("k", "v"):
            x = torch.randn((hi - lo, PS, D), generator=g, device=device, dtype=torch.float32)
            if w == "k" and cfg["outliers"] > 0:
                m = torch.rand(x.shape, generator=g, device=device) < cfg["outliers"]
                x = torch.where(m, 8.0 * torch.sign(x), x)
            x = x.half()
            getattr(pools, f"{w}_fp16")[lo:hi] = x
            t = tags[lo:hi]
            for tag, (pool, sc) in dest.items():
                if tag not in present:
                    continue
                idx = torch.nonzero(t == tag).flatten()
                if idx.numel() == 0:
                    continue
                codes, scales = quantize_pages(x[idx], tag)
                getattr(pools, f"{w}_{pool}")[lo + idx] = codes
                getattr(pools, f"{w}_{sc}")[lo + idx] = scales.to(getattr(pools, f"{w}_{sc}").dtype)
    q = (torch.randn((B, Hq, D), generator=g, device=device) * cfg["q_scale"]).half()
    return dict(cfg=cfg, name=name, q=q, pools=pools, table=table, tables=tables, counts=counts, tags=tags, NP=NP,
                W=W)


# HBM bytes per decode-kernel launch (reads + writes) from rocprofv3 FETCH_SIZE /
# WRITE_SIZE runs of this bench, each scaled by what the counter reads for a
# 1 GiB device copy (--calibrate-copy): profiles/paged_decode_cfg3_hbm_traffic.txt and
# profiles/paged_decode_cfg4_kernel_stats.txt. Each figure holds the digest of the
# decode kernel's sources it was measured on (kernel_source_digest); a build whose
# sources differ reports traffic null (stale) until the counters are run again.
MEASURED_TRAFFIC = {
    "cfg3": {"bytes": 2_105_410_636 + 5_054_464, "src": "4a40bfc181a9e975",
             "source": "profiles/paged_decode_cfg3_hbm_traffic.txt"},
    "cfg4": {"bytes": 189_782_173 + 2_129_920, "src": "4a40bfc181a9e975",
             "source": "profiles/paged_decode_cfg4_kernel_stats.txt"},
    # the same decodes reading 32-byte page descriptors (--page-descriptors) or
    # 32-byte entry records (--entry-records)
    "cfg3-desc": {"bytes": 2_080_208_921 + 5_054_464, "src": "4a40bfc181a9e975",
                  "source": "profiles/paged_decode_cfg3_hbm_traffic.txt"},
    "cfg4-desc": {"bytes": 182_747_550 + 2_129_920, "src": "4a40bfc181a9e975",
                  "source": "profiles/paged_decode_cfg4_kernel_stats.txt"},
    "cfg3-records": {"bytes": 2_005_600_819 + 5_054_464, "src": "4a40bfc181a9e975",
                     "source": "profiles/paged_decode_cfg3_hbm_traffic.txt"},
    "cfg4-records": {"bytes": 178_928_491 + 2_129_920, "src": "4a40bfc181a9e975",
                     "source": "profiles/paged_decode_cfg4_kernel_stats.txt"},
}
KERNEL_SOURCES = ("paged_decode.hip", "iak_device.h", "iak_internal.h")
MLA_KERNEL_SOURCES = ("mla_decode.hip", "iak_device.h", "iak_internal.h")


def source_digest(files) -> str:
    """sha256 (first 16 hex digits) of the named csrc source files, in order."""
    import hashlib
    h = hashlib.sha256()
    for f in files:
        with open(os.path.join(ROOT, "intent-attention-kernel_amd", "csrc", f), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


def kernel_source_digest() -> str:
    """Digest of the decode kernel's source files (profiles/ summaries name it)."""
    return source_digest(KERNEL_SOURCES)


def mla_source_digest() -> str:
    """Digest of the MLA kernel's source files (profiles/ summaries name it)."""
    return source_digest(MLA_KERNEL_SOURCES)


def measured_traffic(config: str):
    """(bytes per launch or None, note) for a config under the current kernel sources."""
    m = MEASURED_TRAFFIC.get(config)
    if m is None:
        return None, None
    if m["src"] != kernel_source_digest():
        return None, f"stale: {m['source']} was measured on kernel sources {m['src']}, not {kernel_source_digest()}"
    return m["bytes"], m["source"]


PAGE_BYTES = {  # K+V code bytes and scale bytes per page (D = 128, fp16 scales, INT4 groups of 32)
    TAG_FP16: (2 * PS * 128 * 2, 0), TAG_FP8: (2 * PS * 128, 2 * 2), TAG_INT8: (2 * PS * 128, 2 * 2),
    TAG_INT4: (2 * PS * 64, 2 * 4 * 2), TAG_INT4R: (2 * PS * 128, 2 * 2 * 4), TAG_SKIP: (0, 0),
}


def algorithmic_bytes(wl, table=None) -> dict:
    """Bytes one step must move: each selected page's K+V codes and scales once
    per KV head (GQA shares them), its page-table entry and tag, the counts,
    Q in and O out (for `table`, default the workload's first page table)."""
    tags_sel = wl["tags"][(wl["table"] if table is None else table).long()].flatten()
    n = {t: int((tags_sel == t).sum()) for t in PAGE_BYTES}
    codes = sum(n[t] * PAGE_BYTES[t][0] for t in n)
    scales = sum(n[t] * PAGE_BYTES[t][1] for t in n)
    meta = tags_sel.numel() * (4 + 4) + wl["counts"].numel() * 4
    qo = 2 * wl["q"].numel() * 2
    return dict(total=codes + scales + meta + qo, codes=codes, scales=scales, meta=meta, qo=qo,
                pages=int(tags_sel.numel()), per_tag={str(k): v for k, v in n.items()})


def flops(wl) -> float:
    cfg = wl["cfg"]
    toks = int(wl["tags"][wl["table"].long()].ne(TAG_SKIP).sum()) * PS
    return 4.0 * toks * (cfg["Hq"] // cfg["Hkv"]) * cfg["D"]


# --------------------------------------------------------------------------- #
# CPU baseline: the oracle on a bounded sample of rows
# --------------------------------------------------------------------------- #

CPU_BUDGET_S = 8.0      # seconds of oracle work per CPU leg (one thread, then all cores)
CPU_WORKERS_MAX = 16    # host cores of the GPU box's share


def cpu_info() -> dict:
    """Host CPU model (lscpu, else /proc/cpuinfo), cores this process may use,
    and the worker count of the all-core leg."""
    import subprocess
    model = None
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        model = next((ln.split(":", 1)[1].strip() for ln in out.splitlines() if ln.startswith("Model name")), None)
    except (OSError, subprocess.SubprocessError):
        pass
    if model is None and os.path.exists("/proc/cpuinfo"):
        model = next((ln.split(":", 1)[1].strip() for ln in open("/proc/cpuinfo") if ln.startswith("model name")),
                     None)
    avail = len(os.sched_getaffinity(0))
    return {"cpu_model": model, "cores_available": avail, "workers": min(CPU_WORKERS_MAX, avail)}


def run_cpu_jobs(job: str, *extra, budget_s: float = CPU_BUDGET_S) -> dict:
    """The oracle's CPU job in a child process (python -m oracle.baseline),
    started before this process touches the GPU: one thread, then one job per
    core at once. Returns its JSON plus cpu_info()."""
    import subprocess
    info = cpu_info()
    cmd = [sys.executable, "-m", "oracle.baseline", job, *map(str, extra), "--workers", str(info["workers"]),
           "--budget", str(budget_s)]
    r = subprocess.run(cmd, cwd=ROOT, capture_output=True, text=True, timeout=4 * budget_s + 180)
    if r.returncode != 0:
        raise RuntimeError(f"CPU baseline job {job} failed ({r.returncode}): {r.stderr[-2000:]}")
    res = json.loads(r.stdout.strip().splitlines()[-1])
    res.update(info)
    return res


def cpu_baseline_entry(raw: dict, unit: str, per_unit_value, step_units: int, sample: str, **extra) -> dict:
    """bench.py's cpu_baseline object from a run_cpu_jobs result: ``value`` is
    the all-core figure (``cores`` = workers used), ``threads_1`` the
    one-thread one; ``per_unit_value(units_per_s)`` converts a job rate into
    the leg's unit and a step takes ``step_units`` units."""
    one = raw["threads_1"]["units_per_s"]
    allc = raw.get("threads_all", raw["threads_1"])["units_per_s"]
    workers = raw.get("threads_all", {}).get("workers", 1)
    out = {"value": round(per_unit_value(allc), 4), "unit": unit, "cores": workers, "kind": "port",
           "us_per_step": round(step_units / allc * 1e6, 1),
           "threads_1": {"value": round(per_unit_value(one), 4), "us_per_step": round(step_units / one * 1e6, 1)},
           "cpu_model": raw["cpu_model"], "cores_available": raw["cores_available"],
           "sample": sample}
    out.update(extra)
    return out


def cpu_baseline_decode(name: str, raw: dict, step_bytes: int, rows: int) -> dict:
    return cpu_baseline_entry(
        raw, "GB/s", lambda ups: step_bytes * ups / rows / 1e9, rows,
        f"oracle.decode.paged_decode_oracle (numpy float32, one BLAS thread per process) on synthetic "
        f"{name} rows (random codes of the configuration's shapes and precision mix); one thread "
        f"{raw['threads_1']['units']} rows in {raw['threads_1']['seconds']:.1f} s, all cores "
        f"{raw.get('threads_all', {}).get('units', 0)} rows in {raw.get('threads_all', {}).get('seconds', 0):.1f} s "
        f"over {raw['workers']} processes; scaled to the {rows}-row step")


# --------------------------------------------------------------------------- #
# MLA latent decode (cfg5)
# --------------------------------------------------------------------------- #

MLA_CONFIGS = {
    # DeepSeek-V3-style latent decode: 512 latent + 64 RoPE dims shared by 128 heads,
    # 16,384-token context in 16-token pages, half the pages selected, latent pages
    # half FP8-e4m3 / half INT8 with one scale per page.
    "cfg5": dict(B=32, H=128, DQK=576, DV=512, T=16384, sel=0.5, mix={TAG_FP8: .5, TAG_INT8: .5}),
}
MLA_SETS = 4          # independent page sets rotated per step (4 x 151 MB > 256 MB MALL)
MFMA_F16_PEAK_TFLOPS = 2500.0


def build_mla_workload(name: str, device: torch.device, seed: int = 4321):
    from intent_attention import LatentPools
    cfg = MLA_CONFIGS[name]
    B, H, DQK, T = cfg["B"], cfg["H"], cfg["DQK"], cfg["T"]
    P = T // PS
    NP = MLA_SETS * B * P
    g = torch.Generator(device=device).manual_seed(seed)
    gc = torch.Generator().manual_seed(seed)
    tags_list = list(cfg["mix"])
    probs = torch.tensor([cfg["mix"][t] for t in tags_list])
    tags = torch.tensor(tags_list, dtype=torch.int32)[torch.multinomial(probs, NP, replacement=True, generator=gc)]
    tags = tags.to(device)
    pools = LatentPools(c_fp8=torch.zeros((NP, PS, DQK), dtype=torch.uint8, device=device),
                        c_fp8_scale=torch.zeros(NP, dtype=torch.float16, device=device),
                        c_int8=torch.zeros((NP, PS, DQK), dtype=torch.int8, device=device),
                        c_int8_scale=torch.zeros(NP, dtype=torch.float16, device=device))
    for lo in range(0, NP, 16384):
        hi = min(NP, lo + 16384)
        x = torch.randn((hi - lo, PS, DQK), generator=g, device=device, dtype=torch.float32).half()
        t = tags[lo:hi]
        for tag, (pool, sc) in ((TAG_FP8, ("c_fp8", "c_fp8_scale")), (TAG_INT8, ("c_int8", "c_int8_scale"))):
            idx = torch.nonzero(t == tag).flatten()
            if idx.numel():
                codes, scales = quantize_pages(x[idx], tag)
                getattr(pools, pool)[lo + idx] = codes
                getattr(pools, sc)[lo + idx] = scales.to(torch.float16)
    nsel = int(cfg["sel"] * P)
    tables = []
    for s in range(MLA_SETS):
        base = s * B * P
        perm = (torch.randperm(B * P, generator=gc) + base).to(torch.int32).reshape(B, P)
        logical = torch.stack([torch.randperm(P, generator=gc)[:nsel].sort().values for _ in range(B)])
        tables.append(torch.gather(perm, 1, logical).contiguous().to(device))
    counts = torch.full((B,), nsel, dtype=torch.int32, device=device)
    q = torch.randn((B, H, DQK), generator=g, device=device).half()
    return dict(cfg=cfg, name=name, q=q, pools=pools, tables=tables, counts=counts, tags=tags, NP=NP, W=nsel)


def mla_step_cost(wl) -> dict:
    cfg = wl["cfg"]
    B, H, DQK, DV = cfg["B"], cfg["H"], cfg["DQK"], cfg["DV"]
    toks = B * wl["W"] * PS
    flop = 2.0 * H * toks * (DQK + DV)
    codes = B * wl["W"] * PS * DQK                    # one byte per latent element
    scales = B * wl["W"] * 2 + B * wl["W"] * (4 + 4)  # fp16 scale + page id + tag per page
    qo = wl["q"].numel() * 2 + B * H * DV * 2
    return dict(flop=flop, bytes=codes + scales + qo, tokens=toks)


def mla_cpu_baseline(wl, raw: dict) -> dict:
    cfg = wl["cfg"]
    flop = mla_step_cost(wl)["flop"]
    return cpu_baseline_entry(
        raw, "TFLOP/s", lambda ups: flop * ups / cfg["B"] / 1e12, cfg["B"],
        f"oracle.mla.mla_paged_decode_oracle (numpy float64, one BLAS thread per process) on synthetic cfg5 "
        f"sequences (128 heads, 512 FP8 / INT8 latent pages); one thread {raw['threads_1']['units']} sequences "
        f"in {raw['threads_1']['seconds']:.1f} s, all cores {raw.get('threads_all', {}).get('units', 0)} over "
        f"{raw['workers']} processes; scaled to the {cfg['B']}-sequence step")


def run_mla(args, cpu=None) -> None:
    from intent_attention.mla_core import make_mla_plan
    dev = torch.device("cuda:0")
    t_build = time.perf_counter()
    wl = build_mla_workload(args.config, dev)
    torch.cuda.synchronize()
    print(f"[bench] built {args.config}: NP={wl['NP']} W={wl['W']} in {time.perf_counter() - t_build:.1f}s",
          file=sys.stderr, flush=True)
    cfg = wl["cfg"]
    out = torch.empty((cfg["B"], cfg["H"], cfg["DV"]), dtype=torch.float16, device=dev)
    plans = [make_mla_plan(wl["q"], wl["pools"], t, wl["counts"], wl["tags"], v_dim=cfg["DV"], out=out,
                           pages_per_split=args.pages_per_split) for t in wl["tables"]]
    stream = torch.cuda.current_stream(dev)
    for i in range(args.warmup):
        plans[i % MLA_SETS].run()
    torch.cuda.synchronize()
    t_start, t_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_start.record(stream)
    for i in range(args.steps):
        plans[i % MLA_SETS].run()
    t_end.record(stream)
    torch.cuda.synchronize()
    ms = t_start.elapsed_time(t_end) / args.steps
    # second pass: events around every step and around the split kernel alone
    ev = kernel_events(args.steps)
    kev = kernel_events(args.steps)
    for i, ((s, e), k) in enumerate(zip(ev, kev)):
        s.record(stream)
        plans[i % MLA_SETS].run(events=k)
        e.record(stream)
    torch.cuda.synchronize()
    per = sorted(s.elapsed_time(e) for s, e in ev)
    kernel_ms_events = sum(b.elapsed_time(e) for b, e in kev) / args.steps
    # the split kernel runs inside each step, so the step time of the timed
    # region bounds it; a per-launch event pair also holds the launch's own
    # dispatch and completion (on some boxes it reads longer than the step)
    kernel_ms = min(ms, kernel_ms_events)
    kernel_timing = ("HIP events around each split-kernel launch" if kernel_ms_events <= ms else
                     "events around the K back-to-back steps of the timed region (the split kernel plus "
                     "the merge: an upper bound on the split kernel, below its per-launch event pairs)")
    cost = mla_step_cost(wl)
    tflops = cost["flop"] / (ms * 1e-3) / 1e12
    kernel_tflops = cost["flop"] / (kernel_ms * 1e-3) / 1e12
    res = {
        "metric": "MLA latent decode µs/step + MFMA TFLOP/s (cfg5, DeepSeek-V3-style)", "value": round(tflops, 1),
        "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
        "us_per_step": round(ms * 1e3, 2),
        "us_per_step_p10_p50_p90": [round(per[len(per) // 10] * 1e3, 2), round(per[len(per) // 2] * 1e3, 2),
                                    round(per[(9 * len(per)) // 10] * 1e3, 2)],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "data": "synthetic (seeded; latent N(0,1) fp16 pages quantised with the reference's fake-quant arithmetic)",
        "config": {"workload": f"{args.config}: MLA decode B={cfg['B']} heads={cfg['H']} latent {cfg['DV']}+"
                               f"{cfg['DQK'] - cfg['DV']} ctx={cfg['T']} page=16 sel={wl['W']} pages/seq "
                               f"mix=FP8/INT8 50/50, {MLA_SETS} page sets rotated",
                   "selected_tokens": cost["tokens"], "algorithmic_bytes": cost["bytes"],
                   "gflop": round(cost["flop"] / 1e9, 3), "pages_per_split": plans[0].args.pages_per_split},
        "roofline": {"bound": "mfma", "achieved": round(kernel_tflops, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(kernel_tflops / MFMA_F16_PEAK_TFLOPS, 4), "traffic": None,
                     "kernel": "mla_decode_kernel", "kernel_us": round(kernel_ms * 1e3, 2),
                     "kernel_timing": kernel_timing,
                     "kernel_us_event_pairs": round(kernel_ms_events * 1e3, 2),
                     "kernel_source_digest": mla_source_digest(),
                     "step_frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
                     "hbm_gbps": round(cost["bytes"] / (kernel_ms * 1e-3) / 1e9, 1)},
    }
    if cpu is not None:
        res["cpu_baseline"] = mla_cpu_baseline(wl, cpu)
    print(json.dumps(res), flush=True)


# --------------------------------------------------------------------------- #
# Quantise-on-write (cfg3-quantize): every quantised page of the cfg3 pools
# --------------------------------------------------------------------------- #

QUANT_CONFIGS = {
    # the cfg3 pools: 32 x 8 x 4096 pages per K and V, 25 % FP16 (stored as is),
    # 25 % FP8, 30 % INT8, 20 % INT4 (groups of 32 channels); fresh float16 pages
    # with 1 % of K elements at 8 sigma, quantised into their pool slots
    "cfg3-quantize": dict(pages=32 * 8 * 4096, D=128, mix={TAG_FP8: .25, TAG_INT8: .30, TAG_INT4: .20},
                          outliers=0.01),
}
QUANT_OUT_BYTES = {TAG_FP8: (PS * 128, 2), TAG_INT8: (PS * 128, 2), TAG_INT4: (PS * 64, 4 * 2)}


def build_quantize_workload(name: str, device: torch.device, seed: int = 99):
    cfg = QUANT_CONFIGS[name]
    NP, D = cfg["pages"], cfg["D"]
    g = torch.Generator(device=device).manual_seed(seed)
    gc = torch.Generator().manual_seed(seed)
    jobs = []
    for w in ("k", "v"):
        slots = torch.randperm(NP, generator=gc)
        lo = 0
        for tag, frac in cfg["mix"].items():
            n = int(frac * NP)
            dst = slots[lo:lo + n].to(torch.int32).to(device)
            lo += n
            src = torch.randn((n, PS, D), generator=g, device=device, dtype=torch.float32)
            if w == "k" and cfg["outliers"] > 0:
                m = torch.rand(src.shape, generator=g, device=device) < cfg["outliers"]
                src = torch.where(m, 8.0 * torch.sign(src), src)
            src = src.half()
            width = D // 2 if tag == TAG_INT4 else D
            codes = torch.zeros((NP, PS, width), dtype=torch.uint8, device=device)
            scales = torch.zeros((NP, D // 32) if tag == TAG_INT4 else (NP,), dtype=torch.float16, device=device)
            jobs.append(dict(w=w, tag=tag, src=src, dst=dst, codes=codes, scales=scales))
    return dict(cfg=cfg, name=name, jobs=jobs)


def quantize_step_bytes(wl) -> int:
    total = 0
    for j in wl["jobs"]:
        n = j["src"].shape[0]
        cb, sb = QUANT_OUT_BYTES[j["tag"]]
        total += n * (PS * wl["cfg"]["D"] * 2 + 4 + cb + sb)     # f16 page in, slot id, codes + scales out
    return total


def quantize_cpu_baseline(wl, raw: dict) -> dict:
    pages = sum(j["src"].shape[0] for j in wl["jobs"])
    step_bytes = quantize_step_bytes(wl)
    return cpu_baseline_entry(
        raw, "GB/s", lambda ups: step_bytes * ups / pages / 1e9, pages,
        f"oracle.quant.quantize_page (numpy, one thread per process) on float16 pages round robin over the "
        f"FP8 / INT8 / INT4 jobs; one thread {raw['threads_1']['units']} pages in "
        f"{raw['threads_1']['seconds']:.1f} s, all cores {raw.get('threads_all', {}).get('units', 0)} over "
        f"{raw['workers']} processes; scaled to the {pages}-page step")


def run_quantize(args, cpu=None) -> None:
    from intent_attention import _native as N
    dev = torch.device("cuda:0")
    t_build = time.perf_counter()
    wl = build_quantize_workload(args.config, dev)
    torch.cuda.synchronize()
    print(f"[bench] built {args.config} in {time.perf_counter() - t_build:.1f}s", file=sys.stderr, flush=True)
    stream = torch.cuda.current_stream(dev)
    argv = []
    for j in wl["jobs"]:
        a = N.QuantizeArgs()
        a.num_pages, a.page_size, a.head_dim = j["src"].shape[0], PS, wl["cfg"]["D"]
        a.src, a.dst_pages, a.pool_pages = j["src"].data_ptr(), j["dst"].data_ptr(), j["codes"].shape[0]
        a.precision, a.mode, a.int4_group = j["tag"], N.QUANT_FAKE_QUANTIZE, 32
        a.codes, a.scales, a.scale_dtype = j["codes"].data_ptr(), j["scales"].data_ptr(), N.DTYPE_F16
        argv.append(a)

    def step():
        for a in argv:
            N.quantize_pages(a, stream.cuda_stream)

    res = _time_steps(step, args, stream)
    ab = quantize_step_bytes(wl)
    ms = res["ms"]
    gbps = ab / (ms * 1e-3) / 1e9
    out = {"metric": "quantise-on-write GB/s (cfg3 pools: FP8 / INT8 / INT4 pages from float16)",
           "value": round(gbps, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": round(ms, 5), "us_per_step": round(ms * 1e3, 2),
           "us_per_step_p10_p50_p90": res["spread"], "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "f16->u8",
           "data": "synthetic (seeded float16 N(0,1) pages, 1 % of K at 8 sigma)",
           "config": {"workload": f"{args.config}: {sum(j['src'].shape[0] for j in wl['jobs'])} pages of 16x128 "
                                  f"quantised into 1,048,576-slot K and V pools (6 launches per step)",
                      "algorithmic_bytes": ab},
           "kernel_source_digest": source_digest(["quantize.hip", "iak_internal.h", "iak_device.h"]),
           "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                        "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None}}
    if cpu is not None:
        out["cpu_baseline"] = quantize_cpu_baseline(wl, cpu)
    print(json.dumps(out), flush=True)


# --------------------------------------------------------------------------- #
# Page tables from routing (cfg3-tables): iak_build_page_tables at cfg3 shape
# --------------------------------------------------------------------------- #

TABLE_CONFIGS = {
    # 32 sequences x 8 KV heads, 65,536 tokens (4096 pages) each; per sequence a
    # routing of blocks of 16..1024 tokens, 40 % of the tokens selected, in a
    # shuffled (routed) order with random page precisions; each (sequence, KV
    # head) row maps its logical pages through its own block-table row into a
    # 1,048,576-page pool; width 1639, precision over every pool page
    "cfg3-tables": dict(B=32, Hkv=8, T=65536, sel=0.40, block=(16, 1024), W=1639),
}


def table_routing(name: str, seed: int = 7):
    """Host part of the cfg3-tables workload: per sequence the routed spans
    (start, end, tag), and the block table [B * Hkv, pages] (numpy only)."""
    cfg = TABLE_CONFIGS[name]
    B, Hkv, T = cfg["B"], cfg["Hkv"], cfg["T"]
    P = T // PS
    rng = np.random.default_rng(seed)
    lists = []
    for b in range(B):
        cuts, t = [], 0
        while t < T:
            ln = int(rng.integers(cfg["block"][0], cfg["block"][1] + 1))
            cuts.append((t, min(T, t + ln)))
            t += ln
        order = rng.permutation(len(cuts))
        spans, got = [], 0
        for i in order:
            if got >= cfg["sel"] * T:
                break
            s, e = cuts[i]
            spans.append((s, e, int(rng.choice([TAG_FP16, TAG_FP8, TAG_INT8, TAG_INT4], p=[.25, .25, .30, .20]))))
            got += e - s
        lists.append(spans)
    NP = B * Hkv * P
    return lists, NP, P, rng.permutation(NP).astype(np.int32).reshape(B * Hkv, P)


def build_table_workload(name: str, device: torch.device, seed: int = 7):
    cfg = TABLE_CONFIGS[name]
    lists, NP, P, bt_host = table_routing(name, seed)
    bt = torch.from_numpy(bt_host).to(device)
    offs, beg, end, tag = [0], [], [], []
    for spans in lists:
        for s, e, t in spans:
            beg.append(s)
            end.append(e)
            tag.append(t)
        offs.append(len(beg))
    dev_i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=device)  # noqa: E731
    return dict(cfg=cfg, name=name, lists=lists, NP=NP, P=P, block_table=bt, offs=dev_i32(offs),
                begin=dev_i32(beg), end=dev_i32(end), tag=dev_i32(tag))


def table_step_bytes(wl, pairs: int) -> int:
    cfg = wl["cfg"]
    R = cfg["B"] * cfg["Hkv"]
    spans = wl["begin"].numel()
    return (spans * 12 * cfg["Hkv"] + wl["offs"].numel() * 4      # span lists, read by each of their rows
            + pairs * 4                                          # block-table entries of the named pages
            + R * cfg["W"] * 4 + R * 4 + wl["NP"] * 4)          # page table, counts, precision out


def run_tables(args, cpu=None) -> None:
    from intent_attention import _native as N
    dev = torch.device("cuda:0")
    wl = build_table_workload(args.config, dev)
    cfg = wl["cfg"]
    R = cfg["B"] * cfg["Hkv"]
    table = torch.empty((R, cfg["W"]), dtype=torch.int32, device=dev)
    counts = torch.empty(R, dtype=torch.int32, device=dev)
    prec = torch.empty(wl["NP"], dtype=torch.int32, device=dev)
    a = N.PageTableArgs()
    a.num_rows, a.rows_per_seq, a.rows_per_list = R, 1, cfg["Hkv"]
    a.table_width, a.page_size, a.num_pages, a.dedupe, a.default_tag = cfg["W"], PS, wl["NP"], 1, TAG_FP16
    a.block_table_width = wl["P"]
    a.span_offsets, a.span_begin, a.span_end, a.span_tag = (t.data_ptr() for t in
                                                            (wl["offs"], wl["begin"], wl["end"], wl["tag"]))
    a.block_table, a.page_table, a.page_counts, a.page_precision = (wl["block_table"].data_ptr(), table.data_ptr(),
                                                                    counts.data_ptr(), prec.data_ptr())
    stream = torch.cuda.current_stream(dev)
    # one step = the three launches (fill, build, tags); replayed as a HIP graph so
    # the host's launch rate does not set the step time
    N.build_page_tables(a, stream.cuda_stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        N.build_page_tables(a, torch.cuda.current_stream(dev).cuda_stream)
    torch.cuda.synchronize()
    res = _time_steps(graph.replay, args, stream)
    pairs = int(sum(min(wl["P"] - 1, (e - 1) // PS) - s // PS + 1 for spans in wl["lists"] for s, e, _ in spans))
    ab = table_step_bytes(wl, pairs * cfg["Hkv"])
    ms = res["ms"]
    gbps = ab / (ms * 1e-3) / 1e9
    out = {"metric": "page-table build µs/step (routing -> page_table / precision / counts, cfg3 shape)",
           "value": round(ms * 1e3, 2), "unit": "us", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": round(ms, 5), "us_per_step_p10_p50_p90": res["spread"], "higher_is_better": False,
           "scaling": "weak", "vs_baseline": None, "dtype": "int32",
           "data": "synthetic (seeded block routings and block tables)",
           "config": {"workload": f"{args.config}: {R} rows (32 sequences x 8 KV heads), "
                                  f"{wl['begin'].numel()} routed blocks, {pairs} selected pages per KV head "
                                  f"summed over sequences, width {cfg['W']}, {wl['NP']}-page precision array",
                      "algorithmic_bytes": ab},
           "kernel_source_digest": source_digest(["page_tables.hip", "iak_internal.h"]),
           "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                        "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None}}
    if cpu is not None:
        out["cpu_baseline"] = cpu_baseline_entry(
            cpu, "us", lambda ups: 1e6 / ups, 1,
            f"oracle.policy.build_page_tables_oracle (Python loops as the reference's routing_to_kernel_metadata "
            f"+ metadata_to_kernel_tensors, one thread per process), the full step: one thread "
            f"{cpu['threads_1']['units']} in {cpu['threads_1']['seconds']:.1f} s, all cores "
            f"{cpu.get('threads_all', {}).get('units', 0)} over {cpu['workers']} processes (independent steps)")
    print(json.dumps(out), flush=True)


# --------------------------------------------------------------------------- #
# KV memory manager transcoding (transcode): iak_transcode_pages on the cfg3
# pool shape. A step demotes a quarter of the pool's pages (random slots) from
# the FP16 pool to the INT8 pool, then promotes them back: the manager's
# demote_cold_pages / promote_hot_pages, one launch each.

TRANSCODE_CONFIGS = {
    "transcode": dict(pool=32 * 8 * 4096, pages=262144, elems=PS * 128),
}


def transcode_page_bytes(elems: int) -> dict:
    """Algorithmic bytes per page: demote reads the float16 page and its slot id
    and writes the codes and the float32 scale; promote reads the codes, the
    scale and the slot id and writes the float16 page."""
    return {"demote": elems * 2 + 4 + elems + 4, "promote": elems + 4 + 4 + elems * 2}


def run_transcode(args, cpu=None) -> None:
    from intent_attention import _native as N
    dev = torch.device("cuda:0")
    cfg = TRANSCODE_CONFIGS[args.config]
    NP, n, E = cfg["pool"], cfg["pages"], cfg["elems"]
    t_build = time.perf_counter()
    g = torch.Generator(device=dev).manual_seed(5)
    fp16 = torch.empty((NP, E), dtype=torch.float16, device=dev)
    for lo in range(0, NP, 65536):
        fp16[lo:lo + 65536] = torch.randn((min(65536, NP - lo), E), generator=g, device=dev).half()
    int8 = torch.zeros((NP, E), dtype=torch.int8, device=dev)
    scales = torch.ones(NP, dtype=torch.float32, device=dev)
    slots = torch.randperm(NP, generator=torch.Generator().manual_seed(6))[:n].to(torch.int32).to(dev)
    torch.cuda.synchronize()
    print(f"[bench] built {args.config} in {time.perf_counter() - t_build:.1f}s", file=sys.stderr, flush=True)
    stream = torch.cuda.current_stream(dev)
    argv = {}
    for name, mode in (("demote", N.TRANSCODE_DEMOTE_INT8), ("promote", N.TRANSCODE_PROMOTE_FP16)):
        a = N.TranscodeArgs()
        a.num_pages, a.page_elems, a.mode, a.pages, a.pool_pages = n, E, mode, slots.data_ptr(), NP
        a.fp16, a.int8, a.scales = fp16.data_ptr(), int8.data_ptr(), scales.data_ptr()
        argv[name] = a

    def step(ev=None):
        for i, name in enumerate(("demote", "promote")):
            if ev is not None:
                ev[i][0].record(stream)
            N.transcode_pages(argv[name], stream.cuda_stream)
            if ev is not None:
                ev[i][1].record(stream)

    res = _time_steps(step, args, stream)
    evs = [kernel_events(2) for _ in range(args.steps)]
    for ev in evs:
        step(ev)
    torch.cuda.synchronize()
    per_page = transcode_page_bytes(E)
    kern = {}
    for i, name in enumerate(("demote", "promote")):
        us = sum(ev[i][0].elapsed_time(ev[i][1]) for ev in evs) / args.steps * 1e3
        kern[name] = {"us": round(us, 2), "GBps": round(per_page[name] * n / (us * 1e-6) / 1e9, 1),
                      "algorithmic_bytes": per_page[name] * n}
    ab = (per_page["demote"] + per_page["promote"]) * n
    ms = res["ms"]
    gbps = ab / (ms * 1e-3) / 1e9
    dom = max(kern, key=lambda k: kern[k]["us"])
    out = {"metric": "KV page transcoding GB/s (demote FP16 -> INT8, then promote INT8 -> FP16)",
           "value": round(gbps, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": round(ms, 5), "us_per_step": round(ms * 1e3, 2),
           "us_per_step_p10_p50_p90": res["spread"], "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "f16<->i8",
           "data": "synthetic (seeded float16 N(0,1) pages)",
           "config": {"workload": f"{args.config}: {n} random slots of a {NP}-page pool of 16x128 float16 pages "
                                  f"demoted to INT8 and promoted back (2 launches per step)",
                      "algorithmic_bytes": ab, "kernels": kern},
           "kernel_source_digest": source_digest(["memory_manager.hip", "iak_internal.h", "iak_device.h"]),
           "roofline": {"bound": "hbm", "achieved": kern[dom]["GBps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                        "frac": round(kern[dom]["GBps"] / HBM_PEAK_GBPS, 4), "traffic": None,
                        "kernel": f"transcode_{dom}_kernel", "kernel_us": kern[dom]["us"]}}
    if cpu is not None:
        out["cpu_baseline"] = cpu_baseline_entry(
            cpu, "GB/s", lambda ups: (per_page["demote"] + per_page["promote"]) * ups / 1e9, n,
            f"oracle.memory.demote_int8 + promote_fp16 (numpy, one thread per process) on 16x128 float16 pages; "
            f"one thread {cpu['threads_1']['units']} pages in {cpu['threads_1']['seconds']:.1f} s, all cores "
            f"{cpu.get('threads_all', {}).get('units', 0)} over {cpu['workers']} processes")
    print(json.dumps(out), flush=True)


# dense_attention (the reference's reference.py:16-45, under intent_quant_attention_reference):
# shapes (leading rows, q_len, kv_len, head_dim, dtype); the first is cfg1's attention
DENSE_CONFIGS = {
    "dense": [((1, 8), 1, 512, 64, torch.float32), ((1, 8), 1, 8192, 128, torch.float16),
              ((1, 32), 1, 4096, 128, torch.bfloat16), ((4, 8), 128, 128, 64, torch.float16)],
}


def run_dense(args) -> None:
    """dense_attention per shape: the C ABI call on resident inputs (kernel(s) only,
    the split workspace allocated once) and the Python entry point. The bytes are
    K + V + Q + O once each (algorithmic; rows of one batch re-read K and V)."""
    from intent_attention import _native as N
    from intent_attention import dense_attention
    from intent_attention.reference import _DTYPES
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    g = torch.Generator(device=dev).manual_seed(7)
    rows = []
    for lead, tq, tk, d, dt in DENSE_CONFIGS[args.config]:
        L = math.prod(lead)
        q = torch.randn(L, tq, d, device=dev, generator=g).to(dt)
        k = torch.randn(L, tk, d, device=dev, generator=g).to(dt)
        v = torch.randn(L, tk, d, device=dev, generator=g).to(dt)
        out = torch.empty(L, tq, d, device=dev, dtype=dt)
        a = N.DenseAttentionArgs()
        a.batch, a.q_len, a.kv_len, a.head_dim, a.v_dim, a.dtype = L, tq, tk, d, d, _DTYPES[dt]
        a.q, a.q_stride_b, a.q_stride_t = q.data_ptr(), q.stride(0), q.stride(1)
        a.k, a.k_stride_b, a.k_stride_t = k.data_ptr(), k.stride(0), k.stride(1)
        a.v, a.v_stride_b, a.v_stride_t = v.data_ptr(), v.stride(0), v.stride(1)
        a.out, a.out_stride_b, a.out_stride_t = out.data_ptr(), out.stride(0), out.stride(1)
        a.sm_scale = 1.0 / math.sqrt(d)
        wsb = N.dense_attention_workspace(a)
        ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=dev)
        h = stream.cuda_stream
        kern = _time_steps(lambda: N.dense_attention(a, h, ws.data_ptr() if wsb else 0, wsb), args, stream)
        qv, kv_, vv = q.view(*lead, tq, d), k.view(*lead, tk, d), v.view(*lead, tk, d)
        api = _time_steps(lambda: dense_attention(qv, kv_, vv), args, stream)
        ab = (2 * L * tk * d + 2 * L * tq * d) * torch.finfo(dt).bits // 8
        rows.append({"shape": {"rows": L * tq, "q_len": tq, "kv_len": tk, "head_dim": d, "dtype": str(dt)[6:]},
                     "split_workspace_bytes": wsb, "us_per_call": round(kern["ms"] * 1e3, 2),
                     "us_p10_p50_p90": kern["spread"], "api_us_per_call": round(api["ms"] * 1e3, 2),
                     "algorithmic_bytes": ab, "gbps": round(ab / (kern["ms"] * 1e-3) / 1e9, 1)})
        print(f"[bench] dense {rows[-1]['shape']}: {rows[-1]['us_per_call']} us", file=sys.stderr, flush=True)
    head = rows[1]
    print(json.dumps({
        "metric": "dense_attention µs per call (the reference's reference.py:16-45 in float32)",
        "value": head["us_per_call"], "unit": "us", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded N(0,1))",
        "config": {"workload": "dense_attention shapes; value = 8 rows x 8,192 keys x 128 (float16), split over keys"},
        "kernel_source_digest": source_digest(["dense_attention.hip", "iak_device.h"]),
        "shapes": rows}), flush=True)


# mla_decode_triton's latent context (the reference's triton_mla_decode.py:47-186,
# float32 row kernel): (batch, latent rows of C, page size, pages listed, d_c, dtype)
MLA_ROWS_CONFIGS = {
    "mla-rows": [(32, 16384, 64, 128, 576, torch.float16), (1, 4096, 64, 32, 576, torch.float32),
                 (4, 8192, 16, 256, 512, torch.bfloat16), (2, 1024, 64, 8, 576, torch.float32)],
}


def run_mla_rows(args) -> None:
    """mla_latent_context per shape: the C ABI call on resident inputs (kernels
    only, the split workspace allocated once) and the Python entry point. The
    bytes are the listed latent rows once, Q and the context (algorithmic)."""
    from intent_attention import _native as N
    from intent_attention.triton_mla_decode import _DT, mla_latent_context
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    g = torch.Generator(device=dev).manual_seed(11)
    rows = []
    for B, T, ps, npages, dc, dt in MLA_ROWS_CONFIGS[args.config]:
        q = torch.randn(B, 1, dc, device=dev, generator=g).to(dt)
        C = torch.randn(T, dc, device=dev, generator=g).to(dt)
        ids = torch.randperm(T // ps, device=dev, generator=g)[:npages].to(torch.int32)
        ctx = torch.empty(B, 1, dc, dtype=torch.float32, device=dev)
        a = N.MlaRowsArgs()
        a.batch, a.q_len, a.latent_dim, a.page_size, a.num_selected, a.num_rows = B, 1, dc, ps, npages, T
        a.q, a.q_dtype, a.q_stride_b, a.q_stride_t = q.data_ptr(), _DT[dt], q.stride(0), q.stride(1)
        a.latents, a.latent_dtype, a.latent_stride = C.data_ptr(), _DT[dt], C.stride(0)
        a.page_ids, a.context, a.sm_scale = ids.data_ptr(), ctx.data_ptr(), 1.0 / math.sqrt(dc)
        wsb = N.mla_decode_rows_workspace(a)
        ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=dev)
        h = stream.cuda_stream
        kern = _time_steps(lambda: N.mla_decode_rows(a, h, ws.data_ptr() if wsb else 0, wsb), args, stream)
        api = _time_steps(lambda: mla_latent_context(q, C, ids, ps), args, stream)
        ab = (npages * ps * dc + 2 * B * dc) * torch.finfo(dt).bits // 8 + B * dc * 4
        rows.append({"shape": {"batch": B, "latent_rows": npages * ps, "page_size": ps, "d_c": dc,
                               "dtype": str(dt)[6:]},
                     "split_workspace_bytes": wsb, "us_per_call": round(kern["ms"] * 1e3, 2),
                     "us_p10_p50_p90": kern["spread"], "api_us_per_call": round(api["ms"] * 1e3, 2),
                     "algorithmic_bytes": ab, "gbps": round(ab / (kern["ms"] * 1e-3) / 1e9, 1)})
        print(f"[bench] mla rows {rows[-1]['shape']}: {rows[-1]['us_per_call']} us", file=sys.stderr, flush=True)
    head = rows[0]
    print(json.dumps({
        "metric": "mla_decode_triton latent context µs per call (the reference's triton_mla_decode.py in float32)",
        "value": head["us_per_call"], "unit": "us", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded N(0,1))",
        "config": {"workload": "mla_latent_context shapes; value = 32 sequences x 8,192 latent rows x 576 (float16)"},
        "kernel_source_digest": source_digest(["mla_rows.hip", "iak_device.h"]),
        "shapes": rows}), flush=True)


# the selected-block fake-quant reconstruction under intent_quant_attention_reference
# (the reference's intent_quant_attention.py:56-84, fake_quantize_tensor per block) in
# float32: (leading rows, tokens, head_dim, [(block tokens, precision), ...]); the first
# is cfg1's (32 pages of 16 tokens, FP16 / INT8 alternating), the second the reference
# benchmark's layout (three quarter-context blocks) at 32 heads x 4,096 tokens
FAKE_QUANT_CONFIGS = {
    "fake-quant": [(8, 512, 64, [(16, p) for _ in range(16) for p in ("FP16", "INT8")]),
                   (32, 4096, 128, [(1024, "INT8"), (1024, "INT4_RESIDUAL"), (1024, "FP8")]),
                   (32, 4096, 128, [(64, "INT8")] * 64),
                   (8, 4096, 64, [(256, "FP8")] * 16)],
}


def run_fake_quant(args) -> None:
    """The selected-block reconstruction per shape: the C ABI call on resident
    inputs and block table (kernels only, the split workspace allocated once)
    and the Python entry point (_reconstruct_selected: block table upload,
    output and workspace allocation, launch). The bytes are the selected K and V
    values read once and their reconstruction written once (algorithmic)."""
    from intent_attention import KVPrecision
    from intent_attention import _native as N
    from intent_attention.block_metadata import BlockPolicy, SemanticBlock
    from intent_attention.intent_quant_attention import _FQ_CODE, _reconstruct_selected
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    g = torch.Generator(device=dev).manual_seed(5)
    rows = []
    for lead, T, d, spec in FAKE_QUANT_CONFIGS[args.config]:
        k = torch.randn(lead, T, d, device=dev, generator=g)
        v = torch.randn(lead, T, d, device=dev, generator=g)
        lens = [n for n, _ in spec]
        precs = [KVPrecision(p) for _, p in spec]
        starts = [sum(lens[:i]) for i in range(len(lens))]
        total = sum(lens)
        meta = torch.tensor([[st, n, st, _FQ_CODE[p]] for st, n, p in zip(starts, lens, precs)],
                            dtype=torch.int32, device=dev)
        out = torch.empty(lead, total, 2 * d, device=dev)
        a = N.FakeQuantBlocksArgs()
        a.lead, a.num_blocks, a.k_dim, a.v_dim = lead, len(spec), d, d
        a.k, a.k_stride_l, a.k_stride_t = k.data_ptr(), k.stride(0), k.stride(1)
        a.v, a.v_stride_l, a.v_stride_t = v.data_ptr(), v.stride(0), v.stride(1)
        a.blocks, a.max_block_tokens = meta.data_ptr(), max(lens)
        a.out, a.out_stride_l, a.out_stride_t = out.data_ptr(), out.stride(0), out.stride(1)
        wsb = N.fake_quant_blocks_workspace(a)
        ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=dev)
        h = stream.cuda_stream
        kern = _time_steps(lambda: N.fake_quant_blocks(a, h, ws.data_ptr() if wsb else 0, wsb), args, stream)
        blocks = [SemanticBlock(f"b{i}", st, st + n, BlockPolicy.ATTEND, 1.0) for i, (st, n) in enumerate(zip(starts, lens))]
        api = _time_steps(lambda: _reconstruct_selected(k, v, blocks, precs), args, stream)
        ab = 2 * lead * total * 2 * d * 4
        rows.append({"shape": {"lead": lead, "tokens": total, "channels": 2 * d, "blocks": len(spec),
                               "block_tokens": sorted(set(lens)), "precisions": sorted({p for _, p in spec})},
                     "split_workspace_bytes": wsb, "us_per_call": round(kern["ms"] * 1e3, 2),
                     "us_p10_p50_p90": kern["spread"], "api_us_per_call": round(api["ms"] * 1e3, 2),
                     "algorithmic_bytes": ab, "gbps": round(ab / (kern["ms"] * 1e-3) / 1e9, 1)})
        print(f"[bench] fake-quant {rows[-1]['shape']}: {rows[-1]['us_per_call']} us", file=sys.stderr, flush=True)
    head = rows[1]
    print(json.dumps({
        "metric": "selected-block fake-quant reconstruction µs per call (the reference's "
                  "intent_quant_attention.py:56-84 in float32)",
        "value": head["us_per_call"], "unit": "us", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded N(0,1))",
        "config": {"workload": "reconstruction shapes; value = 32 heads x 3 blocks of 1,024 tokens x 256 channels "
                               "(INT8, INT4_RESIDUAL, FP8), split"},
        "kernel_source_digest": source_digest(["fake_quant.hip"]),
        "shapes": rows}), flush=True)


def kernel_events(n: int) -> list:
    """n pairs of fence-free timing events (libiak's iak_timing_event_create):
    recording one does not write back and invalidate the caches, so an event
    after a kernel that wrote many MB (the MLA split partials) closes its
    interval when the kernel ends, not after the write-back. The library
    records them around the split kernel of a timed step, the bench around a
    step or a launch."""
    from intent_attention import _native as N
    return [(N.TimingEvent(), N.TimingEvent()) for _ in range(n)]


def _time_steps(step, args, stream) -> dict:
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(args.steps):
        step()
    t1.record(stream)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    for s, e in ev:
        s.record(stream)
        step()
        e.record(stream)
    torch.cuda.synchronize()
    per = sorted(s.elapsed_time(e) for s, e in ev)
    return {"ms": ms, "spread": [round(per[len(per) // 10] * 1e3, 2), round(per[len(per) // 2] * 1e3, 2),
                                 round(per[(9 * len(per)) // 10] * 1e3, 2)]}


# --------------------------------------------------------------------------- #

def cpu_jobs_for(config: str):
    """(job, extra args) of the oracle CPU job that mirrors a leg."""
    if config in CONFIGS and config != "tiny":
        return "decode", (config,)
    if config in MLA_CONFIGS:
        return "mla", ()
    if config in QUANT_CONFIGS:
        return "quantize", ()
    if config == "cfg1":
        return "cfg1", ("loop",)
    if config in TRANSCODE_CONFIGS:
        return "transcode", ()
    return None, ()


def cfg1_attention_step(dev: torch.device, wl: dict):
    """One intent_quant_attention_reference call at cfg1's shape on the product API
    (the selected pages as 16-token blocks, FP16 / INT8 alternating by page id,
    float16 values carried in float32 as the reference's runnable form needs):
    the CPU protocol's `iqa_reference` path, on the GPU."""
    from intent_attention import (BlockLayout, BlockPolicy, KVPrecision, QuantPolicy, SemanticBlock,
                                  intent_quant_attention_reference)
    c = CFG1
    H, D, P = c["H"], c["D"], c["pages"]
    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, H, 1, D, generator=g).half().float().to(dev)
    k = torch.randn(1, H, P * PS, D, generator=g).half().float().to(dev)
    v = torch.randn(1, H, P * PS, D, generator=g).half().float().to(dev)
    pages = sorted(wl["pages"])
    blocks, plan = [], {}
    for r, p in enumerate(pages):
        pol = BlockPolicy.ALWAYS if p < c["always"] else (BlockPolicy.RECENT if p >= P - c["recent"]
                                                           else BlockPolicy.ATTEND)
        blocks.append(SemanticBlock(f"p{p}", p * PS, (p + 1) * PS, pol, 0.9 if pol == BlockPolicy.ATTEND else None))
        plan[f"p{p}"] = KVPrecision.FP16 if r % 2 == 0 else KVPrecision.INT8

    class Plan:
        def assign_block_precision(self, block):
            return QuantPolicy(plan[block.name])

    layout, quantizer = BlockLayout(blocks), Plan()
    return lambda: intent_quant_attention_reference(q, k, v, layout, quantizer)


def run_cfg1(args, cpu=None, cfg1_paths=None) -> None:
    """cfg1: the reference's CPU-runnable shape on the
    GPU. A step is one fused_selected_quant_decode over the routed pages, timed
    as the validated plan's launch (the call the Python entry point makes after
    its argument checks) and as the whole Python call."""
    from intent_attention import fused_selected_quant_decode
    from intent_attention.decode_core import PagePools, make_plan
    from intent_attention.fused_selected_quant_decode import _tag_map
    dev = torch.device("cuda:0")
    wl = build_cfg1(dev)
    c = CFG1
    pools = PagePools(k_fp16=wl["k16"], v_fp16=wl["v16"], k_int8=wl["k8"], v_int8=wl["v8"], k_int8_scale=wl["ks"],
                      v_int8_scale=wl["vs"])
    out = torch.empty((c["B"], c["H"], 1, c["D"]), dtype=torch.float16, device=dev)
    plan = make_plan(wl["q"][:, :, 0, :], pools, wl["table"], wl["counts"], wl["prec"], tag_map=_tag_map(pools),
                     negative_ids=True, sm_scale=1.0 / math.sqrt(c["D"]), out=out[:, :, 0, :], auto_records=False)
    stream = torch.cuda.current_stream(dev)
    res = _time_steps(plan.run, args, stream)
    # the same step captured once in a HIP graph and replayed (a serving loop
    # without the per-launch host work)
    plan.run()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan.run()
    gres = _time_steps(graph.replay, args, stream)
    api = _time_steps(lambda: fused_selected_quant_decode(*cfg1_args(wl)), args, stream)
    iqa = _time_steps(cfg1_attention_step(dev, wl), args, stream)
    kev = kernel_events(args.steps)
    for k in kev:
        plan.run(events=k)
    torch.cuda.synchronize()
    kernel_ms = sum(b.elapsed_time(e) for b, e in kev) / args.steps
    n_sel = len(wl["pages"])
    n_int8 = n_sel // 2
    # K+V codes of every (head, selected page), INT8 scales, table entries and tags, counts, Q and O
    ab = (c["H"] * ((n_sel - n_int8) * 2 * PS * c["D"] * 2 + n_int8 * (2 * PS * c["D"] + 2 * 2))
          + c["H"] * n_sel * (4 + 4) + c["H"] * 4 + 2 * c["B"] * c["H"] * c["D"] * 2)
    ms = res["ms"]
    out_json = {
        "metric": METRIC, "value": round(ab / (ms * 1e-3) / 1e9, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5), "us_per_step": round(ms * 1e3, 2),
        "us_per_step_p10_p50_p90": res["spread"],
        "api_us_per_step": round(api["ms"] * 1e3, 2),
        "graph_replay_us_per_step": round(gres["ms"] * 1e3, 2),
        "intent_quant_attention_us_per_step": round(iqa["ms"] * 1e3, 2),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "data": "synthetic (seeded N(0,1) float16 Q/K/V; INT8 pages by the fused fake_int8_pages_from_fp16)",
        "config": {"workload": "cfg1: B=1 H=8/8 D=64 ctx=1024 (64 pages), 32 selected by BlockRouter (4 ALWAYS, "
                               "8 RECENT, 20 ATTEND), FP16/INT8 alternating by page id, "
                               "routing_to_kernel_metadata -> metadata_to_kernel_tensors -> "
                               "fused_selected_quant_decode",
                   "selected_pages": c["H"] * n_sel, "algorithmic_bytes": ab,
                   "selected_page_ids": wl["meta"]["selected_page_ids"]},
        "roofline": {"bound": "hbm", "achieved": round(ab / (kernel_ms * 1e-3) / 1e9, 2), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(ab / (kernel_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 5),
                     "traffic": None, "kernel": "paged_decode_kernel", "kernel_us": round(kernel_ms * 1e3, 2),
                     "note": "latency-bound: 64 waves read 1.4 MB; the step is launch and dependent-load latency"},
    }
    if cpu is not None:
        out_json["cpu_baseline"] = cpu_baseline_entry(
            cpu, "GB/s", lambda ups: ab * ups / 1e9, 1,
            f"oracle.decode.fused_decode_reference_loop (the reference's per-(b, h, page) loop, numpy float32, one "
            f"thread per process) on synthetic cfg1 inputs; one thread {cpu['threads_1']['units']} steps in "
            f"{cpu['threads_1']['seconds']:.1f} s, all cores {cpu.get('threads_all', {}).get('units', 0)} steps "
            f"over {cpu['workers']} processes (independent steps)",
            paths_1_thread=cfg1_paths,
            published_reference_cpu_us=19454.0,
            published_reference_shape="docs/results_cpu.md:63-69: B=1 H=8 D=64, 16 of 64 pages selected, all FP16, "
                                      "unstated CPU")
    print(json.dumps(out_json), flush=True)


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    # untimed steps before the timed ones: at cfg3 the step time settles over the
    # first ~100 (320.8 us after 10 of them, 316.8 after 30, 315.1 after 100, 314.5
    # after 300 or 1,000), so the default times the steady state
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--config", default="cfg3",
                    choices=sorted(CONFIGS) + ["cfg1"] + sorted(MLA_CONFIGS) + sorted(QUANT_CONFIGS)
                    + sorted(TABLE_CONFIGS) + sorted(TRANSCODE_CONFIGS) + sorted(DENSE_CONFIGS)
                    + sorted(MLA_ROWS_CONFIGS) + sorted(FAKE_QUANT_CONFIGS))
    ap.add_argument("--pages-per-split", type=int, default=0)
    ap.add_argument("--cpu-budget", type=float, default=CPU_BUDGET_S,
                    help="seconds of oracle work per CPU-baseline leg (one thread, then all cores)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--merge", choices=("auto", "kernel", "in-kernel"), default="auto",
                    help="decode legs: where the split partials are merged (auto: the library's choice)")
    ap.add_argument("--page-descriptors", action="store_true",
                    help="decode legs: pack 32-byte page descriptors once (timed apart) and decode from them "
                         "instead of the tag and scale arrays; `value` keeps the reference format's bytes")
    ap.add_argument("--entry-records", action="store_true",
                    help="decode legs: pack 32-byte entry records once per page table (timed apart) and decode "
                         "from them instead of the table, tag and scale arrays; `value` keeps the reference "
                         "format's bytes")
    ap.add_argument("--no-variants", action="store_true",
                    help="cfg3 / cfg4: skip the packed-metadata passes after the headline ones (profiling runs)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="after the timed steps, run a plain device copy of MIB MiB (read + write "
                         "MIB MiB each): the reference point that scales rocprof FETCH_SIZE/WRITE_SIZE")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build's decode runs on a single device "
              f"(--gpus {args.gpus} is not supported; multi-GPU sharding is a design note only)",
              file=sys.stderr)
        sys.exit(2)

    # the CPU baseline runs first, in a child process, before this process touches the GPU
    cpu, cfg1_paths = None, None
    if not args.no_cpu_baseline:
        t0 = time.perf_counter()
        if args.config in TABLE_CONFIGS:
            import tempfile
            lists, NP, P, bt = table_routing(args.config)
            cfg = TABLE_CONFIGS[args.config]
            spec = os.path.join(tempfile.mkdtemp(prefix="iak_bench_"), "tables.npz")
            np.savez(spec, lists=np.array(json.dumps(lists)), R=cfg["B"] * cfg["Hkv"], W=cfg["W"], PS=PS, NP=NP,
                     Hkv=cfg["Hkv"], block_table=bt)
            cpu = run_cpu_jobs("tables", spec, budget_s=args.cpu_budget)
        else:
            job, extra = cpu_jobs_for(args.config)
            if job is not None:
                cpu = run_cpu_jobs(job, *extra, budget_s=args.cpu_budget)
        if args.config == "cfg1":
            import subprocess
            r = subprocess.run([sys.executable, "-c", "import json; from oracle.baseline import cfg1_protocol; "
                                "print(json.dumps(cfg1_protocol()))"], cwd=ROOT, capture_output=True, text=True,
                               timeout=300)
            if r.returncode != 0:
                raise RuntimeError(f"cfg1 CPU protocol failed: {r.stderr[-2000:]}")
            cfg1_paths = json.loads(r.stdout.strip().splitlines()[-1])
        print(f"[bench] CPU baseline in {time.perf_counter() - t0:.1f}s", file=sys.stderr, flush=True)

    if args.config == "cfg1":
        run_cfg1(args, cpu, cfg1_paths)
        return
    if args.config in DENSE_CONFIGS:
        run_dense(args)
        return
    if args.config in MLA_ROWS_CONFIGS:
        run_mla_rows(args)
        return
    if args.config in FAKE_QUANT_CONFIGS:
        run_fake_quant(args)
        return
    if args.config in MLA_CONFIGS:
        run_mla(args, cpu)
        return
    if args.config in QUANT_CONFIGS:
        run_quantize(args, cpu)
        return
    if args.config in TABLE_CONFIGS:
        run_tables(args, cpu)
        return
    if args.config in TRANSCODE_CONFIGS:
        run_transcode(args, cpu)
        return
    run_decode(args, cpu)


def metadata_variants(plans, steps: int, stream, job_bytes: int, config: str) -> dict:
    """The same steps on the same plans reading the optional packed metadata:
    entry records (packed once per page table) and page descriptors (packed
    once for the pools), each timed twice, alternating with the other (the
    mean of the two passes is reported). `value` is the job's reference-format bytes over
    the step time, as on the headline line; the plans return to the reference
    tensors afterwards."""
    def timed(k):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for i in range(min(k, 10)):
            plans[i % len(plans)].run()
        torch.cuda.synchronize()
        e0.record(stream)
        for i in range(k):
            plans[i % len(plans)].run()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / k

    def pack_timed(fn, *arg):
        fn(*arg)   # the first launch of a pack kernel also loads its code
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        fn(*arg)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3

    recs = [torch.empty(p._records_shape(), dtype=torch.int32, device=p.device) for p in plans]
    desc = torch.empty((int(plans[0].args.num_pages), 8), dtype=torch.int32, device=plans[0].device)
    rec_pack = [pack_timed(p.pack_records, r) for p, r in zip(plans, recs)]
    desc_pack = pack_timed(plans[0].pack_descriptors, desc)

    def use(form):
        for p, r in zip(plans, recs):
            p.use_records(r if form == "records" else None)
            p.use_descriptors(desc if form == "desc" else None)

    best = {"records": 0.0, "desc": 0.0}
    for form in ("records", "desc", "records", "desc"):
        use(form)
        best[form] += timed(steps) / 2
    use(None)
    out = {}
    for form, key, extra in (("records", "entry_records", {"pack_us_per_table": round(sum(rec_pack) / len(rec_pack), 2)}),
                             ("desc", "page_descriptors", {"pack_us": round(desc_pack, 2)})):
        ms = best[form]
        out[key] = {"us_per_step": round(ms * 1e3, 2), "value": round(job_bytes / (ms * 1e-3) / 1e9, 1), "unit": "GB/s",
                    **extra, "traffic": measured_traffic(config + ("-records" if form == "records" else "-desc"))[0]}
    return out


def run_decode(args, cpu=None) -> None:
    from intent_attention.decode_core import make_plan
    dev = torch.device("cuda:0")
    t_build = time.perf_counter()
    wl = build_workload(args.config, dev)
    torch.cuda.synchronize()
    print(f"[bench] built {args.config}: NP={wl['NP']} W={wl['W']} in {time.perf_counter() - t_build:.1f}s",
          file=sys.stderr, flush=True)
    cfg = wl["cfg"]
    out = torch.empty((cfg["B"], cfg["Hq"], cfg["D"]), dtype=torch.float16, device=dev)
    # one plan per page table; step i runs table i % sets
    merge = {"auto": None, "kernel": False, "in-kernel": True}[args.merge]
    # the headline reads the reference's tensors on every step (no automatic entry records)
    plans = [make_plan(wl["q"], wl["pools"], t, wl["counts"], wl["tags"], out=out,
                       pages_per_split=args.pages_per_split, merge_in_kernel=merge, auto_records=False)
             for t in wl["tables"]]
    plan = plans[0]
    from intent_attention import _native as N
    desc_info = None
    if args.page_descriptors:
        # one pack serves every plan (same pages, pools and tag map); timed on its own
        desc = plan.pack_descriptors()
        p0, p1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        cur = torch.cuda.current_stream(dev)
        p0.record(cur)
        plan.pack_descriptors(desc)
        p1.record(cur)
        torch.cuda.synchronize()
        for p in plans[1:]:
            p.use_descriptors(desc)
        desc_info = {"pack_us": round(p0.elapsed_time(p1) * 1e3, 2), "bytes": desc.numel() * 4}
    rec_info = None
    if args.entry_records:
        # one pack per page table (a routing decision), each timed on its own
        cur = torch.cuda.current_stream(dev)
        times, nbytes = [], 0
        for p in plans:
            recs = p.pack_records()
            p0, p1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            p0.record(cur)
            p.pack_records(recs)
            p1.record(cur)
            torch.cuda.synchronize()
            times.append(p0.elapsed_time(p1) * 1e3)
            nbytes = recs.numel() * 4
        rec_info = {"pack_us_per_table": round(sum(times) / len(times), 2), "bytes_per_table": nbytes}
    split_plan = N.plan_info(plan.args)
    fused = split_plan["merge_in_kernel"]
    nsets = len(plans)
    stream = torch.cuda.current_stream(dev)
    for i in range(args.warmup):
        plans[i % nsets].run()
    torch.cuda.synchronize()
    # timed region: K back-to-back steps between two events on the kernels' stream
    t_start, t_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record(stream)
    for i in range(args.steps):
        plans[i % nsets].run()
    t_end.record(stream)
    torch.cuda.synchronize()
    total_ms = t_start.elapsed_time(t_end)
    # second pass of K steps: events around every step (spread) and, recorded by
    # the library on the same stream, around the split kernel alone (roofline);
    # event records cost a few microseconds each, so they stay out of `value`
    ev = kernel_events(args.steps)
    kev = kernel_events(args.steps)
    for i, ((s, e), k) in enumerate(zip(ev, kev)):
        s.record(stream)
        plans[i % nsets].run(events=k)
        e.record(stream)
    torch.cuda.synchronize()
    per = sorted(s.elapsed_time(e) for s, e in ev)
    kernel_ms_events = sum(b.elapsed_time(e) for b, e in kev) / args.steps
    ms = total_ms / args.steps
    # The split kernel is timed by the event pair the library records around
    # it, bounded by the step time of the timed region (events around K
    # back-to-back steps): with the merge inside the decode kernel a step is
    # that one launch, the gap between launches included; with a merge kernel
    # the step (split kernel + merge) still bounds the split kernel from above.
    # A per-launch pair adds its records' cost and the launch's dispatch and
    # completion, and on some boxes reads longer than the whole step.
    kernel_ms = min(ms, kernel_ms_events)
    kernel_timing = ("HIP events around each split-kernel launch" if kernel_ms_events <= ms else
                     "events around the K back-to-back launches of the timed region (one launch per step)" if fused
                     else "events around the K back-to-back steps of the timed region (the split kernel plus the "
                          "merge: an upper bound on the split kernel, below its per-launch event pairs)")
    # bytes of the average step over the rotated page sets
    abs_ = [algorithmic_bytes(wl, t) for t in wl["tables"]]
    ab = dict(abs_[0])
    for key in ("total", "codes", "scales", "meta", "qo", "pages"):
        ab[key] = int(round(sum(x[key] for x in abs_) / nsets))
    ab["per_tag"] = {k: int(round(sum(x["per_tag"][k] for x in abs_) / nsets)) for k in abs_[0]["per_tag"]}
    achieved = ab["total"] / (ms * 1e-3) / 1e9
    # the split kernel moves every algorithmic byte but the output, which the
    # merge kernel writes (unless the decode kernel merges itself); with page
    # descriptors or entry records its metadata bytes are theirs: 32 B per
    # selected page (+ its 4 B table entry), or 32 B per table entry
    kernel_alg, kernel_fmt = ab["total"], "reference tensors"
    if rec_info is not None:
        kernel_alg = ab["codes"] + rec_info["bytes_per_table"] + wl["counts"].numel() * 4 + ab["qo"]
        kernel_fmt = "entry records"
    elif desc_info is not None:
        kernel_alg = ab["codes"] + ab["pages"] * (32 + 4) + wl["counts"].numel() * 4 + ab["qo"]
        kernel_fmt = "page descriptors"
    kernel_bytes = kernel_alg - (0 if fused else ab["qo"] // 2)
    kernel_gbps = kernel_bytes / (kernel_ms * 1e-3) / 1e9
    med = per[len(per) // 2]
    traffic_key = args.config + ("-records" if args.entry_records else "-desc" if args.page_descriptors else "")
    res = {
        "metric": METRIC, "value": round(achieved, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
        "us_per_step": round(ms * 1e3, 2), "us_per_step_p10_p50_p90": [round(per[len(per) // 10] * 1e3, 2),
                                                                       round(med * 1e3, 2),
                                                                       round(per[(9 * len(per)) // 10] * 1e3, 2)],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "data": "synthetic (seeded torch generator; codes = reference fake-quant of N(0,1) fp16 pages)",
        "config": {"workload": f"{args.config}: Llama-3-8B GQA decode B={cfg['B']} Hq={cfg['Hq']} "
                               f"Hkv={cfg['Hkv']} D={cfg['D']} ctx={cfg['T']} page=16 "
                               f"sel={wl['W']} pages/row mix={ {int(k): v for k, v in cfg['mix'].items()} }"
                               + (f", {nsets} disjoint page sets rotated" if nsets > 1 else ""),
                   "selected_pages": ab["pages"], "algorithmic_bytes": ab["total"],
                   "bytes_breakdown": {k: ab[k] for k in ("codes", "scales", "meta", "qo")},
                   "pages_per_tag": ab["per_tag"], "pages_per_split": split_plan["pages_per_split"],
                   "splits_per_row": split_plan["splits"],
                   "tail_splits": split_plan["tail_splits"], "tail_pages_per_split": split_plan["tail_pages_per_split"],
                   "merge": "in the decode kernel" if fused else "merge kernel",
                   "page_descriptors": desc_info,
                   "entry_records": rec_info,
                   "gflop": round(flops(wl) / 1e9, 3)},
        "roofline": {"bound": "hbm", "achieved": round(kernel_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(kernel_gbps / HBM_PEAK_GBPS, 4),
                     "traffic": measured_traffic(traffic_key)[0],
                     "kernel": "paged_decode_kernel", "kernel_us": round(kernel_ms * 1e3, 2),
                     "kernel_timing": kernel_timing, "kernel_us_event_pairs": round(kernel_ms_events * 1e3, 2),
                     "kernel_source_digest": kernel_source_digest(),
                     "kernel_bytes": kernel_bytes, "kernel_metadata_format": kernel_fmt,
                     "step_frac": round(achieved / HBM_PEAK_GBPS, 4)},
    }
    if traffic_key in MEASURED_TRAFFIC:
        res["roofline"]["traffic_source"] = measured_traffic(traffic_key)[1]
    plain = not (args.page_descriptors or args.entry_records or args.calibrate_copy or args.no_variants)
    if plain and args.config in MEASURED_TRAFFIC:
        res["variants"] = metadata_variants(plans, args.steps, stream, ab["total"], args.config)
        # the product's default plan: entry records packed by the plan itself at its
        # second run over an unchanged table (the packs fall in the warm-up)
        auto = [make_plan(wl["q"], wl["pools"], t, wl["counts"], wl["tags"], out=out,
                          pages_per_split=args.pages_per_split, merge_in_kernel=merge) for t in wl["tables"]]
        for i in range(max(args.warmup, 2 * nsets)):
            auto[i % nsets].run()
        torch.cuda.synchronize()
        assert all(p.reads_records for p in auto)
        a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a0.record(stream)
        for i in range(args.steps):
            auto[i % nsets].run()
        a1.record(stream)
        torch.cuda.synchronize()
        ams = a0.elapsed_time(a1) / args.steps
        res["variants"]["default_plan"] = {
            "us_per_step": round(ams * 1e3, 2), "value": round(ab["total"] / (ams * 1e-3) / 1e9, 1), "unit": "GB/s",
            "note": "make_plan's default (auto_records): entry records packed by the plan at its second run "
                    "over an unchanged table and read from then on"}
        del auto
    if args.calibrate_copy:
        n = args.calibrate_copy * (1 << 20)
        src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        res["copy_calibration_bytes"] = n
        # the same copy timed: this GPU's read + write streaming rate, the
        # ceiling of kernels that stream as much as they read
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(5):
            dst.copy_(src)
        e1.record(stream)
        torch.cuda.synchronize()
        res["copy_read_write_gbps"] = round(2 * n / (e0.elapsed_time(e1) / 5 * 1e-3) / 1e9, 1)
    if cpu is not None:
        rows = cfg["B"] * cfg["Hkv"]
        res["cpu_baseline"] = cpu_baseline_decode(args.config, cpu, ab["total"], rows)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
