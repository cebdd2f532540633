"""GPU: the bench's workload quantised on the device is bit-exact to the
oracle, and the decode of that workload (all five precisions) matches the
oracle within the quantised-page tolerance.

At the benchmark's full sizes the near-uniform softmax of cfg2-cfg4 (q
scaled by 1/sqrt(128) over 13k-26k tokens) gives outputs of ~6e-3, so the
absolute bars of the task (2e-3 FP16, 1e-2 quantised) are joined by a
relative bar (max|err| / max|ref| <= 1e-2) and a cosine bar per row, a
peaked-softmax variant (q not divided by sqrt(128), and 4x that), and a
negative control: the same plan with one precision class mapped to SKIP must
fail the relative bar, which shows the comparison can see a dropped class."""
import numpy as np
import pytest
import torch

import bench
from oracle.decode import paged_decode_oracle
from tests.test_bench_workload import check_workload_codes

pytestmark = pytest.mark.gpu


def test_device_workload_codes_and_decode():
    print("[gpu-case] bench tiny workload on cuda:0", flush=True)
    dev = torch.device("cuda:0")
    wl = bench.build_workload("tiny", dev, chunk_pages=100)
    check_workload_codes(wl, sample=25)
    from intent_attention import paged_decode
    out = paged_decode(wl["q"], wl["pools"], wl["table"], wl["counts"], wl["tags"], out_dtype=torch.float32)
    p = wl["pools"]
    pools = {"k_fp16": p.k_fp16.cpu().numpy(), "v_fp16": p.v_fp16.cpu().numpy()}
    for nm, src in (("fp8", "fp8"), ("i8", "int8"), ("i4", "int4"), ("i4r", "int4r")):
        for w in ("k", "v"):
            pools[f"{w}_{nm}"] = getattr(p, f"{w}_{src}").cpu().numpy()
            pools[f"{w}_{nm}_scale"] = getattr(p, f"{w}_{src}_scale").cpu().numpy()
    ref = paged_decode_oracle(wl["q"].cpu().numpy(), pools, wl["table"].cpu().numpy(),
                              wl["counts"].cpu().numpy(), wl["tags"].cpu().numpy())
    err = np.abs(out.cpu().numpy() - ref).max()
    print(f"[gpu-case] tiny workload max abs err {err:.2e}", flush=True)
    assert err <= 1e-2


def _row_oracle(wl, rows):
    """Oracle output of the given (batch * kv_head) rows of a bench workload:
    their pages gathered to the host, everything else as the bench builds it."""
    cfg = wl["cfg"]
    B, Hkv, G, D = cfg["B"], cfg["Hkv"], cfg["Hq"] // cfg["Hkv"], cfg["D"]
    table = wl["table"].reshape(B * Hkv, -1)
    ids = table[rows].flatten()
    uniq, inv = torch.unique(ids, return_inverse=True)
    p = wl["pools"]

    def host(t):
        return t[uniq.long()].cpu().numpy()

    pools = {"k_fp16": host(p.k_fp16), "v_fp16": host(p.v_fp16)}
    for nm, src in (("fp8", "fp8"), ("i8", "int8"), ("i4", "int4"), ("i4r", "int4r")):
        for w in ("k", "v"):
            if getattr(p, f"{w}_{src}") is not None:
                pools[f"{w}_{nm}"] = host(getattr(p, f"{w}_{src}"))
                pools[f"{w}_{nm}_scale"] = host(getattr(p, f"{w}_{src}_scale"))
    tags = wl["tags"][uniq.long()].cpu().numpy()
    tbl = inv.reshape(len(rows), 1, -1).cpu().numpy().astype(np.int32)
    cnt = wl["counts"].reshape(B * Hkv)[rows].reshape(len(rows), 1).cpu().numpy()
    q = wl["q"].reshape(B, Hkv, G, D).reshape(B * Hkv, G, D)[rows].cpu().numpy()
    return paged_decode_oracle(q, pools, tbl, cnt, tags, dtype=np.float32)


REL_BAR = 1e-2        # max|got - ref| / max|ref| over the checked rows
COS_BAR = 0.9999      # cosine similarity of every checked (row, head)
# negative controls: (tag mapped to SKIP, its share of the pages)
DROP = {"cfg3": bench.TAG_INT4, "cfg4": bench.TAG_FP16}


def _metrics(got, ref):
    """(max abs err, max abs err / max |ref|, worst per-head cosine)."""
    d = np.abs(got - ref)
    a = got.reshape(-1, got.shape[-1]).astype(np.float64)
    b = ref.reshape(-1, ref.shape[-1]).astype(np.float64)
    cos = (a * b).sum(1) / np.maximum(np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1), 1e-300)
    return float(d.max()), float(d.max() / np.abs(ref).max()), float(cos.min())


@pytest.mark.parametrize("name,tol", [("cfg2", 2e-3), ("cfg3", 1e-2), ("cfg4", 1e-2)])
def test_full_config_sampled_rows(name, tol):
    """The benchmark's own configurations at full size through the same plan the
    bench times; 6 rows spread over the batch checked against the oracle with
    absolute, relative and cosine bars, for the bench's query scale and for
    peaked softmaxes (q times sqrt(128) and 4 sqrt(128)); then the negative
    control. The same decode reading packed page descriptors, and packed entry
    records, gives every output bit-identical."""
    print(f"[gpu-case] full {name} workload, sampled rows", flush=True)
    from intent_attention.decode_core import NATIVE_TAG_MAP, make_plan
    dev = torch.device("cuda:0")
    wl = bench.build_workload(name, dev)
    cfg = wl["cfg"]
    R = cfg["B"] * cfg["Hkv"]
    G = cfg["Hq"] // cfg["Hkv"]
    rows = sorted({0, R - 1, *range(R // 6, R, R // 6)})[:6]
    q0 = wl["q"]
    mults = [1.0, 128 ** 0.5] + ([4 * 128 ** 0.5] if name == "cfg3" else [])
    ref = None
    for mult in mults:
        wl["q"] = (q0.float() * mult).half() if mult != 1.0 else q0
        out = torch.empty((cfg["B"], cfg["Hq"], cfg["D"]), dtype=torch.float32, device=dev)
        plan0 = make_plan(wl["q"], wl["pools"], wl["table"], wl["counts"], wl["tags"], out=out)
        plan0.run()
        torch.cuda.synchronize()
        if mult == 1.0:
            from intent_attention import _native as N
            info = N.plan_info(plan0.args)
            print(f"[gpu-case] {name} plan {info}", flush=True)
            if name == "cfg3":   # the grid the two-tier plan is for
                assert info["tail_splits"] > 0
            for form in ("page descriptors", "entry records"):
                alt = torch.full_like(out, float("nan"))
                plan = make_plan(wl["q"], wl["pools"], wl["table"], wl["counts"], wl["tags"], out=alt)
                packed = plan.pack_descriptors() if form == "page descriptors" else plan.pack_records()
                plan.run()
                torch.cuda.synchronize()
                print(f"[gpu-case] {name} with {form}: bit-identical {bool(torch.equal(alt, out))}", flush=True)
                assert torch.equal(alt, out)
                del alt, plan, packed
        ref = _row_oracle(wl, rows).reshape(len(rows), G, cfg["D"])
        got = out.reshape(R, G, cfg["D"])[rows].cpu().numpy()
        err, rel, cos = _metrics(got, ref)
        print(f"[gpu-case] {name} q x {mult:.2f} rows {rows}: max abs err {err:.2e}, relative {rel:.2e}, "
              f"min cosine {cos:.7f}, max |ref| {np.abs(ref).max():.3e}", flush=True)
        assert err <= tol    # the fixed absolute bar, also for the peaked softmaxes
        assert rel <= REL_BAR and cos >= COS_BAR
        if mult == 1.0 and name in DROP:
            # negative control: one precision class read as SKIP must fail the same bars
            skip = NATIVE_TAG_MAP[2]
            tm = [t if wl["pools"].has(t) else skip for t in NATIVE_TAG_MAP]
            tm[DROP[name]] = skip
            bad = torch.empty_like(out)
            make_plan(wl["q"], wl["pools"], wl["table"], wl["counts"], wl["tags"], out=bad, tag_map=tm).run()
            torch.cuda.synchronize()
            berr, brel, bcos = _metrics(bad.reshape(R, G, cfg["D"])[rows].cpu().numpy(), ref)
            print(f"[gpu-case] {name} negative control (tag {DROP[name]} read as SKIP): max abs err {berr:.2e}, "
                  f"relative {brel:.2e}, min cosine {bcos:.5f}", flush=True)
            assert brel > 5 * REL_BAR and bcos < COS_BAR
    del wl, out
    torch.cuda.empty_cache()


def _mla_seq_oracle(wl, b, v_dim):
    """Oracle latent context of sequence ``b`` of an MLA bench workload (its
    pages gathered to the host)."""
    from oracle.mla import mla_paged_decode_oracle
    p = wl["pools"]
    ids = wl["tables"][0][b].long()
    uniq, inv = torch.unique(ids, return_inverse=True)
    pools = {"c_fp8": p.c_fp8[uniq].cpu().numpy(), "c_fp8_scale": p.c_fp8_scale[uniq].cpu().numpy(),
             "c_i8": p.c_int8[uniq].cpu().numpy(), "c_i8_scale": p.c_int8_scale[uniq].cpu().numpy()}
    return mla_paged_decode_oracle(wl["q"][b:b + 1].cpu().numpy(), pools,
                                   inv[None].cpu().numpy().astype(np.int32), np.array([wl["W"]]),
                                   wl["tags"][uniq].cpu().numpy(), v_dim=v_dim)[0]


def test_full_mla_config_sampled_sequences():
    """cfg5 (MLA) at full size through the bench's plan; 3 sequences against the
    oracle with the absolute bar (1e-2), the relative bar (max err / max |ref|
    <= 1e-2) and the per-head cosine bar (>= 0.9999). cfg5's outputs are small
    (max |out| ~0.2), so the absolute bar alone would pass a 5 % scale error on
    a whole precision class; the negative control maps the FP8 class (half the
    pages) to SKIP and must fail the relative and cosine bars."""
    print("[gpu-case] full cfg5 MLA workload, sampled sequences", flush=True)
    from intent_attention import _native as N
    from intent_attention.mla_core import LATENT_TAG_MAP, make_mla_plan
    dev = torch.device("cuda:0")
    wl = bench.build_mla_workload("cfg5", dev)
    cfg = wl["cfg"]
    seqs = (0, cfg["B"] // 2, cfg["B"] - 1)
    out = torch.empty((cfg["B"], cfg["H"], cfg["DV"]), dtype=torch.float32, device=dev)
    make_mla_plan(wl["q"], wl["pools"], wl["tables"][0], wl["counts"], wl["tags"], v_dim=cfg["DV"], out=out).run()
    tm = [t if wl["pools"].has(t) else N.TAG_SKIP for t in LATENT_TAG_MAP]
    tm[N.TAG_FP8] = N.TAG_SKIP
    bad = torch.empty_like(out)
    make_mla_plan(wl["q"], wl["pools"], wl["tables"][0], wl["counts"], wl["tags"], v_dim=cfg["DV"], out=bad,
                  tag_map=tm).run()
    torch.cuda.synchronize()
    ref = np.stack([_mla_seq_oracle(wl, b, cfg["DV"]) for b in seqs])
    got = out[list(seqs)].cpu().numpy()
    err, rel, cos = _metrics(got, ref)
    print(f"[gpu-case] cfg5 sequences {seqs}: max abs err {err:.2e}, relative {rel:.2e}, min cosine {cos:.7f}, "
          f"max |ref| {np.abs(ref).max():.3e}", flush=True)
    assert err <= 1e-2 and rel <= REL_BAR and cos >= COS_BAR
    berr, brel, bcos = _metrics(bad[list(seqs)].cpu().numpy(), ref)
    print(f"[gpu-case] cfg5 negative control (FP8 pages read as SKIP): max abs err {berr:.2e}, relative {brel:.2e}, "
          f"min cosine {bcos:.5f}", flush=True)
    assert brel > 5 * REL_BAR and bcos < COS_BAR
    del wl, out, bad
    torch.cuda.empty_cache()
