"""GPU: the bench's workload quantised on the device is bit-exact to the
oracle, and the decode of that workload (all five precisions) matches the
oracle within the quantised-page tolerance."""
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
