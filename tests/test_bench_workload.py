"""The bench's synthetic workload: codes and scales of every precision are
bit-exact to the oracle's page-granule quantiser (the reference's
fake_quantize_tensor arithmetic), built here on CPU tensors; the GPU variant
of the same check runs in tests/test_gpu_workload.py."""
import numpy as np
import pytest
import torch

import bench
from oracle import quant as Q


def check_workload_codes(wl, sample=40, seed=0):
    p = wl["pools"]
    tags = wl["tags"].cpu().numpy()
    rng = np.random.default_rng(seed)
    names = {bench.TAG_FP8: "FP8", bench.TAG_INT8: "INT8", bench.TAG_INT4: "INT4",
             bench.TAG_INT4R: "INT4_RESIDUAL"}
    checked = {t: 0 for t in names}
    for pid in rng.permutation(len(tags)):
        t = int(tags[pid])
        if t not in names or checked[t] >= sample:
            continue
        checked[t] += 1
        for w in ("k", "v"):
            page = getattr(p, f"{w}_fp16")[pid].cpu().numpy()
            codes, scales = Q.quantize_page(page, names[t])
            if t == bench.TAG_FP8:
                assert np.array_equal(getattr(p, f"{w}_fp8")[pid].cpu().numpy(), codes)
                assert np.float16(getattr(p, f"{w}_fp8_scale")[pid].item()) == scales[0]
            elif t == bench.TAG_INT8:
                assert np.array_equal(getattr(p, f"{w}_int8")[pid].cpu().numpy(), codes)
                assert np.float16(getattr(p, f"{w}_int8_scale")[pid].item()) == scales[0]
            elif t == bench.TAG_INT4:
                assert np.array_equal(getattr(p, f"{w}_int4")[pid].cpu().numpy(), Q.pack_int4(codes))
                assert np.array_equal(getattr(p, f"{w}_int4_scale")[pid].cpu().numpy(), scales)
            else:
                (q1, q2), (s1, s2) = codes, scales
                assert np.array_equal(getattr(p, f"{w}_int4r")[pid].cpu().numpy(), Q.pack_int4_residual(q1, q2))
                got = getattr(p, f"{w}_int4r_scale")[pid].cpu().numpy()
                assert got[0] == np.float32(s1[0]) and got[1] == s2[0]
    assert all(v > 0 for v in checked.values()), checked
    return checked


def test_tiny_workload_codes_match_oracle():
    wl = bench.build_workload("tiny", torch.device("cpu"), chunk_pages=200)
    check_workload_codes(wl)
    ab = bench.algorithmic_bytes(wl)
    assert ab["pages"] == 2 * 2 * int(0.4 * 128)
    assert ab["total"] > ab["codes"] > 0


def test_bench_refuses_more_than_one_gpu(monkeypatch, capsys):
    monkeypatch.setattr("sys.argv", ["bench.py", "--gpus", "2"])
    with pytest.raises(SystemExit) as e:
        bench.main()
    assert e.value.code == 2 and "one GPU" in capsys.readouterr().err


def test_measured_traffic_is_tied_to_the_kernel_sources(monkeypatch):
    """roofline.traffic comes from counter runs of one build of the decode
    kernel: reported while the kernel's sources hash to the digest it was
    measured on, null (with the reason) for any other sources."""
    digest = bench.kernel_source_digest()
    assert len(digest) == 16
    for key, m in bench.MEASURED_TRAFFIC.items():
        assert m["src"] == digest, f"{key}: measured on {m['src']}, sources are {digest}"
        got, src = bench.measured_traffic(key)
        assert got == m["bytes"] and src == m["source"]
    monkeypatch.setattr(bench, "kernel_source_digest", lambda: "0" * 16)
    got, why = bench.measured_traffic("cfg3")
    assert got is None and "stale" in why
    assert bench.measured_traffic("cfg2") == (None, None)
