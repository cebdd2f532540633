"""Host AddressSanitizer over the C ABI's argument validation (no GPU).

Builds iak_api.hip with host-side ASan (device code uninstrumented), links it
with the library's other objects from the in-tree build and a driver
(tests/native/abi_validation_asan.cpp) that feeds every entry point random,
edge-valued and well-formed arguments that validation either rejects or
answers on the host (workspace sizes, split plans), and checks that ASan
reports nothing and that well-formed plans are consistent."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(ROOT, "intent-attention-kernel_amd", "csrc")
BUILD = os.path.join(CSRC, "_build")
ROCM = "/opt/rocm"
OTHERS = ("paged_decode", "mla_decode", "mla_rows", "dense_attention", "fake_quant", "quantize", "page_tables", "memory_manager")


def test_abi_validation_under_host_asan(tmp_path):
    objs = [os.path.join(BUILD, f"{n}.o") for n in OTHERS]
    if not all(os.path.exists(o) for o in objs) or not os.path.exists(f"{ROCM}/bin/hipcc"):
        pytest.skip("needs the in-tree build (make -C intent-attention-kernel_amd/csrc) and hipcc")
    inc = ["-I", os.path.join(ROOT, "include"), "-I", CSRC]
    api = str(tmp_path / "iak_api_asan.o")
    # host-side instrumentation only: each sanitizer flag applies to the host pass
    subprocess.run([f"{ROCM}/bin/hipcc", "-O1", "-g", "-std=c++17", "-fPIC", "--offload-arch=gfx950", *inc,
                    "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer",
                    "-c", os.path.join(CSRC, "iak_api.hip"), "-o", api], check=True, capture_output=True)
    drv = str(tmp_path / "drv.o")
    subprocess.run([f"{ROCM}/llvm/bin/clang++", "-O1", "-g", "-std=c++17", "-fsanitize=address",
                    "-fno-omit-frame-pointer", *inc, "-c", os.path.join(HERE, "native", "abi_validation_asan.cpp"),
                    "-o", drv], check=True, capture_output=True)
    exe = str(tmp_path / "abi_asan")
    subprocess.run([f"{ROCM}/llvm/bin/clang++", "-fsanitize=address", drv, api, *objs, f"-L{ROCM}/lib",
                    "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib", "-o", exe], check=True, capture_output=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300, env=env)
    assert "AddressSanitizer" not in r.stderr, r.stderr[-4000:]
    assert r.returncode == 0, (r.stdout, r.stderr[-2000:])
    assert "abi-asan:" in r.stdout
    calls, rejected = (int(x) for x in r.stdout.split("abi-asan:")[1].replace(",", "").split()[0:3:2])
    assert calls > 100000 and 0 < rejected < calls
