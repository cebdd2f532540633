"""The quantiser's float16 division (csrc/quantize.hip, div_by_scale): a
reciprocal and one FMA correction instead of an IEEE division per element.
Checked exhaustively on the host over every finite float16 numerator and every
positive finite float16 scale (2.0e9 pairs): the float16-rounded quotient is
bit-identical to the reference's fl16(x / s), signed zeros included. The same
check without the correction step finds mismatches."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CLANG = "/opt/rocm/llvm/bin/clang"


@pytest.mark.skipif(not os.path.exists(CLANG), reason="needs ROCm's clang (host _Float16)")
def test_reciprocal_fma_quotient_is_exact_for_all_float16(tmp_path):
    exe = str(tmp_path / "qc")
    subprocess.run([CLANG, "-O2", "-ffp-contract=off", "-fopenmp", os.path.join(HERE, "native", "f16_quotient_check.c"),
                    "-o", exe, "-lm", "-Wl,-rpath,/opt/rocm/llvm/lib"], check=True)
    out = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout[-2000:]
    assert out.stdout.strip().endswith("checked 2015299584 mismatches 0")
    bad = subprocess.run([exe, "uncorrected"], capture_output=True, text=True, timeout=300)
    assert bad.returncode != 0 and int(bad.stdout.split()[-1]) > 1000
