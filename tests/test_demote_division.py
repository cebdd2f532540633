"""The transcoding kernel's division, checked exhaustively on the host.

The INT8 demote kernel computes each code from Markstein's corrected product
(q0 = x r, e = fma(-q0, s, x), q = fma(e, r, q0) with r = 1 / s) instead of the
reference's float32 division x / s (kv_memory_manager.py:245-247).
tests/csrc/demote_division_check.c compares the two codes for every positive
finite float16 absmax m and every float16 element |x| <= m; a planted mistake
(the bare product x r, no correction) must make it fail.
"""
import os
import shutil
import subprocess

import pytest

SRC = os.path.join(os.path.dirname(os.path.abspath(__file__)), "csrc", "demote_division_check.c")


def _run(tmp_path, *defs):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    exe = str(tmp_path / ("check" + "".join(defs)))
    cmd = ["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-mf16c", "-mfma", "-fopenmp", *defs, "-o", exe,
           SRC, "-lm"]
    subprocess.run(cmd, check=True, capture_output=True)
    return subprocess.run([exe], capture_output=True, text=True, timeout=600)


def test_corrected_product_gives_the_division_codes(tmp_path):
    r = _run(tmp_path)
    assert r.returncode == 0 and r.stdout.startswith("OK 1007713278 pairs"), r.stdout + r.stderr


def test_planted_uncorrected_product_fails(tmp_path):
    r = _run(tmp_path, "-DPLANT_NO_CORRECTION")
    assert r.returncode == 1 and "MISMATCH" in r.stdout, r.stdout + r.stderr
