"""The quotient by an fp16 scale from its reciprocal and one fma correction
(the baseline-format kernels' division, div_fp16_divisor) equals IEEE
division for every pair of significands: an exhaustive CPU check of the
2^23 x 2^10 pairs (a few seconds on 8 threads)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def _has_fma():
    try:
        return " fma " in open("/proc/cpuinfo").read().replace("\n", " ")
    except OSError:
        return False


@pytest.mark.skipif(shutil.which("gcc") is None or not _has_fma(), reason="needs gcc and a CPU with FMA")
def test_reciprocal_quotient_matches_ieee_division(tmp_path):
    exe = tmp_path / "div_fp16_exhaustive"
    subprocess.run(["gcc", "-O2", "-mfma", "-ffp-contract=off", "-pthread", "-o", str(exe),
                    os.path.join(HERE, "native", "div_fp16_exhaustive.c"), "-lm"], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "mismatches: 0" in res.stdout
