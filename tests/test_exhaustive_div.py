"""div_by_scale (the quantizers' x / scale from a per-row reciprocal) against the correctly rounded division, over
every fp16 value and every fp16 absmax: tests/exhaustive_div.c, compiled with the host gcc."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_div_by_scale_exhaustive(tmp_path):
    exe = str(tmp_path / "exhaustive_div")
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", os.path.join(HERE, "exhaustive_div.c"), "-o", exe, "-lm"], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "mismatches: int8 scale 0, int4 scale 0" in r.stdout
