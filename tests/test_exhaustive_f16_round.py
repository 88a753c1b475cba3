"""The quantization passes round r16(a * b) and r16(a + b) of two fp16 values as fp16 products and sums (packed fp16
instructions); over every pair of finite fp16 values both roundings agree: tests/exhaustive_f16_round.c, compiled
with the host gcc. (With the intermediate rounded to 13 significant bits instead of fp32's 24, the same check finds
66.7 million differing sums, so it does distinguish the cases.)"""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_fp16_product_and_sum_rounding_exhaustive(tmp_path):
    exe = str(tmp_path / "exhaustive_f16_round")
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", os.path.join(HERE, "exhaustive_f16_round.c"), "-o", exe, "-lm"], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "mismatches: mul 0, add 0" in r.stdout
