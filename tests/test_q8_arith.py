"""Exhaustive check of the shortened q8_1 quantizer arithmetic of the streaming kernels
(q8_div127 and q8_round_mul in glm-ssd_amd/csrc/kernels.hip): the C program in tests/arith/
compares them with IEEE division and roundf over every input of their ranges (~20 s)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_q8_arith_exhaustive(tmp_path):
    exe = tmp_path / "q8_arith_check"
    subprocess.run(["gcc", "-O2", "-o", str(exe), os.path.join(HERE, "arith", "q8_arith_check.c"), "-lm"],
                   check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout + r.stderr
