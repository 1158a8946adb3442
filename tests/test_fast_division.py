"""The few-token quantiser's division-free scale and reciprocal
(act_scale_reciprocal_fast, fp8_gemm_h20/csrc/fp8bg.hip) are the correctly
rounded quotients on their whole domain: an exhaustive check in C
(tests/fastdiv_check.c), compiled with gcc and run on the CPU.  The
quantiser's scale and reciprocal follow the reference recipe
(/root/reference/scripts/validate.py:21-30: s = amax / 448; the fused path
multiplies by the fp32 reciprocal of s), so the fast sequence must give
bitwise the same s and 1/s as the divisions."""
import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc is not installed")
def test_fast_scale_and_reciprocal_are_correctly_rounded(tmp_path):
    exe = tmp_path / "fastdiv_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), str(HERE / "fastdiv_check.c"), "-lm"],
                   check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    ok, n_div, n_rcp, plain_bad = res.stdout.split()
    assert ok == "ok"
    assert int(n_div) == 0x7f80 - 1                       # every positive finite bf16
    assert int(n_rcp) == 5 * sum(1 for h in range(1, 0x7f80) if h >= 0x0d80)   # x >= 2^-100, five starts each
    assert int(plain_bad) > 10000                         # the FMA correction is needed


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc is not installed")
def test_per_value_division_by_the_scale_is_correctly_rounded(tmp_path):
    # div_by_scale (the standalone activation quantiser's e4m3(x / s), the
    # reference's a / sa at /root/reference/scripts/validate.py:27)
    exe = tmp_path / "divscale_check"
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", "-o", str(exe),
                    str(HERE / "divscale_check.c"), "-lm"], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stdout + res.stderr
    ok, pairs, plain_bad = res.stdout.split()
    assert ok == "ok" and int(pairs) == (1 << 23) * 256
    assert int(plain_bad) > 1000000                       # the FMA correction is needed
