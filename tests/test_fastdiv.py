"""The act-quant kernels divide by the group scale with one IEEE reciprocal
per group and an FMA correction per element (act_quant.hip, div_by_scale).
This checks that formula against IEEE division over its whole input domain
(every bf16 x, every bf16 group amax >= |x|): any quotient that differs is
below 2^-12, where float8_e4m3fn rounds to a signed zero, so the fp8 output
is the one IEEE division gives (the contract q = e4m3fn(x / s) that the
oracle states with IEEE division). The GPU tests then compare the kernels
with the oracle bit for bit."""
import shutil
import subprocess
from pathlib import Path

import pytest


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_fast_division_matches_ieee_for_fp8(tmp_path):
    src = Path(__file__).parent / "fastdiv_check.c"
    exe = tmp_path / "fastdiv_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fopenmp", str(src), "-o", str(exe),
                    "-lm"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    assert r.returncode == 0, r.stdout
    fields = dict(kv.split("=") for kv in r.stdout.split())
    assert int(fields["pairs"]) > 10**9
    assert fields["large"] == "0" and fields["sign"] == "0"


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_division_free_scale_and_reciprocal(tmp_path):
    """The kernels form scale = amax/448 with one multiply and two FMAs and
    its reciprocal from v_rcp_f32 with one Newton step; both must give the
    IEEE results bit for bit on their whole domain (scale_recip_check.c)."""
    src = Path(__file__).parent / "scale_recip_check.c"
    exe = tmp_path / "scale_recip_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", str(src), "-o", str(exe), "-lm"],
                   check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout
    fields = dict(kv.split("=") for kv in r.stdout.split())
    assert int(fields["scales"]) == 0x7F80 and fields["scale_bad"] == "0"
    assert fields["allones_scales"] == "0"
    assert int(fields["recip_bad_mantissas"]) <= 1  # only the all-ones mantissa
