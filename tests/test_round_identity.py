"""The requantizing GEMM epilogues round with
x86_round_cvt(y) = trunc(y + copysign(0.49999997f, y)) plus one range test
(rpl_amd/csrc/hip/common.h) instead of roundf + cvttss2si.  This checks the
identity for all 2^32 float bit patterns on the CPU, against glibc roundf
(the function the reference calls, src/ops_extended.c:119-120)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_round_identity_all_floats(tmp_path):
    exe = tmp_path / "round_identity"
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", "-fno-fast-math", "-o", str(exe),
                    os.path.join(HERE, "round_identity.c"), "-lm"], check=True)
    env = dict(os.environ, OMP_NUM_THREADS=str(min(8, os.cpu_count() or 1)))
    r = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip() == "mismatches 0"


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_quantizer_division_identity(tmp_path):
    """The per-channel quantizer divides by its row scale s as
    fma(fma(-q, s, x), 1/s, q) with q = x * (1/s) when 2^-100 <= s <= 2^125
    (rpl_amd/csrc/hip/quant.hip, div_scale_fast) and rounds that quotient
    to a byte as fminf(fmaxf(q + copysign(0.49999997, q), -128), 127)
    truncated (q8_small).  Against x / s and clamp((int32)roundf(.)) (the
    reference, src/rpl_quantization.c:153-154): the quotient bits for every x
    with s/4 <= |x| <= 128 s and the byte for every x up to 128 s, for twelve
    scales, plus 2^25 random pairs."""
    exe = tmp_path / "quant_div_identity"
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", "-fno-fast-math", "-march=x86-64-v3", "-o",
                    str(exe), os.path.join(HERE, "quant_div_identity.c"), "-lm"], check=True)
    env = dict(os.environ, OMP_NUM_THREADS=str(min(8, os.cpu_count() or 1)))
    r = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=900)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr
    assert r.stdout.strip().endswith("mismatches 0"), r.stdout[-2000:]
