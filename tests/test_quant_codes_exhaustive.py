"""The quant_int4 kernel forms bf16 / fp16 codes without a division per element
(one reciprocal per group and an fma correction; wush_int4_kernel_amd/csrc/quant.hip,
code_plus8).  This CPU test checks that arithmetic against the reference's
division form clamp(rint(RN(v / sf)), -7, 7) (my_int4/rtn_int4.py:50-51) for every
finite bf16 and fp16 v with |v| < 1.8e19 and every bf16 scale sf >= 1e-8: about
2.2e9 pairs, in C (tests/native/quant_codes_exhaustive.c), a few seconds on 8 cores.
The GPU tests then check the kernel bit for bit against the oracle."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_fma_codes_equal_division_for_every_bf16_and_fp16_value(tmp_path):
    exe = tmp_path / "quant_codes_exhaustive"
    src = os.path.join(HERE, "native", "quant_codes_exhaustive.c")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-mfma", "-fopenmp", src, "-o", str(exe), "-lm"],
                   check=True)
    env = dict(os.environ)
    env.setdefault("OMP_NUM_THREADS", str(min(8, os.cpu_count() or 1)))
    out = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=600)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "mismatches 0" in out.stdout


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_fp32_quotients_equal_division_at_ties_and_random(tmp_path):
    # fp32 values (quant_int4 on fp32 input, the fused transform's fp32 x') go
    # through RN(1/sf) and two fma corrections (wush_device.h, quotient_fma);
    # tests/native/quant_codes_fp32.c compares quotient and code with the IEEE
    # division at and next to every rounding tie for every bf16 scale, and on
    # 2^29 random pairs (about 9e8 pairs, a few seconds on 8 cores).  The same
    # pairs check the one-fma codes (wush_device.h, code8_fast) wherever their
    # tie-band test lets them stand.
    exe = tmp_path / "quant_codes_fp32"
    src = os.path.join(HERE, "native", "quant_codes_fp32.c")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-mfma", "-fopenmp", src, "-o", str(exe), "-lm"],
                   check=True)
    env = dict(os.environ)
    env.setdefault("OMP_NUM_THREADS", str(min(8, os.cpu_count() or 1)))
    out = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=600)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "code mismatches 0, quotient mismatches 0, one-fma code mismatches 0" in out.stdout
