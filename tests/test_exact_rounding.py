"""The device quantisers' division-free forms of IEEE operations
(kvm_internal.h: kvm_div127 for d = amax / 127 and kvm_round_away for roundf,
as the q8_0 quantiser of llama-kvmem-stagein.cu:181-207 computes them) equal
the IEEE operations on every input they can see: an exhaustive check over all
finite floats, in C on the host (tests/c/exact_rounding.c).  The reciprocal's
Newton step (kvm_recip_or0) depends on v_rcp_f32 and is covered by the GPU
parity tests of every quantiser."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="no gcc")
def test_div127_and_round_away_exhaustive(tmp_path):
    exe = str(tmp_path / "exact_rounding")
    subprocess.run(["gcc", "-std=c99", "-O2", "-fopenmp", "-ffp-contract=off", "-o", exe,
                    os.path.join(HERE, "c", "exact_rounding.c"), "-lm"], check=True)
    env = dict(os.environ, OMP_NUM_THREADS=str(min(8, os.cpu_count() or 1)))
    r = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "div127 mismatches 0, round_away mismatches 0" in r.stdout
