"""The device quantisers' division-free helpers (kvm_internal.h:
kvm_recip_or0, kvm_div127, kvm_round_away) equal the IEEE operations they
replace on gfx950 for every input: tests/c/exact_rounding_gpu.hip runs them
against the device's own IEEE division and roundf over all finite floats.
The reciprocal's Newton step starts from v_rcp_f32, so only the hardware can
pin it; the host check of the other two is tests/test_exact_rounding.py."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "c", "exact_rounding_gpu")


def test_quantiser_helpers_exhaustive_on_device(tmp_path):
    exe = BIN
    if not os.path.exists(exe):                     # built by __graft_entry__.build()
        exe = str(tmp_path / "exact_rounding_gpu")
        subprocess.run(["sh", os.path.join(HERE, "c", "build_exact_gpu.sh"), exe], check=True)
    print("exhaustive helper check:", exe, flush=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=100)
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)
    assert r.stdout.startswith("ok "), r.stdout
