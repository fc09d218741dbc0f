"""A plain C program drives the library through include/kvm_hotpath.h alone
(tests/c/kvm_abi_decode.c): window import and export of ggml rows, one decode
launch checked against the C oracle, and an error path's status and message."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "c", "kvm_abi_decode")


def test_c_caller_decodes_through_the_abi(tmp_path):
    exe = BIN
    if not os.path.exists(exe):                     # built by __graft_entry__.build()
        exe = str(tmp_path / "kvm_abi_decode")
        subprocess.run(["sh", os.path.join(HERE, "c", "build.sh"), exe], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)
    assert r.stdout.startswith("ok ") and "ok step on the caller's stream" in r.stdout, r.stdout
