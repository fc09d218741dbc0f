"""The C ABI library loads without a GPU and exports every function that
include/kvm_hotpath.h declares (no compute calls here)."""
import ctypes
import re

from kvmem_amd import _lib as L


def _declared():
    src = open(L.HEADER_PATH).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = re.findall(r"^[a-z_][a-z0-9_ \*]*?\b(kvm_[a-z0-9_]+)\s*\(", src, flags=re.M)
    return sorted(set(names))


def test_header_declares_entry_points():
    names = _declared()
    for must in ("kvm_state_create", "kvm_score_topk", "kvm_select_topk", "kvm_stagein_selection",
                 "kvm_stagein_enqueue_k", "kvm_fa_decode", "kvm_fa_prefill", "kvm_fa_decode_lanes"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(L.LIB_PATH)
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_header():
    assert set(_declared()) == set(L.SIGNATURES)


def test_abi_version_without_gpu():
    assert L.load().kvm_abi_version() == 2
