"""The C ABI library loads without a GPU and exports every function that
include/kvm_hotpath.h declares (no compute calls here)."""
import ctypes
import ctypes as C
import os
import re
import subprocess

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
    assert L.load().kvm_abi_version() == 6


# ctypes mirror -> C typedef of include/kvm_hotpath.h
_STRUCTS = {
    "Window": "kvm_window", "QueryAcc": "kvm_query_acc", "MeanKIndex": "kvm_meank_index", "View": "kvm_view",
    "SelectParams": "kvm_select_params", "Selection": "kvm_selection", "RetrievalLane": "kvm_retrieval_lane",
    "RopeParams": "kvm_rope_params", "History": "kvm_history", "StageinLane": "kvm_stagein_lane",
    "Lane": "kvm_lane", "SlotPool": "kvm_slot_pool", "RowRange": "kvm_row_range",
    "SnapshotInfo": "kvm_snapshot_info", "SnapshotLayer": "kvm_snapshot_layer",
}


def test_struct_layouts_match_the_header(tmp_path):
    """Every ctypes struct has the size and field offsets the C compiler gives
    the header's struct (a C program compiled with gcc prints them)."""
    src = open(L.HEADER_PATH).read()
    declared = set(re.findall(r"typedef struct (kvm_[a-z0-9_]+) \{", src))
    assert declared == set(_STRUCTS.values()), declared ^ set(_STRUCTS.values())
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "kvm_hotpath.h"', 'int main(void) {']
    want = []
    for py, c in sorted(_STRUCTS.items()):
        cls = getattr(L, py)
        lines.append(f'  printf("%zu\\n", sizeof({c}));')
        want.append(C.sizeof(cls))
        for name, *_ in cls._fields_:
            lines.append(f'  printf("%zu\\n", offsetof({c}, {name}));')
            want.append(getattr(cls, name).offset)
    lines += ['  return 0;', '}']
    (tmp_path / "layout.c").write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.dirname(L.HEADER_PATH),
                    str(tmp_path / "layout.c"), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()]
    assert got == want


def test_c_caller_builds(tmp_path):
    """tests/c/kvm_abi_decode.c, a C99 caller of the library, compiles against the
    header and links against the library (run on the GPU by test_gpu_c_abi.py)."""
    here = os.path.dirname(os.path.abspath(__file__))
    exe = tmp_path / "kvm_abi_decode"
    subprocess.run(["sh", os.path.join(here, "c", "build.sh"), str(exe)], check=True)
    assert exe.exists()
