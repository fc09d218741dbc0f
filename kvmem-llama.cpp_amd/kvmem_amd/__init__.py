"""MI355X (gfx950) KVMem retrieval + attention hot path: Python host mirror of
the C ABI in include/kvm_hotpath.h.  All compute runs in libkvm_hotpath.so."""
from . import _lib  # noqa: F401
from ._lib import KvmError, load  # noqa: F401
