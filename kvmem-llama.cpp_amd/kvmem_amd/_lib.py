"""ctypes binding of include/kvm_hotpath.h (the C ABI of libkvm_hotpath.so).

The library is the product: every GPU computation goes through it.  Loading
fails loudly when the shared library has not been built.
"""
import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.dirname(_HERE)
LIB_PATH = os.path.join(PKG_DIR, "lib", "libkvm_hotpath.so")
HEADER_PATH = os.path.join(os.path.dirname(PKG_DIR), "include", "kvm_hotpath.h")

KVM_OK, KVM_EINVAL, KVM_EHIP, KVM_ENOMEM, KVM_ERANGE, KVM_EUNSUPPORTED, KVM_ETIMEOUT = 0, -1, -2, -3, -4, -5, -6
WAIT_MERGE, WAIT_PLAN, WAIT_STAGE = 1, 2, 4
WAIT_POLLS_DEFAULT = 1 << 21
T_F32, T_F16, T_Q4_0, T_Q8_0, T_BF16 = 0, 1, 2, 8, 30
TILE_CELLS = 64
MAX_TOPK_BLOCKS = 8192
NOALLOC_SCRATCH_BYTES = 16 << 20
STATUS_NAMES = {0: "KVM_OK", -1: "KVM_EINVAL", -2: "KVM_EHIP", -3: "KVM_ENOMEM",
                -4: "KVM_ERANGE", -5: "KVM_EUNSUPPORTED", -6: "KVM_ETIMEOUT"}


class KvmError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"{STATUS_NAMES.get(code, code)}: {msg}")
        self.code = code


class Window(C.Structure):
    _fields_ = [("n_cells", C.c_uint32), ("n_head_kv", C.c_uint32), ("head_dim", C.c_uint32),
                ("block_tokens", C.c_uint32), ("k_type", C.c_int32), ("v_type", C.c_int32),
                ("k", C.c_void_p), ("v", C.c_void_p), ("cell_pos", C.c_void_p),
                ("slot_block", C.c_void_p), ("slot_base", C.c_void_p),
                ("k_shadow", C.c_void_p), ("shadow_rows", C.c_void_p), ("pending_rows", C.c_void_p)]


class QueryAcc(C.Structure):
    _fields_ = [("n_layer", C.c_uint32), ("n_head", C.c_uint32), ("head_dim", C.c_uint32),
                ("q_sum", C.c_void_p), ("q_count", C.c_void_p), ("n_head_kv", C.c_uint32),
                ("q_vec", C.c_void_p), ("q_norm", C.c_void_p)]


class MeanKIndex(C.Structure):
    _fields_ = [("n_layer", C.c_uint32), ("n_blocks", C.c_uint32), ("n_head_kv", C.c_uint32),
                ("head_dim", C.c_uint32), ("block_tokens", C.c_uint32), ("k_sum", C.c_void_p),
                ("mean_tokens", C.c_void_p), ("present", C.c_void_p), ("acc", C.c_void_p), ("k_norm", C.c_void_p)]


class View(C.Structure):
    _fields_ = [("data", C.c_void_p), ("type", C.c_int), ("ne0", C.c_int64), ("ne1", C.c_int64),
                ("ne2", C.c_int64), ("nb0", C.c_size_t), ("nb1", C.c_size_t), ("nb2", C.c_size_t)]


class SelectParams(C.Structure):
    _fields_ = [("n_blocks", C.c_uint32), ("budget_blocks", C.c_uint32), ("sink_blocks", C.c_uint32),
                ("recent_blocks", C.c_uint32), ("mandatory", C.c_void_p), ("n_mandatory", C.c_uint32),
                ("n_tokens", C.c_void_p)]


class Selection(C.Structure):
    _fields_ = [("cap", C.c_uint32), ("scores", C.c_void_p), ("ids", C.c_void_p),
                ("to_base", C.c_void_p), ("stage_slots", C.c_void_p), ("info", C.c_void_p),
                ("stage_src", C.c_void_p), ("stage_out", C.c_void_p)]


class RetrievalLane(C.Structure):
    _fields_ = [("ix", C.POINTER(MeanKIndex)), ("q", C.POINTER(QueryAcc)), ("p", C.POINTER(SelectParams)),
                ("w", C.POINTER(Window)), ("out", C.POINTER(Selection))]


class RopeParams(C.Structure):
    _fields_ = [("n_rot", C.c_uint32), ("freq_base", C.c_float), ("freq_scale", C.c_float),
                ("hadamard_nrot", C.c_int32)]


class History(C.Structure):
    _fields_ = [("k_raw", C.c_void_p), ("v", C.c_void_p), ("n_tokens", C.c_uint32)]


class StageinLane(C.Structure):
    _fields_ = [("h", C.POINTER(History)), ("w", C.POINTER(Window)), ("sel", C.POINTER(Selection))]


class Lane(C.Structure):
    _fields_ = [("w", C.POINTER(Window)), ("q", C.c_void_p), ("q_pos", C.c_void_p),
                ("out", C.c_void_p), ("n_tokens", C.c_uint32)]


class SlotPool(C.Structure):
    _fields_ = [("n_slots", C.c_uint32), ("n_free", C.c_uint32), ("free_slots", C.c_void_p)]


class RowRange(C.Structure):
    _fields_ = [("begin", C.c_int32), ("end", C.c_int32)]


class SnapshotInfo(C.Structure):
    _fields_ = [("n_layer", C.c_uint32), ("n_embd_k", C.c_uint32), ("n_embd_v", C.c_uint32),
                ("block_tokens", C.c_uint32), ("k_row_bytes", C.c_uint64), ("k_gpu_row_bytes", C.c_uint64),
                ("v_gpu_row_bytes", C.c_uint64), ("n_blocks", C.c_uint64)]


class SnapshotLayer(C.Structure):
    _fields_ = [("k_rows", C.c_void_p), ("k_rows_bytes", C.c_size_t), ("v_rows", C.c_void_p),
                ("v_rows_bytes", C.c_size_t), ("k_sum", C.c_void_p), ("mean_tokens", C.c_void_p),
                ("n_tokens", C.c_void_p), ("max_blocks", C.c_uint64), ("expect", C.POINTER(SnapshotInfo))]


_P = C.c_void_p
_u32, _i32, _i64, _sz, _f = C.c_uint32, C.c_int32, C.c_int64, C.c_size_t, C.c_float
_PW = C.POINTER(Window)

# name -> (restype, argtypes)
SIGNATURES = {
    "kvm_abi_version": (C.c_int, []),
    "kvm_state_create": (_P, [C.c_int]),
    "kvm_state_free": (None, [_P]),
    "kvm_state_set_stream": (C.c_int, [_P, _P]),
    "kvm_state_stream": (_P, [_P]),
    "kvm_state_sync": (C.c_int, [_P]),
    "kvm_state_status": (C.c_int, [_P, C.POINTER(_u32)]),
    "kvm_state_set_wait_polls": (C.c_int, [_P, _u32]),
    "kvm_state_last_error": (C.c_char_p, [_P]),
    "kvm_host_alloc": (_P, [_sz]),
    "kvm_host_free": (None, [_P]),
    "kvm_window_k_bytes": (_sz, [_PW]),
    "kvm_window_v_bytes": (_sz, [_PW]),
    "kvm_window_shadow_bytes": (_sz, [_PW]),
    "kvm_window_check": (C.c_int, [_PW]),
    "kvm_window_reset": (C.c_int, [_P, _PW]),
    "kvm_window_import_rows": (C.c_int, [_P, _PW, _u32, _u32, _P, _P, _P]),
    "kvm_window_export_rows": (C.c_int, [_P, _PW, _u32, _u32, _P, _P]),
    "kvm_slot_pool_reset": (C.c_int, [C.POINTER(SlotPool)]),
    "kvm_slot_alloc": (_i32, [C.POINTER(SlotPool)]),
    "kvm_slot_free": (C.c_int, [C.POINTER(SlotPool), _i32]),
    "kvm_slot_copy_to_host": (C.c_int, [_P, C.POINTER(_PW), _u32, _i32, _P, C.c_uint64]),
    "kvm_slot_copy_from_host": (C.c_int, [_P, C.POINTER(_PW), _u32, _i32, _P, C.c_uint64]),
    "kvm_harvest_block": (C.c_int, [_P, _PW, _u32, _u32, C.POINTER(View), _u32, _P, _P, C.POINTER(MeanKIndex),
                                    _u32, _u32]),
    "kvm_quantize_rows": (C.c_int, [_P, C.c_int, _P, _P, _i64, _i64]),
    "kvm_dequantize_rows": (C.c_int, [_P, C.c_int, _P, _P, _i64, _i64]),
    "kvm_query_reset": (C.c_int, [_P, C.POINTER(QueryAcc)]),
    "kvm_query_refresh": (C.c_int, [_P, C.POINTER(QueryAcc)]),
    "kvm_meank_refresh": (C.c_int, [_P, C.POINTER(MeanKIndex)]),
    "kvm_query_add": (C.c_int, [_P, C.POINTER(QueryAcc), _u32, _P, _u32]),
    "kvm_meank_k_sum_floats": (_sz, [C.POINTER(MeanKIndex)]),
    "kvm_meank_add": (C.c_int, [_P, C.POINTER(MeanKIndex), _u32, _u32, _u32, _P]),
    "kvm_query_add_view": (C.c_int, [_P, C.POINTER(QueryAcc), _u32, C.POINTER(View), _P]),
    "kvm_meank_add_view": (C.c_int, [_P, C.POINTER(MeanKIndex), _u32, _u32, C.POINTER(View)]),
    "kvm_meank_acc_zero": (C.c_int, [_P, C.POINTER(MeanKIndex), _u32]),
    "kvm_meank_acc_add": (C.c_int, [_P, C.POINTER(MeanKIndex), _u32, C.POINTER(View), _u32, _u32]),
    "kvm_meank_acc_flush": (C.c_int, [_P, C.POINTER(MeanKIndex), _u32, _u32, _u32]),
    "kvm_score_topk": (C.c_int, [_P, C.POINTER(MeanKIndex), C.POINTER(QueryAcc),
                                 C.POINTER(SelectParams), _PW, C.POINTER(Selection)]),
    "kvm_score_topk_lanes": (C.c_int, [_P, C.POINTER(RetrievalLane), _u32]),
    "kvm_score_topk_stagein": (C.c_int, [_P, C.POINTER(MeanKIndex), C.POINTER(QueryAcc), C.POINTER(SelectParams),
                                         _PW, C.POINTER(Selection), C.POINTER(History), C.POINTER(RopeParams)]),
    "kvm_score_topk_stagein_lanes": (C.c_int, [_P, C.POINTER(RetrievalLane), C.POINTER(C.POINTER(History)), _u32,
                                               C.POINTER(RopeParams)]),
    "kvm_select_topk": (C.c_int, [_P, _P, C.POINTER(SelectParams), _PW, C.POINTER(Selection)]),
    "kvm_retrieval_mandatory": (C.c_int, [_P, _P, _u32, C.POINTER(RowRange), _u32, _i32, _i32, _i32, _P, _u32,
                                          C.POINTER(_u32)]),
    "kvm_stagein_selection": (C.c_int, [_P, C.POINTER(History), _PW, C.POINTER(Selection),
                                        C.POINTER(RopeParams)]),
    "kvm_stagein_selection_lanes": (C.c_int, [_P, C.POINTER(StageinLane), _u32, C.POINTER(RopeParams)]),
    "kvm_stagein_enqueue_k": (C.c_int, [_P, C.c_int, _P, _sz, _PW, _u32, _i64, _i64, C.c_int,
                                        C.c_int, C.c_int, C.c_int, _i32, _P, C.c_int]),
    "kvm_stagein_enqueue_v": (C.c_int, [_P, _P, _sz, _PW, _u32, _i64]),
    "kvm_stagein_flush": (C.c_int, [_P]),
    "kvm_fa_decode": (C.c_int, [_P, _PW, _P, C.c_int, _P, _u32, _u32, _f, _P]),
    "kvm_fa_decode_lanes": (C.c_int, [_P, C.POINTER(Lane), _u32, C.c_int, _u32, _f]),
    "kvm_fa_decode_noalloc": (C.c_int, [_P, _PW, _P, C.c_int, _P, _u32, _u32, _f, _P]),
    "kvm_stagein_fa_decode": (C.c_int, [_P, C.POINTER(History), C.POINTER(Selection), C.POINTER(RopeParams), _PW, _P,
                                        C.c_int, _P, _u32, _u32, _f, _P]),
    "kvm_stagein_fa_decode_lanes": (C.c_int, [_P, C.POINTER(StageinLane), C.POINTER(Lane), _u32,
                                              C.POINTER(RopeParams), C.c_int, _u32, _f]),
    "kvm_select_topk_stagein_fa_decode": (C.c_int, [_P, _P, C.POINTER(SelectParams), _PW, C.POINTER(Selection),
                                                    C.POINTER(History), C.POINTER(RopeParams), _P, C.c_int, _P,
                                                    _u32, _u32, _f, _P]),
    "kvm_score_topk_stagein_fa_decode": (C.c_int, [_P, C.POINTER(MeanKIndex), C.POINTER(QueryAcc),
                                                   C.POINTER(SelectParams), _PW, C.POINTER(Selection),
                                                   C.POINTER(History), C.POINTER(RopeParams), _P, C.c_int, _P,
                                                   _u32, _u32, _f, _P]),
    "kvm_score_topk_stagein_fa_decode_lanes": (C.c_int, [_P, C.POINTER(RetrievalLane), C.POINTER(C.POINTER(History)),
                                                         C.POINTER(Lane), _u32, C.POINTER(RopeParams), C.c_int,
                                                         _u32, _f]),
    "kvm_fa_prefill": (C.c_int, [_P, _PW, _P, C.c_int, _P, _u32, _u32, _f, _P]),
    "kvm_d2d_batched": (C.c_int, [_P, C.POINTER(_P), C.POINTER(_P), C.POINTER(_sz), C.c_int]),
    "kvm_snapshot_info_read": (C.c_int, [_P, _P, _sz, C.POINTER(SnapshotInfo)]),
    "kvm_snapshot_read_layer": (C.c_int, [_P, _P, _sz, _u32, C.POINTER(SnapshotLayer)]),
}

_lib = None


def load(path=None):
    """Load libkvm_hotpath.so (raises if it is missing) and bind every entry point.

    KVM_HOTPATH_LIB in the environment names another build of the library to
    load in place of the in-tree one.
    """
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = path or os.environ.get("KVM_HOTPATH_LIB") or LIB_PATH
    if not os.path.exists(p):
        raise RuntimeError(f"libkvm_hotpath.so is not built ({p}); run __graft_entry__.build()")
    lib = C.CDLL(p)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib
