"""ctypes wrapper of the C oracle (libkvm_oracle.so) and of the reference's own
kvmem host library built into oracle/_ref/ (libkvmem_ref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, to check results against or as the timed CPU
baseline.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "libkvm_oracle.so")
REF_SO = os.path.join(HERE, "_ref", "libkvmem_ref.so")

T_F32, T_F16, T_Q4_0, T_Q8_0 = 0, 1, 2, 8

_o = None
_r = None


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def lib():
    global _o
    if _o is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"oracle not built: {ORACLE_SO} (make -C oracle)")
        _o = C.CDLL(ORACLE_SO)
        P, u32, i32, i64, f, d = C.c_void_p, C.c_uint32, C.c_int32, C.c_int64, C.c_float, C.c_double
        sig = {
            "oracle_f32_to_f16": (C.c_uint16, [f]),
            "oracle_f16_to_f32": (f, [C.c_uint16]),
            "oracle_quant_q8_0": (None, [P, P, i64]),
            "oracle_dequant_q8_0": (None, [P, P, i64]),
            "oracle_quant_q4_0": (None, [P, P, i64]),
            "oracle_dequant_q4_0": (None, [P, P, i64]),
            "oracle_row_bytes": (i64, [C.c_int, i64]),
            "oracle_rope_theta": (None, [f, f, C.c_int, P]),
            "oracle_rope_cs": (None, [P, C.c_int, i32, P, P]),
            "oracle_rope_neox": (None, [P, i64, C.c_int, C.c_int, C.c_int, i32, P]),
            "oracle_fwht": (None, [P, i64, C.c_int]),
            "oracle_hadamard_nrot_k": (C.c_int, [C.c_int]),
            "oracle_attn_rot_on": (C.c_int, [C.c_int, C.c_int]),
            "oracle_stagein_k": (None, [P, P, i64, C.c_int, C.c_int, C.c_int, C.c_int, i32, P]),
            "oracle_stagein_k_type": (None, [C.c_int, P, P, i64, C.c_int, C.c_int, C.c_int, C.c_int, i32, P]),
            "oracle_meank_add": (None, [P, P, P, u32, u32, C.c_int]),
            "oracle_meank_normalize": (None, [P, u32, P, C.c_int]),
            "oracle_score_retrieval": (None, [C.c_int] * 5 + [P, P, P, P, P, P, C.c_int]),
            "oracle_pick_topk": (u32, [u32, P, u32, u32, u32, P, u32, P]),
            "oracle_window_layout": (u32, [P, u32, P, u32, u32, P, P]),
            "oracle_fa_ggml": (C.c_int, [C.c_int, C.c_int, P, P, P, P, P] + [C.c_int] * 5 + [f, P, C.c_int]),
            "oracle_fa_f64": (C.c_int, [C.c_int, C.c_int, P, P, P, P, P] + [C.c_int] * 5 + [d, P, C.c_int]),
            "oracle_quant_q8_0_rows": (None, [P, P, i64, i64]),
            "oracle_retrieval_mandatory": (u32, [P, u32, P, u32, i32, i32, i32, i32, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(_o, name)
            fn.restype, fn.argtypes = res, args
    return _o


def ref_available():
    return os.path.exists(REF_SO)


def ref():
    global _r
    if _r is None:
        if not ref_available():
            raise RuntimeError(f"reference library not built: {REF_SO} (make -C oracle ref)")
        _r = C.CDLL(REF_SO)
        P, u32, i32, f = C.c_void_p, C.c_uint32, C.c_int32, C.c_float
        _r.ref_pick_topk.restype = C.c_int
        _r.ref_pick_topk.argtypes = [u32, u32, u32, u32, u32, P, u32, P, u32, P, u32]
        _r.ref_set_selection_seq.restype = C.c_int
        _r.ref_set_selection_seq.argtypes = [u32, u32, P, P, u32, P, u32, P, P, P, P, P, u32, P]
        _r.ref_mean_k.restype = C.c_int
        _r.ref_mean_k.argtypes = [u32, u32, u32, u32, P, P]
        _r.ref_raw_snapshot.restype = C.c_longlong
        _r.ref_raw_snapshot.argtypes = [u32, u32, u32, u32, C.c_uint64, C.c_uint64, u32, u32, P, P, P, P,
                                        C.c_uint64]
        _r.ref_block_layout.restype = C.c_int
        _r.ref_block_layout.argtypes = [P, u32, u32, P, P, u32, P, u32, P]
        _r.ref_rope_neox.restype = None
        _r.ref_rope_neox.argtypes = [u32, u32, u32, f, f, P, u32, i32, P]
    return _r


# ---- codecs -------------------------------------------------------------------
def f32_to_f16(x):
    o = lib()
    x = np.asarray(x, dtype=np.float32).reshape(-1)
    return np.array([o.oracle_f32_to_f16(float(v)) for v in x], dtype=np.uint16)


def quant(ty, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.size
    out = np.empty(n // 32 * (34 if ty == T_Q8_0 else 18), dtype=np.uint8)
    (lib().oracle_quant_q8_0 if ty == T_Q8_0 else lib().oracle_quant_q4_0)(_p(x), _p(out), n)
    return out


def dequant(ty, b, n):
    b = np.ascontiguousarray(b, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    (lib().oracle_dequant_q8_0 if ty == T_Q8_0 else lib().oracle_dequant_q4_0)(_p(b), _p(out), n)
    return out


def rope_theta(freq_base, freq_scale, n_rot):
    t = np.empty(n_rot // 2, dtype=np.float32)
    lib().oracle_rope_theta(freq_base, freq_scale, n_rot, _p(t))
    return t


def rope_neox(x, n_head, head_dim, n_rot, pos0, theta):
    x = np.ascontiguousarray(x, dtype=np.float32).copy()
    nt = x.size // (n_head * head_dim)
    lib().oracle_rope_neox(_p(x), nt, n_head, head_dim, n_rot, pos0, _p(np.ascontiguousarray(theta, np.float32)))
    return x


def fwht(x, n):
    x = np.ascontiguousarray(x, dtype=np.float32).copy()
    lib().oracle_fwht(_p(x), x.size // n, n)
    return x


def stagein_k(packed, nt, n_head, head_dim, n_rot, nrot, pos0, theta, k_type=None):
    """Stage-in of raw K rows (q8_0, or q4_0 with k_type=T_Q4_0) at window position pos0."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.empty_like(packed)
    th = _p(np.ascontiguousarray(theta, np.float32))
    if k_type is None or k_type == T_Q8_0:
        lib().oracle_stagein_k(_p(packed), _p(out), nt, n_head, head_dim, n_rot, nrot, pos0, th)
    else:
        lib().oracle_stagein_k_type(k_type, _p(packed), _p(out), nt, n_head, head_dim, n_rot, nrot, pos0, th)
    return out


# ---- mean-K / scoring / selection --------------------------------------------
def meank_sums(k, block_tokens, chunk=None):
    """k: fp32 [n_tokens][n_embd] -> (k_sum [n_blocks][n_embd], mean_tokens [n_blocks]),
    written in chunks of `chunk` tokens like RawKvStore::write_layer_mean_k."""
    k = np.ascontiguousarray(k, dtype=np.float32)
    n, e = k.shape
    nb = (n + block_tokens - 1) // block_tokens
    sums = np.zeros((nb, e), dtype=np.float32)
    mt = np.zeros(nb, dtype=np.uint32)
    chunk = chunk or n
    pos = 0
    while pos < n:
        take_all = min(chunk, n - pos)
        done = 0
        while done < take_all:
            p = pos + done
            b, off = divmod(p, block_tokens)
            take = min(take_all - done, block_tokens - off)
            row = np.ascontiguousarray(k[p:p + take])
            s = sums[b:b + 1].reshape(-1)
            m = mt[b:b + 1]
            lib().oracle_meank_add(s.ctypes.data_as(C.c_void_p), m.ctypes.data_as(C.c_void_p), _p(row), off, take, e)
            done += take
        pos += take_all
    return sums, mt


def score_retrieval(q_sum, q_count, k_sum, mean_tokens, n_head, n_head_kv, head_dim, present=None, n_threads=1):
    """q_sum [L][n_head*D], k_sum [L][n_blocks][n_head_kv*D], mean_tokens [L][n_blocks]."""
    q_sum = np.ascontiguousarray(q_sum, np.float32)
    q_count = np.ascontiguousarray(q_count, np.uint32)
    k_sum = np.ascontiguousarray(k_sum, np.float32)
    mean_tokens = np.ascontiguousarray(mean_tokens, np.uint32)
    n_layer, n_blocks = mean_tokens.shape
    scores = np.zeros(n_blocks, dtype=np.float64)
    pres = None if present is None else np.ascontiguousarray(present, np.uint8)
    lib().oracle_score_retrieval(n_blocks, n_layer, n_head, n_head_kv, head_dim, _p(q_sum), _p(q_count),
                                 _p(k_sum), _p(mean_tokens), _p(pres), _p(scores), n_threads)
    return scores


def pick_topk(scores, budget_blocks, sink_blocks=1, recent_blocks=0, mandatory=()):
    scores = np.ascontiguousarray(scores, np.float64)
    n = scores.size
    out = np.zeros(max(n, 1), dtype=np.uint32)
    mand = np.ascontiguousarray(np.asarray(mandatory, dtype=np.uint32))
    m = lib().oracle_pick_topk(n, _p(scores), budget_blocks, sink_blocks, recent_blocks,
                               _p(mand) if mand.size else None, mand.size, _p(out))
    return out[:m].astype(np.int64)


def window_layout(sel, n_tokens, block_tokens, n_slots):
    sel = np.ascontiguousarray(sel, np.uint32)
    n_tokens = np.ascontiguousarray(n_tokens, np.uint32)
    to_base = np.zeros(max(sel.size, 1), dtype=np.int32)
    cell_pos = np.zeros(n_slots * block_tokens, dtype=np.int32)
    total = lib().oracle_window_layout(_p(sel), sel.size, _p(n_tokens), block_tokens, n_slots, _p(to_base),
                                       _p(cell_pos))
    return to_base[:sel.size].astype(np.int64), cell_pos, int(total)


# ---- attention ----------------------------------------------------------------
def fa_ggml(k_type, v_type, q, k_rows, v_rows, cell_pos, q_pos, n_head, n_head_kv, head_dim, scale, n_threads=8):
    q = np.ascontiguousarray(q, np.float32)
    n_tokens = q.shape[0]
    n_cells = k_rows.shape[0]
    out = np.zeros((n_tokens, n_head, head_dim), dtype=np.float32)
    cp = None if cell_pos is None else np.ascontiguousarray(cell_pos, np.int32)
    qp = np.ascontiguousarray(q_pos, np.int32)
    rc = lib().oracle_fa_ggml(k_type, v_type, _p(q), _p(np.ascontiguousarray(k_rows)),
                              _p(np.ascontiguousarray(v_rows)), _p(cp), _p(qp), n_tokens, n_head, n_head_kv,
                              head_dim, n_cells, scale, _p(out), n_threads)
    assert rc == 0
    return out


def fa_f64(k_type, v_type, q, k_rows, v_rows, cell_pos, q_pos, n_head, n_head_kv, head_dim, scale, n_threads=8):
    q = np.ascontiguousarray(q, np.float32)
    n_tokens = q.shape[0]
    n_cells = k_rows.shape[0]
    out = np.zeros((n_tokens, n_head, head_dim), dtype=np.float64)
    cp = None if cell_pos is None else np.ascontiguousarray(cell_pos, np.int32)
    qp = np.ascontiguousarray(q_pos, np.int32)
    rc = lib().oracle_fa_f64(k_type, v_type, _p(q), _p(np.ascontiguousarray(k_rows)),
                             _p(np.ascontiguousarray(v_rows)), _p(cp), _p(qp), n_tokens, n_head, n_head_kv,
                             head_dim, n_cells, scale, _p(out), n_threads)
    assert rc == 0
    return out


def retrieval_mandatory(n_tokens, ranges=None, query_begin=-1, query_end=0, force_pos=-1):
    """Mandatory block ids (llama-memory-kvmem.cpp:4306-4325) of a store whose
    block b holds n_tokens[b] consecutive positions; ranges None = the turn set
    no explicit spans (the query span applies), [] = explicit and empty."""
    nt = np.ascontiguousarray(n_tokens, np.uint32)
    rg = np.ascontiguousarray(np.asarray([] if ranges is None else ranges, dtype=np.int32).reshape(-1, 2))
    out = np.zeros(nt.size + 1, np.uint32)
    n = lib().oracle_retrieval_mandatory(_p(nt), nt.size, _p(rg) if rg.size else None, rg.shape[0],
                                         0 if ranges is None else 1, query_begin, query_end, force_pos, _p(out))
    return out[:n].astype(np.int64)


# ---- reference library (oracle/_ref) -----------------------------------------
def ref_pick_topk(total_tokens, block_tokens, budget_tokens, sink_blocks, recent_blocks, scores, mandatory=()):
    scores = np.ascontiguousarray(scores, np.float64)
    mand = np.ascontiguousarray(np.asarray(mandatory, dtype=np.uint32))
    out = np.zeros(max(scores.size, 1), dtype=np.uint32)
    m = ref().ref_pick_topk(total_tokens, block_tokens, budget_tokens, sink_blocks, recent_blocks, _p(scores),
                            scores.size, _p(mand) if mand.size else None, mand.size, _p(out), out.size)
    assert m >= 0
    return out[:m].astype(np.int64)


REMAP_DT = np.dtype([("block_id", "<u4"), ("n_tokens", "<u4"), ("from_base", "<i4"), ("to_base", "<i4"),
                     ("skip", "<i4"), ("raw_refresh", "<i4"), ("working_k_resident", "<i4"), ("pad", "<i4")])


def ref_set_selection_seq(total_tokens, block_tokens, selections):
    flat = np.ascontiguousarray(np.concatenate([np.asarray(s, np.uint32) for s in selections]), np.uint32)
    lens = np.ascontiguousarray([len(s) for s in selections], np.uint32)
    cap = max(int((total_tokens + block_tokens - 1) // block_tokens), 1)
    remaps = np.zeros(cap, dtype=REMAP_DT)
    n_remaps = np.zeros(1, np.uint32)
    sin, sout = np.zeros(cap, np.uint32), np.zeros(cap, np.uint32)
    nin, nout, total = np.zeros(1, np.uint32), np.zeros(1, np.uint32), np.zeros(1, np.uint32)
    rc = ref().ref_set_selection_seq(total_tokens, block_tokens, _p(flat), _p(lens), len(selections),
                                     _p(remaps), cap, _p(n_remaps), _p(sin), _p(nin), _p(sout), _p(nout), cap,
                                     _p(total))
    assert rc == 0
    return {"remaps": remaps[:n_remaps[0]], "stage_in": sin[:nin[0]].astype(np.int64),
            "stage_out": sout[:nout[0]].astype(np.int64), "total": int(total[0])}


def ref_raw_snapshot(k_rows, k_f32, v_rows, n_embd_k, n_embd_v, block_tokens, chunk):
    """The reference RawKvStore filled with [n_layer][n_tokens] K rows (+ their fp32
    values for the mean) and packed V rows, then snapshot_write: the snapshot bytes."""
    k_rows, v_rows = np.ascontiguousarray(k_rows, np.uint8), np.ascontiguousarray(v_rows, np.uint8)
    k_f32 = np.ascontiguousarray(k_f32, np.float32)
    n_layer, n_tokens, krb = k_rows.shape
    vrb = v_rows.shape[2]
    args = (n_layer, n_embd_k, n_embd_v, block_tokens, krb, vrb, n_tokens, chunk, _p(k_rows), _p(k_f32), _p(v_rows))
    n = ref().ref_raw_snapshot(*args, None, 0)
    assert n > 0
    out = np.zeros(n, np.uint8)
    assert ref().ref_raw_snapshot(*args, _p(out), n) == n
    return out.tobytes()


def ref_block_layout(appends, block_tokens, positions):
    """The reference store's blocks after register_append of each chunk in
    `appends`: (orig_pos_start, n_tokens) per block, and block_id_containing of
    each position."""
    ap = np.ascontiguousarray(appends, np.uint32)
    cap = int(ap.sum()) // block_tokens + len(ap) + 1
    start, nt = np.zeros(cap, np.uint32), np.zeros(cap, np.uint32)
    pos = np.ascontiguousarray(positions, np.int32)
    cont = np.zeros(max(pos.size, 1), np.int32)
    n = ref().ref_block_layout(_p(ap), ap.size, block_tokens, _p(start), _p(nt), cap, _p(pos), pos.size, _p(cont))
    assert n >= 0
    return start[:n].astype(np.int64), nt[:n].astype(np.int64), cont[:pos.size].astype(np.int64)


def ref_mean_k(k, block_tokens, chunk):
    k = np.ascontiguousarray(k, np.float32)
    n, e = k.shape
    nb = (n + block_tokens - 1) // block_tokens
    out = np.zeros((nb, e), dtype=np.float32)
    r = ref().ref_mean_k(e, block_tokens, n, chunk, _p(k), _p(out))
    assert r == nb
    return out


def ref_rope_neox(k, n_head, head_dim, n_rot, freq_base, freq_scale, pos0):
    k = np.ascontiguousarray(k, np.float32)
    out = np.empty_like(k)
    nt = k.size // (n_head * head_dim)
    ref().ref_rope_neox(n_rot, head_dim, n_head, freq_base, freq_scale, _p(k), nt, pos0, _p(out))
    return out
