"""Host-side mirror of the KVMem hot-path interface over libkvm_hotpath.so.

PyTorch is used only for device memory and the stream; every computation is a
kernel of libkvm_hotpath.so.  Names follow the reference's domain: a window is
the bounded GPU slot pool of one attention layer (llama-memory-kvmem.cpp:611-779),
the mean-K index is RawKvStore's per-block K sums (raw_kv_store.cpp:215-234),
the query accumulator is the adapter's q_sum_/q_count_ (llama-memory-kvmem.cpp:3300-3315).
"""
import ctypes as C

import numpy as np
import torch

from . import _lib as L


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


class State:
    """One execution domain (kvmem_gpu_state, llama-kvmem-stagein.h:12-15)."""

    def __init__(self, device=0, stream=None):
        self.lib = L.load()
        self.device = device
        self.h = self.lib.kvm_state_create(device)
        if not self.h:
            raise L.KvmError(L.KVM_EHIP, f"kvm_state_create({device}) failed")
        s = stream if stream is not None else torch.cuda.current_stream(device).cuda_stream
        self.check(self.lib.kvm_state_set_stream(self.h, C.c_void_p(s)))

    def check(self, rc):
        if rc != L.KVM_OK:
            raise L.KvmError(rc, self.lib.kvm_state_last_error(self.h).decode())
        return rc

    def sync(self):
        """Waits for the state's stream; raises KvmError(KVM_ETIMEOUT) when an
        in-launch wait gave up since the last sync."""
        self.check(self.lib.kvm_state_sync(self.h))

    def status(self):
        """Waits for the stream and returns (and clears) the KVM_WAIT_* bits of
        the in-launch waits that gave up since the last sync / status."""
        v = C.c_uint32(0)
        self.check(self.lib.kvm_state_status(self.h, C.byref(v)))
        return v.value

    def set_wait_polls(self, polls):
        """Polls of an in-launch wait before it gives up (0: every wait gives up at once)."""
        self.check(self.lib.kvm_state_set_wait_polls(self.h, int(polls)))

    def capture(self, fns):
        """Capture the library calls made by fns() (one HIP graph, replayed with
        .replay() on the current stream).  The state's stream is switched to
        the capture stream for the capture and restored after; the calls must
        need no workspace growth (run them once eagerly first)."""
        cap = torch.cuda.Stream(self.device)
        old = self.lib.kvm_state_stream(self.h)
        g = torch.cuda.CUDAGraph()
        torch.cuda.synchronize(self.device)
        self.check(self.lib.kvm_state_set_stream(self.h, C.c_void_p(cap.cuda_stream)))
        try:
            with torch.cuda.graph(g, stream=cap):
                fns()
        finally:
            self.check(self.lib.kvm_state_set_stream(self.h, C.c_void_p(old)))
        return g

    def close(self):
        if self.h:
            self.lib.kvm_state_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


_VIEW_TYPES = {torch.float32: L.T_F32, torch.float16: L.T_F16, torch.bfloat16: L.T_BF16}


def view(t):
    """The kvm_view of a 3-d device tensor [tokens][heads][dims] with its own strides."""
    assert t.dim() == 3, "a view is [tokens][heads][dims]"
    es = t.element_size()
    return L.View(t.data_ptr(), _VIEW_TYPES[t.dtype], t.shape[2], t.shape[1], t.shape[0],
                  t.stride(2) * es, t.stride(1) * es, t.stride(0) * es)


class HostBuffer:
    """Pinned, device-mapped host memory (kvm_host_alloc) viewed as numpy."""

    def __init__(self, nbytes):
        self.lib = L.load()
        self.nbytes = int(nbytes)
        self.ptr = self.lib.kvm_host_alloc(self.nbytes)
        if not self.ptr:
            raise L.KvmError(L.KVM_ENOMEM, f"kvm_host_alloc({nbytes}) failed")
        self.u8 = np.ctypeslib.as_array((C.c_uint8 * self.nbytes).from_address(self.ptr))

    def close(self):
        if self.ptr:
            self.lib.kvm_host_free(C.c_void_p(self.ptr))
            self.ptr = None
            self.u8 = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def row_bytes(ty, n):
    return {L.T_F32: 4 * n, L.T_F16: 2 * n, L.T_Q8_0: n // 32 * 34, L.T_Q4_0: n // 32 * 18}[ty]


class KVWindow:
    """Bounded GPU window of one attention layer in the library's tiled layout."""

    def __init__(self, st, n_cells, n_head_kv, head_dim, block_tokens=128,
                 k_type=L.T_Q8_0, v_type=L.T_Q4_0, shadow=False, pending=False):
        """shadow: keep an HBM copy of the staged blocks' raw K rows, so that a
        later plan re-bases resident blocks from HBM instead of the host.
        pending: count each slot's imported rows not yet harvested, so that a
        plan that would overwrite them is refused."""
        self.st = st
        dev = torch.device("cuda", st.device)
        self.c = L.Window(n_cells, n_head_kv, head_dim, block_tokens, k_type, v_type)
        kb = st.lib.kvm_window_k_bytes(C.byref(self.c))
        vb = st.lib.kvm_window_v_bytes(C.byref(self.c))
        if kb == 0 or vb == 0:
            raise L.KvmError(L.KVM_EINVAL, "bad window geometry")
        self.k = torch.zeros(kb, dtype=torch.uint8, device=dev)
        self.v = torch.zeros(vb, dtype=torch.uint8, device=dev)
        self.cell_pos = torch.full((n_cells,), -1, dtype=torch.int32, device=dev)
        n_slots = n_cells // block_tokens
        self.slot_block = torch.full((n_slots,), -1, dtype=torch.int32, device=dev)
        self.slot_base = torch.full((n_slots,), -1, dtype=torch.int32, device=dev)
        self.c.k, self.c.v = self.k.data_ptr(), self.v.data_ptr()
        self.c.cell_pos = self.cell_pos.data_ptr()
        self.c.slot_block = self.slot_block.data_ptr()
        self.c.slot_base = self.slot_base.data_ptr()
        self.k_shadow = self.shadow_rows = None
        if shadow:
            self.k_shadow = torch.zeros(st.lib.kvm_window_shadow_bytes(C.byref(self.c)), dtype=torch.uint8, device=dev)
            self.shadow_rows = torch.zeros((n_slots,), dtype=torch.int32, device=dev)
            self.c.k_shadow = self.k_shadow.data_ptr()
            self.c.shadow_rows = self.shadow_rows.data_ptr()
        self.pending_rows = None
        if pending:
            self.pending_rows = torch.zeros((n_slots,), dtype=torch.int32, device=dev)
            self.c.pending_rows = self.pending_rows.data_ptr()
        st.check(st.lib.kvm_window_check(C.byref(self.c)))
        self.n_cells, self.n_head_kv, self.head_dim = n_cells, n_head_kv, head_dim
        self.block_tokens, self.k_type, self.v_type = block_tokens, k_type, v_type

    @property
    def bytes(self):
        return self.k.numel() + self.v.numel()

    def k_row_bytes(self):
        return self.n_head_kv * row_bytes(self.k_type, self.head_dim)

    def v_row_bytes(self):
        return self.n_head_kv * row_bytes(self.v_type, self.head_dim)

    def reset(self):
        self.st.check(self.st.lib.kvm_window_reset(self.st.h, C.byref(self.c)))

    def import_rows(self, cell0, k_rows, v_rows, pos=None):
        """k_rows / v_rows: uint8 device tensors of ggml rows ([n][row bytes])."""
        n = (k_rows if k_rows is not None else v_rows).shape[0]
        self.st.check(self.st.lib.kvm_window_import_rows(
            self.st.h, C.byref(self.c), cell0, n, _ptr(k_rows), _ptr(v_rows), _ptr(pos)))

    def export_rows(self, cell0, n):
        dev = self.k.device
        kr = torch.empty((n, self.k_row_bytes()), dtype=torch.uint8, device=dev)
        vr = torch.empty((n, self.v_row_bytes()), dtype=torch.uint8, device=dev)
        self.st.check(self.st.lib.kvm_window_export_rows(
            self.st.h, C.byref(self.c), cell0, n, _ptr(kr), _ptr(vr)))
        return kr, vr


class MeanKIndex:
    """Device mean-K index: ordered fp32 K sums + token counts per (layer, block).

    k_sum is stored in 8-block tiles, [n_layer][tiles][n_head_kv*head_dim][8];
    block_sums() / set_block_sums() convert to and from [n_layer][block][e].
    """

    TILE = 8

    def __init__(self, st, n_layer, n_blocks, n_head_kv, head_dim, block_tokens=128, norms=False):
        """norms: the index also carries the blocks' score term nk (k_norm),
        which add / acc_flush keep current; after writing k_sum or mean_tokens
        directly, call refresh()."""
        dev = torch.device("cuda", st.device)
        self.st = st
        self.n_blocks = n_blocks
        n_tiles = (n_blocks + self.TILE - 1) // self.TILE
        self.k_sum = torch.zeros((n_layer, n_tiles, n_head_kv * head_dim, self.TILE), dtype=torch.float32, device=dev)
        self.mean_tokens = torch.zeros((n_layer, n_blocks), dtype=torch.int32, device=dev)
        self.present = torch.zeros((n_blocks,), dtype=torch.uint8, device=dev)
        self.acc = torch.zeros((n_layer, n_head_kv * head_dim), dtype=torch.float32, device=dev)
        self.k_norm = torch.zeros((n_layer, n_head_kv, n_blocks), dtype=torch.float32, device=dev) if norms else None
        self.c = L.MeanKIndex(n_layer, n_blocks, n_head_kv, head_dim, block_tokens,
                              self.k_sum.data_ptr(), self.mean_tokens.data_ptr(), self.present.data_ptr(),
                              self.acc.data_ptr(), self.k_norm.data_ptr() if norms else None)
        assert self.k_sum.numel() == st.lib.kvm_meank_k_sum_floats(C.byref(self.c))

    def refresh(self):
        self.st.check(self.st.lib.kvm_meank_refresh(self.st.h, C.byref(self.c)))

    def block_sums(self):
        """K sums as [n_layer][n_blocks][n_head_kv*head_dim] (a copy)."""
        Lr, T, E, W = self.k_sum.shape
        return self.k_sum.permute(0, 1, 3, 2).reshape(Lr, T * W, E)[:, :self.n_blocks].contiguous()

    def set_block_sums(self, sums, first=0):
        """Store sums [n_layer][n][e] (device tensor) for blocks first .. first+n-1."""
        Lr, T, E, W = self.k_sum.shape
        n = sums.shape[1]
        view = self.k_sum.permute(0, 1, 3, 2).reshape(Lr, T * W, E).clone()   # (a copy even where reshape can view)
        view[:, first:first + n] = sums
        self.k_sum.copy_(view.reshape(Lr, T, W, E).permute(0, 1, 3, 2))

    def add(self, il, pos0, k_rows):
        """k_rows: device fp32 [n][n_head_kv*head_dim] of pre-RoPE K at positions pos0.."""
        k_rows = k_rows.contiguous()
        self.st.check(self.st.lib.kvm_meank_add(self.st.h, C.byref(self.c), il, pos0,
                                                k_rows.shape[0], _ptr(k_rows)))

    def add_view(self, il, pos0, k):
        """k: device tensor [tokens][heads][dims] (any strides) of fp32 / fp16 / bf16."""
        self.st.check(self.st.lib.kvm_meank_add_view(self.st.h, C.byref(self.c), il, pos0, C.byref(view(k))))

    def acc_zero(self, il):
        self.st.check(self.st.lib.kvm_meank_acc_zero(self.st.h, C.byref(self.c), il))

    def acc_add(self, il, k, tok0, n_keep):
        self.st.check(self.st.lib.kvm_meank_acc_add(self.st.h, C.byref(self.c), il, C.byref(view(k)), tok0, n_keep))

    def acc_flush(self, il, pos0, n):
        self.st.check(self.st.lib.kvm_meank_acc_flush(self.st.h, C.byref(self.c), il, pos0, n))


class QueryAcc:
    """q_sum_ / q_count_ on the device.  With n_head_kv, the accumulator also
    carries the scorer's query terms (q_vec = the group sums times 1 / (q_count
    g), q_norm = their squared norm), which reset / add / add_view keep
    current; after writing q_sum or q_count directly, call refresh()."""

    def __init__(self, st, n_layer, n_head, head_dim, n_head_kv=0):
        dev = torch.device("cuda", st.device)
        self.st = st
        self.q_sum = torch.zeros((n_layer, n_head * head_dim), dtype=torch.float32, device=dev)
        self.q_count = torch.zeros((n_layer,), dtype=torch.int32, device=dev)
        self.q_vec = self.q_norm = None
        if n_head_kv:
            self.q_vec = torch.zeros((n_layer, n_head_kv, head_dim), dtype=torch.float32, device=dev)
            self.q_norm = torch.zeros((n_layer, n_head_kv), dtype=torch.float32, device=dev)
        self.c = L.QueryAcc(n_layer, n_head, head_dim, self.q_sum.data_ptr(), self.q_count.data_ptr(), n_head_kv,
                            self.q_vec.data_ptr() if n_head_kv else None,
                            self.q_norm.data_ptr() if n_head_kv else None)

    def reset(self):
        self.st.check(self.st.lib.kvm_query_reset(self.st.h, C.byref(self.c)))

    def refresh(self):
        self.st.check(self.st.lib.kvm_query_refresh(self.st.h, C.byref(self.c)))

    def add(self, il, q_rows):
        q_rows = q_rows.contiguous()
        self.st.check(self.st.lib.kvm_query_add(self.st.h, C.byref(self.c), il, _ptr(q_rows),
                                                q_rows.shape[0]))

    def add_view(self, il, q, keep=None):
        """q: device tensor [tokens][heads][dims] (any strides) of fp32 / fp16 / bf16;
        keep: host bool / uint8 array per token, or None for every token."""
        kp = None if keep is None else np.ascontiguousarray(keep, np.uint8)
        self.st.check(self.st.lib.kvm_query_add_view(self.st.h, C.byref(self.c), il, C.byref(view(q)),
                                                     None if kp is None else kp.ctypes.data))


class SelectionBuffers:
    """Device outputs of one retrieval (scores, ascending ids, window layout, staging list)."""

    def __init__(self, st, n_blocks, cap):
        dev = torch.device("cuda", st.device)
        self.scores = torch.zeros((max(n_blocks, 1),), dtype=torch.float64, device=dev)
        self.ids = torch.zeros((cap,), dtype=torch.int32, device=dev)
        self.to_base = torch.zeros((cap,), dtype=torch.int32, device=dev)
        self.stage_slots = torch.zeros((cap,), dtype=torch.int32, device=dev)
        self.info = torch.zeros((8,), dtype=torch.int32, device=dev)
        self.stage_src = torch.full((cap,), -1, dtype=torch.int32, device=dev)
        self.stage_out = torch.full((cap,), -1, dtype=torch.int32, device=dev)
        self.c = L.Selection(cap, self.scores.data_ptr(), self.ids.data_ptr(), self.to_base.data_ptr(),
                             self.stage_slots.data_ptr(), self.info.data_ptr(), self.stage_src.data_ptr(),
                             self.stage_out.data_ptr())

    def result(self):
        info = self.info.cpu().numpy().astype(np.int64)
        n = int(info[0])
        return {"ids": self.ids[:n].cpu().numpy().astype(np.int64),
                "to_base": self.to_base[:n].cpu().numpy().astype(np.int64),
                "total": int(info[1]), "stage_slots": self.stage_slots[:int(info[2])].cpu().numpy(),
                "stage_src": self.stage_src[:int(info[2])].cpu().numpy(),
                "stage_out": self.stage_out[:int(info[4])].cpu().numpy().astype(np.int64),
                "status": int(info[3])}


def score_topk(st, index, query, n_blocks, n_tokens, budget_blocks, sink_blocks=1, recent_blocks=0,
               mandatory=None, window=None, sel=None):
    """n_tokens: device int32 [n_blocks]; mandatory: device int32 tensor or None."""
    if sel is None:
        cap = min(n_blocks, budget_blocks) if budget_blocks else n_blocks
        sel = SelectionBuffers(st, n_blocks, max(cap, 1))
    p = L.SelectParams(n_blocks, budget_blocks, sink_blocks, recent_blocks,
                       None if mandatory is None else mandatory.data_ptr(),
                       0 if mandatory is None else mandatory.numel(), n_tokens.data_ptr())
    st.check(st.lib.kvm_score_topk(st.h, C.byref(index.c), C.byref(query.c), C.byref(p),
                                   None if window is None else C.byref(window.c), C.byref(sel.c)))
    return sel


def score_topk_lanes(st, lanes):
    """lanes: list of dicts with index, query, n_blocks, n_tokens, budget_blocks,
    sink_blocks, recent_blocks, window, sel (as score_topk).  One launch sequence."""
    keep = []
    arr = (L.RetrievalLane * len(lanes))()
    for i, ln in enumerate(lanes):
        p = L.SelectParams(ln["n_blocks"], ln["budget_blocks"], ln.get("sink_blocks", 1), ln.get("recent_blocks", 0),
                           None, 0, ln["n_tokens"].data_ptr())
        keep.append(p)
        arr[i] = L.RetrievalLane(C.pointer(ln["index"].c), C.pointer(ln["query"].c), C.pointer(p),
                                 C.pointer(ln["window"].c), C.pointer(ln["sel"].c))
    st.check(st.lib.kvm_score_topk_lanes(st.h, arr, len(lanes)))
    return [ln["sel"] for ln in lanes]


def select_topk(st, scores, n_tokens, budget_blocks, sink_blocks=1, recent_blocks=0, mandatory=None,
                window=None, sel=None):
    """Top-k + layout on given scores (device float64 [n_blocks])."""
    n_blocks = scores.numel()
    if sel is None:
        cap = min(n_blocks, budget_blocks) if budget_blocks else n_blocks
        sel = SelectionBuffers(st, n_blocks, max(cap, 1))
    p = L.SelectParams(n_blocks, budget_blocks, sink_blocks, recent_blocks,
                       None if mandatory is None else mandatory.data_ptr(),
                       0 if mandatory is None else mandatory.numel(), n_tokens.data_ptr())
    st.check(st.lib.kvm_select_topk(st.h, C.c_void_p(scores.data_ptr()), C.byref(p),
                                    None if window is None else C.byref(window.c), C.byref(sel.c)))
    return sel


class SlotPool:
    """Host free list of window slots (kvm_slot_pool: reset_slots / alloc_slot /
    free_slot of the reference adapter)."""

    def __init__(self, n_slots):
        self.lib = L.load()
        self.buf = np.zeros(max(n_slots, 1), np.int32)
        self.c = L.SlotPool(n_slots, 0, self.buf.ctypes.data)
        self.reset()

    def reset(self):
        rc = self.lib.kvm_slot_pool_reset(C.byref(self.c))
        if rc:
            raise L.KvmError(rc, "kvm_slot_pool_reset")

    def alloc(self):
        return self.lib.kvm_slot_alloc(C.byref(self.c))

    def free(self, slot):
        rc = self.lib.kvm_slot_free(C.byref(self.c), slot)
        if rc:
            raise L.KvmError(rc, "kvm_slot_free")


def _layers(windows):
    arr = (C.POINTER(L.Window) * len(windows))()
    for i, w in enumerate(windows):
        arr[i] = C.pointer(w.c)
    return arr


def slot_copy_to_host(st, windows, slot):
    """One slot of every layer's window as bytes: per layer, block_tokens K rows then V rows."""
    need = sum(w.block_tokens * (w.k_row_bytes() + w.v_row_bytes()) for w in windows)
    out = np.zeros(need, np.uint8)
    st.check(st.lib.kvm_slot_copy_to_host(st.h, _layers(windows), len(windows), slot, out.ctypes.data, need))
    return out


def slot_copy_from_host(st, windows, slot, data):
    data = np.ascontiguousarray(data, np.uint8)
    st.check(st.lib.kvm_slot_copy_from_host(st.h, _layers(windows), len(windows), slot, data.ctypes.data, data.nbytes))


def harvest_block(st, window, cell0, n, k_prerope, tok0, k_raw_rows, v_rows, index=None, il=0, pos0=0):
    """kvm_harvest_block: k_raw_rows / v_rows are numpy uint8 arrays (the history
    rows of the tokens); returns after the copies are complete."""
    st.check(st.lib.kvm_harvest_block(st.h, C.byref(window.c), cell0, n, C.byref(view(k_prerope)), tok0,
                                      k_raw_rows.ctypes.data, v_rows.ctypes.data,
                                      None if index is None else C.byref(index.c), il, pos0))
    st.sync()


def retrieval_mandatory(n_tokens, spans=None, query_begin=-1, query_end=0, force_pos=-1):
    """Mandatory block ids of a retrieval (kvm_retrieval_mandatory): n_tokens is
    the host per-block token count, spans the turn's explicit (begin, end) row
    ranges (None = the turn set none: the query span applies; [] = explicit and
    empty)."""
    lib = L.load()
    nt = np.ascontiguousarray(n_tokens, np.uint32)
    arr = None if spans is None else (L.RowRange * max(len(spans), 1))(*[L.RowRange(int(b), int(e)) for b, e in spans])
    out = np.zeros(nt.size + 1, np.uint32)
    n = L._u32(0)
    rc = lib.kvm_retrieval_mandatory(None, nt.ctypes.data, nt.size, arr, 0 if spans is None else len(spans),
                                     query_begin, query_end, force_pos, out.ctypes.data, out.size, C.byref(n))
    if rc:
        raise L.KvmError(rc, "kvm_retrieval_mandatory")
    return out[:n.value].astype(np.int64)


def stagein_selection(st, history, window, sel, n_rot, freq_base, freq_scale=1.0, hadamard_nrot=-1):
    r = L.RopeParams(n_rot, freq_base, freq_scale, hadamard_nrot)
    st.check(st.lib.kvm_stagein_selection(st.h, C.byref(history.c), C.byref(window.c), C.byref(sel.c),
                                          C.byref(r)))


class History:
    """Pinned host history of one layer: raw (pre-RoPE) K rows and V rows in cache format."""

    def __init__(self, k_rows_np, v_rows_np):
        n = k_rows_np.shape[0]
        self.kbuf = HostBuffer(k_rows_np.nbytes)
        self.vbuf = HostBuffer(v_rows_np.nbytes)
        self.kbuf.u8[:] = np.ascontiguousarray(k_rows_np).reshape(-1).view(np.uint8)
        self.vbuf.u8[:] = np.ascontiguousarray(v_rows_np).reshape(-1).view(np.uint8)
        self.c = L.History(self.kbuf.ptr, self.vbuf.ptr, n)
        self.n_tokens = n


def fa_decode(st, window, q, q_pos, n_head, scale, out=None):
    """q: device [n_tokens][n_head][head_dim] fp32 or bf16; q_pos: device int32 [n_tokens]."""
    q = q.contiguous()
    n_tokens = q.shape[0]
    if out is None:
        out = torch.empty((n_tokens, n_head, window.head_dim), dtype=torch.float32, device=q.device)
    qt = L.T_BF16 if q.dtype == torch.bfloat16 else L.T_F32
    st.check(st.lib.kvm_fa_decode(st.h, C.byref(window.c), _ptr(q), qt, _ptr(q_pos), n_tokens, n_head,
                                  float(scale), _ptr(out)))
    return out


def fa_prefill(st, window, q, q_pos, n_head, scale, out=None):
    q = q.contiguous()
    n_tokens = q.shape[0]
    if out is None:
        out = torch.empty((n_tokens, n_head, window.head_dim), dtype=torch.float32, device=q.device)
    qt = L.T_BF16 if q.dtype == torch.bfloat16 else L.T_F32
    st.check(st.lib.kvm_fa_prefill(st.h, C.byref(window.c), _ptr(q), qt, _ptr(q_pos), n_tokens, n_head,
                                   float(scale), _ptr(out)))
    return out


def fa_decode_lanes(st, windows, qs, q_poss, n_head, scale, outs=None):
    n = len(windows)
    if outs is None:
        outs = [torch.empty((q.shape[0], n_head, w.head_dim), dtype=torch.float32, device=q.device)
                for w, q in zip(windows, qs)]
    lanes = (L.Lane * n)()
    keep = []
    for i, (w, q, qp, o) in enumerate(zip(windows, qs, q_poss, outs)):
        q = q.contiguous()
        keep.append(q)
        lanes[i] = L.Lane(C.pointer(w.c), q.data_ptr(), qp.data_ptr(), o.data_ptr(), q.shape[0])
    qt = L.T_BF16 if qs[0].dtype == torch.bfloat16 else L.T_F32
    st.check(st.lib.kvm_fa_decode_lanes(st.h, lanes, n, qt, n_head, float(scale)))
    return outs


class Prepared:
    """One library call with its ctypes arguments built once, for step loops:
    calling it costs one foreign call and no argument marshalling."""

    def __init__(self, st, fn, args, keep=()):
        self.st, self.fn, self.args, self.keep = st, fn, args, keep

    def __call__(self):
        rc = self.fn(*self.args)
        if rc:
            self.st.check(rc)


def prepare_score_topk(st, index, query, n_blocks, n_tokens, budget_blocks, sink_blocks, recent_blocks, window, sel):
    p = L.SelectParams(n_blocks, budget_blocks, sink_blocks, recent_blocks, None, 0, n_tokens.data_ptr())
    return Prepared(st, st.lib.kvm_score_topk,
                    (st.h, C.byref(index.c), C.byref(query.c), C.byref(p), C.byref(window.c), C.byref(sel.c)),
                    (p, index, query, window, sel, n_tokens))


def prepare_score_topk_lanes(st, lanes):
    keep, arr = [], (L.RetrievalLane * len(lanes))()
    for i, ln in enumerate(lanes):
        p = L.SelectParams(ln["n_blocks"], ln["budget_blocks"], ln.get("sink_blocks", 1), ln.get("recent_blocks", 0),
                           None, 0, ln["n_tokens"].data_ptr())
        keep += [p, ln]
        arr[i] = L.RetrievalLane(C.pointer(ln["index"].c), C.pointer(ln["query"].c), C.pointer(p),
                                 C.pointer(ln["window"].c), C.pointer(ln["sel"].c))
    return Prepared(st, st.lib.kvm_score_topk_lanes, (st.h, arr, len(lanes)), (keep, arr))


def prepare_score_topk_stagein(st, index, query, n_blocks, n_tokens, budget_blocks, sink_blocks, recent_blocks,
                               window, sel, history, n_rot, freq_base, freq_scale=1.0, hadamard_nrot=-1):
    """kvm_score_topk_stagein: the scoring grid, the top-k and the stage-in of
    its plan (three launches, every argument checked before the first)."""
    p = L.SelectParams(n_blocks, budget_blocks, sink_blocks, recent_blocks, None, 0, n_tokens.data_ptr())
    r = L.RopeParams(n_rot, freq_base, freq_scale, hadamard_nrot)
    return Prepared(st, st.lib.kvm_score_topk_stagein,
                    (st.h, C.byref(index.c), C.byref(query.c), C.byref(p), C.byref(window.c), C.byref(sel.c),
                     C.byref(history.c), C.byref(r)),
                    (p, r, index, query, window, sel, n_tokens, history))


def score_topk_stagein(st, index, query, n_blocks, n_tokens, budget_blocks, sink_blocks, recent_blocks, window,
                       sel, history, n_rot, freq_base, freq_scale=1.0, hadamard_nrot=-1):
    prepare_score_topk_stagein(st, index, query, n_blocks, n_tokens, budget_blocks, sink_blocks, recent_blocks,
                               window, sel, history, n_rot, freq_base, freq_scale, hadamard_nrot)()
    return sel


def prepare_score_topk_stagein_lanes(st, lanes, n_rot, freq_base, freq_scale=1.0, hadamard_nrot=-1):
    """lanes: score_topk_lanes dicts with a "history" each (kvm_score_topk_stagein_lanes)."""
    keep, arr = [], (L.RetrievalLane * len(lanes))()
    hists = (C.POINTER(L.History) * len(lanes))()
    for i, ln in enumerate(lanes):
        p = L.SelectParams(ln["n_blocks"], ln["budget_blocks"], ln.get("sink_blocks", 1), ln.get("recent_blocks", 0),
                           None, 0, ln["n_tokens"].data_ptr())
        keep += [p, ln]
        arr[i] = L.RetrievalLane(C.pointer(ln["index"].c), C.pointer(ln["query"].c), C.pointer(p),
                                 C.pointer(ln["window"].c), C.pointer(ln["sel"].c))
        hists[i] = C.pointer(ln["history"].c)
    r = L.RopeParams(n_rot, freq_base, freq_scale, hadamard_nrot)
    return Prepared(st, st.lib.kvm_score_topk_stagein_lanes, (st.h, arr, hists, len(lanes), C.byref(r)),
                    (keep, arr, hists, r))


def prepare_stagein(st, history, window, sel, n_rot, freq_base, freq_scale=1.0, hadamard_nrot=-1):
    r = L.RopeParams(n_rot, freq_base, freq_scale, hadamard_nrot)
    return Prepared(st, st.lib.kvm_stagein_selection,
                    (st.h, C.byref(history.c), C.byref(window.c), C.byref(sel.c), C.byref(r)),
                    (r, history, window, sel))


def prepare_stagein_lanes(st, lanes, n_rot, freq_base, freq_scale=1.0, hadamard_nrot=-1):
    """lanes: (history, window, selection) triples, staged in one launch."""
    r = L.RopeParams(n_rot, freq_base, freq_scale, hadamard_nrot)
    arr = (L.StageinLane * len(lanes))()
    for i, (h, w, sel) in enumerate(lanes):
        arr[i] = L.StageinLane(C.pointer(h.c), C.pointer(w.c), C.pointer(sel.c))
    return Prepared(st, st.lib.kvm_stagein_selection_lanes, (st.h, arr, len(lanes), C.byref(r)), (r, arr, lanes))


def stagein_selection_lanes(st, lanes, n_rot, freq_base, freq_scale=1.0, hadamard_nrot=-1):
    prepare_stagein_lanes(st, lanes, n_rot, freq_base, freq_scale, hadamard_nrot)()


def prepare_fa_decode(st, window, q, q_pos, n_head, scale, out):
    qt = L.T_BF16 if q.dtype == torch.bfloat16 else L.T_F32
    return Prepared(st, st.lib.kvm_fa_decode,
                    (st.h, C.byref(window.c), _ptr(q), qt, _ptr(q_pos), q.shape[0], n_head, float(scale), _ptr(out)),
                    (window, q, q_pos, out))


def prepare_fa_decode_lanes(st, windows, qs, q_poss, n_head, scale, outs):
    n = len(windows)
    lanes = (L.Lane * n)()
    for i, (w, q, qp, o) in enumerate(zip(windows, qs, q_poss, outs)):
        lanes[i] = L.Lane(C.pointer(w.c), q.data_ptr(), qp.data_ptr(), o.data_ptr(), q.shape[0])
    qt = L.T_BF16 if qs[0].dtype == torch.bfloat16 else L.T_F32
    return Prepared(st, st.lib.kvm_fa_decode_lanes, (st.h, lanes, n, qt, n_head, float(scale)),
                    (lanes, windows, qs, q_poss, outs))


def prepare_stagein_fa_decode(st, history, sel, window, q, q_pos, n_head, scale, out, n_rot, freq_base,
                              freq_scale=1.0, hadamard_nrot=-1):
    """kvm_stagein_fa_decode: the selection's stage-in plan and the decode
    attention over `window` in one launch."""
    r = L.RopeParams(n_rot, freq_base, freq_scale, hadamard_nrot)
    qt = L.T_BF16 if q.dtype == torch.bfloat16 else L.T_F32
    return Prepared(st, st.lib.kvm_stagein_fa_decode,
                    (st.h, C.byref(history.c), C.byref(sel.c), C.byref(r), C.byref(window.c), _ptr(q), qt,
                     _ptr(q_pos), q.shape[0], n_head, float(scale), _ptr(out)),
                    (r, history, sel, window, q, q_pos, out))


def stagein_fa_decode(st, history, sel, window, q, q_pos, n_head, scale, n_rot, freq_base, freq_scale=1.0,
                      hadamard_nrot=-1, out=None):
    q = q.contiguous()
    if out is None:
        out = torch.empty((q.shape[0], n_head, window.head_dim), dtype=torch.float32, device=q.device)
    prepare_stagein_fa_decode(st, history, sel, window, q, q_pos, n_head, scale, out, n_rot, freq_base, freq_scale,
                              hadamard_nrot)()
    return out


def prepare_stagein_fa_decode_lanes(st, lanes, n_head, scale, n_rot, freq_base, freq_scale=1.0, hadamard_nrot=-1):
    """lanes: dicts with history, sel, window, q, q_pos, out (kvm_stagein_fa_decode_lanes)."""
    n = len(lanes)
    sg, fl = (L.StageinLane * n)(), (L.Lane * n)()
    for i, ln in enumerate(lanes):
        sg[i] = L.StageinLane(C.pointer(ln["history"].c), C.pointer(ln["window"].c), C.pointer(ln["sel"].c))
        fl[i] = L.Lane(C.pointer(ln["window"].c), ln["q"].data_ptr(), ln["q_pos"].data_ptr(), ln["out"].data_ptr(),
                       ln["q"].shape[0])
    r = L.RopeParams(n_rot, freq_base, freq_scale, hadamard_nrot)
    qt = L.T_BF16 if lanes[0]["q"].dtype == torch.bfloat16 else L.T_F32
    return Prepared(st, st.lib.kvm_stagein_fa_decode_lanes, (st.h, sg, fl, n, C.byref(r), qt, n_head, float(scale)),
                    (sg, fl, r, lanes))


def prepare_decode_step(st, index, query, n_blocks, n_tokens, budget_blocks, sink_blocks, recent_blocks, window,
                        sel, history, q, q_pos, n_head, scale, out, n_rot, freq_base, freq_scale=1.0,
                        hadamard_nrot=-1, mandatory=None):
    """kvm_score_topk_stagein_fa_decode: a whole decode step (scoring, top-k,
    stage-in of the plan into `window`, decode attention over it) in two
    launches.  mandatory: device int32 block ids (newest last) or None."""
    p = L.SelectParams(n_blocks, budget_blocks, sink_blocks, recent_blocks,
                       None if mandatory is None else mandatory.data_ptr(),
                       0 if mandatory is None else mandatory.numel(), n_tokens.data_ptr())
    r = L.RopeParams(n_rot, freq_base, freq_scale, hadamard_nrot)
    qt = L.T_BF16 if q.dtype == torch.bfloat16 else L.T_F32
    return Prepared(st, st.lib.kvm_score_topk_stagein_fa_decode,
                    (st.h, C.byref(index.c), C.byref(query.c), C.byref(p), C.byref(window.c), C.byref(sel.c),
                     C.byref(history.c), C.byref(r), _ptr(q), qt, _ptr(q_pos), q.shape[0], n_head, float(scale),
                     _ptr(out)),
                    (p, r, index, query, window, sel, n_tokens, history, q, q_pos, out, mandatory))


def prepare_select_decode_step(st, scores, n_tokens, budget_blocks, sink_blocks, recent_blocks, window, sel,
                               history, q, q_pos, n_head, scale, out, n_rot, freq_base, freq_scale=1.0,
                               hadamard_nrot=-1, mandatory=None):
    """kvm_select_topk_stagein_fa_decode: the decode step from caller scores
    (device float64 [n_blocks]) in one launch."""
    p = L.SelectParams(scores.numel(), budget_blocks, sink_blocks, recent_blocks,
                       None if mandatory is None else mandatory.data_ptr(),
                       0 if mandatory is None else mandatory.numel(), n_tokens.data_ptr())
    r = L.RopeParams(n_rot, freq_base, freq_scale, hadamard_nrot)
    qt = L.T_BF16 if q.dtype == torch.bfloat16 else L.T_F32
    return Prepared(st, st.lib.kvm_select_topk_stagein_fa_decode,
                    (st.h, _ptr(scores), C.byref(p), C.byref(window.c), C.byref(sel.c), C.byref(history.c),
                     C.byref(r), _ptr(q), qt, _ptr(q_pos), q.shape[0], n_head, float(scale), _ptr(out)),
                    (p, r, scores, window, sel, n_tokens, history, q, q_pos, out, mandatory))


def decode_step(st, index, query, n_blocks, n_tokens, budget_blocks, sink_blocks, recent_blocks, window, sel,
                history, q, q_pos, n_head, scale, n_rot, freq_base, freq_scale=1.0, hadamard_nrot=-1, out=None,
                mandatory=None):
    q = q.contiguous()
    if out is None:
        out = torch.empty((q.shape[0], n_head, window.head_dim), dtype=torch.float32, device=q.device)
    prepare_decode_step(st, index, query, n_blocks, n_tokens, budget_blocks, sink_blocks, recent_blocks, window,
                        sel, history, q, q_pos, n_head, scale, out, n_rot, freq_base, freq_scale, hadamard_nrot,
                        mandatory)()
    return out


def prepare_decode_step_lanes(st, lanes, n_head, scale, n_rot, freq_base, freq_scale=1.0, hadamard_nrot=-1):
    """lanes: score_topk_lanes dicts with history, q, q_pos, out as well
    (kvm_score_topk_stagein_fa_decode_lanes)."""
    n = len(lanes)
    keep, arr = [], (L.RetrievalLane * n)()
    hists, fl = (C.POINTER(L.History) * n)(), (L.Lane * n)()
    for i, ln in enumerate(lanes):
        p = L.SelectParams(ln["n_blocks"], ln["budget_blocks"], ln.get("sink_blocks", 1), ln.get("recent_blocks", 0),
                           None, 0, ln["n_tokens"].data_ptr())
        keep += [p, ln]
        arr[i] = L.RetrievalLane(C.pointer(ln["index"].c), C.pointer(ln["query"].c), C.pointer(p),
                                 C.pointer(ln["window"].c), C.pointer(ln["sel"].c))
        hists[i] = C.pointer(ln["history"].c)
        fl[i] = L.Lane(C.pointer(ln["window"].c), ln["q"].data_ptr(), ln["q_pos"].data_ptr(), ln["out"].data_ptr(),
                       ln["q"].shape[0])
    r = L.RopeParams(n_rot, freq_base, freq_scale, hadamard_nrot)
    qt = L.T_BF16 if lanes[0]["q"].dtype == torch.bfloat16 else L.T_F32
    return Prepared(st, st.lib.kvm_score_topk_stagein_fa_decode_lanes,
                    (st.h, arr, hists, fl, n, C.byref(r), qt, n_head, float(scale)), (keep, arr, hists, fl, r))


def quantize_rows(st, ty, x):
    """x: device fp32 [n_rows][n_per_row] -> uint8 ggml rows."""
    x = x.contiguous()
    n_rows, n = x.shape
    out = torch.empty((n_rows, row_bytes(ty, n)), dtype=torch.uint8, device=x.device)
    st.check(st.lib.kvm_quantize_rows(st.h, ty, _ptr(x), _ptr(out), n_rows, n))
    return out


def dequantize_rows(st, ty, rows, n_per_row):
    n_rows = rows.shape[0]
    out = torch.empty((n_rows, n_per_row), dtype=torch.float32, device=rows.device)
    st.check(st.lib.kvm_dequantize_rows(st.h, ty, _ptr(rows), _ptr(out), n_rows, n_per_row))
    return out


def read_snapshot(data, max_blocks=(1 << 64) - 1, expect=None):
    """Parse the reference's raw-store session snapshot (RawKvStore::snapshot_write,
    raw_kv_store.cpp:1225-1247) into per-layer host arrays in the history layout:
    k_rows / v_rows [n_blocks * block_tokens, row bytes] (uint8), k_sum [n_blocks,
    n_embd_k], mean_tokens and n_tokens [n_blocks].  Host-side parsing only.
    max_blocks: the store's block count (the reader accepts max_blocks + 1 blocks,
    raw_kv_store.cpp:1255-1256); expect: dict of the store's geometry
    (SnapshotInfo field names) the header must equal, or None."""
    lib = L.load()
    buf = np.frombuffer(data, dtype=np.uint8)
    info = L.SnapshotInfo()
    rc = lib.kvm_snapshot_info_read(None, buf.ctypes.data, buf.size, C.byref(info))
    if rc:
        raise RuntimeError(f"kvm_snapshot_info_read: {rc}")
    ex = None
    if expect is not None:
        ex = L.SnapshotInfo(**{f: expect.get(f, 0) for f, _ in L.SnapshotInfo._fields_})
    nb, bt = int(info.n_blocks), int(info.block_tokens)
    layers = []
    for il in range(info.n_layer):
        k = np.zeros((nb * bt, int(info.k_row_bytes)), np.uint8)
        v = np.zeros((nb * bt, int(info.v_gpu_row_bytes)), np.uint8)
        ks = np.zeros((nb, int(info.n_embd_k)), np.float32)
        mt = np.zeros(nb, np.uint32)
        nt = np.zeros(nb, np.uint32)
        out = L.SnapshotLayer(k.ctypes.data, k.nbytes, v.ctypes.data if v.size else None, v.nbytes,
                              ks.ctypes.data, mt.ctypes.data, nt.ctypes.data, max_blocks,
                              C.pointer(ex) if ex is not None else None)
        rc = lib.kvm_snapshot_read_layer(None, buf.ctypes.data, buf.size, il, C.byref(out))
        if rc:
            raise RuntimeError(f"kvm_snapshot_read_layer: {rc}")
        layers.append(dict(k_rows=k, v_rows=v, k_sum=ks, mean_tokens=mt, n_tokens=nt))
    return {f: getattr(info, f) for f, _ in L.SnapshotInfo._fields_}, layers
