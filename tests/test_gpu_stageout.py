"""Stage-out side of the window: the slot seam's byte copies (copy_block_to_host
/ _from_host, llama-memory-kvmem.cpp:4073-4147) and the harvest of generated
blocks into the host history (harvest_gpu_v, llama-memory-kvmem.cpp:3583-3690;
stage-out gather + D2H, llama-kvmem-stagein.cu:879-969), then the cycle the
runtime orders (stage-out before stage-in, kvmem_runtime.cpp:121-126, 225-249):
a harvested block leaves the window and a later retrieval stages it back from
the history, byte-equal to the oracle's stage-in of the harvested rows."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import dev, host, rand_rows
from kvmem_amd import api, _lib as L

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kt,vt,H,D", [(L.T_Q8_0, L.T_Q4_0, 4, 256), (L.T_F16, L.T_F16, 2, 128)])
def test_slot_copies_round_trip(kvm_state, kt, vt, H, D):
    rng = np.random.default_rng(31)
    bt, n_cells = 128, 8 * 128
    layers = []
    for il in range(3):
        w = api.KVWindow(kvm_state, n_cells, H, D, bt, kt, vt)
        kr, vr = rand_rows(rng, n_cells, H, D, kt, vt)
        w.import_rows(0, dev(kr), dev(vr), dev(np.arange(n_cells, dtype=np.int32)))
        layers.append((w, kr, vr))
    ws = [w for w, _, _ in layers]
    blob = api.slot_copy_to_host(kvm_state, ws, 3)
    off = 0
    for w, kr, vr in layers:
        kb, vb = bt * w.k_row_bytes(), bt * w.v_row_bytes()
        assert np.array_equal(blob[off:off + kb], kr[3 * bt:4 * bt].reshape(-1))
        assert np.array_equal(blob[off + kb:off + kb + vb], vr[3 * bt:4 * bt].reshape(-1))
        off += kb + vb
    assert off == blob.size
    # into slot 6 of three empty windows: their rows now equal slot 3's
    dst = [api.KVWindow(kvm_state, n_cells, H, D, bt, kt, vt) for _ in range(3)]
    api.slot_copy_from_host(kvm_state, dst, 6, blob)
    for w, (_, kr, vr) in zip(dst, layers):
        ek, ev = w.export_rows(6 * bt, bt)
        assert np.array_equal(host(ek), kr[3 * bt:4 * bt]) and np.array_equal(host(ev), vr[3 * bt:4 * bt])
    with pytest.raises(L.KvmError):                         # too few bytes
        api.slot_copy_from_host(kvm_state, dst, 6, blob[:-1])
    with pytest.raises(L.KvmError):                         # slot past the window
        api.slot_copy_to_host(kvm_state, ws, 8)


@pytest.mark.parametrize("kt", [L.T_Q8_0, L.T_Q4_0])
def test_harvest_then_restage(kvm_state, kt):
    """Generated tokens occupy slot 5 of the window (window positions 640..767,
    original positions 4*128.. of the history); the harvest writes their
    captured pre-RoPE K quantised to the cache's K type (q8_0 or q4_0) and their window V rows as history
    block 4 and adds the K to the mean-K index; a reselect that drops the block
    reuses the slot, and a later one that picks it again stages it back from the
    history exactly as the oracle stages the harvested rows."""
    rng = np.random.default_rng(32)
    H, D, bt, n_hist_blocks = 4, 256, 128, 8
    n_hist = n_hist_blocks * bt
    kr, vr = rand_rows(rng, n_hist, H, D, kt, L.T_Q4_0)
    k_hist = np.zeros_like(kr)
    v_hist = np.zeros_like(vr)
    k_hist[:4 * bt], v_hist[:4 * bt] = kr[:4 * bt], vr[:4 * bt]     # blocks 4.. are not harvested yet
    hist = api.History(k_hist, v_hist)
    w = api.KVWindow(kvm_state, 6 * bt, H, D, bt, kt, L.T_Q4_0)
    # generated block: rotated K rows in the cache (any bytes), V rows, positions
    gk, gv = rand_rows(rng, bt, H, D, kt, L.T_Q4_0)
    w.import_rows(5 * bt, dev(gk), dev(gv), dev(np.arange(5 * bt, 6 * bt, dtype=np.int32)))
    cap = torch.from_numpy(rng.standard_normal((bt + 3, H, D)).astype(np.float32)).to(torch.bfloat16).cuda()
    cap = cap.permute(1, 0, 2).contiguous().permute(1, 0, 2)          # the captured view, heads-major storage
    ix = api.MeanKIndex(kvm_state, 1, n_hist_blocks, H, D, bt, norms=True)
    api.harvest_block(kvm_state, w, 5 * bt, bt, cap, 3, hist.kbuf.u8[4 * bt * w.k_row_bytes():].reshape(-1)[:bt * w.k_row_bytes()],
                      hist.vbuf.u8[4 * bt * w.v_row_bytes():].reshape(-1)[:bt * w.v_row_bytes()], ix, 0, 4 * bt)
    k32 = cap[3:].float().cpu().numpy().reshape(bt, -1)
    want_k = O.quant(kt, k32.reshape(-1)).reshape(bt, -1)
    got_k = hist.kbuf.u8.reshape(n_hist, -1)[4 * bt:5 * bt]
    assert np.array_equal(got_k, want_k)
    assert np.array_equal(hist.vbuf.u8.reshape(n_hist, -1)[4 * bt:5 * bt], gv)
    sums, mt = O.meank_sums(k32, bt)
    assert np.array_equal(host(ix.block_sums())[0][4].view(np.uint32), sums[0].view(np.uint32))
    assert int(host(ix.mean_tokens)[0][4]) == bt
    # the harvest's add kept the block's nk current: a refresh leaves it bit-equal
    kn = ix.k_norm.clone()
    ix.refresh()
    assert torch.equal(kn.view(torch.int32), ix.k_norm.view(torch.int32)) and bool((kn[0, :, 4] > 0).all())
    # the window's slot map: slots 0..3 hold blocks 0..3; block 4 leaves and comes back
    nt = dev(np.full(n_hist_blocks, bt, np.int32))
    s = np.zeros(n_hist_blocks)
    s[[1, 2, 3]] = [3, 2, 1]
    sel = api.select_topk(kvm_state, dev(s), nt, 4, 1, 0, None, window=w)
    api.stagein_selection(kvm_state, hist, w, sel, 64, 1e7)
    s[3], s[4] = 0.0, 5.0                                              # block 4 (harvested) is picked
    sel = api.select_topk(kvm_state, dev(s), nt, 4, 1, 0, None, window=w)
    api.stagein_selection(kvm_state, hist, w, sel, 64, 1e7)
    r = sel.result()
    assert list(r["ids"]) == [0, 1, 2, 4] and r["status"] == 0
    theta = O.rope_theta(1e7, 1.0, 64)
    ek, ev = w.export_rows(3 * bt, bt)
    assert np.array_equal(host(ek).reshape(-1), O.stagein_k(want_k.reshape(-1), bt, H, D, 64, 256, 3 * bt, theta,
                                                          k_type=kt))
    assert np.array_equal(host(ev), gv)


def test_plan_refuses_to_overwrite_unharvested_rows(kvm_state):
    """Stage-out before stage-in (apply_plan_to_kv: harvest_gpu_v of every
    stage_out block, then spill_outgoing and admit_incoming,
    llama-memory-kvmem.cpp:1811-1857, kvmem_runtime.cpp:225-249): a window that
    counts its unharvested rows refuses a plan that would overwrite a slot
    holding generated rows (info[3] bit 2, window untouched, stage_out still
    listing the blocks that leave); after the harvest the same selection
    stages, byte-equal to a fresh stage-in into a window without tracking."""
    st = kvm_state
    rng = np.random.default_rng(33)
    H, D, bt, n_blocks = 4, 256, 128, 12
    kr, vr = rand_rows(rng, n_blocks * bt, H, D, L.T_Q8_0, L.T_Q4_0)
    hist = api.History(kr, vr)
    nt = dev(np.full(n_blocks, bt, np.int32))
    w = api.KVWindow(st, 6 * bt, H, D, bt, pending=True)

    def scores(chosen):
        s = np.zeros(n_blocks)
        s[list(chosen)] = 1.0 + np.arange(len(chosen))
        return dev(s)
    # the first plan: blocks 0 (sink), 3, 5, 7 in slots 0..3
    sel = api.select_topk(st, scores([3, 5, 7]), nt, 4, 1, 0, None, window=w)
    api.stagein_selection(st, hist, w, sel, 64, 1e7)
    r = sel.result()
    assert list(r["ids"]) == [0, 3, 5, 7] and r["status"] == 0 and len(r["stage_out"]) == 0
    # a generated block's rows in slot 4 (window positions 512..639), not harvested
    gk, gv = rand_rows(rng, bt, H, D, L.T_Q8_0, L.T_Q4_0)
    w.import_rows(4 * bt, dev(gk), dev(gv), dev(np.arange(4 * bt, 5 * bt, dtype=np.int32)))
    assert host(w.pending_rows).tolist() == [0, 0, 0, 0, bt, 0]
    before = {k: getattr(w, k).clone() for k in ("k", "v", "cell_pos", "slot_block", "slot_base")}
    # a plan of five blocks: block 3 leaves, and slot 4 would be overwritten
    want = [0, 5, 7, 9, 11]
    sel = api.select_topk(st, scores([5, 7, 9, 11]), nt, 5, 1, 0, None, window=w)
    api.stagein_selection(st, hist, w, sel, 64, 1e7)
    r = sel.result()
    assert list(r["ids"]) == want
    assert r["status"] & 4, r["status"]
    assert list(r["stage_out"]) == [3]
    for k, v in before.items():
        assert torch.equal(getattr(w, k), v), k
    # the harvest takes the generated rows into the host history (as block 11
    # here, whose rows the test then restores), and the plan stages
    cap = torch.from_numpy(rng.standard_normal((bt, H, D)).astype(np.float32)).cuda()
    hk = np.zeros((bt, w.k_row_bytes()), np.uint8)
    hv = np.zeros((bt, w.v_row_bytes()), np.uint8)
    hk_buf, hv_buf = api.HostBuffer(hk.nbytes), api.HostBuffer(hv.nbytes)
    api.harvest_block(st, w, 4 * bt, bt, cap, 0, hk_buf.u8, hv_buf.u8)
    st.sync()
    assert host(w.pending_rows).tolist() == [0] * 6
    assert np.array_equal(hv_buf.u8.reshape(bt, -1), gv)
    sel = api.select_topk(st, scores([5, 7, 9, 11]), nt, 5, 1, 0, None, window=w)
    api.stagein_selection(st, hist, w, sel, 64, 1e7)
    r = sel.result()
    assert list(r["ids"]) == want and r["status"] == 0 and list(r["stage_out"]) == [3]
    fresh = api.KVWindow(st, 6 * bt, H, D, bt)
    sf = api.select_topk(st, scores([5, 7, 9, 11]), nt, 5, 1, 0, None, window=fresh)
    api.stagein_selection(st, hist, fresh, sf, 64, 1e7)
    st.sync()
    for k in ("cell_pos", "slot_block", "slot_base"):
        assert torch.equal(getattr(w, k)[:5 * bt if k == "cell_pos" else 5], getattr(fresh, k)[:5 * bt if k == "cell_pos" else 5]), k
    ka, va = w.export_rows(0, 5 * bt)
    kb, vb = fresh.export_rows(0, 5 * bt)
    assert torch.equal(ka, kb) and torch.equal(va, vb)


def test_pending_rows_record_the_end_of_the_imported_rows(kvm_state):
    """A slot's pending count is the end of its unharvested imported rows: a
    re-import of the same cells (rows rewritten after rejected draft tokens)
    adds nothing, a harvest that stops short of the end leaves it, one that
    reaches it clears it, and a copy of the slot from the host clears it."""
    st = kvm_state
    rng = np.random.default_rng(35)
    H, D, bt = 4, 256, 128
    w = api.KVWindow(st, 4 * bt, H, D, bt, pending=True)

    def imp(c0, n):
        kr, vr = rand_rows(rng, n, H, D, L.T_Q8_0, L.T_Q4_0)
        w.import_rows(c0, dev(kr), dev(vr), dev(np.arange(c0, c0 + n, dtype=np.int32)))

    def harvest(c0, n):
        cap = torch.from_numpy(rng.standard_normal((n, H, D)).astype(np.float32)).cuda()
        hk, hv = api.HostBuffer(n * w.k_row_bytes()), api.HostBuffer(n * w.v_row_bytes())
        api.harvest_block(st, w, c0, n, cap, 0, hk.u8, hv.u8)

    pend = lambda: host(w.pending_rows).tolist()
    imp(bt + 2, 3)
    assert pend() == [0, 5, 0, 0]
    imp(bt + 2, 3)
    assert pend() == [0, 5, 0, 0]
    imp(bt - 3, 15)                        # across the slot boundary
    assert pend() == [bt, 12, 0, 0]
    harvest(bt, 5)                         # stops short of row 12
    assert pend() == [bt, 12, 0, 0]
    harvest(bt + 5, 7)
    assert pend() == [bt, 0, 0, 0]
    blob = api.slot_copy_to_host(st, [w], 0)
    api.slot_copy_from_host(st, [w], 0, blob)
    assert pend() == [0, 0, 0, 0]


def test_stage_out_lists_the_blocks_that_leave(kvm_state):
    """stage_out = the blocks the plan's slots held that the new selection
    drops, ascending (KvMemStore::set_selection's stage_out for GPU-resident
    blocks, kvmem_store.cpp:789-795), against the set difference."""
    st = kvm_state
    rng = np.random.default_rng(34)
    n_blocks, budget, bt = 40, 12, 128
    nt = dev(np.full(n_blocks, bt, np.int32))
    w = api.KVWindow(st, 16 * bt, 2, 128, bt, L.T_F16, L.T_F16)
    prev = None
    for step in range(6):
        s = rng.standard_normal(n_blocks)
        sel = api.select_topk(st, dev(s), nt, budget, 1, 1, None, window=w)
        r = sel.result()
        held = [int(b) for b in host(w.slot_block)[:budget] if 0 <= int(b) < n_blocks]
        want = sorted(set(held) - set(int(i) for i in r["ids"]))
        assert list(r["stage_out"]) == want, (step, list(r["stage_out"]), want)
        # the window takes the plan's layout as a stage-in would (slot map only)
        ids, tb = r["ids"], r["to_base"]
        sb = np.full(16, -1, np.int32)
        sbase = np.full(16, -1, np.int32)
        sb[:len(ids)], sbase[:len(ids)] = ids, tb
        w.slot_block.copy_(dev(sb))
        w.slot_base.copy_(dev(sbase))
        prev = r
    assert prev is not None
