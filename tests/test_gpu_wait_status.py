"""In-launch waits that give up are reported through the ABI.

kvm_state_set_wait_polls(st, 0) makes every in-launch wait (split merge,
selected plan, stage-in barriers) give up
at once, without a look at its flag, so every kernel still runs to its end.
kvm_state_status then hands back the KVM_WAIT_* bits (and kvm_state_sync
returns KVM_ETIMEOUT), clears them and resets the state's sync words; with the
default bound restored, the next calls equal the separate, unforced calls
bit for bit.  The reference's contract is the same: a stage-in that fails
returns false and the caller falls back (llama-kvmem-stagein.cu:93-99,
llama-memory-kvmem.cpp:4032-4038)."""
import numpy as np
import pytest
import torch

from gpu_util import dev, host, rand_rows
from kvmem_amd import api, _lib as L
import test_gpu_decode_step as T

pytestmark = pytest.mark.gpu

H, G, D, BT = T.H, T.G, T.D, T.BT
ALL_STEP = L.WAIT_MERGE | L.WAIT_PLAN


def _step(st, ln):
    d = T._step_dict(ln)
    api.decode_step(st, d["index"], d["query"], d["n_blocks"], d["n_tokens"], d["budget_blocks"], 1, 0,
                    d["window"], d["sel"], d["history"], d["q"], d["q_pos"], H * G, D ** -0.5, 64, 1e7,
                    out=d["out"])


def _fresh_query(ln):
    ln["q"] = dev(ln["rng"].standard_normal((ln["n_tok_q"], H * G, D)).astype(np.float32)).to(torch.bfloat16)
    ln["out"] = torch.zeros((ln["n_tok_q"], H * G, D), dtype=torch.float32, device="cuda")


def test_forced_give_up_in_the_decode_step_is_reported_and_recovers():
    st = api.State(0)
    try:
        ln = T._lane(st, 0x57A7, 40, 12, 16)
        _fresh_query(ln)
        _step(st, ln)                               # the first plan stages the whole selection
        T._reference_step(st, ln)                   # the separate calls on the second window, in step
        assert st.status() == 0
        before = {k: getattr(ln["a"]["window"], k).clone() for k in ("cell_pos", "slot_block", "slot_base")}
        # a new query (another turn), every wait forced to give up
        ln["qa"].q_sum.copy_(dev((ln["rng"].standard_normal((1, H * G * D)) * 2.0).astype(np.float32)))
        _fresh_query(ln)
        st.set_wait_polls(0)
        _step(st, ln)
        bits = st.status()
        assert bits == ALL_STEP, bits
        assert st.status() == 0                     # reported once, then cleared
        res = ln["a"]["sel"].result()
        assert res["status"] == 0 and len(res["stage_slots"]) > 0, res   # a plan was selected ...
        for k, v in before.items():                 # ... and not staged
            assert torch.equal(getattr(ln["a"]["window"], k), v), k
        # the default bound again: the step equals the separate calls
        st.set_wait_polls(L.WAIT_POLLS_DEFAULT)
        _step(st, ln)
        assert st.status() == 0
        ref = T._reference_step(st, ln)
        st.sync()
        T._compare(ln, ref, False, "after recovery")
    finally:
        st.close()


def test_sync_returns_timeout_for_a_forced_merge():
    st = api.State(0)
    try:
        rng = np.random.default_rng(0x71)
        kr, vr = rand_rows(rng, 512, H, D, L.T_Q8_0, L.T_Q4_0)
        w = api.KVWindow(st, 512, H, D, BT)
        w.import_rows(0, dev(kr), dev(vr), dev(np.arange(512, dtype=np.int32)))
        q = dev(rng.standard_normal((2, H * G, D)).astype(np.float32))
        qp = dev(np.array([300, 511], np.int32))
        good = api.fa_decode(st, w, q, qp, H * G, D ** -0.5)
        st.sync()
        st.set_wait_polls(0)
        api.fa_decode(st, w, q, qp, H * G, D ** -0.5)
        with pytest.raises(L.KvmError) as e:
            st.sync()
        assert e.value.code == L.KVM_ETIMEOUT and "split merge" in str(e.value)
        st.sync()                                   # cleared
        st.set_wait_polls(L.WAIT_POLLS_DEFAULT)
        again = api.fa_decode(st, w, q, qp, H * G, D ** -0.5)
        st.sync()
        assert torch.equal(good, again)
    finally:
        st.close()


def test_forced_stage_barrier_empties_the_items_and_recovers():
    """A plan that moves resident blocks within a shadowed window has a gather
    barrier; forced to give up, the stage-in empties the plan's items (info[3]
    bit 16, KVM_WAIT_STAGE), and the same plan staged again with the default
    bound equals a fresh stage-in into a window without a shadow."""
    st = api.State(0)
    try:
        n_blocks, budget = 24, 8
        rng = np.random.default_rng(0x5B)
        kr, vr = rand_rows(rng, n_blocks * BT, H, D, L.T_Q8_0, L.T_Q4_0)
        hist = api.History(kr, vr)
        nt = dev(np.full(n_blocks, BT, np.int32))
        wa = api.KVWindow(st, budget * BT, H, D, BT, shadow=True)
        wb = api.KVWindow(st, budget * BT, H, D, BT)
        sa, sb = api.SelectionBuffers(st, n_blocks, budget), api.SelectionBuffers(st, n_blocks, budget)

        def scores(chosen):
            s = np.zeros(n_blocks)
            s[list(chosen)] = 1.0 + np.arange(len(chosen))
            return dev(s)
        first = [3, 5, 8, 11, 14, 17, 20]            # plus the sink block 0
        api.select_topk(st, scores(first), nt, budget, 1, 0, None, wa, sa)
        api.stagein_selection(st, hist, wa, sa, 64, 1e7)
        assert st.status() == 0
        second = [5, 8, 11, 14, 17, 20, 22]          # block 3 leaves: every later block moves a slot
        api.select_topk(st, scores(second), nt, budget, 1, 0, None, wa, sa)
        st.sync()
        assert (host(sa.stage_src)[:int(host(sa.info)[2])] >= 0).any(), "the plan moves blocks"
        st.set_wait_polls(0)
        api.stagein_selection(st, hist, wa, sa, 64, 1e7)
        assert st.status() == L.WAIT_STAGE
        assert host(sa.info)[3] & 16
        st.set_wait_polls(L.WAIT_POLLS_DEFAULT)
        api.select_topk(st, scores(second), nt, budget, 1, 0, None, wa, sa)
        api.stagein_selection(st, hist, wa, sa, 64, 1e7)
        api.select_topk(st, scores(second), nt, budget, 1, 0, None, wb, sb)
        api.stagein_selection(st, hist, wb, sb, 64, 1e7)
        assert st.status() == 0
        n_used = budget * BT
        for name in ("cell_pos", "slot_block", "slot_base"):
            assert torch.equal(getattr(wa, name), getattr(wb, name)), name
        ka, va = wa.export_rows(0, n_used)
        kb, vb = wb.export_rows(0, n_used)
        assert torch.equal(ka, kb) and torch.equal(va, vb)
    finally:
        st.close()
