"""kvm_stagein_fa_decode(_lanes): a decode step's stage-in and attention in one
launch (the attention's workgroups stage the plan, then meet at an in-launch
barrier) against kvm_stagein_selection + kvm_fa_decode on a second window:
equal windows byte for byte and equal attention outputs (bit for bit where the
launches split the keys alike: the same attention code reads the same bytes)."""
import ctypes as C

import numpy as np
import pytest
import torch

from gpu_util import check_attention, dev, host, rand_rows
from kvmem_amd import api, _lib as L
import oracle as O

pytestmark = pytest.mark.gpu

H, G, D, BT = 4, 6, 256, 128
K_ROW, V_ROW = H * D // 32 * 34, H * D // 32 * 18


def _lane(st, seed, n_blocks, budget, slots, n_tok_q=4, shadow=True):
    rng = np.random.default_rng(seed)
    n_hist = n_blocks * BT - 40                         # the last block partly filled
    kr, vr = rand_rows(rng, n_hist, H, D, L.T_Q8_0, L.T_Q4_0)
    ix = api.MeanKIndex(st, 1, n_blocks, H, D, BT)
    ix.add(0, 0, dev(rng.standard_normal((n_hist, H * D)).astype(np.float32)))
    qa = api.QueryAcc(st, 1, H * G, D)
    qa.reset()
    qa.add(0, dev(rng.standard_normal((4, H * G * D)).astype(np.float32)))
    nt = dev(np.array([min(BT, n_hist - b * BT) for b in range(n_blocks)], np.int32))
    mk = lambda sh: dict(window=api.KVWindow(st, slots * BT, H, D, BT, shadow=sh),
                         sel=api.SelectionBuffers(st, n_blocks, budget), history=api.History(kr, vr))
    return dict(rng=rng, kr=kr, vr=vr, ix=ix, qa=qa, nt=nt, n_blocks=n_blocks, budget=budget, n_hist=n_hist,
                q_pos=dev(np.arange(budget * BT - n_tok_q, budget * BT, dtype=np.int32)), n_tok_q=n_tok_q,
                a=mk(shadow), b=mk(False))


def _resident_full(w, nt_host):
    return sorted({int(b) for b in host(w.slot_block) if 0 <= int(b) < len(nt_host) and nt_host[int(b)] == BT})


def _set_rows(hist, blocks, rows_k, rows_v):
    torch.cuda.synchronize()
    k = hist.kbuf.u8.reshape(hist.n_tokens, K_ROW)
    v = hist.vbuf.u8.reshape(hist.n_tokens, V_ROW)
    for b in blocks:
        k[b * BT:(b + 1) * BT] = rows_k(b)
        v[b * BT:(b + 1) * BT] = rows_v(b)


@pytest.mark.parametrize("n_lanes", [1, 3])
def test_stagein_fa_decode_matches_two_calls(kvm_state, n_lanes):
    """Queries drift over six steps, so plans restage and move blocks within
    windows that carry a K shadow (host rows of the blocks a window holds are
    poisoned while its step runs).  Per lane and step: equal selections, equal
    windows, and outputs bit-equal to kvm_fa_decode's for one lane (the same
    key splits), within the attention tolerance for three (other splits); one
    output also against the oracle."""
    st = kvm_state
    lanes = [_lane(st, 0x5C00 + i, 40 + 6 * i, 12, 16) for i in range(n_lanes)]
    moved = 0
    for step in range(6):
        fused = []
        for ln in lanes:
            if step:
                ln["qa"].q_sum.add_(dev((ln["rng"].standard_normal((1, H * G * D)) * 0.6).astype(np.float32)))
            ln["q"] = dev(ln["rng"].standard_normal((ln["n_tok_q"], H * G, D)).astype(np.float32)).to(torch.bfloat16)
            for side in ("a", "b"):
                api.score_topk(st, ln["ix"], ln["qa"], ln["n_blocks"], ln["nt"], ln["budget"], 1, 0, None,
                               ln[side]["window"], ln[side]["sel"])
            ln["out"] = torch.empty((ln["n_tok_q"], H * G, D), dtype=torch.float32, device="cuda")
            fused.append(dict(history=ln["a"]["history"], sel=ln["a"]["sel"], window=ln["a"]["window"], q=ln["q"],
                              q_pos=ln["q_pos"], out=ln["out"]))
        # poison the host rows of every full block the shadow windows hold
        nts = [host(ln["nt"]) for ln in lanes]
        held = [_resident_full(ln["a"]["window"], nt) for ln, nt in zip(lanes, nts)]
        for ln, hb in zip(lanes, held):
            _set_rows(ln["a"]["history"], hb, lambda b, r=ln["rng"]: r.integers(0, 256, (BT, K_ROW), dtype=np.uint8),
                      lambda b, r=ln["rng"]: r.integers(0, 256, (BT, V_ROW), dtype=np.uint8))
        if n_lanes == 1:
            f = fused[0]
            api.stagein_fa_decode(st, f["history"], f["sel"], f["window"], f["q"], f["q_pos"], H * G, D ** -0.5,
                                  64, 1e7, out=f["out"])
        else:
            api.prepare_stagein_fa_decode_lanes(st, fused, H * G, D ** -0.5, 64, 1e7)()
        for ln, hb in zip(lanes, held):
            _set_rows(ln["a"]["history"], hb, lambda b, ln=ln: ln["kr"][b * BT:(b + 1) * BT],
                      lambda b, ln=ln: ln["vr"][b * BT:(b + 1) * BT])
        for i, ln in enumerate(lanes):
            api.stagein_selection(st, ln["b"]["history"], ln["b"]["window"], ln["b"]["sel"], 64, 1e7)
            ref = api.fa_decode(st, ln["b"]["window"], ln["q"], ln["q_pos"], H * G, D ** -0.5)
            torch.cuda.synchronize()
            ra, rb = ln["a"]["sel"].result(), ln["b"]["sel"].result()
            assert ra["status"] == rb["status"] == 0, (step, i)
            for key in ("ids", "to_base", "stage_slots"):
                assert np.array_equal(ra[key], rb[key]), (step, i, key)
            for name in ("k", "v", "cell_pos", "slot_block", "slot_base"):
                assert torch.equal(getattr(ln["a"]["window"], name), getattr(ln["b"]["window"], name)), (step, i, name)
            if n_lanes == 1:
                assert torch.equal(ln["out"], ref), (step, i)
            else:
                # the lanes' launch splits the keys differently (its grid is capped to
                # what the CUs hold at once): the same sums in another order
                check_attention(host(ln["out"]), host(ref))
            moved += int((ra["stage_src"] >= 0).sum())
    assert moved > 0
    # the oracle on the last step of lane 0 (ggml semantics over the window's bytes)
    ln = lanes[0]
    w = ln["b"]["window"]
    ek, ev = w.export_rows(0, w.n_cells)
    ref = O.fa_ggml(O.T_Q8_0, O.T_Q4_0, ln["q"].float().cpu().numpy(), host(ek), host(ev), host(w.cell_pos),
                    host(ln["q_pos"]), H * G, H, D, D ** -0.5)
    check_attention(host(ln["out"]), ref)


def test_stagein_fa_decode_empty_plan_and_bad_arguments(kvm_state):
    """The steady state (nothing to stage) gives kvm_fa_decode's output; a lane
    that stages one window and attends another is refused."""
    st = kvm_state
    ln = _lane(st, 0x5C10, 24, 8, 10)
    q = dev(ln["rng"].standard_normal((4, H * G, D)).astype(np.float32))
    w, sel, hist = ln["a"]["window"], ln["a"]["sel"], ln["a"]["history"]
    for _ in range(2):
        api.score_topk(st, ln["ix"], ln["qa"], ln["n_blocks"], ln["nt"], ln["budget"], 1, 0, None, w, sel)
        out = api.stagein_fa_decode(st, hist, sel, w, q, ln["q_pos"], H * G, D ** -0.5, 64, 1e7)
    assert len(sel.result()["stage_slots"]) == 0
    assert torch.equal(out, api.fa_decode(st, w, q, ln["q_pos"], H * G, D ** -0.5))
    # lane 0 stages window `w` but attends the reference window: refused
    sg = (L.StageinLane * 1)(L.StageinLane(C.pointer(hist.c), C.pointer(w.c), C.pointer(sel.c)))
    fl = (L.Lane * 1)(L.Lane(C.pointer(ln["b"]["window"].c), q.data_ptr(), ln["q_pos"].data_ptr(), out.data_ptr(), 4))
    rc = st.lib.kvm_stagein_fa_decode_lanes(st.h, sg, fl, 1, C.byref(L.RopeParams(64, 1e7, 1.0, -1)), L.T_F32,
                                            H * G, D ** -0.5)
    assert rc == L.KVM_EINVAL
