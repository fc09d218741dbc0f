"""A decode step (score + top-k + stage-in + FA decode) captured as one HIP
graph: every replay, with eager work and synchronisation between the
replays, gives exactly the eager step's results."""
import numpy as np
import pytest
import torch

from gpu_util import dev, rand_rows
from kvmem_amd import api, _lib as L

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("fused", [False, True])
def test_decode_step_graph_replays_equal_eager(kvm_state, fused):
    """fused: retrieval and stage-in in kvm_score_topk_stagein (the top-k
    workgroup stages the plan) instead of kvm_score_topk + kvm_stagein_selection."""
    st = kvm_state
    rng = np.random.default_rng(21)
    H, G, D, BT, n_blocks = 4, 6, 256, 128, 64
    n_hist = n_blocks * BT
    kr, vr = rand_rows(rng, n_hist, H, D, L.T_Q8_0, L.T_Q4_0)
    hist = api.History(kr, vr)
    ix = api.MeanKIndex(st, 1, n_blocks, H, D, BT)
    ix.add(0, 0, dev(rng.standard_normal((n_hist, H * D)).astype(np.float32)))
    qa = api.QueryAcc(st, 1, H * G, D)
    qa.reset()
    qa.add(0, dev(rng.standard_normal((4, H * G * D)).astype(np.float32)))
    n_tokens = dev(np.full(n_blocks, BT, np.int32))
    w = api.KVWindow(st, 16 * BT, H, D, BT)
    sel = api.SelectionBuffers(st, n_blocks, 8)
    q = dev(rng.standard_normal((4, H * G, D)).astype(np.float32))
    q_pos = dev(np.arange(8 * BT - 4, 8 * BT, dtype=np.int32))
    out = torch.empty((4, H * G, D), dtype=torch.float32, device="cuda")
    score = api.prepare_score_topk(st, ix, qa, n_blocks, n_tokens, 8, 1, 0, w, sel)
    stagein = api.prepare_stagein(st, hist, w, sel, 64, 1e7)
    fa = api.prepare_fa_decode(st, w, q, q_pos, H * G, D ** -0.5, out)

    fused_retrieval = api.prepare_score_topk_stagein(st, ix, qa, n_blocks, n_tokens, 8, 1, 0, w, sel, hist, 64, 1e7)

    def step():
        if fused:
            fused_retrieval()
        else:
            score()
            stagein()
        fa()

    step()                                   # stages the selection, sizes the workspace
    torch.cuda.synchronize()
    step()                                   # steady state: nothing left to stage
    torch.cuda.synchronize()
    want_out, want_ids = out.clone(), sel.ids.clone()
    want_k = w.k.clone()
    g = st.capture(step)
    for r in range(4):
        out.zero_()
        sel.ids.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want_out), r
        assert torch.equal(sel.ids, want_ids), r
        assert torch.equal(w.k, want_k), r
        step()                               # eager work between the replays
        torch.cuda.synchronize()
        assert torch.equal(out, want_out), r


@pytest.mark.parametrize("mode", ["retrieval_stagein", "staged", "step"])
def test_back_to_back_replays_follow_changing_inputs(kvm_state, monkeypatch, mode):
    """Replays of one captured decode step with nothing of the library's in
    between, while the inputs change: the query accumulator drifts (so plans
    restage and move blocks within a window with a K shadow, through the
    stage-in's in-launch barrier) and the attention query changes every
    replay.  Each replay's window equals an eager retrieval + stage-in of the
    same plans into a second window, and each replay's attention output equals
    an eager attention over the replay's window: the launches' in-launch
    flags take their epochs from the device, not from the captured arguments.
    mode: kvm_score_topk_stagein + kvm_fa_decode ("retrieval_stagein"),
    kvm_score_topk + kvm_stagein_fa_decode (the attention launch stages the
    plan, "staged"), or kvm_score_topk_stagein_fa_decode (the attention launch
    also selects, "step"; both attention paths take 32 key splits)."""
    monkeypatch.setenv("KVM_FA_SPLITS", "32")
    st = kvm_state
    rng = np.random.default_rng(23)
    H, G, D, BT, n_blocks, budget = 4, 6, 256, 128, 48, 12
    n_hist = n_blocks * BT
    kr, vr = rand_rows(rng, n_hist, H, D, L.T_Q8_0, L.T_Q4_0)
    hist = api.History(kr, vr)
    ix = api.MeanKIndex(st, 1, n_blocks, H, D, BT)
    ix.add(0, 0, dev(rng.standard_normal((n_hist, H * D)).astype(np.float32)))
    qa = api.QueryAcc(st, 1, H * G, D)
    qa.reset()
    qa.add(0, dev(rng.standard_normal((4, H * G * D)).astype(np.float32)))
    n_tokens = dev(np.full(n_blocks, BT, np.int32))
    w = api.KVWindow(st, 16 * BT, H, D, BT, shadow=True)
    sel = api.SelectionBuffers(st, n_blocks, budget)
    wr = api.KVWindow(st, 16 * BT, H, D, BT)
    selr = api.SelectionBuffers(st, n_blocks, budget)
    q = dev(rng.standard_normal((4, H * G, D)).astype(np.float32))
    q_pos = dev(np.arange(budget * BT - 4, budget * BT, dtype=np.int32))
    out = torch.empty((4, H * G, D), dtype=torch.float32, device="cuda")
    if mode == "staged":
        retrieval = api.prepare_score_topk(st, ix, qa, n_blocks, n_tokens, budget, 1, 0, w, sel)
        fa = api.prepare_stagein_fa_decode(st, hist, sel, w, q, q_pos, H * G, D ** -0.5, out, 64, 1e7)
    elif mode == "step":
        retrieval = api.prepare_decode_step(st, ix, qa, n_blocks, n_tokens, budget, 1, 0, w, sel, hist, q, q_pos,
                                            H * G, D ** -0.5, out, 64, 1e7)
        fa = lambda: None
    else:
        retrieval = api.prepare_score_topk_stagein(st, ix, qa, n_blocks, n_tokens, budget, 1, 0, w, sel, hist, 64,
                                                   1e7)
        fa = api.prepare_fa_decode(st, w, q, q_pos, H * G, D ** -0.5, out)

    def step():
        retrieval()
        fa()

    step()
    api.score_topk(st, ix, qa, n_blocks, n_tokens, budget, 1, 0, None, wr, selr)
    api.stagein_selection(st, hist, wr, selr, 64, 1e7)
    torch.cuda.synchronize()
    g = st.capture(step)
    n_rep = 6
    qs = [dev(rng.standard_normal((4, H * G, D)).astype(np.float32)) for _ in range(n_rep)]
    drift = [dev((rng.standard_normal((1, H * G * D)) * 0.6).astype(np.float32)) for _ in range(n_rep)]
    outs, moved = [], 0
    for r in range(n_rep):
        # the inputs change on the replay stream's side of the graph: torch work only
        q.copy_(qs[r])
        qa.q_sum.add_(drift[r].view_as(qa.q_sum))
        g.replay()
        outs.append(out.clone())
        # the same plan eagerly, into the reference window (read after the replay)
        api.score_topk(st, ix, qa, n_blocks, n_tokens, budget, 1, 0, None, wr, selr)
        api.stagein_selection(st, hist, wr, selr, 64, 1e7)
        torch.cuda.synchronize()
        ra, rb = sel.result(), selr.result()
        assert np.array_equal(ra["ids"], rb["ids"]) and np.array_equal(ra["stage_slots"], rb["stage_slots"]), r
        for name in ("k", "v", "cell_pos", "slot_block", "slot_base"):
            assert torch.equal(getattr(w, name), getattr(wr, name)), (r, name)
        moved += int((ra["stage_src"] >= 0).sum())
        # eager attention over the same window and query
        ref = api.fa_decode(st, w, qs[r], q_pos, H * G, D ** -0.5)
        torch.cuda.synchronize()
        assert torch.equal(outs[r], ref), r
    assert moved > 0
    # replays back to back with nothing of the library's between them: only the
    # query changes (the plan stays put), every output still matches its query
    outs = []
    for r in range(n_rep):
        q.copy_(qs[r])
        g.replay()
        outs.append(out.clone())
    torch.cuda.synchronize()
    for r in range(n_rep):
        assert torch.equal(outs[r], api.fa_decode(st, w, qs[r], q_pos, H * G, D ** -0.5)), r
