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
