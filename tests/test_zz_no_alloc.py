"""kvm_fa_decode_noalloc (split partials in the library's fixed per-device
scratch array, no allocation) against kvm_fa_decode (partials in the state's
workspace) through the C ABI: two calls in a row, the second with a smaller
window and fewer query tokens, each equal to the allocating entry point's
output and within the attention tolerance of the ggml-semantics oracle."""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import check_attention, dev, host, rand_rows
from kvmem_amd import api, _lib as L

pytestmark = pytest.mark.gpu


def _case(st, seed, n_cells, T, H=4, G=6, D=256):
    rng = np.random.default_rng(seed)
    w = api.KVWindow(st, n_cells, H, D, 128)
    kr, vr = rand_rows(rng, n_cells, H, D, L.T_Q8_0, L.T_Q4_0)
    cp = np.arange(n_cells, dtype=np.int32)
    cp[rng.choice(n_cells, n_cells // 50, replace=False)] = -1
    w.import_rows(0, dev(kr), dev(vr), dev(cp))
    qt = torch.from_numpy(rng.standard_normal((T, H * G, D)).astype(np.float32)).to(torch.bfloat16)
    qp = np.arange(n_cells - T, n_cells, dtype=np.int32)
    return w, kr, vr, cp, qt, qp


def test_fa_decode_noalloc_matches_fa_decode(kvm_state):
    st = kvm_state
    H, G, D = 4, 6, 256
    scale = D ** -0.5
    for seed, n_cells, T in ((1, 32768, 4), (2, 4096, 1)):          # second call: smaller input
        w, kr, vr, cp, qt, qp = _case(st, seed, n_cells, T)
        q, qpd = qt.cuda(), dev(qp)
        want = torch.empty((T, H * G, D), dtype=torch.float32, device="cuda")
        got = torch.full((T, H * G, D), float("nan"), dtype=torch.float32, device="cuda")
        st.check(st.lib.kvm_fa_decode(st.h, C.byref(w.c), C.c_void_p(q.data_ptr()), L.T_BF16,
                                      C.c_void_p(qpd.data_ptr()), T, H * G, scale, C.c_void_p(want.data_ptr())))
        st.check(st.lib.kvm_fa_decode_noalloc(st.h, C.byref(w.c), C.c_void_p(q.data_ptr()), L.T_BF16,
                                              C.c_void_p(qpd.data_ptr()), T, H * G, scale,
                                              C.c_void_p(got.data_ptr())))
        got, want = host(got), host(want)
        assert np.array_equal(got, want), (n_cells, T, float(np.abs(got - want).max()))
        ref = O.fa_ggml(L.T_Q8_0, L.T_Q4_0, qt.float().numpy(), kr, vr, cp, qp, H * G, H, D, scale)
        check_attention(got, ref)

