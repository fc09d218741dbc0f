"""Capture-side index upkeep from captured graph views (typed, strided), bit for
bit against ordered fp32 sums on the host: the query accumulator with the
query-span row filter (llama-memory-kvmem.cpp:3417-3433, 3470-3483), the
mean-K sums (write_layer_mean_k, raw_kv_store.cpp:685-705) and the decode
running sum with its flush (kvmem_meank_*, llama-kvmem-stagein.cu:1066-1097;
write_layer_mean_sum, raw_kv_store.cpp:707-731)."""
import numpy as np
import pytest
import torch

from gpu_util import host
from kvmem_amd import api

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def _captured(rng, n_tok, heads, dims, dt, layout):
    """A [tokens][heads][dims] view of the given dtype: contiguous, or the
    [heads][tokens][dims] tensor ggml captures before a permute (strided), or
    every other dim of a wider tensor (nb0 of two elements)."""
    x = torch.from_numpy((rng.standard_normal((n_tok, heads, dims)) * 3).astype(np.float32)).to(DT[dt]).cuda()
    if layout == "contiguous":
        return x
    if layout == "heads_major":
        return x.permute(1, 0, 2).contiguous().permute(1, 0, 2)
    wide = torch.zeros((n_tok, heads, 2 * dims), dtype=DT[dt], device="cuda")
    wide[:, :, ::2] = x
    return wide[:, :, ::2]


def _f32_rows(v):
    return v.float().cpu().numpy().reshape(v.shape[0], -1)


def _ordered_sum(acc, rows):
    acc = acc.astype(np.float32).copy()
    for r in rows:
        acc = (acc + r).astype(np.float32)
    return acc


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("layout", ["contiguous", "heads_major", "strided_dim"])
def test_query_add_view(kvm_state, dt, layout):
    rng = np.random.default_rng(len(dt) * 7 + len(layout))
    n_head, D = 24, 256
    qa = api.QueryAcc(kvm_state, 2, n_head, D)
    qa.reset()
    q = _captured(rng, 9, n_head, D, dt, layout)
    keep = rng.random(9) < 0.6
    keep[0] = True
    qa.add_view(1, q, keep)
    qa.add_view(1, q[:3], None)
    rows = _f32_rows(q)
    want = _ordered_sum(np.zeros(n_head * D, np.float32), list(rows[keep]) + list(rows[:3]))
    got = host(qa.q_sum)
    assert np.array_equal(got[1].view(np.uint32), want.view(np.uint32))
    assert not got[0].any() and list(host(qa.q_count)) == [0, int(keep.sum()) + 3]


def test_query_add_view_more_rows_than_one_launch(kvm_state):
    rng = np.random.default_rng(5)
    qa = api.QueryAcc(kvm_state, 1, 2, 128)
    qa.reset()
    q = _captured(rng, 2100 + 37, 2, 128, "f16", "heads_major")
    keep = rng.random(q.shape[0]) < 0.5
    qa.add_view(0, q, keep)
    want = _ordered_sum(np.zeros(256, np.float32), _f32_rows(q)[keep])
    assert np.array_equal(host(qa.q_sum)[0].view(np.uint32), want.view(np.uint32))
    assert int(host(qa.q_count)[0]) == int(keep.sum())


@pytest.mark.parametrize("dt,layout", [("f16", "heads_major"), ("bf16", "strided_dim"), ("f32", "contiguous")])
def test_meank_add_view(kvm_state, dt, layout):
    """Prefill ubatches at positions 0.. and 300.. (the second continues the
    block the first left partly filled), as the capture hook hands them over."""
    rng = np.random.default_rng(11)
    H, D, bt = 4, 256, 128
    ix = api.MeanKIndex(kvm_state, 2, 8, H, D, bt)
    k1 = _captured(rng, 300, H, D, dt, layout)
    k2 = _captured(rng, 150, H, D, dt, layout)
    ix.add_view(1, 0, k1)
    ix.add_view(1, 300, k2)
    rows = np.concatenate([_f32_rows(k1), _f32_rows(k2)])
    got = host(ix.block_sums())[1]
    for b in range(4):
        n = min(bt, 450 - b * bt)
        want = _ordered_sum(np.zeros(H * D, np.float32), rows[b * bt:b * bt + n])
        assert np.array_equal(got[b].view(np.uint32), want.view(np.uint32)), b
    assert list(host(ix.mean_tokens)[1][:5]) == [128, 128, 128, 66, 0]
    assert list(host(ix.present)[:5]) == [1, 1, 1, 1, 0]


def test_meank_decode_running_sum_and_flush(kvm_state):
    """Accepted decode tokens go to the running sum (two commits, the second
    keeping 2 of 3 MTP tokens), which is flushed into a block the prompt left
    partly filled (its sum += the running sum, not a continued ordered sum) and,
    after a zero, into a fresh block (its sum = the running sum)."""
    rng = np.random.default_rng(13)
    H, D, bt = 4, 256, 128
    ix = api.MeanKIndex(kvm_state, 1, 4, H, D, bt)
    prompt = _captured(rng, 200, H, D, "f32", "contiguous")
    ix.add_view(0, 0, prompt)                        # block 1 holds positions 128..199
    ix.acc_zero(0)
    d1 = _captured(rng, 2, H, D, "bf16", "heads_major")
    d2 = _captured(rng, 3, H, D, "bf16", "heads_major")
    ix.acc_add(0, d1, 0, 2)
    ix.acc_add(0, d2, 0, 2)
    ix.acc_flush(0, 200, 4)                          # positions 200..203 of block 1
    ix.acc_zero(0)
    d3 = _captured(rng, 5, H, D, "f16", "strided_dim")
    ix.acc_add(0, d3, 1, 4)
    ix.acc_flush(0, 256, 4)                          # positions 256..259: block 2 starts
    rows = _f32_rows(prompt)
    block1 = _ordered_sum(np.zeros(H * D, np.float32), rows[128:200])
    acc1 = _ordered_sum(np.zeros(H * D, np.float32), list(_f32_rows(d1)) + list(_f32_rows(d2)[:2]))
    acc2 = _ordered_sum(np.zeros(H * D, np.float32), _f32_rows(d3)[1:5])
    got = host(ix.block_sums())[0]
    assert np.array_equal(got[1].view(np.uint32), (block1 + acc1).astype(np.float32).view(np.uint32))
    assert np.array_equal(got[2].view(np.uint32), acc2.view(np.uint32))
    assert np.array_equal(host(ix.acc)[0].view(np.uint32), acc2.view(np.uint32))     # flush keeps it
    assert list(host(ix.mean_tokens)[0]) == [128, 76, 4, 0]


def test_view_shape_is_checked(kvm_state):
    qa = api.QueryAcc(kvm_state, 1, 8, 128)
    with pytest.raises(api.L.KvmError):
        qa.add_view(0, torch.zeros((2, 4, 128), dtype=torch.float16, device="cuda"))
    ix = api.MeanKIndex(kvm_state, 1, 4, 2, 128, 128)
    k = torch.zeros((2, 2, 128), dtype=torch.float32, device="cuda")
    v = api.view(k)
    v.type = api.L.T_Q8_0                            # a quantised view is not a captured output
    assert kvm_state.lib.kvm_meank_add_view(kvm_state.h, api.C.byref(ix.c), 0, 0, api.C.byref(v)) == api.L.KVM_EUNSUPPORTED
