"""Shared helpers of the GPU parity tests (inputs are built on the CPU and the
oracle computes the expected results)."""
import numpy as np
import torch

import oracle as O
from kvmem_amd import api, _lib as L


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.detach().cpu().numpy()


def rand_rows(rng, n_cells, n_head_kv, d, kt, vt, scale=1.0):
    """Random K / V rows in ggml cache format (and their fp32 sources)."""
    k = (rng.standard_normal((n_cells, n_head_kv * d)) * scale).astype(np.float32)
    v = rng.standard_normal((n_cells, n_head_kv * d)).astype(np.float32)

    def enc(ty, x):
        if ty == L.T_F16:
            return x.astype(np.float16).view(np.uint8).reshape(n_cells, -1)
        return O.quant(ty, x.reshape(-1)).reshape(n_cells, -1)
    return enc(kt, k), enc(vt, v)


def check_attention(out, ref, atol=2e-3, rtol=1e-3):
    """max |out - ref| <= atol and <= rtol * max |ref|."""
    err = float(np.abs(out - ref).max())
    scale = float(np.abs(ref).max())
    assert err <= atol, (err, scale)
    assert err <= rtol * scale, (err, scale)
    return err, scale


def golden_snapshot(name):
    """A raw-store snapshot the reference's RawKvStore wrote (tests/golden/, made by
    make_snapshots.py on the CPU): (snapshot bytes, case metadata, the K rows, V
    rows and fp32 K the store was filled with, regenerated from the seed and
    checked against the digest recorded with the fixture)."""
    import gzip
    import json
    import os
    import make_snapshots as MS
    here = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    with open(os.path.join(here, "snapshots.json")) as f:
        meta = json.load(f)[name]
    with open(os.path.join(here, name + ".bin.gz"), "rb") as f:
        snap = gzip.decompress(f.read())
    kr, vr, kf = MS.case_inputs(meta["seed"], meta["n_head_kv"], meta["head_dim"], meta["block_tokens"],
                                meta["n_blocks"], meta["short"], meta["random_rows"])
    assert MS.digest(kr, vr, kf) == meta["inputs_sha256"], "regenerated inputs differ from the fixture's"
    return snap, meta, kr, vr, kf
