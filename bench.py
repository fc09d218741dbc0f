"""Benchmark: KVMem decode attention + retrieval on one MI355X.

Workload (256K history, 32K window): one attention layer with 24 query heads,
4 kv heads (GQA 6), head_dim 256; a 262,144-token history in 128-token blocks
held in pinned host memory as raw q8_0 K / q4_0 V rows plus a device mean-K
index; a 32,768-cell GPU window (16,384 retrieved cells incl. the sink block +
16,384 generation cells); 4 bf16 query tokens (MTP verify) with 16 planted
relevant blocks.  Synthetic N(0,1) data from a fixed seed.

One step = score_retrieval over 2,048 blocks -> top-k + window layout + stage
plan -> stage-in of the changed slots (none in steady state) -> quantised
flash-attention decode over the full window.  Steps cycle through 8 layer
replicas of window + index (504 MB), more than the 256 MB Infinity Cache, so
every step streams its window and index from HBM as a multi-layer model does.

Prints one JSON line (time per decode step in microseconds, lower is better).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "kvmem-llama.cpp_amd"))

HIST_TOKENS = 262144
BT = 128
H_KV, G, D = 4, 6, 256
N_HEAD = H_KV * G
WINDOW = 32768
RETRIEVED = 16384
MTP = 4
PLANTED = 16
N_ROT, FREQ_BASE = 64, 1e7
HBM_PEAK_GBPS = 8000.0

K_ROW = H_KV * D // 32 * 34          # 1088 B per token (q8_0)
V_ROW = H_KV * D // 32 * 18          # 576 B per token (q4_0)
FA_KV_BYTES = WINDOW * (K_ROW + V_ROW)                        # 54,525,952
QO_BYTES = MTP * N_HEAD * D * 2 + MTP * N_HEAD * D * 4       # bf16 Q + fp32 O = 147,456
SCORE_BYTES = (HIST_TOKENS // BT) * H_KV * D * 4             # mean-K index, 8,388,608
TOPK_BYTES = (HIST_TOKENS // BT) * 8                         # scores, 16 KiB
STEP_BYTES = SCORE_BYTES + TOPK_BYTES + FA_KV_BYTES + QO_BYTES


def log(msg):
    print(msg, file=sys.stderr, flush=True)


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "fa_decode_256k_32k_hbm_traffic.txt")


def measured_traffic():
    """HBM bytes per flash-attention launch (split + combine) from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary of this workload, or None."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def build_workload(st, api, L, torch, np, n_rep, seed=0xC0FFEE02, hist_tokens=HIST_TOKENS, mtp=MTP):
    from kvmem_amd import workload as W
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    n_blocks = hist_tokens // BT
    # pinned host history: raw (pre-RoPE) K as q8_0 rows, V as q4_0 rows
    kbuf = api.HostBuffer(hist_tokens * K_ROW)
    vbuf = api.HostBuffer(hist_tokens * V_ROW)
    ix0 = api.MeanKIndex(st, 1, n_blocks, H_KV, D, BT)
    chunk = 16384
    for t0 in range(0, hist_tokens, chunk):
        k = torch.randn((chunk, H_KV * D), generator=gen, device=dev)
        v = torch.randn((chunk, H_KV * D), generator=gen, device=dev)
        ix0.add(0, t0, k)
        kq = api.quantize_rows(st, L.T_Q8_0, k)
        vq = api.quantize_rows(st, L.T_Q4_0, v)
        torch.from_numpy(kbuf.u8[t0 * K_ROW:(t0 + chunk) * K_ROW]).copy_(kq.view(-1).cpu())
        torch.from_numpy(vbuf.u8[t0 * V_ROW:(t0 + chunk) * V_ROW]).copy_(vq.view(-1).cpu())
    hist = api.History.__new__(api.History)
    hist.kbuf, hist.vbuf, hist.n_tokens = kbuf, vbuf, hist_tokens
    hist.c = L.History(kbuf.ptr, vbuf.ptr, hist_tokens)
    # query: 4 tokens whose pre-RoPE rows point at 16 planted blocks
    planted = W.distinct_ids(seed, 0, PLANTED, 1, n_blocks)
    means = ix0.block_sums()[0][torch.from_numpy(planted).to(dev)].T / float(BT)   # [H*D, 16]
    qsum_kv = means.sum(1).view(H_KV, D)
    qrows = qsum_kv.repeat_interleave(G, 0).reshape(1, N_HEAD * D).repeat(mtp, 1)
    qrows = qrows + 0.1 * torch.randn(qrows.shape, generator=gen, device=dev)
    # the accumulator carries the scorer's query terms, kept current by add
    qa = api.QueryAcc(st, 1, N_HEAD, D, n_head_kv=H_KV)
    qa.reset()
    qa.add(0, qrows)
    n_tokens = torch.full((n_blocks,), BT, dtype=torch.int32, device=dev)
    # generation cells: synthetic decoded tokens at window positions 16384..32767
    ng = WINDOW - RETRIEVED
    gk = api.quantize_rows(st, L.T_Q8_0, torch.randn((ng, H_KV * D), generator=gen, device=dev))
    gv = api.quantize_rows(st, L.T_Q4_0, torch.randn((ng, H_KV * D), generator=gen, device=dev))
    gpos = torch.arange(RETRIEVED, WINDOW, dtype=torch.int32, device=dev)
    reps = []
    for r in range(n_rep):
        # the index carries the blocks' score term nk (formed after the copies)
        ix = api.MeanKIndex(st, 1, n_blocks, H_KV, D, BT, norms=True)
        ix.k_sum.copy_(ix0.k_sum)
        ix.mean_tokens.copy_(ix0.mean_tokens)
        ix.present.copy_(ix0.present)
        ix.refresh()
        w = api.KVWindow(st, WINDOW, H_KV, D, BT)
        sel = api.SelectionBuffers(st, n_blocks, RETRIEVED // BT)
        api.score_topk(st, ix, qa, n_blocks, n_tokens, RETRIEVED // BT, 1, 0, None, w, sel)
        api.stagein_selection(st, hist, w, sel, N_ROT, FREQ_BASE)
        w.import_rows(RETRIEVED, gk, gv, gpos)
        reps.append((ix, w, sel))
    torch.cuda.synchronize()
    res = reps[0][2].result()
    assert res["status"] == 0 and len(res["ids"]) == RETRIEVED // BT, res
    assert set(planted.tolist()) <= set(res["ids"].tolist()), "planted blocks not retrieved"
    q = torch.randn((mtp, N_HEAD, D), generator=gen, device=dev).to(torch.bfloat16)
    q_pos = torch.arange(WINDOW - mtp, WINDOW, dtype=torch.int32, device=dev)
    return dict(hist=hist, qa=qa, n_tokens=n_tokens, reps=reps, q=q, q_pos=q_pos, planted=planted,
                ids=res["ids"], hist_tokens=hist_tokens)


def prepare_decode(st, api, wl, out):
    """A decode step for every layer replica, marshalled once, as
    (step, retrieval, attention): the step is one call in two launches
    (kvm_score_topk_stagein_fa_decode: the scoring grid, then one launch whose
    selector workgroup picks the blocks while the attention workgroups attend,
    staging the plan and attending again when it stages anything); retrieval
    (kvm_score_topk: scoring grid + top-k workgroup) and attention
    (kvm_stagein_fa_decode: the attention's workgroups stage the plan, then
    attend) are the same step as three launches."""
    n_blocks = wl["hist_tokens"] // BT
    return [(api.prepare_decode_step(st, ix, wl["qa"], n_blocks, wl["n_tokens"], RETRIEVED // BT, 1, 0, w, sel,
                                     wl["hist"], wl["q"], wl["q_pos"], N_HEAD, D ** -0.5, out, N_ROT, FREQ_BASE),
             api.prepare_score_topk(st, ix, wl["qa"], n_blocks, wl["n_tokens"], RETRIEVED // BT, 1, 0, w, sel),
             api.prepare_stagein_fa_decode(st, wl["hist"], sel, w, wl["q"], wl["q_pos"], N_HEAD, D ** -0.5, out,
                                           N_ROT, FREQ_BASE))
            for ix, w, sel in wl["reps"]]


def prepare_select(st, api, torch, wl, preps, out):
    """The step's second launch alone, per replica: the selecting attention
    launch (kvm_select_topk_stagein_fa_decode) on the scores the replica's
    step computed (a copy: the launch writes the selection's score array), so
    the top-k, the (empty) plan and the attention are the step's own."""
    n_blocks = wl["hist_tokens"] // BT
    calls = []
    for (step, _, _), (ix, w, sel) in zip(preps, wl["reps"]):
        step()
        torch.cuda.synchronize()
        scores = sel.scores[:n_blocks].clone()
        calls.append(api.prepare_select_decode_step(st, scores, wl["n_tokens"], RETRIEVED // BT, 1, 0, w, sel,
                                                    wl["hist"], wl["q"], wl["q_pos"], N_HEAD, D ** -0.5, out, N_ROT,
                                                    FREQ_BASE))
    return calls


def time_steps(torch, step, fa, steps, warmup, *more):
    """Eager ms per call of each loop, each from one pair of events around
    the loop: an event recorded between two launches would itself open a gap
    of several microseconds in the stream.  `step(i)` runs step i; `fa(i)` runs
    only the attention launch of step i (back to back over the replicas, so
    every launch streams its window from HBM); `more`: further loops."""
    def timed(fn):
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for i in range(steps):
            fn(i)
        stop.record()
        torch.cuda.synchronize()
        return start.elapsed_time(stop) / steps
    return tuple(timed(fn) for fn in (step, fa) + more)


def check_full_size(st, api, L, torch, np, wl):
    """Size-independent checks at full size: planted blocks retrieved, layout contiguous,
    nothing to restage, stage-in bytes of one block equal the oracle's, and the
    attention output equals the ggml-semantics oracle on a sampled head."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    ix, w, sel = wl["reps"][0]
    api.score_topk(st, ix, wl["qa"], wl["hist_tokens"] // BT, wl["n_tokens"], RETRIEVED // BT, 1, 0, None, w, sel)
    res = sel.result()
    assert np.array_equal(res["to_base"], np.arange(0, RETRIEVED, BT)), "window layout"
    assert len(res["stage_slots"]) == 0 and res["total"] == RETRIEVED, "steady state restages nothing"
    assert np.array_equal(res["ids"], wl["ids"])
    cp = w.cell_pos.cpu().numpy()
    assert np.array_equal(cp, np.arange(WINDOW)), "cell positions"
    k, s = 37, int(res["ids"][37])
    ek, ev = w.export_rows(k * BT, BT)
    hk = wl["hist"].kbuf.u8[s * BT * K_ROW:(s + 1) * BT * K_ROW]
    theta = O.rope_theta(FREQ_BASE, 1.0, N_ROT)
    want = O.stagein_k(hk, BT, H_KV, D, N_ROT, 256, k * BT, theta)
    assert np.array_equal(ek.cpu().numpy().reshape(-1), want), "stage-in bytes"
    assert np.array_equal(ev.cpu().numpy().reshape(-1), wl["hist"].vbuf.u8[s * BT * V_ROW:(s + 1) * BT * V_ROW])
    return O


def cpu_threads():
    """Threads for the CPU baseline: the cores this process may use (its
    affinity set), capped by OMP_NUM_THREADS where the host sets a CPU share
    (16 per GPU on the MI355X boxes), and the counts reported beside them."""
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    n = min(avail, share) if share > 0 else avail
    return max(1, n), {"cpu_count": os.cpu_count(), "affinity": avail, "omp_num_threads": share or None}


def median_time(fn, runs):
    """Median wall time of `runs` calls of fn() after one untimed (warm-cache) call."""
    fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2], ts


def cpu_baseline(O, np, wl, out_gpu, runs=21):
    """The oracle's ggml-semantics restatement (C, OpenMP) of one whole decode
    step on this host's cores: scoring over the full 2,048-block index, top-k,
    and flash attention for all 96 query rows over the full 32,768-cell window;
    the median of `runs` warm runs."""
    import torch
    n_threads, counts = cpu_threads()
    ix, w, sel = wl["reps"][0]
    n_blocks = HIST_TOKENS // BT
    k_sum = ix.block_sums().cpu().numpy()                                   # [1][blocks][e]
    mt = ix.mean_tokens.cpu().numpy().astype(np.uint32)
    q_sum = wl["qa"].q_sum.cpu().numpy()
    q_cnt = wl["qa"].q_count.cpu().numpy().astype(np.uint32)
    ek, ev = w.export_rows(0, WINDOW)
    ek, ev = ek.cpu().numpy(), ev.cpu().numpy()
    cp = w.cell_pos.cpu().numpy()
    q = wl["q"].float().cpu().numpy()
    qp = wl["q_pos"].cpu().numpy()
    res = {}

    def step():
        scores = O.score_retrieval(q_sum, q_cnt, k_sum, mt, N_HEAD, H_KV, D, n_threads=n_threads)
        res["ids"] = O.pick_topk(scores, RETRIEVED // BT, 1, 0)
        res["scores"] = scores
        res["out"] = O.fa_ggml(O.T_Q8_0, O.T_Q4_0, q, ek, ev, cp, qp, N_HEAD, H_KV, D, D ** -0.5,
                               n_threads=n_threads)

    med, ts = median_time(step, runs)
    assert np.array_equal(res["scores"].view(np.uint64), sel.scores.cpu().numpy()[:n_blocks].view(np.uint64))
    assert np.array_equal(res["ids"], wl["ids"])
    err = float(np.abs(out_gpu - res["out"]).max())
    assert err <= 2e-3 and err <= 1e-3 * float(np.abs(res["out"]).max()), err
    return {"value": round(med * 1e6, 1), "unit": "us/step", "cores": n_threads, "kind": "port", **counts,
            "runs": runs, "min_us": round(min(ts) * 1e6, 1), "max_us": round(max(ts) * 1e6, 1),
            "sample": f"the whole step on {n_threads} threads, median of {runs} warm runs: oracle ggml-semantics "
                      f"C (OpenMP) scoring over all {n_blocks} blocks + top-k + attention for all "
                      f"{MTP * N_HEAD} query rows over the full {WINDOW}-cell window; outputs checked "
                      f"against the GPU's (scores and ids bit-exact, attention max err {err:.1e})"}


# ---- chunked prefill over the window (2,048-token chunk, MFMA) ----------------
PF_CHUNK = 2048
PF_CELLS = WINDOW + PF_CHUNK
# useful (query, key) pairs per query head: the whole window plus the causal chunk
PF_PAIRS = PF_CHUNK * WINDOW + PF_CHUNK * (PF_CHUNK + 1) // 2          # 69,207,040
PF_FLOP = 4 * D * PF_PAIRS * N_HEAD                                     # 1.7008 TFLOP
MFMA_F16_PEAK_TFLOPS = 2500.0


def run_prefill(args, st, api, L, torch, np):
    """Chunked prefill: a 2,048-token bf16 query chunk at positions 32768..34815,
    causal, against a 32,768-cell q8_0/q4_0 window plus the chunk's own cells
    (written quantised), 24 q heads / 4 kv heads / head_dim 256."""
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0xC0FFEE04)
    reps = []
    for r in range(args.replicas):
        w = api.KVWindow(st, PF_CELLS, H_KV, D, BT)
        for c0 in range(0, PF_CELLS, 8192):
            n = min(8192, PF_CELLS - c0)
            k = api.quantize_rows(st, L.T_Q8_0, torch.randn((n, H_KV * D), generator=gen, device=dev))
            v = api.quantize_rows(st, L.T_Q4_0, torch.randn((n, H_KV * D), generator=gen, device=dev))
            w.import_rows(c0, k, v, torch.arange(c0, c0 + n, dtype=torch.int32, device=dev))
        reps.append(w)
    q = torch.randn((PF_CHUNK, N_HEAD, D), generator=gen, device=dev).to(torch.bfloat16)
    q_pos = torch.arange(WINDOW, WINDOW + PF_CHUNK, dtype=torch.int32, device=dev)
    out = torch.empty((PF_CHUNK, N_HEAD, D), dtype=torch.float32, device=dev)
    scale = D ** -0.5
    for i in range(args.warmup):
        api.fa_prefill(st, reps[i % len(reps)], q, q_pos, N_HEAD, scale, out)
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(args.steps):
        api.fa_prefill(st, reps[i % len(reps)], q, q_pos, N_HEAD, scale, out)
    stop.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / args.steps
    out_gpu = out.cpu().numpy()
    # full-size check: sampled tokens (first, middle, last of the chunk), all heads,
    # against the float64 softmax over the same fp16 operands
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    w = reps[(args.steps - 1) % len(reps)]
    ek, ev = w.export_rows(0, PF_CELLS)
    ek, ev = ek.cpu().numpy(), ev.cpu().numpy()
    cp = w.cell_pos.cpu().numpy()
    kh = O.dequant(O.T_Q8_0, ek.reshape(-1), PF_CELLS * H_KV * D).astype(np.float16).view(np.uint8).reshape(PF_CELLS, -1)
    vh = O.dequant(O.T_Q4_0, ev.reshape(-1), PF_CELLS * H_KV * D).astype(np.float16).view(np.uint8).reshape(PF_CELLS, -1)
    qf = q.float().cpu().numpy()
    qp = q_pos.cpu().numpy()
    toks = np.array([0, 1, PF_CHUNK // 2, PF_CHUNK - 1])
    ref = O.fa_f64(O.T_F16, O.T_F16, qf[toks], kh, vh, cp, qp[toks], N_HEAD, H_KV, D, scale,
                   n_threads=min(16, os.cpu_count() or 1))
    err = float(np.abs(out_gpu[toks] - ref).max())
    assert err <= 2e-3 and err <= 1e-3 * float(np.abs(ref).max()), err
    log("prefill sampled-token check passed (max err %.2e)" % err)
    tflops = PF_FLOP / (ms * 1e-3) / 1e12
    rec = {
        "metric": "chunked prefill attention TFLOP/s (2048-token chunk over a 32K q8_0/q4_0 window)",
        "value": round(tflops, 1), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16 MFMA (K/V dequantised to f16), bf16 Q, fp32 softmax/accumulate",
        "data": "synthetic N(0,1), seed 0xC0FFEE04",
        "config": {"workload": "chunked prefill: 2048 bf16 query tokens at positions 32768..34815, causal, "
                               "over a 34816-cell q8_0/q4_0 window (32768 window cells + the chunk's own), "
                               "24 q heads / 4 kv heads / head_dim 256",
                   "useful_pairs_per_head": PF_PAIRS, "flop": PF_FLOP},
        "roofline": {"bound": "mfma", "kernel": "kvm_fa_prefill (k_pf_stage + k_pf_attn + k_pf_combine)",
                     "achieved": round(tflops, 1), "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4), "traffic": None,
                     "launch_us": round(ms * 1e3, 2)},
    }
    if not args.no_cpu_baseline:
        log("timing the CPU baseline")
        n_threads, counts = cpu_threads()
        # one query token (24 heads) per run, 21 tokens spread over the chunk:
        # a token at chunk position i sees 32768 + i + 1 keys, so the chunk's
        # cost is the per-key cost times its 69,207,040 (query, key) pairs
        ts, keys = [], []
        O.fa_ggml(O.T_Q8_0, O.T_Q4_0, qf[:1], ek, ev, cp, qp[:1], N_HEAD, H_KV, D, scale, n_threads=n_threads)
        for i in np.linspace(0, PF_CHUNK - 1, 21).astype(int):
            tok = np.array([i])
            t1 = time.perf_counter()
            O.fa_ggml(O.T_Q8_0, O.T_Q4_0, qf[tok], ek, ev, cp, qp[tok], N_HEAD, H_KV, D, scale, n_threads=n_threads)
            ts.append((time.perf_counter() - t1) / (WINDOW + i + 1))
        per_key = sorted(ts)[len(ts) // 2]
        total = per_key * PF_PAIRS
        rec["cpu_baseline"] = {
            "value": round(PF_FLOP / total / 1e12, 5), "unit": "TFLOP/s", "cores": n_threads, "kind": "port",
            **counts, "runs": len(ts),
            "sample": f"oracle ggml-semantics C (OpenMP over the 24 heads) attention of one query token per run "
                      f"over the 34816-cell window, 21 tokens spread over the chunk; median time per visible key "
                      f"({per_key * 1e9:.1f} ns) times the chunk's {PF_PAIRS} pairs = {total:.1f} s"}
    print(json.dumps(rec), flush=True)


# ---- stage-in + RoPE re-application (128 selected blocks) --------------------
SI_BLOCKS = 128
SI_BYTES = SI_BLOCKS * BT * (K_ROW + V_ROW)                             # 27,262,976


def run_stagein(args, st, api, L, torch, np):
    """Stage-in of 128 selected 128-token blocks (q8_0 K re-RoPE'd from its
    original position to its window position, FWHT and requantised; q4_0 V moved
    unchanged) from pinned host memory into a 16,384-cell window.  Every step
    restages all 128 blocks (the window's slot table is reset first)."""
    from kvmem_amd import workload as W
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0xC0FFEE03)
    n_blocks = HIST_TOKENS // BT
    kbuf = api.HostBuffer(HIST_TOKENS * K_ROW)
    vbuf = api.HostBuffer(HIST_TOKENS * V_ROW)
    chunk = 16384
    for t0 in range(0, HIST_TOKENS, chunk):
        k = torch.randn((chunk, H_KV * D), generator=gen, device=dev)
        v = torch.randn((chunk, H_KV * D), generator=gen, device=dev)
        torch.from_numpy(kbuf.u8[t0 * K_ROW:(t0 + chunk) * K_ROW]).copy_(api.quantize_rows(st, L.T_Q8_0, k).view(-1).cpu())
        torch.from_numpy(vbuf.u8[t0 * V_ROW:(t0 + chunk) * V_ROW]).copy_(api.quantize_rows(st, L.T_Q4_0, v).view(-1).cpu())
    hist = api.History.__new__(api.History)
    hist.kbuf, hist.vbuf, hist.n_tokens = kbuf, vbuf, HIST_TOKENS
    hist.c = L.History(kbuf.ptr, vbuf.ptr, HIST_TOKENS)
    chosen = np.sort(W.distinct_ids(0xC0FFEE03, 0, SI_BLOCKS, 0, n_blocks))
    scores = torch.zeros(n_blocks, dtype=torch.float64, device=dev)
    scores[torch.from_numpy(chosen).to(dev)] = 1.0
    n_tokens = torch.full((n_blocks,), BT, dtype=torch.int32, device=dev)
    w = api.KVWindow(st, SI_BLOCKS * BT, H_KV, D, BT)
    sel = api.select_topk(st, scores, n_tokens, SI_BLOCKS, 0, 0, None, w)
    res = sel.result()
    assert np.array_equal(res["ids"], chosen) and len(res["stage_slots"]) == SI_BLOCKS, res

    def step():
        w.reset()
        api.select_topk(st, scores, n_tokens, SI_BLOCKS, 0, 0, None, w, sel)
        api.stagein_selection(st, hist, w, sel, N_ROT, FREQ_BASE)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    for i in range(args.steps):
        w.reset()
        api.select_topk(st, scores, n_tokens, SI_BLOCKS, 0, 0, None, w, sel)
        evs[i][0].record()
        api.stagein_selection(st, hist, w, sel, N_ROT, FREQ_BASE)
        evs[i][1].record()
    torch.cuda.synchronize()
    ms = sum(a.elapsed_time(b) for a, b in evs) / args.steps
    # the same bytes as one plain pinned-host -> device copy, for the link's reach
    dst = torch.empty(SI_BYTES, dtype=torch.uint8, device=dev)
    src = torch.from_numpy(kbuf.u8[:SI_BYTES])
    dst.copy_(src, non_blocking=True)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(10):
        dst.copy_(src, non_blocking=True)
    e1.record()
    torch.cuda.synchronize()
    copy_gbps = SI_BYTES * 10 / (e0.elapsed_time(e1) * 1e-3) / 1e9
    # bit-exact check of every staged block against the oracle
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    theta = O.rope_theta(FREQ_BASE, 1.0, N_ROT)
    ek, ev = w.export_rows(0, SI_BLOCKS * BT)
    ek, ev = ek.cpu().numpy(), ev.cpu().numpy()
    for k, b in enumerate(chosen):
        hk = kbuf.u8[b * BT * K_ROW:(b + 1) * BT * K_ROW]
        want = O.stagein_k(hk, BT, H_KV, D, N_ROT, 256, k * BT, theta)
        assert np.array_equal(ek[k * BT:(k + 1) * BT].reshape(-1), want), f"K of block {b}"
        assert np.array_equal(ev[k * BT:(k + 1) * BT].reshape(-1), vbuf.u8[b * BT * V_ROW:(b + 1) * BT * V_ROW])
    log("stage-in bytes of all %d blocks equal the oracle's" % SI_BLOCKS)
    # CPU baseline: the oracle's stage-in of all 128 blocks (K chain per block,
    # one block per task on a thread pool: ctypes releases the GIL) plus the V
    # byte copies into a staging buffer, median of 21 warm runs
    from concurrent.futures import ThreadPoolExecutor
    n_threads, counts = cpu_threads()
    vdst = np.empty(SI_BLOCKS * BT * V_ROW, np.uint8)

    def one(kb):
        k, b = kb
        O.stagein_k(kbuf.u8[b * BT * K_ROW:(b + 1) * BT * K_ROW], BT, H_KV, D, N_ROT, 256, k * BT, theta)
        vdst[k * BT * V_ROW:(k + 1) * BT * V_ROW] = vbuf.u8[b * BT * V_ROW:(b + 1) * BT * V_ROW]

    with ThreadPoolExecutor(n_threads) as pool:
        t_cpu, _ = median_time(lambda: list(pool.map(one, enumerate(chosen))), 21)
    gbps = SI_BYTES / (ms * 1e-3) / 1e9
    rec = {
        "metric": "stage-in + RoPE re-application host->device GB/s (128 selected blocks)",
        "value": round(gbps, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q8_0 K (fp32 RoPE/FWHT, requantised) / q4_0 V bytes", "data": "synthetic N(0,1), seed 0xC0FFEE03",
        "config": {"workload": "stage-in: 128 distinct 128-token blocks drawn uniformly from 2048, pinned host "
                               "q8_0 K / q4_0 V -> 16384-cell window, 4 kv heads, head_dim 256, NeoX RoPE on 64 dims "
                               "(theta 1e7) from the original to the window position, FWHT 256, q8_0 requant",
                   "bytes_h2d": SI_BYTES},
        "roofline": {"bound": "host-link", "kernel": "kvm_stagein_selection (k_stagein)",
                     "achieved": round(gbps, 2), "peak": round(copy_gbps, 2), "unit": "GB/s",
                     "frac": round(gbps / copy_gbps, 4), "traffic": None, "launch_us": round(ms * 1e3, 2),
                     "peak_source": "plain pinned-host->device copy of the same bytes on this box"},
        "cpu_baseline": {"value": round(SI_BYTES / t_cpu / 1e9, 3), "unit": "GB/s", "cores": n_threads,
                         "kind": "port", **counts, "runs": 21,
                         "sample": f"oracle C stage-in (dequant, RoPE, FWHT, requant) of K plus the V byte copy for "
                                   f"all {SI_BLOCKS} blocks, one block per task on {n_threads} threads, median of 21 "
                                   f"warm runs ({t_cpu * 1e3:.1f} ms)"},
    }
    print(json.dumps(rec), flush=True)


# ---- churn: the decode step with one block swapped per step ------------------
def pinned_history(st, api, L, torch, seed):
    """A 262,144-token pinned host history of q8_0 K / q4_0 V rows of N(0,1) values."""
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    kbuf = api.HostBuffer(HIST_TOKENS * K_ROW)
    vbuf = api.HostBuffer(HIST_TOKENS * V_ROW)
    chunk = 16384
    for t0 in range(0, HIST_TOKENS, chunk):
        k = torch.randn((chunk, H_KV * D), generator=gen, device=dev)
        v = torch.randn((chunk, H_KV * D), generator=gen, device=dev)
        torch.from_numpy(kbuf.u8[t0 * K_ROW:(t0 + chunk) * K_ROW]).copy_(api.quantize_rows(st, L.T_Q8_0, k).view(-1).cpu())
        torch.from_numpy(vbuf.u8[t0 * V_ROW:(t0 + chunk) * V_ROW]).copy_(api.quantize_rows(st, L.T_Q4_0, v).view(-1).cpu())
    hist = api.History.__new__(api.History)
    hist.kbuf, hist.vbuf, hist.n_tokens = kbuf, vbuf, HIST_TOKENS
    hist.c = L.History(kbuf.ptr, vbuf.ptr, HIST_TOKENS)
    return hist


def run_churn(args, st, api, L, torch, np):
    """The headline decode step (256K history, 32K window, 4 bf16 query tokens)
    when each step's selection differs from the previous one by one early block:
    the second-oldest selected block leaves and one past the newest joins, or
    the reverse, so the 126 blocks between move one slot and must be re-rotated
    to their new window positions.  The mean-K index makes two alternating
    queries select exactly those two sets.  Timed with a window that keeps a K
    shadow (moved blocks re-based from HBM, one block read from the host) and
    with one that does not (127 blocks restaged over PCIe), against the same
    step with an unchanging query; the step as three launches (value:
    kvm_score_topk, then kvm_stagein_fa_decode, whose attention workgroups
    stage the plan), as four (kvm_score_topk_stagein, whose stage-in kernel
    runs two workgroups per CU, then kvm_fa_decode) and as two
    (kvm_score_topk_stagein_fa_decode: a changed plan is staged after a pass of
    the attention over the window as it was, which then runs again)."""
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0xC0FFEE06)
    n_blocks, nsel = HIST_TOKENS // BT, RETRIEVED // BT
    hist = pinned_history(st, api, L, torch, 0xC0FFEE06)
    rng = np.random.default_rng(0xC0FFEE06)
    sa = np.concatenate([[0], np.sort(rng.choice(np.arange(1, n_blocks - 1), nsel - 1, replace=False))])
    sb = np.sort(np.concatenate([np.setdiff1d(sa, [sa[1]]), [n_blocks - 1]]))
    sums = torch.zeros((1, n_blocks, H_KV * D), device=dev)
    sums[0, torch.from_numpy(sa).to(dev), 0] = float(BT)
    sums[0, torch.from_numpy(sb).to(dev), 1] = float(BT)
    ix = api.MeanKIndex(st, 1, n_blocks, H_KV, D, BT, norms=True)
    ix.set_block_sums(sums)
    ix.mean_tokens[:, :n_blocks] = BT
    ix.present[:n_blocks] = 1
    ix.refresh()
    qas = []
    for dim in (0, 1):
        qa = api.QueryAcc(st, 1, N_HEAD, D, n_head_kv=H_KV)
        qa.q_sum.zero_()
        qa.q_sum[0, dim] = 1.0
        qa.q_count.fill_(1)
        qa.refresh()
        qas.append(qa)
    n_tokens = torch.full((n_blocks,), BT, dtype=torch.int32, device=dev)
    ng = WINDOW - RETRIEVED
    gk = api.quantize_rows(st, L.T_Q8_0, torch.randn((ng, H_KV * D), generator=gen, device=dev))
    gv = api.quantize_rows(st, L.T_Q4_0, torch.randn((ng, H_KV * D), generator=gen, device=dev))
    gpos = torch.arange(RETRIEVED, WINDOW, dtype=torch.int32, device=dev)
    q = torch.randn((MTP, N_HEAD, D), generator=gen, device=dev).to(torch.bfloat16)
    q_pos = torch.arange(WINDOW - MTP, WINDOW, dtype=torch.int32, device=dev)
    out = torch.empty((MTP, N_HEAD, D), dtype=torch.float32, device=dev)
    res = {}
    for shadow in (True, False):
        w = api.KVWindow(st, WINDOW, H_KV, D, BT, shadow=shadow)
        sel = api.SelectionBuffers(st, n_blocks, nsel)
        w.import_rows(RETRIEVED, gk, gv, gpos)
        calls = [(api.prepare_score_topk(st, ix, qa, n_blocks, n_tokens, nsel, 1, 0, w, sel),
                  api.prepare_stagein_fa_decode(st, hist, sel, w, q, q_pos, N_HEAD, D ** -0.5, out, N_ROT, FREQ_BASE))
                 for qa in qas]
        # the step as four launches: kvm_score_topk_stagein (scoring, top-k, the
        # stage-in kernel at two workgroups per CU), then kvm_fa_decode
        calls4 = [(api.prepare_score_topk_stagein(st, ix, qa, n_blocks, n_tokens, nsel, 1, 0, w, sel, hist, N_ROT,
                                                  FREQ_BASE),
                   api.prepare_fa_decode(st, w, q, q_pos, N_HEAD, D ** -0.5, out)) for qa in qas]

        def churn4(i):
            r, f = calls4[i % 2]
            r()
            f()

        def churn(i):
            r, f = calls[i % 2]
            r()
            f()

        def steady(i):
            r, f = calls[0]
            r()
            f()

        # the same steps in two launches (kvm_score_topk_stagein_fa_decode): the
        # attention runs over the window as it was, then the plan is staged and
        # the attention runs again
        steps2 = [api.prepare_decode_step(st, ix, qa, n_blocks, n_tokens, nsel, 1, 0, w, sel, hist, q, q_pos, N_HEAD,
                                          D ** -0.5, out, N_ROT, FREQ_BASE) for qa in qas]
        churn(0)
        torch.cuda.synchronize()
        assert np.array_equal(sel.result()["ids"], sa)
        steady2_ms, churn2_ms = time_steps(torch, lambda i: steps2[0](), lambda i: steps2[i % 2](), args.steps,
                                           args.warmup)
        churn(0)
        steady_ms, _ = time_steps(torch, steady, lambda i: None, args.steps, args.warmup)
        churn_ms, churn4_ms = time_steps(torch, churn, churn4, args.steps, args.warmup)
        r = sel.result()
        last = sb if (args.steps - 1) % 2 == 1 else sa            # the timed loop's last call
        assert np.array_equal(r["ids"], last) and r["status"] == 0, r["status"]
        moved = int((r["stage_src"] >= 0).sum())
        assert len(r["stage_slots"]) == nsel - 1 and moved == (nsel - 2 if shadow else 0), (len(r["stage_slots"]), moved)
        # the window equals a fresh stage-in of the last plan
        wf = api.KVWindow(st, WINDOW, H_KV, D, BT)
        sf = api.select_topk(st, sel.scores[:n_blocks].clone(), n_tokens, nsel, 1, 0, None, wf)
        api.stagein_selection(st, hist, wf, sf, N_ROT, FREQ_BASE)
        ka, va = w.export_rows(0, RETRIEVED)
        kb, vb = wf.export_rows(0, RETRIEVED)
        assert torch.equal(ka, kb) and torch.equal(va, vb), "churned window differs from a fresh stage-in"
        res[shadow] = dict(churn_us=churn_ms * 1e3, churn4_us=churn4_ms * 1e3, steady_us=steady_ms * 1e3, moved=moved,
                           host_blocks=len(r["stage_slots"]) - moved, churn2_us=churn2_ms * 1e3,
                           steady2_us=steady2_ms * 1e3)
        log("shadow=%s: steady %.2f us, churn %.2f us (four launches %.2f) per step"
            % (shadow, steady_ms * 1e3, churn_ms * 1e3, churn4_ms * 1e3))
        del w, sel, calls, calls4, steps2, wf, sf
        torch.cuda.synchronize()
    a, b = res[True], res[False]
    # least HBM traffic of the shadow restage: a moved block's raw K read from the
    # shadow and its K tile written, its V tiles read and written; the new block's
    # rows cross the host link
    hbm_min = a["moved"] * BT * 2 * (K_ROW + V_ROW)
    rec = {
        "metric": "decode step with one selected block swapped per step, µs/token @256K history, 32K window",
        "value": round(a["churn_us"], 2), "unit": "us/step", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(a["churn_us"] * 1e-3, 5), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "q8_0/q4_0 KV (int8 + fp16 MFMA), bf16 Q, fp32 softmax",
        "data": "synthetic N(0,1) history and query, seed 0xC0FFEE06; mean-K index built for two alternating selections",
        "config": {"workload": "decode step (score + top-k + stage-in + FA decode over a 32768-cell window, 4 bf16 "
                               "query tokens) whose 128-block selection alternates between two sets differing in "
                               "the second-oldest and the newest block: 127 slots restaged per step, 126 of them "
                               "blocks already in the window that move one slot",
                   "history_tokens": HIST_TOKENS, "window_cells": WINDOW},
        "shadow": {"churn_us": round(a["churn_us"], 2), "four_launch_churn_us": round(a["churn4_us"], 2),
                   "steady_us": round(a["steady_us"], 2),
                   "restage_us": round(a["churn_us"] - a["steady_us"], 2), "moved_blocks": a["moved"],
                   "host_blocks": a["host_blocks"], "hbm_bytes_min": hbm_min,
                   "h2d_bytes": a["host_blocks"] * BT * (K_ROW + V_ROW),
                   "two_launch_churn_us": round(a["churn2_us"], 2), "two_launch_steady_us": round(a["steady2_us"], 2)},
        "host_restage": {"churn_us": round(b["churn_us"], 2), "four_launch_churn_us": round(b["churn4_us"], 2),
                         "steady_us": round(b["steady_us"], 2),
                         "restage_us": round(b["churn_us"] - b["steady_us"], 2), "host_blocks": b["host_blocks"],
                         "h2d_bytes": b["host_blocks"] * BT * (K_ROW + V_ROW),
                         "two_launch_churn_us": round(b["churn2_us"], 2),
                         "two_launch_steady_us": round(b["steady2_us"], 2)},
    }
    print(json.dumps(rec), flush=True)


# ---- multi-lane decode (4 conversations) -------------------------------------
LANE_HIST = (65536, 131072, 196608, 262144)


def run_lanes(args, st, api, L, torch, np):
    """Four conversations, each with its own 32K-cell window, mean-K index and
    pinned host history (64K / 128K / 192K / 256K tokens), one bf16 query token
    each.  A step is two launches for all lanes
    (kvm_score_topk_stagein_fa_decode_lanes: the scoring grid over every lane's
    blocks, then one launch whose selector workgroup per lane picks the blocks
    while the lanes' attention workgroups attend); the same step as three
    launches (retrieval for all lanes: scoring grid + one top-k workgroup per
    lane; then stage-in and attention for all lanes in one launch) is timed
    beside it."""
    n_rep = 2
    wls = []
    for i, ht in enumerate(LANE_HIST):
        log("building lane %d (%d-token history)" % (i, ht))
        wls.append(build_workload(st, api, L, torch, np, n_rep, seed=0xC0FFEE05 + i, hist_tokens=ht, mtp=1))
    outs = [torch.empty((1, N_HEAD, D), dtype=torch.float32, device="cuda") for _ in wls]
    scale = D ** -0.5
    preps = []
    for r in range(n_rep):
        lanes = [dict(index=wl["reps"][r][0], query=wl["qa"], n_blocks=wl["hist_tokens"] // BT,
                      n_tokens=wl["n_tokens"], budget_blocks=RETRIEVED // BT, sink_blocks=1,
                      window=wl["reps"][r][1], sel=wl["reps"][r][2], history=wl["hist"]) for wl in wls]
        fa_lanes = [dict(history=wl["hist"], sel=wl["reps"][r][2], window=wl["reps"][r][1], q=wl["q"],
                         q_pos=wl["q_pos"], out=o) for wl, o in zip(wls, outs)]
        steps = [dict(ln, q=fl["q"], q_pos=fl["q_pos"], out=fl["out"]) for ln, fl in zip(lanes, fa_lanes)]
        preps.append((api.prepare_decode_step_lanes(st, steps, N_HEAD, scale, N_ROT, FREQ_BASE),
                      api.prepare_score_topk_lanes(st, lanes),
                      api.prepare_stagein_fa_decode_lanes(st, fa_lanes, N_HEAD, scale, N_ROT, FREQ_BASE)))

    def three_launch(i):
        _, retrieve, fa = preps[i % n_rep]
        retrieve()
        fa()

    ms, fa_ms, three_ms = time_steps(torch, lambda i: preps[i % n_rep][0](), lambda i: preps[i % n_rep][2](),
                                     args.steps, args.warmup, three_launch)
    # checks: each lane's selection equals its single-lane one, nothing to restage,
    # and its attention equals the single-lane kernel's and the oracle's
    r = (args.steps - 1) % n_rep
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    for i, wl in enumerate(wls):
        ix, w, sel = wl["reps"][r]
        res = sel.result()
        assert np.array_equal(res["ids"], wl["ids"]) and len(res["stage_slots"]) == 0, i
        one = api.fa_decode(st, w, wl["q"], wl["q_pos"], N_HEAD, scale).cpu().numpy()
        np.testing.assert_allclose(outs[i].cpu().numpy(), one, rtol=1e-3, atol=1e-4)
    ek, ev = wls[0]["reps"][r][1].export_rows(0, WINDOW)
    ref = O.fa_ggml(O.T_Q8_0, O.T_Q4_0, wls[0]["q"].float().cpu().numpy()[:, :G], ek.cpu().numpy()[:, :K_ROW // H_KV],
                    ev.cpu().numpy()[:, :V_ROW // H_KV], wls[0]["reps"][r][1].cell_pos.cpu().numpy(),
                    wls[0]["q_pos"].cpu().numpy(), G, 1, D, scale, n_threads=min(16, os.cpu_count() or 1))
    got = outs[0].cpu().numpy()[:, :G]
    err = float(np.abs(got - ref).max())
    assert err <= 2e-3 and err <= 1e-3 * float(np.abs(ref).max()), err
    log("multi-lane checks passed")
    n_blocks = [h // BT for h in LANE_HIST]
    fa_bytes = len(wls) * (FA_KV_BYTES + N_HEAD * D * (2 + 4))
    step_bytes = fa_bytes + sum(nb * (H_KV * D * 4 + 8) for nb in n_blocks)
    fa_gbps = fa_bytes / (fa_ms * 1e-3) / 1e9
    rec = {
        "metric": "multi-lane decode aggregate tokens/s (4 lanes, 64K-256K histories, 32K windows)",
        "value": round(len(wls) / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "q8_0/q4_0 KV (int8 + fp16 MFMA), bf16 Q, fp32 softmax",
        "data": "synthetic N(0,1), seeds 0xC0FFEE05 + lane, 16 planted blocks per lane",
        "config": {"workload": "4 lanes: histories of 65536/131072/196608/262144 tokens (pinned host q8_0 K / "
                               "q4_0 V), 32768-cell windows, 1 bf16 query token per lane; the scoring grid for all "
                               "lanes, then one launch that selects, stages and attends for all lanes "
                               "(kvm_score_topk_stagein_fa_decode_lanes); 24 q heads / 4 kv heads / head_dim 256; "
                               "2 replicas cycled",
                   "lanes": len(wls), "step_bytes": step_bytes},
        "three_launch_ms_per_step": round(three_ms, 5),
        "hbm_gbps": round(step_bytes / (ms * 1e-3) / 1e9, 1),
        "roofline": {"bound": "hbm", "kernel": "kvm_stagein_fa_decode_lanes (k_fa_decode_staged: split-K "
                                               "attention over every lane, splits merged in-launch)",
                     "achieved": round(fa_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(fa_gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                     "launch_us": round(fa_ms * 1e3, 3), "algorithmic_bytes": fa_bytes},
    }
    print(json.dumps(rec), flush=True)


# ---- history sweep of the decode step ------------------------------------------
SWEEP_HIST = (32768, 65536, 131072, 262144)


def run_sweep(args, st, api, L, torch, np):
    """The decode step at 32K / 64K / 128K / 256K-token histories (same window,
    query and replicas); one JSON line with a row per history size."""
    rows = []
    out = torch.empty((MTP, N_HEAD, D), dtype=torch.float32, device="cuda")
    for ht in SWEEP_HIST:
        log("history %d" % ht)
        wl = build_workload(st, api, L, torch, np, args.replicas, hist_tokens=ht)
        preps = prepare_decode(st, api, wl, out)

        ms, fa_ms = time_steps(torch, lambda i: preps[i % len(preps)][0](), lambda i: preps[i % len(preps)][2](),
                               args.steps, args.warmup)
        nb = ht // BT
        step_bytes = nb * (H_KV * D * 4 + 8) + FA_KV_BYTES + QO_BYTES
        rows.append({"history_tokens": ht, "blocks": nb, "us_per_step": round(ms * 1e3, 2),
                     "fa_us": round(fa_ms * 1e3, 2), "step_bytes": step_bytes,
                     "hbm_gbps": round(step_bytes / (ms * 1e-3) / 1e9, 1),
                     "roofline_step_us": round(step_bytes / (HBM_PEAK_GBPS * 1e9) * 1e6, 3)})
        log(json.dumps(rows[-1]))
        del preps, wl
        torch.cuda.synchronize()
    last = rows[-1]
    rec = {
        "metric": "decode attn+retrieval µs/token and HBM GB/s, history sweep 32K-256K, 32K window",
        "value": last["us_per_step"], "unit": "us/step", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "q8_0/q4_0 KV (int8 + fp16 MFMA), bf16 Q, fp32 softmax", "data": "synthetic N(0,1), seed 0xC0FFEE02",
        "config": {"workload": "decode step (score + top-k + stage plan + stage-in + FA decode over a 32768-cell "
                               "window, 4 bf16 query tokens) at each history size", "replicas": args.replicas},
        "sweep": rows,
    }
    print(json.dumps(rec), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--workload", default="decode",
                    choices=["decode", "prefill", "stagein", "lanes", "sweep", "churn"],
                    help="decode: the headline decode step (default); prefill: chunked-prefill attention; "
                         "stagein: stage-in + RoPE of 128 blocks; lanes: 4-lane decode; sweep: decode step "
                         "at 32K-256K histories; churn: the decode step with one block swapped per step")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--replicas", type=int, default=8)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="after the timed region, copy 256 MiB device-to-device once (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for {args.gpus}): the path is not sharded across GPUs",
              file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch
    from kvmem_amd import api, _lib as L

    st = api.State(0)
    if args.workload == "prefill":
        return run_prefill(args, st, api, L, torch, np)
    if args.workload == "stagein":
        return run_stagein(args, st, api, L, torch, np)
    if args.workload == "lanes":
        return run_lanes(args, st, api, L, torch, np)
    if args.workload == "sweep":
        return run_sweep(args, st, api, L, torch, np)
    if args.workload == "churn":
        return run_churn(args, st, api, L, torch, np)
    log("building workload (256K history, 32K window, %d replicas)" % args.replicas)
    t0 = time.time()
    wl = build_workload(st, api, L, torch, np, args.replicas)
    log("workload ready in %.1f s" % (time.time() - t0))
    O = check_full_size(st, api, L, torch, np, wl)
    log("full-size checks passed")

    out = torch.empty((MTP, N_HEAD, D), dtype=torch.float32, device="cuda")
    preps = prepare_decode(st, api, wl, out)
    selects = prepare_select(st, api, torch, wl, preps, out)

    def three_launch(i):
        _, retrieve, fa = preps[i % len(preps)]
        retrieve()
        fa()

    step_ms, fa_ms, three_ms, sel_ms = time_steps(torch, lambda i: preps[i % len(preps)][0](),
                                                  lambda i: preps[i % len(preps)][2](), args.steps, args.warmup,
                                                  three_launch, lambda i: selects[i % len(selects)]())
    out_gpu = out.cpu().numpy()
    if args.calibrate_copy:
        a = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        b = torch.empty_like(a)
        b.copy_(a)
        torch.cuda.synchronize()

    fa_bytes = FA_KV_BYTES + QO_BYTES
    # the selecting launch also reads the scores and the blocks' token counts
    # and writes the per-block scores and the selection
    n_blocks = HIST_TOKENS // BT
    sel_bytes = fa_bytes + n_blocks * (8 + 4 + 8) + (RETRIEVED // BT) * 12
    sel_gbps = sel_bytes / (sel_ms * 1e-3) / 1e9
    step_us = step_ms * 1e3
    rec = {
        "metric": "decode attn+retrieval µs/token and HBM GB/s @256K history, 32K window",
        "value": round(step_us, 2),
        # one decode step: 4 query tokens (an MTP verify step) against the window
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8_0/q4_0 KV (int8 + fp16 MFMA), bf16 Q, fp32 softmax",
        "data": "synthetic N(0,1), seed 0xC0FFEE02, 16 planted blocks",
        "config": {"workload": "decode step: 262144-token history (2048 x 128-token blocks, pinned host "
                               "q8_0 K / q4_0 V) -> score + top-k(128 blocks incl. sink) + stage plan + "
                               "stage-in + FA decode over a 32768-cell q8_0/q4_0 window; 4 bf16 query tokens "
                               "(MTP verify), 24 q heads / 4 kv heads / head_dim 256; 1 layer per step, "
                               f"{args.replicas} layer replicas cycled; two launches "
                               "(kvm_score_topk_stagein_fa_decode)",
                   "history_tokens": HIST_TOKENS, "window_cells": WINDOW, "query_tokens": MTP},
        "hbm_gbps": round(STEP_BYTES / (step_ms * 1e-3) / 1e9, 1),
        # the same step as three launches (kvm_score_topk, then kvm_stagein_fa_decode)
        "three_launch_step_us": round(three_ms * 1e3, 2),
        # the reference retrieves once per query (tools/llama-kvmem-server.cpp:1466):
        # the step above is the worst case (a retrieval every token); split into
        # what retrieval adds per event (score + top-k + stage plan) and
        # attention per token, from the step and the separately timed attention loop
        "us_per_query_token": round(step_us / MTP, 3),
        "per_event": {"retrieval_us": round(step_us - fa_ms * 1e3, 2),
                      "attention_us_per_step": round(fa_ms * 1e3, 3)},
        "step_bytes": STEP_BYTES,
        "roofline_step_us": round(STEP_BYTES / (HBM_PEAK_GBPS * 1e9) * 1e6, 3),
        # the step's dominant kernel: its second launch, timed alone on the
        # step's own scores (the same top-k, empty plan and attention)
        "roofline": {"bound": "hbm", "kernel": "k_fa_decode_select (the step's second launch: the selector "
                                               "column's top-k while the split-K attention runs, splits merged "
                                               "in-launch)",
                     "achieved": round(sel_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(sel_gbps / HBM_PEAK_GBPS, 4), "traffic": measured_traffic(),
                     "traffic_source": os.path.relpath(TRAFFIC_PROFILE, ROOT),
                     "launch_us": round(sel_ms * 1e3, 3), "algorithmic_bytes": sel_bytes},
        # the attention launch of the three-launch form (k_fa_decode_staged)
        "attention_only": {"kernel": "k_fa_decode_staged", "launch_us": round(fa_ms * 1e3, 3),
                           "achieved": round(fa_bytes / (fa_ms * 1e-3) / 1e9, 1),
                           "frac": round(fa_bytes / (fa_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)},
    }
    if not args.no_cpu_baseline:
        log("timing the CPU baseline")
        rec["cpu_baseline"] = cpu_baseline(O, np, wl, out_gpu)
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
