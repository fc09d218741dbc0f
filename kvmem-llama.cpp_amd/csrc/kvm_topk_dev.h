// kvm_topk_dev.h -- device side of the top-k block selection and window
// layout (pick_topk_blocks + set_selection, kvmem_store.cpp:357-623 and
// llama-memory-kvmem.cpp:4256-4340), shared by the top-k kernel of
// kvm_retrieval.hip (1,024 threads, up to 8,192 blocks) and the decode
// attention launch whose selector workgroup runs it (512 threads, up to 4,096
// blocks) while the other workgroups attend.
//
// One workgroup of NTH threads per lane; thread t owns the blocks t, t + NTH,
// ... for loading and the contiguous range [t*per, (t+1)*per) for compaction.
// Every global read is issued before any use; barriers order LDS only.
#pragma once
#include "kvm_score_dev.h"

struct topk_args {
    const double *scores_in;   // caller's scores (kvm_select_topk), or null
    const double *layer_score; // per-layer contributions [layer][cap] (kvm_score_topk)
    const uint32_t *q_count;
    const uint8_t *present;
    double *scores_out;        // scores reduced from the layer contributions
    const uint32_t *n_tokens;
    const uint32_t *mandatory;
    const uint32_t *slot_block;
    const int32_t *slot_base;
    uint32_t *ids;
    int32_t *to_base;
    uint32_t *stage_slots;
    uint32_t *info;
    uint32_t n, budget, sink, recent, n_mand, n_slots, cap, n_layer, ls_cap;
    const uint32_t *shadow_rows;   // the window's shadow row counts, or null
    int32_t *stage_src;            // per staged entry, the old slot it moves from (-1: host)
    uint32_t bt;                   // the window's block_tokens
    const uint32_t *pending_rows;  // the window's unharvested rows per slot, or null
    uint32_t *stage_out;           // the blocks leaving the plan's slots, or null
};

// Independent retrievals (conversation lanes) in one launch.
#define KVM_RET_LANES 8
struct topk_lanes {
    topk_args lane[KVM_RET_LANES];
};

#define KVM_TOPK_FINE 1024        // linear bins of the one-pass select (64 coarse bins of 16)
#define KVM_TOPK_GATHER 64        // largest threshold bin ranked exactly

// order-preserving map of a double to uint64 (-0.0 folded onto +0.0, so the
// two compare equal as in the reference's `sa != sb` test)
__device__ inline uint64_t ord_key(double x) {
    if (x == 0.0) x = 0.0;
    const uint64_t u = (uint64_t)__double_as_longlong(x);
    return (u >> 63) ? ~u : (u | 0x8000000000000000ull);
}

// exclusive prefix sums of two values over the NTH threads (DPP wave scans,
// one LDS exchange of the wave totals); totals through t1, t2.  s_tmp holds
// 2 * waves words; consecutive calls must use different s_tmp buffers (a call
// returns without a second barrier, while other waves may still read its buffer)
template <int NTH>
__device__ void block_scan2(uint32_t v1, uint32_t v2, uint32_t *s_tmp, uint32_t &e1, uint32_t &e2,
                            uint32_t &t1, uint32_t &t2) {
    constexpr uint32_t NW = NTH / 64;
    const uint32_t lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const uint32_t x1 = kvm_wave_incl_scan(v1), x2 = kvm_wave_incl_scan(v2);
    if (lane == 63) { s_tmp[wid] = x1; s_tmp[NW + wid] = x2; }
    KVM_LDS_BARRIER();
    const uint32_t w1 = lane < NW ? s_tmp[lane] : 0u, w2 = lane < NW ? s_tmp[NW + lane] : 0u;
    const uint32_t i1 = kvm_wave_incl_scan(w1), i2 = kvm_wave_incl_scan(w2);
    e1 = x1 - v1 + __builtin_amdgcn_readlane(i1 - w1, wid);
    e2 = x2 - v2 + __builtin_amdgcn_readlane(i2 - w2, wid);
    t1 = __builtin_amdgcn_readlane(i1, NW - 1);
    t2 = __builtin_amdgcn_readlane(i2, NW - 1);
}

// s_hist[bin] += 1 for every active lane, one atomic per distinct bin run:
// the lanes sharing the first active lane's bin are counted with a ballot
// (the skewed top digits put most keys in one bin), the rest individually.
__device__ inline void hist_add(uint32_t *s_hist, uint32_t bin, bool active) {
    const uint64_t act = __builtin_amdgcn_ballot_w64(active);
    if (!act) return;
    const uint32_t lead = (uint32_t)__builtin_ctzll(act);
    const uint32_t lbin = __builtin_amdgcn_readlane(bin, lead);
    const uint64_t same = __builtin_amdgcn_ballot_w64(active && bin == lbin);
    if ((threadIdx.x & 63) == lead) atomicAdd(&s_hist[lbin], (uint32_t)__builtin_popcountll(same));
    if (active && bin != lbin) atomicAdd(&s_hist[bin], 1u);
}

// The selection's LDS: keys, token counts and kept flags of up to MAXB blocks,
// the first SLOTS entries of the window's slot map, and the select's small
// buffers.  The top-k kernel declares it statically; the decode attention's
// selector places it in the launch's dynamic LDS.
template <int NTH, int MAXB, int SLOTS>
struct topk_lds {
    static constexpr uint32_t NW = NTH / 64;
    kvm_u32x4 gath[KVM_TOPK_GATHER];
    uint32_t fine[KVM_TOPK_FINE];
    uint64_t key[MAXB];
    uint64_t prefix;
    uint32_t ntok[MAXB];
    uint32_t sblk[SLOTS];
    int32_t sbase[SLOTS];
    uint32_t spend[SLOTS];        // unharvested rows per slot (0 without tracking)
    uint32_t hist[2][256];
    uint32_t tmp[2][2 * NW];      // block_scan2 buffers, used alternately
    float wmm[2][NW];
    uint32_t wc[NW];
    uint32_t rank[KVM_TOPK_GATHER];
    uint32_t sel[4];
    uint32_t count, k, done, need;
    uint8_t kept[MAXB];
};

// Selection of the `need` best candidates under the strict order
// (score desc, block id desc): a one-pass select over a linear histogram of
// the fp32-rounded scores, or an MSB-first radix select over the
// order-preserving 64-bit keys that narrows to the bin holding the need-th
// largest key; it stops as soon as that bin is taken whole, otherwise ties on
// the full key are broken by descending block id.  Then the ascending
// compaction with window positions and the stage plan.  Returns the plan's
// length to stage (0 when the layout does not fit), the same in every thread.
template <int NTH, int MAXB, int SLOTS>
__device__ __forceinline__ uint32_t topk_body(const topk_args &a, topk_lds<NTH, MAXB, SLOTS> &T) {
#pragma clang fp contract(off)
    static_assert(NTH >= 256 && NTH % 64 == 0 && KVM_TOPK_GATHER * KVM_TOPK_GATHER % NTH == 0, "top-k threads");
    static_assert(MAXB % NTH == 0 && MAXB / NTH <= 32 && SLOTS % NTH == 0, "top-k capacities");
    constexpr uint32_t LOAD = MAXB / NTH;
    uint64_t *const s_key = T.key;
    uint32_t *const s_ntok = T.ntok;
    uint8_t *const s_kept = T.kept;
    uint32_t *const s_sblk = T.sblk;
    int32_t *const s_sbase = T.sbase;
    auto &s_hist = T.hist;
    auto &s_tmp = T.tmp;
    uint32_t &s_count = T.count, &s_k = T.k, &s_done = T.done, &s_need = T.need;
    uint64_t &s_prefix = T.prefix;
    uint32_t *const s_fine = T.fine;
    auto &s_wmm = T.wmm;
    uint32_t *const s_wc = T.wc;
    uint32_t *const s_sel = T.sel;
    kvm_u32x4 *const s_gath = T.gath;
    uint32_t *const s_rank = T.rank;
    const uint32_t tid = threadIdx.x, lane = tid & 63, n = a.n;
    const bool all = a.budget == 0 || n <= a.budget;
    // the window's slot map for the ranks the stage plan compares (loaded with
    // the scores, so the compaction needs no second memory round trip)
    const uint32_t n_sl = a.slot_block ? (a.n_slots < a.cap ? a.n_slots : a.cap) : 0u;
    const uint32_t n_sl_lds = n_sl < SLOTS ? n_sl : SLOTS;
    // ---- phase A: every load issued before any use and none under a branch
    // (the compiler waits for all loads in flight at a branch's join): indices
    // are clamped, and absent inputs read a stand-in whose values are unused
    constexpr uint32_t SLT = SLOTS / NTH;
    const uint32_t *sbp = a.slot_block ? a.slot_block : a.n_tokens;
    const int32_t *sbb = a.slot_base ? a.slot_base : (const int32_t *)a.n_tokens;
    // blocks may move within the window (from the shadow of their old slot)
    const bool moves = a.stage_src && a.shadow_rows && a.slot_block;
    // (without moves the shadow counts are unused: the stand-in is the slot
    // map itself, which holds as many entries as the loop below reads)
    const uint32_t *srp = moves ? a.shadow_rows : sbp;
    const uint32_t nsl1 = n_sl_lds ? n_sl_lds - 1 : 0u, n1 = n ? n - 1 : 0u;
    const uint32_t *spp = a.pending_rows && a.slot_block ? a.pending_rows : sbp;
    uint32_t sl_blk[SLT], sl_rows[SLT], sl_pend[SLT];
    int32_t sl_base[SLT];
#pragma unroll
    for (uint32_t j = 0; j < SLT; ++j) {
        const uint32_t i = tid + j * NTH;
        sl_blk[j] = sbp[i < nsl1 ? i : nsl1];
        sl_base[j] = sbb[i < nsl1 ? i : nsl1];
        sl_rows[j] = srp[i < nsl1 ? i : nsl1];
        sl_pend[j] = spp[i < nsl1 ? i : nsl1];
    }
    const uint32_t kpt = (n + NTH - 1) / NTH;
    const bool have_ls = a.layer_score != nullptr, have_pr = have_ls && a.present != nullptr;
    const double *scp = have_ls ? a.layer_score : a.scores_in;
    const uint8_t *prp = have_pr ? a.present : (const uint8_t *)a.n_tokens;
    double sv[LOAD];
    uint64_t kr[LOAD];          // keys of blocks tid + NTH k (kept for the select)
    float sf[LOAD];             // their scores rounded to fp32
    uint32_t nt[LOAD];
    uint32_t pr[LOAD];
    // (unconditional, through a stand-in pointer: a load under a branch would be
    // waited for at the branch's join, ahead of the score loads)
    const uint32_t *qcp = have_ls ? a.q_count : a.n_tokens;
    const uint32_t qc0 = qcp[0];
#pragma unroll
    for (uint32_t k = 0; k < LOAD; ++k) {
        const uint32_t i = tid + k * NTH, ic = i < n1 ? i : n1;
        sv[k] = kvm_ld_f64_dev(scp + ic);
        nt[k] = a.n_tokens[ic];
        pr[k] = prp[ic];
    }
#pragma unroll
    for (uint32_t k = 0; k < LOAD; ++k) pr[k] = have_pr ? pr[k] : 1u;
#pragma unroll
    for (uint32_t j = 0; j < SLT; ++j) {
        const uint32_t i = tid + j * NTH;
        if (i < n_sl_lds) {
            s_sblk[i] = sl_blk[j];
            s_sbase[i] = sl_base[j];
            T.spend[i] = a.pending_rows ? sl_pend[j] : 0u;
        }
    }
    if (tid < 256) s_hist[0][tid] = 0;
    for (uint32_t i = tid; i < KVM_TOPK_FINE; i += NTH) s_fine[i] = 0;
    if (tid < KVM_TOPK_GATHER) s_rank[tid] = 0;
    if (tid == 0) {
        s_sel[3] = 0;
        s_prefix = 0;
        s_done = 0;
    }
    // With no mandatory ids the sink / recent pass (kvmem_store.cpp:520-545)
    // has a closed form: the sink_c oldest blocks (sink_c = min(sink, budget))
    // and, newest first, the recent blocks not in the sink while the budget
    // lasts, i.e. blocks [n - tail_c, n).  Every thread knows its own flags.
    const bool closed = !all && a.n_mand == 0;
    uint32_t sink_c = 0, tail_c = 0;
    if (closed) {
        const uint32_t sink = a.sink < n ? a.sink : n, recent = a.recent < n ? a.recent : n;
        sink_c = sink < a.budget ? sink : a.budget;
        const uint32_t lo = sink_c > n - recent ? sink_c : n - recent;
        tail_c = n - lo < a.budget - sink_c ? n - lo : a.budget - sink_c;
    }
    auto kept0 = [&](uint32_t i) { return all || (closed && (i < sink_c || i >= n - tail_c)); };
#pragma unroll
    for (uint32_t k = 0; k < LOAD; ++k) {
        const uint32_t i = tid + k * NTH;
        if (k < kpt && i < n) {
            double sc = sv[k];
            if (a.layer_score) {
                // average of the layers with queries, in layer order
                double acc = 0.0;
                uint32_t nlay = 0;
                if (qc0) { acc += sc; nlay++; }
                for (uint32_t il = 1; il < a.n_layer; ++il)
                    if (a.q_count[il]) { acc += kvm_ld_f64_dev(a.layer_score + (uint64_t)il * a.ls_cap + i); nlay++; }
                sc = nlay ? acc / (double)nlay : 0.0;
                if (!pr[k]) sc = 0.0;
                a.scores_out[i] = sc;
            }
            kr[k] = ord_key(sc);
            sf[k] = (float)sc;
            s_key[i] = kr[k];
            s_ntok[i] = nt[k];
            s_kept[i] = kept0(i) ? 1 : 0;
        }
    }
    KVM_LDS_BARRIER();
    const uint32_t per = (n + NTH - 1) / NTH;
    const uint32_t i0 = tid * per < n ? tid * per : n, i1 = i0 + per < n ? i0 + per : n;
    if (!all) {
        // sink prefix, mandatory ids newest first, recent tail (kvmem_store.cpp:520-545):
        // in closed form above, or one thread walks it when mandatory ids are given
        uint32_t count = sink_c + tail_c;
        if (!closed) {
            if (tid == 0) {
                uint32_t c = 0;
                const uint32_t sink = a.sink < n ? a.sink : n, recent = a.recent < n ? a.recent : n;
                for (uint32_t i = 0; i < sink && c < a.budget; ++i)
                    if (!s_kept[i]) { s_kept[i] = 1; ++c; }
                for (uint32_t i = a.n_mand; i > 0 && c < a.budget; --i) {
                    const uint32_t id = a.mandatory[i - 1];
                    if (id < n && !s_kept[id]) { s_kept[id] = 1; ++c; }
                }
                for (uint32_t i = 0; i < recent && c < a.budget; ++i) {
                    const uint32_t id = n - 1 - i;
                    if (!s_kept[id]) { s_kept[id] = 1; ++c; }
                }
                s_count = c;
            }
            KVM_LDS_BARRIER();
            count = s_count;
        }
        bool fallback = count < a.budget;
        if (count < a.budget) {
            // ---- one pass over a linear histogram of the fp32 scores.  Rounding
            // to fp32 and the bin map are monotonic, so a key in a higher bin is
            // larger; only the bin holding the need-th key is ranked exactly (by
            // 64-bit key, then id).  A crowded bin, or scores that are not finite,
            // fall back to the radix select below.
            constexpr uint32_t NW = NTH / 64;
            const uint32_t wid = tid >> 6;
            uint32_t cand = 0;
            float fmn = INFINITY, fmx = -INFINITY;
            uint32_t c = 0, kept_bits = 0;
            if (closed) {
#pragma unroll
                for (uint32_t k = 0; k < LOAD; ++k) kept_bits |= (uint32_t)kept0(tid + k * NTH) << k;
            } else {
#pragma unroll
                for (uint32_t k = 0; k < LOAD; ++k) {
                    const uint32_t i = tid + k * NTH;
                    kept_bits |= (uint32_t)(k < kpt && i < n && s_kept[i] != 0) << k;
                }
            }
#pragma unroll
            for (uint32_t k = 0; k < LOAD; ++k) {
                const uint32_t i = tid + k * NTH;
                if (k < kpt && i < n && !(kept_bits >> k & 1u)) {
                    cand |= 1u << k;
                    fmn = fminf(fmn, sf[k]);
                    fmx = sf[k] != sf[k] ? INFINITY : fmaxf(fmx, sf[k]);   // a NaN score: fall back
                    ++c;
                }
            }
            fmn = kvm_wave_min_f32(fmn);
            fmx = kvm_wave_max_f32(fmx);
            c = __builtin_amdgcn_readlane(kvm_wave_incl_scan(c), 63);
            if (lane == 0) {
                s_wmm[0][wid] = fmn;
                s_wmm[1][wid] = fmx;
                s_wc[wid] = c;
            }
            KVM_LDS_BARRIER();
            const float mn = kvm_wave_min_f32(lane < NW ? s_wmm[0][lane] : INFINITY);
            const float mx = kvm_wave_max_f32(lane < NW ? s_wmm[1][lane] : -INFINITY);
            const uint32_t ncand = __builtin_amdgcn_readlane(kvm_wave_incl_scan(lane < NW ? s_wc[lane] : 0u), 63);
            const uint32_t need = a.budget - count < ncand ? a.budget - count : ncand;
            const bool finite = mn >= -3.0e38f && mx <= 3.0e38f;
            if (need == ncand || finite) {
                const float sc = mx > mn ? (float)KVM_TOPK_FINE / (mx - mn) : 0.0f;
                auto bin_of = [&](float f) {
                    const float b = (f - mn) * sc;
                    return b >= (float)(KVM_TOPK_FINE - 1) ? KVM_TOPK_FINE - 1 : (b > 0.0f ? (uint32_t)b : 0u);
                };
                uint32_t T = 0, above = 0, cnt = ncand;
                if (need < ncand) {
#pragma unroll
                    for (uint32_t k = 0; k < LOAD; ++k)
                        if (cand >> k & 1u) {
                            const uint32_t b = bin_of(sf[k]);
                            atomicAdd(&s_fine[b], 1u);
                        }
                    KVM_LDS_BARRIER();
                    if (tid < 64) {
                        // coarse bin 63 - lane (descending) = its 16 fine bins, then
                        // the 16 fine bins of the one holding the need-th key
                        const kvm_u32x4 *fb = (const kvm_u32x4 *)&s_fine[(63 - lane) * 16];
                        const kvm_u32x4 f0 = fb[0], f1 = fb[1], f2 = fb[2], f3 = fb[3];
                        const kvm_u32x4 fs = f0 + f1 + f2 + f3;
                        const uint32_t cc = fs[0] + fs[1] + fs[2] + fs[3];
                        const uint32_t ci = kvm_wave_incl_scan(cc);
                        const uint64_t h1 = __builtin_amdgcn_ballot_w64(ci - cc < need && need <= ci);
                        const uint32_t l1 = (uint32_t)__builtin_ctzll(h1);
                        const uint32_t cb = 63u - l1, above_c = __builtin_amdgcn_readlane(ci - cc, l1);
                        const uint32_t cf = lane < 16 ? s_fine[cb * 16 + 15 - lane] : 0u;
                        const uint32_t fi = above_c + kvm_wave_incl_scan(cf);
                        const uint64_t h2 = __builtin_amdgcn_ballot_w64(fi - cf < need && need <= fi);
                        const uint32_t l2 = (uint32_t)__builtin_ctzll(h2);
                        if (lane == l2) {
                            s_sel[0] = cb * 16 + 15 - lane;
                            s_sel[1] = fi - cf;
                            s_sel[2] = cf;
                        }
                    }
                    KVM_LDS_BARRIER();
                    T = s_sel[0];
                    above = s_sel[1];
                    cnt = s_sel[2];
                }
                const uint32_t kk = need - above;      // keys still to take, from bin T
                if (kk == cnt || cnt <= KVM_TOPK_GATHER) {
                    fallback = false;
                    // keys above bin T are taken, and bin T whole when kk == cnt;
                    // otherwise its keys are gathered and ranked
                    // a wave reserves its gathered keys' slots with one atomic
#pragma unroll
                    for (uint32_t k = 0; k < LOAD; ++k) {
                        if (k >= kpt) break;                 // uniform: no thread holds block tid + NTH k
                        const bool ck = (cand >> k & 1u) != 0;
                        const uint32_t i = tid + k * NTH, b = ck && need != ncand ? bin_of(sf[k]) : 0u;
                        const bool take = ck && (need == ncand || b > T || (b == T && kk == cnt));
                        const bool gath = ck && !take && b == T;
                        if (take) s_kept[i] = 2;
                        const uint64_t gm = __builtin_amdgcn_ballot_w64(gath);
                        if (gm) {
                            const uint32_t lead = (uint32_t)__builtin_ctzll(gm);
                            uint32_t base = 0;
                            if (lane == lead) base = atomicAdd(&s_sel[3], (uint32_t)__builtin_popcountll(gm));
                            base = __builtin_amdgcn_readlane(base, lead);
                            const uint32_t below = __builtin_amdgcn_mbcnt_hi((uint32_t)(gm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)gm, 0u));
                            if (gath) s_gath[base + below] = kvm_u32x4{(uint32_t)kr[k], (uint32_t)(kr[k] >> 32), i, 0u};
                        }
                    }
                    if (kk != cnt) {
                        KVM_LDS_BARRIER();
                        // rank of entry j among the cnt gathered: keys larger, or equal
                        // with a larger id; thread (part, j) counts 4 of them
                        const uint32_t j = tid & (KVM_TOPK_GATHER - 1), part = tid / KVM_TOPK_GATHER;
                        constexpr uint32_t PER = KVM_TOPK_GATHER * KVM_TOPK_GATHER / NTH;
                        if (j < cnt) {
                            const kvm_u32x4 e = s_gath[j];
                            const uint64_t kj = (uint64_t)e[0] | ((uint64_t)e[1] << 32);
                            uint32_t r = 0;
#pragma unroll
                            for (uint32_t q = 0; q < PER; ++q) {
                                const uint32_t o = part * PER + q;
                                if (o < cnt) {
                                    const kvm_u32x4 x = s_gath[o];
                                    const uint64_t ko = (uint64_t)x[0] | ((uint64_t)x[1] << 32);
                                    r += ko > kj || (ko == kj && x[2] > e[2]);
                                }
                            }
                            if (r) atomicAdd(&s_rank[j], r);
                        }
                        KVM_LDS_BARRIER();
                        if (tid < cnt && s_rank[tid] < kk) s_kept[s_gath[tid][2]] = 2;
                    }
                    KVM_LDS_BARRIER();
                }
            }
        }
        if (fallback) {
            // radix passes: histogram into buffer p&1 -> barrier -> wave 0 picks
            // the bin and clears the other buffer -> barrier
            uint64_t mask = 0;
            uint32_t need = 1;                       // known after the first pass
            for (int shift = 56, p = 0; shift >= 0 && need; shift -= 8, ++p) {
                uint32_t *hist = s_hist[p & 1];
                const uint64_t prefix = s_prefix;
                for (uint32_t k = 0; k < per; ++k) {
                    const uint32_t i = i0 + k;
                    const bool act = i < i1 && !s_kept[i] && (s_key[i] & mask) == prefix;
                    hist_add(hist, act ? (uint32_t)(s_key[i] >> shift) & 255u : 0u, act);
                }
                KVM_LDS_BARRIER();
                if (tid < 64) {
                    // lane l owns bins 255-4l .. 252-4l (descending)
                    uint32_t c[4], tot = 0;
#pragma unroll
                    for (int j = 0; j < 4; ++j) { c[j] = hist[255 - 4 * lane - j]; tot += c[j]; }
                    const uint32_t incl = kvm_wave_incl_scan(tot);
                    uint32_t k;
                    if (p == 0) {
                        // candidates = keys in the first histogram
                        const uint32_t ncand = __builtin_amdgcn_readlane(incl, 63);
                        k = a.budget - count < ncand ? a.budget - count : ncand;
                        if (lane == 0) s_need = k;
                    } else {
                        k = s_k;
                    }
                    uint32_t run = incl - tot;           // keys in higher bins
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        if (run < k && k <= run + c[j]) {
                            s_prefix = prefix | ((uint64_t)(255 - 4 * lane - j) << shift);
                            s_k = k - run;
                            s_done = k - run == c[j];    // the whole bin is taken
                        }
                        run += c[j];
                    }
                    s_hist[(p + 1) & 1][4 * lane] = 0;
                    s_hist[(p + 1) & 1][4 * lane + 1] = 0;
                    s_hist[(p + 1) & 1][4 * lane + 2] = 0;
                    s_hist[(p + 1) & 1][4 * lane + 3] = 0;
                }
                mask |= (uint64_t)0xff << shift;
                KVM_LDS_BARRIER();
                need = s_need;
                if (s_done) break;
            }
            // keys above the bin are selected; a bin taken whole is selected;
            // otherwise (full 64-bit ties) the s_k highest ids among equal keys
            const uint64_t T = s_prefix;
            const uint32_t ktie = s_k;
            const bool whole = s_done;
            uint32_t ties = 0;
            if (!whole && need)
                for (uint32_t i = i0; i < i1; ++i) ties += !s_kept[i] && (s_key[i] & mask) == T;
            uint32_t before = 0, n_ties = 0, z0, z1;
            if (!whole && need) block_scan2<NTH>(ties, 0u, s_tmp[1], before, z0, n_ties, z1);
            for (uint32_t i = i0; i < i1 && need; ++i) {
                if (s_kept[i]) continue;
                const uint64_t km = s_key[i] & mask;
                if (km > T) {
                    s_kept[i] = 2;
                } else if (km == T) {
                    if (whole || n_ties - 1 - before < ktie) s_kept[i] = 2;     // rank by descending id
                    if (!whole) ++before;
                }
            }
            KVM_LDS_BARRIER();
        }
    }
    // ---- the old slot of every block the window holds with a complete shadow
    // (a full block), in the keys' buffer, which the selection no longer
    // reads: s_inv[b] = slot, or -1 for a slot whose shadow is incomplete.
    // Entries of blocks in no slot are not written; a lookup accepts slot j
    // only where the slot map names the block, so stale entries are harmless.
    int32_t *const s_inv = (int32_t *)T.key;
    if (moves) {
#pragma unroll
        for (uint32_t j = 0; j < SLT; ++j) {
            const uint32_t i = tid + j * NTH;
            if (i < n_sl_lds && sl_blk[j] < n) s_inv[sl_blk[j]] = sl_rows[j] == a.bt ? (int32_t)i : -1;
        }
        KVM_LDS_BARRIER();
    }
    // ---- ascending compaction with window positions: ranks and token
    // offsets of this thread's blocks come from one scan
    uint32_t local = 0, tok = 0;
    for (uint32_t i = i0; i < i1; ++i)
        if (s_kept[i]) { ++local; tok += s_ntok[i]; }
    uint32_t rank0, base0, n_sel, total;
    block_scan2<NTH>(local, tok, s_tmp[0], rank0, base0, n_sel, total);
    const bool fits = n_sel <= a.cap;
    const uint32_t ns = fits ? (n_sel < a.n_slots ? n_sel : a.n_slots) : 0;
    // slots whose (block, base) differ from the new layout; a plan that would
    // overwrite a slot holding unharvested rows is refused
    uint32_t need_mask = 0, need_local = 0, refuse = 0;
    if (fits) {
        uint32_t rank = rank0, base = base0, k = 0;
        for (uint32_t i = i0; i < i1; ++i) {
            if (!s_kept[i]) continue;
            a.ids[rank] = i;
            a.to_base[rank] = (int32_t)base;
            const bool in_lds = rank < n_sl_lds;
            if (rank < ns && (!a.slot_block ||
                              (in_lds ? s_sblk[rank] : a.slot_block[rank]) != i ||
                              (in_lds ? s_sbase[rank] : a.slot_base[rank]) != (int32_t)base)) {
                need_mask |= 1u << k;
                ++need_local;
                if (a.pending_rows && a.slot_block && (in_lds ? T.spend[rank] : a.pending_rows[rank]) != 0u) refuse = 1;
            }
            base += s_ntok[i];
            ++rank;
            ++k;
        }
    }
    // stage-out: the blocks of slots [tid * SLT, ...) of the plan's first
    // n_sl_lds slots that the selection does not keep, in slot order (the
    // chronological layout keeps blocks ascending)
    uint32_t out_local = 0;
    const uint32_t so0 = tid * SLT;
#pragma unroll
    for (uint32_t j = 0; j < SLT; ++j) {
        const uint32_t sl = so0 + j;
        const uint32_t b = sl < n_sl_lds ? s_sblk[sl] : 0xffffffffu;
        out_local += b < n && !s_kept[b] ? 1u : 0u;
    }
    uint32_t pos, out_pos, n_stage, n_out;
    block_scan2<NTH>(need_local, out_local, s_tmp[1], pos, out_pos, n_stage, n_out);
    if (a.stage_out && out_local) {
#pragma unroll
        for (uint32_t j = 0; j < SLT; ++j) {
            const uint32_t sl = so0 + j;
            const uint32_t b = sl < n_sl_lds ? s_sblk[sl] : 0xffffffffu;
            if (b < n && !s_kept[b] && out_pos < a.cap) a.stage_out[out_pos++] = b;
        }
    }
    refuse = __syncthreads_or(refuse) ? 1u : 0u;
    if (need_mask) {
        uint32_t rank = rank0, k = 0;
        for (uint32_t i = i0; i < i1; ++i) {
            if (!s_kept[i]) continue;
            if (need_mask >> k & 1u) {
                a.stage_slots[pos] = rank;
                if (a.stage_src) {
                    // a full block in a slot with a complete shadow moves from there
                    int32_t src = -1;
                    if (moves && s_ntok[i] == a.bt) {
                        const int32_t j = s_inv[i];
                        if (j >= 0 && (uint32_t)j < n_sl_lds && s_sblk[j] == i) src = j;
                    }
                    a.stage_src[pos] = src;
                }
                ++pos;
            }
            ++rank;
            ++k;
        }
    }
    const uint32_t status = (fits ? (n_sel <= a.n_slots || a.n_slots == 0 ? 0u : 2u) : 1u) | (refuse ? 4u : 0u);
    if (tid == 0) {
        a.info[0] = n_sel;
        a.info[1] = total;
        a.info[2] = n_stage;
        a.info[3] = status;
        a.info[4] = a.stage_out ? (n_out < a.cap ? n_out : a.cap) : 0u;
        a.info[5] = 0u;
        a.info[6] = 0u;
        a.info[7] = 0u;
    }
    return status ? 0u : n_stage;
}

// Host side (kvm_retrieval.hip): checks every lane's retrieval and fills its
// top-k arguments (nothing is launched); the scoring grid of the prepared
// lanes, whose per-layer contributions the top-k arguments read; the top-k
// kernel over them.
int kvm_retrieval_prepare(kvm_state *st, const kvm_retrieval_lane *lanes, uint32_t n_lanes, topk_lanes *tl);
int kvm_retrieval_score(kvm_state *st, const kvm_retrieval_lane *lanes, uint32_t n_lanes, const topk_lanes &tl);
// The scoring grid's arguments of prepared lanes (what kvm_retrieval_score
// launches), for a launch that scores them itself.
void kvm_retrieval_score_args(const kvm_retrieval_lane *lanes, uint32_t n_lanes, const topk_lanes &tl,
                              score_args *out);
int kvm_topk_launch(kvm_state *st, const topk_lanes &tl, uint32_t n_lanes);
// Checks a selection from caller scores (kvm_select_topk) and fills its top-k
// arguments; nothing is launched.
int kvm_select_prepare(kvm_state *st, const double *scores, const kvm_select_params *p, const kvm_window *w,
                       const kvm_selection *out, topk_args *ta);
