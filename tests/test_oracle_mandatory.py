"""Mandatory blocks of a retrieval (llama-memory-kvmem.cpp:4306-4325): the
oracle against brute force on the reference store's own block layout and its
block_id_containing (oracle/_ref, where the reference sources are present),
and the library's host entry point kvm_retrieval_mandatory against the oracle."""
import numpy as np
import pytest

import oracle as O
from kvmem_amd import api

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (needs the reference sources)")


def _brute(n_tokens, spans, query_begin, query_end, force_pos):
    """Position by position: a block is mandatory if any position it holds lies in a range."""
    starts = np.concatenate([[0], np.cumsum(n_tokens)[:-1]]).astype(np.int64)
    total = int(np.sum(n_tokens))
    ranges = list(spans) if spans is not None else ([(query_begin, query_end if query_end > 0 else total)]
                                                    if query_begin >= 0 else [])
    ids = [b for b, (s, n) in enumerate(zip(starts, n_tokens))
           if any(any(r0 <= p < r1 for r0, r1 in ranges) for p in range(s, s + n))]
    if 0 <= force_pos < total:
        ids.append(int(np.searchsorted(starts, force_pos, side="right") - 1))
    return np.array(ids, np.int64)


KATS = [
    # (n_tokens, spans, query_begin, query_end, force_pos, expected)
    ([128] * 10 + [77], [(200, 300)], -1, 0, 1000, [1, 2, 7]),
    ([128] * 10 + [77], None, 1200, 0, -1, [9, 10]),            # query span to the store's end
    ([128] * 10 + [77], None, 1200, 1290, 5, [9, 10, 0]),
    ([128] * 10 + [77], [(0, 1), (1279, 1290)], -1, 0, 5000, [0, 9, 10]),   # force_pos past the end: none
    ([128] * 4, [(128, 128)], 5, 0, 130, [1]),                  # empty span; spans override the query span
    ([128] * 4, [(100, 140)], -1, 0, 130, [0, 1, 1]),           # force_pos block listed again
    ([], [(0, 10)], 0, 0, 0, []),
    # an inverted query span: the reference's overlap test (block end > begin and
    # block start < end) still keeps the block that straddles it
    ([128] * 10, None, 950, 930, -1, [7]),
    # the turn set explicit spans, none of them mandatory: the query span does
    # not stand in (explicit_spans_ with an empty turn_spans_.mandatory), only
    # the force_pos block is kept
    ([128] * 4, [], 5, 0, 130, [1]),
    ([128] * 4, [], 5, 0, -1, []),
]


@pytest.mark.parametrize("case", range(len(KATS)))
def test_known_answers(case):
    nt, spans, qb, qe, fp, want = KATS[case]
    assert list(O.retrieval_mandatory(nt, spans, qb, qe, fp)) == want
    assert list(api.retrieval_mandatory(nt, spans, qb, qe, fp)) == want
    if qe <= 0 or qe >= qb:
        assert list(_brute(np.array(nt, np.int64), spans, qb, qe, fp)) == want


@needs_ref
def test_oracle_on_the_reference_store_layout():
    rng = np.random.default_rng(3)
    for _ in range(60):
        appends = rng.integers(1, 400, rng.integers(1, 8))
        pos = rng.integers(-5, int(appends.sum()) + 5, 6)
        starts, nt, containing = O.ref_block_layout(appends, 128, pos)
        assert np.array_equal(starts, np.concatenate([[0], np.cumsum(nt)[:-1]]))
        for p, c in zip(pos, containing):                       # force_pos alone
            got = O.retrieval_mandatory(nt, None, -1, 0, int(p))
            assert list(got) == ([] if c < 0 else [c])
        spans = [tuple(sorted(rng.integers(-3, int(appends.sum()) + 3, 2))) for _ in range(rng.integers(0, 4))]
        spans = None if not spans and rng.random() < 0.5 else spans
        qb, fp = int(rng.integers(-1, 300)), int(pos[0])
        qe = int(rng.integers(qb, 600)) if qb >= 0 and rng.random() < 0.7 else 0
        assert np.array_equal(O.retrieval_mandatory(nt, spans, qb, qe, fp), _brute(nt, spans, qb, qe, fp))


def test_library_matches_oracle():
    rng = np.random.default_rng(4)
    for _ in range(300):
        nb = int(rng.integers(0, 40))
        nt = np.full(nb, 128, np.int64)
        if nb:
            nt[-1] = rng.integers(1, 129)
        total = int(nt.sum())
        spans = [tuple(sorted(rng.integers(-10, total + 10, 2))) for _ in range(rng.integers(0, 5))]
        spans = None if not spans and rng.random() < 0.5 else spans
        qb, qe, fp = int(rng.integers(-2, total + 2)), int(rng.integers(-1, total + 2)), int(rng.integers(-2, total + 3))
        want = O.retrieval_mandatory(nt, spans, qb, qe, fp)
        assert np.array_equal(api.retrieval_mandatory(nt, spans, qb, qe, fp), want)
        if qe <= 0 or qe >= qb:                      # brute force knows no inverted span
            assert np.array_equal(want, _brute(nt, spans, qb, qe, fp))


def test_library_refuses_a_small_output():
    lib = api.L.load()
    nt = np.full(5, 128, np.uint32)
    out = np.zeros(2, np.uint32)
    n = api.L._u32(0)
    rr = (api.L.RowRange * 1)(api.L.RowRange(0, 640))
    assert lib.kvm_retrieval_mandatory(None, nt.ctypes.data, 5, rr, 1, -1, 0, -1, out.ctypes.data, 2,
                                       api.C.byref(n)) == api.L.KVM_ERANGE
