"""Deterministic block choices for the synthetic workloads (the planted
blocks of the decode step, the stage-in's selected blocks): a counter-based
splitmix64 stream, so value k of stream `seed` is a pure function of
(seed, k)."""
import numpy as np

_GOLD = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)

def splitmix64(seed, idx):
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + (idx.astype(np.uint64) + np.uint64(1)) * _GOLD
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform_ints(seed, offset, n, hi):
    """n integers uniform in [0, hi) (multiply-shift on 32 random bits)."""
    k = np.arange(offset, offset + n, dtype=np.uint64)
    z = splitmix64(seed, k) >> np.uint64(32)
    return ((z * np.uint64(hi)) >> np.uint64(32)).astype(np.int64)


def distinct_ids(seed, offset, count, lo, hi):
    """`count` distinct integers in [lo, hi), drawn in stream order (rejection of repeats)."""
    got, seen, k = [], set(), offset
    while len(got) < count:
        batch = uniform_ints(seed, k, 4 * count, hi - lo) + lo
        k += 4 * count
        for v in batch.tolist():
            if v not in seen:
                seen.add(v)
                got.append(v)
                if len(got) == count:
                    break
    return np.array(got, dtype=np.int64)
