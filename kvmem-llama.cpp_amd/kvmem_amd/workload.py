"""Deterministic synthetic workloads for the KVMem hot path.

Normal variates: a counter-based splitmix64 stream, two 53-bit uniforms per
value, Box-Muller in double, rounded to fp32.  Value k of stream `seed` is a
pure function of (seed, k), so any slice can be regenerated independently.
"""
import numpy as np

_GOLD = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)

SEEDS = {"cfg1": 0xC0FFEE01, "cfg2": 0xC0FFEE02, "cfg3": 0xC0FFEE03, "cfg4": 0xC0FFEE04,
         "cfg5": 0xC0FFEE05}


def splitmix64(seed, idx):
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + (idx.astype(np.uint64) + np.uint64(1)) * _GOLD
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def normals(seed, offset, n, chunk=1 << 22):
    """n standard normals (fp32) of stream `seed` starting at value index `offset`."""
    out = np.empty(n, dtype=np.float32)
    for s in range(0, n, chunk):
        k = np.arange(offset + s, offset + min(n, s + chunk), dtype=np.uint64)
        a = splitmix64(seed, np.uint64(2) * k)
        b = splitmix64(seed, np.uint64(2) * k + np.uint64(1))
        u1 = ((a >> np.uint64(11)).astype(np.float64) + 1.0) * (2.0 ** -53)
        u2 = (b >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)
        out[s:s + len(k)] = (np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)).astype(np.float32)
    return out


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
