"""Shared helpers for the test-suite (seeded key generators, comparisons)."""
import numpy as np

RESERVED_MASK = np.uint64(0xFFFFFFFFFFFFFFFC)
M1 = np.uint64(0xff51afd7ed558ccd)
M2 = np.uint64(0xc4ceb9fe1a85ec53)


def murmur3_np(k):
    """Vectorised MurmurHash3 fmix64 over a uint64 array."""
    k = np.asarray(k, dtype=np.uint64).copy()
    with np.errstate(over="ignore"):
        k ^= k >> np.uint64(33)
        k *= M1
        k ^= k >> np.uint64(33)
        k *= M2
        k ^= k >> np.uint64(33)
    return k


def uniform_keys(rng, n, exclude=None):
    """Unique uniform uint64 keys, none of them reserved (top 4 values)."""
    out = np.empty(0, np.uint64)
    seen = set() if exclude is None else set(int(x) for x in exclude)
    while out.size < n:
        c = rng.integers(0, 2**64, size=2 * (n - out.size), dtype=np.uint64,
                         endpoint=False)
        c = c[(c & RESERVED_MASK) != RESERVED_MASK]
        c = np.unique(c)
        if seen:
            c = np.array([x for x in c if int(x) not in seen], np.uint64)
        rng.shuffle(c)
        out = np.concatenate([out, c])
        out = out[np.sort(np.unique(out, return_index=True)[1])]
        seen.update(int(x) for x in c)
    return out[:n].copy()


def keys_in_bucket(rng, n, capacity, bucket, bucket_size=128, lo=0,
                   hi=0xFFFFFFFFFFFFFFFD):
    """`n` distinct keys in [lo, hi) whose bucket is `bucket` (power-of-2
    capacity), as the reference's create_keys_in_one_buckets builds them."""
    got = []
    seen = set()
    span = hi - lo
    while len(got) < n:
        c = rng.integers(0, 2**63, size=1 << 16, dtype=np.uint64)
        c = (c % np.uint64(span)) + np.uint64(lo)
        b = (murmur3_np(c) & np.uint64(capacity - 1)) // np.uint64(bucket_size)
        for x in c[b == np.uint64(bucket)]:
            if int(x) not in seen:
                seen.add(int(x))
                got.append(x)
                if len(got) == n:
                    break
    return np.array(got, np.uint64)


def values_for(keys, dim, dtype=np.float32):
    """Row i = key_i * 1e-5 in every column (the reference's fixture rule)."""
    return np.repeat((np.asarray(keys, np.float64) * 0.00001).astype(dtype)
                     [:, None], dim, axis=1)


def sort_records(keys, values, scores):
    o = np.argsort(keys, kind="stable")
    return keys[o], values[o], scores[o] if scores is not None else None
