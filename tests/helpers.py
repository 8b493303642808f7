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


def zipf_ranks(rng, n, alpha, universe):
    """n Zipf(alpha) ranks in [1, universe], by Hormann-Derflinger
    rejection-inversion ("Rejection-inversion to generate variates from
    monotone discrete distributions", ACM TOMACS 6(3), 1996), vectorised:
    candidates are drawn in bulk and rejected ones redrawn."""
    a = float(alpha)
    N = float(universe)

    def h(x):
        return np.exp(-a * np.log(x))

    def H(x):  # integral of h, written to stay exact as (1 - a) -> 0
        lx = np.log(x)
        t = (1.0 - a) * lx
        return np.where(np.abs(t) > 1e-8, np.expm1(t) / np.where(t == 0, 1, t), 1.0) * lx

    def H_inv(y):
        t = y * (1.0 - a)
        g = np.where(np.abs(t) > 1e-8, np.log1p(t) / np.where(t == 0, 1, t), 1.0)
        return np.exp(g * y)

    hx1 = float(H(np.array(1.5))) - 1.0
    hN = float(H(np.array(N + 0.5)))
    s = 2.0 - float(H_inv(H(np.array(2.5)) - h(np.array(2.0))))
    out = np.empty(n, np.uint64)
    todo = np.arange(n)
    while todo.size:
        u = hN + rng.random(todo.size) * (hx1 - hN)
        x = H_inv(u)
        k = np.clip(np.floor(x + 0.5), 1, N)
        ok = (k - x <= s) | (u >= H(k + 0.5) - h(k))
        out[todo[ok]] = k[ok].astype(np.uint64)
        todo = todo[~ok]
    return out


def scramble30(r):
    """A fixed bijection of [0, 2^30) (odd multiply, xor-shift, odd multiply),
    applied to rank - 1 so that a key's value says nothing of its rank."""
    m = np.uint64((1 << 30) - 1)
    x = (np.asarray(r, np.uint64) - np.uint64(1)) & m
    with np.errstate(over="ignore"):
        x = (x * np.uint64(0x2545F491)) & m
        x ^= x >> np.uint64(15)
        x = (x * np.uint64(0x1B873593)) & m
        x ^= x >> np.uint64(13)
    return x


def zipf_keys(rng, n, alpha=1.05, universe=1 << 30):
    return scramble30(zipf_ranks(rng, n, alpha, universe))


def uniform_keys_fast(rng, n):
    """n distinct non-reserved uniform uint64 keys (vectorised; for batches
    too large for uniform_keys' exclusion sets)."""
    out = np.empty(0, np.uint64)
    while out.size < n:
        c = rng.integers(0, 2**64, size=n - out.size + 64, dtype=np.uint64)
        c = c[(c & RESERVED_MASK) != RESERVED_MASK]
        out = np.unique(np.concatenate([out, c]))
    rng.shuffle(out)
    return out[:n].copy()
