"""GPU parity of contains, assign and assign_values against the oracle."""
import numpy as np
import pytest

import oracle as O
from gpu_pair import Pair, to_dev, to_np
from helpers import uniform_keys, values_for

pytestmark = pytest.mark.gpu


def _pair(strategy, dim=16, **kw):
    p = Pair(1 << 13, dim=dim, strategy=strategy, **kw)
    if strategy in (O.EPOCH_LFU, O.EPOCH_LRU):
        p.set_global_epoch(4)
    return p


def _fill(p, rng, n=4000):
    ks = uniform_keys(rng, n)
    uses = p.strategy not in (O.LRU, O.EPOCH_LRU)
    sc = rng.integers(1, 1 << 30, size=n, dtype=np.uint64) if uses else None
    p.insert_or_assign(ks, values_for(ks, p.dim), sc, clock=20)
    return ks


@pytest.mark.parametrize("hybrid", [False, True])
def test_contains_matches_oracle(hybrid):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(1)
    p = _pair(O.CUSTOMIZED, max_hbm=(1 << 13) * 64 // 4 if hybrid else None)
    ks = _fill(p, rng)
    q = np.concatenate([ks[:2000], uniform_keys(rng, 1000, exclude=ks),
                        np.array([0xFFFFFFFFFFFFFFFF, 0xFFFFFFFFFFFFFFFD], np.uint64)])
    f = torch.zeros(q.size, dtype=torch.uint8, device="cuda")
    p.g.contains(q.size, to_dev(q), f)
    np.testing.assert_array_equal(to_np(f, np.uint8).astype(bool), p.o.contains(q))


@pytest.mark.parametrize("strategy", [O.LFU, O.CUSTOMIZED, O.LRU, O.EPOCH_LFU, O.EPOCH_LRU])
@pytest.mark.parametrize("dim", [16, 7])
def test_assign_matches_oracle(strategy, dim):
    rng = np.random.default_rng(2 + dim)
    p = _pair(strategy, dim=dim)
    ks = _fill(p, rng)
    q = np.concatenate([ks[1000:3000], uniform_keys(rng, 800, exclude=ks),
                        np.array([0xFFFFFFFFFFFFFFFF], np.uint64)])
    rng.shuffle(q)
    uses = strategy not in (O.LRU, O.EPOCH_LRU)
    sc = rng.integers(1, 1 << 30, size=q.size, dtype=np.uint64) if uses else None
    rows = rng.standard_normal((q.size, dim)).astype(np.float32)
    p.o.assign(q, rows, sc, clock=77)
    p.g.set_lru_clock(77)
    p.g.assign(q.size, to_dev(q), to_dev(rows), None if sc is None else to_dev(sc))
    p.assert_same_state()
    # assign_values: rows only
    rows2 = rng.standard_normal((q.size, dim)).astype(np.float32)
    p.o.assign_values(q, rows2)
    p.g.assign_values(q.size, to_dev(q), to_dev(rows2))
    p.assert_same_state()


def test_assign_hybrid_rows():
    # rows in pinned host slices: assign and assign_values write them in place
    rng = np.random.default_rng(13)
    p = _pair(O.LFU, dim=16, max_hbm=(1 << 13) * 64 // 4)
    assert not p.g.is_pure_hbm_mode()
    ks = _fill(p, rng)
    q = np.concatenate([ks[:2500], uniform_keys(rng, 500, exclude=ks)])
    sc = rng.integers(1, 1 << 30, size=q.size, dtype=np.uint64)
    rows = rng.standard_normal((q.size, 16)).astype(np.float32)
    p.o.assign(q, rows, sc)
    p.g.assign(q.size, to_dev(q), to_dev(rows), to_dev(sc))
    p.assert_same_state()
    rows2 = rng.standard_normal((q.size, 16)).astype(np.float32)
    p.o.assign_values(q, rows2)
    p.g.assign_values(q.size, to_dev(q), to_dev(rows2))
    p.assert_same_state()


@pytest.mark.parametrize("strategy", [O.LFU, O.CUSTOMIZED])
def test_assign_repeated_keys(strategy):
    # unique_key=False: scores apply in batch order (exact); for a repeated
    # key the row of one of its occurrences lands.
    rng = np.random.default_rng(9)
    p = _pair(strategy, dim=8)
    ks = _fill(p, rng, 3000)
    base = ks[:1500]
    q = np.concatenate([base, base[:500], base[:200]])
    rng.shuffle(q)
    sc = rng.integers(1, 1 << 20, size=q.size, dtype=np.uint64)
    rows = rng.standard_normal((q.size, 8)).astype(np.float32)
    p.o.assign(q, rows, sc)
    p.g.assign(q.size, to_dev(q), to_dev(rows), to_dev(sc), 0, False)
    (ok, ov, os_), (gk, gv, gs) = p.export()
    np.testing.assert_array_equal(gk, ok)
    np.testing.assert_array_equal(gs, os_)
    occ = {}
    for i, k in enumerate(q.tolist()):
        occ.setdefault(k, []).append(i)
    for j, k in enumerate(gk.tolist()):
        if k in occ:
            cands = rows[occ[k]]
            assert any(np.array_equal(gv[j], c) for c in cands)
        else:
            np.testing.assert_array_equal(gv[j], ov[j])
    assert p.g.size() == p.o.size() == 3000
