"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py
from the oracle on fixed seeds): short call sequences with their expected
outputs.  The CPU test pins the oracle to the committed vectors (any change
to its semantics shows up here); the GPU test replays the same inputs on the
gfx950 table through the C ABI and compares with the vectors alone, with no
oracle in the loop."""
import glob
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import oracle as O  # noqa: E402
from make_golden import run_sequence  # noqa: E402

FILES = sorted(glob.glob(os.path.join(HERE, "golden", "golden_*.npz")))


def load(path):
    d = np.load(path)  # plain arrays only (allow_pickle stays False)
    cap, mcap, dim, st = (int(x) for x in d["table"])
    seq = []
    for j, op in enumerate(d["ops"]):
        pre = f"in{j}_"
        seq.append((str(op), {k[len(pre):]: d[k] for k in d.files if k.startswith(pre)}))
    out = {k[4:]: d[k] for k in d.files if k.startswith("out_")}
    return (cap, mcap, dim, st), seq, out


def test_fixtures_present():
    assert len(FILES) >= 7


@pytest.mark.parametrize("path", FILES, ids=os.path.basename)
def test_oracle_reproduces_golden(path):
    (cap, mcap, dim, st), seq, want = load(path)
    t = O.Oracle(cap, mcap, dim=dim, strategy=st)
    got = run_sequence(t, seq)
    assert set(got) == set(want)
    for k in want:
        np.testing.assert_array_equal(np.asarray(got[k]).view(np.uint8),
                                      want[k].view(np.uint8), err_msg=k)


@pytest.mark.gpu
@pytest.mark.parametrize("path", FILES, ids=os.path.basename)
def test_gpu_matches_golden(path):
    import torch
    import hkv_amd
    from gpu_pair import records_equal, to_dev, to_np
    (cap, mcap, dim, st), seq, want = load(path)
    g = hkv_amd.HashTable("u64", "f32", st)
    g.init(hkv_amd.HashTableOptions(init_capacity=cap, max_capacity=mcap,
                                    max_hbm_for_vectors=1 << 40, dim=dim))

    def sc(a):
        return to_dev(a["scores"]) if "scores" in a else None
    for j, (op, a) in enumerate(seq):
        if op == "epoch":
            g.set_global_epoch(int(a["epoch"]))
            continue
        if "clock" in a:
            g.set_lru_clock(int(a["clock"]))
        k = a.get("keys")
        n = 0 if k is None else k.size
        if op == "insert_or_assign":
            g.insert_or_assign(n, to_dev(k), to_dev(a["values"]), sc(a), 0, bool(a["unique"]))
        elif op == "find_or_insert":
            v = to_dev(a["values"])
            g.find_or_insert(n, to_dev(k), v, sc(a), 0, bool(a["unique"]))
            np.testing.assert_array_equal(to_np(v, np.float32).reshape(n, dim),
                                          want[f"{j}_values"])
        elif op == "insert_and_evict":
            ek = torch.zeros(n, dtype=torch.int64, device="cuda")
            ev = torch.zeros((n, dim), dtype=torch.float32, device="cuda")
            es = torch.zeros(n, dtype=torch.int64, device="cuda")
            c = g.insert_and_evict(n, to_dev(k), to_dev(a["values"]), sc(a), ek, ev, es,
                                   None, 0, bool(a["unique"]))
            records_equal((want[f"{j}_ev_keys"], want[f"{j}_ev_values"], want[f"{j}_ev_scores"]),
                          (to_np(ek, np.uint64)[:c], to_np(ev, np.float32).reshape(n, dim)[:c],
                           to_np(es, np.uint64)[:c]))
        elif op == "find":
            v = to_dev(a["fill"])
            f = torch.zeros(n, dtype=torch.uint8, device="cuda")
            s = torch.zeros(n, dtype=torch.int64, device="cuda")
            g.find(n, to_dev(k), v, f, s)
            fn = to_np(f, np.uint8).astype(bool)
            np.testing.assert_array_equal(fn, want[f"{j}_founds"])
            np.testing.assert_array_equal(to_np(v, np.float32).reshape(n, dim), want[f"{j}_values"])
            np.testing.assert_array_equal(np.where(fn, to_np(s, np.uint64), 0), want[f"{j}_scores"])
        elif op == "erase":
            g.erase(n, to_dev(k))
        elif op == "assign_scores":
            g.assign_scores(n, to_dev(k), sc(a))
        elif op == "accum_or_assign":
            g.accum_or_assign(n, to_dev(k), to_dev(a["values"]), to_dev(a["flags"]), sc(a))
    c = g.capacity()
    ek = torch.zeros(c, dtype=torch.int64, device="cuda")
    ev = torch.zeros((c, dim), dtype=torch.float32, device="cuda")
    es = torch.zeros(c, dtype=torch.int64, device="cuda")
    m = g.export_batch(c, 0, ek, ev, es)
    np.testing.assert_array_equal(to_np(ek, np.uint64)[:m], want["export_keys"])
    np.testing.assert_array_equal(to_np(es, np.uint64)[:m], want["export_scores"])
    np.testing.assert_array_equal(to_np(ev, np.float32).reshape(c, dim)[:m], want["export_values"])
    assert g.size() == int(want["size"][0])
