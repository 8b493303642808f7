"""Writes the golden fixtures of this directory from the oracle (the host
restatement of the reference table), on fixed seeds.

Each fixture is an .npz of plain arrays (no pickles): the inputs of a short
sequence of API calls and the expected outputs -- returned rows, founds,
evicted records and the table's slot-order export after the sequence.
tests/test_golden.py replays them on the oracle (CPU) and on the gfx950 table
(GPU).  Run from the repository root: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")]

import oracle as O  # noqa: E402
from helpers import keys_in_bucket, uniform_keys  # noqa: E402


def run_sequence(t, seq):
    """Applies `seq` (list of (op, args dict)) to oracle table t; returns the
    per-call outputs as a dict of arrays named after the call index."""
    out = {}
    for j, (op, a) in enumerate(seq):
        if op == "epoch":
            t.set_global_epoch(int(a["epoch"]))
        elif op == "insert_or_assign":
            t.insert_or_assign(a["keys"], a["values"], a.get("scores"),
                               bool(a["unique"]), False, int(a["clock"]))
        elif op == "find_or_insert":
            out[f"{j}_values"] = t.find_or_insert(a["keys"], a["values"], a.get("scores"),
                                                  bool(a["unique"]), False, int(a["clock"]))
        elif op == "insert_and_evict":
            k, v, s = t.insert_and_evict(a["keys"], a["values"], a.get("scores"),
                                         bool(a["unique"]), False, int(a["clock"]))
            o = np.lexsort((s, k))
            out[f"{j}_ev_keys"], out[f"{j}_ev_values"], out[f"{j}_ev_scores"] = k[o], v[o], s[o]
        elif op == "find":
            v, f, s = t.find(a["keys"], a["fill"].copy(), with_scores=True)
            out[f"{j}_values"], out[f"{j}_founds"], out[f"{j}_scores"] = v, f, np.where(f, s, 0)
        elif op == "erase":
            t.erase(a["keys"])
        elif op == "assign_scores":
            t.assign_scores(a["keys"], a.get("scores"), int(a["clock"]))
        elif op == "accum_or_assign":
            t.accum_or_assign(a["keys"], a["values"], a["flags"], a.get("scores"), False,
                              int(a["clock"]))
    k, v, s = t.export_batch(t.capacity(), 0)
    out["export_keys"], out["export_values"], out["export_scores"] = k, v, s
    out["size"] = np.array([t.size()], np.uint64)
    return out


def pack(name, table, seq, out):
    d = {"table": np.array([table["capacity"], table["max_capacity"], table["dim"],
                            table["strategy"]], np.uint64),
         "ops": np.array([op for op, _ in seq])}
    for j, (op, a) in enumerate(seq):
        for k, v in a.items():
            d[f"in{j}_{k}"] = np.asarray(v)
    for k, v in out.items():
        d[f"out_{k}"] = v
    np.savez_compressed(os.path.join(HERE, name), **d)


def fixtures():
    rng = np.random.default_rng(20240601)
    fx = []
    # config-1 shape at reduced size: Customized, 64 buckets, dim 4
    cap, dim = 1 << 13, 4
    allk = uniform_keys(rng, 4096)
    seq = []
    for b in range(4):
        ks = allk[b * 1024:(b + 1) * 1024]
        seq.append(("insert_or_assign", {
            "keys": ks, "values": rng.uniform(-1, 1, (ks.size, dim)).astype(np.float32),
            "scores": rng.integers(0, 2**64 - 1, ks.size, dtype=np.uint64),
            "unique": 1, "clock": 1}))
    q = np.concatenate([rng.choice(allk, 512, replace=False), uniform_keys(rng, 512, exclude=allk)])
    rng.shuffle(q)
    seq.append(("find", {"keys": q, "fill": np.full((q.size, dim), 7, np.float32)}))
    seq.append(("erase", {"keys": rng.choice(allk, 410, replace=False)}))
    seq.append(("find", {"keys": q, "fill": np.full((q.size, dim), 3, np.float32)}))
    fx.append(("golden_c1_small.npz",
               {"capacity": cap, "max_capacity": cap, "dim": dim, "strategy": O.CUSTOMIZED}, seq))
    # each strategy, 4 buckets filled well past full (evictions, tie-breaks)
    for st in (O.LRU, O.LFU, O.EPOCH_LRU, O.EPOCH_LFU, O.CUSTOMIZED):
        cap, dim = 512, 2
        seq = [("epoch", {"epoch": 3})]
        pool = uniform_keys(rng, 1500)
        for b in range(4):
            ks = pool[b * 300:(b + 1) * 300]
            sc = None if st in (O.LRU, O.EPOCH_LRU) else rng.integers(0, 40, ks.size, dtype=np.uint64)
            a = {"keys": ks, "values": rng.uniform(-1, 1, (ks.size, dim)).astype(np.float32),
                 "unique": 1, "clock": (b + 1) << 20}
            if sc is not None:
                a["scores"] = sc
            seq.append(("insert_or_assign", a))
        dup = rng.choice(pool[:1200], 400)
        a = {"keys": dup, "values": rng.uniform(-1, 1, (dup.size, dim)).astype(np.float32),
             "unique": 0, "clock": 9 << 20}
        if st not in (O.LRU, O.EPOCH_LRU):
            a["scores"] = rng.integers(0, 40, dup.size, dtype=np.uint64)
        seq.append(("find_or_insert", a))
        fx.append((f"golden_strategy_{st}.npz",
                   {"capacity": cap, "max_capacity": cap, "dim": dim, "strategy": st}, seq))
    # insert_and_evict with low scores refused and accum_or_assign (Customized)
    cap, dim = 4 * 128, 3
    hi = keys_in_bucket(rng, 128, cap, 1, lo=1, hi=10_000_000)
    lo = keys_in_bucket(rng, 64, cap, 1, lo=100_000_000, hi=200_000_000)
    seq = [("insert_and_evict", {"keys": hi, "values": rng.uniform(-1, 1, (128, dim)).astype(np.float32),
                                 "scores": np.arange(500, 628, dtype=np.uint64), "unique": 1, "clock": 1}),
           ("insert_and_evict", {"keys": lo, "values": rng.uniform(-1, 1, (64, dim)).astype(np.float32),
                                 "scores": np.arange(450, 514, dtype=np.uint64), "unique": 1, "clock": 2})]
    q = np.concatenate([hi[:40], lo[:40], uniform_keys(rng, 20)])
    seq.append(("accum_or_assign", {
        "keys": q, "values": rng.uniform(-0.01, 0.01, (q.size, dim)).astype(np.float32),
        "flags": (np.arange(q.size) % 3 != 0).astype(np.uint8),
        "scores": rng.integers(400, 700, q.size, dtype=np.uint64), "clock": 3}))
    seq.append(("assign_scores", {"keys": q[::2].copy(), "scores": rng.integers(0, 900, q[::2].size,
                                                                         dtype=np.uint64), "clock": 4}))
    fx.append(("golden_evict_accum.npz",
               {"capacity": cap, "max_capacity": cap, "dim": dim, "strategy": O.CUSTOMIZED}, seq))
    return fx


def main():
    for name, table, seq in fixtures():
        t = O.Oracle(table["capacity"], table["max_capacity"], dim=table["dim"],
                     strategy=table["strategy"])
        pack(name, table, seq, run_sequence(t, seq))
        print("wrote", name, os.path.getsize(os.path.join(HERE, name)), "bytes")


if __name__ == "__main__":
    main()
