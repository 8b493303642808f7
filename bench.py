"""Benchmark: find and insert_or_assign on one MI355X.

Workload (the headline lookup/upsert shape): kLru table, capacity 2^26 slots
in 128-slot buckets, dim 64 fp32 values all in HBM, batches of 2^20
uniform-random uint64 keys.  One step = insert_or_assign of one batch of new
keys + find of one batch of resident keys (100% hit).  The table is filled
so that the load factor crosses 0.5 in the middle of the timed steps.
Inputs are resident in HBM before timing starts.

Prints one JSON line.  Also reported: insert_or_assign and find (100% and
0% hit, plain and missed-keys overloads) at load factors 0.75 and 1.0, the
other benchmark configurations, and the host reference (the oracle) timed on
a bounded sample of the same workload at one thread and at all threads.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "hierarchicalkv-ascend_amd"))

METRIC = ("find & insert_or_assign Mkeys/s at cap 64M dim 64, lf 0.5/1.0; "
          "% HBM peak")
HBM_PEAK_GBS = 8000.0
S = 64          # bytes charged per random touch of bucket metadata
CAP = 1 << 26
DIM = 64
BATCH = 1 << 20


# HBM bytes per key that each operation's kernels move at this workload,
# measured by rocprofv3 FETCH_SIZE and WRITE_SIZE passes (scaled by what the
# same counters read for a plain 1 GiB device copy) and kept, with the
# command that measured them, in profiles/hbm_traffic.json.
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic.json")


def measured_bytes_per_key(op):
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)["bytes_per_key"][op]
    except (OSError, KeyError, ValueError):
        return None


def algo_bytes(op, dim=DIM):
    """Algorithmic bytes per key (fixed model: S per random metadata touch,
    x2 when read-modify-write; V = 4*dim per row direction)."""
    V = 4 * dim
    return {
        "find_hit": 9 + 2 * S + 2 * V,
        "find_miss": 9 + S,
        "insert_new": 8 + 2 * V + 8 * S,
        "insert_evict": 8 + 2 * V + 8 * S + 2048,
    }[op]


def rand_keys(torch, n, gen):
    k = torch.randint(-(2**63), 2**63 - 1, (n,), dtype=torch.int64,
                      device="cuda", generator=gen)
    # Reserved keys are 0xFFFFFFFFFFFFFFFC..FF (-4..-1 as int64).
    bad = (k >= -4) & (k < 0)
    return torch.where(bad, k - 4, k)


def zipf_keys_gpu(torch, n, gen, alpha=1.05, universe=1 << 30):
    """n Zipf(alpha) keys over [0, universe) on the GPU: Hormann-Derflinger
    rejection-inversion ranks, mapped through a fixed bijection of the
    30-bit range so that a key's value says nothing of its rank."""
    a, N = alpha, float(universe)
    one = torch.ones((), dtype=torch.float64, device="cuda")

    def H(x):
        lx = torch.log(x)
        t = (1.0 - a) * lx
        return torch.expm1(t) / t * lx

    def H_inv(y):
        t = y * (1.0 - a)
        return torch.exp(torch.log1p(t) / t * y)

    hx1 = float(H(one * 1.5)) - 1.0
    hN = float(H(one * (N + 0.5)))
    s_ = 2.0 - float(H_inv(H(one * 2.5) - 2.0 ** -a))
    out = torch.empty(n, dtype=torch.int64, device="cuda")
    todo = torch.arange(n, device="cuda")
    while todo.numel():
        u = hN + torch.rand(todo.numel(), dtype=torch.float64, device="cuda",
                            generator=gen) * (hx1 - hN)
        x = H_inv(u)
        k = torch.clamp(torch.floor(x + 0.5), 1, N)
        ok = (k - x <= s_) | (u >= H(k + 0.5) - torch.exp(-a * torch.log(k)))
        out[todo[ok]] = k[ok].to(torch.int64)
        todo = todo[~ok]
    m = (1 << 30) - 1
    x = (out - 1) & m
    x = (x * 0x2545F491) & m
    x ^= x >> 15
    x = (x * 0x1B873593) & m
    x ^= x >> 13
    return x


def _events(torch, k):
    return [torch.cuda.Event(enable_timing=True) for _ in range(k)]


def bench_c3(torch, hkv_amd, stream, gen, batches=200):
    """kEpochLfu, capacity 2^27, dim 32: find_or_insert of 2^20 Zipf(1.05)
    keys per batch (duplicates: unique_key=false, score increment 1),
    epoch + 1 every 10 batches."""
    cap, dim, B = 1 << 27, 32, 1 << 20
    t = hkv_amd.HashTable("u64", "f32", hkv_amd.EvictStrategy.kEpochLfu)
    t.init(hkv_amd.HashTableOptions(init_capacity=cap, max_capacity=cap,
                                    max_hbm_for_vectors=cap * dim * 4, dim=dim))
    keys = [zipf_keys_gpu(torch, B, gen) for _ in range(batches)]
    vals = torch.rand((B, dim), device="cuda", generator=gen)
    ones = torch.ones(B, dtype=torch.int64, device="cuda")
    ev = _events(torch, 2 * batches)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for b in range(batches):
            t.set_global_epoch(b // 10)
            ev[2 * b].record(stream)
            t.find_or_insert(B, keys[b], vals, ones, stream, False)
            ev[2 * b + 1].record(stream)
    torch.cuda.synchronize()
    ms = [ev[2 * b].elapsed_time(ev[2 * b + 1]) for b in range(batches)]
    size = t.size()
    del t, keys
    tot = sum(ms)
    return {"op": "find_or_insert (unique_key=false)", "batches": batches,
            "mkeys_s": round(B * batches / tot / 1e3, 1),
            "ms_per_batch_mean": round(tot / batches, 4),
            "ms_last_10": round(sum(ms[-10:]) / 10, 4), "final_size": size}


def bench_c4(torch, hkv_amd, stream, gen, reps=3):
    """kLfu, capacity 2^26, dim 128, prefilled to load factor 1.0 with uint32
    scores: insert_and_evict, accum_or_assign and assign_scores on 2^20-key
    batches of 50% new / 50% resident keys."""
    cap, dim, B = 1 << 26, 128, 1 << 20
    t = hkv_amd.HashTable("u64", "f32", hkv_amd.EvictStrategy.kLfu)
    t.init(hkv_amd.HashTableOptions(init_capacity=cap, max_capacity=cap,
                                    max_hbm_for_vectors=cap * dim * 4, dim=dim))
    vals = torch.rand((B, dim), device="cuda", generator=gen) * 2 - 1

    def u32s(n):
        return torch.randint(0, 1 << 32, (n,), dtype=torch.int64, device="cuda",
                             generator=gen)
    with torch.cuda.stream(stream):
        guard = 0
        filled = []
        while t.size(stream) < cap and guard < 200:
            ks = rand_keys(torch, B, gen)
            t.insert_or_assign(B, ks, vals, u32s(B), stream)
            filled.append(ks)
            guard += 1
        filled = torch.cat(filled)
        fv = torch.empty((2 * B, dim), dtype=torch.float32, device="cuda")
        ff = torch.empty(2 * B, dtype=torch.uint8, device="cuda")
        ek = torch.empty(B, dtype=torch.int64, device="cuda")
        evv = torch.empty((B, dim), dtype=torch.float32, device="cuda")
        es = torch.empty(B, dtype=torch.int64, device="cuda")
        cnt = torch.zeros(1, dtype=torch.int64, device="cuda")

        def mixed():
            # resident keys drawn uniformly: prefill keys that find reports
            cand = filled[torch.randint(0, filled.numel(), (2 * B,), device="cuda",
                                        generator=gen)]
            t.find(2 * B, cand, fv, ff, None, stream)
            res = torch.unique(cand[ff.bool()])
            res = res[torch.randperm(res.numel(), device="cuda", generator=gen)[:B // 2]]
            q = torch.cat([res, rand_keys(torch, B - res.numel(), gen)])
            fl = torch.cat([torch.ones(res.numel(), dtype=torch.uint8, device="cuda"),
                            torch.zeros(B - res.numel(), dtype=torch.uint8, device="cuda")])
            perm = torch.randperm(B, device="cuda", generator=gen)
            return q[perm], fl[perm]  # accumulate resident keys, assign new ones
        out = {}
        for name in ("insert_and_evict", "accum_or_assign", "assign_scores"):
            qs = [mixed() for _ in range(reps)]
            sc = [u32s(B) for _ in range(reps)]
            deltas = (torch.rand((B, dim), device="cuda", generator=gen) * 0.02 - 0.01)
            torch.cuda.synchronize()
            e = _events(torch, 2 * reps)
            n_ev = 0
            for r in range(reps):
                q, fl = qs[r]
                e[2 * r].record(stream)
                if name == "insert_and_evict":
                    cnt.zero_()
                    t.insert_and_evict(B, q, vals, sc[r], ek, evv, es, cnt, stream)
                elif name == "accum_or_assign":
                    t.accum_or_assign(B, q, deltas, fl, sc[r], stream)
                else:
                    t.assign_scores(B, q, sc[r], stream)
                e[2 * r + 1].record(stream)
            torch.cuda.synchronize()
            if name == "insert_and_evict":
                n_ev = int(cnt.item())
            ms = sum(e[2 * r].elapsed_time(e[2 * r + 1]) for r in range(reps)) / reps
            out[name] = {"mkeys_s": round(B / ms / 1e3, 1), "ms": round(ms, 4)}
            if name == "insert_and_evict":
                out[name]["evicted_last_batch"] = n_ev
                # half the keys evict: model bytes (evicting upsert + victim
                # row out + record) for them, present-key upsert for the rest
                V = 4 * dim
                b_ev = 8 + 2 * V + 8 * S + 2048 + 8 + V + 16
                b_hit = 8 + 2 * V + 6 * S + 8
                gbs = (b_ev + b_hit) / 2 * B / (ms * 1e-3) / 1e9
                out[name]["algo_gbs"] = round(gbs, 1)
                out[name]["frac_hbm"] = round(gbs / HBM_PEAK_GBS, 4)
    del t, filled, fv
    return out


def bench_c5(torch, hkv_amd, stream, gen):
    """kCustomized, init 2^27 growing to 2^28, dim 64, max_hbm_for_vectors
    16 GiB (after growth 3/4 of the rows are pinned host memory): fill with
    2^20-key insert_or_assign batches until auto-growth, time the growing
    call, mixed find / insert_or_assign batches, then export_batch over the
    whole table in 2^22-slot chunks."""
    init, mx, dim, B = 1 << 27, 1 << 28, 64, 1 << 20
    t = hkv_amd.HashTable("u64", "f32", hkv_amd.EvictStrategy.kCustomized)
    t.init(hkv_amd.HashTableOptions(init_capacity=init, max_capacity=mx,
                                    max_hbm_for_vectors=16 << 30, dim=dim))
    vals = torch.rand((B, dim), device="cuda", generator=gen) * 2 - 1
    out_v = torch.empty((B, dim), dtype=torch.float32, device="cuda")
    fnd = torch.empty(B, dtype=torch.uint8, device="cuda")
    res = {}
    with torch.cuda.stream(stream):
        inserted = []
        grow_ms = None
        for b in range(80):
            ks = rand_keys(torch, B, gen)
            sc = torch.randint(0, 1 << 62, (B,), dtype=torch.int64, device="cuda",
                               generator=gen)
            cap0 = t.capacity()
            torch.cuda.synchronize()
            a = time.perf_counter()
            t.insert_or_assign(B, ks, vals, sc, stream)
            torch.cuda.synchronize()
            dt = (time.perf_counter() - a) * 1e3
            if t.capacity() != cap0:
                grow_ms = round(dt, 2)
            inserted.append(ks)
            if t.capacity() == mx and b >= 70:
                break
        res["growth_call_ms"] = grow_ms
        res["capacity"] = t.capacity()
        allk = torch.cat(inserted)
        e = _events(torch, 8)
        for r in range(4):
            q = allk[torch.randint(0, allk.numel(), (B,), device="cuda", generator=gen)]
            ks = rand_keys(torch, B, gen)
            sc = torch.randint(0, 1 << 62, (B,), dtype=torch.int64, device="cuda",
                               generator=gen)
            torch.cuda.synchronize()
            e[0].record(stream)
            t.find(B, q, out_v, fnd, None, stream)
            e[1].record(stream)
            t.insert_or_assign(B, ks, vals, sc, stream)
            e[2].record(stream)
            torch.cuda.synchronize()
            if r == 3:
                res["find_ms"] = round(e[0].elapsed_time(e[1]), 4)
                res["insert_or_assign_ms"] = round(e[1].elapsed_time(e[2]), 4)
        res["find_mkeys_s"] = round(B / res["find_ms"] / 1e3, 1)
        res["insert_or_assign_mkeys_s"] = round(B / res["insert_or_assign_ms"] / 1e3, 1)
        C = 1 << 22
        ek = torch.empty(C, dtype=torch.int64, device="cuda")
        ev = torch.empty((C, dim), dtype=torch.float32, device="cuda")
        es = torch.empty(C, dtype=torch.int64, device="cuda")
        cnt = torch.zeros(1, dtype=torch.int64, device="cuda")
        total = 0
        torch.cuda.synchronize()
        a = time.perf_counter()
        for off in range(0, t.capacity(), C):
            t.export_batch(C, off, ek, ev, es, cnt, stream)
        torch.cuda.synchronize()
        dt = time.perf_counter() - a
        total = t.size(stream)
        res["export_s"] = round(dt, 4)
        res["export_gbs"] = round(total * (8 + 4 * dim + 8) / dt / 1e9, 1)
        res["size"] = total
        # host link ceiling for the host-resident rows
        h = torch.empty(1 << 28, dtype=torch.float32, pin_memory=True)
        d = torch.empty(1 << 28, dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        a = time.perf_counter()
        d.copy_(h, non_blocking=True)
        torch.cuda.synchronize()
        res["h2d_gbs"] = round((1 << 30) / (time.perf_counter() - a) / 1e9, 1)
        a = time.perf_counter()
        h.copy_(d, non_blocking=True)
        torch.cuda.synchronize()
        res["d2h_gbs"] = round((1 << 30) / (time.perf_counter() - a) / 1e9, 1)
        del h, d
    del t
    return res


def bench_at_load_factor(torch, hkv_amd, stream, gen, target, calls=3):
    """The headline table (kLru, 2^26 slots, dim 64) filled with batches of
    2^20 new keys to the load factor `target`, then `calls` insert_or_assign
    calls of new keys and `calls` find calls of keys just inserted, each
    timed with events on the stream they run on.  Counter passes read the
    last `calls` dispatches of each kernel."""
    t = hkv_amd.HashTable("u64", "f32", hkv_amd.EvictStrategy.kLru)
    t.init(hkv_amd.HashTableOptions(init_capacity=CAP, max_capacity=CAP,
                                    max_hbm_for_vectors=CAP * DIM * 4, dim=DIM))
    vals = torch.rand((BATCH, DIM), device="cuda", generator=gen) * 2 - 1
    out = torch.empty((BATCH, DIM), dtype=torch.float32, device="cuda")
    fnd = torch.empty(BATCH, dtype=torch.uint8, device="cuda")
    with torch.cuda.stream(stream):
        guard = 0
        while t.load_factor(stream) < target - 1e-9 and guard < 200:
            if target < 1.0 and t.load_factor(stream) + BATCH / CAP > target:
                break
            t.insert_or_assign(BATCH, rand_keys(torch, BATCH, gen), vals, None, stream)
            guard += 1
        lf0 = t.load_factor(stream)
        ks = [rand_keys(torch, BATCH, gen) for _ in range(calls)]
        e = _events(torch, 2 * calls + 1)
        torch.cuda.synchronize()
        for r in range(calls):
            e[r].record(stream)
            t.insert_or_assign(BATCH, ks[r], vals, None, stream)
        e[calls].record(stream)
        for r in range(calls):
            t.find(BATCH, ks[r], out, fnd, None, stream)
            e[calls + 1 + r].record(stream)
        torch.cuda.synchronize()
    ins = [e[r].elapsed_time(e[r + 1]) for r in range(calls)]
    fi = [e[calls + r].elapsed_time(e[calls + 1 + r]) for r in range(calls)]
    del t
    return {"load_factor_at_start": round(lf0, 4),
            "insert_or_assign_ms": [round(x, 4) for x in ins],
            "find_hit_ms": [round(x, 4) for x in fi], "hits_last": int(fnd.sum().item())}


def run_configs(torch, hkv_amd, stream, gen, only=None):
    import gc
    out = {}
    for tag, name, fn in (("zipf", "zipf_epoch_lfu_cap2^27_dim32", bench_c3),
                          ("lfu", "lfu_full_table_cap2^26_dim128", bench_c4),
                          ("hybrid", "hybrid_customized_cap2^27to2^28_dim64", bench_c5)):
        if only and tag != only:
            continue
        try:
            out[name] = fn(torch, hkv_amd, stream, gen)
        except Exception as exc:  # reported, never fatal for the main line
            out[name] = {"error": repr(exc)}
        gc.collect()
        torch.cuda.empty_cache()
    return out


def cpu_info():
    """CPU model, physical and logical core counts of this host, and the CPUs
    this process may run on."""
    model, cores, phys = None, set(), None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if ":" not in line:
                    continue
                k, v = (x.strip() for x in line.split(":", 1))
                if k == "model name" and model is None:
                    model = v
                elif k == "physical id":
                    phys = v
                elif k == "core id":
                    cores.add((phys, v))
    except OSError:
        pass
    try:
        allowed = len(os.sched_getaffinity(0))
    except AttributeError:
        allowed = os.cpu_count()
    return {"cpu_model": model, "physical_cores": len(cores) or None,
            "logical_cores": os.cpu_count(), "cpus_allowed": allowed}


def cpu_baseline(batches=4):
    """The oracle on the host cores: kLru, capacity 2^26, dim 64, filled to
    load factor ~0.47, then `batches` rounds of insert_or_assign of 2^20 new
    keys plus find of 2^20 resident keys, at one thread and at all the
    threads the box gives this process (at most 16).  insert_or_assign is
    split by bucket range across threads and find by batch range, both with
    the one-thread results."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle as O
    info = cpu_info()
    threads = max(1, min(16, info["cpus_allowed"] or 1))
    t = O.Oracle(CAP, dim=DIM, strategy=O.LRU, threads=threads)
    rng = np.random.default_rng(7)
    resident = []
    vals = rng.uniform(-1, 1, (BATCH, DIM)).astype(np.float32)
    clk = 1
    for b in range(30):  # fill to ~0.47
        ks = rng.integers(0, 2**62, BATCH, dtype=np.uint64)
        t.insert_or_assign(ks, vals, clock=clk)
        clk += 1
        resident.append(ks)
    resident = np.concatenate(resident)
    out = np.empty((BATCH, DIM), np.float32)

    def run(th):
        t.set_threads(th)
        t_ins = t_find = 0.0
        for _ in range(batches):
            ks = rng.integers(0, 2**62, BATCH, dtype=np.uint64)
            q = rng.choice(resident, BATCH)
            a = time.perf_counter()
            t.insert_or_assign(ks, vals, clock=clk + _)
            b_ = time.perf_counter()
            t.find(q, out)
            c = time.perf_counter()
            t_ins += b_ - a
            t_find += c - b_
        n = batches * BATCH
        return (2 * n / (t_ins + t_find) / 1e6, n / t_ins / 1e6, n / t_find / 1e6)

    one = run(1)
    clk += batches
    allc = run(threads)
    return {"value": round(allc[0], 3), "unit": "Mkeys/s", "cores": threads,
            "kind": "port",
            "sample": ("oracle, kLru cap 2^26 dim 64 at load factor ~0.47-0.6: "
                       f"{batches} insert_or_assign + {batches} find batches of 2^20 keys "
                       f"at 1 thread, then {batches} + {batches} at {threads} threads"),
            "insert_mkeys_s": round(allc[1], 3), "find_mkeys_s": round(allc[2], 3),
            "value_1thread": round(one[0], 3), "insert_mkeys_s_1thread": round(one[1], 3),
            "find_mkeys_s_1thread": round(one[2], 3), **info}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=8)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the load factor 0.75/1.0 and miss points")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the other benchmark configurations (Zipf "
                         "find_or_insert, full-table Lfu eviction and "
                         "accumulation, hybrid HBM/host table)")
    ap.add_argument("--configs-only", action="store_true",
                    help="run only the other benchmark configurations and print "
                         "their figures as one JSON object")
    ap.add_argument("--only", choices=("zipf", "lfu", "hybrid"),
                    help="with --configs-only: run just this configuration")
    ap.add_argument("--at-load-factor", type=float, default=None,
                    help="only: fill the headline table to this load factor, then "
                         "time 3 insert_or_assign and 3 find calls (counter passes)")
    ap.add_argument("--calibrate", action="store_true",
                    help="first run a plain 1 GiB device-to-device copy (the "
                         "reference kernel for scaling HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: the table is a single-device "
              "structure here (multi-GPU sharding is a design note, not a "
              "measured path). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    import hkv_amd

    K, W = args.steps, args.warmup
    dev = torch.device("cuda:0")
    if args.calibrate:
        a = torch.empty(1 << 28, dtype=torch.float32, device=dev).fill_(1.0)
        b_ = torch.empty_like(a)
        torch.cuda.synchronize()
        b_.copy_(a)
        torch.cuda.synchronize()
        del a, b_
    stream = torch.cuda.Stream(device=dev)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1234)
    if args.at_load_factor is not None:
        print(json.dumps(bench_at_load_factor(torch, hkv_amd, stream, gen,
                                              args.at_load_factor)), flush=True)
        return
    if args.configs_only:
        print(json.dumps(run_configs(torch, hkv_amd, stream, gen, args.only)), flush=True)
        return
    table = hkv_amd.HashTable("u64", "f32", hkv_amd.EvictStrategy.kLru)
    table.init(hkv_amd.HashTableOptions(
        init_capacity=CAP, max_capacity=CAP,
        max_hbm_for_vectors=CAP * DIM * 4, dim=DIM))
    values = torch.rand((BATCH, DIM), dtype=torch.float32, device=dev,
                        generator=gen) * 2 - 1
    out_vals = torch.empty((BATCH, DIM), dtype=torch.float32, device=dev)
    founds = torch.empty(BATCH, dtype=torch.uint8, device=dev)
    batches_to_half = (CAP // 2) // BATCH
    fill = batches_to_half - W - K // 2
    resident = []
    with torch.cuda.stream(stream):
        for _ in range(fill):
            ks = rand_keys(torch, BATCH, gen)
            table.insert_or_assign(BATCH, ks, values, None, stream)
            resident.append(ks)
        # Inputs of warmup and timed steps, generated before timing.
        ins_keys = [rand_keys(torch, BATCH, gen) for _ in range(W + K)]
        res_all = torch.cat(resident)
        find_keys = [res_all[torch.randint(0, res_all.numel(), (BATCH,),
                                           device=dev, generator=gen)]
                     for _ in range(W + K)]
    torch.cuda.synchronize()
    lf_start = None
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)]
          for _ in range(K)]
    with torch.cuda.stream(stream):
        for s in range(W):
            table.insert_or_assign(BATCH, ins_keys[s], values, None, stream)
            table.find(BATCH, find_keys[s], out_vals, founds, None, stream)
        torch.cuda.synchronize()
        lf_start = table.load_factor(stream)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for s in range(K):
            e = ev[s]
            e[0].record(stream)
            table.insert_or_assign(BATCH, ins_keys[W + s], values, None, stream)
            e[1].record(stream)
            table.find(BATCH, find_keys[W + s], out_vals, founds, None, stream)
            e[2].record(stream)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
    lf_end = table.load_factor(stream)
    hit = int(founds.sum().item())
    ins_ms = sum(e[0].elapsed_time(e[1]) for e in ev) / K
    find_ms = sum(e[1].elapsed_time(e[2]) for e in ev) / K
    wall = t1 - t0
    value = 2 * BATCH * K / wall / 1e6

    def gbs(op, ms):
        return algo_bytes(op) * BATCH / (ms * 1e-3) / 1e9

    ins_gbs = gbs("insert_new", ins_ms)
    find_gbs = gbs("find_hit", find_ms)
    breakdown = {
        "insert_or_assign_lf0.5": {
            "mkeys_s": round(BATCH / ins_ms / 1e3, 1), "ms": round(ins_ms, 4),
            "algo_gbs": round(ins_gbs, 1),
            "frac_hbm": round(ins_gbs / HBM_PEAK_GBS, 4),
            "bytes_per_key": algo_bytes("insert_new")},
        "find_hit_lf0.5": {
            "mkeys_s": round(BATCH / find_ms / 1e3, 1), "ms": round(find_ms, 4),
            "algo_gbs": round(find_gbs, 1),
            "frac_hbm": round(find_gbs / HBM_PEAK_GBS, 4),
            "bytes_per_key": algo_bytes("find_hit"), "hits": hit},
        "load_factor_range": [round(lf_start, 4), round(lf_end, 4)],
    }

    # The same K finds back to back (one event pair): the per-launch rate
    # without the event split between the step's insert and find.
    with torch.cuda.stream(stream):
        fb0 = torch.cuda.Event(enable_timing=True)
        fb1 = torch.cuda.Event(enable_timing=True)
        fb0.record(stream)
        for s in range(K):
            table.find(BATCH, find_keys[W + s], out_vals, founds, None, stream)
        fb1.record(stream)
        torch.cuda.synchronize()
    fbb_ms = fb0.elapsed_time(fb1) / K
    fbb_gbs = gbs("find_hit", fbb_ms)
    breakdown["find_hit_lf0.5_back_to_back"] = {
        "mkeys_s": round(BATCH / fbb_ms / 1e3, 1), "ms": round(fbb_ms, 4),
        "algo_gbs": round(fbb_gbs, 1), "frac_hbm": round(fbb_gbs / HBM_PEAK_GBS, 4),
        "calls": K}

    if not args.no_extra:
        with torch.cuda.stream(stream):
            def time_op(fn, reps=3):
                es = [torch.cuda.Event(enable_timing=True) for _ in range(2 * reps)]
                for r in range(reps):
                    es[2 * r].record(stream)
                    fn(r)
                    es[2 * r + 1].record(stream)
                torch.cuda.synchronize()
                return sum(es[2 * r].elapsed_time(es[2 * r + 1])
                           for r in range(reps)) / reps
            miss_keys = rand_keys(torch, BATCH, gen)
            fm_ms = time_op(lambda r: table.find(BATCH, miss_keys, out_vals,
                                                 founds, None, stream))
            mk = torch.empty(BATCH, dtype=torch.int64, device=dev)
            mi = torch.empty(BATCH, dtype=torch.int32, device=dev)
            ms_ = torch.empty(1, dtype=torch.int32, device=dev)
            fmm_ms = time_op(lambda r: table.find_missed(
                BATCH, miss_keys, out_vals, mk, mi, ms_, None, stream))
            breakdown["find_miss_lf0.5"] = {
                "mkeys_s": round(BATCH / fm_ms / 1e3, 1), "ms": round(fm_ms, 4),
                "algo_gbs": round(gbs("find_miss", fm_ms), 1)}
            breakdown["find_missed_overload_lf0.5"] = {
                "mkeys_s": round(BATCH / fmm_ms / 1e3, 1), "ms": round(fmm_ms, 4)}
            # Pointer, assign and predicate APIs on the same table (load
            # factor ~0.5, resident keys).
            hit_keys = find_keys[0]
            vptrs = torch.empty(BATCH, dtype=torch.int64, device=dev)
            kptrs = [torch.empty(BATCH, dtype=torch.int64, device=dev) for _ in range(3)]
            api = {}
            # One untimed call of each API first (first-launch costs).
            few = 1024
            table.find_ptr(few, hit_keys, vptrs, founds, None, stream)
            table.find_and_update(few, hit_keys, vptrs, founds, None, stream)
            table.contains(few, hit_keys, founds, stream)
            table.assign_values(few, hit_keys, values, stream)
            table.find_or_insert_ptr(few, hit_keys, vptrs, founds, None, stream)
            cnt = torch.zeros(1, dtype=torch.int64, device=dev)
            table.size_if(hkv_amd.PRED_SCORE_GE, 0, 0, cnt, stream)
            win = 1 << 22
            ek = torch.empty(win, dtype=torch.int64, device=dev)
            evv = torch.empty((win, DIM), dtype=torch.float32, device=dev)
            table.export_batch_if(hkv_amd.PRED_SCORE_GE, 0, 0, few, 0, cnt, ek, evv, None,
                                  stream)
            torch.cuda.synchronize()
            api["find_ptr_hit"] = time_op(lambda r: table.find_ptr(
                BATCH, hit_keys, vptrs, founds, None, stream))
            api["find_and_update_hit"] = time_op(lambda r: table.find_and_update(
                BATCH, hit_keys, vptrs, founds, None, stream))
            api["contains_hit"] = time_op(lambda r: table.contains(
                BATCH, hit_keys, founds, stream))
            api["assign_values_hit"] = time_op(lambda r: table.assign_values(
                BATCH, hit_keys, values, stream))
            fp_keys = [rand_keys(torch, BATCH, gen) for _ in range(3)]
            api["find_or_insert_ptr_new"] = time_op(lambda r: table.find_or_insert_ptr(
                BATCH, fp_keys[r], vptrs, founds, None, stream))
            api["find_or_insert_ptr_hit_locked"] = time_op(lambda r: table.find_or_insert_ptr(
                BATCH, fp_keys[r], vptrs, founds, None, stream, True, False, kptrs[r]))
            api["unlock_keys"] = time_op(lambda r: table.unlock_keys(
                BATCH, kptrs[r], fp_keys[r], None, stream))
            api["size_if_full_table"] = time_op(lambda r: table.size_if(
                hkv_amd.PRED_SCORE_GE, 0, 0, cnt, stream))
            api["export_batch_if_4M_slots"] = time_op(lambda r: table.export_batch_if(
                hkv_amd.PRED_SCORE_GE, 0, 0, win, r * win, cnt, ek, evv, None, stream))
            for name, ms in api.items():
                per = CAP if name == "size_if_full_table" else (
                    win if name.startswith("export") else BATCH)
                breakdown[name] = {"ms": round(ms, 4),
                                   "mitems_s": round(per / ms / 1e3, 1),
                                   "items": "slots" if per != BATCH else "keys"}
            del ek, evv
            for target, name, model in ((0.75, "insert_or_assign_lf0.75", "insert_new"),
                                        (1.0, "insert_or_assign_lf1.0", "insert_evict")):
                guard = 0
                while table.load_factor(stream) < target - 1e-9 and guard < 200:
                    lf = table.load_factor(stream)
                    if target < 1.0 and lf + BATCH / CAP > target:
                        break
                    table.insert_or_assign(BATCH, rand_keys(torch, BATCH, gen),
                                           values, None, stream)
                    guard += 1
                lf0 = table.load_factor(stream)
                nk = [rand_keys(torch, BATCH, gen) for _ in range(3)]
                torch.cuda.synchronize()
                t_ms = time_op(lambda r: table.insert_or_assign(
                    BATCH, nk[r], values, None, stream))
                g = gbs(model, t_ms)
                breakdown[name] = {
                    "mkeys_s": round(BATCH / t_ms / 1e3, 1), "ms": round(t_ms, 4),
                    "algo_gbs": round(g, 1), "frac_hbm": round(g / HBM_PEAK_GBS, 4),
                    "load_factor_at_start": round(lf0, 4)}
                # find at this load factor: the batches just inserted (hits),
                # then fresh keys (misses) through both overloads.
                lf_tag = "lf%.2f" % target if target < 1.0 else "lf1.0"
                hf = time_op(lambda r: table.find(BATCH, nk[r], out_vals, founds,
                                                  None, stream))
                hits = int(founds.sum().item())
                g = gbs("find_hit", hf)
                breakdown["find_hit_" + lf_tag] = {
                    "mkeys_s": round(BATCH / hf / 1e3, 1), "ms": round(hf, 4),
                    "algo_gbs": round(g, 1), "frac_hbm": round(g / HBM_PEAK_GBS, 4),
                    "bytes_per_key": algo_bytes("find_hit"), "hits": hits,
                    "load_factor": round(table.load_factor(stream), 4)}
                mks = [rand_keys(torch, BATCH, gen) for _ in range(3)]
                fm = time_op(lambda r: table.find(BATCH, mks[r], out_vals, founds,
                                                  None, stream))
                fmm = time_op(lambda r: table.find_missed(
                    BATCH, mks[r], out_vals, mk, mi, ms_, None, stream))
                breakdown["find_miss_" + lf_tag] = {
                    "mkeys_s": round(BATCH / fm / 1e3, 1), "ms": round(fm, 4),
                    "algo_gbs": round(gbs("find_miss", fm), 1),
                    "missed_overload_ms": round(fmm, 4),
                    "missed_overload_mkeys_s": round(BATCH / fmm / 1e3, 1)}

    if not args.no_configs:
        breakdown.update(run_configs(torch, hkv_amd, stream, gen))

    # The dominant operation of the step sets the roofline line.
    if ins_ms >= find_ms:
        roof = {"kernel": "insert_or_assign (k_pcount + k_pscan + k_pscatter + "
                          "k_apply_fast + k_apply_deferred + k_apply_part)",
                "achieved": round(ins_gbs, 1), "bytes_per_key": algo_bytes("insert_new"),
                "ms_per_launch": round(ins_ms, 4), "op": "insert_new"}
    else:
        roof = {"kernel": "find (k_find)", "achieved": round(find_gbs, 1),
                "bytes_per_key": algo_bytes("find_hit"),
                "ms_per_launch": round(find_ms, 4), "op": "find_hit"}
    bpk = measured_bytes_per_key(roof["op"])
    traffic = round(bpk * BATCH) if bpk is not None else None
    roofline = {"bound": "hbm", "achieved": roof["achieved"], "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(roof["achieved"] / HBM_PEAK_GBS, 4),
                "traffic": traffic, "traffic_unit": "bytes per launch (rocprofv3 "
                "FETCH_SIZE + WRITE_SIZE, copy-calibrated)",
                "kernel": roof["kernel"],
                "keys_per_launch": BATCH, "bytes_per_key": roof["bytes_per_key"],
                "ms_per_launch": roof["ms_per_launch"]}

    cpu = None
    if not args.no_cpu_baseline:
        try:
            cpu = cpu_baseline()
        except Exception as exc:  # reported, never fatal for the GPU line
            cpu = {"error": repr(exc)}

    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "Mkeys/s",
        "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(wall / K * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "u64",
        "data": "synthetic",
        "config": {"workload": "kLru cap 2^26 (128-slot buckets) dim 64 fp32 in HBM, "
                               "2^20-key batches: insert_or_assign new keys + find "
                               "resident keys around load factor 0.5",
                   "capacity": CAP, "dim": DIM, "batch": BATCH,
                   "strategy": "kLru", "parallelism": "single GPU"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "breakdown": breakdown,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
