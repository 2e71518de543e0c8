"""Regenerates the golden fixtures of this directory from the seeded generators
and the CPU oracle (oracle/oracle.c), cross-checked where a closed form exists.

    python tests/golden/make_golden.py [--full]

Writes fixtures.json (counts, iteration counts, per-iteration delta sizes,
FNV-1a-64 digests of the sorted packed output and of the generated inputs) and
c1_closure.npz (the full config-1 closure as a packed 1000x1000 bit matrix).
--full also computes the full-size C2 / C3 / C4 entries (minutes of CPU time).
--sparse computes the transitive closures with ids spread over the u32 range
(tcs, tcs_crit: G(2^20, m) digraphs, beyond any dense bit-matrix domain).
--c5 computes the larger Andersen instances (10,000, 20,000 and 40,000 variables; the
naive fixpoint cross-checks the first two, the third is past its time budget).
--c5-stated computes, for C5 at its stated 500,000 variables / 2,000,000 facts, the
row counts of the first recursive iteration's joins in the order the join route
evaluates them (the seed delta, rule 2's join, and rule 3's two-join body with the
delta in its first pointsTo atom), which decide where a join-row limit trips.
"""
from __future__ import annotations

import argparse
import json
import sys
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402
from xlog_amd import andersen_plan, datagen, pack, tc_plan  # noqa: E402


def fnv_inputs(*arrays) -> int:
    h = 0
    parts = []
    for a in arrays:
        parts.append(oracle.fnv1a64(np.asarray(a).astype(np.uint64)))
    for x in parts:
        h = (h * 0x100000001B3) ^ x
        h &= (1 << 64) - 1
    return h


def tc_entry(nv, src, dst):
    b = oracle.bfs_tc(nv, src, dst)
    it = b["iterations"]
    return {"vertices": nv, "edges": int(len(src)), "input_digest": fnv_inputs(src, dst),
            "tuples": b["total"], "iterations": it, "digest": b["digest"],
            "delta_sizes": [int(x) for x in b["dist_count"][1:it + 1]] + [0]}


def sparse_tc_entry(cfg):
    """Closure of a G(n, m) digraph (seed_for(6)) with ids remapped by datagen.sparse_ids: the
    BFS closed form gives the relation, iterations and per-iteration delta sizes (invariant under
    the relabelling); the digest is over the relabelled, re-sorted tuples."""
    nv, m = cfg["n_vertices"], cfg["n_edges"]
    src, dst = datagen.random_digraph(nv, m, datagen.seed_for(6))
    b = oracle.bfs_tc(nv, src, dst, want_relation=True, digest=False)
    it = b["iterations"]
    rel = b["relation"]
    hi = datagen.sparse_ids((rel >> np.uint64(32)).astype(np.uint32)).astype(np.uint64)
    lo = datagen.sparse_ids((rel & np.uint64(0xFFFFFFFF)).astype(np.uint32)).astype(np.uint64)
    del rel
    keys = np.sort((hi << np.uint64(32)) | lo)
    del hi, lo
    s2, d2 = datagen.sparse_ids(src), datagen.sparse_ids(dst)
    return {"vertices": nv, "edges": int(m), "id_map": "datagen.sparse_ids", "input_digest": fnv_inputs(s2, d2),
            "tuples": int(len(keys)), "iterations": it,
            "delta_sizes": [int(x) for x in b["dist_count"][1:it + 1]] + [0], "digest": oracle.fnv1a64(keys)}


def c5_entry(nv, nf, check_naive=True):
    f = datagen.andersen(nv, nf, 1.5, datagen.seed_for(5))
    rels = [pack(*f[k]) for k in ("assign", "addressOf", "load", "store")]
    outs, it, deltas = oracle.seminaive(andersen_plan(), rels + [None])
    if check_naive:
        nouts, rounds = oracle.naive(andersen_plan(), rels + [None])
        assert np.array_equal(nouts[4], outs[4]) and rounds == it
    return {"n_vars": nv, "n_facts": nf, "alpha": 1.5,
            "input_digest": fnv_inputs(*[x for k in ("assign", "addressOf", "load", "store") for x in f[k]]),
            "tuples": int(len(outs[4])), "iterations": it, "delta_sizes": deltas,
            "digest": oracle.fnv1a64(outs[4]), "checked_against_naive": bool(check_naive)}


def c5_stated_entry():
    """C5 at its stated size, first recursive iteration.  After the seed, pointsTo = delta = addressOf
    (rule 1; the other rules read pointsTo, still empty).  The join route then evaluates, in rule order,
    rule 2 (assign join delta on W) and rule 3 with the delta in atom 1: load(V,W) join delta(W,P) projected
    to (V,P), then joined with pointsTo(P,O) (= addressOf) on P.  The library's join step keeps a first join
    of more than 2^30 - 1 rows as a sorted set (chunked sort + dedup), so the second join's bag is counted
    over the distinct (V,P) pairs; the reference keeps the bag (bag2_over_bag1)."""
    cfg = datagen.C5
    f = datagen.andersen(cfg["n_vars"], cfg["n_facts"], cfg["alpha"], datagen.seed_for(5))
    assign, addr, load = (oracle.sort_dedup(pack(*f[k])) for k in ("assign", "addressOf", "load"))
    r2 = oracle.chain2_counts(assign, addr, np.zeros(0, np.uint64))
    r3 = oracle.chain2_counts(load, addr, addr)
    return {"n_vars": cfg["n_vars"], "n_facts": cfg["n_facts"], "alpha": cfg["alpha"],
            "seed_delta": int(len(addr)), "rule2_bag": r2["bag1"], "rule2_tuples": r2["set1"],
            "rule3_first_join_bag": r3["bag1"], "rule3_first_join_set": r3["set1"],
            "rule3_second_join_bag_over_set": r3["bag2_over_set1"],
            "rule3_second_join_bag_over_bag": r3["bag2_over_bag1"]}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--full", action="store_true")
    ap.add_argument("--sparse", action="store_true")
    ap.add_argument("--c5", action="store_true")
    ap.add_argument("--c5-stated", action="store_true")
    ap.add_argument("--threads", type=int, default=1)
    args = ap.parse_args()
    oracle.set_threads(args.threads)
    fx = {"_about": "Generated by tests/golden/make_golden.py from the seeded generators and the CPU oracle. "
                    "digest = FNV-1a-64 over the little-endian bytes of the sorted packed (c0<<32|c1) tuples."}
    path = HERE / "fixtures.json"
    if path.exists():
        fx.update(json.loads(path.read_text()))

    # C1 -------------------------------------------------------------------------
    src, dst = datagen.random_digraph(1000, 5000, datagen.seed_for(1))
    e = tc_entry(1000, src, dst)
    outs, it, deltas = oracle.seminaive(tc_plan(), [pack(src, dst), None])
    # semi-naive loop == BFS closed form: iteration count and per-iteration deltas
    assert it == e["iterations"] and deltas == e["delta_sizes"], (it, deltas, e)
    assert oracle.fnv1a64(outs[1]) == e["digest"] and len(outs[1]) == e["tuples"]
    fx["c1"] = e
    rel = outs[1]
    bits = np.zeros((1000, 1000), np.uint8)
    bits[(rel >> np.uint64(32)).astype(np.int64), (rel & np.uint64(0xFFFFFFFF)).astype(np.int64)] = 1
    np.savez_compressed(HERE / "c1_closure.npz", bits=np.packbits(bits, axis=1))

    # C2 small (sample shape with the same generator) ------------------------------
    r_a, r_b, s_b, s_c = datagen.zipf_join(1 << 16, 1 << 16, 1 << 12, 1.1, datagen.seed_for(2))
    j = oracle.join_project(pack(r_a, r_b), pack(s_b, s_c), 1, 0, 0, 3)
    u = oracle.sort_dedup(j)
    fx["c2_small"] = {"n_r": 1 << 16, "n_s": 1 << 16, "n_keys": 1 << 12, "zipf_s": 1.1,
                      "input_digest": fnv_inputs(r_a, r_b, s_b, s_c), "join_rows": int(len(j)),
                      "unique": int(len(u)), "digest": oracle.fnv1a64(u)}

    # C3 small ------------------------------------------------------------------------
    keys = datagen.dup_tuples(1 << 20, datagen.seed_for(3))
    u = oracle.sort_dedup(keys)
    fx["c3_small"] = {"n": 1 << 20, "input_digest": oracle.fnv1a64(keys), "unique": int(len(u)),
                      "digest": oracle.fnv1a64(u)}

    # C5 small (same generator, scaled down) --------------------------------------------
    for nv, nf in ((2000, 8000), (5000, 20000)):
        f = datagen.andersen(nv, nf, 1.5, datagen.seed_for(5))
        rels = [pack(*f[k]) for k in ("assign", "addressOf", "load", "store")]
        outs, it, deltas = oracle.seminaive(andersen_plan(), rels + [None])
        nouts, rounds = oracle.naive(andersen_plan(), rels + [None])
        assert np.array_equal(nouts[4], outs[4]) and rounds == it
        fx[f"c5_{nv}_{nf}"] = {"n_vars": nv, "n_facts": nf, "alpha": 1.5,
                               "input_digest": fnv_inputs(*[x for k in ("assign", "addressOf", "load", "store")
                                                            for x in f[k]]),
                               "tuples": int(len(outs[4])), "iterations": it, "delta_sizes": deltas,
                               "digest": oracle.fnv1a64(outs[4])}

    if args.sparse:
        for name, cfg in (("tcs", datagen.TCS), ("tcs_crit", datagen.TCS_CRIT)):
            t = time.time()
            fx[name] = sparse_tc_entry(cfg)
            print(f"{name} {time.time() - t:.0f}s", flush=True)
    if args.c5:
        for nv in (10_000, 20_000, 40_000):
            t = time.time()
            fx[f"c5_{nv}_{4 * nv}"] = c5_entry(nv, 4 * nv, check_naive=nv <= 20_000)
            print(f"c5 {nv} {time.time() - t:.0f}s", flush=True)
            path.write_text(json.dumps(fx, indent=1) + "\n")
    if args.c5_stated:
        t = time.time()
        fx["c5_stated"] = c5_stated_entry()
        print(f"c5 stated {time.time() - t:.0f}s {fx['c5_stated']}", flush=True)
    if args.full:
        t = time.time()
        src, dst = datagen.random_digraph(32768, 3 * 32768, datagen.seed_for(4))
        fx["c4"] = tc_entry(32768, src, dst)
        print(f"c4 {time.time() - t:.0f}s", flush=True)
        t = time.time()
        keys = datagen.dup_tuples(1 << 28, datagen.seed_for(3))
        ik = oracle.fnv1a64(keys)
        u = oracle.sort_dedup(keys)
        del keys
        fx["c3"] = {"n": 1 << 28, "input_digest": ik, "unique": int(len(u)), "digest": oracle.fnv1a64(u)}
        del u
        print(f"c3 {time.time() - t:.0f}s", flush=True)
        t = time.time()
        r_a, r_b, s_b, s_c = datagen.zipf_join(1 << 24, 1 << 24, 1 << 20, 1.1, datagen.seed_for(2))
        ik = fnv_inputs(r_a, r_b, s_b, s_c)
        j = oracle.join_project(pack(r_a, r_b), pack(s_b, s_c), 1, 0, 0, 3)
        nj = int(len(j))
        u = oracle.sort_dedup(j)
        del j
        fx["c2"] = {"n_r": 1 << 24, "n_s": 1 << 24, "n_keys": 1 << 20, "zipf_s": 1.1, "input_digest": ik,
                    "join_rows": nj, "unique": int(len(u)), "digest": oracle.fnv1a64(u)}
        print(f"c2 {time.time() - t:.0f}s", flush=True)
    path.write_text(json.dumps(fx, indent=1) + "\n")
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
