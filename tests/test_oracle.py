"""Pins the CPU oracle (oracle/oracle.c) with checks independent of its own
formulas: numpy / Python-set algebra, nested-loop brute force, closed forms
(BFS layers, chain, cycle, K_{n,n}), the naive fixpoint, and the reference's
own known-answer vectors (tests/golden/reference_kats.json)."""
import itertools
import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from xlog_amd import andersen_plan, copy_points_to_plan, datagen, pack, tc_plan, unpack

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def rows_to_keys(rows):
    return np.array([(r[0] << 32) | r[1] for r in rows], dtype=np.uint64)


def keys_to_rows(keys):
    return [[int(k >> 32), int(k & 0xFFFFFFFF)] for k in keys]


# ---- sort / dedup -------------------------------------------------------------
@pytest.mark.parametrize("n", [0, 1, 2, 3, 255, 256, 257, 10000, 100003])
def test_sort_dedup_vs_numpy(n):
    rng = np.random.default_rng(n)
    k = rng.integers(0, 1 << 64, n, dtype=np.uint64)
    if n > 3:
        k[: n // 3] = k[n // 3: 2 * (n // 3)]
    assert np.array_equal(oracle.sort_u64(k), np.sort(k))
    assert np.array_equal(oracle.sort_dedup(k), np.unique(k))


def test_sort_skips_constant_digits_correctly():
    k = pack(np.full(5000, 7, np.uint32), np.arange(5000, dtype=np.uint32)[::-1])
    assert np.array_equal(oracle.sort_u64(k), np.sort(k))


def test_sort_kats():
    for kat in KATS["sort"]:
        col = np.array(kat["cols"][0], dtype=np.uint64)
        if len(kat["cols"]) == 1:
            assert oracle.sort_u64(col).tolist() == kat["expect"][0], kat["src"]
        else:
            k = pack(kat["cols"][0], kat["cols"][1])
            got = keys_to_rows(oracle.sort_u64(k))
            assert [r[0] for r in got] == kat["expect"][0] and [r[1] for r in got] == kat["expect"][1], kat["src"]


def test_dedup_kats():
    for kat in KATS["dedup_full_row"]:
        assert keys_to_rows(oracle.sort_dedup(rows_to_keys(kat["rows"]))) == kat["expect"], kat["src"]


def test_diff_kats():
    for kat in KATS["diff_full_row"]:
        a = oracle.sort_dedup(rows_to_keys(kat["a"]))
        b = oracle.sort_dedup(rows_to_keys(kat["b"]))
        assert keys_to_rows(oracle.diff_sorted(a, b)) == kat["expect"], kat["src"]


@pytest.mark.parametrize("seed", range(6))
def test_set_algebra_identities(seed):
    rng = np.random.default_rng(seed)
    a = np.unique(rng.integers(0, 3000, rng.integers(0, 2000), dtype=np.uint64))
    b = np.unique(rng.integers(0, 3000, rng.integers(0, 2000), dtype=np.uint64))
    u, d = oracle.union_sorted(a, b), oracle.diff_sorted(a, b)
    sa, sb = set(a.tolist()), set(b.tolist())
    assert u.tolist() == sorted(sa | sb)
    assert d.tolist() == sorted(sa - sb)
    assert len(u) == len(a) + len(b) - len(sa & sb)
    assert sorted(set(d.tolist()) | (sa & sb)) == a.tolist()


# ---- join ------------------------------------------------------------------------
@pytest.mark.parametrize("seed", range(5))
@pytest.mark.parametrize("lk,rk", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_join_vs_nested_loop(seed, lk, rk):
    rng = np.random.default_rng(seed * 10 + lk * 2 + rk)
    l = pack(rng.integers(0, 6, 40), rng.integers(0, 6, 40))
    r = pack(rng.integers(0, 6, 30), rng.integers(0, 6, 30))
    L = [(int(x >> 32), int(x & 0xFFFFFFFF)) for x in l]
    R = [(int(x >> 32), int(x & 0xFFFFFFFF)) for x in r]
    for oc in [(0, 3), (1, 2), (3, 0), (2, 1)]:
        brute = sorted(((lr + rr)[oc[0]] << 32) | (lr + rr)[oc[1]]
                       for lr in L for rr in R if lr[lk] == rr[rk])
        got = sorted(oracle.join_project(l, r, lk, rk, *oc).tolist())
        assert got == brute
    # multiset size from the key histograms
    cl = np.bincount([x[lk] for x in L], minlength=6)
    cr = np.bincount([x[rk] for x in R], minlength=6)
    assert oracle.join_count(l, r, lk, rk) == int((cl * cr).sum())


@pytest.mark.parametrize("seed", range(6))
def test_chain2_counts_vs_python(seed):
    """The two-join body head(v, o) :- l(v, w), a(w, p), b(p, o) counted by the
    oracle equals the sizes of the joined lists and sets built in Python."""
    rng = np.random.default_rng(900 + seed)
    n = int(rng.integers(3, 12))

    def rel(m):
        return oracle.sort_dedup(pack(rng.integers(0, n, m), rng.integers(0, n, m)))
    l, a, b = rel(int(rng.integers(0, 60))), rel(int(rng.integers(0, 60))), rel(int(rng.integers(0, 60)))
    L, A, B = ([(int(x >> 32), int(x & 0xFFFFFFFF)) for x in r] for r in (l, a, b))
    bag1 = [(v, p) for v, w in L for w2, p in A if w == w2]
    set1 = set(bag1)
    got = oracle.chain2_counts(l, a, b)
    assert got["bag1"] == len(bag1)
    assert got["set1"] == len(set1)
    assert got["bag2_over_set1"] == len([1 for v, p in set1 for p2, o in B if p == p2])
    assert got["bag2_over_bag1"] == len([1 for v, p in bag1 for p2, o in B if p == p2])
    # the first join's bag is also the plain join count
    assert got["bag1"] == oracle.join_count(l, a, 1, 0)


def test_join_kats():
    for kat in KATS["join_inner_key0"]:
        l, r = rows_to_keys(kat["left"]), rows_to_keys(kat["right"])
        got = oracle.join_project(l, r, 0, 0, 0, 3)
        exp = [(row[0] << 32) | row[3] for row in kat["expect"]]
        assert sorted(got.tolist()) == sorted(exp), kat["src"]


# ---- fixpoint: transitive closure ---------------------------------------------------
def floyd_warshall(nv, edges):
    m = np.zeros((nv, nv), bool)
    for a, b in edges:
        m[a, b] = True
    for k in range(nv):
        m |= m[:, [k]] & m[[k], :]
    return m


@pytest.mark.parametrize("seed", range(8))
def test_bfs_vs_floyd_warshall(seed):
    rng = np.random.default_rng(seed)
    nv = int(rng.integers(2, 30))
    edges = [(int(a), int(b)) for a, b in rng.integers(0, nv, (int(rng.integers(0, 60)), 2))]
    src = np.array([e[0] for e in edges], np.uint32)
    dst = np.array([e[1] for e in edges], np.uint32)
    b = oracle.bfs_tc(nv, src, dst)
    m = floyd_warshall(nv, edges)
    xs, zs = np.nonzero(m)
    exp = np.sort(pack(xs.astype(np.uint32), zs.astype(np.uint32)))
    assert np.array_equal(b["relation"], exp)


@pytest.mark.parametrize("seed", range(8))
def test_seminaive_tc_equals_bfs_layers(seed):
    rng = np.random.default_rng(100 + seed)
    nv = int(rng.integers(2, 200))
    m = int(rng.integers(0, 4 * nv))
    src = rng.integers(0, nv, m).astype(np.uint32)
    dst = rng.integers(0, nv, m).astype(np.uint32)
    b = oracle.bfs_tc(nv, src, dst)
    outs, it, deltas = oracle.seminaive(tc_plan(), [pack(src, dst), None])
    assert np.array_equal(outs[1], b["relation"])
    assert it == b["iterations"]
    if m:
        assert deltas == [int(x) for x in b["dist_count"][1:it + 1]] + [0]


@pytest.mark.parametrize("shape", ["chain", "cycle", "kbip"])
def test_tc_closed_forms(shape):
    n = 25
    src, dst = {"chain": datagen.chain, "cycle": datagen.cycle, "kbip": datagen.complete_bipartite}[shape](n)
    outs, it, _ = oracle.seminaive(tc_plan(), [pack(src, dst), None])
    exp = {"chain": ((n - 1) * n // 2, n - 1), "cycle": (n * n, n), "kbip": (n * n, 1)}[shape]
    assert (len(outs[1]), it) == exp


def test_tc_empty_edges_runs_one_iteration():
    outs, it, deltas = oracle.seminaive(tc_plan(), [np.zeros(0, np.uint64), None])
    assert len(outs[1]) == 0 and it == 1 and deltas == [0, 0]


def test_tc_kats():
    kat = KATS["tc"][0]
    src, dst = zip(*kat["edges"])
    outs, it, _ = oracle.seminaive(tc_plan(), [pack(src, dst), None])
    pairs = keys_to_rows(outs[1])
    assert sorted(z for x, z in pairs if x == 1) == kat["expect_from"]["1"], kat["src"]
    kat = KATS["tc"][1]
    src, dst = zip(*kat["edges"])
    outs, it, _ = oracle.seminaive(tc_plan(), [pack(src, dst), None])
    m = floyd_warshall(12, kat["edges"])
    xs, zs = np.nonzero(m)
    assert np.array_equal(outs[1], np.sort(pack(xs.astype(np.uint32), zs.astype(np.uint32)))), kat["src"]


def test_iteration_limit():
    src, dst = datagen.chain(30)
    with pytest.raises(RuntimeError) as e:
        oracle.seminaive(tc_plan(), [pack(src, dst), None], max_iter=10)
    assert e.value.code == -4 and e.value.iterations == 10


# ---- fixpoint: other programs vs the independent naive evaluation ------------------
def test_points_to_copy_kat():
    kat = KATS["points_to_copy"][0]
    outs, it, _ = oracle.seminaive(copy_points_to_plan(), [rows_to_keys(kat["addr_of"]), rows_to_keys(kat["copy"]), None])
    assert keys_to_rows(outs[2]) == kat["expect"], kat["src"]


@pytest.mark.parametrize("nv,nf", [(30, 60), (200, 600), (800, 3000)])
def test_andersen_seminaive_equals_naive(nv, nf):
    f = datagen.andersen(nv, nf, 1.5, datagen.seed_for(5) + nv)
    rels = [pack(*f[k]) for k in ("assign", "addressOf", "load", "store")]
    outs, it, _ = oracle.seminaive(andersen_plan(), rels + [None])
    nouts, rounds = oracle.naive(andersen_plan(), rels + [None])
    assert np.array_equal(outs[4], nouts[4]) and it == rounds


def andersen_python(f):
    """Direct set-based restatement of the four rules, iterated to a fixpoint."""
    pts = set(zip(*[x.tolist() for x in f["addressOf"]]))
    assign = list(zip(*[x.tolist() for x in f["assign"]]))
    load = list(zip(*[x.tolist() for x in f["load"]]))
    store = list(zip(*[x.tolist() for x in f["store"]]))
    while True:
        by = {}
        for v, o in pts:
            by.setdefault(v, set()).add(o)
        new = set(pts)
        for v, w in assign:
            new |= {(v, o) for o in by.get(w, ())}
        for v, w in load:
            for p in by.get(w, ()):
                new |= {(v, o) for o in by.get(p, ())}
        for v, w in store:
            for p in by.get(v, ()):
                new |= {(p, o) for o in by.get(w, ())}
        if new == pts:
            return pts
        pts = new


@pytest.mark.parametrize("nv,nf", [(40, 100), (150, 500)])
def test_andersen_vs_python_sets(nv, nf):
    f = datagen.andersen(nv, nf, 1.5, 77 + nv)
    rels = [pack(*f[k]) for k in ("assign", "addressOf", "load", "store")]
    outs, _, _ = oracle.seminaive(andersen_plan(), rels + [None])
    exp = np.array(sorted((a << 32) | b for a, b in andersen_python(f)), dtype=np.uint64)
    assert np.array_equal(outs[4], exp)


def test_planted_mistake_is_caught():
    """A wrong plan (join on the wrong column, i.e. reach(X,Z) :- reach(X,Y), edge(Z,Y))
    must disagree with the BFS closed form on a graph with asymmetric edges."""
    src, dst = datagen.random_digraph(60, 200, 5)
    X, Y, Z = 0, 1, 2
    wrong = [2, 1, X, Y, 1, 0, X, Y, 1, X, Z, 2, 1, X, Y, 0, Z, Y]
    outs, it, _ = oracle.seminaive(wrong, [pack(src, dst), None])
    b = oracle.bfs_tc(60, src, dst)
    assert not np.array_equal(outs[1], b["relation"])


# ---- the multi-threaded paths (CPU baseline) against the single-threaded ones --
def test_parallel_paths_match_serial():
    """or_set_threads(t > 1) switches the sort, join probe and BFS to OpenMP versions; they must give
    exactly the single-threaded results (which the tests above pin)."""
    rng = np.random.default_rng(2024)
    keys = rng.integers(0, 1 << 64, 400_000, dtype=np.uint64)
    keys[::7] = keys[1::7][: len(keys[::7])]  # duplicates
    l = pack(rng.integers(0, 1 << 31, 60_000, dtype=np.uint64), rng.integers(0, 5_000, 60_000, dtype=np.uint64))
    r = pack(rng.integers(0, 5_000, 50_000, dtype=np.uint64), rng.integers(0, 1 << 31, 50_000, dtype=np.uint64))
    src, dst = datagen.random_digraph(1200, 5000, datagen.seed_for(1))
    f = datagen.andersen(1500, 6000, 1.5, datagen.seed_for(5))
    rels = [pack(*f[k]) for k in ("assign", "addressOf", "load", "store")] + [None]
    tc_rel = [pack(src, dst), None]

    def run():
        return (oracle.sort_dedup(keys.copy()), oracle.join_project(l, r, 1, 0, 0, 3),
                oracle.seminaive(tc_plan(), tc_rel), oracle.seminaive(andersen_plan(), rels),
                oracle.bfs_tc(1200, src, dst, want_relation=False, digest=False))

    serial = run()
    try:
        assert oracle.set_threads(4) == 4
        par = run()
    finally:
        oracle.set_threads(1)
    assert np.array_equal(serial[0], par[0])
    assert np.array_equal(serial[1], par[1])  # same bag, same order
    for s_, p_ in ((serial[2], par[2]), (serial[3], par[3])):
        assert s_[1:] == p_[1:]
        assert all((a is None and b is None) or np.array_equal(a, b) for a, b in zip(s_[0], p_[0]))
    assert serial[4]["total"] == par[4]["total"] and serial[4]["iterations"] == par[4]["iterations"]
    assert np.array_equal(serial[4]["dist_count"], par[4]["dist_count"])


# ---- FNV-1a-64, the digest of every fixture ------------------------------------
@pytest.mark.parametrize("data,digest", [
    # published FNV-1a 64-bit test vectors (the FNV reference test suite, isthe.com/chongo/tech/comp/fnv)
    (b"", 0xCBF29CE484222325),
    (b"a", 0xAF63DC4C8601EC8C),
    (b"foobar", 0x85944171F73967E8),
])
def test_fnv1a64_published_vectors(data, digest):
    assert oracle.fnv1a64_bytes(data) == digest


def test_fnv1a64_keys_are_little_endian_bytes():
    # the fixture digest is FNV-1a over the keys' little-endian bytes in row order
    rng = np.random.default_rng(3)
    for n in (0, 1, 2, 7, 1000):
        keys = rng.integers(0, 1 << 64, size=n, dtype=np.uint64)
        assert oracle.fnv1a64(keys) == oracle.fnv1a64_bytes(keys.astype("<u8").tobytes()), n
    assert oracle.fnv1a64(np.zeros(0, np.uint64)) == 0xCBF29CE484222325
    # one key's bytes in order: 0x0102030405060708 hashes the bytes 08 07 ... 01
    k = np.array([0x0102030405060708], np.uint64)
    assert oracle.fnv1a64(k) == oracle.fnv1a64_bytes(bytes([8, 7, 6, 5, 4, 3, 2, 1]))
    assert oracle.fnv1a64(k) != oracle.fnv1a64_bytes(bytes([1, 2, 3, 4, 5, 6, 7, 8]))
