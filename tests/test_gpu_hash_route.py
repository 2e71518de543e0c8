"""GPU parity of the hash-set route (the transitive closure with R in a device
hash set, one fused expand + insert pass per iteration) and of the sparse
factorized delta operator (fj_delta_sparse_novel_u32_recorded,
crates/xlog-cuda/src/provider/fj_delta_sparse.rs:66).

Expected values: the BFS closed form of the CPU oracle (relation, iteration
count = max finite distance, delta of iteration k = pairs at distance k + 1),
brute force on tiny graphs, the committed fixtures (C1, C4, and the
sparse-id closures tcs / tcs_crit whose ids span the whole u32 range), and the
dense factorized delta operator on dense domains."""
import json
import sys
from pathlib import Path

import numpy as np
import pytest

import oracle
from xlog_amd import FJ_DELTA_CANONICAL, ROUTE_AUTO, ROUTE_HASH, ROUTE_JOIN, XlogError, datagen, pack, tc_plan

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).parent / "golden"
FIX = json.loads((GOLDEN / "fixtures.json").read_text())
UNSUPPORTED = 7


def _note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _tc(p, src, dst, route):
    E = p.create_buffer_from_u32_columns([np.asarray(src, np.uint32), np.asarray(dst, np.uint32)])
    outs, st = p.fixpoint(tc_plan(), [E, None], route=route)
    return outs[1], st


def _bfs_expect(nv, src, dst):
    b = oracle.bfs_tc(nv, src, dst)
    it = b["iterations"]
    return b["relation"], it, [int(x) for x in b["dist_count"][1:it + 1]] + [0]


@pytest.mark.parametrize("nv,m,seed", [(200, 300, 1), (1000, 5000, 2), (3000, 3100, 3), (5000, 4000, 4)])
def test_hash_route_random_graphs_vs_bfs(provider, nv, m, seed):
    p = provider
    src, dst = datagen.random_digraph(nv, m, seed)
    rel, it, deltas = _bfs_expect(nv, src, dst)
    # duplicated edges and a shuffled order give the same closure
    src2, dst2 = np.concatenate([src, src[:50]]), np.concatenate([dst, dst[:50]])
    order = np.random.default_rng(seed).permutation(len(src2))
    out, st = _tc(p, src2[order], dst2[order], ROUTE_HASH)
    assert st["route"] == ROUTE_HASH
    assert np.array_equal(p.download_packed(out), rel)
    assert out.is_canonical()
    assert (st["iterations"], st["delta_sizes"]) == (it, deltas)
    # one read-back per iteration (plus a handful of set-up and final waits)
    assert st["host_waits"] <= st["iterations"] + 8, st


def test_hash_route_grow_and_rerun(provider, monkeypatch):
    # a 64-slot table and 100 appends per attempt force every step through the overflow protocol
    p = provider
    src, dst = datagen.random_digraph(3000, 3600, 9)
    rel, it, deltas = _bfs_expect(3000, src, dst)
    monkeypatch.setenv("XLOG_HIP_HASH_SLOTS", "64")
    monkeypatch.setenv("XLOG_HIP_HASH_APPENDS", "100")
    out, st = _tc(p, src, dst, ROUTE_HASH)
    assert np.array_equal(p.download_packed(out), rel)
    assert (st["iterations"], st["delta_sizes"]) == (it, deltas)
    assert st["host_waits"] > st["iterations"] + 8  # the reruns took extra read-backs


def _closure_brute(edges):
    succ = {}
    for a, b in edges:
        succ.setdefault(a, set()).add(b)
    out = set()
    for s in succ:
        seen, stack = set(), [s]
        while stack:
            for b in succ.get(stack.pop(), ()):
                if b not in seen:
                    seen.add(b)
                    stack.append(b)
        out |= {(s, b) for b in seen}
    return sorted(out)


def test_hash_route_all_ones_ids(provider):
    # 0xFFFFFFFF is the table's empty slot: the all-ones tuple (M, M) travels by its flag
    p = provider
    M = 0xFFFFFFFF
    edges = [(M, 5), (5, M), (M, 0), (0, M - 1), (M - 1, 7), (7, 7), (12, M)]
    src, dst = zip(*edges)
    out, st = _tc(p, src, dst, ROUTE_HASH)
    exp = _closure_brute(edges)
    assert (M, M) in exp
    assert p.download_rows(out) == exp
    j, st_j = _tc(p, src, dst, ROUTE_JOIN)
    assert p.download_rows(j) == exp
    assert (st["iterations"], st["delta_sizes"]) == (st_j["iterations"], st_j["delta_sizes"])


@pytest.mark.parametrize("plan_name", ["tc", "nonlinear_tc"])
def test_hash_route_all_ones_in_initial_head(provider, plan_name):
    """The starting IDB relation holds the all-ones tuple (M, M), which the table
    keeps in its flag: it must count as present from the start (never re-derived
    as new, never a duplicate row of an indexed relation), on the linear plan and
    on the non-linear one whose IDB relation is read through an index."""
    import chain_plans as cp
    p = provider
    M = 0xFFFFFFFF
    edges = [(M, 5), (5, M), (M, 0), (0, M - 1), (M - 1, 7), (7, 7), (12, M), (9, 12)]
    head = [(M, M), (3, 9), (M, 0)]
    plan = tc_plan() if plan_name == "tc" else cp.nonlinear_tc_plan()
    e = pack(np.array([a for a, _ in edges], np.uint32), np.array([b for _, b in edges], np.uint32))
    h = pack(np.array([a for a, _ in head], np.uint32), np.array([b for _, b in head], np.uint32))
    outs_o, it_o, deltas_o = oracle.seminaive(plan, [e, h])
    assert M * (2 ** 32) + M in set(int(x) for x in outs_o[1])
    for route in (ROUTE_HASH, ROUTE_JOIN):
        _note(f"all-ones initial head plan={plan_name} route={route}")
        dev = [p.create_buffer_from_packed(e), p.create_buffer_from_packed(h)]
        outs, st = p.fixpoint(plan, dev, route=route)
        assert st["route"] == route
        assert np.array_equal(p.download_packed(outs[1]), outs_o[1]), route
        assert outs[1].is_canonical()
        assert (st["iterations"], st["delta_sizes"]) == (it_o, deltas_o), route


def test_fj_delta_sparse_all_ones_in_full(provider):
    """The one-step sparse operator over a full relation holding (M, M): that
    tuple is not novel."""
    p = provider
    M = 0xFFFFFFFF
    delta = p.create_buffer_from_u32_columns([np.array([M, 4], np.uint32), np.array([5, 5], np.uint32)])
    edge = p.create_buffer_from_u32_columns([np.array([5, 5], np.uint32), np.array([M, 6], np.uint32)])
    full = p.create_buffer_from_u32_columns([np.array([M, 4], np.uint32), np.array([M, 6], np.uint32)])
    out = p.fj_delta_sparse_novel_u32_recorded(delta, edge, full, FJ_DELTA_CANONICAL)
    # candidates (M, M), (M, 6), (4, M), (4, 6); (M, M) and (4, 6) are in full
    assert p.download_rows(out) == [(4, M), (M, 6)]


def test_hash_route_empty_and_unsupported(provider):
    p = provider
    out, st = _tc(p, [], [], ROUTE_HASH)
    assert out.num_rows() == 0 and st["iterations"] == 1 and st["delta_sizes"] == [0, 0]
    # a body of four atoms is beyond the hash route's two hops
    import chain_plans as cp
    s, d = datagen.random_digraph(100, 150, 3)
    e = p.create_buffer_from_u32_columns([np.asarray(s, np.uint32), np.asarray(d, np.uint32)])
    with pytest.raises(XlogError) as ex:
        p.fixpoint(cp.quad_plan(), [e, e, None], route=ROUTE_HASH)
    assert ex.value.status == UNSUPPORTED


def test_hash_route_c1_fixture(provider):
    p = provider
    fx = FIX["c1"]
    src, dst = datagen.random_digraph(fx["vertices"], fx["edges"], datagen.seed_for(1))
    out, st = _tc(p, src, dst, ROUTE_HASH)
    bits = np.unpackbits(np.load(GOLDEN / "c1_closure.npz")["bits"], axis=1)[:, :fx["vertices"]]
    xs, zs = np.nonzero(bits)
    assert np.array_equal(p.download_packed(out), np.sort(pack(xs.astype(np.uint32), zs.astype(np.uint32))))
    assert (st["iterations"], st["delta_sizes"]) == (fx["iterations"], fx["delta_sizes"])
    assert st["host_waits"] <= st["iterations"] + 8


def _sparse_graph(cfg):
    src, dst = datagen.random_digraph(cfg["n_vertices"], cfg["n_edges"], datagen.seed_for(6))
    return datagen.sparse_ids(src), datagen.sparse_ids(dst)


def _check_fixture(p, out, st, fx):
    assert out.num_rows() == fx["tuples"]
    assert st["iterations"] == fx["iterations"]
    assert st["delta_sizes"] == fx["delta_sizes"]
    assert p.digest(out) == fx["digest"]


def test_tcs_sparse_ids_fixture_auto_and_join(provider):
    # 2^20 vertices with ids spread over the u32 range: beyond the bit-matrix domain, AUTO takes the hash route
    p = provider
    fx = FIX["tcs"]
    s, d = _sparse_graph(datagen.TCS)
    assert _fnv_inputs(s, d) == fx["input_digest"]
    _note("tcs: AUTO")
    out, st = _tc(p, s, d, ROUTE_AUTO)
    assert st["route"] == ROUTE_HASH
    _check_fixture(p, out, st, fx)
    assert st["host_waits"] <= st["iterations"] + 8
    _note("tcs: join route")
    out_j, st_j = _tc(p, s, d, ROUTE_JOIN)
    _check_fixture(p, out_j, st_j, fx)


def test_tcs_crit_sparse_ids_fixture(provider):
    # critical G(2^20, 2^20): 418 iterations, ~2.6e8 tuples, one read-back per iteration
    p = provider
    fx = FIX["tcs_crit"]
    s, d = _sparse_graph(datagen.TCS_CRIT)
    _note("tcs_crit: hash route")
    out, st = _tc(p, s, d, ROUTE_HASH)
    _check_fixture(p, out, st, fx)
    assert st["host_waits"] <= st["iterations"] + 8


def test_hash_route_c4_fixture(provider):
    # C4 (9.5e8 tuples, 23 iterations) forced onto the hash route: the table grows to 2^31 slots
    p = provider
    fx = FIX["c4"]
    src, dst = datagen.random_digraph(fx["vertices"], fx["edges"], datagen.seed_for(4))
    _note("c4: hash route")
    out, st = _tc(p, src, dst, ROUTE_HASH)
    _check_fixture(p, out, st, fx)
    del out
    p.trim()


def _fnv_inputs(*arrays):
    h = 0
    for a in arrays:
        h = ((h * 0x100000001B3) ^ oracle.fnv1a64(np.asarray(a).astype(np.uint64))) & ((1 << 64) - 1)
    return h


# ---- the one-step sparse operator ---------------------------------------------
def _fj_expected(delta, edge, full):
    j = oracle.join_project(delta, edge, 1, 0, 0, 3)
    return oracle.diff_sorted(oracle.sort_dedup(j), oracle.sort_dedup(full))


def test_fj_delta_sparse_matches_dense(provider):
    p = provider
    rng = np.random.default_rng(11)
    dom = 3000
    edge = oracle.sort_dedup(pack(rng.integers(0, dom, 20_000, dtype=np.uint32),
                                  rng.integers(0, dom, 20_000, dtype=np.uint32)))
    delta = pack(rng.integers(0, dom, 8_000, dtype=np.uint32), rng.integers(0, dom, 8_000, dtype=np.uint32))
    full = pack(rng.integers(0, dom, 200_000, dtype=np.uint32), rng.integers(0, dom, 200_000, dtype=np.uint32))
    E, D, F = (p.create_buffer_from_packed(x) for x in (edge, delta, full))
    exp = _fj_expected(delta, edge, full)
    sp = p.fj_delta_sparse_novel_u32_recorded(D, E, F, FJ_DELTA_CANONICAL)
    dn = p.fj_delta_novel_u32_recorded(D, E, F, FJ_DELTA_CANONICAL, dom)
    assert sp.is_canonical()
    assert np.array_equal(p.download_packed(sp), exp)
    assert np.array_equal(p.download_packed(dn), exp)
    # column roles: delta stored (y, x), full and head stored (z, x)
    swap = lambda k: (k << np.uint64(32)) | (k >> np.uint64(32))  # noqa: E731
    out2 = p.fj_delta_sparse_novel_u32_recorded(p.create_buffer_from_packed(swap(delta)), E,
                                                p.create_buffer_from_packed(swap(full)), (1, 0, 1, 0))
    assert np.array_equal(p.download_packed(out2), np.sort(swap(exp)))
    # delta stored (x, y), full and head stored (z, x)
    out3 = p.fj_delta_sparse_novel_u32_recorded(D, E, p.create_buffer_from_packed(swap(full)), (0, 1, 1, 0))
    assert np.array_equal(p.download_packed(out3), np.sort(swap(exp)))


def test_fj_delta_sparse_large_ids(provider):
    # ids over the whole u32 range (no dense domain exists); the all-ones id included
    p = provider
    rng = np.random.default_rng(21)
    ids = datagen.sparse_ids(np.arange(5000))
    e_s, e_d = ids[rng.integers(0, 5000, 30_000)], ids[rng.integers(0, 5000, 30_000)]
    edge = oracle.sort_dedup(pack(e_s, e_d))
    delta = pack(ids[rng.integers(0, 5000, 10_000)], ids[rng.integers(0, 5000, 10_000)])
    full = pack(ids[rng.integers(0, 5000, 100_000)], ids[rng.integers(0, 5000, 100_000)])
    E, D, F = (p.create_buffer_from_packed(x) for x in (edge, delta, full))
    out = p.fj_delta_sparse_novel_u32_recorded(D, E, F)
    assert np.array_equal(p.download_packed(out), _fj_expected(delta, edge, full))


def test_fj_delta_sparse_budget_and_empty(provider):
    p = provider
    E = p.create_buffer_from_u32_columns([[0, 1], [1, 2]])
    D = p.create_buffer_from_u32_columns([[0], [0]])
    F = p.create_empty_buffer(2)
    assert p.download_rows(p.fj_delta_sparse_novel_u32_recorded(D, E, F)) == [(0, 1)]
    assert p.fj_delta_sparse_novel_u32_recorded(p.create_empty_buffer(2), E, F).num_rows() == 0
    # a table above the budget declines (the reference's Ok(None))
    assert p.fj_delta_sparse_novel_u32_recorded(D, E, F, FJ_DELTA_CANONICAL, max_table_bytes=1024) is None
    assert p.fj_delta_sparse_novel_u32_recorded(D, E, F, FJ_DELTA_CANONICAL, max_table_bytes=1 << 30) is not None
    with pytest.raises(XlogError):
        p.fj_delta_sparse_novel_u32_recorded(D, E, F, (0, 0, 0, 1))
    with pytest.raises(XlogError):
        p.fj_delta_sparse_novel_u32_recorded(p.create_buffer_from_u32_columns([[0]]), E, F)
