"""GPU parity of the semi-naive fixpoint driver (both transitive-closure routes
and the generic join route) against the CPU oracle, the BFS closed form and
the reference's own recursion tests."""
import sys

import numpy as np
import pytest

import oracle
from xlog_amd import ROUTE_BITMAP, ROUTE_JOIN, XlogError, andersen_plan, copy_points_to_plan, datagen, pack, tc_plan

pytestmark = pytest.mark.gpu

ROUTES = [ROUTE_BITMAP, ROUTE_JOIN]


def _note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _tc(p, src, dst, route):
    e = p.create_buffer_from_u32_columns([np.asarray(src, np.uint32), np.asarray(dst, np.uint32)])
    outs, st = p.fixpoint(tc_plan(), [e, None], route=route)
    assert st["route"] == route
    return p.download_packed(outs[1]), st


@pytest.mark.parametrize("route", ROUTES)
def test_tc_reference_kat_chain(provider, route):
    """e2e_integration_tests.rs:247-300 / examples/xlog/00-basics/01_tc_reachability.xlog"""
    rel, st = _tc(provider, [1, 2, 3], [2, 3, 4], route)
    pairs = [(int(k >> 32), int(k & 0xFFFFFFFF)) for k in rel]
    assert sorted(z for x, z in pairs if x == 1) == [2, 3, 4]
    assert len(pairs) == 6 and st["iterations"] == 3


@pytest.mark.parametrize("route", ROUTES)
def test_tc_reference_irregular_digraph(provider, route):
    """test_factorized_delta_e2e.rs:256-272 edges, oracle_tc :218-241 semantics."""
    edges = [(0, 1), (1, 2), (2, 0), (3, 4), (3, 5), (4, 6), (5, 6), (6, 7), (8, 0), (8, 3), (8, 7), (8, 9),
             (9, 9), (11, 1)]
    src, dst = zip(*edges)
    rel, st = _tc(provider, src, dst, route)
    bfs = oracle.bfs_tc(12, src, dst)
    assert np.array_equal(rel, bfs["relation"])
    assert st["iterations"] == bfs["iterations"]


@pytest.mark.parametrize("route", ROUTES)
@pytest.mark.parametrize("shape,n", [("chain", 50), ("cycle", 40), ("kbip", 30), ("empty", 0)])
def test_tc_closed_forms(provider, route, shape, n):
    _note(f"tc closed form {shape} n={n} route={route}")
    if shape == "chain":
        src, dst = datagen.chain(n)
        exp_n, exp_it = (n - 1) * n // 2, n - 1
    elif shape == "cycle":
        src, dst = datagen.cycle(n)
        exp_n, exp_it = n * n, n
    elif shape == "kbip":
        src, dst = datagen.complete_bipartite(n)
        exp_n, exp_it = n * n, 1
    else:
        src, dst = np.zeros(0, np.uint32), np.zeros(0, np.uint32)
        exp_n, exp_it = 0, 1
    if shape == "empty" and route == ROUTE_BITMAP:
        route = ROUTE_JOIN  # an empty edge set has no domain for the bitmap route
    rel, st = _tc(provider, src, dst, route)
    assert len(rel) == exp_n
    assert st["iterations"] == exp_it


@pytest.mark.parametrize("route", ROUTES)
def test_tc_config1_full(provider, route):
    """Config 1: 1,000 vertices, 5,000 distinct edges; bit-exact relation, count,
    iterations and per-iteration delta sizes against the oracle and BFS."""
    src, dst = datagen.random_digraph(1000, 5000, datagen.seed_for(1))
    rel, st = _tc(provider, src, dst, route)
    bfs = oracle.bfs_tc(1000, src, dst)
    assert np.array_equal(rel, bfs["relation"])
    assert st["iterations"] == bfs["iterations"] == 9
    _, it, deltas = oracle.seminaive(tc_plan(), [pack(src, dst), None])
    assert st["delta_sizes"] == deltas
    assert [int(x) for x in bfs["dist_count"][1:it + 1]] == deltas[:it]


def test_tc_reference_random_graph_with_duplicates(provider):
    """The reference bench's own generator keeps duplicate edges and self-loops."""
    src, dst = datagen.ref_random_graph(300, 1500, 42)
    for route in ROUTES:
        rel, st = _tc(provider, src, dst, route)
        bfs = oracle.bfs_tc(300, src, dst)
        assert np.array_equal(rel, bfs["relation"]) and st["iterations"] == bfs["iterations"]


def test_points_to_copy_kat(provider):
    """real_world_tests.rs:739-800: {(3,1),(4,2),(5,1),(6,1)}."""
    p = provider
    addr = p.create_buffer_from_u32_columns([[3, 4], [1, 2]])
    copy = p.create_buffer_from_u32_columns([[5, 6], [3, 5]])
    outs, st = p.fixpoint(copy_points_to_plan(), [addr, copy, None])
    assert sorted(p.download_rows(outs[2])) == [(3, 1), (4, 2), (5, 1), (6, 1)]


@pytest.mark.parametrize("n_vars,n_facts", [(50, 150), (400, 1500), (2000, 8000)])
def test_andersen_small_vs_oracle(provider, n_vars, n_facts):
    p = provider
    _note(f"andersen n_vars={n_vars} n_facts={n_facts}")
    f = datagen.andersen(n_vars, n_facts, 1.5, datagen.seed_for(5))
    rels = [pack(*f["assign"]), pack(*f["addressOf"]), pack(*f["load"]), pack(*f["store"])]
    outs_o, it_o, deltas_o = oracle.seminaive(andersen_plan(), rels + [None])
    dev = [p.create_buffer_from_packed(r) for r in rels] + [None]
    outs, st = p.fixpoint(andersen_plan(), dev)
    assert np.array_equal(p.download_packed(outs[4]), outs_o[4])
    assert st["iterations"] == it_o
    assert st["delta_sizes"] == deltas_o


def test_chunked_join_fold_parity(provider, monkeypatch):
    """Join outputs above the chunk size are produced as sorted sets chunk by
    chunk; forcing tiny chunks must not change any fixpoint result
    (the reference's multi-chunk fold parity, set_ops_tests.rs:524-587)."""
    p = provider
    f = datagen.andersen(400, 1500, 1.5, datagen.seed_for(5))
    rels = [pack(*f[k]) for k in ("assign", "addressOf", "load", "store")]
    outs_o, it_o, deltas_o = oracle.seminaive(andersen_plan(), rels + [None])
    src, dst = datagen.random_digraph(300, 1200, 11)
    tc_o = oracle.bfs_tc(300, src, dst)
    for chunk in ("1", "777", "100000"):
        monkeypatch.setenv("XLOG_HIP_JOIN_CHUNK_ROWS", chunk)
        dev = [p.create_buffer_from_packed(r) for r in rels] + [None]
        outs, st = p.fixpoint(andersen_plan(), dev, route=ROUTE_JOIN)
        assert np.array_equal(p.download_packed(outs[4]), outs_o[4])
        assert st["iterations"] == it_o and st["delta_sizes"] == deltas_o
        e = p.create_buffer_from_u32_columns([src, dst])
        o2, st2 = p.fixpoint(tc_plan(), [e, None], route=ROUTE_JOIN)
        assert np.array_equal(p.download_packed(o2[1]), tc_o["relation"]) and st2["iterations"] == tc_o["iterations"]


def test_iteration_limit_is_an_error(provider):
    src, dst = datagen.chain(20)
    e = provider.create_buffer_from_u32_columns([src, dst])
    for route in ROUTES:
        with pytest.raises(XlogError) as ex:
            provider.fixpoint(tc_plan(), [e, None], route=route, max_iterations=5)
        assert ex.value.status == 4
