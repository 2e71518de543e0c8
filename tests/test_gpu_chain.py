"""GPU parity of the routes that take chain-rule programs (rule bodies that are
paths of binary relations) against the CPU oracle, which the CPU suite pins
against boolean-matrix closed forms: the dense bitmap route, the join route,
and the hash-set route (bodies of up to three atoms, two hops around the delta
atom).  All must agree to the tuple, the iteration count and every
per-iteration delta size.  Programs over ids spread across u32 take the
hash-set route under AUTO."""
import sys

import numpy as np
import pytest

import oracle
from xlog_amd import (ROUTE_AUTO, ROUTE_BITMAP, ROUTE_HASH, ROUTE_JOIN, XlogError, andersen_plan, datagen, pack,
                      tc_plan)

import chain_plans as cp

pytestmark = pytest.mark.gpu

UNSUPPORTED, ITERATION_LIMIT = 7, 4


def _note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _graph(n, m, seed):
    s, d = datagen.random_digraph(n, m, seed)
    return np.asarray(s, np.uint32), np.asarray(d, np.uint32)


def _run(p, plan, rels, route, **kw):
    dev = [p.create_buffer_from_packed(r) if r is not None else None for r in rels]
    return p.fixpoint(plan, dev, route=route, **kw)


def _parity(p, name, plan, rels, idb, routes=(ROUTE_BITMAP, ROUTE_JOIN, ROUTE_HASH)):
    outs_o, it_o, deltas_o = oracle.seminaive(plan, rels)
    for route in routes:
        _note(f"chain {name} route={route}")
        outs, st = _run(p, plan, rels, route)
        assert st["route"] == route
        for q in idb:
            assert np.array_equal(p.download_packed(outs[q]), outs_o[q]), f"{name} route {route} pred {q}"
        assert st["iterations"] == it_o
        assert st["delta_sizes"] == deltas_o


@pytest.mark.parametrize("n,m,seed", [(300, 600, 1), (1000, 2500, 2)])
def test_tc_variants(provider, n, m, seed):
    s, d = _graph(n, m, seed)
    e = pack(s, d)
    _parity(provider, "left tc", cp.left_tc_plan(), [e, None], [1])
    _parity(provider, "nonlinear tc", cp.nonlinear_tc_plan(), [e, None], [1])


def test_tc_with_initial_head(provider):
    """A non-empty head relation leaves the transitive-closure bitmap kernel to the chain route."""
    s, d = _graph(800, 1600, 3)
    hs, hd = _graph(800, 300, 4)
    _parity(provider, "tc initial head", tc_plan(), [pack(s, d), pack(hs, hd)], [1])
    outs, st = _run(provider, tc_plan(), [pack(s, d), pack(hs, hd)], ROUTE_AUTO)
    assert st["route"] == ROUTE_BITMAP


@pytest.mark.parametrize("n,seed", [(500, 5), (3000, 6)])
def test_same_generation(provider, n, seed):
    rng = np.random.default_rng(seed)
    child = np.arange(1, n, dtype=np.uint32)
    parent = np.array([rng.integers(max(0, int(c) - 40), int(c)) for c in child], dtype=np.uint32)
    fs = rng.integers(0, n, n // 4).astype(np.uint32)
    fd = rng.integers(0, n, n // 4).astype(np.uint32)
    _parity(provider, "sg up/down", cp.same_generation_plan(),
            [pack(fs, fd), pack(child, parent), pack(parent, child), None], [3])
    _parity(provider, "sg par backward", cp.same_generation_par_plan(), [pack(fs, fd), pack(child, parent), None], [2])


@pytest.mark.parametrize("n,m,seed", [(200, 320, 7), (2000, 3500, 8)])
def test_parity_mutual_recursion(provider, n, m, seed):
    s, d = _graph(n, m, seed)
    _parity(provider, "parity", cp.parity_plan(), [pack(s, d), None, None], [1, 2])
    _parity(provider, "parity left-linear", cp.parity_left_plan(), [pack(s, d), None, None], [1, 2])


@pytest.mark.parametrize("n,m,seed", [(150, 200, 9), (1500, 2200, 10)])
def test_symmetric_closure(provider, n, m, seed):
    s, d = _graph(n, m, seed)
    _parity(provider, "symmetric", cp.symmetric_plan(), [pack(s, d), None], [1])


@pytest.mark.parametrize("n,seed", [(100, 11), (400, 12)])
def test_four_atom_chain(provider, n, seed):
    a_s, a_d = _graph(n, n, seed)
    b_s, b_d = _graph(n, n // 2, seed + 100)
    rels = [pack(a_s, a_d), pack(b_s, b_d), None]
    _parity(provider, "quad", cp.quad_plan(), rels, [2], routes=(ROUTE_BITMAP, ROUTE_JOIN))
    with pytest.raises(XlogError) as ex:  # four atoms: three hops
        _run(provider, cp.quad_plan(), rels, ROUTE_HASH)
    assert ex.value.status == UNSUPPORTED


def test_scrambled_body_order(provider):
    """A path whose atoms are listed out of order: the chain route runs it and matches the oracle on the
    same program in path order; the join route (left-deep, like the reference's lowering) rejects it."""
    p = provider
    a_s, a_d = _graph(600, 900, 13)
    b_s, b_d = _graph(600, 500, 14)
    rels = [pack(a_s, a_d), pack(b_s, b_d), None]
    outs_o, it_o, deltas_o = oracle.seminaive(cp.ordered_chain_plan(), rels)
    for route, taken in ((ROUTE_AUTO, ROUTE_BITMAP), (ROUTE_HASH, ROUTE_HASH)):
        outs, st = _run(p, cp.scrambled_chain_plan(), rels, route)
        assert st["route"] == taken
        assert np.array_equal(p.download_packed(outs[2]), outs_o[2])
        assert st["iterations"] == it_o and st["delta_sizes"] == deltas_o
    with pytest.raises(XlogError) as ex:
        _run(p, cp.scrambled_chain_plan(), rels, ROUTE_JOIN)
    assert ex.value.status == UNSUPPORTED


@pytest.mark.parametrize("n_vars,n_facts", [(50, 150), (400, 1500), (2000, 8000)])
def test_andersen_both_routes(provider, n_vars, n_facts):
    f = datagen.andersen(n_vars, n_facts, 1.5, datagen.seed_for(5))
    rels = [pack(*f[k]) for k in ("assign", "addressOf", "load", "store")] + [None]
    _parity(provider, f"andersen {n_vars}", andersen_plan(), rels, [4])


def test_domain_edges(provider):
    """Ids at the top of the 2^17 domain (2048-word rows, more stripes than waves), then one id past it:
    AUTO takes the hash-set route (the join route when a join-row limit is set) and an explicit bitmap
    request is refused."""
    p = provider
    rng = np.random.default_rng(15)
    ids = np.sort(rng.choice(1 << 17, 400, replace=False)).astype(np.uint32)
    ids[-1] = (1 << 17) - 1
    s = ids[rng.integers(0, 400, 900)]
    d = ids[rng.integers(0, 400, 900)]
    hs, hd = ids[rng.integers(0, 400, 50)], ids[rng.integers(0, 400, 50)]
    _parity(p, "tc top of domain", tc_plan(), [pack(s, d), pack(hs, hd)], [1])
    _parity(p, "symmetric top of domain", cp.symmetric_plan(), [pack(s, d), None], [1])
    big = np.array([1 << 17], np.uint32)
    rels = [pack(np.append(s, big), np.append(d, ids[:1])), pack(hs, hd)]
    outs_o, it_o, deltas_o = oracle.seminaive(tc_plan(), rels)
    for kw, taken in (({}, ROUTE_HASH), ({"max_join_rows": 1 << 40}, ROUTE_JOIN)):
        outs, st = _run(p, tc_plan(), rels, ROUTE_AUTO, **kw)
        assert st["route"] == taken
        assert np.array_equal(p.download_packed(outs[1]), outs_o[1])
        assert st["iterations"] == it_o and st["delta_sizes"] == deltas_o
    with pytest.raises(XlogError) as ex:
        _run(p, tc_plan(), rels, ROUTE_BITMAP)
    assert ex.value.status == UNSUPPORTED


def test_chain_route_errors(provider):
    p = provider
    s, d = datagen.chain(30)
    e = pack(np.asarray(s, np.uint32), np.asarray(d, np.uint32))
    h = pack(np.array([0], np.uint32), np.array([1], np.uint32))
    with pytest.raises(XlogError) as ex:
        _run(p, tc_plan(), [e, h], ROUTE_BITMAP, max_iterations=5)
    assert ex.value.status == ITERATION_LIMIT
    assert ex.value.stats["iterations"] == 5
    # an intersection body is no chain
    both = [1, 2, 0, 1, 2, 0, 0, 1, 1, 0, 1]
    with pytest.raises(XlogError) as ex:
        _run(p, both, [e, e, None], ROUTE_BITMAP)
    assert ex.value.status == UNSUPPORTED


def _spread(*cols):
    """The same relations with every id mapped by the bijection onto u32 that the sparse fixtures use."""
    return [datagen.sparse_ids(np.asarray(c, np.uint32)) for c in cols]


def _sparse_parity(p, name, plan, rels, idb, auto=ROUTE_HASH):
    outs_o, it_o, deltas_o = oracle.seminaive(plan, rels)
    for route in (ROUTE_AUTO, ROUTE_HASH, ROUTE_JOIN):
        _note(f"sparse {name} route={route}")
        outs, st = _run(p, plan, rels, route)
        assert st["route"] == (auto if route == ROUTE_AUTO else route)
        for q in idb:
            assert np.array_equal(p.download_packed(outs[q]), outs_o[q]), f"{name} route {route} pred {q}"
            assert outs[q].is_canonical()
        assert st["iterations"] == it_o
        assert st["delta_sizes"] == deltas_o
        if st["route"] == ROUTE_HASH:  # one read-back per iteration, plus set-up
            assert st["host_waits"] <= 2 * st["iterations"] + 40, st


@pytest.mark.parametrize("n,m,seed", [(400, 700, 21), (1200, 1900, 22)])
def test_sparse_ids_programs(provider, n, m, seed):
    """Programs over ids spread across u32 (beyond the bitmap route's 2^17) on the hash-set route."""
    p = provider
    s, d = _spread(*_graph(n, m, seed))
    e = pack(s, d)
    _sparse_parity(p, "nonlinear tc", cp.nonlinear_tc_plan(), [e, None], [1])
    _sparse_parity(p, "left tc", cp.left_tc_plan(), [e, None], [1])
    _sparse_parity(p, "parity", cp.parity_plan(), [e, None, None], [1, 2])
    _sparse_parity(p, "symmetric", cp.symmetric_plan(), [e, None], [1])
    hs, hd = _spread(*_graph(n, m // 5, seed + 50))
    _sparse_parity(p, "tc initial head", tc_plan(), [e, pack(hs, hd)], [1])


@pytest.mark.parametrize("n,seed", [(600, 23), (4000, 24)])
def test_sparse_ids_same_generation(provider, n, seed):
    rng = np.random.default_rng(seed)
    child = np.arange(1, n, dtype=np.uint32)
    parent = np.array([rng.integers(max(0, int(c) - 40), int(c)) for c in child], dtype=np.uint32)
    fs, fd = rng.integers(0, n, n // 4).astype(np.uint32), rng.integers(0, n, n // 4).astype(np.uint32)
    c2, p2, f2s, f2d = _spread(child, parent, fs, fd)
    _sparse_parity(provider, "sg up/down", cp.same_generation_plan(), [pack(f2s, f2d), pack(c2, p2), pack(p2, c2), None], [3])
    _sparse_parity(provider, "sg par backward", cp.same_generation_par_plan(), [pack(f2s, f2d), pack(c2, p2), None], [2])


@pytest.mark.parametrize("n_vars,n_facts", [(300, 1000), (3000, 12000)])
def test_sparse_ids_andersen(provider, n_vars, n_facts):
    """Andersen's points-to (the three-atom load and store rules: two hops around the delta atom, with
    the full relation read through its indexes in both directions) over spread ids.  AUTO keeps such
    rules (two IDB atoms in a three-atom body) on the join route."""
    f = datagen.andersen(n_vars, n_facts, 1.5, datagen.seed_for(5))
    rels = [pack(*_spread(*f[k])) for k in ("assign", "addressOf", "load", "store")] + [None]
    _sparse_parity(provider, f"andersen {n_vars}", andersen_plan(), rels, [4], auto=ROUTE_JOIN)


def test_hash_route_programs_rerun(provider, monkeypatch):
    """A 64-slot table and 100 appends per attempt: every iteration of every head goes through the
    grow-and-rerun protocol, with several variants sharing one head."""
    p = provider
    monkeypatch.setenv("XLOG_HIP_HASH_SLOTS", "64")
    monkeypatch.setenv("XLOG_HIP_HASH_APPENDS", "100")
    f = datagen.andersen(400, 1500, 1.5, datagen.seed_for(5))
    rels = [pack(*f[k]) for k in ("assign", "addressOf", "load", "store")] + [None]
    outs_o, it_o, deltas_o = oracle.seminaive(andersen_plan(), rels)
    outs, st = _run(p, andersen_plan(), rels, ROUTE_HASH)
    assert np.array_equal(p.download_packed(outs[4]), outs_o[4])
    assert st["iterations"] == it_o and st["delta_sizes"] == deltas_o
    s, d = _graph(500, 900, 25)
    outs_o, it_o, deltas_o = oracle.seminaive(cp.parity_plan(), [pack(s, d), None, None])
    outs, st = _run(p, cp.parity_plan(), [pack(s, d), None, None], ROUTE_HASH)
    for q in (1, 2):
        assert np.array_equal(p.download_packed(outs[q]), outs_o[q])
    assert st["iterations"] == it_o and st["delta_sizes"] == deltas_o


def test_hash_route_queued_steps(provider, monkeypatch):
    """Linear programs (no IDB atom read in full by a variant) queue several iterations per read-back on
    the hash-set route: the same relations and deltas as one read-back per iteration, with fewer waits."""
    p = provider
    s, d = _spread(*_graph(1500, 1700, 26))
    for name, plan, rels, idb in (("left tc", cp.left_tc_plan(), [pack(s, d), None], [1]),
                                  ("parity", cp.parity_plan(), [pack(s, d), None, None], [1, 2])):
        outs_o, it_o, deltas_o = oracle.seminaive(plan, rels)
        waits = {}
        for queue in ("1", "8"):
            monkeypatch.setenv("XLOG_HIP_HASH_QUEUE", queue)
            _note(f"queued {name} queue={queue}")
            outs, st = _run(p, plan, rels, ROUTE_HASH)
            for q in idb:
                assert np.array_equal(p.download_packed(outs[q]), outs_o[q]), f"{name} queue {queue} pred {q}"
            assert st["iterations"] == it_o and st["delta_sizes"] == deltas_o
            waits[queue] = st["host_waits"]
        assert it_o > 16 and waits["8"] < waits["1"] - it_o // 2, (name, it_o, waits)


def test_hash_route_queued_indexed(provider, monkeypatch):
    """Programs whose variants read an IDB relation in full (non-linear closure, Andersen) queue on the
    hash-set route too: before each queued step the relation's appends of the step before are sorted and
    merged into it and its indexes rebuilt, all on the device.  The same relations and deltas as one
    read-back per iteration, with fewer waits; then with 100 appends per step in a 64-slot table, so that
    queued steps overflow and are rerun from the host."""
    p = provider
    s, d = _spread(*_graph(1500, 2600, 28))
    f = datagen.andersen(800, 3000, 1.5, datagen.seed_for(5))
    progs = (("nonlinear tc", cp.nonlinear_tc_plan(), [pack(s, d), None], [1]),
             ("andersen", andersen_plan(), [pack(*f[k]) for k in ("assign", "addressOf", "load", "store")] + [None],
              [4]))
    for name, plan, rels, idb in progs:
        outs_o, it_o, deltas_o = oracle.seminaive(plan, rels)
        waits = {}
        for queue in ("1", "8"):
            monkeypatch.setenv("XLOG_HIP_HASH_QUEUE", queue)
            _note(f"queued indexed {name} queue={queue}")
            outs, st = _run(p, plan, rels, ROUTE_HASH)
            for q in idb:
                assert np.array_equal(p.download_packed(outs[q]), outs_o[q]), f"{name} queue {queue} pred {q}"
                assert outs[q].is_canonical()
            assert st["iterations"] == it_o and st["delta_sizes"] == deltas_o
            waits[queue] = st["host_waits"]
        _note(f"queued indexed {name}: {it_o} iterations, host waits {waits}")
        assert waits["8"] < waits["1"], (name, it_o, waits)
    monkeypatch.delenv("XLOG_HIP_HASH_QUEUE")
    monkeypatch.setenv("XLOG_HIP_HASH_SLOTS", "64")
    monkeypatch.setenv("XLOG_HIP_HASH_APPENDS", "100")
    for name, plan, rels, idb in progs:
        _note(f"queued indexed overflow {name}")
        outs_o, it_o, deltas_o = oracle.seminaive(plan, rels)
        outs, st = _run(p, plan, rels, ROUTE_HASH)
        for q in idb:
            assert np.array_equal(p.download_packed(outs[q]), outs_o[q]), name
        assert st["iterations"] == it_o and st["delta_sizes"] == deltas_o


def test_hash_route_queued_overflow(provider, monkeypatch):
    """Queued steps of at most 100 appends each in a 64-slot table: steps overflow inside the queue (the
    later ones then do nothing), and the half-load budget cuts steps short; each such step is rerun
    from the host's sizes and the queue resumes."""
    p = provider
    monkeypatch.setenv("XLOG_HIP_HASH_SLOTS", "64")
    monkeypatch.setenv("XLOG_HIP_HASH_APPENDS", "100")
    s, d = _spread(*_graph(900, 1000, 27))
    for name, plan, rels, idb in (("left tc", cp.left_tc_plan(), [pack(s, d), None], [1]),
                                  ("symmetric", cp.symmetric_plan(), [pack(s, d), None], [1])):
        _note(f"queued overflow {name}")
        outs_o, it_o, deltas_o = oracle.seminaive(plan, rels)
        outs, st = _run(p, plan, rels, ROUTE_HASH)
        for q in idb:
            assert np.array_equal(p.download_packed(outs[q]), outs_o[q]), name
        assert st["iterations"] == it_o and st["delta_sizes"] == deltas_o


def test_staged_emit(provider, monkeypatch):
    """The bitmap route's final emit of dense rows stages each group of 64 words in LDS and writes it with
    line-aligned stores (rows of 8192 tuples or more on average).  A hub graph (every vertex to 0 and back)
    closes to every pair of its 8,200 vertices (rows of 8,200 tuples, 129-word rows); then programs of the
    other tests with the staged emit forced on every row size (XLOG_HIP_EMIT_STAGED_ROW=0), including
    2048-word rows (four chunks of 512 words per row)."""
    p = provider
    v = 8200
    others = np.arange(1, v, dtype=np.uint32)
    s = np.concatenate([others, np.zeros(v - 1, np.uint32)])
    d = np.concatenate([np.zeros(v - 1, np.uint32), others])
    _note("staged emit: hub graph")
    outs, st = _run(p, tc_plan(), [pack(s, d), None], ROUTE_BITMAP)
    got = p.download_packed(outs[1])
    x = np.arange(v, dtype=np.uint64)
    assert np.array_equal(got, ((x[:, None] << np.uint64(32)) | x[None, :]).ravel())
    monkeypatch.setenv("XLOG_HIP_EMIT_STAGED_ROW", "0")
    for n, m, seed in ((300, 600, 1), (1000, 2500, 2)):
        s, d = _graph(n, m, seed)
        _parity(p, f"staged emit tc {n}", cp.left_tc_plan(), [pack(s, d), None], [1], routes=(ROUTE_BITMAP,))
    rng = np.random.default_rng(15)
    ids = np.sort(rng.choice(1 << 17, 400, replace=False)).astype(np.uint32)
    ids[-1] = (1 << 17) - 1
    s, d = ids[rng.integers(0, 400, 900)], ids[rng.integers(0, 400, 900)]
    _parity(p, "staged emit top of domain", tc_plan(), [pack(s, d), None], [1], routes=(ROUTE_BITMAP,))
    f = datagen.andersen(400, 1500, 1.5, datagen.seed_for(5))
    rels = [pack(*f[k]) for k in ("assign", "addressOf", "load", "store")] + [None]
    _parity(p, "staged emit andersen", andersen_plan(), rels, [4], routes=(ROUTE_BITMAP,))
