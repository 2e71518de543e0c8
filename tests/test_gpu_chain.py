"""GPU parity of the dense chain-rule route of the fixpoint (any program whose
rule bodies are paths of binary relations) against the CPU oracle, which the
CPU suite pins against boolean-matrix closed forms.  Every program also runs
on the join route, and both must agree to the tuple, the iteration count and
every per-iteration delta size."""
import sys

import numpy as np
import pytest

import oracle
from xlog_amd import ROUTE_AUTO, ROUTE_BITMAP, ROUTE_JOIN, XlogError, andersen_plan, datagen, pack, tc_plan

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


def _parity(p, name, plan, rels, idb, routes=(ROUTE_BITMAP, ROUTE_JOIN)):
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
    _parity(provider, "quad", cp.quad_plan(), [pack(a_s, a_d), pack(b_s, b_d), None], [2])


def test_scrambled_body_order(provider):
    """A path whose atoms are listed out of order: the chain route runs it and matches the oracle on the
    same program in path order; the join route (left-deep, like the reference's lowering) rejects it."""
    p = provider
    a_s, a_d = _graph(600, 900, 13)
    b_s, b_d = _graph(600, 500, 14)
    rels = [pack(a_s, a_d), pack(b_s, b_d), None]
    outs_o, it_o, deltas_o = oracle.seminaive(cp.ordered_chain_plan(), rels)
    outs, st = _run(p, cp.scrambled_chain_plan(), rels, ROUTE_AUTO)
    assert st["route"] == ROUTE_BITMAP
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
    AUTO falls back to the join route and an explicit bitmap request is refused."""
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
    outs, st = _run(p, tc_plan(), rels, ROUTE_AUTO)
    assert st["route"] == ROUTE_JOIN
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
