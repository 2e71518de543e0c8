"""GPU parity of cyclic rule bodies against the CPU oracle (which the CPU suite
pins against boolean-matrix closed forms): an atom whose two variables are
both bound when it is joined is a join on both keys in the reference's
left-deep lowering (crates/xlog-logic/src/lower.rs build_join_tree /
compute_join_keys), here a filter step of the join route (a lookup of the row
in the atom's index on its first column).  A triangle-shaped body whose head
drops one variable is evaluated by the generic join instead when that reads
less (each row of the atom over the head's variables intersects two sorted
runs; XLOG_HIP_WCOJ=1 / =0 forces it / the left-deep plan): both must give the
oracle's result.  Such bodies are not paths, so AUTO takes the join route and
the bitmap and hash routes decline them."""
import sys

import numpy as np
import pytest

import oracle
from xlog_amd import ROUTE_AUTO, ROUTE_BITMAP, ROUTE_HASH, ROUTE_JOIN, XlogError, datagen, pack

import chain_plans as cp

pytestmark = pytest.mark.gpu

UNSUPPORTED = 7


def _note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _graph(n, m, seed):
    s, d = datagen.random_digraph(n, m, seed)
    return np.asarray(s, np.uint32), np.asarray(d, np.uint32)


def _run(p, plan, rels, route, **kw):
    dev = [p.create_buffer_from_packed(r) if r is not None else None for r in rels]
    return p.fixpoint(plan, dev, route=route, **kw)


def _wcoj(monkeypatch, mode):
    if mode == "default":
        monkeypatch.delenv("XLOG_HIP_WCOJ", raising=False)
    else:
        monkeypatch.setenv("XLOG_HIP_WCOJ", mode)


def _parity(p, name, plan, rels, idb):
    outs_o, it_o, deltas_o = oracle.seminaive(plan, rels)
    for route in (ROUTE_AUTO, ROUTE_JOIN):
        _note(f"cyclic {name} route={route}")
        outs, st = _run(p, plan, rels, route)
        assert st["route"] == ROUTE_JOIN
        for q in idb:
            got = p.download_packed(outs[q])
            assert np.array_equal(got, outs_o[q]), f"{name} route {route} pred {q}"
            assert outs[q].is_canonical()
        assert st["iterations"] == it_o
        assert st["delta_sizes"] == deltas_o
    return outs_o


@pytest.mark.parametrize("wcoj", ["default", "0", "1"])
@pytest.mark.parametrize("n,m,seed", [(200, 1500, 41), (2000, 30000, 42)])
def test_triangle_closure(provider, monkeypatch, n, m, seed, wcoj):
    _wcoj(monkeypatch, wcoj)
    s, d = _graph(n, m, seed)
    outs = _parity(provider, "triangle closure", cp.triangle_closure_plan(), [pack(s, d), None], [1])
    assert len(outs[1]) > len(set(zip(s.tolist(), d.tolist())))  # the closing atom derives rows


@pytest.mark.parametrize("wcoj", ["default", "0", "1"])
@pytest.mark.parametrize("n,m,seed", [(300, 4000, 43), (3000, 60000, 44)])
def test_triangles(provider, monkeypatch, n, m, seed, wcoj):
    _wcoj(monkeypatch, wcoj)
    s, d = _graph(n, m, seed)
    outs = _parity(provider, "triangles", cp.triangles_plan(), [pack(s, d), None], [1])
    assert len(outs[1]) > 0


@pytest.mark.parametrize("n,seed", [(400, 45), (3000, 46)])
def test_filtered_tc(provider, n, seed):
    a_s, a_d = _graph(n, 3 * n, seed)
    k_s, k_d = _graph(n, 6 * n, seed + 100)
    b_s, b_d = _graph(n, 2 * n, seed + 200)
    _parity(provider, "filtered tc", cp.filtered_tc_plan(), [pack(a_s, a_d), pack(k_s, k_d), pack(b_s, b_d), None],
            [3])


@pytest.mark.parametrize("n,seed", [(500, 47), (4000, 48)])
def test_flat_same_generation(provider, n, seed):
    rng = np.random.default_rng(seed)
    child = np.arange(1, n, dtype=np.uint32)
    parent = np.array([rng.integers(max(0, int(c) - 8), int(c)) for c in child], dtype=np.uint32)
    fs = rng.integers(0, n, 4 * n).astype(np.uint32)
    fd = rng.integers(0, n, 4 * n).astype(np.uint32)
    _parity(provider, "flat sg", cp.flat_sg_plan(), [pack(fs, fd), pack(child, parent), None], [2])


def test_sparse_ids_and_edges(provider):
    """Ids spread over u32 (the filter's index lookups hash them), an empty filter atom, and the
    bitmap and hash routes declining a cyclic body."""
    s, d = _graph(1500, 12000, 49)
    ss, sd = datagen.sparse_ids(s), datagen.sparse_ids(d)
    _parity(provider, "sparse triangle closure", cp.triangle_closure_plan(), [pack(ss, sd), None], [1])
    a_s, a_d = _graph(300, 900, 50)
    b_s, b_d = _graph(300, 600, 51)
    _parity(provider, "empty filter atom", cp.filtered_tc_plan(),
            [pack(a_s, a_d), np.zeros(0, np.uint64), pack(b_s, b_d), None], [3])
    for route in (ROUTE_BITMAP, ROUTE_HASH):
        _note(f"cyclic declined route={route}")
        with pytest.raises(XlogError) as ex:
            _run(provider, cp.triangle_closure_plan(), [pack(s, d), None], route)
        assert ex.value.status == UNSUPPORTED
        del ex


def _brute_triangle(plan, n, s, d):
    """The single rule of `plan` (three atoms over variables 0..2 of relation 0, head two of them) by brute
    force over an n x n x n boolean tensor."""
    head, hv0, hv1, nb = plan[1], plan[2], plan[3], plan[4]
    E = np.zeros((n, n), dtype=bool)
    E[s.astype(np.int64), d.astype(np.int64)] = True
    T = np.ones((n, n, n), dtype=bool)
    for j in range(nb):
        _, a, b = plan[5 + 3 * j: 8 + 3 * j]
        shape = [1, 1, 1]
        shape[a], shape[b] = n, n
        M = E if a < b else E.T  # M[i, k] indexed by (min axis, max axis)
        T &= M.reshape(shape)
    (w,) = {0, 1, 2} - {hv0, hv1}
    R = T.any(axis=w)  # axes in increasing order of the remaining variables
    if hv0 > hv1:
        R = R.T
    x, z = np.nonzero(R)
    return np.sort(pack(x.astype(np.uint32), z.astype(np.uint32)))


@pytest.mark.parametrize("wcoj", ["default", "0", "1"])
def test_triangle_orientations(provider, monkeypatch, wcoj):
    """Triangle bodies with their atoms in every column orientation and body order (the generic join's index
    columns and the closing atom's word order follow the atoms), heads over each pair of variables, on a
    graph with a hub, checked against brute force.  One of them has no left-deep plan (after its first
    join three variables are live): the generic join is its only evaluation, and with it forced off
    (XLOG_HIP_WCOJ=0) it is UNSUPPORTED."""
    _wcoj(monkeypatch, wcoj)
    X, Y, Z = 0, 1, 2
    n = 400
    s, d = _graph(n, 5000, 52)
    hub = np.arange(1, n, dtype=np.uint32)
    s = np.concatenate([s, np.zeros(n - 1, np.uint32), hub])
    d = np.concatenate([d, hub, np.zeros(n - 1, np.uint32)])
    e = pack(s, d)
    plans = [
        ([1, 1, X, Z, 3, 0, Y, X, 0, Z, Y, 0, X, Z], True),   # tri(X,Z) :- e(Y,X), e(Z,Y), e(X,Z)
        ([1, 1, Z, X, 3, 0, X, Y, 0, Y, Z, 0, Z, X], True),   # the head reversed
        ([1, 1, X, Y, 3, 0, Z, X, 0, X, Y, 0, Y, Z], False),  # the head drops Z: no left-deep plan
        ([1, 1, Y, Z, 3, 0, X, Y, 0, Z, X, 0, Y, Z], True),   # the head drops X
    ]
    for k, (plan, left_deep) in enumerate(plans):
        _note(f"triangle orientation {k} wcoj={wcoj}")
        want = _brute_triangle(plan, n, s, d)
        if wcoj == "0" and not left_deep:
            with pytest.raises(XlogError) as ex:
                _run(provider, plan, [e, None], ROUTE_JOIN)
            assert ex.value.status == UNSUPPORTED
            del ex
            continue
        outs, st = _run(provider, plan, [e, None], ROUTE_AUTO)
        assert st["route"] == ROUTE_JOIN
        assert np.array_equal(provider.download_packed(outs[1]), want), k
        assert st["iterations"] == 1 and st["delta_sizes"] == [len(want), 0]
    ss, sd = datagen.sparse_ids(s), datagen.sparse_ids(d)
    _parity(provider, "sparse triangles", cp.triangles_plan(), [pack(ss, sd), None], [1])
