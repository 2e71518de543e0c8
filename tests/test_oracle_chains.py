"""Pins the CPU oracle's semi-naive evaluation (oracle.c or_seminaive, after
crates/xlog-runtime/src/executor/recursive.rs:447-957) on chain-rule programs
other than transitive closure and Andersen: every result is checked against
Kleene iteration of the program written as boolean matrix algebra in numpy.

The semi-naive delta of iteration k is T(R_{k-1}) minus R_{k-1} (T the
immediate-consequence operator, R_{-1} the initial relations), so the matrix
iteration fixes the final relations, every per-iteration delta size and the
iteration count independently of the join-based evaluation."""
import numpy as np
import pytest

import oracle
from xlog_amd import datagen, pack

import chain_plans as cp


def _mat(n, src, dst):
    m = np.zeros((n, n), dtype=bool)
    m[np.asarray(src, np.int64), np.asarray(dst, np.int64)] = True
    return m


def _mm(a, b):
    return (a.astype(np.int32) @ b.astype(np.int32)) > 0


def _rows(m):
    x, z = np.nonzero(m)
    return np.sort(pack(x.astype(np.uint32), z.astype(np.uint32)))


def _kleene(step, init):
    """step(R) -> T(R) for a tuple of IDB matrices; returns (final, iterations, delta sizes)."""
    R = tuple(m.copy() for m in init)
    T = step(R)
    D = tuple(t & ~r for t, r in zip(T, R))
    deltas = [int(sum(d.sum() for d in D))]
    R = tuple(r | d for r, d in zip(R, D))
    it = 0
    while True:
        it += 1
        T = step(R)
        D = tuple(t & ~r for t, r in zip(T, R))
        n = int(sum(d.sum() for d in D))
        deltas.append(n)
        if n == 0:
            return R, it, deltas
        R = tuple(r | d for r, d in zip(R, D))


def _graph(n, m, seed):
    s, d = datagen.random_digraph(n, m, seed)
    return np.asarray(s, np.uint32), np.asarray(d, np.uint32)


def _check(plan, rels, idb, expect):
    outs, it, deltas = oracle.seminaive(plan, rels)
    R, it_m, deltas_m = expect
    for p, m in zip(idb, R):
        assert np.array_equal(outs[p], _rows(m)), f"pred {p}"
    assert it == it_m
    assert deltas == deltas_m


@pytest.mark.parametrize("n,m,seed", [(40, 60, 1), (120, 200, 2)])
def test_left_and_nonlinear_tc(n, m, seed):
    s, d = _graph(n, m, seed)
    E = _mat(n, s, d)
    e = pack(s, d)
    _check(cp.left_tc_plan(), [e, None], [1], _kleene(lambda R: (E | _mm(E, R[0]),), [np.zeros_like(E)]))
    _check(cp.nonlinear_tc_plan(), [e, None], [1], _kleene(lambda R: (E | _mm(R[0], R[0]),), [np.zeros_like(E)]))


@pytest.mark.parametrize("n,seed", [(60, 3), (150, 4)])
def test_same_generation(n, seed):
    rng = np.random.default_rng(seed)
    child = np.arange(1, n, dtype=np.uint32)
    parent = np.array([rng.integers(0, c) for c in child], dtype=np.uint32)
    fs = rng.integers(0, n, n // 5).astype(np.uint32)
    fd = rng.integers(0, n, n // 5).astype(np.uint32)
    F, Up = _mat(n, fs, fd), _mat(n, child, parent)
    Dn = Up.T.copy()
    expect = _kleene(lambda R: (F | _mm(_mm(Up, R[0]), Dn),), [np.zeros_like(F)])
    _check(cp.same_generation_plan(), [pack(fs, fd), pack(child, parent), pack(parent, child), None], [3], expect)
    _check(cp.same_generation_par_plan(), [pack(fs, fd), pack(child, parent), None], [2], expect)


@pytest.mark.parametrize("n,m,seed", [(30, 45, 5), (90, 160, 6)])
def test_parity_mutual_recursion(n, m, seed):
    s, d = _graph(n, m, seed)
    E = _mat(n, s, d)
    step = lambda R: (E | _mm(R[1], E), _mm(R[0], E))  # (odd, even)
    _check(cp.parity_plan(), [pack(s, d), None, None], [1, 2], _kleene(step, [np.zeros_like(E)] * 2))


@pytest.mark.parametrize("n,m,seed", [(30, 45, 5), (90, 160, 6)])
def test_parity_left_linear(n, m, seed):
    s, d = _graph(n, m, seed)
    E = _mat(n, s, d)
    step = lambda R: (E | _mm(E, R[1]), _mm(E, R[0]))  # (odd, even)
    _check(cp.parity_left_plan(), [pack(s, d), None, None], [1, 2], _kleene(step, [np.zeros_like(E)] * 2))


@pytest.mark.parametrize("n,m,seed", [(30, 40, 7), (100, 150, 8)])
def test_symmetric_closure(n, m, seed):
    s, d = _graph(n, m, seed)
    E = _mat(n, s, d)
    step = lambda R: (E.T | R[0].T | _mm(R[0], E),)
    _check(cp.symmetric_plan(), [pack(s, d), None], [1], _kleene(step, [np.zeros_like(E)]))


@pytest.mark.parametrize("n,seed", [(40, 9), (80, 10)])
def test_four_atom_chain(n, seed):
    a_s, a_d = _graph(n, n, seed)
    b_s, b_d = _graph(n, n // 2, seed + 100)
    A, B = _mat(n, a_s, a_d), _mat(n, b_s, b_d)
    step = lambda R: (A | _mm(_mm(_mm(A, R[0]), B), R[0]),)
    _check(cp.quad_plan(), [pack(a_s, a_d), pack(b_s, b_d), None], [2], _kleene(step, [np.zeros_like(A)]))


def test_ordered_chain_and_initial_head():
    n = 70
    a_s, a_d = _graph(n, 90, 11)
    b_s, b_d = _graph(n, 60, 12)
    h_s, h_d = _graph(n, 25, 13)
    A, B, H0 = _mat(n, a_s, a_d), _mat(n, b_s, b_d), _mat(n, h_s, h_d)
    step = lambda R: (A | _mm(_mm(A, R[0]), B),)
    _check(cp.ordered_chain_plan(), [pack(a_s, a_d), pack(b_s, b_d), pack(h_s, h_d)], [2], _kleene(step, [H0]))


def test_scrambled_body_is_outside_left_deep_evaluation():
    """The oracle (like the join route) evaluates bodies left-deep and rejects an atom that shares
    no variable with the running binding."""
    with pytest.raises(RuntimeError) as ex:
        oracle.seminaive(cp.scrambled_chain_plan(), [pack([1], [2]), pack([2], [3]), None])
    assert ex.value.code == -3


# Cyclic bodies: an atom whose two variables are both bound is a join on both keys (a filter of the
# binding), lower.rs build_join_tree / compute_join_keys.
@pytest.mark.parametrize("n,m,seed", [(30, 120, 21), (90, 700, 22)])
def test_triangle_closure(n, m, seed):
    s, d = _graph(n, m, seed)
    E = _mat(n, s, d)
    step = lambda R: (E | (_mm(R[0], E) & E.T),)
    _check(cp.triangle_closure_plan(), [pack(s, d), None], [1], _kleene(step, [np.zeros((n, n), bool)]))


@pytest.mark.parametrize("n,m,seed", [(25, 150, 23), (60, 600, 24)])
def test_triangles(n, m, seed):
    s, d = _graph(n, m, seed)
    E = _mat(n, s, d)
    step = lambda R: (_mm(E, E) & E.T,)
    _check(cp.triangles_plan(), [pack(s, d), None], [1], _kleene(step, [np.zeros((n, n), bool)]))


@pytest.mark.parametrize("n,seed", [(40, 25), (100, 26)])
def test_filtered_tc(n, seed):
    a_s, a_d = _graph(n, 3 * n, seed)
    k_s, k_d = _graph(n, 4 * n, seed + 100)
    b_s, b_d = _graph(n, 2 * n, seed + 200)
    A, K, B = _mat(n, a_s, a_d), _mat(n, k_s, k_d), _mat(n, b_s, b_d)
    step = lambda R: (A | _mm(R[0] & K.T, B),)
    rels = [pack(a_s, a_d), pack(k_s, k_d), pack(b_s, b_d), None]
    _check(cp.filtered_tc_plan(), rels, [3], _kleene(step, [np.zeros((n, n), bool)]))


@pytest.mark.parametrize("n,seed", [(60, 27), (150, 28)])
def test_flat_same_generation(n, seed):
    rng = np.random.default_rng(seed)
    child = np.arange(1, n, dtype=np.uint32)
    parent = np.array([rng.integers(max(0, int(c) - 6), int(c)) for c in child], dtype=np.uint32)
    fs = rng.integers(0, n, 3 * n).astype(np.uint32)
    fd = rng.integers(0, n, 3 * n).astype(np.uint32)
    F, P = _mat(n, fs, fd), _mat(n, child, parent)
    step = lambda R: (F | (_mm(_mm(P, R[0]), P.T) & F),)
    rels = [pack(fs, fd), pack(child, parent), None]
    _check(cp.flat_sg_plan(), rels, [2], _kleene(step, [np.zeros((n, n), bool)]))
