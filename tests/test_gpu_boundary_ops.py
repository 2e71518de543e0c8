"""GPU parity of the provider methods that complete the drop-in surface:
dedup_sorted, the reusable join index (build_join_index_v2 /
hash_join_v2_with_index), the nested-loop join and the factorized TC delta
step (fj_delta_novel_u32_recorded).  Every call goes through libxlog_hip.so;
expected values come from the CPU oracle, from brute force on small inputs
and from the committed C1 closure fixture."""
import json
import sys
from collections import Counter
from pathlib import Path

import numpy as np
import pytest

import oracle
from xlog_amd import FJ_DELTA_CANONICAL, JOIN_ANTI, JOIN_INNER, JOIN_SEMI, XlogError, datagen, pack

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).parent / "golden"


def _note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _cols(rows, arity):
    return [[r[c] for r in rows] for c in range(arity)]


def _brute_join(l_rows, r_rows, lk, rk):
    """All (left ++ right) rows with equal keys, left-row major then right order."""
    return [tuple(a) + tuple(b) for a in l_rows for b in r_rows if a[lk] == b[rk]]


# ---- dedup_sorted (relational.rs:288-420) ------------------------------------
def test_dedup_sorted_adjacent_runs(provider):
    p = provider
    # key column 0 sorted: first row of each key run, input order, no sort
    rows = [(1, 9), (1, 3), (2, 7), (2, 7), (2, 1), (5, 0), (7, 4), (7, 2)]
    d = p.dedup_sorted(p.create_buffer_from_u32_columns(_cols(rows, 2)), [0])
    assert p.download_rows(d) == [(1, 9), (2, 7), (5, 0), (7, 4)]
    # unsorted input: adjacent runs only, exactly like the reference's mark-and-compact
    rows = [(3, 1), (3, 2), (1, 5), (3, 7), (3, 7)]
    d = p.dedup_sorted(p.create_buffer_from_u32_columns(_cols(rows, 2)), [0])
    assert p.download_rows(d) == [(3, 1), (1, 5), (3, 7)]
    # key column 1 on an input sorted by column 1
    rows = [(9, 1), (4, 1), (8, 2), (0, 3), (5, 3)]
    d = p.dedup_sorted(p.create_buffer_from_u32_columns(_cols(rows, 2)), [1])
    assert p.download_rows(d) == [(9, 1), (8, 2), (0, 3)]
    # arity 1, full key: adjacent unique of a sorted column
    d = p.dedup_sorted(p.create_buffer_from_u32_columns([[1, 1, 2, 3, 3, 3, 9]]), [0])
    assert p.download_column(d, 0).tolist() == [1, 2, 3, 9]
    # full-row key on arity 2: the full-row dedup (sorted, unique)
    rows = [(2, 1), (1, 1), (2, 1), (0, 5)]
    d = p.dedup_sorted(p.create_buffer_from_u32_columns(_cols(rows, 2)), [0, 1])
    assert p.download_rows(d) == [(0, 5), (1, 1), (2, 1)] and d.is_canonical()
    assert p.dedup_sorted(p.create_empty_buffer(2), [0]).num_rows() == 0
    one = p.create_buffer_from_u32_columns([[4], [2]])
    assert p.download_rows(p.dedup_sorted(one, [1])) == [(4, 2)]
    with pytest.raises(XlogError):
        p.dedup_sorted(one, [])
    with pytest.raises(XlogError):
        p.dedup_sorted(one, [2])


@pytest.mark.parametrize("n", [2, 4097, 300_000])
def test_dedup_sorted_random_vs_numpy(provider, n):
    p = provider
    rng = np.random.default_rng(n)
    a = np.sort(rng.integers(0, max(2, n // 7), n, dtype=np.uint32))
    b = rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32)
    d = p.dedup_sorted(p.create_buffer_from_u32_columns([a, b]), [0])
    first = np.ones(n, bool)
    first[1:] = a[1:] != a[:-1]
    assert np.array_equal(p.download_column(d, 0), a[first])
    assert np.array_equal(p.download_column(d, 1), b[first])


# ---- reusable join index (relational.rs:3728-4000) ---------------------------
def test_join_index_reuse_matches_hash_join(provider):
    p = provider
    rng = np.random.default_rng(7)
    r = p.create_buffer_from_u32_columns([rng.integers(0, 500, 20_000, dtype=np.uint32),
                                          rng.integers(0, 1 << 31, 20_000, dtype=np.uint32)])
    for rk in (0, 1):
        ix = p.build_join_index_v2(r, [rk])
        for seed in range(3):
            g = np.random.default_rng(100 + seed)
            lkeys = g.integers(0, 600, 5_000, dtype=np.uint32) if rk == 0 else \
                p.download_column(r, 1)[g.integers(0, 20_000, 5_000)]
            left = p.create_buffer_from_u32_columns([lkeys, g.integers(0, 1 << 31, 5_000, dtype=np.uint32)])
            for jt in (JOIN_INNER, JOIN_SEMI, JOIN_ANTI):
                a = p.hash_join_v2_with_index(left, r, [0], [rk], jt, ix)
                b = p.hash_join_v2(left, r, [0], [rk], jt)
                assert a.arity == b.arity
                assert Counter(p.download_rows(a)) == Counter(p.download_rows(b)), (rk, seed, jt)
        ix.free()


def test_join_index_max_output_and_errors(provider):
    p = provider
    left = p.create_buffer_from_u32_columns([[1, 2, 2, 3], [10, 20, 21, 30]])
    right = p.create_buffer_from_u32_columns([[2, 2, 3, 9], [200, 201, 300, 900]])
    ix = p.build_join_index_v2(right, [0])
    full = p.hash_join_v2_with_index(left, right, [0], [0], JOIN_INNER, ix)
    rows = p.download_rows(full)
    assert Counter(rows) == Counter(_brute_join(list(zip([1, 2, 2, 3], [10, 20, 21, 30])),
                                                list(zip([2, 2, 3, 9], [200, 201, 300, 900])), 0, 0))
    for cap in (1, 3, 5, 100):
        t = p.hash_join_v2_with_index(left, right, [0], [0], JOIN_INNER, ix, max_output=cap)
        assert p.download_rows(t) == rows[:min(cap, len(rows))]
    with pytest.raises(XlogError):  # index built over another key column
        p.hash_join_v2_with_index(left, right, [0], [1], JOIN_INNER, ix)
    with pytest.raises(XlogError):  # the reference refuses an index over an empty relation
        p.build_join_index_v2(p.create_empty_buffer(2), [0])
    empty_left = p.create_empty_buffer(2)
    assert p.hash_join_v2_with_index(empty_left, right, [0], [0], JOIN_INNER, ix).num_rows() == 0


# ---- nested-loop join (relational.rs:3041-3255) ------------------------------
@pytest.mark.parametrize("la,ra", [(1, 1), (1, 2), (2, 1), (2, 2)])
def test_nested_loop_join_brute_force(provider, la, ra):
    p = provider
    rng = np.random.default_rng(la * 10 + ra)
    nl, nr = 700, 900
    l_cols = [rng.integers(0, 40, nl, dtype=np.uint32) for _ in range(la)]
    r_cols = [rng.integers(0, 40, nr, dtype=np.uint32) for _ in range(ra)]
    lk, rk = la - 1, 0
    out = p.nested_loop_join_v2_inner_u32_1key(p.create_buffer_from_u32_columns(l_cols),
                                               p.create_buffer_from_u32_columns(r_cols), lk, rk)
    assert out.arity == la + ra
    l_rows = list(zip(*[c.tolist() for c in l_cols]))
    r_rows = list(zip(*[c.tolist() for c in r_cols]))
    # deterministic order: left-row major, then right-row order
    assert p.download_rows(out) == _brute_join(l_rows, r_rows, lk, rk)


def test_nested_loop_join_caps_and_edges(provider):
    p = provider
    a = p.create_buffer_from_u32_columns([[1, 2, 3], [4, 5, 6]])
    assert p.nested_loop_join_v2_inner_u32_1key(a, p.create_empty_buffer(1), 0, 0).arity == 3
    assert p.nested_loop_join_v2_inner_u32_1key(p.create_empty_buffer(2), a, 0, 0).num_rows() == 0
    no_match = p.create_buffer_from_u32_columns([[7, 8]])
    assert p.nested_loop_join_v2_inner_u32_1key(a, no_match, 0, 0).num_rows() == 0
    # rows_l * rows_r = 2001 * 2000 > 4,000,000: refused like the reference
    big_l = p.create_buffer_from_u32_columns([np.zeros(2001, np.uint32)])
    big_r = p.create_buffer_from_u32_columns([np.zeros(2000, np.uint32)])
    with pytest.raises(XlogError) as e:
        p.nested_loop_join_v2_inner_u32_1key(big_l, big_r, 0, 0)
    assert e.value.status == 3  # CAPACITY_OVERFLOW
    # exactly at the threshold: 2000 * 2000 all-equal keys = 4,000,000 rows
    eq = p.nested_loop_join_v2_inner_u32_1key(big_r, big_r, 0, 0)
    assert eq.num_rows() == 4_000_000
    with pytest.raises(XlogError):
        p.nested_loop_join_v2_inner_u32_1key(a, a, 2, 0)


# ---- factorized delta step (fj_delta.rs:117-490) -----------------------------
def _fj_expected(delta, edge, full):
    """{(x, z) : (x, y) in delta, (y, z) in edge} minus full, as sorted unique packed keys."""
    j = oracle.join_project(delta, edge, 1, 0, 0, 3)
    return oracle.diff_sorted(oracle.sort_dedup(j), oracle.sort_dedup(full))


def test_fj_delta_step_vs_oracle(provider):
    p = provider
    rng = np.random.default_rng(11)
    dom = 3000
    edge = oracle.sort_dedup(pack(rng.integers(0, dom, 20_000, dtype=np.uint32),
                                  rng.integers(0, dom, 20_000, dtype=np.uint32)))
    delta = pack(rng.integers(0, dom, 8_000, dtype=np.uint32), rng.integers(0, dom, 8_000, dtype=np.uint32))
    full = pack(rng.integers(0, dom, 200_000, dtype=np.uint32), rng.integers(0, dom, 200_000, dtype=np.uint32))
    E = p.create_buffer_from_packed(edge)
    D = p.create_buffer_from_packed(delta)
    F = p.create_buffer_from_packed(full)
    out = p.fj_delta_novel_u32_recorded(D, E, F, FJ_DELTA_CANONICAL, dom)
    exp = _fj_expected(delta, edge, full)
    assert out.is_canonical()
    assert np.array_equal(p.download_packed(out), exp)
    # column roles: delta stored (y, x), full and head stored (z, x)
    swap = lambda k: (k << np.uint64(32)) | (k >> np.uint64(32))  # noqa: E731
    out2 = p.fj_delta_novel_u32_recorded(p.create_buffer_from_packed(swap(delta)), E,
                                         p.create_buffer_from_packed(swap(full)), (1, 0, 1, 0), dom)
    assert np.array_equal(p.download_packed(out2), np.sort(swap(exp)))
    # an unsorted edge relation with duplicates gives the same set
    shuffled = np.concatenate([edge, edge[:500]])
    rng.shuffle(shuffled)
    out3 = p.fj_delta_novel_u32_recorded(D, p.create_buffer_from_packed(shuffled), F, FJ_DELTA_CANONICAL, dom)
    assert np.array_equal(p.download_packed(out3), exp)


def test_fj_delta_iterated_is_the_c1_closure(provider):
    """Seminaive TC driven step by step through the operator reproduces the
    committed C1 closure, its iteration count and its per-iteration delta sizes."""
    p = provider
    fx = json.loads((GOLDEN / "fixtures.json").read_text())["c1"]
    src, dst = datagen.random_digraph(fx["vertices"], fx["edges"], datagen.seed_for(1))
    edge = oracle.sort_dedup(pack(src, dst))
    E = p.create_buffer_from_packed(edge)
    R = p.create_buffer_from_packed(edge)
    D = p.create_buffer_from_packed(edge)
    deltas, it = [len(edge)], 0
    while True:
        it += 1
        N = p.fj_delta_novel_u32_recorded(D, E, R, FJ_DELTA_CANONICAL, fx["vertices"])
        deltas.append(N.num_rows())
        if N.num_rows() == 0:
            break
        R = p.union_gpu(R, N)
        D = N
    bits = np.unpackbits(np.load(GOLDEN / "c1_closure.npz")["bits"], axis=1)[:, :fx["vertices"]]
    xs, zs = np.nonzero(bits)
    assert np.array_equal(p.download_packed(R), np.sort(pack(xs.astype(np.uint32), zs.astype(np.uint32))))
    assert (it, deltas) == (fx["iterations"], fx["delta_sizes"])


def test_fj_delta_errors_and_empty(provider):
    p = provider
    E = p.create_buffer_from_u32_columns([[0, 1], [1, 2]])
    D = p.create_buffer_from_u32_columns([[0], [0]])
    F = p.create_empty_buffer(2)
    assert p.download_rows(p.fj_delta_novel_u32_recorded(D, E, F, FJ_DELTA_CANONICAL, 3)) == [(0, 1)]
    assert p.fj_delta_novel_u32_recorded(p.create_empty_buffer(2), E, F, FJ_DELTA_CANONICAL, 3).num_rows() == 0
    for bad_domain in (0, 2, (1 << 16) + 1):  # 2: id 2 lies outside the domain
        with pytest.raises(XlogError):
            p.fj_delta_novel_u32_recorded(D, E, F, FJ_DELTA_CANONICAL, bad_domain)
    with pytest.raises(XlogError):
        p.fj_delta_novel_u32_recorded(D, E, F, (0, 0, 0, 1), 3)
    with pytest.raises(XlogError):
        p.fj_delta_novel_u32_recorded(p.create_buffer_from_u32_columns([[0]]), E, F, FJ_DELTA_CANONICAL, 3)
