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


def _brute_keys(l_rows, r_rows, lk, rk, kind=JOIN_INNER):
    """Join on key lists: INNER rows left ++ right in left-row-major, right-row order;
    SEMI / ANTI the left rows with / without a match, input order."""
    match = lambda a, b: all(a[x] == b[y] for x, y in zip(lk, rk))
    if kind == JOIN_INNER:
        return [tuple(a) + tuple(b) for a in l_rows for b in r_rows if match(a, b)]
    want = kind == JOIN_SEMI
    return [tuple(a) for a in l_rows if any(match(a, b) for b in r_rows) == want]


def _rel(p, rows, arity):
    return p.create_buffer_from_u32_columns([[r[c] for r in rows] for c in range(arity)])


def test_join_index_reference_key_list_shapes(provider):
    """The reference builds indexes over five key columns and over two
    (crates/xlog-cuda/tests/pack_keys_gpu.rs:12-38, 53-65); here the index is
    also probed and checked against brute force."""
    p = provider
    five = [(1, 4, 7, 10, 13), (2, 5, 8, 11, 14), (3, 6, 9, 12, 15)]
    r5 = _rel(p, five, 5)
    ix5 = p.build_join_index_v2(r5, [0, 1, 2, 3, 4])
    probe = [(2, 5, 8, 11, 14), (3, 6, 9, 12, 0), (1, 4, 7, 10, 13), (2, 5, 8, 11, 14), (1, 4, 7, 10, 14)]
    l5 = _rel(p, probe, 5)
    keys = [0, 1, 2, 3, 4]
    for kind in (JOIN_SEMI, JOIN_ANTI):
        got = p.download_rows(p.hash_join_v2_with_index(l5, r5, keys, keys, kind, ix5))
        assert got == _brute_keys(probe, five, keys, keys, kind), kind
    # five key columns with the left's columns permuted, INNER (output arity 3 + 5)
    l3 = [(10, 7, 4), (11, 8, 5), (10, 7, 5), (12, 9, 6)]
    ix_perm = p.build_join_index_v2(r5, [3, 2, 1])
    got = p.download_rows(p.hash_join_v2_with_index(_rel(p, l3, 3), r5, [0, 1, 2], [3, 2, 1], JOIN_INNER, ix_perm))
    assert got == _brute_keys(l3, five, [0, 1, 2], [3, 2, 1]) == [(10, 7, 4) + five[0], (11, 8, 5) + five[1],
                                                               (12, 9, 6) + five[2]]
    two = [(1, 10), (2, 20), (3, 30), (4, 40)]
    r2 = _rel(p, two, 2)
    ix2 = p.build_join_index_v2(r2, [0, 1])
    left = [(1, 10, 7), (1, 20, 8), (4, 40, 9), (3, 30, 1), (4, 40, 2)]
    got = p.download_rows(p.hash_join_v2_with_index(_rel(p, left, 3), r2, [0, 1], [0, 1], JOIN_INNER, ix2))
    assert got == _brute_keys(left, two, [0, 1], [0, 1])
    # the index remembers its key list: another list or another relation is refused
    with pytest.raises(XlogError) as ex:
        p.hash_join_v2_with_index(_rel(p, left, 3), r2, [1, 0], [1, 0], JOIN_INNER, ix2)
    assert ex.value.status == 1
    with pytest.raises(XlogError) as ex:
        p.hash_join_v2_with_index(_rel(p, left, 3), r5, [0, 1], [0, 1], JOIN_INNER, ix2)
    assert ex.value.status == 1


@pytest.mark.parametrize("seed", range(5))
@pytest.mark.parametrize("la,ra,nk", [(3, 3, 2), (2, 2, 2), (4, 3, 3), (2, 4, 2), (4, 4, 4), (1, 5, 1), (3, 2, 1)])
def test_join_index_key_lists_reused_vs_brute_force(provider, seed, la, ra, nk):
    """One index over a key list, probed by three left relations with every
    join type, against brute force (exact row order) and against the
    one-shot keyed join; max_output keeps a prefix of that order."""
    p = provider
    rng = np.random.default_rng(1000 * seed + 100 * la + 10 * ra + nk)
    rk = [int(x) for x in rng.permutation(ra)[:nk]]
    vals = int(rng.integers(2, 7))
    nr = int(rng.integers(1, 250))
    r_rows = [tuple(int(v) for v in rng.integers(0, vals, ra)) for _ in range(nr)]
    if seed == 0:  # all-ones key values
        r_rows = [tuple(0xFFFFFFFF if v == 0 else v for v in row) for row in r_rows]
    right = _rel(p, r_rows, ra)
    ix = p.build_join_index_v2(right, rk)
    for probe in range(3):
        lk = [int(x) for x in rng.permutation(la)[:nk]]
        nl = int(rng.integers(0, 250))
        l_rows = [tuple(int(v) for v in rng.integers(0, vals, la)) for _ in range(nl)]
        if seed == 0:
            l_rows = [tuple(0xFFFFFFFF if v == 0 else v for v in row) for row in l_rows]
        _note(f"join index key list la={la} ra={ra} lk={lk} rk={rk} nl={nl} nr={nr} probe={probe}")
        left = _rel(p, l_rows, la)
        for kind in (JOIN_INNER, JOIN_SEMI, JOIN_ANTI):
            if kind == JOIN_INNER and la + ra > 8:
                continue
            exp = _brute_keys(l_rows, r_rows, lk, rk, kind)
            got = p.hash_join_v2_with_index(left, right, lk, rk, kind, ix)
            assert got.arity == (la + ra if kind == JOIN_INNER else la)
            assert p.download_rows(got) == exp, (kind, probe)
            assert p.download_rows(p.hash_join_v2(left, right, lk, rk, kind)) == exp, (kind, probe)
            if kind == JOIN_INNER and exp:
                cap = int(rng.integers(1, len(exp) + 1))
                t = p.hash_join_v2_with_index(left, right, lk, rk, kind, ix, max_output=cap)
                assert p.download_rows(t) == exp[:cap]
    ix.free()


def test_join_index_larger_random_key_lists(provider):
    """Two and three key columns over 200,000-row relations, index reused, against numpy."""
    p = provider
    rng = np.random.default_rng(42)
    n = 200_000
    r_cols = [rng.integers(0, 60, n, dtype=np.uint32), rng.integers(0, 2000, n, dtype=np.uint32),
              rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32)]
    right = p.create_buffer_from_u32_columns(r_cols)
    for rk in ([0, 1], [1, 0, 2]):
        ix = p.build_join_index_v2(right, rk)
        for probe in range(2):
            m = 50_000
            pick = rng.integers(0, n, m)
            l_cols = [r_cols[rk[t]][pick].copy() for t in range(len(rk))]
            l_cols[0][: m // 3] = rng.integers(0, 70, m // 3, dtype=np.uint32)  # some keys absent
            left = p.create_buffer_from_u32_columns(l_cols)
            lk = list(range(len(rk)))
            semi = p.download_rows(p.hash_join_v2_with_index(left, right, lk, rk, JOIN_SEMI, ix))
            rkeys = set(zip(*[r_cols[c].tolist() for c in rk]))
            lrows = list(zip(*[c.tolist() for c in l_cols]))
            assert semi == [r for r in lrows if r in rkeys]
            anti = p.download_rows(p.hash_join_v2_with_index(left, right, lk, rk, JOIN_ANTI, ix))
            assert anti == [r for r in lrows if r not in rkeys]
            inner = p.hash_join_v2_with_index(left, right, lk, rk, JOIN_INNER, ix)
            cnt = Counter(zip(*[r_cols[c].tolist() for c in rk]))
            assert inner.num_rows() == sum(cnt[r] for r in lrows)
            assert Counter(p.download_rows(inner)) == Counter(p.download_rows(
                p.hash_join_v2(left, right, lk, rk, JOIN_INNER)))
        ix.free()


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
