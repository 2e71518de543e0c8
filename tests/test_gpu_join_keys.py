"""GPU parity of equi-joins on key column lists and of joins over inputs wider
than two columns (provider hash_join_v2 with key lists, the C ABI's
xlog_hip_hash_join_keys; reference hash_join_v2, relational.rs:2926-2992).

Expected rows come from a nested-loop brute force on small inputs (rows in
left-row-major, then right-row order, which is the order the library
documents), from a numpy sort-based join on larger inputs, and from the
reference's own known answer for a two-column key
(crates/xlog-cuda/tests/join_v2_tests.rs:303-353)."""
import sys

import numpy as np
import pytest

from xlog_amd import JOIN_ANTI, JOIN_INNER, JOIN_SEMI, XlogError

pytestmark = pytest.mark.gpu
INVALID_ARG, CAPACITY_OVERFLOW, UNSUPPORTED = 1, 3, 7


def _note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _rel(p, rows, arity):
    return p.create_buffer_from_u32_columns([[r[c] for r in rows] for c in range(arity)])


def _brute(l_rows, r_rows, lk, rk, kind=JOIN_INNER):
    if kind == JOIN_INNER:
        return [tuple(a) + tuple(b) for a in l_rows for b in r_rows
                if all(a[x] == b[y] for x, y in zip(lk, rk))]
    hit = [any(all(a[x] == b[y] for x, y in zip(lk, rk)) for b in r_rows) for a in l_rows]
    want = kind == JOIN_SEMI
    return [tuple(a) for a, h in zip(l_rows, hit) if h == want]


def test_reference_multi_column_join(provider):
    # join_v2_tests.rs:303-353: left (a, b, payload), right (x, y, value), on (a, b) = (x, y)
    p = provider
    left = p.create_buffer_from_u32_columns([[1, 1, 2], [10, 20, 10], [100, 200, 300]])
    right = p.create_buffer_from_u32_columns([[1, 2, 1], [10, 10, 20], [1000, 2000, 3000]])
    out = p.hash_join_v2(left, right, [0, 1], [0, 1], JOIN_INNER)
    assert out.num_rows() == 3 and out.arity == 6
    assert p.download_rows(out) == [(1, 10, 100, 1, 10, 1000), (1, 20, 200, 1, 20, 3000),
                                    (2, 10, 300, 2, 10, 2000)]


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("la,ra", [(1, 3), (3, 1), (2, 3), (3, 3), (4, 4), (4, 2)])
def test_keyed_join_vs_brute_force(provider, seed, la, ra):
    p = provider
    rng = np.random.default_rng(100 * seed + 10 * la + ra)
    nk = int(rng.integers(1, min(la, ra) + 1))
    lk = [int(x) for x in rng.permutation(la)[:nk]]
    rk = [int(x) for x in rng.permutation(ra)[:nk]]
    nl, nr = int(rng.integers(0, 300)), int(rng.integers(0, 300))
    vals = int(rng.integers(2, 6))
    l_rows = [tuple(int(v) for v in rng.integers(0, vals, la)) for _ in range(nl)]
    r_rows = [tuple(int(v) for v in rng.integers(0, vals, ra)) for _ in range(nr)]
    _note(f"keyed join la={la} ra={ra} keys {lk}/{rk} nl={nl} nr={nr}")
    left, right = _rel(p, l_rows, la), _rel(p, r_rows, ra)
    for kind in (JOIN_INNER, JOIN_SEMI, JOIN_ANTI):
        out = p.hash_join_v2(left, right, lk, rk, kind)
        exp = _brute(l_rows, r_rows, lk, rk, kind)
        assert out.arity == (la + ra if kind == JOIN_INNER else la)
        assert out.num_rows() == len(exp), kind
        assert p.download_rows(out) == exp, kind


def test_single_key_wide_inputs_and_all_ones_keys(provider):
    # one key column over arity-3 / arity-4 inputs, and key values 0xFFFFFFFF on both sides
    p = provider
    M = 0xFFFFFFFF
    l_rows = [(M, 1, 2), (5, 3, 4), (M, 9, 9), (7, 0, 0)]
    r_rows = [(0, M, 1, 1), (0, 5, 2, 2), (0, M, 3, 3), (0, 8, 4, 4)]
    left, right = _rel(p, l_rows, 3), _rel(p, r_rows, 4)
    for lk, rk in (([0], [1]), ([0, 1], [1, 0])):
        for kind in (JOIN_INNER, JOIN_SEMI, JOIN_ANTI):
            out = p.hash_join_v2(left, right, lk, rk, kind)
            assert p.download_rows(out) == _brute(l_rows, r_rows, lk, rk, kind), (lk, kind)


def test_keyed_join_output_arity_8_and_projection(provider):
    p = provider
    rng = np.random.default_rng(8)
    l_rows = [tuple(int(v) for v in rng.integers(0, 4, 4)) for _ in range(120)]
    r_rows = [tuple(int(v) for v in rng.integers(0, 4, 4)) for _ in range(90)]
    left, right = _rel(p, l_rows, 4), _rel(p, r_rows, 4)
    out = p.hash_join_v2(left, right, [3, 1], [0, 2], JOIN_INNER)
    exp = _brute(l_rows, r_rows, [3, 1], [0, 2])
    assert out.arity == 8 and p.download_rows(out) == exp
    # every column downloads on its own too
    for c in range(8):
        assert p.download_column(out, c).tolist() == [e[c] for e in exp]
    # join + projection over wide inputs (ChainJoin = Project(Join))
    pj = p.join_project(left, right, 3, 0, [0, 7])
    assert sorted(p.download_rows(pj)) == sorted((e[0], e[7]) for e in _brute(l_rows, r_rows, [3], [0]))
    # set semantics of the same: sort + dedup over an arity-8 relation
    d = p.dedup_full_row(out)
    assert p.download_rows(d) == sorted(set(exp))


def test_keyed_join_errors(provider):
    p = provider
    a = p.create_buffer_from_u32_columns([[1], [2], [3], [4], [5]])
    b = p.create_buffer_from_u32_columns([[1], [2], [3], [4]])
    with pytest.raises(XlogError) as ex:
        p.hash_join_v2(a, b, [0, 1], [0], JOIN_INNER)
    assert ex.value.status == INVALID_ARG
    with pytest.raises(XlogError) as ex:
        p.hash_join_v2(a, b, [5], [0], JOIN_INNER)
    assert ex.value.status == INVALID_ARG
    with pytest.raises(XlogError) as ex:  # 5 + 4 output columns
        p.hash_join_v2(a, b, [0], [0], JOIN_INNER)
    assert ex.value.status == UNSUPPORTED
    # SEMI / ANTI keep the left arity, so they are fine
    assert p.download_rows(p.hash_join_v2(a, b, [0, 1], [0, 1], JOIN_SEMI)) == [(1, 2, 3, 4, 5)]
    e = p.create_empty_buffer(3)
    assert p.hash_join_v2(e, b, [0], [0], JOIN_INNER).num_rows() == 0
    assert p.hash_join_v2(b, e, [0, 1], [0, 1], JOIN_ANTI).num_rows() == 1


def _np_join(lcols, rcols, lk, rk):
    """Rows (as a list of column arrays) of the inner join, built with numpy."""
    def key(cols, ks):
        k = np.zeros(len(cols[0]), np.uint64)
        for c in ks:  # values below 2^16 here, so 16 bits per key column suffice
            k = (k << np.uint64(16)) | cols[c].astype(np.uint64)
        return k
    lkey, rkey = key(lcols, lk), key(rcols, rk)
    order = np.argsort(rkey, kind="stable")
    rs = rkey[order]
    lo = np.searchsorted(rs, lkey, "left")
    cnt = np.searchsorted(rs, lkey, "right") - lo
    li = np.repeat(np.arange(len(lkey)), cnt)
    ri = order[np.arange(len(li)) + np.repeat(lo - np.concatenate([[0], np.cumsum(cnt)[:-1]]), cnt)]
    return [c[li] for c in lcols] + [c[ri] for c in rcols]


def test_keyed_join_large_vs_numpy(provider):
    # several probe tiles, skewed keys: rows in left-row then right-row order
    p = provider
    rng = np.random.default_rng(77)
    nl, nr = 300_000, 200_000
    lcols = [rng.integers(0, 300, nl).astype(np.uint32), rng.integers(0, 1 << 16, nl).astype(np.uint32),
             rng.integers(0, 20, nl).astype(np.uint32)]
    rcols = [rng.integers(0, 20, nr).astype(np.uint32), rng.integers(0, 300, nr).astype(np.uint32),
             rng.integers(0, 1 << 16, nr).astype(np.uint32)]
    lcols[0][:5000] = 7  # a hot key
    rcols[1][:400] = 7
    lk, rk = [0, 2], [1, 0]
    exp = _np_join(lcols, rcols, lk, rk)
    _note(f"keyed join large: expecting {len(exp[0])} rows")
    out = p.hash_join_v2(p.create_buffer_from_u32_columns(lcols), p.create_buffer_from_u32_columns(rcols),
                         lk, rk, JOIN_INNER)
    assert out.num_rows() == len(exp[0])
    for c in range(6):
        assert np.array_equal(p.download_column(out, c), exp[c]), c
