"""GPU parity of the merge-path sort-merge join (xlog_hip_sort_merge_join,
reference sort_merge_join_v2_inner_u32_1key, relational.rs:3401-3571).

The reference's own tests (crates/xlog-integration/tests/test_sort_merge_dispatch.rs:231-500)
compare the operator's row set with hash_join_v2 on sorted unique keys, on 250 keys x 4
duplicates per side (4000 rows) and on empty inputs; those fixtures are restated here.
Beyond them: the exact row order (left rows in key order, right rows of a run in input
order) against brute force, unsorted inputs (sorted by the operator), merge paths spanning
many 2048-item tiles, and a skewed hot key against the hash join and the closed-form count
sum_k cnt_L(k) * cnt_R(k)."""
import sys
from collections import Counter

import numpy as np
import pytest

from xlog_amd import JOIN_INNER

pytestmark = pytest.mark.gpu


def _note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _stable_by(rows, k):
    return sorted(rows, key=lambda r: r[k])  # Python's sort is stable


def _expected(l_rows, r_rows, lk, rk):
    """Left rows in key order (stable), each followed by its right matches in key-stable order."""
    ls, rs = _stable_by(l_rows, lk), _stable_by(r_rows, rk)
    by_key = {}
    for b in rs:
        by_key.setdefault(b[rk], []).append(b)
    return [tuple(a) + tuple(b) for a in ls for b in by_key.get(a[lk], [])]


def _rel(p, rows, arity):
    return p.create_buffer_from_u32_columns([np.array([r[c] for r in rows], dtype=np.uint32)
                                             for c in range(arity)])


# ---- the reference's fixtures (test_sort_merge_dispatch.rs) -------------------
def test_smj_sorted_unique_keys(provider):
    p = provider
    left = _rel(p, [(i, 1000 + i) for i in range(100)], 2)
    right = _rel(p, [(i, 2000 + i) for i in range(100)], 2)
    sm = p.sort_merge_join_v2_inner_u32_1key(left, right, 0, 0)
    hj = p.hash_join_v2(left, right, [0], [0], JOIN_INNER)
    assert sm.arity == 4 and sm.num_rows() == 100
    assert set(p.download_rows(sm)) == set(p.download_rows(hj))
    assert p.download_rows(sm) == [(i, 1000 + i, i, 2000 + i) for i in range(100)]


def test_smj_duplicate_keys(provider):
    p = provider
    l_rows = [(i // 4, 1000 + i) for i in range(1000)]
    r_rows = [(i // 4, 2000 + i) for i in range(1000)]
    left, right = _rel(p, l_rows, 2), _rel(p, r_rows, 2)
    got = p.download_rows(p.sort_merge_join_v2_inner_u32_1key(left, right, 0, 0))
    assert len(got) == 4000 and len(set(got)) == 4000
    assert set(got) == set(p.download_rows(p.hash_join_v2(left, right, [0], [0], JOIN_INNER)))
    assert got == _expected(l_rows, r_rows, 0, 0)


@pytest.mark.parametrize("empty_side", ["left", "right", "both"])
def test_smj_empty_inputs(provider, empty_side):
    p = provider
    full = _rel(p, [(1, 2), (3, 4)], 2)
    empty = p.create_empty_buffer(2)
    left = empty if empty_side in ("left", "both") else full
    right = empty if empty_side in ("right", "both") else full
    out = p.sort_merge_join_v2_inner_u32_1key(left, right, 0, 0)
    assert out.num_rows() == 0 and out.arity == 4


# ---- exact order against brute force -----------------------------------------
@pytest.mark.parametrize("la,ra,lk,rk", [(1, 1, 0, 0), (1, 2, 0, 1), (2, 1, 1, 0), (2, 2, 0, 0), (2, 2, 1, 0),
                                         (2, 2, 0, 1), (2, 2, 1, 1)])
@pytest.mark.parametrize("presorted", [True, False])
def test_smj_brute_force(provider, la, ra, lk, rk, presorted):
    p = provider
    rng = np.random.default_rng(100 * la + 10 * ra + 3 * lk + rk + (7 if presorted else 0))
    nl, nr = 900, 700
    l_rows = [tuple(int(x) for x in rng.integers(0, 60, la)) for _ in range(nl)]
    r_rows = [tuple(int(x) for x in rng.integers(0, 60, ra)) for _ in range(nr)]
    if presorted:
        l_rows, r_rows = _stable_by(l_rows, lk), _stable_by(r_rows, rk)
    _note(f"smj brute force la={la} ra={ra} lk={lk} rk={rk} presorted={presorted}")
    out = p.sort_merge_join_v2_inner_u32_1key(_rel(p, l_rows, la), _rel(p, r_rows, ra), lk, rk)
    assert out.arity == la + ra
    assert p.download_rows(out) == _expected(l_rows, r_rows, lk, rk)


@pytest.mark.parametrize("case", ["disjoint", "left_below", "interleaved", "one_key"])
def test_smj_merge_path_shapes(provider, case):
    """Merge paths over many 2048-item tiles with every mix of left rows and runs per tile."""
    p = provider
    rng = np.random.default_rng(len(case))
    if case == "disjoint":      # even keys left, odd keys right: no match at all
        lk_ = 2 * rng.integers(0, 50000, 60000)
        rk_ = 2 * rng.integers(0, 50000, 40000) + 1
    elif case == "left_below":  # every left key below every right key, then one shared key at the boundary
        lk_ = np.concatenate([rng.integers(0, 1000, 30000), [5000] * 3])
        rk_ = np.concatenate([[5000] * 2, rng.integers(5001, 9000, 30000)])
    elif case == "interleaved":
        lk_ = rng.integers(0, 20000, 50000)
        rk_ = rng.integers(0, 20000, 30000)
    else:                       # a single key on both sides
        lk_ = np.full(3000, 7)
        rk_ = np.full(1500, 7)
    l_rows = list(zip(lk_.tolist(), range(len(lk_))))
    r_rows = list(zip(rk_.tolist(), range(len(rk_))))
    _note(f"smj merge path case={case} nl={len(l_rows)} nr={len(r_rows)}")
    out = p.sort_merge_join_v2_inner_u32_1key(_rel(p, l_rows, 2), _rel(p, r_rows, 2), 0, 0)
    cl, cr = Counter(lk_.tolist()), Counter(rk_.tolist())
    assert out.num_rows() == sum(c * cr.get(k, 0) for k, c in cl.items())
    if out.num_rows() <= 5_000_000:
        assert p.download_rows(out) == _expected(l_rows, r_rows, 0, 0)


def _mix(w0, w1):
    """64-bit row hash of two packed words (splitmix64 finaliser over w0 ^ rotated w1)."""
    with np.errstate(over="ignore"):
        x = w0 ^ ((w1 << np.uint64(29)) | (w1 >> np.uint64(35))) ^ (w1 * np.uint64(0x9E3779B97F4A7C15))
        x = (x ^ (x >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        x = (x ^ (x >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return x ^ (x >> np.uint64(31))


def _host_join_words(lk_, lpay, rpay, rk_):
    """Packed words of left(lk, lpay) join right(rpay, rk) on lk = rk, output
    (lk, lpay, rpay, rk), built with numpy from the sorted right keys."""
    order = np.argsort(rk_, kind="stable")
    rks, rps = rk_[order], rpay[order]
    lo = np.searchsorted(rks, lk_, side="left")
    hi = np.searchsorted(rks, lk_, side="right")
    cnt = (hi - lo).astype(np.int64)
    li = np.repeat(np.arange(len(lk_)), cnt)
    starts = np.repeat(lo - np.concatenate([[0], np.cumsum(cnt)[:-1]]), cnt)
    ri = np.arange(len(li)) + starts
    w0 = (lk_[li].astype(np.uint64) << np.uint64(32)) | lpay[li].astype(np.uint64)
    w1 = (rps[ri].astype(np.uint64) << np.uint64(32)) | rks[ri].astype(np.uint64)
    return w0, w1


def test_smj_skewed_hot_key(provider):
    """A hot key with 3000 left x 2000 right rows among uniform keys: same multiset as the hash join
    (about 6.5e6 rows, 6e6 of them from the hot key)."""
    p = provider
    rng = np.random.default_rng(11)
    nl, nr = 200000, 120000
    lk_ = rng.integers(0, 50000, nl).astype(np.uint32)
    rk_ = rng.integers(0, 50000, nr).astype(np.uint32)
    lk_[:3000] = 424242
    rk_[:2000] = 424242
    lpay = rng.integers(0, 1 << 32, nl, dtype=np.uint64).astype(np.uint32)
    rpay = rng.integers(0, 1 << 32, nr, dtype=np.uint64).astype(np.uint32)
    left = p.create_buffer_from_u32_columns([lk_, lpay])
    right = p.create_buffer_from_u32_columns([rpay, rk_])  # right key in column 1
    cl, cr = Counter(lk_.tolist()), Counter(rk_.tolist())
    expect_n = sum(c * cr.get(k, 0) for k, c in cl.items())
    _note(f"smj skewed: expecting {expect_n} rows")
    sm = p.sort_merge_join_v2_inner_u32_1key(left, right, 0, 1)
    hj = p.hash_join_v2(left, right, [0], [1], JOIN_INNER)
    assert sm.num_rows() == expect_n == hj.num_rows()
    # as multisets against a host join: rows are hashed from their packed words
    # ((c0 << 32) | c1, (c2 << 32) | c3) and the sorted hash arrays compared
    exp_rows = _host_join_words(lk_, lpay, rpay, rk_)

    def row_hashes(rel):
        c = [p.download_column(rel, i).astype(np.uint64) for i in range(4)]
        return _mix((c[0] << np.uint64(32)) | c[1], (c[2] << np.uint64(32)) | c[3])
    want = np.sort(_mix(*exp_rows))
    assert np.array_equal(np.sort(row_hashes(sm)), want)
    assert np.array_equal(np.sort(row_hashes(hj)), want)
    # left rows come out in key order
    k0 = p.download_column(sm, 0)
    assert np.all(k0[1:] >= k0[:-1])
