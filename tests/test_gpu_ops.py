"""GPU parity of the relational operators against the CPU oracle and the
reference's own known-answer tests.  Every call goes through libxlog_hip.so."""
import sys

import numpy as np
import pytest

import oracle
from xlog_amd import JOIN_ANTI, JOIN_INNER, JOIN_SEMI, XlogError, pack, unpack

pytestmark = pytest.mark.gpu

# the last three span 129, 513 and 769 sort tiles of 8192 keys: tile chunks of
# 2 and 8 per XCD, and a last group of blocks partly without a tile
SIZES = [0, 1, 2, 63, 64, 65, 255, 256, 4095, 4096, 4097, 8191, 70000, (1 << 20) + 17, (1 << 22) + 3,
         3 * (1 << 21) + 5]


def _note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _rng(seed):
    return np.random.default_rng(seed)


def _rows(p, rel):
    return p.download_rows(rel)


# ---- reference KATs: crates/xlog-cuda/tests/sort_tests.rs:7-154 ------------
def test_sort_kats(provider):
    p = provider
    b = p.create_buffer_from_u32_columns([[5, 2, 8, 1, 9, 3]])
    assert p.download_column(p.sort(b, [0]), 0).tolist() == [1, 2, 3, 5, 8, 9]
    b = p.create_buffer_from_u32_columns([[3, 1, 2], [30, 10, 20]])
    s = p.sort(b, [0])
    assert p.download_column(s, 0).tolist() == [1, 2, 3]
    assert p.download_column(s, 1).tolist() == [10, 20, 30]
    assert p.sort(p.create_empty_buffer(1), [0]).num_rows() == 0
    b = p.create_buffer_from_u32_columns([[1, 2, 3, 4, 5]])
    assert p.download_column(p.sort(b, [0]), 0).tolist() == [1, 2, 3, 4, 5]
    b = p.create_buffer_from_u32_columns([[3, 1, 2, 1, 3, 2]])
    assert p.download_column(p.sort(b, [0]), 0).tolist() == [1, 1, 2, 2, 3, 3]
    b = p.create_buffer_from_u32_columns([[5, 4, 3, 2, 1]])
    assert p.download_column(p.sort(b, [0]), 0).tolist() == [1, 2, 3, 4, 5]


# ---- test_full_row_set_algebra.rs:60-163 --------------------------------------
def test_full_row_set_algebra_kats(provider):
    p = provider

    def rel(rows):
        if not rows:
            return p.create_buffer_from_u32_columns([[], []])
        return p.create_buffer_from_u32_columns([[r[0] for r in rows], [r[1] for r in rows]])

    def s(rel_):
        return sorted(_rows(p, rel_))

    assert s(p.dedup_full_row(rel([(1, 10), (2, 20), (3, 30)]))) == [(1, 10), (2, 20), (3, 30)]
    assert s(p.dedup_full_row(rel([(1, 10), (1, 10), (1, 10)]))) == [(1, 10)]
    assert s(p.dedup_full_row(rel([(1, 10), (1, 10), (1, 20), (2, 20), (2, 20)]))) == [(1, 10), (1, 20), (2, 20)]
    assert s(p.dedup_full_row(rel([(1, 10), (1, 20), (1, 30)]))) == [(1, 10), (1, 20), (1, 30)]
    assert p.dedup_full_row(rel([])).num_rows() == 0
    assert s(p.dedup_full_row(rel([(7, 8)]))) == [(7, 8)]
    assert s(p.diff_full_row(rel([(1, 10), (1, 10), (1, 20)]), rel([(1, 10)]))) == [(1, 20)]
    assert s(p.diff_full_row(rel([(1, 20), (1, 20), (2, 30)]), rel([(1, 10)]))) == [(1, 20), (2, 30)]
    assert p.diff_full_row(rel([(1, 10), (2, 20)]), rel([(2, 20), (1, 10)])).num_rows() == 0
    assert s(p.diff_full_row(rel([(1, 10), (1, 10), (2, 20)]), rel([(3, 30)]))) == [(1, 10), (2, 20)]
    assert s(p.diff_full_row(rel([(1, 10), (1, 20), (2, 10)]), rel([(1, 10)]))) == [(1, 20), (2, 10)]


# ---- join_collision_test.rs:19-130 ----------------------------------------------
def test_join_collision_kats(provider):
    p = provider
    l = p.create_buffer_from_u32_columns([[100], [1]])
    r = p.create_buffer_from_u32_columns([[200], [2]])
    assert p.hash_join_v2(l, r, [0], [0]).num_rows() == 0
    l = p.create_buffer_from_u32_columns([[100, 200], [1, 2]])
    r = p.create_buffer_from_u32_columns([[200, 300], [10, 20]])
    assert _rows(p, p.hash_join_v2(l, r, [0], [0])) == [(200, 2, 200, 10)]
    l = p.create_buffer_from_u32_columns([[100, 200], [1, 2]])
    r = p.create_buffer_from_u32_columns([[300, 400], [5, 6]])
    assert p.hash_join_v2(l, r, [0], [0], JOIN_SEMI).num_rows() == 0
    assert sorted(_rows(p, p.hash_join_v2(l, r, [0], [0], JOIN_ANTI))) == [(100, 1), (200, 2)]


@pytest.mark.parametrize("n", SIZES)
def test_sort_dedup_random(provider, n):
    p = provider
    _note(f"sort_dedup n={n}")
    rng = _rng(n + 11)
    keys = rng.integers(0, 1 << 64, size=n, dtype=np.uint64)
    if n > 4:
        keys[rng.integers(0, n, size=n // 3)] = keys[rng.integers(0, n, size=n // 3)]
    rel = p.create_buffer_from_packed(keys)
    s = p.sort(rel, [0, 1])
    assert np.array_equal(p.download_packed(s), oracle.sort_u64(keys))
    d = p.dedup_full_row(rel)
    assert d.is_canonical()
    assert np.array_equal(p.download_packed(d), oracle.sort_dedup(keys))


@pytest.mark.parametrize("n", [0, 1, 100, 4097, 300000])
def test_sort_narrow_keys_skip_passes(provider, n):
    """TC-shaped keys (both columns < 2^15) exercise the digit-skip logic."""
    p = provider
    _note(f"sort narrow n={n}")
    rng = _rng(n + 5)
    keys = pack(rng.integers(0, 1 << 15, n), rng.integers(0, 1 << 15, n))
    rel = p.create_buffer_from_packed(keys)
    assert np.array_equal(p.download_packed(p.dedup_full_row(rel)), oracle.sort_dedup(keys))


@pytest.mark.parametrize("key_cols", [[0], [1], [1, 0]])
def test_sort_by_key_cols_is_stable(provider, key_cols):
    p = provider
    _note(f"sort key_cols={key_cols}")
    rng = _rng(7)
    n = 50000
    c0 = rng.integers(0, 50, n).astype(np.uint32)
    c1 = rng.integers(0, 50, n).astype(np.uint32)
    rel = p.create_buffer_from_u32_columns([c0, c1])
    out = p.sort(rel, key_cols)
    got = list(zip(p.download_column(out, 0).tolist(), p.download_column(out, 1).tolist()))
    rows = list(zip(c0.tolist(), c1.tolist()))
    exp = sorted(rows, key=lambda r: tuple(r[c] for c in key_cols))  # Python sort is stable
    assert got == exp


def test_sort_arity4_and_dedup(provider):
    p = provider
    rng = _rng(3)
    n = 20000
    cols = [rng.integers(0, 4, n).astype(np.uint32) for _ in range(4)]
    rel = p.create_buffer_from_u32_columns(cols)
    rows = list(zip(*[c.tolist() for c in cols]))
    s = p.sort(rel, [2, 0])
    assert _rows(p, s) == sorted(rows, key=lambda r: (r[2], r[0]))
    d = p.dedup_full_row(rel)
    assert _rows(p, d) == sorted(set(rows))
    d2 = p.dedup(rel, [3])
    got = _rows(p, d2)
    first = {}
    for r in sorted(rows, key=lambda r: r[3]):
        first.setdefault(r[3], r)
    assert got == [first[k] for k in sorted(first)]


# diff windows: (5000, 300000) searches B in HBM (window above 16 keys per row), (50000, 600000) streams
# windows of about 10^5 keys through LDS in several 8192-key chunks, the others stream one chunk
@pytest.mark.parametrize("na,nb", [(0, 0), (0, 10), (10, 0), (1000, 1000), (5000, 300000), (300000, 4099),
                                   (50000, 600000)])
def test_union_diff_random(provider, na, nb):
    p = provider
    _note(f"union/diff na={na} nb={nb}")
    rng = _rng(na * 7 + nb)
    a = rng.integers(0, 1 << 20, na, dtype=np.uint64)
    b = np.concatenate([rng.integers(0, 1 << 20, nb, dtype=np.uint64), a[: na // 2]])
    ra, rb = p.create_buffer_from_packed(a), p.create_buffer_from_packed(b)
    ua, ub = oracle.sort_dedup(a), oracle.sort_dedup(b)
    assert np.array_equal(p.download_packed(p.union_gpu(ra, rb)), oracle.union_sorted(ua, ub))
    assert np.array_equal(p.download_packed(p.diff_gpu(ra, rb)), oracle.diff_sorted(ua, ub))
    # canonical inputs take the merge path
    ca, cb = p.dedup_full_row(ra), p.dedup_full_row(rb)
    assert np.array_equal(p.download_packed(p.union_gpu(ca, cb)), oracle.union_sorted(ua, ub))
    parts = [p.create_buffer_from_packed(x) for x in np.array_split(b, 3)]
    assert np.array_equal(p.download_packed(p.union_many_gpu(parts + [ra])), oracle.union_sorted(ua, ub))


def test_diff_window_pass_regions(provider):
    """A set difference of 2,200,007 rows: 256 tiles of 8192 rows or more, so every
    tile's window of B comes from the separate window pass (k_diff_windows).  Three
    regions of keys give the three ways a tile reads its window: A every 8th key
    under a dense B (windows of about 65,536 keys, within 16 per row: streamed
    through LDS in eight 8192-key chunks), A every 32nd key under a dense B
    (windows of about 262,144 keys, above 16 per row: searched in HBM), and A
    dense over a sparse B (one chunk); half of the A keys of each region are in B."""
    p = provider
    rng = _rng(2200007)
    n1, n2 = 1_000_003, 600_001
    n3 = 2_200_007 - n1 - n2
    base2, base3 = 1 << 26, 1 << 28
    a1 = np.arange(n1, dtype=np.uint64) * 8
    b1 = np.arange(n1 * 8, dtype=np.uint64)[rng.random(n1 * 8) < 0.9]
    a2 = base2 + np.arange(n2, dtype=np.uint64) * 32
    b2 = base2 + np.arange(n2 * 32, dtype=np.uint64)[rng.random(n2 * 32) < 0.9]
    a3 = base3 + np.arange(n3, dtype=np.uint64)
    b3 = base3 + np.sort(rng.choice(n3, n3 // 8, replace=False)).astype(np.uint64)
    a = np.concatenate([a1, a2, a3])
    b = np.concatenate([b1, b2, b3])
    assert len(a) == 2_200_007 and len(a) % 8192
    ra = p.create_buffer_from_packed(rng.permutation(a))
    rb = p.create_buffer_from_packed(b)
    ua, ub = oracle.sort_dedup(a), oracle.sort_dedup(b)
    exp = oracle.diff_sorted(ua, ub)
    assert 0 < len(exp) < len(ua)
    _note(f"diff window pass: |A| {len(ua)} |B| {len(ub)} |A minus B| {len(exp)}")
    assert np.array_equal(p.download_packed(p.diff_gpu(ra, rb)), exp)
    # canonical inputs (no re-sort), and the union of the same sets
    ca, cb = p.dedup_full_row(ra), p.dedup_full_row(rb)
    assert np.array_equal(p.download_packed(p.diff_gpu(ca, cb)), exp)
    assert np.array_equal(p.download_packed(p.union_gpu(ca, cb)), oracle.union_sorted(ua, ub))


@pytest.mark.parametrize("nl,nr,keys", [(0, 10, 5), (10, 0, 5), (1, 1, 1), (5000, 3000, 100), (200000, 100000, 5000),
                                        (100000, 1000, 3)])
def test_join_project_random(provider, nl, nr, keys):
    p = provider
    _note(f"join nl={nl} nr={nr} keys={keys}")
    rng = _rng(nl + 3 * nr + keys)
    l = pack(rng.integers(0, 1 << 32, nl, dtype=np.uint64), rng.integers(0, keys, nl))
    r = pack(rng.integers(0, keys, nr), rng.integers(0, 1 << 32, nr, dtype=np.uint64))
    L, R = p.create_buffer_from_packed(l), p.create_buffer_from_packed(r)
    # Delta(x,y) join E(y,z) -> (x,z): left key col 1, right key col 0, out (0, 3)
    got = p.join_project(L, R, 1, 0, [0, 3])
    exp = oracle.join_project(l, r, 1, 0, 0, 3)
    assert got.num_rows() == len(exp) == oracle.join_count(l, r, 1, 0)
    assert np.array_equal(np.sort(p.download_packed(got)), np.sort(exp))
    # full hash join: left ++ right columns
    full = p.hash_join_v2(L, R, [1], [0])
    assert full.arity == 4 and full.num_rows() == len(exp)
    if nl * nr and len(exp) < 200000:
        rows = sorted(_rows(p, full))
        lc0, lc1 = unpack(l)
        rc0, rc1 = unpack(r)
        byk = {}
        for a, b in zip(rc0.tolist(), rc1.tolist()):
            byk.setdefault(a, []).append(b)
        brute = sorted((x, y, y, z) for x, y in zip(lc0.tolist(), lc1.tolist()) for z in byk.get(y, []))
        assert rows == brute


@pytest.mark.parametrize("nl,nr,lkeys,avals,seed", [
    (0, 10, 5, 100, 1), (10, 0, 5, 100, 2), (1, 1, 1, 1, 3), (5000, 3000, 100, 50, 4),
    (200000, 100000, 5000, 1 << 32, 5), (100000, 20000, 50, 7, 6), (300000, 50000, 3000, 2000, 7)])
def test_join_project_dedup_ordered(provider, nl, nr, lkeys, avals, seed):
    """The order-preserving fused join+project+dedup equals dedup(project(join)); small `avals`
    forces many probe rows to share an output column (interleaved runs, including runs longer
    than one LDS segment)."""
    p = provider
    _note(f"join_project_dedup nl={nl} nr={nr}")
    rng = _rng(seed)
    l = pack(rng.integers(0, avals, nl, dtype=np.uint64), rng.integers(0, lkeys, nl))
    r = pack(rng.integers(0, lkeys, nr), rng.integers(0, 1 << 32, nr, dtype=np.uint64))
    if nr > 10:
        r[: nr // 10] = r[nr // 10: 2 * (nr // 10)]  # duplicate build rows
    L, R = p.create_buffer_from_packed(l), p.create_buffer_from_packed(r)
    exp = oracle.sort_dedup(oracle.join_project(l, r, 1, 0, 0, 3))
    got = p.join_project_dedup(L, R, 1, 0, [0, 3])
    assert got.is_canonical()
    assert np.array_equal(p.download_packed(got), exp)
    # the right key column 1 (payload = column 0) and the generic shapes
    exp2 = oracle.sort_dedup(oracle.join_project(l, r, 1, 1, 0, 2))
    assert np.array_equal(p.download_packed(p.join_project_dedup(L, R, 1, 1, [0, 2])), exp2)
    exp3 = oracle.sort_dedup(oracle.join_project(l, r, 1, 0, 3, 0))
    assert np.array_equal(p.download_packed(p.join_project_dedup(L, R, 1, 0, [3, 0])), exp3)
    # a canonical build side (already a sorted set) takes the index without re-sorting
    Rc = p.dedup_full_row(R)
    got_c = p.join_project_dedup(L, Rc, 1, 0, [0, 3])
    assert got_c.is_canonical() and np.array_equal(p.download_packed(got_c), exp)


@pytest.mark.parametrize("all_unmatched", [False, True])
def test_join_project_dedup_groups_without_outputs(provider, all_unmatched):
    """Probe rows sharing their output column whose keys match nothing: groups with no outputs (some
    groups, or every group, so that the side probe emits nothing), next to lone rows that match."""
    p = provider
    rng = _rng(31 if all_unmatched else 32)
    n = 40000
    a = np.arange(n, dtype=np.uint64)
    grouped = a < 20000
    a[grouped] = a[grouped] // 4  # groups of 4 rows sharing their out column
    a[~grouped] += 1 << 20
    key = rng.integers(0, 100, n).astype(np.uint64)
    unmatched = grouped if all_unmatched else grouped & ((a % 2) == 1)
    key[unmatched] = (1 << 30) + np.arange(int(unmatched.sum()), dtype=np.uint64)
    l = pack(a, key)
    r = pack(rng.integers(0, 100, 3000), rng.integers(0, 1 << 32, 3000, dtype=np.uint64))
    exp = oracle.sort_dedup(oracle.join_project(l, r, 1, 0, 0, 3))
    got = p.join_project_dedup(p.create_buffer_from_packed(l), p.create_buffer_from_packed(r), 1, 0, [0, 3])
    assert got.is_canonical()
    assert np.array_equal(p.download_packed(got), exp)


def test_join_skewed_hot_key(provider):
    """One key holds most probe rows and a long build run (cooperative expansion)."""
    p = provider
    rng = _rng(99)
    nl, nr = 300000, 20000
    lk = np.where(rng.random(nl) < 0.6, 7, rng.integers(0, 1000, nl)).astype(np.uint64)
    rk = np.where(rng.random(nr) < 0.3, 7, rng.integers(0, 1000, nr)).astype(np.uint64)
    l = pack(rng.integers(0, 1 << 32, nl, dtype=np.uint64), lk)
    r = pack(rk, rng.integers(0, 1 << 32, nr, dtype=np.uint64))
    got = p.join_project(p.create_buffer_from_packed(l), p.create_buffer_from_packed(r), 1, 0, [0, 3])
    assert got.num_rows() == oracle.join_count(l, r, 1, 0)
    d = p.dedup_full_row(got)
    exp = oracle.sort_dedup(oracle.join_project(l, r, 1, 0, 0, 3))
    assert np.array_equal(p.download_packed(d), exp)


def test_project_and_is_sorted(provider):
    p = provider
    rel = p.create_buffer_from_u32_columns([[3, 1, 2], [30, 10, 20], [7, 8, 9]])
    pr = p.project(rel, [2, 0])
    assert _rows(p, pr) == [(7, 3), (8, 1), (9, 2)]
    assert not p.is_sorted_ascending_u32(rel, 0)
    assert p.is_sorted_ascending_u32(rel, 2)


def test_errors_fail_closed(provider):
    p = provider
    a = p.create_buffer_from_u32_columns([[1, 2]])
    b = p.create_buffer_from_u32_columns([[1, 2], [3, 4]])
    with pytest.raises(XlogError) as e:
        p.union_gpu(a, b)
    assert e.value.status == 2
    with pytest.raises(XlogError):
        p.sort(b, [5])
