"""GPU parity of the radix sort at every tile-order chunk size.

The digit passes deal tiles to the XCDs in chunks of consecutive tiles by
workgroup index (xlog_amd/csrc/sort.hip, chunk_tile): 8 tiles per chunk from
512 tiles up, and tiles / 64 below that, so sorts of 64-511 tiles run with
chunks of 1..7 and a last group of blocks partly without a tile.  The tests of
this module take XLOG_HIP_SORT_TICKETS=0 (the fused short-run unique by
workgroup index too), except test_tile_orders, which runs every order and the
look-back's counting fallback.  Keys-only sorts use 8192-key tiles;
sorts that carry a row payload (the keyed sort of arity-3/4 rows, join index
builds) use 4096-key tiles.  Every size here is checked against numpy: the full
sort + dedup, a stable sort on one key column, and narrow keys whose constant
digits are skipped, and sorts whose lowest digit (the pass queued before the
histograms are read back) is constant."""
import sys

import numpy as np
import pytest

import oracle
from xlog_amd import pack

pytestmark = pytest.mark.gpu

TILE_K = 8192  # keys-only tile


@pytest.fixture(autouse=True)
def _index_order(monkeypatch):
    """The chunked workgroup-index order, whose chunk sizes these tests walk."""
    monkeypatch.setenv("XLOG_HIP_SORT_TICKETS", "0")


def _note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


# tile counts covering chunk = 1..8 (tiles // 64, capped at 8) with ragged last tiles
TILES = [64, 130, 200, 260, 330, 400, 450, 511, 512, 700]


@pytest.mark.parametrize("tiles", TILES)
def test_sort_dedup_every_chunk(provider, tiles):
    p = provider
    n = tiles * TILE_K - (tiles * 37) % 5000  # ragged last tile
    _note(f"sort sizes: tiles={tiles} n={n} chunk={min(8, max(1, (n + TILE_K - 1) // TILE_K // 64))}")
    rng = np.random.default_rng(tiles)
    keys = rng.integers(0, 1 << 64, size=n, dtype=np.uint64)
    keys[rng.integers(0, n, size=n // 4)] = keys[rng.integers(0, n, size=n // 4)]
    rel = p.create_buffer_from_packed(keys)
    assert np.array_equal(p.download_packed(p.sort(rel, [0, 1])), np.sort(keys))
    assert np.array_equal(p.download_packed(p.dedup_full_row(rel)), oracle.sort_dedup(keys))


@pytest.mark.parametrize("tiles", [70, 150, 333])
def test_stable_column_sort_every_chunk(provider, tiles):
    """Sort by the second column only: a 4-digit pass range, stable (equal keys keep input order)."""
    p = provider
    n = tiles * TILE_K - 123
    rng = np.random.default_rng(1000 + tiles)
    c0 = np.arange(n, dtype=np.uint32)  # input order, to check stability
    c1 = rng.integers(0, 5000, n, dtype=np.uint32)
    rel = p.create_buffer_from_u32_columns([c0, c1])
    got = p.download_packed(p.sort(rel, [1]))
    order = np.argsort(c1, kind="stable")
    assert np.array_equal(got, pack(c0[order], c1[order]))


@pytest.mark.parametrize("tiles", [90, 260, 480])
def test_narrow_keys_every_chunk(provider, tiles):
    """Transitive-closure-shaped keys (both columns < 2^15): four of the eight digits are constant and skipped."""
    p = provider
    n = tiles * TILE_K - 777
    rng = np.random.default_rng(2000 + tiles)
    keys = pack(rng.integers(0, 1 << 15, n), rng.integers(0, 1 << 15, n))
    rel = p.create_buffer_from_packed(keys)
    assert np.array_equal(p.download_packed(p.dedup_full_row(rel)), oracle.sort_dedup(keys))


@pytest.mark.parametrize("rows", [300_000, 1_100_000, 2_000_001])
def test_payload_sort_every_chunk(provider, rows):
    """Arity-4 rows sorted on two columns: the key + row-index (payload) sort with 4096-key tiles."""
    p = provider
    rng = np.random.default_rng(rows)
    cols = [rng.integers(0, 50, rows, dtype=np.uint32) for _ in range(2)] + \
           [rng.integers(0, 1 << 32, rows, dtype=np.uint64).astype(np.uint32) for _ in range(2)]
    rel = p.create_buffer_from_u32_columns(cols)
    out = p.sort(rel, [1, 0])
    order = np.lexsort((cols[0], cols[1]))  # primary column 1, then column 0, stable
    for c in range(4):
        assert np.array_equal(p.download_column(out, c), cols[c][order])


@pytest.mark.parametrize("n", [1000, 70_001, 300 * TILE_K + 5])
def test_constant_lowest_digit(provider, n):
    """Keys whose lowest byte is the same everywhere.  The lowest digit's pass is
    queued before the histograms are read back, so here it runs as a stable copy
    and the later digits must still give the exact order."""
    p = provider
    rng = np.random.default_rng(3000 + n)
    keys = (rng.integers(0, 1 << 50, n, dtype=np.uint64) << np.uint64(8)) | np.uint64(0x5A)
    keys[rng.integers(0, n, n // 3)] = keys[rng.integers(0, n, n // 3)]
    rel = p.create_buffer_from_packed(keys)
    assert np.array_equal(p.download_packed(p.sort(rel, [0, 1])), np.sort(keys))
    assert np.array_equal(p.download_packed(p.dedup_full_row(rel)), oracle.sort_dedup(keys))


@pytest.mark.parametrize("n", [2, 4097, 200 * TILE_K + 9])
def test_all_keys_equal(provider, n):
    """Every digit is constant: only the speculative pass runs, and it must leave the rows intact."""
    p = provider
    keys = np.full(n, 0x0123456789ABCDEF, dtype=np.uint64)
    rel = p.create_buffer_from_packed(keys)
    assert np.array_equal(p.download_packed(p.sort(rel, [0, 1])), keys)
    assert np.array_equal(p.download_packed(p.dedup_full_row(rel)), keys[:1])


@pytest.mark.parametrize("n", [5000, 150 * TILE_K - 17])
def test_stable_sort_column_with_constant_low_byte(provider, n):
    """Sort by a column whose values are multiples of 256: its lowest digit's pass is a stable copy."""
    p = provider
    rng = np.random.default_rng(4000 + n)
    c0 = np.arange(n, dtype=np.uint32)
    c1 = (rng.integers(0, 3000, n, dtype=np.uint32) * 256).astype(np.uint32)
    rel = p.create_buffer_from_u32_columns([c0, c1])
    got = p.download_packed(p.sort(rel, [1]))
    order = np.argsort(c1, kind="stable")
    assert np.array_equal(got, pack(c0[order], c1[order]))


# the counting fallback reads a whole tile per wait, so its mode runs up to a few hundred tiles
_TILE_ORDER_CASES = [(o, t) for o in ("default", "ticket", "index", "fallback") for t in (1, 64, 260, 700, 2100)
                     if not (o == "fallback" and t > 260)]


@pytest.mark.parametrize("order,tiles", _TILE_ORDER_CASES)
def test_tile_orders(provider, monkeypatch, tiles, order):
    # default: digit passes by workgroup index in XCD chunks with the bounded look-back wait, the fused
    # short-run unique by start tickets; XLOG_HIP_SORT_TICKETS=1 tickets for both, =0 workgroup index for
    # both; fallback: XLOG_HIP_SORT_SPIN=0 (up to 64 tiles: every wait on an unpublished tile counts that
    # tile's keys instead of polling again) or 2 (after two polls; a digit thread reads a whole tile per
    # count, so this mode is kept to a few hundred tiles)
    p = provider
    monkeypatch.delenv("XLOG_HIP_SORT_TICKETS", raising=False)
    if order == "ticket":
        monkeypatch.setenv("XLOG_HIP_SORT_TICKETS", "1")
    elif order == "index":
        monkeypatch.setenv("XLOG_HIP_SORT_TICKETS", "0")
    elif order == "fallback":
        monkeypatch.setenv("XLOG_HIP_SORT_SPIN", "0" if tiles <= 64 else "2")
    n = tiles * TILE_K - (tiles * 53) % 3000
    _note(f"sort tile order {order}: tiles={tiles} n={n}")
    rng = np.random.default_rng(1000 + tiles)
    keys = rng.integers(0, 1 << 64, size=n, dtype=np.uint64)
    keys[rng.integers(0, n, n // 4)] = keys[rng.integers(0, n, n // 4)]  # duplicates
    d = p.dedup_full_row(p.create_buffer_from_packed(keys))
    assert np.array_equal(p.download_packed(d), np.unique(keys))
    # a stable keyed sort (payload passes) under the same order
    c0 = rng.integers(0, 1000, size=min(n, 400_000), dtype=np.uint32)
    c1 = np.arange(len(c0), dtype=np.uint32)
    c2 = rng.integers(0, 7, size=len(c0), dtype=np.uint32)
    s = p.sort(p.create_buffer_from_u32_columns([c0, c1, c2]), [2, 0])
    order = np.lexsort((c0, c2))  # stable: by c2, then c0, ties in input order
    assert np.array_equal(p.download_column(s, 1), c1[order])


@pytest.mark.parametrize("n", [2, 3, 1000, 1024, 1025, 4097, 8191, 8192, 8193])
def test_small_sort_unique(provider, n):
    """Sort + dedup of one tile or less and just past it: random keys, many duplicates, all-equal keys and keys
    of all ones (the largest u64)."""
    p = provider
    _note(f"small sort unique n={n}")
    rng = np.random.default_rng(n + 5)
    cases = [rng.integers(0, 1 << 64, size=n, dtype=np.uint64),
             rng.integers(0, max(2, n // 3), size=n, dtype=np.uint64),
             np.full(n, 12345, dtype=np.uint64)]
    top = rng.integers(0, 1 << 64, size=n, dtype=np.uint64)
    top[rng.choice(n, max(1, n // 4), replace=False)] = np.uint64(0xFFFFFFFFFFFFFFFF)
    cases.append(top)
    for keys in cases:
        got = p.download_packed(p.dedup_full_row(p.create_buffer_from_packed(keys)))
        assert np.array_equal(got, np.unique(keys))
