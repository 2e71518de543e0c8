"""GPU parity of the exported scan and compaction (the C ABI's
xlog_hip_exclusive_scan_u32 and xlog_hip_compact, provider
exclusive_scan_u32_inplace / compact_by_device_mask).

Expected values come from numpy (cumsum modulo 2^32, boolean indexing) and
from the reference's own known answers (crates/xlog-cuda/tests/scan_tests.rs:6-92,
large_prefix_sum_test.rs:23-166: mask prefix sums at 6, 10, 256, 257, 512,
1,000, 5,000 and 10,000 elements; compact_device_count.rs: compaction by a
device mask).  Device arrays are the packed words of a relation: u32 element
2i is the low half of word i, element 2i + 1 the high half."""
import sys

import numpy as np
import pytest

from xlog_amd import pack

pytestmark = pytest.mark.gpu

TILE = 1024 * 16  # values per scan tile


def _note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _as_words(vals: np.ndarray) -> np.ndarray:
    """u32 values (padded to even length) as the packed u64 words holding them."""
    v = np.asarray(vals, dtype=np.uint32)
    if len(v) % 2:
        v = np.concatenate([v, np.array([0xDEADBEEF], dtype=np.uint32)])
    if len(v) == 0:
        v = np.array([0xDEADBEEF, 0xDEADBEEF], dtype=np.uint32)
    return v.view(np.uint64)


def _scan_on_device(p, vals: np.ndarray, offset_elems: int = 0):
    """Uploads vals (preceded by offset_elems sentinel values), scans len(vals)
    values in place starting offset_elems values into the buffer, and returns
    (scanned values, whole buffer after, total)."""
    pre = np.full(offset_elems, 0xA5A5A5A5, dtype=np.uint32)
    buf = np.concatenate([pre, np.asarray(vals, dtype=np.uint32)])
    words = _as_words(buf)
    rel = p.create_buffer_from_packed(words.copy())
    ptr = p.device_words(rel, 0) + 4 * offset_elems
    total = p.exclusive_scan_u32_inplace(ptr, len(vals))
    after = p.download_packed(rel).view(np.uint32)
    return after[offset_elems:offset_elems + len(vals)], after, total, len(buf)


def _expect(vals):
    v = np.asarray(vals, dtype=np.uint64)
    excl = np.concatenate([np.zeros(1, np.uint64), np.cumsum(v)[:-1]]) if len(v) else np.zeros(0, np.uint64)
    return (excl & np.uint64(0xFFFFFFFF)).astype(np.uint32), int(v.sum())


@pytest.mark.parametrize("mask,prefix,count", [
    ([1, 0, 1, 1, 0, 1], [0, 1, 1, 2, 3, 3], 4),  # scan_tests.rs:6-19
    ([0] * 10, [0] * 10, 0),                      # scan_tests.rs:23-33
    ([1] * 5, [0, 1, 2, 3, 4], 5),                # scan_tests.rs:37-47
])
def test_scan_reference_kats(provider, mask, prefix, count):
    got, _, total, _ = _scan_on_device(provider, np.array(mask))
    assert got.tolist() == prefix and total == count


def test_scan_reference_sizes(provider):
    p = provider
    # 256 with ones at 0, 127, 255 (scan_tests.rs:51-68)
    m = np.zeros(256, np.uint32)
    m[[0, 127, 255]] = 1
    got, _, total, _ = _scan_on_device(p, m)
    assert total == 3 and got[0] == 0 and got[127] == 1 and got[255] == 2
    # all ones at 257, 512 and 5,000 (scan_tests.rs:72-90, large_prefix_sum_test.rs:78-166)
    for n in (257, 512, 5000):
        got, _, total, _ = _scan_on_device(p, np.ones(n, np.uint32))
        assert total == n and np.array_equal(got, np.arange(n, dtype=np.uint32)), n
    # alternating at 1,000 and 257 (large_prefix_sum_test.rs:23-49,107-134)
    for n in (1000, 257):
        m = (np.arange(n) % 2 == 0).astype(np.uint32)
        got, _, total, _ = _scan_on_device(p, m)
        exp, cnt = _expect(m)
        assert total == cnt and np.array_equal(got, exp), n


@pytest.mark.parametrize("n", [0, 1, 2, 63, 64, 65, 1023, 1024, TILE - 1, TILE, TILE + 1, 3 * TILE + 5,
                               (1 << 20) + 3, 1 << 22])
def test_scan_sizes_vs_numpy(provider, n):
    _note(f"scan n={n}")
    rng = np.random.default_rng(1000 + n)
    vals = rng.integers(0, 1 << 12, size=n, dtype=np.uint32)
    got, after, total, blen = _scan_on_device(provider, vals)
    exp, cnt = _expect(vals)
    assert total == cnt
    assert np.array_equal(got, exp)
    # nothing past the n scanned values is written
    assert np.all(after[n:blen] == 0xDEADBEEF) if blen > n else True


@pytest.mark.parametrize("offset", [1, 2, 3])
def test_scan_unaligned_start(provider, offset):
    # a start that is not 16-byte aligned takes the scalar load path
    n = 2 * TILE + 77
    rng = np.random.default_rng(7 + offset)
    vals = rng.integers(0, 1 << 20, size=n, dtype=np.uint32)
    got, after, total, _ = _scan_on_device(provider, vals, offset_elems=offset)
    exp, cnt = _expect(vals)
    assert total == cnt and np.array_equal(got, exp)
    assert np.all(after[:offset] == 0xA5A5A5A5)


def test_scan_wraps_modulo_2_32(provider):
    # prefixes past 2^32 wrap like the reference's u32 arithmetic; the total is exact
    n = 5 * TILE + 11
    rng = np.random.default_rng(99)
    vals = rng.integers(1 << 31, 1 << 32, size=n, dtype=np.uint64).astype(np.uint32)
    got, _, total, _ = _scan_on_device(provider, vals)
    exp, cnt = _expect(vals)
    assert cnt > (1 << 40)
    assert total == cnt and np.array_equal(got, exp)


def test_scan_repeated_calls_share_state(provider):
    # consecutive scans reuse the look-back status buffer (epoch tags) and tickets
    p = provider
    for i, n in enumerate((3 * TILE, TILE + 9, 7, 4 * TILE + 1)):
        vals = np.random.default_rng(i).integers(0, 1000, size=n, dtype=np.uint32)
        got, _, total, _ = _scan_on_device(p, vals)
        exp, cnt = _expect(vals)
        assert total == cnt and np.array_equal(got, exp), n


# ---- compaction by a device mask (filter.rs:1820-1935) ------------------------
def _mask_device(p, mask: np.ndarray):
    m = np.asarray(mask, dtype=np.uint8)
    pad = (-len(m)) % 8
    b = np.concatenate([m, np.zeros(pad + (8 if len(m) == 0 else 0), np.uint8)])
    rel = p.create_buffer_from_packed(b.view(np.uint64).copy(), arity=2)
    return rel, p.device_words(rel, 0)


@pytest.mark.parametrize("kind", ["zeros", "ones", "random", "sparse"])
@pytest.mark.parametrize("n", [1, 257, 16384, 100_003])
def test_compact_vs_numpy(provider, kind, n):
    p = provider
    rng = np.random.default_rng(n)
    a = rng.integers(0, 1 << 32, size=n, dtype=np.uint64).astype(np.uint32)
    b = rng.integers(0, 1 << 32, size=n, dtype=np.uint64).astype(np.uint32)
    mask = {"zeros": np.zeros(n, np.uint8), "ones": np.ones(n, np.uint8),
            "random": rng.integers(0, 2, size=n).astype(np.uint8),
            "sparse": (rng.random(n) < 0.01).astype(np.uint8) * rng.integers(1, 256, size=n).astype(np.uint8)}[kind]
    rel = p.create_buffer_from_u32_columns([a, b])
    mrel, mptr = _mask_device(p, mask)
    out = p.compact_by_device_mask(rel, mptr)
    keep = mask != 0
    assert out.num_rows() == int(keep.sum())
    assert np.array_equal(p.download_packed(out), pack(a, b)[keep])


def test_compact_arity4_and_canonical_flag(provider):
    p = provider
    n = 40_000
    rng = np.random.default_rng(5)
    cols = [rng.integers(0, 50, size=n, dtype=np.uint32) for _ in range(4)]
    rel = p.create_buffer_from_u32_columns(cols)
    mask = rng.integers(0, 2, size=n).astype(np.uint8)
    mrel, mptr = _mask_device(p, mask)
    out = p.compact_by_device_mask(rel, mptr)
    keep = mask != 0
    for c in range(4):
        assert np.array_equal(p.download_column(out, c), cols[c][keep]), c
    assert not out.is_canonical()
    # a subset of a canonical set keeps the certificate (compact_rel keeps the order)
    canon = p.dedup_full_row(p.create_buffer_from_u32_columns([cols[0], cols[1]]))
    m2 = (np.arange(canon.num_rows()) % 3 != 0).astype(np.uint8)
    m2rel, m2ptr = _mask_device(p, m2)
    sub = p.compact_by_device_mask(canon, m2ptr)
    assert sub.is_canonical()
    assert np.array_equal(p.download_packed(sub), p.download_packed(canon)[m2 != 0])
