"""GPU parity of the segment route of the radix sort.

A keys-only sort of the whole key over at least 2^22 keys, or of the high word
when its caller accepts the whole key's order (the fused join's two sorts),
whose histograms of digits 6 and 7 predict segments of at most 0.85 x 5,120
keys (xlog_amd/csrc/sort.hip, segment_route) takes two digit passes, which
order the keys by their top 16 bits, then sorts every segment on chip
(select.hip, k_seg_sort: one counting pass through LDS over the 4,096 bins of
the 12 bits below the segment's, every bin ranked by the whole key, and the
unique keys written at an offset from decoupled look-back, for sort + dedup).
A segment is the keys of 2^g consecutive top-16-bit values, g the largest (at
most 6) that keeps 4,096 keys or fewer per segment on average (6 at 2^22 keys;
XLOG_HIP_SORT_SEG_GSHIFT fixes it, and g = 0 -- C3's segments, one top-16-bit
value each -- is tested here at 2^22 keys).  A segment of more than 5,120 keys,
or a bin of more than 256 keys that are not all equal, makes the sort run every
digit's pass instead (the high-word sort: its own digits' passes).  Each case
is checked against numpy (sort) and the oracle (sort + dedup, join + project +
dedup); the route it took is read from the kernel profile."""
import sys

import numpy as np
import pytest

import oracle
from xlog_amd import datagen, pack

pytestmark = pytest.mark.gpu

N = 1 << 22
U64 = np.uint64


def _note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _route(p, fn):
    p.profile_reset()
    p.profile_enable(True)
    try:
        out = fn()
        prof = p.profile_read()
    finally:
        p.profile_enable(False)
    return out, prof["sort_segments"]["launches"], prof["sort_pass"]["launches"], prof["sort_runs"]["launches"]


def _check(p, keys, want_segments, want_passes, want_runs=0):
    """dedup_full_row against the oracle and the full-key sort against numpy, both with the expected route."""
    exp = oracle.sort_dedup(keys)
    got, segs, passes, runs = _route(p, lambda: p.download_packed(p.dedup_full_row(p.create_buffer_from_packed(keys))))
    assert np.array_equal(got, exp)
    assert (segs, passes, runs) == (want_segments, want_passes, want_runs)
    srt, segs, passes, runs = _route(
        p, lambda: p.download_packed(p.sort(p.create_buffer_from_packed(keys), [0, 1])))
    assert np.array_equal(srt, np.sort(keys))
    assert (segs, passes, runs) == (want_segments, want_passes, want_runs)


@pytest.fixture
def g0(monkeypatch):
    """Segments of one top-16-bit value each (C3's shape) at 2^22 keys."""
    monkeypatch.setenv("XLOG_HIP_SORT_SEG_GSHIFT", "0")


@pytest.mark.parametrize("n", [N, N + 12345, 3 * N - 7])
def test_uniform_keys_take_segment_route(provider, n):
    """Uniform 64-bit keys: two digit passes and one segment pass (segments of 2^6, 2^5 or 2^4 top-16-bit
    values)."""
    _note(f"segment sort: uniform n={n}")
    keys = np.random.default_rng(n).integers(0, 1 << 64, size=n, dtype=U64)
    _check(provider, keys, 1, 2)


@pytest.mark.parametrize("g", [0, 3])
def test_fixed_segment_widths(provider, monkeypatch, g):
    """XLOG_HIP_SORT_SEG_GSHIFT: segments of one and of eight top-16-bit values (about 64 and 512 keys)."""
    monkeypatch.setenv("XLOG_HIP_SORT_SEG_GSHIFT", str(g))
    _note(f"segment sort: fixed g={g}")
    _check(provider, datagen.dup_tuples(N + 99, 50 + g), 1, 2)
    _check(provider, np.random.default_rng(g).integers(0, 1 << 64, size=N + 12345, dtype=U64), 1, 2)


def test_c3_shaped_duplicates(provider):
    """C3's generator (30 % exact duplicates) at 2^23 tuples."""
    n = 2 * N
    _note(f"segment sort: c3-shaped n={n}")
    _check(provider, datagen.dup_tuples(n, datagen.seed_for(3)), 1, 2)


def test_c3_shaped_at_2_26(provider):
    """C3-shaped tuples at 2^26 (segments of 4 top-16-bit values)."""
    n = 1 << 26
    _note(f"segment sort: c3-shaped n={n}")
    keys = datagen.dup_tuples(n, 26)
    got, segs, passes, runs = _route(
        provider, lambda: provider.download_packed(provider.dedup_full_row(provider.create_buffer_from_packed(keys))))
    assert (segs, passes, runs) == (1, 2, 0)
    assert np.array_equal(got, oracle.sort_dedup(keys))


def test_constant_middle_bits(provider, g0):
    """Bits 32..47 constant: every segment is one bin (about 64 keys) ranked by the whole key."""
    rng = np.random.default_rng(3247)
    top = rng.integers(0, 1 << 16, size=N, dtype=U64)
    keys = (top << U64(48)) | (U64(0xABCD) << U64(32)) | rng.integers(0, 1 << 32, size=N, dtype=U64)
    _note("segment sort: constant bits 32..47")
    _check(provider, keys, 1, 2)


def test_constant_middle_bits_grouped(provider):
    """Bits 32..47 constant with the default width: a bin is one top-16-bit value (about 64 keys)."""
    rng = np.random.default_rng(3248)
    top = rng.integers(0, 1 << 16, size=N, dtype=U64)
    keys = (top << U64(48)) | (U64(0x1357) << U64(32)) | rng.integers(0, 1 << 32, size=N, dtype=U64)
    _note("segment sort: constant bits 32..47, grouped")
    _check(provider, keys, 1, 2)


def test_one_constant_middle_digit(provider, g0):
    """Bits 40..47 constant: the bins of bits 36..47 use 16 of their 4,096 values (bins of about 4 keys)."""
    rng = np.random.default_rng(4047)
    keys = rng.integers(0, 1 << 64, size=N, dtype=U64)
    keys = (keys & ~(U64(0xFF) << U64(40))) | (U64(0x5A) << U64(40))
    _note("segment sort: constant bits 40..47")
    _check(provider, keys, 1, 2)


def test_runs_of_exactly_256(provider, g0):
    """2^14 high words with distinct bits 36..63, each carrying exactly 256 keys: the longest bins (keys that
    share bits 36..63) the segment pass ranks; segments hold a few of them, within capacity."""
    rng = np.random.default_rng(256)
    top = rng.permutation(np.unique(rng.integers(0, 1 << 28, size=N // 128, dtype=U64)))[: N // 256]
    hi = (top << U64(4)) | rng.integers(0, 16, size=len(top), dtype=U64)
    keys = (np.repeat(hi, 256) << U64(32)) | rng.integers(0, 1 << 32, size=N, dtype=U64)
    rng.shuffle(keys)
    _note("segment sort: runs of 256")
    _check(provider, keys, 1, 2)


def test_long_bin_of_equal_keys(provider, g0):
    """One key repeated 3,000 times (alone in its bin of bits 36..63): a bin above 256 keys whose keys are all
    equal stays on the route."""
    rng = np.random.default_rng(3000)
    keys = rng.integers(0, 1 << 64, size=N, dtype=U64)
    keys[rng.choice(N, 3000, replace=False)] = U64(0x0123456789ABCDEF)
    _note("segment sort: 3,000 equal keys")
    _check(provider, keys, 1, 2)


def test_run_of_257_falls_back(provider):
    """One high word carries 257 keys (not all equal): the segment pass flags its bin and every digit takes its
    pass."""
    rng = np.random.default_rng(257)
    keys = rng.integers(0, 1 << 64, size=N + 1, dtype=U64)
    keys[rng.choice(N + 1, 257, replace=False)] = (U64(0xDEADBEEF) << U64(32)) | rng.integers(
        0, 1 << 32, size=257, dtype=U64)
    _note("segment sort: a run of 257")
    _check(provider, keys, 1, 2 + 8)


@pytest.mark.parametrize("extra", [5120 - 64, 5121])
def test_segment_at_capacity(provider, g0, extra):
    """One top-16-bit value carries about `extra` + 64 keys: 5,120 keys are sorted on chip, more fall back."""
    rng = np.random.default_rng(extra)
    keys = rng.integers(0, 1 << 64, size=N, dtype=U64)
    top = U64(0x1234)
    have = int(np.count_nonzero((keys >> U64(48)) == top))
    idx = rng.choice(np.flatnonzero((keys >> U64(48)) != top), extra + 64 - have, replace=False)
    keys[idx] = (top << U64(48)) | rng.integers(0, 1 << 48, size=len(idx), dtype=U64)
    size = int(np.count_nonzero((keys >> U64(48)) == top))
    _note(f"segment sort: a segment of {size} keys")
    _check(provider, keys, 1, 2 if size <= 5120 else 2 + 8)


def test_correlated_top_digits_fall_back(provider):
    """Top 16 bits x * 0x0101: each digit looks uniform, but the keys fill 256 of the 65,536 top-16-bit values
    (n / 256 keys each): the segments holding them are above capacity and the sort runs every digit."""
    rng = np.random.default_rng(77)
    x = rng.integers(0, 256, size=N + 3, dtype=U64)
    keys = ((x * U64(0x0101)) << U64(48)) | rng.integers(0, 1 << 48, size=N + 3, dtype=U64)
    _note("segment sort: correlated top digits")
    _check(provider, keys, 1, 2 + 8)


def test_skewed_top_bits_keep_other_routes(provider):
    """Half the keys below 2^48: the estimate rules the segment route out before any pass."""
    rng = np.random.default_rng(5)
    keys = rng.integers(0, 1 << 64, size=N + 5, dtype=U64)
    keys[: (N + 5) // 2] &= U64((1 << 48) - 1)
    _note("segment sort: skewed top bits")
    exp = oracle.sort_dedup(keys)
    got, segs, _, _ = _route(provider, lambda: provider.download_packed(
        provider.dedup_full_row(provider.create_buffer_from_packed(keys))))
    assert segs == 0
    assert np.array_equal(got, exp)


def test_index_order(provider, monkeypatch):
    """XLOG_HIP_SORT_TICKETS=0: the segment unique takes its segments in workgroup-index order."""
    keys = datagen.dup_tuples(N + 777, 11)
    monkeypatch.setenv("XLOG_HIP_SORT_TICKETS", "0")
    _note("segment sort: index order")
    got, segs, passes, _ = _route(provider, lambda: provider.download_packed(
        provider.dedup_full_row(provider.create_buffer_from_packed(keys))))
    assert (segs, passes) == (1, 2)
    assert np.array_equal(got, oracle.sort_dedup(keys))


def test_route_off_matches(provider, monkeypatch):
    """XLOG_HIP_SORT_SEGMENTS=0 turns the route off; the result is the same."""
    keys = datagen.dup_tuples(N + 99, 12)
    on = provider.download_packed(provider.dedup_full_row(provider.create_buffer_from_packed(keys)))
    monkeypatch.setenv("XLOG_HIP_SORT_SEGMENTS", "0")
    off, segs, _, _ = _route(provider, lambda: provider.download_packed(
        provider.dedup_full_row(provider.create_buffer_from_packed(keys))))
    assert segs == 0
    assert np.array_equal(on, off)


def _join_case(p, r_a, r_b, s_b, s_c, want_segments):
    R = p.create_buffer_from_u32_columns([r_a, r_b])
    S = p.create_buffer_from_u32_columns([s_b, s_c])
    exp = oracle.sort_dedup(oracle.join_project(pack(r_a, r_b), pack(s_b, s_c), 1, 0, 0, 3))
    got, segs, _, runs = _route(p, lambda: p.download_packed(p.join_project_dedup(R, S, 1, 0, [0, 3])))
    assert np.array_equal(got, exp)
    assert segs == want_segments
    return runs


def test_fused_join_sorts_take_segment_route(provider):
    """C2's shape at 2^22 rows a side (2^20 keys): the probe rows (ordered by their out column) and the build
    rows (by key, then payload) both come from the segment route, so the build side takes no short-run pass."""
    r_a, r_b, s_b, s_c = datagen.zipf_join(N, N, 1 << 20, 1.1, datagen.seed_for(2))
    _note("segment sort: fused join, C2 shape")
    assert _join_case(provider, r_a, r_b, s_b, s_c, want_segments=2) == 0


def test_fused_join_word_sort_falls_back(provider):
    """Probe out column x * 0x01010101 (each digit uniform, 256 values in all): the probe sort's segments are
    above capacity, so it runs its key-word passes instead; the build side (keys spread over u32) still takes the
    segment route.  The result is the same."""
    rng = np.random.default_rng(9)
    x = rng.integers(0, 256, size=N, dtype=np.uint64)
    r_a = (x * np.uint64(0x01010101)).astype(np.uint32)
    s_b = rng.integers(0, 1 << 32, size=N, dtype=np.uint64).astype(np.uint32)
    s_c = rng.integers(0, 1 << 32, size=N, dtype=np.uint64).astype(np.uint32)
    r_b = s_b[rng.integers(0, N, size=N)]
    _note("segment sort: fused join fallback")
    assert _join_case(provider, r_a, r_b, s_b, s_c, want_segments=2) == 0
