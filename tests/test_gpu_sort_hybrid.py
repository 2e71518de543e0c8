"""GPU parity of the high-word route of the radix sort.

A keys-only sort of the whole key over at least 2^22 keys reads its digit
histograms back first.  When they predict that the high word leaves runs of a
few keys (xlog_amd/csrc/sort.hip, short_high_runs), only the high word's digits
take radix passes and k_sort_short_runs orders every run of equal high word by
its low word; a run longer than 256 keys makes the sort run every digit's pass
instead.  Each case is checked against numpy, the route it took is read from
the kernel profile (short-run launches, digit passes), and the result is
compared with the same sort with the route switched off
(XLOG_HIP_SORT_HYBRID=0)."""
import sys

import numpy as np
import pytest

import oracle
from xlog_amd import datagen

pytestmark = pytest.mark.gpu

N_MIN = 1 << 22  # smallest sort that may take the route


@pytest.fixture(autouse=True)
def _no_segment_route(monkeypatch):
    """These sorts would take the segment route (tests/test_gpu_sort_segments.py); it is switched off so
    that the high-word route is the one under test."""
    monkeypatch.setenv("XLOG_HIP_SORT_SEGMENTS", "0")


def _note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _dedup_with_route(p, keys):
    rel = p.create_buffer_from_packed(keys)
    p.profile_reset()
    p.profile_enable(True)
    try:
        out = p.download_packed(p.dedup_full_row(rel))
        prof = p.profile_read()
    finally:
        p.profile_enable(False)
    return out, prof["sort_runs"]["launches"], prof["sort_pass"]["launches"]


def _check(p, keys, monkeypatch, want_runs, want_passes):
    exp = oracle.sort_dedup(keys)
    got, runs, passes = _dedup_with_route(p, keys)
    assert np.array_equal(got, exp)
    assert (runs, passes) == (want_runs, want_passes)
    srt = p.download_packed(p.sort(p.create_buffer_from_packed(keys), [0, 1]))
    assert np.array_equal(srt, np.sort(keys))
    monkeypatch.setenv("XLOG_HIP_SORT_HYBRID", "0")
    off, runs0, _ = _dedup_with_route(p, keys)
    monkeypatch.delenv("XLOG_HIP_SORT_HYBRID")
    assert runs0 == 0
    assert np.array_equal(off, exp)


@pytest.mark.parametrize("n", [N_MIN, N_MIN + 12345, 3 * N_MIN - 7])
def test_uniform_keys_take_high_word_route(provider, monkeypatch, n):
    """Uniform 64-bit keys: four high-word passes and one short-run pass."""
    _note(f"hybrid sort: uniform n={n}")
    keys = np.random.default_rng(n).integers(0, 1 << 64, size=n, dtype=np.uint64)
    _check(provider, keys, monkeypatch, want_runs=1, want_passes=4)


def test_c3_shaped_duplicates(provider, monkeypatch):
    """C3's generator (30 % exact duplicates) at 2^23 tuples."""
    n = 1 << 23
    _note(f"hybrid sort: c3-shaped n={n}")
    keys = datagen.dup_tuples(n, datagen.seed_for(3))
    _check(provider, keys, monkeypatch, want_runs=1, want_passes=4)


def test_runs_of_exactly_256(provider, monkeypatch):
    """2^14 random high words, each carrying exactly 256 keys: the longest runs the pass places."""
    n = N_MIN
    rng = np.random.default_rng(256)
    hi = rng.permutation(np.unique(rng.integers(0, 1 << 32, size=n // 128, dtype=np.uint64)))[: n // 256]
    keys = (np.repeat(hi, 256) << np.uint64(32)) | rng.integers(0, 1 << 32, size=n, dtype=np.uint64)
    rng.shuffle(keys)
    _note("hybrid sort: runs of 256")
    _check(provider, keys, monkeypatch, want_runs=1, want_passes=4)


def test_run_of_257_falls_back(provider, monkeypatch):
    """One high word carries 257 keys: the short-run pass flags it and every digit takes its pass."""
    n = N_MIN + 1
    rng = np.random.default_rng(257)
    keys = rng.integers(0, 1 << 64, size=n, dtype=np.uint64)
    keys[rng.choice(n, 257, replace=False)] = (np.uint64(0xDEADBEEF) << np.uint64(32)) | rng.integers(
        0, 1 << 32, size=257, dtype=np.uint64)
    _note("hybrid sort: a run of 257")
    _check(provider, keys, monkeypatch, want_runs=1, want_passes=4 + 8)


def test_correlated_high_digits_fall_back(provider, monkeypatch):
    """High words x * 0x01010101: each digit looks uniform, the word has 256 values (runs of n / 256)."""
    n = N_MIN + 3
    rng = np.random.default_rng(77)
    x = rng.integers(0, 256, size=n, dtype=np.uint64)
    keys = ((x * np.uint64(0x01010101)) << np.uint64(32)) | rng.integers(0, 1 << 32, size=n, dtype=np.uint64)
    _note("hybrid sort: correlated high digits")
    _check(provider, keys, monkeypatch, want_runs=1, want_passes=4 + 8)


def test_skewed_high_word_keeps_digit_passes(provider, monkeypatch):
    """Half the keys share one high word: the histograms rule the route out before any pass."""
    n = N_MIN + 5
    rng = np.random.default_rng(5)
    keys = rng.integers(0, 1 << 64, size=n, dtype=np.uint64)
    keys[: n // 2] &= np.uint64(0xFFFFFFFF)
    _note("hybrid sort: skewed high word")
    _check(provider, keys, monkeypatch, want_runs=0, want_passes=8)


def test_lookback_fallback(provider, monkeypatch):
    """XLOG_HIP_SORT_SPIN=2: a look-back wait of a digit pass on a tile still unpublished after two polls
    counts that tile's keys itself; the result is the same."""
    n = N_MIN + 4321
    keys = datagen.dup_tuples(n, 12)
    _note("hybrid sort: look-back fallback")
    monkeypatch.setenv("XLOG_HIP_SORT_SPIN", "2")
    got, runs, passes = _dedup_with_route(provider, keys)
    assert (runs, passes) == (1, 4)
    assert np.array_equal(got, oracle.sort_dedup(keys))


def test_index_order(provider, monkeypatch):
    """XLOG_HIP_SORT_TICKETS=0: the radix passes and the short-run unique take their tiles in workgroup-index
    order (the default numbers them by start tickets, as every other test here runs)."""
    n = N_MIN + 777
    keys = datagen.dup_tuples(n, 11)
    _note("hybrid sort: index order")
    monkeypatch.setenv("XLOG_HIP_SORT_TICKETS", "0")
    got, runs, passes = _dedup_with_route(provider, keys)
    assert (runs, passes) == (1, 4)
    assert np.array_equal(got, oracle.sort_dedup(keys))
