"""GPU test of xlog_hip_exclusive_scan_u32_noalloc, the scan whose scratch is a
fixed device array instead of allocated memory.  It is called through the C ABI
and checked against the allocating entry point (xlog_hip_exclusive_scan_u32)
on the same inputs, on consecutive calls whose second input is smaller (the
shared scratch keeps the previous call's contents), and against numpy."""
import ctypes as C
import sys

import numpy as np
import pytest

from xlog_amd.provider import library

pytestmark = pytest.mark.gpu

TILE = 1024 * 16


def _note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _noalloc(p, ptr, n):
    lib = library()
    lib.xlog_hip_exclusive_scan_u32_noalloc.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64,
                                                        C.POINTER(C.c_uint64)]
    lib.xlog_hip_exclusive_scan_u32_noalloc.restype = C.c_int
    t = C.c_uint64(12345)
    st = lib.xlog_hip_exclusive_scan_u32_noalloc(p.ctx, C.c_void_p(ptr), n, C.byref(t))
    return st, t.value


def _device_copy(p, vals):
    v = np.asarray(vals, dtype=np.uint32)
    if len(v) % 2:
        v = np.concatenate([v, np.array([0xDEADBEEF], np.uint32)])
    if len(v) == 0:
        v = np.array([0xDEADBEEF, 0xDEADBEEF], np.uint32)
    rel = p.create_buffer_from_packed(v.view(np.uint64).copy())
    return rel, p.device_words(rel, 0)


def _both(p, vals):
    """(noalloc result, noalloc total, allocating result, allocating total) on copies of vals."""
    n = len(vals)
    r1, p1 = _device_copy(p, vals)
    st, t1 = _noalloc(p, p1, n)
    assert st == 0, st
    r2, p2 = _device_copy(p, vals)
    t2 = p.exclusive_scan_u32_inplace(p2, n)
    a1 = p.download_packed(r1).view(np.uint32)
    a2 = p.download_packed(r2).view(np.uint32)
    return a1, t1, a2, t2


@pytest.mark.parametrize("sizes", [(5 * TILE + 123, 2 * TILE + 7), (3 * TILE, 1000), ((1 << 22) + 5, 257),
                                   (TILE + 1, 0)])
def test_noalloc_scan_matches_allocating_scan(provider, sizes):
    p = provider
    for i, n in enumerate(sizes):
        _note(f"noalloc scan call {i} n={n}")
        rng = np.random.default_rng(17 * n + i)
        vals = rng.integers(0, 1 << 32, size=n, dtype=np.uint64).astype(np.uint32)
        a1, t1, a2, t2 = _both(p, vals)
        assert t1 == t2 == int(vals.astype(np.uint64).sum())
        assert np.array_equal(a1, a2)
        excl = (np.concatenate([np.zeros(1, np.uint64), np.cumsum(vals.astype(np.uint64))[:-1]]) & np.uint64(0xFFFFFFFF)).astype(np.uint32) \
            if n else np.zeros(0, np.uint32)
        assert np.array_equal(a1[:n], excl)


def test_noalloc_scan_unaligned_and_repeated(provider):
    p = provider
    n = 2 * TILE + 99
    vals = np.random.default_rng(4).integers(0, 1 << 16, size=n + 1, dtype=np.uint32)
    vals[0] = 0xA5A5A5A5
    for _ in range(3):
        rel, ptr = _device_copy(p, vals)
        st, t = _noalloc(p, ptr + 4, n)  # starts one value in: the scalar load path
        assert st == 0
        got = p.download_packed(rel).view(np.uint32)
        assert got[0] == 0xA5A5A5A5
        exp = (np.concatenate([np.zeros(1, np.uint64), np.cumsum(vals[1:].astype(np.uint64))[:-1]]) & np.uint64(0xFFFFFFFF)).astype(np.uint32)
        assert np.array_equal(got[1:n + 1], exp)
        assert t == int(vals[1:].astype(np.uint64).sum())


def test_noalloc_scan_rejects_above_maximum(provider):
    # checked on the host before any launch: 2^32 + 1 values is CAPACITY_OVERFLOW
    p = provider
    rel, ptr = _device_copy(p, np.zeros(4, np.uint32))
    st, _ = _noalloc(p, ptr, (1 << 32) + 1)
    assert st == 3
    assert b"exceeds the maximum" in library().xlog_hip_last_error()


def test_noalloc_scan_allocates_nothing(provider):
    # the pool's live and cached bytes do not change across the call
    p = provider
    vals = np.arange(3 * TILE, dtype=np.uint32)
    rel, ptr = _device_copy(p, vals)
    before = p.memory_stats()
    st, t = _noalloc(p, ptr, len(vals))
    after = p.memory_stats()
    assert st == 0 and t == int(vals.astype(np.uint64).sum())
    assert before["in_use"] == after["in_use"] and before["cached"] == after["cached"]
