"""CPU oracle for the semi-naive fixpoint path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this package, and only as the checker; the product path (xlog_amd) never calls
it.  `oracle.c` restates the reference semantics (see its header for the
file:line it follows); this module is a thin ctypes wrapper.

Pinning (what checks each function beyond retyping it):
  or_sort_u64 / or_unique_sorted / or_sort_dedup : numpy sort/unique, sortedness,
      the reference KATs (sort_tests.rs, test_full_row_set_algebra.rs).
  or_diff_sorted / or_union_sorted : Python set algebra, |A u B| = |A|+|B|-|A n B|,
      KATs of test_full_row_set_algebra.rs:112-163.
  or_join_project / or_join_count : nested-loop brute force on small inputs and
      the histogram identity sum_k cntL(k)*cntR(k); collision KATs join_collision_test.rs.
  or_seminaive : BFS closed form for TC (count, per-iteration deltas =
      pairs at distance k+1, iterations = max finite distance), chain / cycle /
      K_{n,n} closed forms, the reference TC and points-to KATs, and the
      independent naive fixpoint for every other plan.
  or_bfs_tc : brute-force Floyd-Warshall style reachability on tiny graphs.
  or_chain2_counts : Python sets and lists over the joined rows on small
      random relations (tests/test_oracle.py).
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

_DIR = Path(__file__).resolve().parent
_LIB_PATH = _DIR / "liboracle.so"


def build() -> Path:
    from . import _build_recipe

    return _build_recipe.build()


def _load() -> C.CDLL:
    if not _LIB_PATH.exists():
        build()
    lib = C.CDLL(str(_LIB_PATH))
    P, U64, I = C.c_void_p, C.c_uint64, C.c_int
    lib.or_sort_u64.argtypes = [P, U64]
    lib.or_sort_u64.restype = I
    lib.or_unique_sorted.argtypes = [P, U64]
    lib.or_unique_sorted.restype = U64
    lib.or_sort_dedup.argtypes = [P, U64]
    lib.or_sort_dedup.restype = U64
    lib.or_diff_sorted.argtypes = [P, U64, P, U64, P]
    lib.or_diff_sorted.restype = U64
    lib.or_union_sorted.argtypes = [P, U64, P, U64, P]
    lib.or_union_sorted.restype = U64
    lib.or_fnv1a64.argtypes = [P, U64]
    lib.or_fnv1a64.restype = U64
    lib.or_fnv1a64_bytes.argtypes = [P, U64]
    lib.or_fnv1a64_bytes.restype = U64
    lib.or_join_project.argtypes = [P, U64, P, U64, I, I, I, I, C.POINTER(P)]
    lib.or_join_project.restype = C.c_int64
    lib.or_join_count.argtypes = [P, U64, P, U64, I, I]
    lib.or_join_count.restype = U64
    lib.or_chain2_counts.argtypes = [P, U64, P, U64, P, U64, P]
    lib.or_chain2_counts.restype = I
    lib.or_free.argtypes = [P]
    lib.or_free.restype = None
    lib.or_seminaive.argtypes = [P, I, P, P, U64, P, P, C.POINTER(U64), P, U64]
    lib.or_seminaive.restype = I
    lib.or_naive.argtypes = [P, I, P, P, U64, P, P, C.POINTER(U64)]
    lib.or_naive.restype = I
    lib.or_bfs_tc.argtypes = [C.c_uint32, P, P, U64, P, U64, P, C.POINTER(U64), C.POINTER(U64)]
    lib.or_bfs_tc.restype = C.c_int64
    lib.or_set_threads.argtypes = [I]
    lib.or_set_threads.restype = I
    lib.or_max_threads.argtypes = []
    lib.or_max_threads.restype = I
    return lib


_lib = _load()


def _p(a: np.ndarray):
    return a.ctypes.data if a.size else None


def _u64(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint64))


def sort_u64(keys) -> np.ndarray:
    a = _u64(keys).copy()
    if _lib.or_sort_u64(_p(a), len(a)) != 0:
        raise MemoryError("or_sort_u64")
    return a


def sort_dedup(keys) -> np.ndarray:
    a = _u64(keys).copy()
    n = _lib.or_sort_dedup(_p(a), len(a))
    return a[:n].copy()


def diff_sorted(a, b) -> np.ndarray:
    a, b = _u64(a), _u64(b)
    out = np.empty(max(1, len(a)), np.uint64)
    n = _lib.or_diff_sorted(_p(a), len(a), _p(b), len(b), out.ctypes.data)
    return out[:n].copy()


def union_sorted(a, b) -> np.ndarray:
    a, b = _u64(a), _u64(b)
    out = np.empty(max(1, len(a) + len(b)), np.uint64)
    n = _lib.or_union_sorted(_p(a), len(a), _p(b), len(b), out.ctypes.data)
    return out[:n].copy()


def fnv1a64(keys) -> int:
    a = _u64(keys)
    return int(_lib.or_fnv1a64(_p(a), len(a)))


def fnv1a64_bytes(data: bytes) -> int:
    """FNV-1a 64 of a byte string."""
    buf = C.create_string_buffer(bytes(data), max(1, len(data)))
    return int(_lib.or_fnv1a64_bytes(C.cast(buf, C.c_void_p), len(data)))


def join_project(l, r, lk: int, rk: int, oc0: int, oc1: int) -> np.ndarray:
    """Bag of (row[oc0], row[oc1]) over L join R on L.c[lk] == R.c[rk], row = L ++ R."""
    l, r = _u64(l), _u64(r)
    outp = C.c_void_p()
    n = _lib.or_join_project(_p(l), len(l), _p(r), len(r), lk, rk, oc0, oc1, C.byref(outp))
    if n < 0:
        raise MemoryError("or_join_project")
    if n == 0:
        if outp.value:
            _lib.or_free(outp)
        return np.empty(0, np.uint64)
    buf = np.ctypeslib.as_array(C.cast(outp, C.POINTER(C.c_uint64)), shape=(n,)).copy()
    _lib.or_free(outp)
    return buf


def chain2_counts(l, a, b) -> dict:
    """Row counts of head(v, o) :- l(v, w), a(w, p), b(p, o) evaluated left-deep
    (inputs sorted unique packed rows, ids below 2^28): the first join's bag,
    its distinct (v, p) pairs, and the second join's bag over those pairs and
    over the first join's bag."""
    l, a, b = _u64(l), _u64(a), _u64(b)
    out = np.zeros(4, np.uint64)
    rc = _lib.or_chain2_counts(_p(l), len(l), _p(a), len(a), _p(b), len(b), out.ctypes.data)
    if rc != 0:
        raise ValueError(f"or_chain2_counts failed ({rc})")
    return {"bag1": int(out[0]), "set1": int(out[1]), "bag2_over_set1": int(out[2]), "bag2_over_bag1": int(out[3])}


def join_count(l, r, lk: int, rk: int) -> int:
    l, r = _u64(l), _u64(r)
    return int(_lib.or_join_count(_p(l), len(l), _p(r), len(r), lk, rk))


def _run_plan(fn_name: str, plan, relations, max_iter: int, trace_cap: int = 0):
    n = len(relations)
    rels = [_u64(r if r is not None else []) for r in relations]
    plan_arr = np.ascontiguousarray(np.asarray(plan, dtype=np.int32))
    relp = (C.c_void_p * n)(*[_p(r) for r in rels])
    reln = (C.c_uint64 * n)(*[len(r) for r in rels])
    outp = (C.c_void_p * n)()
    outn = (C.c_uint64 * n)()
    it = C.c_uint64()
    if fn_name == "seminaive":
        trace = (C.c_uint64 * max(1, trace_cap))()
        rc = _lib.or_seminaive(plan_arr.ctypes.data, n, relp, reln, max_iter, outp, outn, C.byref(it), trace,
                               trace_cap)
    else:
        trace = None
        rc = _lib.or_naive(plan_arr.ctypes.data, n, relp, reln, max_iter, outp, outn, C.byref(it))
    outs = []
    for i in range(n):
        if outp[i]:
            k = outn[i]
            arr = np.ctypeslib.as_array(C.cast(outp[i], C.POINTER(C.c_uint64)), shape=(k,)).copy() if k else \
                np.empty(0, np.uint64)
            _lib.or_free(C.c_void_p(outp[i]))
            outs.append(arr)
        else:
            outs.append(None)
    deltas = [trace[i] for i in range(min(it.value + 1, trace_cap))] if trace is not None else None
    return rc, outs, it.value, deltas


def seminaive(plan, relations, max_iter: int = 1_000_000, trace_cap: int = 4096):
    """Semi-naive fixpoint (recursive.rs:447-957).  Returns (outputs, iterations, delta_sizes);
    raises RuntimeError with code -4 when the iteration limit is hit."""
    rc, outs, it, deltas = _run_plan("seminaive", plan, relations, max_iter, trace_cap)
    if rc != 0:
        err = RuntimeError(f"or_seminaive failed ({rc})")
        err.code = rc
        err.iterations = it
        raise err
    return outs, it, deltas


def naive(plan, relations, max_rounds: int = 1_000_000):
    rc, outs, it, _ = _run_plan("naive", plan, relations, max_rounds)
    if rc != 0:
        raise RuntimeError(f"or_naive failed ({rc})")
    return outs, it


def set_threads(n: int) -> int:
    """Threads of the parallel sort / join probe / BFS paths (1 = single-threaded); returns the value set."""
    return int(_lib.or_set_threads(int(n)))


def max_threads() -> int:
    """OpenMP's default thread count (OMP_NUM_THREADS or the host's cores)."""
    return int(_lib.or_max_threads())


def bfs_tc(n_vertices: int, src, dst, want_relation: bool = True, max_dist: int = 4096, digest: bool = True):
    """Closed-form TC by BFS from every source.  Returns dict(iterations, total, digest (None when not
    asked for), dist_count (index d = #pairs at shortest distance d), relation (sorted) or None)."""
    src = np.ascontiguousarray(np.asarray(src, np.uint32))
    dst = np.ascontiguousarray(np.asarray(dst, np.uint32))
    dist = np.zeros(max_dist, np.uint64)
    total, digest_v = C.c_uint64(), C.c_uint64()
    out = None
    if want_relation:
        # first pass for the size
        _lib.or_bfs_tc(n_vertices, _p(src), _p(dst), len(src), None, 0, None, C.byref(total), C.byref(digest_v))
        out = np.empty(max(1, total.value), np.uint64)
    # the digest needs the rows in source order: with digest=False and no relation the parallel path
    # (counts only) runs when set_threads(n > 1) is in effect
    it = _lib.or_bfs_tc(n_vertices, _p(src), _p(dst), len(src), dist.ctypes.data, max_dist,
                        out.ctypes.data if out is not None else None, C.byref(total),
                        C.byref(digest_v) if (digest or want_relation) else None)
    if it < 0:
        raise MemoryError("or_bfs_tc")
    rel = out[: total.value].copy() if out is not None else None
    return {"iterations": int(it), "total": int(total.value),
            "digest": int(digest_v.value) if (digest or want_relation) else None,
            "dist_count": dist, "relation": rel}
