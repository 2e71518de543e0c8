"""Host-side mirror of the reference operator provider over the C ABI.

`HipKernelProvider` exposes the inherent methods of
`xlog_cuda::CudaKernelProvider` (crates/xlog-cuda/src/provider/mod.rs:1139) that
the reference runtime calls on the semi-naive path, with the same names,
argument meaning and error behaviour (a failed call raises `XlogError`, the
counterpart of `XlogError::Kernel`, crates/xlog-core/src/error.rs).  Every
operator is a call into libxlog_hip.so; there is no host fallback: if the
library is missing the import of this module raises.
"""
from __future__ import annotations

import ctypes as C
import weakref
from pathlib import Path
from typing import Iterable, Optional, Sequence

import numpy as np

_PKG = Path(__file__).resolve().parent
_LIB_PATH = _PKG / "libxlog_hip.so"

OK = 0
STATUS_NAMES = {
    0: "OK",
    1: "INVALID_ARG",
    2: "TYPE_MISMATCH",
    3: "CAPACITY_OVERFLOW",
    4: "ITERATION_LIMIT",
    5: "OOM",
    6: "DEVICE_ERROR",
    7: "UNSUPPORTED",
}
JOIN_INNER, JOIN_SEMI, JOIN_ANTI = 0, 1, 2
ROUTE_AUTO, ROUTE_JOIN, ROUTE_BITMAP, ROUTE_HASH = 0, 1, 2, 3


class XlogError(RuntimeError):
    """Raised for every non-OK status of the C ABI."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status
        self.message = message


class FixpointStats(C.Structure):
    _fields_ = [
        ("iterations", C.c_uint64),
        ("max_iterations", C.c_uint64),
        ("delta_sizes", C.POINTER(C.c_uint64)),
        ("delta_cap", C.c_uint64),
        ("route", C.c_uint64),
        ("wall_ms", C.c_double),
        ("max_join_rows", C.c_uint64),
        ("host_waits", C.c_uint64),
        ("delta_count", C.c_uint64),
    ]


class FjDeltaCols(C.Structure):
    """Column roles of one factorized delta step (reference FjDeltaCols,
    crates/xlog-cuda/src/provider/fj_delta.rs:50-84)."""

    _fields_ = [
        ("delta_carry", C.c_uint32),
        ("delta_key", C.c_uint32),
        ("r_carry", C.c_uint32),
        ("r_value", C.c_uint32),
    ]


#: right-linear TC orientation: delta (x, y), head (x, z)
FJ_DELTA_CANONICAL = (0, 1, 0, 1)


def _load() -> C.CDLL:
    if not _LIB_PATH.exists():
        raise ImportError(
            f"{_LIB_PATH} is not built; run `python xlog_amd/_build.py` (the HIP path has no fallback)"
        )
    lib = C.CDLL(str(_LIB_PATH))
    P, U32, U64, I32 = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int
    PP = C.POINTER(C.c_void_p)
    sig = {
        "xlog_hip_last_error": (C.c_char_p, []),
        "xlog_hip_version": (C.c_char_p, []),
        "xlog_hip_ctx_create": (I32, [I32, PP]),
        "xlog_hip_ctx_destroy": (None, [P]),
        "xlog_hip_synchronize": (I32, [P]),
        "xlog_hip_stream": (P, [P]),
        "xlog_hip_memory_stats": (I32, [P, C.POINTER(U64), C.POINTER(U64), C.POINTER(U64)]),
        "xlog_hip_trim": (I32, [P]),
        "xlog_hip_set_memory_budget": (I32, [P, U64]),
        "xlog_hip_rel_create_empty": (I32, [P, U32, PP]),
        "xlog_hip_rel_from_host_columns": (I32, [P, PP, U32, U64, PP]),
        "xlog_hip_rel_from_device_columns": (I32, [P, PP, U32, U64, PP]),
        "xlog_hip_rel_from_host_packed": (I32, [P, P, U32, U64, PP]),
        "xlog_hip_rel_download_column": (I32, [P, P, U32, P, U64]),
        "xlog_hip_rel_download_packed": (I32, [P, P, P, U64]),
        "xlog_hip_rel_num_rows": (I32, [P, C.POINTER(U64)]),
        "xlog_hip_rel_arity": (I32, [P, C.POINTER(U32)]),
        "xlog_hip_rel_is_canonical": (I32, [P, C.POINTER(I32)]),
        "xlog_hip_rel_device_words": (I32, [P, U32, PP]),
        "xlog_hip_rel_clone": (I32, [P, P, PP]),
        "xlog_hip_rel_free": (None, [P]),
        "xlog_hip_sort": (I32, [P, P, P, U32, PP]),
        "xlog_hip_dedup": (I32, [P, P, P, U32, PP]),
        "xlog_hip_dedup_full_row": (I32, [P, P, PP]),
        "xlog_hip_dedup_sorted": (I32, [P, P, P, U32, PP]),
        "xlog_hip_join_index_build": (I32, [P, P, P, U32, PP]),
        "xlog_hip_hash_join_with_index": (I32, [P, P, P, P, P, U32, I32, P, U64, PP]),
        "xlog_hip_join_index_free": (None, [P]),
        "xlog_hip_nested_loop_join": (I32, [P, P, P, U32, U32, PP]),
        "xlog_hip_fj_delta_novel": (I32, [P, P, P, P, C.POINTER(FjDeltaCols), U32, PP]),
        "xlog_hip_fj_delta_sparse_novel": (I32, [P, P, P, P, C.POINTER(FjDeltaCols), U64, PP]),
        "xlog_hip_union": (I32, [P, P, P, PP]),
        "xlog_hip_union_many": (I32, [P, PP, U32, PP]),
        "xlog_hip_diff": (I32, [P, P, P, PP]),
        "xlog_hip_hash_join": (I32, [P, P, P, U32, U32, I32, PP]),
        "xlog_hip_hash_join_keys": (I32, [P, P, P, P, P, U32, I32, PP]),
        "xlog_hip_sort_merge_join": (I32, [P, P, P, U32, U32, PP]),
        "xlog_hip_join_project": (I32, [P, P, P, U32, U32, P, U32, PP]),
        "xlog_hip_join_project_dedup": (I32, [P, P, P, U32, U32, P, U32, PP]),
        "xlog_hip_project": (I32, [P, P, P, U32, PP]),
        "xlog_hip_is_sorted": (I32, [P, P, U32, C.POINTER(I32)]),
        "xlog_hip_exclusive_scan_u32": (I32, [P, P, U64, C.POINTER(U64)]),
        "xlog_hip_exclusive_scan_u32_noalloc": (I32, [P, P, U64, C.POINTER(U64)]),
        "xlog_hip_compact": (I32, [P, P, P, PP]),
        "xlog_hip_fixpoint": (I32, [P, P, U32, PP, PP, C.POINTER(FixpointStats)]),
        "xlog_hip_fixpoint_tc": (I32, [P, P, PP, C.POINTER(FixpointStats)]),
        "xlog_hip_rel_digest": (I32, [P, P, C.POINTER(U64)]),
        "xlog_hip_profile_enable": (I32, [P, I32]),
        "xlog_hip_profile_reset": (I32, [P]),
        "xlog_hip_profile_read": (I32, [P, U32, C.POINTER(U64), C.POINTER(C.c_double), C.POINTER(C.c_double)]),
        "xlog_hip_arrow_ipc_decode_u32": (I32, [P, U64, C.POINTER(U32), C.POINTER(U64), P, U64]),
        "xlog_hip_arrow_ipc_encode_u32": (I32, [PP, U32, U64, C.POINTER(C.c_char_p), PP, C.POINTER(U64)]),
        "xlog_hip_bytes_free": (None, [P]),
        "xlog_hip_rel_from_arrow_ipc": (I32, [P, P, U64, PP]),
        "xlog_hip_rel_to_arrow_ipc": (I32, [P, P, C.POINTER(C.c_char_p), PP, C.POINTER(U64)]),
        "xlog_hip_read_arrow_ipc_stream_file": (I32, [P, C.c_char_p, PP]),
        "xlog_hip_write_arrow_ipc_stream_file": (I32, [P, P, C.POINTER(C.c_char_p), C.c_char_p]),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


_lib = _load()

#: exported symbol names the C header declares (checked by the CPU test-suite)
ABI_SYMBOLS = (
    "xlog_hip_last_error", "xlog_hip_version", "xlog_hip_ctx_create", "xlog_hip_ctx_destroy",
    "xlog_hip_synchronize", "xlog_hip_stream", "xlog_hip_memory_stats", "xlog_hip_trim", "xlog_hip_set_memory_budget",
    "xlog_hip_rel_create_empty", "xlog_hip_rel_from_host_columns", "xlog_hip_rel_from_device_columns",
    "xlog_hip_rel_from_host_packed", "xlog_hip_rel_download_column", "xlog_hip_rel_download_packed",
    "xlog_hip_rel_num_rows", "xlog_hip_rel_arity", "xlog_hip_rel_is_canonical", "xlog_hip_rel_device_words",
    "xlog_hip_rel_clone", "xlog_hip_rel_free", "xlog_hip_sort", "xlog_hip_dedup", "xlog_hip_dedup_full_row",
    "xlog_hip_dedup_sorted", "xlog_hip_join_index_build", "xlog_hip_hash_join_with_index",
    "xlog_hip_join_index_free", "xlog_hip_nested_loop_join", "xlog_hip_fj_delta_novel", "xlog_hip_fj_delta_sparse_novel",
    "xlog_hip_union", "xlog_hip_union_many", "xlog_hip_diff", "xlog_hip_hash_join", "xlog_hip_hash_join_keys",
    "xlog_hip_sort_merge_join", "xlog_hip_join_project", "xlog_hip_join_project_dedup", "xlog_hip_project",
    "xlog_hip_is_sorted",
    "xlog_hip_exclusive_scan_u32", "xlog_hip_exclusive_scan_u32_noalloc", "xlog_hip_compact", "xlog_hip_fixpoint", "xlog_hip_fixpoint_tc",
    "xlog_hip_rel_digest", "xlog_hip_profile_enable", "xlog_hip_profile_reset", "xlog_hip_profile_read",
    "xlog_hip_arrow_ipc_decode_u32", "xlog_hip_arrow_ipc_encode_u32", "xlog_hip_bytes_free",
    "xlog_hip_rel_from_arrow_ipc", "xlog_hip_rel_to_arrow_ipc", "xlog_hip_read_arrow_ipc_stream_file",
    "xlog_hip_write_arrow_ipc_stream_file",
)

KERNEL_KINDS = {
    "sort_pass": 0, "sort_hist": 1, "select": 2, "merge": 3, "probe_count": 4, "probe_emit": 5, "tc_step": 6,
    "tc_emit": 7, "chain_product": 8, "chain_finalize": 9, "chain_emit": 10, "hash_insert": 11, "sort_runs": 12,
    "sort_segments": 13,
}


def library() -> C.CDLL:
    return _lib


def library_path() -> Path:
    return _LIB_PATH


def _check(status: int) -> None:
    if status != OK:
        msg = _lib.xlog_hip_last_error()
        raise XlogError(status, msg.decode() if msg else "")


def _names_arg(names: Sequence[str] | None, arity: int):
    if names is None:
        return None
    if len(names) != arity:
        raise XlogError(1, f"{len(names)} column names for {arity} columns")
    return (C.c_char_p * arity)(*[n.encode() for n in names])


def _take_bytes(ptr: C.c_void_p, n: int) -> bytes:
    try:
        return C.string_at(ptr, n) if n else b""
    finally:
        _lib.xlog_hip_bytes_free(ptr)


def arrow_ipc_decode_u32(data: bytes) -> list[np.ndarray]:
    """Host-only decode of an Arrow IPC stream of UInt32 columns (one record batch) into numpy columns."""
    buf = np.frombuffer(data, dtype=np.uint8)
    arity, rows = C.c_uint32(), C.c_uint64()
    ptr = buf.ctypes.data if len(buf) else None
    _check(_lib.xlog_hip_arrow_ipc_decode_u32(ptr, len(buf), C.byref(arity), C.byref(rows), None, 0))
    out = np.empty((arity.value, rows.value), dtype=np.uint32)
    _check(_lib.xlog_hip_arrow_ipc_decode_u32(ptr, len(buf), C.byref(arity), C.byref(rows),
                                              out.ctypes.data if out.size else None, out.size))
    return list(out)


def arrow_ipc_encode_u32(columns: Sequence[np.ndarray], names: Sequence[str] | None = None) -> bytes:
    """Host-only encode of UInt32 columns as an Arrow IPC stream (schema, one record batch, end marker)."""
    cols = [np.ascontiguousarray(np.asarray(c, dtype=np.uint32)) for c in columns]
    rows = len(cols[0]) if cols else 0
    ptrs = (C.c_void_p * max(1, len(cols)))(*[c.ctypes.data for c in cols])
    out, n = C.c_void_p(), C.c_uint64()
    _check(_lib.xlog_hip_arrow_ipc_encode_u32(ptrs, len(cols), rows, _names_arg(names, len(cols)), C.byref(out),
                                              C.byref(n)))
    return _take_bytes(out, n.value)


def _u32_array(values: Iterable[int]):
    vals = list(values)
    return (C.c_uint32 * max(1, len(vals)))(*vals), len(vals)


class Relation:
    """Device-resident relation handle (the CudaBuffer counterpart,
    crates/xlog-cuda/src/memory.rs:1758-1930).  Freed when garbage collected."""

    __slots__ = ("_h", "_provider", "__weakref__")

    def __init__(self, provider: "HipKernelProvider", handle: C.c_void_p):
        self._provider = provider
        self._h = handle

    @property
    def handle(self) -> C.c_void_p:
        if not self._h:
            raise XlogError(1, "relation already freed")
        return self._h

    def num_rows(self) -> int:
        n = C.c_uint64()
        _check(_lib.xlog_hip_rel_num_rows(self.handle, C.byref(n)))
        return n.value

    def __len__(self) -> int:
        return self.num_rows()

    @property
    def arity(self) -> int:
        a = C.c_uint32()
        _check(_lib.xlog_hip_rel_arity(self.handle, C.byref(a)))
        return a.value

    def is_canonical(self) -> bool:
        v = C.c_int()
        _check(_lib.xlog_hip_rel_is_canonical(self.handle, C.byref(v)))
        return bool(v.value)

    def free(self) -> None:
        # After the provider's context is destroyed the device memory is already released and the
        # handle must not reach the library again; that happens when the provider and its relations
        # are collected in one batch (weak references are cleared before finalizers run, so close()
        # cannot see them).
        if self._h:
            if self._provider._ctx is not None:
                _lib.xlog_hip_rel_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class JoinIndex:
    """Reusable join index over one key column (the JoinIndexV2 counterpart,
    relational.rs:3728).  Freed when garbage collected or when its provider closes."""

    __slots__ = ("_h", "_provider", "right_keys", "__weakref__")

    def __init__(self, provider: "HipKernelProvider", handle: C.c_void_p, right_keys: Sequence[int]):
        self._provider = provider
        self._h = handle
        self.right_keys = tuple(right_keys)

    @property
    def handle(self) -> C.c_void_p:
        if not self._h:
            raise XlogError(1, "join index already freed")
        return self._h

    def free(self) -> None:
        if self._h:
            if self._provider._ctx is not None:  # see Relation.free
                _lib.xlog_hip_join_index_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class HipKernelProvider:
    """Operators over device relations on one MI355X (one context, one stream).

    Method names follow `CudaKernelProvider` (relational.rs / io.rs / transfer.rs)."""

    def __init__(self, device: int = 0):
        self._ctx = None
        self._live = weakref.WeakSet()
        h = C.c_void_p()
        _check(_lib.xlog_hip_ctx_create(device, C.byref(h)))
        self._ctx = h
        self.device = device

    # -- lifecycle --------------------------------------------------------
    def close(self) -> None:
        if getattr(self, "_ctx", None):
            # relations are context-owned device memory: release them first
            for r in list(getattr(self, "_live", ())):
                r.free()
            _lib.xlog_hip_ctx_destroy(self._ctx)
            self._ctx = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def ctx(self) -> C.c_void_p:
        if not self._ctx:
            raise XlogError(1, "provider closed")
        return self._ctx

    def synchronize(self) -> None:
        _check(_lib.xlog_hip_synchronize(self.ctx))

    def stream(self) -> int:
        return _lib.xlog_hip_stream(self.ctx) or 0

    def memory_stats(self) -> dict:
        a, b, c = C.c_uint64(), C.c_uint64(), C.c_uint64()
        _check(_lib.xlog_hip_memory_stats(self.ctx, C.byref(a), C.byref(b), C.byref(c)))
        return {"in_use": a.value, "peak": b.value, "cached": c.value}

    def trim(self) -> None:
        _check(_lib.xlog_hip_trim(self.ctx))

    def set_memory_budget(self, device_bytes: int) -> None:
        """Device memory budget in bytes, 0 for none (MemoryBudget::with_limit,
        crates/xlog-core/src/config.rs:39-45): an allocation past it raises
        XlogError with status OOM."""
        _check(_lib.xlog_hip_set_memory_budget(self.ctx, device_bytes))

    # -- kernel timing (HIP events on the context stream) --------------------
    def profile_enable(self, on: bool = True) -> None:
        _check(_lib.xlog_hip_profile_enable(self.ctx, 1 if on else 0))

    def profile_reset(self) -> None:
        _check(_lib.xlog_hip_profile_reset(self.ctx))

    def profile_read(self) -> dict:
        out = {}
        for name, kind in KERNEL_KINDS.items():
            n, ms, b = C.c_uint64(), C.c_double(), C.c_double()
            _check(_lib.xlog_hip_profile_read(self.ctx, kind, C.byref(n), C.byref(ms), C.byref(b)))
            out[name] = {"launches": n.value, "total_ms": ms.value, "algo_bytes": b.value}
        return out

    def _rel(self, h: C.c_void_p) -> Relation:
        r = Relation(self, h)
        self._live.add(r)
        return r

    # -- buffers (provider/mod.rs:3018, io.rs:75, transfer.rs:22) ---------
    def create_empty_buffer(self, arity: int) -> Relation:
        h = C.c_void_p()
        _check(_lib.xlog_hip_rel_create_empty(self.ctx, arity, C.byref(h)))
        return self._rel(h)

    def create_buffer_from_u32_columns(self, columns: Sequence[Sequence[int] | np.ndarray]) -> Relation:
        cols = [np.ascontiguousarray(np.asarray(c, dtype=np.uint32)) for c in columns]
        if not cols:
            raise XlogError(1, "at least one column is required")
        rows = len(cols[0])
        if any(len(c) != rows for c in cols):
            raise XlogError(1, "columns have different lengths")
        ptrs = (C.c_void_p * len(cols))(*[c.ctypes.data for c in cols])
        h = C.c_void_p()
        _check(_lib.xlog_hip_rel_from_host_columns(self.ctx, ptrs, len(cols), rows, C.byref(h)))
        return self._rel(h)

    create_buffer_from_slices = create_buffer_from_u32_columns

    def create_buffer_from_packed(self, keys: np.ndarray, arity: int = 2) -> Relation:
        k = np.ascontiguousarray(np.asarray(keys, dtype=np.uint64))
        h = C.c_void_p()
        _check(_lib.xlog_hip_rel_from_host_packed(self.ctx, k.ctypes.data, arity, len(k), C.byref(h)))
        return self._rel(h)

    def create_buffer_from_device_columns(self, dev_ptrs: Sequence[int], rows: int) -> Relation:
        ptrs = (C.c_void_p * len(dev_ptrs))(*dev_ptrs)
        h = C.c_void_p()
        _check(_lib.xlog_hip_rel_from_device_columns(self.ctx, ptrs, len(dev_ptrs), rows, C.byref(h)))
        return self._rel(h)

    # -- Arrow IPC streams (provider/io.rs:697-773) ---------------------
    def from_arrow_ipc_stream(self, data: bytes) -> Relation:
        buf = np.frombuffer(data, dtype=np.uint8)
        h = C.c_void_p()
        _check(_lib.xlog_hip_rel_from_arrow_ipc(self.ctx, buf.ctypes.data if len(buf) else None, len(buf),
                                                C.byref(h)))
        return self._rel(h)

    def to_arrow_ipc_stream(self, rel: Relation, names: Sequence[str] | None = None) -> bytes:
        out, n = C.c_void_p(), C.c_uint64()
        _check(_lib.xlog_hip_rel_to_arrow_ipc(self.ctx, rel.handle, _names_arg(names, rel.arity), C.byref(out),
                                              C.byref(n)))
        return _take_bytes(out, n.value)

    def read_arrow_ipc_stream_file(self, path: str | Path) -> Relation:
        h = C.c_void_p()
        _check(_lib.xlog_hip_read_arrow_ipc_stream_file(self.ctx, str(path).encode(), C.byref(h)))
        return self._rel(h)

    def write_arrow_ipc_stream_file(self, rel: Relation, path: str | Path, names: Sequence[str] | None = None) -> None:
        _check(_lib.xlog_hip_write_arrow_ipc_stream_file(self.ctx, rel.handle, _names_arg(names, rel.arity),
                                                         str(path).encode()))

    def download_column(self, rel: Relation, col: int) -> np.ndarray:
        n = rel.num_rows()
        out = np.empty(n, dtype=np.uint32)
        _check(_lib.xlog_hip_rel_download_column(self.ctx, rel.handle, col, out.ctypes.data if n else None, n))
        return out

    def download_packed(self, rel: Relation) -> np.ndarray:
        n = rel.num_rows()
        out = np.empty(n, dtype=np.uint64)
        _check(_lib.xlog_hip_rel_download_packed(self.ctx, rel.handle, out.ctypes.data if n else None, n))
        return out

    def download_rows(self, rel: Relation) -> list[tuple[int, ...]]:
        cols = [self.download_column(rel, c) for c in range(rel.arity)]
        return list(zip(*[c.tolist() for c in cols]))

    def device_row_count(self, rel: Relation) -> int:
        return rel.num_rows()

    def device_words(self, rel: Relation, word: int = 0) -> int:
        p = C.c_void_p()
        _check(_lib.xlog_hip_rel_device_words(rel.handle, word, C.byref(p)))
        return p.value or 0

    def clone_buffer(self, rel: Relation) -> Relation:
        h = C.c_void_p()
        _check(_lib.xlog_hip_rel_clone(self.ctx, rel.handle, C.byref(h)))
        return self._rel(h)

    def digest(self, rel: Relation) -> int:
        d = C.c_uint64()
        _check(_lib.xlog_hip_rel_digest(self.ctx, rel.handle, C.byref(d)))
        return d.value

    # -- operators (relational.rs) ------------------------------------------
    def sort(self, rel: Relation, key_cols: Sequence[int]) -> Relation:
        arr, n = _u32_array(key_cols)
        h = C.c_void_p()
        _check(_lib.xlog_hip_sort(self.ctx, rel.handle, arr, n, C.byref(h)))
        return self._rel(h)

    def dedup(self, rel: Relation, key_cols: Sequence[int]) -> Relation:
        arr, n = _u32_array(key_cols)
        h = C.c_void_p()
        _check(_lib.xlog_hip_dedup(self.ctx, rel.handle, arr, n, C.byref(h)))
        return self._rel(h)

    def dedup_sorted(self, rel: Relation, key_cols: Sequence[int]) -> Relation:
        """First row of every run of adjacent rows equal on key_cols (input already ordered)."""
        arr, n = _u32_array(key_cols)
        h = C.c_void_p()
        _check(_lib.xlog_hip_dedup_sorted(self.ctx, rel.handle, arr, n, C.byref(h)))
        return self._rel(h)

    def dedup_full_row(self, rel: Relation) -> Relation:
        h = C.c_void_p()
        _check(_lib.xlog_hip_dedup_full_row(self.ctx, rel.handle, C.byref(h)))
        return self._rel(h)

    def union_gpu(self, a: Relation, b: Relation) -> Relation:
        h = C.c_void_p()
        _check(_lib.xlog_hip_union(self.ctx, a.handle, b.handle, C.byref(h)))
        return self._rel(h)

    def union_many_gpu(self, rels: Sequence[Relation]) -> Relation:
        arr = (C.c_void_p * max(1, len(rels)))(*[r.handle for r in rels])
        h = C.c_void_p()
        _check(_lib.xlog_hip_union_many(self.ctx, arr, len(rels), C.byref(h)))
        return self._rel(h)

    def diff_gpu(self, a: Relation, b: Relation) -> Relation:
        h = C.c_void_p()
        _check(_lib.xlog_hip_diff(self.ctx, a.handle, b.handle, C.byref(h)))
        return self._rel(h)

    diff_full_row = diff_gpu

    def hash_join_v2(self, left: Relation, right: Relation, left_keys: Sequence[int], right_keys: Sequence[int],
                     join_type: int = JOIN_INNER) -> Relation:
        """Equi-join on key column lists (relational.rs:2926-2992); INNER output is
        left columns ++ right columns, SEMI / ANTI the matching / unmatched left rows."""
        if len(left_keys) != len(right_keys) or not left_keys:
            raise XlogError(1, "key column lists must be non-empty and of equal length")
        (lk, _), (rk, _) = _u32_array(left_keys), _u32_array(right_keys)
        h = C.c_void_p()
        _check(_lib.xlog_hip_hash_join_keys(self.ctx, left.handle, right.handle, lk, rk, len(left_keys),
                                            join_type, C.byref(h)))
        return self._rel(h)

    def build_join_index_v2(self, right: Relation, right_keys: Sequence[int]) -> JoinIndex:
        """Reusable index over a key list of the build side (relational.rs:3728-3880)."""
        if not right_keys:
            raise XlogError(1, "Join requires at least one key column")
        rk, _ = _u32_array(right_keys)
        h = C.c_void_p()
        _check(_lib.xlog_hip_join_index_build(self.ctx, right.handle, rk, len(right_keys), C.byref(h)))
        ix = JoinIndex(self, h, right_keys)
        self._live.add(ix)
        return ix

    def hash_join_v2_with_index(self, left: Relation, right: Relation, left_keys: Sequence[int],
                                right_keys: Sequence[int], join_type: int, index: JoinIndex,
                                max_output: Optional[int] = None) -> Relation:
        """hash_join_v2 against an index built over (right, right_keys) (relational.rs:3882-4000)."""
        if len(left_keys) != len(right_keys) or not left_keys:
            raise XlogError(1, "key column lists must be non-empty and of equal length")
        (lk, _), (rk, _) = _u32_array(left_keys), _u32_array(right_keys)
        h = C.c_void_p()
        _check(_lib.xlog_hip_hash_join_with_index(self.ctx, left.handle, right.handle, lk, rk, len(left_keys),
                                                  join_type, index.handle, max_output or 0, C.byref(h)))
        return self._rel(h)

    def nested_loop_join_v2_inner_u32_1key(self, left: Relation, right: Relation, left_key: int,
                                           right_key: int) -> Relation:
        h = C.c_void_p()
        _check(_lib.xlog_hip_nested_loop_join(self.ctx, left.handle, right.handle, left_key, right_key,
                                              C.byref(h)))
        return self._rel(h)

    def fj_delta_novel_u32_recorded(self, delta: Relation, edge: Relation, full_r: Relation,
                                    cols: Sequence[int] = FJ_DELTA_CANONICAL, domain: int = 1 << 16) -> Relation:
        """One factorized TC delta step: novel head tuples of delta x edge not in full_r (canonical).

        cols = (delta_carry, delta_key, r_carry, r_value); the reference's launch stream is the
        provider's stream."""
        roles = FjDeltaCols(*cols)
        h = C.c_void_p()
        _check(_lib.xlog_hip_fj_delta_novel(self.ctx, delta.handle, edge.handle, full_r.handle, C.byref(roles),
                                            domain, C.byref(h)))
        return self._rel(h)

    def fj_delta_sparse_novel_u32_recorded(self, delta: Relation, edge: Relation, full_r: Relation,
                                           cols: Sequence[int] = FJ_DELTA_CANONICAL,
                                           max_table_bytes: int = 0) -> Optional[Relation]:
        """The factorized delta step over a device hash set, no domain bound
        (fj_delta_sparse.rs:66); None when the table would exceed max_table_bytes."""
        roles = FjDeltaCols(*cols)
        h = C.c_void_p()
        _check(_lib.xlog_hip_fj_delta_sparse_novel(self.ctx, delta.handle, edge.handle, full_r.handle,
                                                   C.byref(roles), max_table_bytes, C.byref(h)))
        return self._rel(h) if h.value else None

    def sort_merge_join_v2_inner_u32_1key(self, left: Relation, right: Relation, left_key: int,
                                          right_key: int) -> Relation:
        h = C.c_void_p()
        _check(_lib.xlog_hip_sort_merge_join(self.ctx, left.handle, right.handle, left_key, right_key, C.byref(h)))
        return self._rel(h)

    def join_project(self, left: Relation, right: Relation, left_key: int, right_key: int,
                     out_cols: Sequence[int]) -> Relation:
        arr, n = _u32_array(out_cols)
        h = C.c_void_p()
        _check(_lib.xlog_hip_join_project(self.ctx, left.handle, right.handle, left_key, right_key, arr, n,
                                          C.byref(h)))
        return self._rel(h)

    def join_project_dedup(self, left: Relation, right: Relation, left_key: int, right_key: int,
                           out_cols: Sequence[int]) -> Relation:
        """Canonical set of the projected join (one rule contribution, join -> project -> dedup)."""
        arr, n = _u32_array(out_cols)
        h = C.c_void_p()
        _check(_lib.xlog_hip_join_project_dedup(self.ctx, left.handle, right.handle, left_key, right_key, arr, n,
                                                C.byref(h)))
        return self._rel(h)

    def project(self, rel: Relation, cols: Sequence[int]) -> Relation:
        arr, n = _u32_array(cols)
        h = C.c_void_p()
        _check(_lib.xlog_hip_project(self.ctx, rel.handle, arr, n, C.byref(h)))
        return self._rel(h)

    def is_sorted_ascending_u32(self, rel: Relation, col: int) -> bool:
        v = C.c_int()
        _check(_lib.xlog_hip_is_sorted(self.ctx, rel.handle, col, C.byref(v)))
        return bool(v.value)

    def exclusive_scan_u32_inplace(self, dev_ptr: int, n: int) -> int:
        t = C.c_uint64()
        _check(_lib.xlog_hip_exclusive_scan_u32(self.ctx, C.c_void_p(dev_ptr), n, C.byref(t)))
        return t.value

    def exclusive_scan_u32_inplace_noalloc(self, dev_ptr: int, n: int) -> int:
        """exclusive_scan_u32_inplace without any device allocation (scratch in
        a fixed device array; n <= 2^32; overlapping calls on one GPU race)."""
        t = C.c_uint64()
        _check(_lib.xlog_hip_exclusive_scan_u32_noalloc(self.ctx, C.c_void_p(dev_ptr), n, C.byref(t)))
        return t.value

    def compact_by_device_mask(self, rel: Relation, dev_mask_ptr: int) -> Relation:
        h = C.c_void_p()
        _check(_lib.xlog_hip_compact(self.ctx, rel.handle, C.c_void_p(dev_mask_ptr), C.byref(h)))
        return self._rel(h)

    # -- fixpoint (executor/recursive.rs:447-957) -----------------------------
    def fixpoint(self, plan: Sequence[int], relations: Sequence[Relation | None], route: int = ROUTE_AUTO,
                 max_iterations: int = 0, trace_cap: int = 4096, max_join_rows: int = 0):
        """Run a plan (see include/xlog_hip.h) to fixpoint.

        Returns (outputs, stats) where outputs[p] is the final relation of every
        IDB predicate p (None for EDB ones) and stats is a dict with
        iterations, delta_sizes (index 0 = seed), route, wall_ms and host_waits.
        max_join_rows > 0 fails a rule body's join whose output would exceed it
        (CAPACITY_OVERFLOW; 2**32 - 1 is the reference's u32 limit).  On failure
        the raised XlogError carries .stats with the iterations and delta sizes
        reached."""
        n = len(relations)
        plan_arr = (C.c_int32 * len(plan))(*plan)
        rels = (C.c_void_p * n)(*[r.handle if r is not None else None for r in relations])
        outs = (C.c_void_p * n)()
        trace = (C.c_uint64 * trace_cap)()
        st = FixpointStats(0, max_iterations, trace, trace_cap, route, 0.0, max_join_rows, 0, 0)
        status = _lib.xlog_hip_fixpoint(self.ctx, plan_arr, n, rels, outs, C.byref(st))
        stats = {"iterations": st.iterations, "route": int(st.route), "wall_ms": st.wall_ms,
                 "host_waits": st.host_waits}
        # the seed's and every completed iteration's delta size (after a failure inside an iteration,
        # "iterations" counts that iteration and the list stops before it)
        stats["delta_sizes"] = [trace[i] for i in range(min(st.delta_count, trace_cap))]
        if status != OK:
            err = XlogError(status, (_lib.xlog_hip_last_error() or b"").decode())
            err.stats = stats
            raise err
        out = [self._rel(C.c_void_p(outs[i])) if outs[i] else None for i in range(n)]
        return out, stats


# plans (int32 arrays, see include/xlog_hip.h)
def tc_plan(edge: int = 0, reach: int = 1) -> list[int]:
    """reach(X,Y) :- edge(X,Y).  reach(X,Z) :- reach(X,Y), edge(Y,Z).  (logic_bench.rs:102-110)"""
    X, Y, Z = 0, 1, 2
    return [2, reach, X, Y, 1, edge, X, Y, reach, X, Z, 2, reach, X, Y, edge, Y, Z]


def andersen_plan(assign: int = 0, addr: int = 1, load: int = 2, store: int = 3, pts: int = 4) -> list[int]:
    """Andersen points-to:
         pointsTo(V,O) :- addressOf(V,O).
         pointsTo(V,O) :- assign(V,W), pointsTo(W,O).
         pointsTo(V,O) :- load(V,W), pointsTo(W,P), pointsTo(P,O).
         pointsTo(P,O) :- store(V,W), pointsTo(V,P), pointsTo(W,O)."""
    V, W, O, P = 0, 1, 2, 3
    return [4,
            pts, V, O, 1, addr, V, O,
            pts, V, O, 2, assign, V, W, pts, W, O,
            pts, V, O, 3, load, V, W, pts, W, P, pts, P, O,
            pts, P, O, 3, store, V, W, pts, V, P, pts, W, O]


def copy_points_to_plan(addr_of: int = 0, copy: int = 1, points_to: int = 2) -> list[int]:
    """points_to(P,T) :- addr_of(P,T).  points_to(D,T) :- copy(D,S), points_to(S,T).
    (examples/xlog/50-program-analysis/01_points_to_copy.xlog)"""
    P, T, D, S = 0, 1, 2, 3
    return [2, points_to, P, T, 1, addr_of, P, T, points_to, D, T, 2, copy, D, S, points_to, S, T]


def pack(c0, c1) -> np.ndarray:
    return (np.asarray(c0, dtype=np.uint64) << np.uint64(32)) | np.asarray(c1, dtype=np.uint64)


def unpack(keys: np.ndarray):
    k = np.asarray(keys, dtype=np.uint64)
    return (k >> np.uint64(32)).astype(np.uint32), (k & np.uint64(0xFFFFFFFF)).astype(np.uint32)
