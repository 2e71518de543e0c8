"""Seeded synthetic inputs for the five workloads (wrapper over csrc/datagen.c).

Seeds are 0x5EED0000 + config id.  Every generator returns numpy arrays; the
same arrays feed the GPU library, the CPU checker and the benchmark.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

_LIB_PATH = Path(__file__).resolve().parent / "libxlog_datagen.so"


def _load() -> C.CDLL:
    if not _LIB_PATH.exists():
        raise ImportError(f"{_LIB_PATH} is not built; run `python xlog_amd/_build.py`")
    lib = C.CDLL(str(_LIB_PATH))
    P, U32, U64, D = C.c_void_p, C.c_uint32, C.c_uint64, C.c_double
    lib.xlog_gen_random_digraph.argtypes = [U32, U64, U64, P, P]
    lib.xlog_gen_random_digraph.restype = C.c_int
    lib.xlog_gen_zipf_join.argtypes = [U64, U64, U32, D, U64, P, P, P, P]
    lib.xlog_gen_zipf_join.restype = C.c_int
    lib.xlog_gen_dup_tuples.argtypes = [U64, U32, U32, U64, P]
    lib.xlog_gen_dup_tuples.restype = C.c_int
    lib.xlog_gen_andersen.argtypes = [U32, D, U64] + [U64, P, P] * 4
    lib.xlog_gen_andersen.restype = C.c_int
    lib.xlog_gen_chain.argtypes = [U32, P, P]
    lib.xlog_gen_chain.restype = U64
    lib.xlog_gen_cycle.argtypes = [U32, P, P]
    lib.xlog_gen_cycle.restype = U64
    lib.xlog_gen_complete_bipartite.argtypes = [U32, P, P]
    lib.xlog_gen_complete_bipartite.restype = U64
    lib.xlog_gen_ref_random_graph.argtypes = [U32, U64, U64, P, P]
    lib.xlog_gen_ref_random_graph.restype = None
    lib.xlog_gen_key_of_rank.argtypes = [U32, U64]
    lib.xlog_gen_key_of_rank.restype = U32
    return lib


_lib = _load()

SEED_BASE = 0x5EED0000


def seed_for(config_id: int) -> int:
    return SEED_BASE + config_id


def _p(a: np.ndarray):
    return a.ctypes.data if a.size else None


def random_digraph(n_vertices: int, n_edges: int, seed: int):
    """G(n, m): n_edges distinct (src, dst) pairs, src != dst, generation order."""
    src = np.empty(n_edges, np.uint32)
    dst = np.empty(n_edges, np.uint32)
    rc = _lib.xlog_gen_random_digraph(n_vertices, n_edges, seed, _p(src), _p(dst))
    if rc != 0:
        raise ValueError(f"random_digraph failed ({rc})")
    return src, dst


def chain(n: int):
    m = max(0, n - 1)
    src, dst = np.empty(m, np.uint32), np.empty(m, np.uint32)
    _lib.xlog_gen_chain(n, _p(src), _p(dst))
    return src, dst


def cycle(n: int):
    src, dst = np.empty(n, np.uint32), np.empty(n, np.uint32)
    _lib.xlog_gen_cycle(n, _p(src), _p(dst))
    return src, dst


def complete_bipartite(n: int):
    src, dst = np.empty(n * n, np.uint32), np.empty(n * n, np.uint32)
    _lib.xlog_gen_complete_bipartite(n, _p(src), _p(dst))
    return src, dst


def ref_random_graph(n: int, m: int, seed: int):
    """The reference bench generator (logic_bench.rs:48-62): duplicates and self-loops kept."""
    src, dst = np.empty(m, np.uint32), np.empty(m, np.uint32)
    _lib.xlog_gen_ref_random_graph(n, m, seed, _p(src), _p(dst))
    return src, dst


def zipf_join(n_r: int, n_s: int, n_keys: int, zipf_s: float, seed: int):
    """R(a, b): a uniform u32, b = key(Zipf(s) rank); S(b, c): b = key(uniform rank), c uniform."""
    r_a, r_b = np.empty(n_r, np.uint32), np.empty(n_r, np.uint32)
    s_b, s_c = np.empty(n_s, np.uint32), np.empty(n_s, np.uint32)
    rc = _lib.xlog_gen_zipf_join(n_r, n_s, n_keys, zipf_s, seed, _p(r_a), _p(r_b), _p(s_b), _p(s_c))
    if rc != 0:
        raise ValueError(f"zipf_join failed ({rc})")
    return r_a, r_b, s_b, s_c


def key_of_rank(rank: int, seed: int) -> int:
    return int(_lib.xlog_gen_key_of_rank(rank, seed))


def dup_tuples(n: int, seed: int, dup_num: int = 3, dup_den: int = 10) -> np.ndarray:
    """n packed u64 tuples, floor(n*dup_num/dup_den) of them exact copies of fresh ones."""
    out = np.empty(n, np.uint64)
    rc = _lib.xlog_gen_dup_tuples(n, dup_num, dup_den, seed, _p(out))
    if rc != 0:
        raise ValueError(f"dup_tuples failed ({rc})")
    return out


def andersen(n_vars: int, n_facts: int, alpha: float, seed: int):
    """assign / addressOf / load / store, 40/20/20/20 of n_facts distinct pairs each."""
    counts = [n_facts * 4 // 10, n_facts * 2 // 10, n_facts * 2 // 10, n_facts * 2 // 10]
    arrs = [(np.empty(c, np.uint32), np.empty(c, np.uint32)) for c in counts]
    args = []
    for c, (v, w) in zip(counts, arrs):
        args += [c, _p(v), _p(w)]
    rc = _lib.xlog_gen_andersen(n_vars, alpha, seed, *args)
    if rc != 0:
        raise ValueError(f"andersen failed ({rc})")
    return {"assign": arrs[0], "addressOf": arrs[1], "load": arrs[2], "store": arrs[3]}


# ---- the five configurations (BASELINE.json "configs") ----------------------
# Vertex ids spread over the whole u32 range (id v -> (v * A + B) mod 2^32, A odd,
# so a bijection; B puts vertex 7 on 0xFFFFFFFF, the all-ones id): graphs whose
# max id + 1 is ~2^32, beyond any dense bit-matrix domain.
SPARSE_ID_MUL = 2654435761
SPARSE_ID_ADD = (0xFFFFFFFF - 7 * SPARSE_ID_MUL) % (1 << 32)


def sparse_ids(v) -> np.ndarray:
    v = np.asarray(v, dtype=np.uint64)
    return ((v * np.uint64(SPARSE_ID_MUL) + np.uint64(SPARSE_ID_ADD)) & np.uint64(0xFFFFFFFF)).astype(np.uint32)


C1 = dict(n_vertices=1000, n_edges=5000)
C2 = dict(n_r=1 << 24, n_s=1 << 24, n_keys=1 << 20, zipf_s=1.1)
C3 = dict(n=1 << 28)
C4 = dict(n_vertices=32768, n_edges=3 * 32768)
C5 = dict(n_vars=500_000, n_facts=2_000_000, alpha=1.5)
# transitive closure above the dense domain: G(2^20, m) digraphs with sparse ids (seed_for(6))
TCS = dict(n_vertices=1 << 20, n_edges=int(0.9 * (1 << 20)))      # subcritical: ~9.4M tuples, 64 iterations
TCS_CRIT = dict(n_vertices=1 << 20, n_edges=1 << 20)              # critical: ~2.6e8 tuples, 418 iterations
