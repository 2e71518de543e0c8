"""Queued iterations of the join route: programs whose recursive rules each
read one IDB atom (transitive closure, left-linear closure, mutual recursion,
same generation) run several iterations per read-back with every row count on
the device (libxlog_hip's Driver::run_queue); so do programs whose rules read
an IDB relation in full beside the delta (non-linear closure, Andersen, a
four-atom body with two IDB atoms), whose indexes over R are rebuilt on the
device at the start of every queued iteration.  Checked against the oracle
(relations, iteration count, every delta size) with the queue on and off, with
its bounds shrunk so that queues stop and the stopped iteration runs from the
host (XLOG_HIP_JOIN_QUEUE_MARGIN_PCT / XLOG_HIP_JOIN_QUEUE_SLACK), at the
iteration limit and at the join-row limit (the reference's u32 limit,
relational.rs:4550-4555), whose failure must match the unqueued loop's."""
import sys

import numpy as np
import pytest

import oracle
from xlog_amd import ROUTE_JOIN, XlogError, andersen_plan, datagen, pack, tc_plan

import chain_plans as cp

pytestmark = pytest.mark.gpu

CAPACITY_OVERFLOW, ITERATION_LIMIT = 3, 4


def _note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _graph(n, m, seed):
    s, d = datagen.random_digraph(n, m, seed)
    return np.asarray(s, np.uint32), np.asarray(d, np.uint32)


def _run(p, plan, rels, **kw):
    dev = [p.create_buffer_from_packed(r) if r is not None else None for r in rels]
    return p.fixpoint(plan, dev, route=ROUTE_JOIN, **kw)


def _programs():
    s, d = _graph(1500, 2600, 31)
    e = pack(s, d)
    rng = np.random.default_rng(32)
    n = 3000
    child = np.arange(1, n, dtype=np.uint32)
    parent = np.array([rng.integers(max(0, int(c) - 40), int(c)) for c in child], dtype=np.uint32)
    fs = rng.integers(0, n, n // 4).astype(np.uint32)
    fd = rng.integers(0, n, n // 4).astype(np.uint32)
    # ids spread over u32: the sorts inside the loop run every digit pass
    ss, sd = (datagen.sparse_ids(x) for x in _graph(1200, 1500, 33))
    return [
        ("tc", tc_plan(), [e, None], [1]),
        ("left tc", cp.left_tc_plan(), [e, None], [1]),
        ("parity", cp.parity_plan(), [e, None, None], [1, 2]),
        ("same generation", cp.same_generation_plan(), [pack(fs, fd), pack(child, parent), pack(parent, child), None],
         [3]),
        ("sparse-id tc", tc_plan(), [pack(ss, sd), None], [1]),
    ]


def _nonlinear_programs():
    s, d = _graph(1500, 2600, 31)
    f = datagen.andersen(600, 2400, 1.5, datagen.seed_for(5))
    a_s, a_d = _graph(400, 600, 36)
    b_s, b_d = _graph(400, 380, 37)
    ss, sd = (datagen.sparse_ids(x) for x in _graph(1200, 1700, 38))
    return [
        ("nonlinear tc", cp.nonlinear_tc_plan(), [pack(s, d), None], [1]),
        ("andersen", andersen_plan(), [pack(*f[k]) for k in ("assign", "addressOf", "load", "store")] + [None], [4]),
        ("quad", cp.quad_plan(), [pack(a_s, a_d), pack(b_s, b_d), None], [2]),
        ("sparse-id nonlinear tc", cp.nonlinear_tc_plan(), [pack(ss, sd), None], [1]),
    ]


def _check(p, name, plan, rels, idb, ref):
    outs_o, it_o, deltas_o = ref
    outs, st = _run(p, plan, rels)
    assert st["route"] == ROUTE_JOIN
    for q in idb:
        got = p.download_packed(outs[q])
        assert np.array_equal(got, outs_o[q]), f"{name} pred {q}"
        assert outs[q].is_canonical()
    assert st["iterations"] == it_o, name
    assert st["delta_sizes"] == deltas_o, name
    return st


def test_queued_join_route_matches_oracle(provider, monkeypatch):
    """Queue on (8 iterations per read-back) and off (XLOG_HIP_JOIN_QUEUE=1): the same relations,
    iterations and deltas; the queue takes fewer read-backs (after the seed and one host iteration,
    about one per 8 iterations)."""
    p = provider
    for name, plan, rels, idb in _programs():
        ref = oracle.seminaive(plan, rels)
        waits = {}
        for queue in ("1", "8"):
            monkeypatch.setenv("XLOG_HIP_JOIN_QUEUE", queue)
            _note(f"join queue {name} queue={queue}")
            waits[queue] = _check(p, name, plan, rels, idb, ref)["host_waits"]
        it = ref[1]
        assert it > 16, (name, it)
        assert waits["8"] < waits["1"] - it // 2, (name, it, waits)
        assert waits["8"] <= it // 8 + 12, (name, it, waits)


def test_queued_join_route_nonlinear(provider, monkeypatch):
    """Variants that read an IDB relation in full (through an index rebuilt on the device every queued
    iteration from R's two runs, by its first or second column): queue on and off give the oracle's
    relations, iterations and deltas, and the queue takes fewer read-backs."""
    p = provider
    for name, plan, rels, idb in _nonlinear_programs():
        ref = oracle.seminaive(plan, rels)
        waits = {}
        for queue in ("1", "8"):
            monkeypatch.setenv("XLOG_HIP_JOIN_QUEUE", queue)
            _note(f"join queue {name} queue={queue}")
            waits[queue] = _check(p, name, plan, rels, idb, ref)["host_waits"]
        it = ref[1]
        assert it >= 4, (name, it)
        # an iteration whose candidates pass one sort (2^30 - 1 keys) still runs from the host, in pieces
        _note(f"join queue {name}: {it} iterations, host waits {waits}")
        assert waits["8"] <= waits["1"] // 2, (name, it, waits)


@pytest.mark.parametrize("margin,slack", [(50, 16), (90, 64), (100, 1024)])
def test_queued_join_route_stops_and_resumes(provider, monkeypatch, margin, slack):
    """Bounds below the real sizes: queues stop (a check kernel raises the stop flag, every later launch
    of the queue returns), the completed iterations are kept and the stopped one runs again; the
    result is still the oracle's."""
    p = provider
    monkeypatch.setenv("XLOG_HIP_JOIN_QUEUE_MARGIN_PCT", str(margin))
    monkeypatch.setenv("XLOG_HIP_JOIN_QUEUE_SLACK", str(slack))
    for name, plan, rels, idb in _programs() + _nonlinear_programs():
        _note(f"join queue stops {name} margin={margin} slack={slack}")
        _check(p, name, plan, rels, idb, oracle.seminaive(plan, rels))


@pytest.mark.parametrize("mode,filt", [("0", "1"), ("1", "1"), ("2", "1"), ("3", "1"), ("3", "0"), ("0", "0")])
def test_queued_join_route_group_bitmap_modes(provider, monkeypatch, mode, filt):
    """Grouped heads over a small domain find their new rows by per-group LDS bitmaps.
    XLOG_HIP_GROUP_BITMAP: 0 sort + set difference instead; 1 R's rows read from its two runs; 2 from R
    as a bit matrix that every iteration brings up to date, the runs merged as before; 3 (the default)
    R kept only in the matrix, from queue to queue, by heads that no index reads in full, and written
    back to R's runs when a host iteration or the end of the fixpoint reads them.  Heads whose
    candidates are not grouped (left-linear closure, same generation, the non-linear programs) filter
    their join outputs against R's matrix and the outputs already taken, and every step before a last
    one drops repeated outputs (XLOG_HIP_JOIN_FILTER=0: sort + set difference instead).  Each setting
    with the queue's own bounds and with bounds shrunk so that queues stop and host iterations come
    between them (R's runs written back, the matrix rebuilt after the host iteration); every result is
    the oracle's."""
    p = provider
    monkeypatch.setenv("XLOG_HIP_GROUP_BITMAP", mode)
    monkeypatch.setenv("XLOG_HIP_JOIN_FILTER", filt)
    for name, plan, rels, idb in _programs() + _nonlinear_programs():
        ref = oracle.seminaive(plan, rels)
        for stops in (False, True):
            if stops:
                monkeypatch.setenv("XLOG_HIP_JOIN_QUEUE_MARGIN_PCT", "50")
                monkeypatch.setenv("XLOG_HIP_JOIN_QUEUE_SLACK", "16")
            else:
                monkeypatch.delenv("XLOG_HIP_JOIN_QUEUE_MARGIN_PCT", raising=False)
                monkeypatch.delenv("XLOG_HIP_JOIN_QUEUE_SLACK", raising=False)
            _note(f"join queue group bitmap mode={mode} filter={filt} {name} stops={stops}")
            _check(p, name, plan, rels, idb, ref)


def test_queued_join_route_small_and_empty(provider):
    """Edge cases: no edges, one edge, a cycle (the last iterations derive nothing), a head with
    initial contents, and an iteration limit reached inside a queue."""
    p = provider
    cyc = np.arange(40, dtype=np.uint32)
    cases = [
        ("no edges", [np.zeros(0, np.uint64), None]),
        ("one edge", [pack(np.array([3], np.uint32), np.array([7], np.uint32)), None]),
        ("cycle", [pack(cyc, (cyc + 1) % 40), None]),
        ("chain", [pack(cyc[:-1], cyc[1:]), None]),
    ]
    s, d = _graph(600, 900, 34)
    hs, hd = _graph(600, 200, 35)
    cases.append(("initial head", [pack(s, d), pack(hs, hd)]))
    for name, rels in cases:
        _note(f"join queue edge case {name}")
        _check(p, name, tc_plan(), rels, [1], oracle.seminaive(tc_plan(), rels))
    # the 40-cycle needs 40 iterations: a limit of 25 stops inside a queue
    cycle = cases[2][1]
    with pytest.raises(XlogError) as ex:
        _run(p, tc_plan(), cycle, max_iterations=25)
    assert ex.value.status == ITERATION_LIMIT
    assert ex.value.stats["iterations"] == 25
    assert ex.value.stats["delta_sizes"] == oracle.seminaive(tc_plan(), cycle)[2][:26]


def test_queued_join_route_join_row_limit(provider, monkeypatch):
    """A join-row limit trips inside a queue: the error, its iteration and the delta sizes reached are
    those of the loop without a queue."""
    p = provider
    s, d = _graph(1500, 2600, 31)
    rels = [pack(s, d), None]
    _, it_o, deltas_o = oracle.seminaive(tc_plan(), rels)
    # the largest delta times the largest out-degree bounds every join; a limit below the peak join trips
    peak = max(deltas_o)
    limit = peak  # the join of the peak delta with the edges has more rows than the delta itself
    results = {}
    for queue in ("1", "8"):
        monkeypatch.setenv("XLOG_HIP_JOIN_QUEUE", queue)
        with pytest.raises(XlogError) as ex:
            _run(p, tc_plan(), rels, max_join_rows=limit)
        e = ex.value
        assert e.status == CAPACITY_OVERFLOW
        assert "exceeds the row limit" in e.message
        results[queue] = (e.message, e.stats["iterations"], e.stats["delta_sizes"])
        del ex
    assert results["1"] == results["8"]
    assert results["8"][2] == deltas_o[:len(results["8"][2])]
