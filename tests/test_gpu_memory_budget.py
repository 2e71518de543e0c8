"""GPU checks of the context's device memory budget (the reference's
MemoryBudget::with_limit, crates/xlog-core/src/config.rs:39-45, enforced by
GpuMemoryManager, crates/xlog-cuda/src/memory.rs:756-770): an allocation past
it fails closed with OOM, the context stays usable, and the fixpoint's AUTO
route choice keeps its bit matrices within it (the result, iteration count
and delta sizes stay those of the oracle)."""
import gc
import sys

import numpy as np
import pytest

import oracle
from xlog_amd import ROUTE_AUTO, ROUTE_BITMAP, ROUTE_HASH, ROUTE_JOIN, XlogError, datagen, pack, tc_plan

pytestmark = pytest.mark.gpu
OOM = 5


def _note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture
def p():
    """A context of its own: its pool holds nothing of the other tests (the
    session context keeps per-context look-back state sized by the largest
    sort it ran), so the budget counts only what these tests allocate."""
    from xlog_amd import HipKernelProvider

    gc.collect()
    prov = HipKernelProvider(0)
    try:
        yield prov
    finally:
        gc.collect()
        prov.close()


def test_budget_refuses_then_recovers(p):
    rng = np.random.default_rng(5)
    keys = rng.integers(0, 1 << 64, 1 << 20, dtype=np.uint64)
    rel = p.create_buffer_from_packed(keys)  # 8 MiB held
    p.trim()
    p.set_memory_budget(4 << 20)  # below what a sort of it needs
    with pytest.raises(XlogError) as ex:
        p.dedup_full_row(rel)
    assert ex.value.status == OOM
    assert "budget" in ex.value.message
    p.set_memory_budget(0)
    d = p.dedup_full_row(rel)
    assert np.array_equal(p.download_packed(d), oracle.sort_dedup(keys))
    # a budget that allows the operation gives the same result, within the budget
    p.set_memory_budget(256 << 20)
    d2 = p.dedup_full_row(rel)
    assert np.array_equal(p.download_packed(d2), oracle.sort_dedup(keys))
    st = p.memory_stats()
    assert st["in_use"] + st["cached"] <= 256 << 20, st
    p.set_memory_budget(0)


def test_budget_steers_auto_off_the_bitmap_route(p):
    """A transitive closure over 2^17 ids takes the bitmap route (2 GiB bit
    matrices) without a budget; with a 1 GiB budget AUTO takes the hash-set
    route instead, with the same relation, iterations and delta sizes."""
    nv = 1 << 17
    src, dst = datagen.random_digraph(nv, nv // 2, 77)  # sparse: short paths, small closure
    e = pack(src, dst)
    b = oracle.bfs_tc(nv, src, dst)
    it = b["iterations"]
    deltas = [int(x) for x in b["dist_count"][1:it + 1]] + [0]
    for budget, route in ((0, ROUTE_BITMAP), (1 << 30, ROUTE_HASH)):
        _note(f"budget {budget}: tc over {nv} ids")
        p.trim()
        p.set_memory_budget(budget)
        outs, st = p.fixpoint(tc_plan(), [p.create_buffer_from_packed(e), None], route=ROUTE_AUTO)
        assert st["route"] == route
        assert np.array_equal(p.download_packed(outs[1]), b["relation"])
        assert (st["iterations"], st["delta_sizes"]) == (it, deltas)
        del outs
    p.set_memory_budget(0)
    # an explicit bitmap request under a budget too small for it fails closed
    p.trim()
    p.set_memory_budget(1 << 30)
    with pytest.raises(XlogError) as ex:
        p.fixpoint(tc_plan(), [p.create_buffer_from_packed(e), None], route=ROUTE_BITMAP)
    assert ex.value.status == OOM
    p.set_memory_budget(0)


@pytest.mark.parametrize("where", ["rule2", "rule3_second_join"])
def test_failed_fixpoint_frees_its_device_memory(p, where):
    """A fixpoint stopped by the join-row limit (CAPACITY_OVERFLOW, the
    reference's relational.rs:4550-4555) gives back every block it took.  The
    limit trips in the first recursive iteration either on rule 2's join or on
    rule 3's second join, when rule 2's head tuples and rule 3's first join
    are held (join sizes from the oracle's counts, as for C5 at its stated
    size)."""
    from xlog_amd import andersen_plan

    f = datagen.andersen(2000, 8000, 1.5, datagen.seed_for(5))
    assign, addr, load = (oracle.sort_dedup(pack(*f[k])) for k in ("assign", "addressOf", "load"))
    r2 = oracle.chain2_counts(assign, addr, np.zeros(0, np.uint64))
    r3 = oracle.chain2_counts(load, addr, addr)
    if where == "rule2":
        limit = r2["bag1"] - 1
    else:
        limit = max(r2["bag1"], r3["bag1"])
        assert r3["bag2_over_bag1"] > limit
    rels = [p.create_buffer_from_u32_columns(list(f[k])) for k in ("assign", "addressOf", "load", "store")]

    def fail_once():
        with pytest.raises(XlogError) as ex:
            p.fixpoint(andersen_plan(), rels + [None], route=ROUTE_JOIN, max_join_rows=limit)
        assert ex.value.status == 3  # CAPACITY_OVERFLOW
        assert ex.value.stats["iterations"] == 1
        del ex
        gc.collect()
        return p.memory_stats()["in_use"]

    # the first run also sizes the context's persistent look-back state; the
    # second must end with exactly the live bytes it started with
    before = fail_once()
    assert fail_once() == before
