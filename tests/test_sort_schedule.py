"""CPU check of the radix pass's tile order (xlog_amd/csrc/sort.hip, chunk_tile and
radix_sort_u64's grid): a threaded model of workgroup dispatch (in index order and
shuffled) with the kernel's start-order tickets or workgroup-index tiles, its tile
formula and decoupled look-back, with and without the look-back's bounded wait
(tests/sim/sort_schedule_sim.cpp).

With room for at least 8 * chunk blocks at once (the condition the host sizes
chunk for) every tile must run exactly once with its exact exclusive prefix and
no run may stall; with fewer slots the same model must be able to stall, which
shows the watchdog would catch a schedule that breaks the condition."""
import subprocess
from pathlib import Path

import pytest

SRC = Path(__file__).parent / "sim" / "sort_schedule_sim.cpp"


@pytest.fixture(scope="module")
def sim(tmp_path_factory):
    exe = tmp_path_factory.mktemp("sortsim") / "sort_schedule_sim"
    subprocess.run(["g++", "-O2", "-std=c++17", "-pthread", "-o", str(exe), str(SRC)], check=True)
    return exe


def _run(exe, trials, watchdog, mode):
    out = subprocess.run([str(exe), str(trials), str(watchdog), mode], capture_output=True, text=True,
                         check=True, timeout=600).stdout
    last = out.strip().splitlines()[-1].split()
    return dict(zip(last[0::2], map(int, last[1::2]))), out


def test_tile_order_never_stalls_with_the_host_chunk(sim):
    res, out = _run(sim, 200, 30, "ok")
    assert res == {"runs": 200, "failures": 0, "hangs": 0}, out


def test_tile_order_never_stalls_under_any_dispatch_order(sim):
    # tiles come from start-order tickets, so a shuffled dispatch order changes nothing
    res, out = _run(sim, 100, 30, "shuffled")
    assert res == {"runs": 100, "failures": 0, "hangs": 0}, out


def test_tile_order_can_stall_below_the_condition(sim):
    res, out = _run(sim, 3, 1, "tight")
    assert res["failures"] == 0 and res["hangs"] >= 1, out


def test_index_order_with_bounded_wait_never_stalls(sim):
    # the default order of the digit passes: workgroup index, shuffled dispatch, too few slots for a chunk
    # group; the bounded wait counts an unpublished predecessor itself, so every run ends with exact prefixes
    res, out = _run(sim, 40, 60, "tight-shuffled-index-fallback")
    assert res == {"runs": 40, "failures": 0, "hangs": 0}, out
    res, out = _run(sim, 60, 60, "shuffled-index-fallback")
    assert res == {"runs": 60, "failures": 0, "hangs": 0}, out


def test_index_order_without_the_bound_can_stall(sim):
    # the same schedule with an unbounded wait
    res, out = _run(sim, 3, 1, "tight-shuffled-index")
    assert res["failures"] == 0 and res["hangs"] >= 1, out
