"""CPU check of the radix pass's tile order (xlog_amd/csrc/sort.hip, chunk_tile and
radix_sort_u64's grid): a threaded model of workgroup dispatch (in index order and
shuffled) with the kernel's start-order tickets, tile formula and decoupled look-back
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
