"""CPU checks of the C-ABI library: it loads, exports every symbol the header
declares, and reports errors as status codes (no compute calls here)."""
import ctypes
import re
import subprocess
import sys
from pathlib import Path

import pytest

import xlog_amd
from xlog_amd import provider as prov

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "xlog_hip.h"


def declared():
    txt = HEADER.read_text()
    return sorted(set(re.findall(r"\b(xlog_hip_[a-z0-9_]+)\s*\(", txt)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(xlog_amd.library_path()))
    names = declared()
    assert len(names) >= 35
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(xlog_amd.ABI_SYMBOLS)


def test_library_is_gfx950_code_object():
    # the offload bundle embedded in the library names its target
    data = Path(xlog_amd.library_path()).read_bytes()
    assert b"amdgcn-amd-amdhsa--gfx950" in data


def test_version_and_null_arguments_fail_closed():
    lib = prov.library()
    assert b"gfx950" in lib.xlog_hip_version()
    rows = ctypes.c_uint64()
    assert lib.xlog_hip_rel_num_rows(None, ctypes.byref(rows)) == 1  # INVALID_ARG
    assert b"NULL" in lib.xlog_hip_last_error()
    assert lib.xlog_hip_synchronize(None) == 1


def test_context_without_gpu_reports_status():
    if Path("/dev/kfd").exists():
        pytest.skip("a GPU driver is present")
    with pytest.raises(prov.XlogError) as e:
        prov.HipKernelProvider(0)
    assert e.value.status in (1, 6)


def test_bench_rejects_multi_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stdout


def test_plans_have_expected_layout():
    assert xlog_amd.tc_plan() == [2, 1, 0, 1, 1, 0, 0, 1, 1, 0, 2, 2, 1, 0, 1, 0, 1, 2]
    p = xlog_amd.andersen_plan()
    assert p[0] == 4 and len(p) == 1 + 4 * 4 + 3 * (1 + 2 + 3 + 3)
