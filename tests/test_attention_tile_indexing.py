"""CPU replay of the stored-tile attention backward's addressing (no GPU).

Builds tests/attention_tile_index_check.hip, which calls the kernels' own
__host__ __device__ index functions for every workgroup, wave, lane, register
and block of the dQ kernel's tile stores and the dK/dV kernel's tile loads, at
every degree 0..8 and head dim, over square, ragged, causal, windowed and
randomly masked shapes. The float32 layout in use must be in bounds, aligned,
written once per element and read back from the element written for the same
(query, key) pair. The float64 layout of the first stored-tile build (the one
that took a GPU memory fault) is in bounds and consistent as well, so its
addressing is not the fault's cause. The float32 layout with float64's
accumulator rows (acc_row = 4 r + h) misassigns values, which is why the
stored-tile kernels refuse float64 at compile time.
"""

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


@pytest.fixture(scope="module")
def report(tmp_path_factory):
    if not (os.path.exists(HIPCC) or shutil.which("hipcc")):
        pytest.skip("hipcc is not available")
    exe = str(tmp_path_factory.mktemp("tile_check") / "tile_check")
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-O2", "-std=c++17", "-I", os.path.join(ROOT, "include"),
                    "-I", os.path.join(ROOT, "polytensors_amd", "csrc"),
                    os.path.join(ROOT, "tests", "attention_tile_index_check.hip"), "-o", exe],
                   check=True, capture_output=True, text=True)
    out = subprocess.run([exe], check=True, capture_output=True, text=True, timeout=300).stdout
    modes = {}
    for line in out.splitlines():
        name, *fields = line.split()
        modes[name] = {k: int(v) for k, v in (f.split("=") for f in fields)}
    return modes


def test_float32_tile_layout_in_use_is_consistent(report):
    n = report["current"]
    assert n["cases"] > 900 and n["stores"] > 0 and n["loads"] > 0
    assert n["bounds"] == n["dup"] == n["align"] == n["mismatch"] == n["uncovered"] == 0, n


def test_old_float64_tile_layout_was_in_bounds_and_consistent(report):
    n = report["old-double"]
    assert n["cases"] > 800
    assert n["bounds"] == n["dup"] == n["align"] == n["mismatch"] == n["uncovered"] == 0, n


def test_float32_layout_with_float64_rows_would_misassign_values(report):
    # the check detects a layout mismatch (in bounds, but the wrong (query, key) values)
    n = report["current-double"]
    assert n["bounds"] == 0 and n["mismatch"] > 0, n
