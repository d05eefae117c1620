"""The attention kernels classify key blocks (SKIP / PARTIAL / FULL) per wave from closed-form bit
ranges; this builds the host check of tests/native/block_classes_check.hip, which compares them
with the per-block predicate on random spans and plans, and runs it on the CPU."""

import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


@pytest.mark.skipif(shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(),
                    reason="hipcc not available")
def test_closed_form_block_classes(tmp_path):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    exe = tmp_path / "block_classes_check"
    subprocess.run([hipcc, "--offload-arch=gfx950", "-O2", "-std=c++17", "-w",
                    str(HERE / "native" / "block_classes_check.hip"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe), "200000"], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.strip().endswith("bad 0")


@pytest.mark.skipif(shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(),
                    reason="hipcc not available")
def test_lane_intervals_are_monotone(tmp_path):
    # The kernels read a wave's span from four lanes (wave_span_monotone); this holds only while the
    # lanes' intervals never decrease along the lanes, which the host check verifies by brute force.
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    exe = tmp_path / "lane_spans_check"
    subprocess.run([hipcc, "--offload-arch=gfx950", "-O2", "-std=c++17", "-w",
                    str(HERE / "native" / "lane_spans_check.hip"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe), "400"], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.strip().endswith("bad 0")


@pytest.mark.skipif(shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(),
                    reason="hipcc not available")
def test_closed_form_tile_plans(tmp_path):
    # The row-layout prepass derives each tile's plan from the tile's first and last few rows
    # (q_tile_union / k_tile_union); the host check compares that with the union over every row.
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    exe = tmp_path / "tile_plan_check"
    subprocess.run([hipcc, "--offload-arch=gfx950", "-O2", "-std=c++17", "-w",
                    str(HERE / "native" / "tile_plan_check.hip"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe), "20000"], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.strip().endswith("bad 0")


@pytest.mark.skipif(shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(),
                    reason="hipcc not available")
def test_fast_division_and_slot_rotation(tmp_path):
    # The attention kernels map workgroups to (row, head, rank) with fast_div (multiply-high by a
    # launch-time reciprocal); the host check compares it with integer division, exhaustively for
    # small divisors and dividends and at random up to 2^31, and the slot rotation with its
    # definition (j + rank H) mod B H.
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    exe = tmp_path / "fast_div_check"
    subprocess.run([hipcc, "--offload-arch=gfx950", "-O2", "-std=c++17", "-w",
                    str(HERE / "native" / "fast_div_check.hip"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe), "20000"], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.strip().endswith("bad 0")
