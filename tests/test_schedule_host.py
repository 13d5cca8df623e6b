"""Row schedules of the TP kernels, checked on the host.

The persistent forward and backward kernels (o2mi_tp.hpp ``row_schedule``)
give each block a fixed set of row chunks, in forward or reverse order.  This
compiles ``tests/native/schedule_check.cpp`` against the kernel header and runs
it: every row must be visited exactly once, and every iteration a kernel may
address -- including the next-row prefetch of the iteration after the last --
must either lie inside [0, n_rows) or cover no rows (a reverse schedule whose
prefetch started before row 0 once read past the start of the inputs).
"""
import shutil
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]


def _hipcc():
    for candidate in ("/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and Path(candidate).exists():
            return candidate
    return None


def test_row_schedules_cover_rows_once_and_stay_in_bounds(tmp_path):
    hipcc = _hipcc()
    if hipcc is None:
        pytest.skip("hipcc not available")
    exe = tmp_path / "schedule_check"
    subprocess.run([hipcc, "-std=c++20", "-O1", f"-I{REPO / 'ictc-o2-hp_amd' / 'csrc'}",
                    str(REPO / "tests" / "native" / "schedule_check.cpp"), "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    proc = subprocess.run([str(exe)], capture_output=True, text=True)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert proc.stdout.strip().endswith(", 0 bad")


def test_per_row_weight_mapping_covers_every_edge_and_channel_once(tmp_path):
    """The per-row-weight streamed kernels (V = 1) put a block's wave pairs on
    shared 16-edge groups and deal each group's 32-channel tiles round-robin
    (``row_wave``), over a grid from ``row_grid``.  Compiled against those
    headers, ``tests/native/row_mapping_check.cpp`` checks over many (edges,
    channels, channel span) that every (edge, channel) belongs to exactly one
    wave and every 16-channel range stays inside its block's span."""
    hipcc = _hipcc()
    if hipcc is None:
        pytest.skip("hipcc not available")
    exe = tmp_path / "row_mapping_check"
    subprocess.run([hipcc, "-std=c++20", "-O1", f"-I{REPO / 'ictc-o2-hp_amd' / 'csrc'}",
                    str(REPO / "tests" / "native" / "row_mapping_check.cpp"), "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    proc = subprocess.run([str(exe)], capture_output=True, text=True)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert proc.stdout.strip().endswith(", 0 bad")
