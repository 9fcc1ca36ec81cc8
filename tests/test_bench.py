"""bench.py's contract where no GPU is needed: one GPU only, and the roofline's traffic figure read from the
committed rocprofv3 summary (the FETCH_SIZE / WRITE_SIZE table of the headline kernel, scaled by the calibration
copy) agreeing with the table's own rows."""
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    run = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                         text=True, timeout=120, cwd=ROOT)
    assert run.returncode == 2
    assert "one GPU" in run.stderr and run.stdout == ""


def test_traffic_figure_is_the_table_average():
    sys.path.insert(0, ROOT)
    try:
        import bench
    finally:
        sys.path.remove(ROOT)
    figure = bench.traffic_per_launch()
    assert figure is not None
    text = open(os.path.join(ROOT, "profiles", "gemv_q8r_8b_decode_traffic.md")).read()
    # the phases' scaled bytes a launch, each phase 32 launches a step but the lm-head's one (129 a step)
    rows = re.findall(r"^\| (q/k/v|o|gate\+up|down|lm-head) \| .*\| (\d+) \|$", text, re.M)
    assert [r[0] for r in rows] == ["q/k/v", "o", "gate+up", "down", "lm-head"]
    step = sum((1 if name == "lm-head" else 32) * int(b) for name, b in rows)
    assert figure == pytest.approx(step / 129, abs=1.0)
    # and the rows are the FETCH_SIZE / WRITE_SIZE columns scaled by the stated factors (2 and 1)
    for line in re.findall(r"^\| (?:q/k/v|o|gate\+up|down|lm-head) \|.*$", text, re.M):
        cells = [c.strip() for c in line.strip("|").split("|")]
        fetch, write, scaled = float(cells[3]), float(cells[4]), int(cells[5])
        assert scaled == pytest.approx(1024 * (2.0 * fetch + write), rel=2e-4)
