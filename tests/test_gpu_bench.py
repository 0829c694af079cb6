"""bench.py end to end at the driver's short settings: the run must emit one
parsed JSON line whose batch-0 parity check and row-status check passed,
whatever the number of steps (a short run writes only some rotated sets)."""
import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.gpu
@pytest.mark.parametrize("steps,warmup", [(1, 1), (20, 5)])
def test_bench_short_run_emits_line(steps, warmup):
    out = subprocess.run(
        [sys.executable, str(ROOT / "bench.py"), "--steps", str(steps), "--warmup", str(warmup),
         "--cpu-seconds", "0.5", "--set-gb", "0.5"],
        capture_output=True, text=True, timeout=300, check=True)
    line = json.loads(out.stdout.strip().splitlines()[-1])
    assert line["steps"] == steps and line["n_gpus"] == 1
    assert line["parity"].startswith("64/64")
    assert line["roofline"]["frac"] > 0 and line["cpu_baseline"]["cores"] >= 1
