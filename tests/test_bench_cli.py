"""CPU checks of bench.py's command line: it measures one GPU only and says so
for --gpus above 1, before importing torch or touching a device."""
import pathlib
import subprocess
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


@pytest.mark.parametrize("n", [2, 8])
def test_bench_refuses_several_gpus(n):
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", str(n), "--steps", "1", "--warmup", "0"],
                       capture_output=True, text=True, timeout=60, cwd=ROOT)
    assert r.returncode == 2
    assert r.stdout == ""
    assert "one GPU only" in r.stderr and f"--gpus {n}" in r.stderr
