"""bench.py's command-line contract that needs no GPU.

More than one GPU is not measured here (one MI355X per box): `--gpus N` with
N > 1 exits with status 2 and says why, before touching torch or the GPU.
"""

import subprocess
import sys
from pathlib import Path

BENCH = Path(__file__).resolve().parents[1] / "bench.py"


def test_more_than_one_gpu_is_refused_with_a_message():
    result = subprocess.run([sys.executable, str(BENCH), "--gpus", "2"], capture_output=True,
                            text=True, timeout=120)
    assert result.returncode == 2
    assert "single GPU" in result.stderr and "--gpus 2" in result.stderr
    assert result.stdout == ""


def test_help_lists_the_measurement_modes():
    result = subprocess.run([sys.executable, str(BENCH), "--help"], capture_output=True,
                            text=True, timeout=120)
    assert result.returncode == 0
    for flag in ("--steps", "--warmup", "--sweep", "--prenorm", "--reference-table"):
        assert flag in result.stdout
