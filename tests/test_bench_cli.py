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
    for flag in ("--steps", "--warmup", "--sweep", "--prenorm", "--reference-table", "--config"):
        assert flag in result.stdout


def test_unknown_config_is_refused_with_the_list_of_names():
    result = subprocess.run([sys.executable, str(BENCH), "--config", "C9"], capture_output=True,
                            text=True, timeout=120)
    assert result.returncode == 2
    assert "unknown --config ['C9']" in result.stderr
    for name in ("C0", "C2 H=1024", "C3", "W H=1600"):
        assert f"'{name}'" in result.stderr
    assert result.stdout == ""


def test_kernel_names_follow_the_library_backward_shapes():
    """bench.py labels the dominant kernel with the shape the library runs;
    the backward's waves per row are visible through the C ABI's workspace
    size (one partial per block; 8-wave blocks hold 8 / parts rows)."""
    import importlib.util

    from gfx1010_kernels import _cabi

    spec = importlib.util.spec_from_file_location("bench_under_test", BENCH)
    bench = importlib.util.module_from_spec(spec)
    sys.modules["bench_under_test"] = bench
    spec.loader.exec_module(bench)
    rows = 41
    for hidden in range(128, 8193, 64):
        if hidden in bench.SPECIALIZED_HIDDEN and hidden != 1024:
            continue
        blocks = _cabi.backward_workspace_bytes(rows, hidden, True) // (2 * hidden * 4)
        parts = bench.wide_parts(hidden, "rln_backward_kernel")
        assert blocks == -(-rows // (8 // parts)), hidden
