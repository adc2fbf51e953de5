"""The C ABI's argument validation under the host sanitizers (CPU only).

tests/sanitize/ builds the host code of the C ABI (gfx1010-kernels_amd/csrc/
rln_api.hip: the checks that replace the reference's TORCH_CHECKs,
csrc/residual_layer_norm_kernel.hip:26-166) with AddressSanitizer and
UndefinedBehaviorSanitizer and runs a plain C driver that makes every
entry point reject bad arguments (null pointers, bad dtypes, sizes that
overflow, bad dropout probabilities and Philox settings, small workspaces)
and asks every size and metadata query. Nothing reaches a device, so it
runs without a GPU; any sanitizer report fails the run.
"""

import os
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent / "sanitize"
OBJECTS = HERE.parents[1] / "gfx1010-kernels_amd" / "_build"


def test_validation_paths_run_clean_under_host_sanitizers():
    if not list(OBJECTS.glob("rln_hidden_*.o")):
        pytest.skip("library objects not built (gfx1010-kernels_amd/build.py)")
    build = subprocess.run(["make", "-s", "-C", str(HERE)], capture_output=True, text=True,
                           timeout=900)
    assert build.returncode == 0, build.stdout + build.stderr
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", HIP_VISIBLE_DEVICES="")
    run = subprocess.run([str(HERE / "rln_validate")], capture_output=True, text=True,
                         timeout=300, env=env)
    assert run.returncode == 0, run.stdout + run.stderr
    assert run.stdout.strip().splitlines()[-1] == "ok", run.stdout + run.stderr
