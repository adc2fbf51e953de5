"""Build the MI355X residual LayerNorm native code in-tree.

Produces, inside ``gfx1010_kernels/``:

* ``librln_gfx950.so`` - the HIP kernels for gfx950 and the C ABI declared in
  ``include/rln.h`` (hipcc, device code for gfx950 only);
* ``_C<EXT_SUFFIX>`` - the PyTorch glue module (g++, host code only), linked
  against ``librln_gfx950.so`` with an ``$ORIGIN`` run path;
and, outside the package, ``benchmarks/librln_probe_gfx950.so`` - the
streaming-probe kernels bench.py times beside the operator
(``benchmarks/rln_probe.hip``; not part of the operator).

Run ``python gfx1010-kernels_amd/build.py`` or call :func:`build`.
"""

from __future__ import annotations

import os
import shlex
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

ROOT = Path(__file__).resolve().parent
REPO = ROOT.parent
PACKAGE = ROOT / "gfx1010_kernels"
INCLUDE = REPO / "include"
CSRC = ROOT / "csrc"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = "gfx950"
LIBRARY = PACKAGE / f"librln_{ARCH}.so"
GLUE = PACKAGE / f"_C{sysconfig.get_config_var('EXT_SUFFIX')}"
PROBE_SOURCE = REPO / "benchmarks" / "rln_probe.hip"
PROBE = REPO / "benchmarks" / f"librln_probe_{ARCH}.so"

# Device-code flags. Packed fp32 instructions are disabled (the compiler may
# otherwise form v_pk_{add,mul,fma}_f32 from float code); FP contraction is
# off so that the bit-exact residual update is never fused into an FMA.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-ffp-contract=off",
    "-mcode-object-version=5",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
]

# One translation unit per row shape (every dtype and alignment variant of
# its kernels), plus the C ABI; compiled in parallel, linked into one library.
# Specialized hidden sizes, and the (slots per lane, waves per row) pairs of
# the run-time-length kernels that serve every other multiple of 64 up to
# 8192, per pass (the lists RLN_FOR_EACH_WIDE_FORWARD / _BACKWARD in
# rln_device.h; the link fails on a pair missing here). The backward of 1024
# columns runs the (1, 4) run-time-length kernel, that of large 768-column
# launches the (1, 3) one (backward_runs_wide), and that of large launches of
# 6657-8192 columns the (2, 16) one.
HIDDEN_SIZES = (128, 256, 384, 512, 768, 1024)
FIXED_BACKWARD = (128, 256, 384, 512, 768)
WIDE_FORWARD = ((1, 1), (2, 1), (3, 1), (4, 1), (3, 2), (4, 2), (3, 4), (4, 4), (3, 8), (4, 8))
WIDE_BACKWARD = ((1, 1), (2, 1), (3, 1), (1, 3), (1, 4), (3, 2), (2, 4), (3, 4), (2, 8), (3, 8),
                 (4, 8), (2, 16))
BUILD_DIR = ROOT / "_build"


def _run(command: list[str]) -> None:
    printable = " ".join(shlex.quote(part) for part in command)
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(
            f"build step failed ({result.returncode}): {printable}\n"
            f"{result.stdout}\n{result.stderr}"
        )


def _compile_object(source: Path, output: Path, defines: list[str]) -> Path:
    hipcc = str(ROCM / "bin" / "hipcc")
    _run([hipcc, *HIP_FLAGS, *defines, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(source),
          "-o", str(output)])
    return output


def build_library(jobs: int | None = None, defines: tuple[str, ...] = (),
                  output: Path = LIBRARY, build_dir: Path = BUILD_DIR) -> Path:
    """Compile the gfx950 kernels and C ABI into librln_gfx950.so (or, with
    extra -D `defines`, a variant build at `output`)."""
    build_dir.mkdir(parents=True, exist_ok=True)
    extra = [f"-D{define}" for define in defines]
    units = [(CSRC / "rln_api.hip", build_dir / "rln_api.o", extra)]
    units += [
        (CSRC / "rln_hidden.hip", build_dir / f"rln_hidden_{hidden}.o",
         [*extra, f"-DRLN_HIDDEN={hidden}",
          f"-DRLN_PASSES={1 | (hidden in FIXED_BACKWARD) << 1}"])
        for hidden in HIDDEN_SIZES
    ]
    units += [
        (CSRC / "rln_hidden.hip", build_dir / f"rln_wide_{v}x{p}.o",
         [*extra, f"-DRLN_WIDE_V={v}", f"-DRLN_WIDE_P={p}",
          f"-DRLN_PASSES={((v, p) in WIDE_FORWARD) | ((v, p) in WIDE_BACKWARD) << 1}"])
        for v, p in sorted(set(WIDE_FORWARD) | set(WIDE_BACKWARD))
    ]
    workers = jobs or min(len(units), max(1, (os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(lambda unit: _compile_object(*unit), units))
    hipcc = str(ROCM / "bin" / "hipcc")
    output.parent.mkdir(parents=True, exist_ok=True)
    temporary = output.with_name(output.name + ".tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects),
          f"-Wl,-soname,{output.name}", "-Wl,-z,defs", "-o", str(temporary)])
    os.replace(temporary, output)
    return output


VARIANTS = REPO / "benchmarks" / "variants"


def variant_path(name: str) -> Path:
    return VARIANTS / f"librln_{ARCH}_{name}.so"


def build_variant(name: str, defines: tuple[str, ...], jobs: int | None = None) -> Path:
    """A variant build of the library with compile-time switches (the RLN_*
    macros of rln_device.h) for the benchmark's A/B runs (bench.py --ab),
    at benchmarks/variants/librln_gfx950_<name>.so."""
    if not name.replace("_", "").replace("-", "").isalnum():
        raise ValueError(f"variant name {name!r}: letters, digits, '-' and '_' only")
    return build_library(jobs, defines, variant_path(name), BUILD_DIR / "variants" / name)


def build_probe() -> Path:
    """Compile the benchmark's streaming-probe kernels into their own library,
    beside their source (not in the package)."""
    hipcc = str(ROCM / "bin" / "hipcc")
    temporary = PROBE.with_name(PROBE.name + ".tmp")
    _run([hipcc, *HIP_FLAGS, "-shared", str(PROBE_SOURCE), f"-Wl,-soname,{PROBE.name}",
          "-Wl,-z,defs", "-o", str(temporary)])
    os.replace(temporary, PROBE)
    return PROBE


def _torch_paths() -> tuple[list[str], Path, bool]:
    import torch
    from torch.utils import cpp_extension

    return (
        cpp_extension.include_paths(),
        Path(torch.__file__).resolve().parent / "lib",
        bool(torch.compiled_with_cxx11_abi()),
    )


def build_glue() -> Path:
    """Compile the torch glue module linked against librln_gfx950.so."""
    includes, torch_lib, cxx11_abi = _torch_paths()
    python_include = sysconfig.get_paths()["include"]
    temporary = GLUE.with_name(GLUE.name + ".tmp")
    command = [
        "g++",
        "-O2",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-Wall",
        "-Wno-unused-function",
        "-D__HIP_PLATFORM_AMD__=1",
        "-DUSE_ROCM=1",
        "-DTORCH_API_INCLUDE_EXTENSION_H",
        "-DTORCH_EXTENSION_NAME=_C",
        f"-D_GLIBCXX_USE_CXX11_ABI={1 if cxx11_abi else 0}",
        f"-I{INCLUDE}",
        *[f"-I{path}" for path in includes],
        f"-I{python_include}",
        f"-I{ROCM / 'include'}",
        str(CSRC / "rln_torch.cpp"),
        f"-L{torch_lib}",
        f"-L{PACKAGE}",
        "-lc10",
        "-lc10_hip",
        "-ltorch",
        "-ltorch_cpu",
        "-ltorch_hip",
        "-ltorch_python",
        f"-l:{LIBRARY.name}",
        "-Wl,-rpath,$ORIGIN",
        "-o",
        str(temporary),
    ]
    _run(command)
    os.replace(temporary, GLUE)
    return GLUE


def build() -> tuple[Path, Path]:
    """Build both artefacts (the library first: the glue links against it)."""
    PACKAGE.mkdir(parents=True, exist_ok=True)
    library = build_library()
    glue = build_glue()
    build_probe()
    return library, glue


if __name__ == "__main__":
    for artefact in build():
        print(artefact.relative_to(REPO))
    sys.exit(0)
