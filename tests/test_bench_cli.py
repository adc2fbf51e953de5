"""bench.py's command-line contract that needs no GPU.

More than one GPU is not measured here (one MI355X per box): `--gpus N` with
N > 1 exits with status 2 and says why, before touching torch or the GPU.
"""

import subprocess
import sys
from pathlib import Path

import pytest


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
    for flag in ("--steps", "--warmup", "--sweep", "--prenorm", "--reference-table", "--config",
                 "--ceiling", "--quick", "--traffic-summary", "--char-gpt", "--alternation",
                 "--dwdb-placement", "--ab-rows"):
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
    size (one partial per block; 8-wave blocks hold 8 / parts rows, the
    12-wave blocks of four-wave rows of one or two slots at small launches
    12 / 4)."""
    import importlib.util

    from gfx1010_kernels import _cabi

    spec = importlib.util.spec_from_file_location("bench_under_test", BENCH)
    bench = importlib.util.module_from_spec(spec)
    sys.modules["bench_under_test"] = bench
    spec.loader.exec_module(bench)
    from dataclasses import replace

    for rows in (41, 8192, 8193):
        for hidden in range(128, 8193, 64):
            if hidden in bench.SPECIALIZED_HIDDEN and hidden != 1024:
                continue
            blocks = _cabi.backward_workspace_bytes(rows, hidden, True) // (2 * hidden * 4)
            parts = bench.wide_parts(hidden, "rln_backward_kernel", rows)
            name = bench.kernel_name("rln_backward_kernel",
                                     replace(bench.C1, hidden=hidden, rows=rows))
            waves = 12 if "StaggeredWideShape" in name or parts == 3 else 16 if parts == 16 else 8
            assert blocks == min(-(-rows // (waves // parts)), 256), (rows, hidden, name)


def _bench_module():
    import importlib.util

    spec = importlib.util.spec_from_file_location("bench_under_test", BENCH)
    bench = importlib.util.module_from_spec(spec)
    sys.modules["bench_under_test"] = bench
    spec.loader.exec_module(bench)
    return bench


def test_mask_decoding_matches_the_oracle_layout():
    """The parity self-check decodes the kernel's mask words on the device with
    bit c % 32 of word r * H / 32 + c / 32; it must agree with the oracle's
    decoder (pinned against the reference's layout in test_oracle.py)."""
    import numpy as np
    import torch

    from oracle import rln_oracle as oracle

    bench = _bench_module()
    rows, hidden = 5, 96
    words = np.random.default_rng(3).integers(0, 2 ** 32, rows * hidden // 32, dtype=np.uint64)
    words = words.astype(np.uint32)
    keep = bench.decode_mask(torch, torch.from_numpy(words.view(np.int32)), rows, hidden)
    assert np.array_equal(keep.numpy(), oracle.decode_mask(words, rows, hidden).astype(bool))


# The two C1 kernels as rocprofv3's counter csv names them (mangled).
MANGLED_BACKWARD = ("_ZN3rln19rln_backward_kernelINS_15TwelveWaveShapeILi768EEEDF16_fLb1EEEvPKfPKT1_"
                    "S4_S4_S4_S4_PKjPfPT0_SA_SA_SA_lT_ifii")
MANGLED_FORWARD = ("_ZN3rln18rln_forward_kernelINS_10FixedShapeILi768ELi64EEEDF16_fLb1ELb1EEEvPKfPKT0_"
                   "S4_S4_PfPT1_S8_S8_PjS8_S8_lT_fifjNS_10PhiloxArgsEii")


def test_traffic_summary_scales_counters_and_stamps_the_sources(tmp_path, monkeypatch):
    """--traffic-summary turns two rocprofv3 --pmc csv directories into the
    traffic record: kernel rows matched by their mangled names, each counter scaled by its value for the 256 MiB calibration copy (the
    largest copyBuffer dispatch, among the runtime's small ones); the record
    carries the kernel-source digest, and a record with another digest is
    reported stale instead of used."""
    import json

    bench = _bench_module()
    rows = {"FETCH_SIZE": [("__amd_rocclr_copyBuffer", 131072.0), ("__amd_rocclr_copyBuffer", 1.5),
                           (MANGLED_BACKWARD, 37000.0), (MANGLED_FORWARD, 18500.0)],
            "WRITE_SIZE": [("__amd_rocclr_copyBuffer", 262144.0), ("__amd_rocclr_copyBuffer", 3.0),
                           (MANGLED_BACKWARD, 38000.0), (MANGLED_FORWARD, 50000.0)]}
    for counter, values in rows.items():
        directory = tmp_path / counter / "host"
        directory.mkdir(parents=True)
        lines = ["Kernel_Name,Counter_Name,Counter_Value"]
        for name, value in values:
            jitters = (0.0,) if name.startswith("__") else (-1.0, 1.0)
            for jitter in jitters:
                lines.append(f'"{name}",{counter},{value + jitter}')
        (directory / "1_counter_collection.csv").write_text("\n".join(lines) + "\n")
    target = tmp_path / "traffic.json"
    monkeypatch.setattr(bench, "TRAFFIC_FILE", target)
    assert bench.traffic_summary(str(tmp_path / "FETCH_SIZE"), str(tmp_path / "WRITE_SIZE")) == 0
    record = json.loads(target.read_text())
    assert record["fetch_scale"] == 2.0 and record["write_scale"] == 1.0
    assert record["hbm_bytes_per_launch"] == 1024 * (37000 * 2 + 38000)
    assert record["forward_hbm_bytes_per_launch"] == 1024 * (18500 * 2 + 50000)
    assert record["sources_digest"] == bench.kernel_sources_digest()
    traffic, note = bench.load_traffic()
    assert traffic == record["hbm_bytes_per_launch"] and "commit" in note
    record["sources_digest"] = "0" * 16
    target.write_text(json.dumps(record))
    traffic, note = bench.load_traffic()
    assert traffic is None and note.startswith("stale")


def test_mangled_kernel_names_are_the_library_symbols():
    """mangled_kernel_name() gives the prefix rocprofv3 prints for the C1
    kernels, and, where the built library and llvm-readelf are at hand, every
    kernel bench.py names for its workloads is a symbol of the library."""
    bench = _bench_module()
    for kernel, mangled in (("rln_backward_kernel", MANGLED_BACKWARD),
                            ("rln_forward_kernel", MANGLED_FORWARD)):
        prefix = bench.mangled_kernel_name(bench.kernel_name(kernel, bench.C1))
        assert mangled.startswith(prefix) and mangled[len(prefix):].startswith("vPK")
    readelf = Path("/opt/rocm/llvm/bin/llvm-readelf")
    library = BENCH.parent / "gfx1010-kernels_amd" / "gfx1010_kernels" / "librln_gfx950.so"
    if not (readelf.exists() and library.exists()):
        return
    symbols = subprocess.run([str(readelf), "-s", "--wide", str(library)], capture_output=True,
                             text=True, check=True).stdout
    for workload in [bench.C1, *bench.sweep_workloads()]:
        kernels = ["rln_forward_kernel"] + (["rln_backward_kernel"] if workload.backward else [])
        for kernel in kernels:
            prefix = bench.mangled_kernel_name(bench.kernel_name(kernel, workload))
            assert prefix in symbols, (workload.describe(), kernel, prefix)


def test_ab_row_workloads_are_c1_shaped():
    """bench.py --ab-rows re-measures row-count-dependent launch rules on
    C1-shaped workloads: C1's branch, dropout and seed at other row counts."""
    import argparse

    bench = _bench_module()
    args = argparse.Namespace(ab_rows="2048, 8192", ab_hidden=768, ab_bf16=True)
    workloads = bench.ab_row_workloads(args)
    assert [w.name for w in workloads] == ["[2048,768]", "[8192,768]", "[2048,768] bf16-out",
                                           "[8192,768] bf16-out"]
    assert [w.rows for w in workloads] == [2048, 8192, 2048, 8192]
    for workload in workloads[:2]:
        assert (workload.branch, workload.normalized) == (bench.C1.branch, bench.C1.normalized)
        assert (workload.dropout_p, workload.seed, workload.hidden) == (0.1, bench.C1.seed, 768)
    for workload in workloads[2:]:
        assert (workload.branch, workload.normalized) == ("bf16", "bf16")
    assert bench.ab_row_workloads(argparse.Namespace(ab_rows="", ab_hidden=768,
                                                     ab_bf16=False)) == []
    with pytest.raises(SystemExit):
        bench.ab_row_workloads(argparse.Namespace(ab_rows="0", ab_hidden=768, ab_bf16=False))


def test_dwdb_placement_distances_cover_the_32k_period():
    """--dwdb-placement walks grad_bias over every KiB of four 32 KiB periods
    (from 3 KiB, past C1's 3 KiB arrays) and then coarser distances."""
    bench = _bench_module()
    offsets = bench.DWDB_OFFSETS
    assert list(offsets) == sorted(set(offsets))
    assert offsets[0] == 3 * 1024 and 4 * 768 <= offsets[0]
    assert all(k * 1024 in offsets for k in range(3, 129))
    assert offsets[-1] == 4 << 20
