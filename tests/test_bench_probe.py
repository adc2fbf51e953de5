"""The benchmark's streaming probe (benchmarks/rln_probe.hip): its variant
table and argument checks, without a GPU.

The probe gives every configuration bench.py measures a floor: the fastest
of its variants moving exactly that configuration's streams. So every
workload of the sweep that the probe applies to must find forward (and,
with a backward, backward) variants of its stream configuration, and a
launch must refuse NULL buffers its pass uses before touching the GPU.
"""

import ctypes
import importlib.util
import sys
from pathlib import Path

import pytest

BENCH = Path(__file__).resolve().parents[1] / "bench.py"


def _bench():
    spec = importlib.util.spec_from_file_location("bench_probe_under_test", BENCH)
    bench = importlib.util.module_from_spec(spec)
    sys.modules["bench_probe_under_test"] = bench
    spec.loader.exec_module(bench)
    return bench


def _library(bench):
    if not bench.PROBE_LIBRARY.exists():
        pytest.skip("benchmarks/librln_probe_gfx950.so is not built")
    return bench.probe_library()


def test_stream_configurations_of_the_sweep():
    bench = _bench()
    by_name = {w.name: w for w in bench.sweep_workloads()}
    assert bench.probe_config(bench.C1) == 0
    assert bench.probe_config(by_name["C0"]) == 5  # fp32 branch, eval: no mask
    assert bench.probe_config(by_name["C4 tail p=0.0"]) == 5
    assert bench.probe_config(by_name["C4 tail p=0.1"]) == 1
    assert bench.probe_config(by_name["C1 bf16-out"]) == 2
    assert bench.probe_config(by_name["C2 H=768 bf16-out"]) == 2
    # Every sweep workload has a floor, except launches past 2^31 bytes per
    # fp32 tensor (the probe's 32-bit offsets).
    for workload in bench.sweep_workloads():
        fits = workload.rows * workload.hidden * 4 <= 1 << 31
        assert bench.probe_applies(workload) == fits, workload.name


def test_every_configuration_has_both_passes():
    bench = _bench()
    library = _library(bench)
    kinds = {}
    for index in range(library.rln_probe_variant_count()):
        config = library.rln_probe_variant_config(index)
        kind = library.rln_probe_variant_kind(index)
        name = library.rln_probe_variant_name(index).decode()
        assert kind in (0, 1, 2)
        if kind == 2:
            continue
        assert config in bench.PROBE_CONFIGS, name
        assert name.startswith(("fwd " if kind == 0 else "bwd ")), name
        assert (" b32" in name) == bool(config & 1) and (" n16" in name) == bool(config & 2)
        assert (" nomask" in name) == bool(config & 4)
        kinds.setdefault(config, set()).add(kind)
    assert kinds == {config: {0, 1} for config in bench.PROBE_CONFIGS}
    assert library.rln_probe_variant_config(-1) == -1
    assert library.rln_probe_variant_config(library.rln_probe_variant_count()) == -1


def test_launch_refuses_missing_buffers_without_launching():
    bench = _bench()
    library = _library(bench)
    count = library.rln_probe_variant_count()
    forward = next(i for i in range(count) if library.rln_probe_variant_kind(i) == 0
                   and library.rln_probe_variant_config(i) == 0)
    backward = next(i for i in range(count) if library.rln_probe_variant_kind(i) == 1
                    and library.rln_probe_variant_config(i) == 5)
    fake = 0x1000  # never dereferenced: every call below returns before a launch
    rows, hidden = ctypes.c_int64(64), ctypes.c_int64(768)
    blocks = ctypes.c_int64(1)

    def launch(index, pointers):
        array = (ctypes.c_void_p * 15)(*pointers)
        return library.rln_probe_launch(index, array, rows, hidden, blocks, None)

    # The forward's buffers 0-6; its mask (4) is required with a mask.
    pointers = [fake] * 7 + [None] * 8
    pointers[4] = None
    assert launch(forward, pointers) == 1
    # The backward's buffers 7-14; a configuration without a mask needs no
    # mask (10), but every other buffer.
    pointers = [None] * 7 + [fake] * 8
    pointers[13] = None
    assert launch(backward, pointers) == 1
    # Bad shapes.
    assert library.rln_probe_launch(forward, (ctypes.c_void_p * 15)(*([fake] * 15)),
                                    ctypes.c_int64(64), ctypes.c_int64(100), blocks, None) == 1
    assert library.rln_probe_launch(-1, (ctypes.c_void_p * 15)(*([fake] * 15)), rows, hidden,
                                    blocks, None) == 1


def test_alternation_study_names_existing_probe_passes():
    """bench.py --alternation pairs the op with two probe variants by name;
    both must be variants of the headline stream configuration."""
    bench = _bench()
    library = _library(bench)
    by_name = {library.rln_probe_variant_name(i).decode(): i
               for i in range(library.rln_probe_variant_count())}
    for (name, blocks), kind in zip(bench.ALTERNATION_PROBES, (0, 1)):
        assert name in by_name, name
        assert library.rln_probe_variant_kind(by_name[name]) == kind
        assert library.rln_probe_variant_config(by_name[name]) == 0
        assert blocks > 0
