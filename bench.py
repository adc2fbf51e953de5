#!/usr/bin/env python
"""Throughput of the fused residual + dropout + LayerNorm on one MI355X.

Workload (the north-star shape): x fp32 [8, 1024, 768]
~ N(0, 1), branch fp16 ~ N(0, 0.5), weight = 1 + 0.02 N(0, 1), bias = 0.02 N(0, 1),
dropout_p = 0.1, eps = 1e-5, upstream gradients fp32 ~ N(0, 1), atomic
weight/bias reduction. One step = the forward kernel plus the backward kernel
through the C ABI (librln_gfx950.so), with a fresh Philox offset each step and
the weight/bias gradients accumulated across steps (micro-batch gradient
accumulation; the atomic backward is then a single kernel).

Inputs are resident in HBM before the timed region. One input set moves about
200 MB, under MI355X's 256 MB Infinity Cache, so steps rotate through
``--sets`` independent copies (800 MB by default) and every step reads inputs
that were last touched three steps earlier.

Prints one JSON line:
  value        fwd+bwd algorithmic HBM bytes / wall time per step (GB/s), the
               step = forward then backward of the same batch, back to back
  roofline     dominant kernel (backward): algorithmic bytes / its average
               duration, from HIP events around a batch of back-to-back
               backward launches on the launch stream, against 8 TB/s
  cold_step    the same step with the backward lagging two batches behind,
               so that its saved forward state is no longer cache resident
  cpu_baseline the reference's CPU decomposition (F.dropout + add +
               F.layer_norm, forward + autograd) on this host's cores
  step_us_spread  p20 / median / p80 of the step time over batches of 25
  copy_ceiling    a plain device copy's GB/s at ~100 MB per launch
  ceiling_us   the measured streaming floor of this workload: the fastest of
               benchmarks/rln_probe.hip's streaming kernels (block size,
               bytes in flight per lane, look-ahead, 128-bit fp16, cache
               policy, LDS staging, grid) with the forward's and the
               backward's exact streams, timed like the op's kernels over
               the same buffers, and the op's times as a fraction of them
  parity       the timed C-ABI step (set 0, its Philox offset, weight/bias
               sums accumulated from zero) checked before timing against the
               PyTorch decomposition in float64 on this GPU, with the kernel's
               own dropout mask applied: updated bitwise, the rest normwise at
               the test suite's bars; a miss ends the run with status 1
  public_api      whole autograd steps through the public Python API on this
               GPU: these kernels (implementation="gfx950") and the
               reference's decomposition run by PyTorch-ROCm ("torch")
  reference_method  the reference's own published metric, speedup of the
               public call over the PyTorch decomposition on the same GPU
               (B = 1, H = 384), at T = 262144 where the GPU work dominates,
               beside the best ratios the reference publishes for gfx1010

The roofline kernel's average duration comes from a fixed 400 back-to-back
launches, whatever ``--steps`` is; those kernel timings run first, then the
``--warmup`` untimed steps, then exactly ``--steps`` timed steps. ``roofline.traffic`` is read from
profiles/rln_backward_c1_traffic.json only when that file's kernel-source
digest matches the sources in this tree (else null, with ``traffic_note``);
``--traffic-summary FETCH_DIR WRITE_DIR`` writes that file from two
``rocprofv3 --pmc FETCH_SIZE`` / ``WRITE_SIZE`` runs of ``bench.py --quick
--calibrate-copy-mib 256``. ``--quick`` runs the C1 line alone (no public-API,
reference-method, ceiling or CPU legs), for profiler passes.

``--sweep`` adds one JSON line per other BASELINE.json configuration (C0, the
C2 hidden-size sweep, C3 deterministic, the C4 cases), each with the same
fields for its own shape. ``--reference-table`` adds the reference's own
published measurement, run on this GPU: public-API forward and training-step
speedups over the PyTorch decomposition at B = 1, H = 384, T = 128 .. 4096,
beside the speedups the reference publishes for gfx1010. ``--config NAME``
(repeatable) runs only the named sweep configurations and skips the C1 line,
so that a profiler run sees one configuration's launches. ``--ceiling`` prints
every probe point of C1 (one ``probe_table`` line) and adds one line per
other configuration with the probe's streams (or the ``--config`` ones) with
the op's and the probe floor's times side by side.

Algorithmic bytes per row (H = hidden, bb = branch bytes, mask H/8 bytes when
dropping):
  forward  H * (4 + bb + 4 + 4) + 8 + H/8, plus 8H once (weight, bias)
  backward H * (4 + 4 + 4 + 4 + bb) + 8 + H/8, plus 12H once (weight; dW, db)
"""

from __future__ import annotations

import argparse
import ctypes
import hashlib
import json
import os
import platform
import statistics
import sys
import time
from dataclasses import dataclass, replace
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _path in (REPO, REPO / "gfx1010-kernels_amd"):
    if str(_path) not in sys.path:
        sys.path.insert(0, str(_path))

HBM_PEAK_GBPS = 8000.0
METRIC = "fwd & fwd+bwd achieved HBM GB/s (% of ~8 TB/s peak), rows/s at H=768"
EPS = 1e-5
TRAFFIC_FILE = REPO / "profiles" / "rln_backward_c1_traffic.json"
CSRC = REPO / "gfx1010-kernels_amd" / "csrc"
KERNEL_SOURCES = ("rln_device.h", "rln_api.hip", "rln_hidden.hip")
PROBE_LIBRARY = REPO / "benchmarks" / "librln_probe_gfx950.so"
# Back-to-back launches timed for the roofline kernel and the ceiling kernels.
ROOFLINE_LAUNCHES = 400


# The reference's threads per row (reference _normalization_native.py:5-12),
# which fix its dropout stream; the public API passes the same table.
REFERENCE_THREADS = {128: 128, 256: 128, 384: 128, 512: 128, 768: 128, 1024: 192}
DTYPE_BYTES = {"f32": 4, "f16": 2, "bf16": 2}
DTYPE_NAMES = {"f32": "float32", "f16": "float16", "bf16": "bfloat16"}


@dataclass(frozen=True)
class Workload:
    name: str
    rows: int
    hidden: int
    branch: str  # "f32", "f16" or "bf16"
    branch_std: float
    dropout_p: float
    training: bool = True
    backward: bool = True
    deterministic: bool = False
    x_mean: float = 0.0
    seed: int = 1001
    normalized: str = "f32"  # dtype of normalized and of its upstream gradient
    # Dropout stream layout (rln_philox_t.threads): None = what the public API
    # draws (the reference's hipRAND stream with its threads table on its
    # hidden sizes, else the library's own layout); 0 = the library's layout.
    threads: int | None = None

    @property
    def stream_threads(self) -> int:
        if self.threads is not None:
            return self.threads
        return REFERENCE_THREADS.get(self.hidden, 0)

    @property
    def branch_bytes(self) -> int:
        return DTYPE_BYTES[self.branch]

    @property
    def normalized_bytes(self) -> int:
        return DTYPE_BYTES[self.normalized]

    @property
    def dropping(self) -> bool:
        return self.training and self.dropout_p > 0.0

    def forward_bytes(self) -> int:
        mask = self.hidden // 8 if self.dropping else 0
        per_row = self.hidden * (4 + self.branch_bytes + 4 + self.normalized_bytes) + 8 + mask
        return self.rows * per_row + 8 * self.hidden

    def backward_bytes(self) -> int:
        if not self.backward:
            return 0
        mask = self.hidden // 8 if self.dropping else 0
        per_row = (self.hidden * (4 + self.normalized_bytes + 4 + 4 + self.branch_bytes)
                   + 8 + mask)
        return self.rows * per_row + 12 * self.hidden

    def describe(self) -> str:
        mode = "fwd+bwd" if self.backward else "fwd"
        reduction = "deterministic" if self.deterministic else "atomic"
        suffix = f", {reduction} dW/db" if self.backward else ""
        output = "" if self.normalized == "f32" else f", normalized {self.normalized}"
        stream = ""
        if self.dropping:
            stream = (f", reference hipRAND stream (threads={self.stream_threads})"
                      if self.stream_threads else ", library Philox layout")
        return (f"{self.name} {mode}: x fp32 [{self.rows},{self.hidden}], branch {self.branch}"
                f"{output}, dropout_p={self.dropout_p}, training={self.training}{stream}"
                f"{suffix}")


C1 = Workload("C1", 8 * 1024, 768, "f16", 0.5, 0.1, seed=1001)


def ab_row_workloads(args) -> list[Workload]:
    """C1-shaped workloads at the --ab-rows row counts: the row sweeps that
    decided row-count-dependent launch rules (the twelve- and nine-wave
    backwards of 768 and 384 columns) are re-measured through them."""
    rows = [int(value) for value in args.ab_rows.split(",") if value.strip()]
    if any(value <= 0 for value in rows) or args.ab_hidden <= 0:
        raise SystemExit("bench.py: --ab-rows and --ab-hidden take positive integers")
    workloads = [replace(C1, name=f"[{value},{args.ab_hidden}]", rows=value,
                         hidden=args.ab_hidden) for value in rows]
    if args.ab_bf16:
        workloads += [replace(workload, name=workload.name + " bf16-out", branch="bf16",
                              normalized="bf16") for workload in workloads]
    return workloads


def sweep_workloads() -> list[Workload]:
    """The other BASELINE.json configurations."""
    workloads = [Workload("C0", 4 * 1024, 768, "f32", 1.0, 0.0, training=False,
                          backward=False, seed=1000)]
    for hidden in (128, 256, 384, 512, 768, 1024):
        workloads.append(Workload(f"C2 H={hidden}", 262144, hidden, "f16", 1.0, 0.15,
                                  seed=1002 + hidden))
    workloads.append(Workload("C3", 32 * 2048, 1024, "f16", 0.5, 0.15, deterministic=True,
                              seed=1003))
    for dropout_p in (0.0, 0.1):
        workloads.append(Workload(f"C4 tail p={dropout_p}", 3 * 4097, 384, "f32", 1.0,
                                  dropout_p, x_mean=100.0, seed=1004))
    workloads.append(Workload("C4 large", 64 * 4096, 1024, "f16", 1.0, 0.1, seed=1006))
    # Half-precision interfaces (beyond the reference): bf16 branch, bf16
    # normalized output and upstream gradient, at the C1 and C2 H=768 shapes.
    workloads.append(Workload("C1 bf16-out", 8 * 1024, 768, "bf16", 0.5, 0.1, seed=1001,
                              normalized="bf16"))
    # The library's own Philox layout (a quarter fewer Philox blocks than the
    # reference's stream at H = 768, three quarters fewer at H = 128) at the
    # C1, C2 H=768 and C2 H=128 shapes.
    workloads.append(Workload("C1 own-stream", 8 * 1024, 768, "f16", 0.5, 0.1, seed=1001,
                              threads=0))
    workloads.append(Workload("C2 H=768 own-stream", 262144, 768, "f16", 1.0, 0.15,
                              seed=1002 + 768, threads=0))
    workloads.append(Workload("C2 H=128 own-stream", 262144, 128, "f16", 1.0, 0.15,
                              seed=1002 + 128, threads=0))
    workloads.append(Workload("C2 H=768 bf16-out", 262144, 768, "bf16", 1.0, 0.15,
                              seed=1770, normalized="bf16"))
    # Hidden sizes the reference does not serve natively (run-time row length,
    # several waves per row above 1024): GPT-2 XL's 1600 at the C1 batch, and
    # ~134 M-element sweeps like C2's.
    workloads.append(Workload("W H=1600 [8,1024]", 8 * 1024, 1600, "f16", 0.5, 0.1, seed=1600))
    for hidden in (640, 1280, 1600, 2048, 4096, 8192):
        workloads.append(Workload(f"W H={hidden}", (1 << 27) // hidden, hidden, "f16", 1.0, 0.15,
                                  seed=2000 + hidden))
    return workloads


def parse_args():
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=500)
    parser.add_argument("--warmup", type=int, default=50)
    parser.add_argument("--sets", type=int, default=4, help="rotated input sets")
    parser.add_argument("--cpu-seconds", type=float, default=15.0,
                        help="time budget of the CPU baseline sample")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--sweep", action="store_true",
                        help="also print one line per other BASELINE.json configuration")
    parser.add_argument("--calibrate-copy-mib", type=int, default=0,
                        help="also launch one device copy of this many MiB (PMC calibration)")
    parser.add_argument("--prenorm", action="store_true",
                        help="also time a pre-norm transformer stack, fused vs unfused")
    parser.add_argument("--char-gpt", action="store_true",
                        help="also time the reference's char-GPT AMP microstep (B=1, T=1024, "
                             "C=384, L=8), original vs fused normalization flow")
    parser.add_argument("--reference-table", action="store_true",
                        help="also print the reference's published speedup table, measured here")
    parser.add_argument("--reference-matrix", action="store_true",
                        help="also print the reference's end-to-end matrix (every native hidden "
                             "size, forward and train, fused vs torch) at B=1, T=1024/2048/4096")
    parser.add_argument("--ceiling", action="store_true",
                        help="add op-vs-streaming-ceiling lines per configuration")
    parser.add_argument("--alternation", action="store_true",
                        help="only time C1's forward and backward alternating with each other "
                             "and with the streaming probe's passes (one JSON line)")
    parser.add_argument("--dwdb-placement", action="store_true",
                        help="only time C1's backward with grad_weight and grad_bias placed "
                             "at a range of distances from each other (one JSON line)")
    parser.add_argument("--quick", action="store_true",
                        help="C1 line only (with --sweep or --config: those lines), kernels "
                             "launched only as the step launches them (no input-grads-only "
                             "backward, public-API, reference, ceiling or CPU legs): the "
                             "profiling runs")
    parser.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                        help="write profiles/rln_backward_c1_traffic.json from two rocprofv3 "
                             "--pmc output directories (no GPU needed)")
    parser.add_argument("--ab", action="append", default=[], metavar="NAME=DEFINES",
                        help="A/B run: also time a variant build of the library with the "
                             "comma-separated compile-time switches (e.g. "
                             "'nt=RLN_SMALL_STORE_POLICY=2'), built into benchmarks/variants/ if "
                             "missing, alternated round by round with the default build on C1 "
                             "(or the --config workloads); repeatable")
    parser.add_argument("--ab-rounds", type=int, default=5,
                        help="rounds of an A/B run (each times every build once)")
    parser.add_argument("--ab-build", action="store_true",
                        help="rebuild the --ab variants even where a build exists")
    parser.add_argument("--ab-rows", default="", metavar="ROWS[,ROWS...]",
                        help="A/B run on C1-shaped workloads (fp16 branch, p = 0.1) of these "
                             "row counts instead of C1, at --ab-hidden columns; with "
                             "--ab-bf16 also with a bf16 branch and output")
    parser.add_argument("--ab-hidden", type=int, default=768)
    parser.add_argument("--ab-bf16", action="store_true")
    parser.add_argument("--config", action="append", default=[], metavar="NAME",
                        help="run only this sweep configuration (repeatable; e.g. 'C2 H=1024'), "
                             "without the C1 line: one kernel's launches per run, for counters")
    return parser.parse_args()


# The reference's published speedups over its PyTorch decomposition on the
# RX 5600 XT (gfx1010): B = 1, H = 384, fp32 x, fp16 branch, p = 0.15, median
# of 1000 event-timed calls after 100 warmup calls (reference README.md:403-416).
REFERENCE_SPEEDUPS = {128: (1.273, 1.269), 256: (1.262, 1.265), 512: (1.303, 1.292),
                      1024: (1.242, 1.299), 2048: (1.792, 1.846), 4096: (1.839, 2.021)}
# Sequence lengths added on MI355X, where the reference's ones are host-bound
# (a call is done before its launch overhead): the same measurement where
# the GPU work dominates.
EXTRA_SEQUENCES = (16384, 65536, 262144)


def reference_table(torch, warmup: int = 100, reps: int = 1000,
                    sequences: tuple[int, ...] | None = None) -> list[dict]:
    """The reference's own headline measurement, on this GPU: the public
    forward and forward + backward (autograd.grad) call, fused native path
    against implementation="torch" (the decomposition), one CUDA-event pair
    around each call on the current stream, median / p20 / p80 of `reps`
    calls after `warmup` (as the reference's
    benchmarks/benchmark_residual_layer_norm.py:30-44, :213-264 measures).
    `sequences` picks some of the sequence lengths (default: all)."""
    from gfx1010_kernels import residual_layer_norm

    def timed(call):
        for _ in range(warmup):
            call()
        torch.cuda.synchronize()
        events = []
        for _ in range(reps):
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record()
            call()
            end.record()
            events.append((start, end))
        torch.cuda.synchronize()
        samples = sorted(start.elapsed_time(end) for start, end in events)
        pick = lambda fraction: samples[round(fraction * (len(samples) - 1))]  # noqa: E731
        return {"median_ms": round(pick(0.5), 5), "p20_ms": round(pick(0.2), 5),
                "p80_ms": round(pick(0.8), 5)}

    hidden, dropout_p = 384, 0.15
    lines = []
    cases = [*REFERENCE_SPEEDUPS.items(), *((sequence, (None, None)) for sequence in EXTRA_SEQUENCES)]
    if sequences is not None:
        cases = [case for case in cases if case[0] in sequences]
    for sequence, published in cases:
        generator = torch.Generator(device="cuda").manual_seed(sequence)
        shape = (1, sequence, hidden)
        inputs = (
            torch.randn(shape, device="cuda", generator=generator).requires_grad_(True),
            torch.randn(shape, device="cuda", generator=generator).half().requires_grad_(True),
            torch.randn(hidden, device="cuda", generator=generator).requires_grad_(True),
            torch.randn(hidden, device="cuda", generator=generator).requires_grad_(True),
        )
        grads = tuple(torch.randn(shape, device="cuda", generator=generator) for _ in range(2))
        line = {"kind": "reference_table", "B": 1, "T": sequence, "C": hidden,
                "dropout_p": dropout_p, "branch": "float16", "warmup": warmup, "reps": reps}
        for mode, index in (("forward", 0), ("train", 1)):
            results = {}
            for implementation in ("torch", "gfx950"):
                def call(implementation=implementation, mode=mode):
                    outputs = residual_layer_norm(*inputs, dropout_p=dropout_p, training=True,
                                                  implementation=implementation)
                    if mode == "train":
                        torch.autograd.grad(outputs, inputs, grads)

                results[implementation] = timed(call)
            line[mode] = {
                **results,
                "speedup": round(results["torch"]["median_ms"] / results["gfx950"]["median_ms"], 3),
                "reference_speedup_gfx1010": published[index],
            }
        lines.append(line)
    return lines


# The reference's matrix script: every native hidden size at one (B, T), its
# seed, branch dtype and dropout (benchmarks/benchmark_residual_layer_norm_matrix.py:
# 13-14, :135-152 defaults B = 1, T = 1024, p = 0.15, fp16 branch, 50 warmup
# and 500 timed calls).
MATRIX_HIDDEN = (128, 256, 384, 512, 768, 1024)
MATRIX_SEED = 29_072_026
MATRIX_SEQUENCES = (1024, 2048, 4096)


def reference_matrix(torch, batch: int = 1, sequences: tuple[int, ...] = MATRIX_SEQUENCES,
                     dropout_p: float = 0.15, warmup: int = 50, reps: int = 500) -> list[dict]:
    """The reference's end-to-end matrix on this GPU
    (benchmarks/benchmark_residual_layer_norm_matrix.py:52-227): for every
    hidden size, the public forward call and the forward + autograd.grad
    "train" call over fresh leaves, implementation="gfx950" against
    implementation="torch" on the same inputs (x, weight, bias fp32 and an
    fp16 branch from torch.randn after seeding SEED + hidden; upstream
    gradients randn_like), one CUDA-event pair around each call, median /
    p20 / p80 (linear quantiles, as its quantile()) of `reps` calls after
    `warmup`, and speedup = torch median / fused median. One line per
    (T, hidden, mode)."""
    from gfx1010_kernels import residual_layer_norm

    def quantile(values, fraction):
        ordered = sorted(values)
        position = (len(ordered) - 1) * fraction
        lower, upper = int(position // 1), -int(-position // 1)
        weight = position - lower
        return ordered[lower] * (1.0 - weight) + ordered[upper] * weight

    def timed(call, seed):
        torch.manual_seed(seed)
        for _ in range(warmup):
            call()
        torch.cuda.synchronize()
        torch.manual_seed(seed)
        events = []
        for _ in range(reps):
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record()
            call()
            end.record()
            events.append((start, end))
        torch.cuda.synchronize()
        samples = [start.elapsed_time(end) for start, end in events]
        return {"median_ms": round(quantile(samples, 0.5), 5),
                "p20_ms": round(quantile(samples, 0.2), 5),
                "p80_ms": round(quantile(samples, 0.8), 5)}

    lines = []
    for sequence in sequences:
        for hidden in MATRIX_HIDDEN:
            seed = MATRIX_SEED + hidden
            torch.manual_seed(seed)
            shape = (batch, sequence, hidden)
            source = (torch.randn(shape, device="cuda"),
                      torch.randn(shape, device="cuda", dtype=torch.float16),
                      torch.randn(hidden, device="cuda"), torch.randn(hidden, device="cuda"))
            grads = (torch.randn_like(source[0]), torch.randn_like(source[0]))
            for mode in ("forward", "train"):
                results = {}
                for implementation in ("torch", "gfx950"):
                    leaves = tuple(t.detach().clone().requires_grad_(True) for t in source)

                    def call(leaves=leaves, implementation=implementation, mode=mode):
                        outputs = residual_layer_norm(*leaves, dropout_p=dropout_p,
                                                      training=True,
                                                      implementation=implementation)
                        if mode == "train":
                            torch.autograd.grad(outputs, leaves, grads)

                    results[implementation] = timed(call, seed + (mode == "train"))
                lines.append({
                    "kind": "reference_matrix", "B": batch, "T": sequence, "C": hidden,
                    "mode": mode, "branch_dtype": "float16", "dropout_p": dropout_p,
                    "warmup": warmup, "reps": reps, **results,
                    "speedup": round(results["torch"]["median_ms"]
                                     / results["gfx950"]["median_ms"], 3)})
    return lines


def prenorm_stack(torch, stream, depth: int = 12, hidden: int = 768, tokens: int = 8192,
                  dropout_p: float = 0.1, steps: int = 20) -> dict:
    """A GPT-2-small-shaped pre-norm stack (12 blocks, H = 768, 8 x 1024 tokens;
    attention replaced by one H x H projection, MLP H -> 4H -> H with GELU;
    bf16 sublayers, fp32 residual stream and LayerNorm parameters), one
    training step = forward + backward of the whole stack. "unfused" runs
    `x = x + dropout(sublayer(ln(x)))` in PyTorch; "fused" runs
    prenorm_forward, every residual add fused into the LayerNorm after it
    (normalized output in bf16 for the sublayers)."""
    from torch import nn
    from torch.nn import functional as F

    from gfx1010_kernels import prenorm_forward

    torch.manual_seed(0)

    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.ln_1 = nn.LayerNorm(hidden)
            self.attn = nn.Linear(hidden, hidden, dtype=torch.bfloat16)
            self.ln_2 = nn.LayerNorm(hidden)
            self.mlp = nn.Sequential(nn.Linear(hidden, 4 * hidden, dtype=torch.bfloat16),
                                     nn.GELU(),
                                     nn.Linear(4 * hidden, hidden, dtype=torch.bfloat16))

    blocks = nn.ModuleList(Block() for _ in range(depth)).cuda()
    final = nn.LayerNorm(hidden).cuda()
    x = torch.randn(tokens, hidden, device="cuda", requires_grad=True)
    grad = torch.randn(tokens, hidden, device="cuda", dtype=torch.bfloat16)
    half = torch.bfloat16

    def unfused():
        h = x
        for block in blocks:
            h = h + F.dropout(block.attn(block.ln_1(h).to(half)).float(), dropout_p, True)
            h = h + F.dropout(block.mlp(block.ln_2(h).to(half)).float(), dropout_p, True)
        return final(h).to(half)

    def fused():
        _, out = prenorm_forward(x, blocks, final, dropout_p=dropout_p, training=True,
                                 implementation="gfx950", normalized_dtype=half)
        return out

    result = {}
    with torch.cuda.stream(stream):
        for name, forward in (("unfused", unfused), ("fused", fused)):
            def step():
                torch.autograd.backward(forward(), grad)

            for _ in range(3):
                step()
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            start.record(stream)
            for _ in range(steps):
                step()
            end.record(stream)
            end.synchronize()
            result[name] = {"ms_per_step": round(start.elapsed_time(end) / steps, 3)}
    result["speedup"] = round(result["unfused"]["ms_per_step"] / result["fused"]["ms_per_step"], 3)
    result["config"] = {"depth": depth, "hidden": hidden, "tokens": tokens,
                        "dropout_p": dropout_p, "sublayers": "bf16", "steps": steps}
    return result


def char_gpt_microstep(torch, stream, batch: int = 1, sequence: int = 1024, hidden: int = 384,
                       depth: int = 8, heads: int = 6, vocab: int = 65, dropout_p: float = 0.2,
                       warmup: int = 10, samples: int = 40) -> dict:
    """The reference's model-level measurement (docs/residual_layer_norm.md:
    380-385): a character-level GPT with B = 1, T = 1024, C = 384, L = 8, one
    complete AMP (fp16 autocast) forward + backward microstep, 10 warmups and
    40 event-timed samples, "original" normalization flow against the fused
    one. The model is nanoGPT-shaped (its shakespeare-char vocabulary of 65
    and dropout 0.2; the reference states neither): token + position
    embeddings with dropout, pre-norm blocks of causal self-attention (6
    heads, fused attention kernels only: a missing one raises rather than
    falling back to the math path) and a 4x GELU MLP, each with residual
    dropout, a final LayerNorm, an untied vocabulary projection and the
    cross-entropy loss. "original" runs `x = x + dropout(sublayer(ln(x)))`;
    "fused" runs prenorm_forward (every residual add + dropout fused into the
    LayerNorm after it, implementation="gfx950"). Weights are random, the
    tokens synthetic. Returns medians in milliseconds."""
    from torch import nn
    from torch.nn import functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    from gfx1010_kernels import prenorm_forward

    class Attention(nn.Module):
        def __init__(self):
            super().__init__()
            self.qkv = nn.Linear(hidden, 3 * hidden)
            self.proj = nn.Linear(hidden, hidden)

        def forward(self, h):
            b, t, c = h.shape
            q, k, v = self.qkv(h).split(hidden, dim=2)
            q, k, v = (z.view(b, t, heads, c // heads).transpose(1, 2) for z in (q, k, v))
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                y = F.scaled_dot_product_attention(q, k, v, is_causal=True)
            return self.proj(y.transpose(1, 2).reshape(b, t, c))

    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.ln_1 = nn.LayerNorm(hidden)
            self.attn = Attention()
            self.ln_2 = nn.LayerNorm(hidden)
            self.mlp = nn.Sequential(nn.Linear(hidden, 4 * hidden), nn.GELU(),
                                     nn.Linear(4 * hidden, hidden))

    class CharGPT(nn.Module):
        def __init__(self):
            super().__init__()
            self.tokens = nn.Embedding(vocab, hidden)
            self.positions = nn.Embedding(sequence, hidden)
            self.h = nn.ModuleList(Block() for _ in range(depth))
            self.ln_f = nn.LayerNorm(hidden)
            self.head = nn.Linear(hidden, vocab, bias=False)

        def forward(self, index, fused):
            positions = torch.arange(sequence, device=index.device)
            x = F.dropout(self.tokens(index) + self.positions(positions), dropout_p, True)
            if fused:
                _, out = prenorm_forward(x, self.h, self.ln_f, dropout_p=dropout_p, training=True,
                                         implementation="gfx950")
            else:
                for block in self.h:
                    x = x + F.dropout(block.attn(block.ln_1(x)), dropout_p, True)
                    x = x + F.dropout(block.mlp(block.ln_2(x)), dropout_p, True)
                out = self.ln_f(x)
            return self.head(out)

    torch.manual_seed(0)
    model = CharGPT().cuda()
    generator = torch.Generator(device="cuda").manual_seed(1)
    index = torch.randint(0, vocab, (batch, sequence), device="cuda", generator=generator)
    targets = torch.randint(0, vocab, (batch, sequence), device="cuda", generator=generator)

    def microstep(fused):
        with torch.autocast(device_type="cuda", dtype=torch.float16):
            logits = model(index, fused)
            loss = F.cross_entropy(logits.view(-1, vocab).float(), targets.view(-1))
        loss.backward()

    result = {}
    with torch.cuda.stream(stream):
        for name, fused in (("original", False), ("fused", True)):
            times = []
            for sample in range(warmup + samples):
                model.zero_grad(set_to_none=True)
                start = torch.cuda.Event(enable_timing=True)
                end = torch.cuda.Event(enable_timing=True)
                start.record(stream)
                microstep(fused)
                end.record(stream)
                end.synchronize()
                if sample >= warmup:
                    times.append(start.elapsed_time(end))
            result[name] = {"median_ms": round(statistics.median(times), 4),
                            "p20_ms": round(sorted(times)[len(times) // 5], 4),
                            "p80_ms": round(sorted(times)[(4 * len(times)) // 5], 4)}
    result["speedup"] = round(result["original"]["median_ms"] / result["fused"]["median_ms"], 4)
    result["config"] = {"batch": batch, "sequence": sequence, "hidden": hidden, "depth": depth,
                        "heads": heads, "vocab": vocab, "dropout_p": dropout_p, "amp": "fp16",
                        "warmup": warmup, "samples": samples}
    result["reference_published"] = {"original_ms": 150.119, "fused_ms": 148.946,
                                     "speedup": 1.008, "gpu": "gfx1010 (RX 5600 XT)"}
    return result


GRAPH_STEPS = (1, 8, 32)
PUBLIC_API_SETS = 4


def public_api_steps(torch, workload: Workload, stream, steps: int = 96) -> dict:
    """Whole autograd steps through the public API on this GPU, as a user runs
    them: `implementation="gfx950"` (these kernels) and
    `implementation="torch"` (the reference's decomposition, F.dropout + add +
    F.layer_norm, run by PyTorch-ROCm on the same GPU), over 4 input sets
    rotated from step to step. `eager` includes Python dispatch, autograd and
    allocation per step; `host_us` is the CPU
    time to issue one eager forward and one eager step (perf_counter over
    `steps` calls, no synchronization inside: when it exceeds the GPU's time
    the eager step is host-bound), `forward_no_grad` that of one forward
    under torch.no_grad() (an inference call, which records no graph; for the
    fused path also `forward_no_grad_auto`, the same call with
    implementation="auto"), and `engine_floor` that of
    torch.autograd.grad over one elementwise op (x * 2), PyTorch's own floor
    for a step with a CUDA backward; `graph_steps` replays HIP graphs holding 1,
    8 and 32 consecutive steps (the op draws a fresh dropout mask on every
    replay of every step), per step; `graph` is the one-step graph."""
    from gfx1010_kernels import residual_layer_norm

    generator = torch.Generator(device="cuda").manual_seed(workload.seed)
    shape = (workload.rows, workload.hidden)
    branch_type = getattr(torch, DTYPE_NAMES[workload.branch])
    weight = (1.0 + 0.02 * torch.randn(workload.hidden, device="cuda",
                                       generator=generator)).requires_grad_(True)
    bias = (0.02 * torch.randn(workload.hidden, device="cuda",
                               generator=generator)).requires_grad_(True)
    # Input sets rotated from step to step, as in the C-ABI timing: each
    # step's inputs and upstream gradients are other tensors than the last's.
    sets = []
    for _ in range(PUBLIC_API_SETS):
        x = torch.randn(shape, device="cuda", generator=generator).requires_grad_(True)
        branch = (workload.branch_std * torch.randn(shape, device="cuda", generator=generator)).to(
            branch_type).requires_grad_(True)
        grads = [torch.randn(shape, device="cuda", generator=generator) for _ in range(2)]
        sets.append(((x, branch, weight, bias), grads))
    total = workload.forward_bytes() + workload.backward_bytes()
    counter = [0]

    def next_set():
        counter[0] += 1
        return sets[counter[0] % len(sets)]

    def timed(body, calls, steps_per_call=1):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record(stream)
        for _ in range(calls):
            body()
        end.record(stream)
        end.synchronize()
        ms = start.elapsed_time(end) / (calls * steps_per_call)
        return {"us_per_step": round(ms * 1e3, 3), "gbps": round(total / (ms * 1e-3) / 1e9, 1)}

    def host_us(body, calls):
        torch.cuda.synchronize()
        began = time.perf_counter()
        for _ in range(calls):
            body()
        issued = time.perf_counter() - began
        torch.cuda.synchronize()
        return round(issued * 1e6 / calls, 2)

    result = {}
    with torch.cuda.stream(stream):
        for implementation in ("gfx950", "torch"):
            def forward(leaves=None):
                x, branch, weight_, bias_ = leaves or next_set()[0]
                return residual_layer_norm(
                    x, branch, weight_, bias_, dropout_p=workload.dropout_p, eps=EPS,
                    training=workload.training, implementation=implementation)

            def step():
                leaves, grads = next_set()
                return torch.autograd.grad(forward(leaves), leaves, grads)

            def engine_floor():
                # One elementwise CUDA node through the same autograd engine.
                (x, *_), grads = next_set()
                return torch.autograd.grad((x * 2.0,), (x,), (grads[0],))

            def forward_auto():
                x, branch, weight_, bias_ = next_set()[0]
                return residual_layer_norm(
                    x, branch, weight_, bias_, dropout_p=workload.dropout_p, eps=EPS,
                    training=workload.training)

            for _ in range(10):
                step()
            entry = {"eager": timed(step, steps),
                     "host_us": {"forward": host_us(forward, steps), "step": host_us(step, steps),
                                 "engine_floor": host_us(engine_floor, steps)}}
            with torch.no_grad():
                entry["host_us"]["forward_no_grad"] = host_us(forward, steps)
                if implementation == "gfx950":
                    entry["host_us"]["forward_no_grad_auto"] = host_us(forward_auto, steps)
            graph_steps = {}
            for count in GRAPH_STEPS:
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, stream=stream):
                    for _ in range(count):
                        step()
                graph.replay()
                graph_steps[str(count)] = timed(graph.replay, max(steps // count, 4), count)
                del graph
            entry["graph"] = graph_steps["1"]
            entry["graph_steps"] = graph_steps
            result[implementation] = entry
    result["kind"] = ("fwd+bwd through residual_layer_norm(..., implementation=...) and "
                      f"torch.autograd.grad, {steps} steps back to back, {PUBLIC_API_SETS} "
                      "input sets rotated")
    return result


def cpu_baseline(torch, workload: Workload, budget_seconds: float) -> dict:
    """The reference's CPU path on this host, on a bounded sample of steps
    (forward plus autograd backward; forward only for a forward workload)."""
    from oracle.torch_path import fwd_bwd_step, residual_layer_norm_torch

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    generator = torch.Generator().manual_seed(workload.seed)
    shape = (workload.rows, workload.hidden)
    x = torch.randn(shape, generator=generator).requires_grad_(True)
    branch = (workload.branch_std * torch.randn(shape, generator=generator))
    branch = branch.to(getattr(torch, DTYPE_NAMES[workload.branch])).requires_grad_(True)
    weight = (1.0 + 0.02 * torch.randn(workload.hidden, generator=generator)).requires_grad_(True)
    bias = (0.02 * torch.randn(workload.hidden, generator=generator)).requires_grad_(True)
    grad_updated = torch.randn(shape, generator=generator)
    grad_normalized = torch.randn(shape, generator=generator)
    if workload.backward:
        step = lambda: fwd_bwd_step(x, branch, weight, bias, grad_updated,  # noqa: E731
                                    grad_normalized, workload.dropout_p, EPS)
    else:
        def step():
            with torch.no_grad():
                residual_layer_norm_torch(x, branch, weight, bias, workload.dropout_p, EPS,
                                          workload.training)
    for _ in range(2):
        step()
    samples = []
    start = time.perf_counter()
    while len(samples) < 10 or (time.perf_counter() - start < budget_seconds and len(samples) < 1000):
        began = time.perf_counter()
        step()
        samples.append(time.perf_counter() - began)
    median = statistics.median(samples)
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    total = workload.forward_bytes() + workload.backward_bytes()
    return {
        "value": round(total / median / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"{len(samples)} {'fwd+bwd' if workload.backward else 'fwd'} steps of "
                   f"{workload.name} [{workload.rows},{workload.hidden}] (F.dropout + add + "
                   f"F.layer_norm{', autograd.grad' if workload.backward else ''}), "
                   f"median {median * 1e3:.2f} ms/step, torch {torch.__version__} on {model}"),
        "rows_per_s": round(workload.rows / median, 1),
        "ms_per_step": round(median * 1e3, 3),
    }


class Runner:
    """Device buffers for one workload and the C ABI launches over them."""

    def __init__(self, torch, library, cabi, workload: Workload, sets: int, stream):
        self.torch = torch
        self.library = library
        self.cabi = cabi
        self.w = workload
        self.stream = stream
        self.handle = stream.cuda_stream
        generator = torch.Generator().manual_seed(workload.seed)
        self.weight = (1.0 + 0.02 * torch.randn(workload.hidden, generator=generator)).cuda()
        self.bias = (0.02 * torch.randn(workload.hidden, generator=generator)).cuda()
        self.sets = [self._make_set(workload.seed + 17 * index) for index in range(sets)]
        self.workspace = None
        workspace_bytes = cabi.backward_workspace_bytes(
            workload.rows, workload.hidden, workload.deterministic)
        if workload.backward and workspace_bytes:
            self.workspace = torch.empty(workspace_bytes, device="cuda", dtype=torch.uint8)
        self.seed = 0x5EED_0000 + workload.seed
        self.increment = max(cabi.philox_increment(workload.hidden, workload.stream_threads), 4)

    def _make_set(self, seed: int) -> dict:
        torch, w = self.torch, self.w
        generator = torch.Generator(device="cuda").manual_seed(seed)
        shape = (w.rows, w.hidden)
        f32 = dict(device="cuda", dtype=torch.float32)
        branch = torch.randn(shape, generator=generator, **f32) * w.branch_std
        normalized_type = getattr(torch, DTYPE_NAMES[w.normalized])
        tensors = {
            "x": torch.randn(shape, generator=generator, **f32) + w.x_mean,
            "branch": branch.to(getattr(torch, DTYPE_NAMES[w.branch])),
            "updated": torch.empty(shape, **f32),
            "normalized": torch.empty(shape, device="cuda", dtype=normalized_type),
            "mean": torch.empty(w.rows, **f32),
            "rstd": torch.empty(w.rows, **f32),
            "mask": torch.empty(max(w.rows * w.hidden // 32, 1), device="cuda",
                                dtype=torch.int32),
        }
        if w.backward:
            tensors.update(
                grad_updated=torch.randn(shape, generator=generator, **f32),
                grad_normalized=torch.randn(shape, generator=generator, **f32).to(normalized_type),
                grad_x=torch.empty(shape, **f32),
                grad_branch=torch.empty(shape, device="cuda",
                                        dtype=getattr(torch, DTYPE_NAMES[w.branch])),
                grad_weight=torch.zeros(w.hidden, **f32),
                grad_bias=torch.zeros(w.hidden, **f32),
            )
        return tensors

    def code(self, name: str) -> int:
        return {"f32": self.cabi.RLN_DTYPE_F32, "f16": self.cabi.RLN_DTYPE_F16,
                "bf16": self.cabi.RLN_DTYPE_BF16}[name]

    def _launch_arguments(self):
        """Per set, the C-ABI argument tuples of its forward and backward,
        built once (ctypes-converted), so that a launch from the timing loops
        costs the host as little as the C call itself: the forward's ~9 us at
        C0 is shorter than building the arguments anew each time."""
        w, cabi = self.w, self.cabi
        p, i64, f64 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_double
        self._philox = cabi.RlnPhilox(self.seed, 0, None, None, w.stream_threads)
        philox = ctypes.byref(self._philox)
        handle = p(self.handle)
        workspace = self.workspace
        self._forward_args, self._backward_args = [], []
        for t in self.sets:
            self._forward_args.append((
                p(t["x"].data_ptr()), p(t["branch"].data_ptr()), self.code(w.branch),
                p(self.weight.data_ptr()), p(self.bias.data_ptr()), p(t["updated"].data_ptr()),
                p(t["normalized"].data_ptr()), self.code(w.normalized), p(t["mean"].data_ptr()),
                p(t["rstd"].data_ptr()), p(t["mask"].data_ptr()), None, None, i64(w.rows),
                i64(w.hidden), f64(w.dropout_p), f64(EPS), int(w.training), philox, handle))
            if w.backward:
                self._backward_args.append((
                    p(t["grad_updated"].data_ptr()), p(t["grad_normalized"].data_ptr()),
                    self.code(w.normalized), p(t["updated"].data_ptr()), p(self.weight.data_ptr()),
                    p(t["mean"].data_ptr()), p(t["rstd"].data_ptr()), p(t["mask"].data_ptr()),
                    p(t["grad_x"].data_ptr()), p(t["grad_branch"].data_ptr()), self.code(w.branch),
                    p(t["grad_weight"].data_ptr()), p(t["grad_bias"].data_ptr()), i64(w.rows),
                    i64(w.hidden), f64(w.dropout_p), int(w.training), int(w.deterministic), 1,
                    p(workspace.data_ptr()) if workspace is not None else None,
                    workspace.numel() if workspace is not None else 0, handle))
        # The same backwards with grad_weight and grad_bias (arguments 11 and
        # 12 of rln_backward) NULL.
        self._input_grad_args = [args[:11] + (None, None) + args[13:]
                                 for args in self._backward_args]

    def forward(self, step: int):
        """The forward of `step` (its set, its Philox offset) through rln_forward."""
        if not hasattr(self, "_forward_args"):
            self._launch_arguments()
        self._philox.offset = self.increment * step
        if self.library.rln_forward(*self._forward_args[step % len(self.sets)]):
            raise RuntimeError(self.cabi.last_error())

    def backward(self, step: int):
        """The backward of `step`'s set through rln_backward (weight/bias
        gradients accumulated into the set's sums)."""
        if not hasattr(self, "_forward_args"):
            self._launch_arguments()
        if self.library.rln_backward(*self._backward_args[step % len(self.sets)]):
            raise RuntimeError(self.cabi.last_error())

    def backward_input_grads(self, step: int):
        """The backward of `step`'s set with the weight/bias gradients not
        requested (both NULL): the input gradients alone, which shows what
        the parameter sums add to the backward."""
        if not hasattr(self, "_forward_args"):
            self._launch_arguments()
        if self.library.rln_backward(*self._input_grad_args[step % len(self.sets)]):
            raise RuntimeError(self.cabi.last_error())

    def step(self, index: int):
        self.forward(index)
        if self.w.backward:
            self.backward(index)

    def timed(self, body, count: int) -> float:
        """Milliseconds per iteration of `body` over `count` iterations, from
        HIP events recorded on the launch stream around the whole batch."""
        torch = self.torch
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record(self.stream)
        for index in range(count):
            body(index)
        end.record(self.stream)
        end.synchronize()
        return start.elapsed_time(end) / count

    def measure(self, warmup: int, steps: int, launches: int = ROOFLINE_LAUNCHES,
                input_grads: bool = True) -> dict:
        """Per-kernel averages (the roofline) over `launches` back-to-back
        launches of one kernel, whatever `steps` is; then `warmup` untimed
        steps and the step time over exactly `steps` timed steps (the
        contract's W and K), with the GPU already busy for the kernel timings
        before them; then the spread and the cold step. With `input_grads`,
        also the backward with dW/db not requested, over `launches`."""
        w = self.w
        # Untimed steps until the GPU has run about 25 ms of this work: its
        # clocks ramp up under load, and the first kernel timings after an
        # idle GPU came out ~4 % slow (C1 forward 17.7 against 17.0 us).
        first_ms = self.timed(lambda i: self.step(i), 2 * len(self.sets))
        base = 2 * len(self.sets)
        ramp = min(int(25.0 / max(first_ms, 1e-3)), 5000)
        for index in range(ramp):
            self.step(base + index)
        base += ramp
        forward_ms = self.timed(lambda i: self.forward(base + i), launches)
        base += launches
        result = {"forward_ms": forward_ms, "launches": launches}
        if w.backward:
            # Every set holds the saved state of a forward; re-running the
            # backward on it is the same work as the step's backward.
            result["backward_ms"] = self.timed(lambda i: self.backward(base + i), launches)
            base += launches
            if input_grads:
                result["backward_input_grads_ms"] = self.timed(
                    lambda i: self.backward_input_grads(base + i), launches)
                base += launches
        for index in range(warmup):
            self.step(base + index)
        base += warmup
        result["step_ms"] = self.timed(lambda i: self.step(base + i), steps)
        base += steps
        # Spread: the same steps timed in batches of 25 (p20 / median / p80
        # of the per-batch step time).
        batches = []
        for _ in range(max(steps // 25, 4)):
            batches.append(self.timed(lambda i: self.step(base + i), 25))
            base += 25
        result["step_batches_ms"] = batches
        if w.backward:
            # Backward on the set forwarded `lag` steps earlier (two, or one
            # when only two sets rotate).
            lag = min(2, len(self.sets) - 1)

            def cold(index):
                self.forward(base + index)
                self.backward(base + index - lag + len(self.sets))

            result["cold_ms"] = self.timed(cold, steps)
        return result


def copy_ceiling(torch, stream, mib: int = 50, copies: int = 200) -> dict:
    """A plain device copy (torch copy_) of `mib` MiB, four buffer pairs in
    rotation (400 MiB of sources, beyond the 256 MB MALL), back to back on
    the bench stream: the streaming ceiling the op's kernels compare with."""
    elements = mib * (1 << 20) // 4
    pairs = [(torch.ones(elements, device="cuda"), torch.empty(elements, device="cuda"))
             for _ in range(4)]
    with torch.cuda.stream(stream):
        for source, target in pairs:
            target.copy_(source)
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record(stream)
        for index in range(copies):
            source, target = pairs[index % 4]
            target.copy_(source)
        end.record(stream)
        end.synchronize()
    us = start.elapsed_time(end) * 1e3 / copies
    moved = 2 * elements * 4
    return {"gbps": round(moved / (us * 1e-6) / 1e9, 1), "us_per_copy": round(us, 3),
            "bytes_moved": moved, "kind": f"torch copy_ of {mib} MiB, 4 buffer pairs rotated"}


def kernel_sources_digest() -> str:
    """Digest of the kernel sources a traffic profile describes."""
    digest = hashlib.sha256()
    for name in KERNEL_SOURCES:
        digest.update(name.encode())
        digest.update((CSRC / name).read_bytes())
    return digest.hexdigest()[:16]


def load_traffic() -> tuple[int | None, str]:
    """HBM bytes per C1 backward launch from the committed PMC summary, when it
    profiles the kernel sources in this tree; else (None, why not)."""
    if not TRAFFIC_FILE.exists():
        return None, f"no {TRAFFIC_FILE.name}"
    record = json.loads(TRAFFIC_FILE.read_text())
    digest = kernel_sources_digest()
    if record.get("sources_digest") != digest:
        return None, (f"stale: {TRAFFIC_FILE.name} profiles kernel sources "
                      f"{record.get('sources_digest')}, this tree has {digest}")
    return record["hbm_bytes_per_launch"], (
        f"rocprofv3 PMC FETCH_SIZE x {record['fetch_scale']} + WRITE_SIZE x "
        f"{record['write_scale']} per dispatch, kernel sources {digest}, commit "
        f"{record.get('commit')}")


def mangled_kernel_name(name: str) -> str:
    """The Itanium-ABI mangled prefix (through the template arguments) of a
    kernel_name() instance, e.g. rln::rln_backward_kernel<rln::FixedShape<768,
    64>, _Float16, float, true> -> _ZN3rln19rln_backward_kernelINS_10Fixed
    ShapeILi768ELi64EEEDF16_fLb1EEE. rocprofv3 leaves names with _Float16 or
    __bf16 arguments mangled, so counter csv rows are matched on this too."""
    import re

    match = re.fullmatch(r"rln::(\w+)<rln::(\w+)<(\d+)(?:, (\d+))?>, ([\w ]+), ([\w ]+), "
                         r"(true|false)(?:, (true|false))?>", name)
    if match is None:
        raise ValueError(f"not a kernel_name() instance: {name}")
    kernel, shape, first, second, branch, normalized, aligned, ring = match.groups()
    types = {"float": "f", "_Float16": "DF16_", "__bf16": "DF16b"}
    flags = f"Lb{int(aligned == 'true')}E" + (f"Lb{int(ring == 'true')}E" if ring else "")
    shape_args = f"ILi{first}E" + (f"Li{second}E" if second is not None else "")
    return (f"_ZN3rln{len(kernel)}{kernel}INS_{len(shape)}{shape}{shape_args}EE"
            f"{types[branch]}{types[normalized]}{flags}EE")


def _counter_values(directory: str) -> tuple[str, dict[str, list[float]]]:
    """(counter name, the value of every dispatch by kernel name) of one
    rocprofv3 --pmc csv output directory."""
    import csv
    from collections import defaultdict

    files = sorted(Path(directory).rglob("*counter_collection.csv"))
    if not files:
        raise SystemExit(f"bench.py: no *counter_collection.csv under {directory}")
    values, counter = defaultdict(list), None
    for path in files:
        with path.open() as handle:
            for row in csv.DictReader(handle):
                counter = row["Counter_Name"]
                values[row["Kernel_Name"]].append(float(row["Counter_Value"]))
    return counter, dict(values)


def traffic_summary(fetch_dir: str, write_dir: str) -> int:
    """Writes TRAFFIC_FILE from a FETCH_SIZE and a WRITE_SIZE pass of
    `bench.py --quick --calibrate-copy-mib 256`: each counter (KiB per
    dispatch, averaged over the kernel's dispatches) is scaled by what it reads
    for the 256 MiB calibration copy (the runtime's largest copyBuffer
    dispatch: 262144 KiB read and written)."""
    fetch_counter, fetch = _counter_values(fetch_dir)
    write_counter, write = _counter_values(write_dir)
    if (fetch_counter, write_counter) != ("FETCH_SIZE", "WRITE_SIZE"):
        raise SystemExit(f"bench.py: expected FETCH_SIZE and WRITE_SIZE, got "
                         f"{fetch_counter} and {write_counter}")

    def lookup(table, prefix):
        mangled = mangled_kernel_name(prefix)
        matches = [v for name, v in table.items()
                   if name.startswith(prefix) or name.startswith(mangled)]
        if len(matches) != 1:
            raise SystemExit(f"bench.py: {len(matches)} kernels named {prefix}")
        return sum(matches[0]) / len(matches[0])

    def calibration(table):
        copies = [v for name, v in table.items() if name.startswith("__amd_rocclr_copyBuffer")]
        largest = max((value for v in copies for value in v), default=0.0)
        if largest < 0.25 * 262144:
            raise SystemExit("bench.py: no 256 MiB calibration copy in the counters "
                             "(run the passes with --calibrate-copy-mib 256)")
        return largest

    fetch_scale = 262144.0 / calibration(fetch)
    write_scale = 262144.0 / calibration(write)
    record = {"workload": C1.describe(), "sources_digest": kernel_sources_digest()}
    try:
        import subprocess

        record["commit"] = subprocess.run(["git", "-C", str(REPO), "rev-parse", "--short=12",
                                           "HEAD"], capture_output=True, text=True,
                                          check=True).stdout.strip()
    except (OSError, subprocess.CalledProcessError):
        record["commit"] = None
    record.update(fetch_scale=round(fetch_scale, 5), write_scale=round(write_scale, 5))
    for kernel, key, algorithmic in (("rln_backward_kernel", "", C1.backward_bytes()),
                                     ("rln_forward_kernel", "forward_", C1.forward_bytes())):
        name = kernel_name(kernel, C1)
        fetch_kib, write_kib = lookup(fetch, name), lookup(write, name)
        hbm = round(1024 * (fetch_kib * fetch_scale + write_kib * write_scale))
        record[f"{key}kernel"] = name
        record[f"{key}fetch_kib_per_dispatch"] = round(fetch_kib, 2)
        record[f"{key}write_kib_per_dispatch"] = round(write_kib, 2)
        record[f"{key}hbm_bytes_per_launch"] = hbm
        record[f"{key}algorithmic_bytes_per_launch"] = algorithmic
    TRAFFIC_FILE.write_text(json.dumps(record, indent=1) + "\n")
    print(json.dumps(record))
    return 0


def decode_mask(torch, words, rows: int, hidden: int):
    """keep[r, c] = bit c % 32 of int32 word r * hidden / 32 + c / 32, on the device."""
    shifts = torch.arange(32, device=words.device, dtype=torch.int32)
    bits = (words.view(rows, hidden // 32, 1) >> shifts) & 1
    return bits.view(rows, hidden).bool()


def parity_self_check(torch, runner: "Runner") -> dict:
    """One step of exactly the path the benchmark times (set 0, step 0's Philox
    offset, the weight/bias gradients accumulated into zeroed sums), checked
    against the reference's decomposition (dropout -> add -> LayerNorm, and its
    gradients, reference gfx1010_kernels/normalization.py:15-33) in float64 on
    this GPU, with the kernel's own dropout mask applied explicitly: `updated`
    bitwise; normalized, mean, rstd, grad_x (normwise <= 1e-5), grad_branch
    (one ulp of its type + 1e-5 of the largest value), dW/db (normwise <= 1e-4),
    and the mask's keep ratio within 6 sigma of 1 - p."""
    w, t = runner.w, runner.sets[0]
    if w.backward:
        t["grad_weight"].zero_()
        t["grad_bias"].zero_()
    runner.forward(0)
    if w.backward:
        runner.backward(0)
    torch.cuda.synchronize()
    f64 = torch.float64
    rows, hidden = w.rows, w.hidden
    branch = t["branch"].float()
    errors, ok = {}, True
    if w.dropping:
        # 1.0f / (1.0f - float(p)), in fp32 as the library computes it
        # (reference csrc/residual_layer_norm_kernel.hip:898-899).
        one = torch.tensor(1.0, dtype=torch.float32)
        scale = (one / (one - torch.tensor(w.dropout_p, dtype=torch.float32))).item()
        keep = decode_mask(torch, t["mask"], rows, hidden)
        dropped = ((branch * keep.float()) * scale).to(t["branch"].dtype).float()
        kept = keep.double().mean().item()
        sigma = (w.dropout_p * (1 - w.dropout_p) / (rows * hidden)) ** 0.5
        errors["keep_ratio"] = round(kept, 6)
        ok &= abs(kept - (1 - w.dropout_p)) <= 6 * sigma
    else:
        keep, scale, dropped = None, 1.0, branch
    updated = t["x"] + dropped
    errors["updated_bitwise"] = bool(torch.equal(updated.view(torch.int32),
                                                 t["updated"].view(torch.int32)))
    ok &= errors["updated_bitwise"]

    def normwise(actual, expected):
        return (actual.to(f64) - expected).abs().max().item() / max(expected.abs().max().item(),
                                                                   1e-30)

    def ulp_excess(actual, expected, dtype):
        if dtype == torch.float32:
            return normwise(actual, expected) - 1e-5
        bits = 10 if dtype == torch.float16 else 7
        floor = -14 if dtype == torch.float16 else -126
        exponent = torch.floor(torch.log2(expected.abs().clamp_min(2.0 ** floor)))
        bound = torch.exp2(exponent - bits) + 1e-5 * expected.abs().max()
        return ((actual.to(f64) - expected).abs() - bound).max().item()

    u = updated.to(f64)
    mean = u.mean(dim=1)
    centred = u - mean[:, None]
    rstd = 1.0 / torch.sqrt((centred * centred).mean(dim=1) + EPS)
    xhat = centred * rstd[:, None]
    weight, bias = runner.weight.to(f64), runner.bias.to(f64)
    normalized = xhat * weight + bias
    errors["mean"] = normwise(t["mean"], mean)
    errors["rstd"] = normwise(t["rstd"], rstd)
    errors["normalized"] = (normwise(t["normalized"], normalized)
                            if t["normalized"].dtype == torch.float32
                            else ulp_excess(t["normalized"], normalized, t["normalized"].dtype))
    ok &= errors["mean"] <= 1e-5 and errors["rstd"] <= 1e-5
    ok &= errors["normalized"] <= (1e-5 if t["normalized"].dtype == torch.float32 else 0.0)
    if w.backward:
        gu, gy = t["grad_updated"].to(f64), t["grad_normalized"].to(f64)
        q = gy * weight
        grad_x = gu + rstd[:, None] * (q - q.mean(dim=1, keepdim=True)
                                       - xhat * (q * xhat).mean(dim=1, keepdim=True))
        grad_branch = grad_x * (keep.to(f64) * scale if keep is not None else 1.0)
        errors["grad_x"] = normwise(t["grad_x"], grad_x)
        errors["grad_branch_ulp_excess"] = ulp_excess(t["grad_branch"], grad_branch,
                                                      t["grad_branch"].dtype)
        errors["grad_weight"] = normwise(t["grad_weight"], (gy * xhat).sum(dim=0))
        errors["grad_bias"] = normwise(t["grad_bias"], gy.sum(dim=0))
        ok &= errors["grad_x"] <= 1e-5 and errors["grad_branch_ulp_excess"] <= 0.0
        ok &= errors["grad_weight"] <= 1e-4 and errors["grad_bias"] <= 1e-4
    for name, value in errors.items():
        if isinstance(value, float):
            errors[name] = float(f"{value:.3e}")
    errors["pass"] = bool(ok)
    errors["checked"] = ("one step of the timed C-ABI path vs float64 dropout/add/LayerNorm "
                         "on this GPU with the kernel's mask")
    return errors


def probe_library():
    library = ctypes.CDLL(str(PROBE_LIBRARY))
    library.rln_probe_variant_count.restype = ctypes.c_int
    library.rln_probe_variant_name.restype = ctypes.c_char_p
    library.rln_probe_variant_name.argtypes = [ctypes.c_int]
    library.rln_probe_variant_kind.argtypes = [ctypes.c_int]
    library.rln_probe_variant_threads.argtypes = [ctypes.c_int]
    library.rln_probe_variant_config.argtypes = [ctypes.c_int]
    library.rln_probe_one_step_blocks.restype = ctypes.c_int64
    library.rln_probe_one_step_blocks.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_int64]
    library.rln_probe_launch.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int64,
                                         ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p]
    library.rln_probe_atomic_combine.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                                                 ctypes.c_int, ctypes.c_int64, ctypes.c_int,
                                                 ctypes.c_void_p]
    library.rln_probe_empty_launches.argtypes = [ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                                 ctypes.c_void_p]
    library.rln_probe_atomic_policy.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                                                ctypes.c_int64, ctypes.c_int, ctypes.c_void_p]
    library.rln_probe_atomic_fold.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                              ctypes.c_int64, ctypes.c_int, ctypes.c_int64,
                                              ctypes.c_int, ctypes.c_void_p]
    return library


# Copies of the weight/bias sums the atomic-combine probe spreads 256 blocks over.
PROBE_ATOMIC_COPIES = (1, 2, 4, 8, 16, 64, 256)
# Copies of the in-launch fold combine.
PROBE_FOLD_COPIES = (1, 2, 4, 8, 16)
PROBE_EMPTY_BLOCKS = (1, 256, 768, 2048, 3072)


def probe_fixed_costs(torch, runner: "Runner", library, hidden: int, repeats: int = 200) -> dict:
    """Two fixed costs of a pass, each from `repeats` launches issued back to
    back by a C loop (microseconds per launch): the weight/bias combine alone
    (256 blocks of 512 threads adding 2 x hidden fp32 values each with
    atomics, spread over 1..256 copies of the sums, consecutive blocks in
    different copies or in the same one; by the atomics' cache policy; and
    folded inside the launch - copies, agent-scope release fences, a ticket,
    the last block swapping the copies into the output), and an empty kernel
    of 1..3072 blocks of 256 threads (a launch's own cost on the GPU)."""
    handle = ctypes.c_void_p(runner.handle)
    sums = torch.zeros(max(PROBE_ATOMIC_COPIES) * 2 * hidden, device="cuda")
    atomic = {}
    for ranges, label in ((0, "interleaved"), (1, "block ranges")):
        atomic[label] = {}
        for copies in PROBE_ATOMIC_COPIES:
            def batch(_, copies=copies, ranges=ranges):
                if library.rln_probe_atomic_combine(sums.data_ptr(), hidden, copies, ranges, 256,
                                                    repeats, handle):
                    raise RuntimeError("rln_probe_atomic_combine failed")
            batch(0)
            atomic[label][str(copies)] = round(runner.timed(batch, 1) * 1e3 / repeats, 3)
    policies = {}
    for policy, label in ((0, "plain"), (2, "nt"), (16, "sc1"), (18, "nt sc1")):
        one = torch.zeros(2 * hidden, device="cuda")

        def batch(_, policy=policy, one=one):
            if library.rln_probe_atomic_policy(one.data_ptr(), hidden, policy, 256, repeats,
                                               handle):
                raise RuntimeError("rln_probe_atomic_policy failed")
        us = runner.timed(batch, 1) * 1e3 / repeats
        # Every float received exactly 256 * repeats additions of 1.0.
        exact = bool(torch.all(one == float(256 * repeats)).item())
        policies[label] = {"us": round(us, 3), "sums_exact": exact}
    atomic["one copy, buffer atomics by cache policy"] = policies
    # The fold inside one launch: adds into copies, release fence, ticket; the
    # last block swaps the copies for zeros and adds their total into the
    # output. After the launches every output value must be 256 * repeats and
    # every copy zero.
    fold = {}
    for copies in PROBE_FOLD_COPIES:
        copy_sums = torch.zeros(copies * 2 * hidden, device="cuda")
        out = torch.zeros(2 * hidden, device="cuda")
        counter = torch.zeros(1, device="cuda", dtype=torch.int32)

        def batch(_, copies=copies, copy_sums=copy_sums, out=out, counter=counter):
            if library.rln_probe_atomic_fold(copy_sums.data_ptr(), out.data_ptr(),
                                             counter.data_ptr(), hidden, copies, 256, repeats,
                                             handle):
                raise RuntimeError("rln_probe_atomic_fold failed")
        us = runner.timed(batch, 1) * 1e3 / repeats
        exact = bool(torch.all(out == float(256 * repeats)).item()
                     and torch.all(copy_sums == 0).item() and int(counter.item()) == 0)
        fold[str(copies)] = {"us": round(us, 3), "sums_exact": exact}
    atomic["fold in the launch, by copies"] = fold
    empty = {}
    for blocks in PROBE_EMPTY_BLOCKS:
        def batch(_, blocks=blocks):
            if library.rln_probe_empty_launches(blocks, 256, repeats, handle):
                raise RuntimeError("rln_probe_empty_launches failed")
        batch(0)
        empty[str(blocks)] = round(runner.timed(batch, 1) * 1e3 / repeats, 3)
    return {"atomic_combine_us_by_copies": atomic, "empty_kernel_us_by_blocks": empty}


# Persistent grids of the probe: waves per CU (each a whole number of blocks).
PROBE_WAVES_PER_CU = (4, 8, 12, 16, 24, 32)
# Probe points re-timed at the full launch count, per pass.
PROBE_FINALISTS = 6


# Stream configurations benchmarks/rln_probe.hip instantiates (its Cfg bits).
PROBE_CONFIGS = (0, 1, 2, 5)


def probe_config(workload: Workload) -> int:
    """The probe's stream configuration of a workload: bit 0 an fp32 branch
    (else 16-bit), bit 1 a 16-bit normalized output and upstream gradient
    (else fp32), bit 2 no mask (not dropping)."""
    return ((workload.branch_bytes == 4) | (workload.normalized_bytes == 2) << 1
            | (not workload.dropping) << 2)


def probe_applies(workload: Workload) -> bool:
    """Whether the probe moves this workload's streams: a configuration it
    instantiates, over at most 2^31 bytes per fp32 tensor."""
    return (probe_config(workload) in PROBE_CONFIGS
            and workload.rows * workload.hidden * 4 <= (1 << 31))


def probe_floor(torch, runner: "Runner", library, launches: int = ROOFLINE_LAUNCHES,
                table: bool = False) -> dict:
    """The measured streaming floor of the runner's workload: every variant of
    benchmarks/rln_probe.hip (block size, units per lane, look-ahead, 128-bit
    fp16, cache policy, LDS staging) on every grid (one step per thread, and
    persistent grids of PROBE_WAVES_PER_CU waves per CU), over the runner's
    own rotated sets. Each point is timed over launches / 4 back-to-back
    launches; the PROBE_FINALISTS fastest per pass are timed again over
    `launches`, twice, interleaved (the faster run counts); then the fastest
    forward and backward are timed alternating, as the step runs them.
    Microseconds per launch."""
    w = runner.w
    config = probe_config(w)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    arrays = []
    for t in runner.sets:
        names = ("x", "branch", "updated", "normalized", "mask", "mean", "rstd", "grad_updated",
                 "grad_normalized", "updated", "mask", "mean", "rstd", "grad_x", "grad_branch")
        # NULL for what the workload lacks (a forward-only one's gradients).
        arrays.append((ctypes.c_void_p * len(names))(
            *[t[name].data_ptr() if name in t else None for name in names]))
    handle = ctypes.c_void_p(runner.handle)
    rows, hidden = ctypes.c_int64(w.rows), ctypes.c_int64(w.hidden)

    def launcher(index, blocks):
        count = ctypes.c_int64(blocks)

        def launch(step):
            if library.rln_probe_launch(index, arrays[step % len(arrays)], rows, hidden, count,
                                        handle):
                raise RuntimeError(f"rln_probe_launch({index}, {blocks}) failed")
        return launch

    points = {0: [], 1: []}
    for index in range(library.rln_probe_variant_count()):
        kind = library.rln_probe_variant_kind(index)
        if library.rln_probe_variant_config(index) != config or (kind == 1 and not w.backward):
            continue
        threads = library.rln_probe_variant_threads(index)
        one_step = library.rln_probe_one_step_blocks(index, w.rows, w.hidden)
        grids = {"one step per thread": one_step}
        for waves in PROBE_WAVES_PER_CU:
            if waves % (threads // 64) == 0:
                blocks = waves * cus // (threads // 64)
                if blocks < one_step:
                    grids[f"{waves} waves/CU"] = blocks
        if threads >= 512:
            # One block on each of half the CUs: whether half the CUs can
            # stream the pass as fast (half the blocks to combine).
            grids["one block on half the CUs"] = cus // 2
        if kind == 2:
            continue
        name = library.rln_probe_variant_name(index).decode()
        for grid, blocks in grids.items():
            launch = launcher(index, blocks)
            for step in range(2 * len(arrays)):
                launch(step)
            us = runner.timed(launch, max(launches // 4, 1)) * 1e3
            points[kind].append({"variant": name, "grid": grid, "blocks": blocks,
                                 "index": index, "us": round(us, 3)})
    best = {}
    for kind, label in ((0, "fwd"), (1, "bwd")):
        if not points[kind]:
            continue
        finalists = sorted(points[kind], key=lambda point: point["us"])[:PROBE_FINALISTS]
        for point in finalists:
            point["us_full"] = []
        for _ in range(2):
            for point in finalists:
                point["us_full"].append(
                    runner.timed(launcher(point["index"], point["blocks"]), launches) * 1e3)
        for point in finalists:
            point["us_full"] = round(min(point["us_full"]), 3)
        best[label] = min(finalists, key=lambda point: point["us_full"])
    result = {}
    for label, point in best.items():
        result[label] = point["us_full"]
        result[f"{label}_probe"] = f'{point["variant"]}, {point["grid"]} ({point["blocks"]} blocks)'
    if "bwd" in best:
        forward = launcher(best["fwd"]["index"], best["fwd"]["blocks"])
        backward = launcher(best["bwd"]["index"], best["bwd"]["blocks"])

        def step(index):
            forward(index)
            backward(index)

        result["step"] = round(runner.timed(step, launches) * 1e3, 3)
    result.update({
        "fixed_costs": probe_fixed_costs(torch, runner, library, w.hidden),
        "points": len(points[0]) + len(points[1]),
        "kind": ("fastest of the benchmarks/rln_probe.hip streaming variants with the op's "
                 f"exact streams, {launches} launches back to back, {len(runner.sets)} rotated "
                 "sets; step = the fastest forward and backward alternating"),
    })
    if table:
        result["table"] = sorted(points[0] + points[1],
                                 key=lambda point: (point["variant"][:3], point["us"]))
    return result


def percentiles_us(batches_ms) -> dict:
    ordered = sorted(batches_ms)

    def pick(fraction):
        return round(ordered[min(len(ordered) - 1, int(fraction * len(ordered)))] * 1e3, 3)

    return {"p20": pick(0.2), "median": round(statistics.median(ordered) * 1e3, 3),
            "p80": pick(0.8), "batches": len(ordered), "steps_per_batch": 25}


def gbps(nbytes: int, ms: float) -> float:
    return nbytes / (ms * 1e-3) / 1e9


SPECIALIZED_HIDDEN = (128, 256, 384, 512, 768, 1024)


def wide_parts(hidden: int, kernel: str, rows: int = 0) -> int:
    """Waves per row of a run-time row length (rln_device.h wide_parts, and
    shape_info's sixteen-wave backward of large launches)."""
    if kernel == "rln_forward_kernel":
        return 1 if hidden <= 1024 else 2 if hidden <= 2048 else 4 if hidden <= 4096 else 8
    parts = (1 if hidden <= 704 else 3 if hidden <= 768 else 4 if hidden <= 1024 else
             2 if hidden <= 1216 else 4 if hidden <= 2432 else 8)
    if parts == 8 and hidden >= 6657 and rows * hidden >= 1 << 26:
        return 16
    return parts


def kernel_name(kernel: str, workload: Workload) -> str:
    """The template instance of `kernel` this workload launches (as rocprofv3
    names it): its row shape, branch type, normalized / gradient type, and the
    aligned access path. Mirrors the dispatch of rln_device.h: the specialized
    sizes' lanes per row (the forward's forward_lanes), and the run-time-length
    shapes each pass runs, 1024's backward and that of 768 columns from 65536
    rows among them (backward_runs_wide), the sixteen-wave backward of large
    launches of 6657-8192 columns, and the twelve-, nine- and twelve-wave
    (four waves per row, at most 8192 rows) backwards of small launches."""
    forward = kernel == "rln_forward_kernel"
    hidden = workload.hidden
    runs_wide = hidden == 1024 or (hidden == 768 and workload.rows >= 65536)
    if not forward and backward_twelve_waves(hidden, workload.rows):
        shape = f"rln::TwelveWaveShape<{hidden}>"
    elif not forward and backward_nine_waves(hidden, workload.rows):
        shape = f"rln::NineWaveShape<{hidden}>"
    elif hidden in SPECIALIZED_HIDDEN and (forward or not runs_wide):
        lanes = 64 if (hidden // 4) % 64 == 0 else 32
        if forward:
            lanes = {128: 16, 768: 64, 1024: 64}.get(hidden, 32)
        shape = f"rln::FixedShape<{hidden}, {lanes}>"
    else:
        parts = wide_parts(hidden, kernel, workload.rows)
        vectors = -(-hidden // (256 * parts))
        if not forward and parts == 4 and vectors <= 2 and workload.rows <= 8192:
            shape = f"rln::StaggeredWideShape<{vectors}>"
        else:
            shape = f"rln::WideShape<{vectors}, {parts}>"
    types = {"f32": "float", "f16": "_Float16", "bf16": "__bf16"}
    ring = ", true" if forward_ring(workload.rows, hidden) else ", false"
    return (f"rln::{kernel}<{shape}, {types[workload.branch]}, "
            f"{types[workload.normalized]}, true{ring if forward else ''}>")


def backward_twelve_waves(hidden: int, rows: int) -> bool:
    """Whether the backward runs twelve-wave blocks (rln_device.h
    backward_twelve_waves): 768 columns over 2048-9216 rows whose last row
    step keeps at least half of the 256 x 12 waves busy, or all of them."""
    teams = 256 * 12
    if hidden != 768 or rows < 2048 or rows > 3 * teams:
        return False
    last = rows % teams
    return last == 0 or 2 * last >= teams


def backward_nine_waves(hidden: int, rows: int) -> bool:
    """Whether the backward runs nine-wave blocks (rln_device.h
    backward_nine_waves): 384 columns over 11520-13056 rows, a third row step
    of the 256 x 9 two-row teams one-half to five-sixths full."""
    slots = 256 * 9 * 2
    return hidden == 384 and 2 * rows >= 5 * slots and 6 * rows <= 17 * slots


def forward_ring(rows: int, hidden: int) -> bool:
    """Whether the forward runs its ring-walk instance (rln_device.h
    forward_ring and forward_paced): launches that are not paced and whose
    grid gives teams several rows."""
    elements = rows * hidden
    parts = wide_parts(hidden, "rln_forward_kernel")
    vectors = -(-hidden // (256 * parts))
    specialized_four_slots = hidden in (512, 1024)
    if hidden >= 256 and elements >= 1 << 23:
        if parts == 1 or (elements >= 1 << 26 and not (parts == 8 and vectors == 4)):
            return False
    if parts > 1:
        return elements < (1 << 24 if parts < 8 else 1 << 27)
    if specialized_four_slots and elements < 1 << 24:
        return True
    return elements < 1 << 23


def result_line(torch, workload: Workload, timing: dict, steps: int, warmup: int,
                sets: int, traffic) -> dict:
    total = workload.forward_bytes() + workload.backward_bytes()
    value = gbps(total, timing["step_ms"])
    forward_gbps = gbps(workload.forward_bytes(), timing["forward_ms"])
    if workload.backward:
        dominant, dominant_ms = "rln_backward_kernel", timing["backward_ms"]
        dominant_bytes = workload.backward_bytes()
    else:
        dominant, dominant_ms = "rln_forward_kernel", timing["forward_ms"]
        dominant_bytes = workload.forward_bytes()
    dominant_gbps = gbps(dominant_bytes, dominant_ms)
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(timing["step_ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded torch.randn, BASELINE.json distributions)",
        "config": {
            "workload": workload.describe() + f", {sets} rotated input sets",
            "rows": workload.rows,
            "hidden": workload.hidden,
            "dropout_p": workload.dropout_p,
            "branch_dtype": DTYPE_NAMES[workload.branch],
            "normalized_dtype": DTYPE_NAMES[workload.normalized],
            "parallelism": "single GPU",
        },
        "pct_of_peak": round(100.0 * value / HBM_PEAK_GBPS, 2),
        "step_us_spread": percentiles_us(timing["step_batches_ms"]),
        "rows_per_s": round(workload.rows / (timing["step_ms"] * 1e-3), 1),
        "fwd_gbps": round(forward_gbps, 2),
        "fwd_pct_of_peak": round(100.0 * forward_gbps / HBM_PEAK_GBPS, 2),
        "fwd_us": round(timing["forward_ms"] * 1e3, 3),
        "algorithmic_bytes_per_step": total,
        "roofline": {
            "bound": "hbm",
            "kernel": kernel_name(dominant, workload),
            "achieved": round(dominant_gbps, 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(dominant_gbps / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "algorithmic_bytes_per_launch": dominant_bytes,
            "avg_us_per_launch": round(dominant_ms * 1e3, 3),
            "launches": timing["launches"],
        },
        "cpu_baseline": None,
        "device": torch.cuda.get_device_name(0),
        "host": platform.node(),
    }
    if workload.backward:
        cold = gbps(total, timing["cold_ms"])
        line["bwd_us"] = round(timing["backward_ms"] * 1e3, 3)
        # The same backward with dW/db not requested: the difference is the
        # cost of the weight/bias sums (block combine + fp32 atomics).
        if "backward_input_grads_ms" in timing:
            line["bwd_input_grads_only_us"] = round(timing["backward_input_grads_ms"] * 1e3, 3)
        line["cold_step"] = {
            "us_per_step": round(timing["cold_ms"] * 1e3, 3),
            "gbps": round(cold, 2),
            "pct_of_peak": round(100.0 * cold / HBM_PEAK_GBPS, 2),
        }
    return line


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures a single GPU; --gpus {args.gpus} is not supported "
              "(one MI355X per box; the operator is row-parallel and would shard rows "
              "with no communication besides DDP's all-reduce of dW/db).", file=sys.stderr)
        return 2
    names = [workload.name for workload in sweep_workloads()]
    unknown = [name for name in args.config if name not in names]
    if unknown:
        print(f"bench.py: unknown --config {unknown}; the configurations are {names}",
              file=sys.stderr)
        return 2
    if args.traffic_summary:
        return traffic_summary(*args.traffic_summary)
    import torch

    from gfx1010_kernels import _cabi, residual_layer_norm_status

    status = residual_layer_norm_status(0)
    if not status.available:
        raise RuntimeError(f"native backend unavailable: {status.reason}")
    library = _cabi.library()
    stream = torch.cuda.Stream()

    traffic, traffic_note = load_traffic()

    if args.calibrate_copy_mib:
        with torch.cuda.stream(stream):
            elements = args.calibrate_copy_mib * (1 << 20) // 4
            source = torch.ones(elements, device="cuda")
            destination = torch.empty_like(source)
            destination.copy_(source)
            torch.cuda.synchronize()
            print(f"[bench] calibration copy of {args.calibrate_copy_mib} MiB done", flush=True)
            del source, destination

    if args.ab:
        chosen = [workload for workload in sweep_workloads() if workload.name in args.config]
        return run_ab(torch, _cabi, stream, args, chosen + ab_row_workloads(args)
                      or [C1])

    if args.dwdb_placement:
        with torch.cuda.stream(stream):
            print(json.dumps(dwdb_placement_study(torch, library, cabi=_cabi, stream=stream)),
                  flush=True)
        return 0

    if args.alternation:
        with torch.cuda.stream(stream):
            print(json.dumps(alternation_study(torch, library, _cabi, stream)), flush=True)
        return 0

    if args.config:
        chosen = [workload for workload in sweep_workloads() if workload.name in args.config]
        if args.ceiling:
            run_ceilings(torch, library, _cabi, stream, args, chosen)
        else:
            run_sweep(torch, library, _cabi, stream, args, chosen)
        return 0

    with torch.cuda.stream(stream):
        runner = Runner(torch, library, _cabi, C1, args.sets, stream)
        parity = parity_self_check(torch, runner)
        print(f"[bench] C1 parity self-check: {parity}", flush=True)
        if not parity["pass"]:
            print("bench.py: the timed path misses the parity bars; not timing it",
                  file=sys.stderr)
            return 1
        # --quick (the profiling runs) launches the kernels only as the step
        # does, so per-kernel counter averages describe the step's launches.
        timing = runner.measure(args.warmup, args.steps, input_grads=not args.quick)
        ceiling = None if args.quick else probe_floor(torch, runner, probe_library(),
                                                      table=args.ceiling)
        del runner
        print(f"[bench] C1: step {timing['step_ms'] * 1e3:.2f} us, forward "
              f"{timing['forward_ms'] * 1e3:.2f} us, backward {timing['backward_ms'] * 1e3:.2f} us, "
              f"cold step {timing['cold_ms'] * 1e3:.2f} us", flush=True)
    result = result_line(torch, C1, timing, args.steps, args.warmup, args.sets, traffic)
    result["roofline"]["traffic_note"] = traffic_note
    result["parity"] = parity
    if args.quick:
        print(json.dumps(result), flush=True)
        if args.sweep:
            run_sweep(torch, library, _cabi, stream, args, sweep_workloads())
        if args.reference_matrix:
            for line in reference_matrix(torch):
                print(json.dumps(line), flush=True)
        return 0
    probe_table = ceiling.pop("table", None)
    result["ceiling_us"] = {
        **ceiling,
        "op_fwd": round(timing["forward_ms"] * 1e3, 3),
        "op_bwd": round(timing["backward_ms"] * 1e3, 3),
        "op_step": round(timing["step_ms"] * 1e3, 3),
        "op_over_ceiling_step": round(timing["step_ms"] * 1e3 / ceiling["step"], 4),
    }
    result["copy_ceiling"] = copy_ceiling(torch, stream)
    result["public_api"] = public_api_steps(torch, C1, stream)
    # The reference's own published metric (speedup over its PyTorch
    # decomposition on the same GPU, H = 384) at a length where the GPU work
    # dominates; the full table is --reference-table.
    (line,) = reference_table(torch, warmup=20, reps=200, sequences=(262144,))
    result["reference_method"] = {
        "shape": "B=1, T=262144, H=384, fp16 branch, p=0.15",
        "forward_speedup_vs_torch": line["forward"]["speedup"],
        "train_speedup_vs_torch": line["train"]["speedup"],
        "reference_best_published_gfx1010": {"forward": max(v[0] for v in REFERENCE_SPEEDUPS.values()),
                                              "train": max(v[1] for v in REFERENCE_SPEEDUPS.values())},
        "kind": "median of 200 event-timed public calls, implementation='gfx950' vs 'torch'",
    }
    if not args.no_cpu_baseline:
        print(f"[bench] CPU baseline (~{args.cpu_seconds:.0f} s)", flush=True)
        result["cpu_baseline"] = cpu_baseline(torch, C1, args.cpu_seconds)
    print(json.dumps(result), flush=True)
    if probe_table is not None:
        print(json.dumps({"kind": "probe_table", "workload": C1.describe(),
                          "points": probe_table}), flush=True)

    if args.prenorm:
        line = {"metric": "pre-norm stack fwd+bwd step time (ms)", "higher_is_better": False,
                **prenorm_stack(torch, stream)}
        print(json.dumps(line), flush=True)

    if args.char_gpt:
        line = {"metric": "char-GPT AMP fwd+bwd microstep time (ms)", "higher_is_better": False,
                **char_gpt_microstep(torch, stream)}
        print(json.dumps(line), flush=True)

    if args.reference_table:
        for line in reference_table(torch):
            print(json.dumps(line), flush=True)

    if args.reference_matrix:
        for line in reference_matrix(torch):
            print(json.dumps(line), flush=True)

    if args.sweep:
        run_sweep(torch, library, _cabi, stream, args, sweep_workloads())
    if args.ceiling:
        run_ceilings(torch, library, _cabi, stream, args, sweep_workloads())
    return 0


# The probe variants and grids the alternation study pairs with the op: the
# fastest C1 forward and backward of the probe tables measured so far.
ALTERNATION_PROBES = (("fwd t512 u1 ld2 st17 ahead0 wide0", 256),
                      ("bwd t256 u4 ld2 st17 ahead1 wide0", 1024))


# Byte distances from grad_weight to grad_bias for --dwdb-placement: every
# KiB from 3 to 128, then multiples of 128 KiB to 4 MiB.
DWDB_OFFSETS = tuple(k * 1024 for k in range(3, 129)) + tuple(k << 17 for k in range(2, 33))


def dwdb_placement_study(torch, library, cabi, stream, launches: int = 200) -> dict:
    """C1's backward (atomic dW/db) with grad_weight at the start of a
    buffer and grad_bias DWDB_OFFSETS bytes after it, against the same
    backward without the sums: what the 256 blocks' weight/bias atomics add
    to the kernel for each relative placement of the two sums (the C ABI
    takes them as two independent pointers)."""
    runner = Runner(torch, library, cabi, C1, 4, stream)
    if not parity_self_check(torch, runner)["pass"]:
        raise SystemExit("bench.py: the timed path misses the parity bars")
    hidden = C1.hidden
    pool = torch.zeros((DWDB_OFFSETS[-1] + 4 * hidden) // 4 + 1024, device="cuda",
                       dtype=torch.float32)
    points = []
    for offset in DWDB_OFFSETS:
        for tensors in runner.sets:
            tensors["grad_weight"] = pool[:hidden]
            tensors["grad_bias"] = pool[offset // 4: offset // 4 + hidden]
        runner._launch_arguments()
        for index in range(20):
            runner.step(index)
        backward = runner.timed(lambda i: runner.backward(i), launches) * 1e3
        input_grads = runner.timed(lambda i: runner.backward_input_grads(i), launches) * 1e3
        points.append({"offset_bytes": offset, "backward_us": round(backward, 3),
                       "input_grads_us": round(input_grads, 3),
                       "sums_us": round(backward - input_grads, 3)})
    sums = sorted(point["sums_us"] for point in points)
    return {"kind": "dwdb_placement", "workload": C1.describe(), "launches": launches,
            "weight_address_mod_64k": pool.data_ptr() % 65536,
            "sums_us_median": sums[len(sums) // 2], "points": points}


def alternation_study(torch, library, cabi, stream, launches: int = 400) -> dict:
    """How a C1 pass's time depends on the kernel before it: the op's forward
    and backward and the streaming probe's C1-shaped forward and backward
    (ALTERNATION_PROBES), alone and in alternating pairs, and the op's forward
    after the op's backward with a 64-row launch of the same forward between
    them (the forward's code then warm). Each sequence runs 12 untimed
    iterations, then `launches` timed ones between two events on the launch
    stream; microseconds per iteration, and for each pair the excess over its
    two members timed alone."""
    runner = Runner(torch, library, cabi, C1, 4, stream)
    if not parity_self_check(torch, runner)["pass"]:
        raise SystemExit("bench.py: the timed path misses the parity bars")
    tiny = Runner(torch, library, cabi, replace(C1, name="C1 64 rows", rows=64), 4, stream)
    probe = probe_library()
    names = {probe.rln_probe_variant_name(i).decode(): i
             for i in range(probe.rln_probe_variant_count())}
    arrays = []
    for t in runner.sets:
        tensors = (t["x"], t["branch"], t["updated"], t["normalized"], t["mask"], t["mean"],
                   t["rstd"], t["grad_updated"], t["grad_normalized"], t["updated"], t["mask"],
                   t["mean"], t["rstd"], t["grad_x"], t["grad_branch"])
        arrays.append((ctypes.c_void_p * len(tensors))(*[x.data_ptr() for x in tensors]))
    handle = ctypes.c_void_p(runner.handle)
    rows, hidden = ctypes.c_int64(C1.rows), ctypes.c_int64(C1.hidden)

    def probe_pass(name, blocks):
        index, count = names[name], ctypes.c_int64(blocks)

        def launch(step):
            if probe.rln_probe_launch(index, arrays[step % len(arrays)], rows, hidden, count,
                                      handle):
                raise RuntimeError(f"rln_probe_launch({name}) failed")
        return launch

    passes = {"op_fwd": runner.forward, "op_bwd": runner.backward,
              "probe_fwd": probe_pass(*ALTERNATION_PROBES[0]),
              "probe_bwd": probe_pass(*ALTERNATION_PROBES[1]), "op_fwd_64_rows": tiny.forward}
    sequences = [("op_fwd",), ("op_bwd",), ("probe_fwd",), ("probe_bwd",), ("op_fwd_64_rows",),
                 ("op_fwd", "op_bwd"), ("op_fwd", "probe_bwd"), ("probe_fwd", "op_bwd"),
                 ("probe_fwd", "probe_bwd"), ("op_bwd", "op_fwd_64_rows"),
                 ("op_bwd", "op_fwd_64_rows", "op_fwd")]
    timed = {}
    for sequence in sequences:
        def body(step, sequence=sequence):
            for name in sequence:
                passes[name](step)
        for step in range(12):
            body(step)
        timed[" + ".join(sequence)] = round(runner.timed(body, launches) * 1e3, 3)
    excess = {}
    for key, us in timed.items():
        parts = key.split(" + ")
        if len(parts) == 2 and all(part in timed for part in parts):
            excess[key] = round(us - sum(timed[part] for part in parts), 3)
    after_warm = round(timed["op_bwd + op_fwd_64_rows + op_fwd"]
                       - timed["op_bwd + op_fwd_64_rows"], 3)
    return {"kind": "alternation", "workload": C1.describe(), "us_per_iteration": timed,
            "pair_excess_us": excess,
            "op_fwd_after_op_bwd_and_a_64_row_forward_us": after_warm,
            "probe_passes": {"fwd": list(ALTERNATION_PROBES[0]),
                             "bwd": list(ALTERNATION_PROBES[1])},
            "launches": launches}


def run_ceilings(torch, library, cabi, stream, args, workloads) -> None:
    """One line per workload whose streams the probe moves (probe_applies):
    the op's kernels and the probe's measured streaming floor over the same
    buffers, microseconds per launch."""
    probe = probe_library()
    for workload in workloads:
        if not probe_applies(workload):
            continue
        torch.cuda.empty_cache()
        large = workload.rows * workload.hidden >= (1 << 26)
        launches = 40 if large else ROOFLINE_LAUNCHES
        with torch.cuda.stream(stream):
            runner = Runner(torch, library, cabi, workload, 2 if large else args.sets, stream)
            timing = runner.measure(min(args.warmup, 10), max(args.steps // 10, 20) if large
                                    else args.steps, launches)
            limit = probe_floor(torch, runner, probe, launches)
            del runner
        line = {"kind": "ceiling", "workload": workload.describe(),
                "op_us": {"fwd": round(timing["forward_ms"] * 1e3, 3)}, "ceiling_us": limit}
        if workload.backward:
            line["op_us"].update(bwd=round(timing["backward_ms"] * 1e3, 3),
                                 step=round(timing["step_ms"] * 1e3, 3))
        for key in ("fwd", "bwd", "step"):
            if key in line["op_us"]:
                line[f"op_over_ceiling_{key}"] = round(line["op_us"][key] / limit[key], 4)
        print(json.dumps(line), flush=True)


def parse_ab(specs) -> list[tuple[str, tuple[str, ...]]]:
    variants = []
    for spec in specs:
        name, _, defines = spec.partition("=")
        if not name or name == "default":
            raise SystemExit(f"bench.py: --ab {spec!r}: give the variant a name other than "
                             "'default'")
        variants.append((name, tuple(define for define in defines.split(",") if define)))
    return variants


def run_ab(torch, cabi, stream, args, workloads) -> int:
    """Times the default build and each --ab variant build of the library on
    the same inputs (one Runner per build, same seeds), round by round, so
    that every build is timed on the same box in alternation. Prints one
    line per workload with the per-round kernel times of every build and
    their medians (microseconds); each build's timed path passes the parity
    self-check first."""
    import importlib.util

    spec = importlib.util.spec_from_file_location(
        "rln_build", REPO / "gfx1010-kernels_amd" / "build.py")
    build = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(build)
    builds = [("default", (), cabi.library())]
    for name, defines in parse_ab(args.ab):
        path = build.variant_path(name)
        if args.ab_build or not path.exists():
            print(f"[bench] building variant {name}: {', '.join(defines)}", flush=True)
            build.build_variant(name, defines)
        builds.append((name, defines, cabi.load(path)))
    for workload in workloads:
        torch.cuda.empty_cache()
        large = workload.rows * workload.hidden >= (1 << 26)
        sets = 2 if large else args.sets
        launches = 40 if large else ROOFLINE_LAUNCHES
        steps = max(args.steps // 10, 20) if large else args.steps
        rounds = {name: [] for name, _, _ in builds}
        with torch.cuda.stream(stream):
            runners = []
            for name, _, library in builds:
                runner = Runner(torch, library, cabi, workload, sets, stream)
                parity = parity_self_check(torch, runner)
                if not parity["pass"]:
                    print(f"bench.py: build {name} misses the parity bars on {workload.name}: "
                          f"{parity}", file=sys.stderr)
                    return 1
                runners.append((name, runner))
            for index in range(args.ab_rounds):
                for name, runner in runners:
                    timing = runner.measure(min(args.warmup, 10), steps, launches,
                                            input_grads=workload.backward)
                    rounds[name].append({key[:-3]: round(value * 1e3, 3)
                                         for key, value in timing.items()
                                         if key.endswith("_ms") and isinstance(value, float)})
                print(f"[bench] A/B {workload.name} round {index + 1}/{args.ab_rounds}: "
                      + ", ".join(f"{name} step {rounds[name][-1]['step']:.2f} us"
                                  for name, _ in runners), flush=True)
            del runners
        line = {"kind": "ab", "workload": workload.describe(), "rounds": args.ab_rounds,
                "builds": {}}
        for name, defines, _ in builds:
            keys = rounds[name][0].keys()
            line["builds"][name] = {
                "defines": list(defines),
                "median_us": {key: round(statistics.median(r[key] for r in rounds[name]), 3)
                              for key in keys},
                "rounds_us": rounds[name],
            }
        print(json.dumps(line), flush=True)
    return 0


def run_sweep(torch, library, cabi, stream, args, workloads) -> None:
    """One JSON line per workload (the configurations other than C1)."""
    for workload in workloads:
        torch.cuda.empty_cache()
        large = workload.rows * workload.hidden >= (1 << 26)
        sets = 2 if large else args.sets
        steps = max(args.steps // 10, 20) if large else args.steps
        with torch.cuda.stream(stream):
            runner = Runner(torch, library, cabi, workload, sets, stream)
            parity = parity_self_check(torch, runner)
            timing = runner.measure(min(args.warmup, 10) if large else args.warmup, steps,
                                    input_grads=not args.quick)
            del runner
        torch.cuda.empty_cache()
        line = result_line(torch, workload, timing, steps, args.warmup, sets, None)
        line["sweep"] = True
        line["parity"] = parity
        if not workload.backward and not args.no_cpu_baseline:
            # C0's forward-only CPU path is cheap to sample (~0.5 ms per step).
            line["cpu_baseline"] = cpu_baseline(torch, workload, min(args.cpu_seconds, 5.0))
        print(json.dumps(line), flush=True)


if __name__ == "__main__":
    sys.exit(main())
