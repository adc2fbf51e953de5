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

Algorithmic bytes per row (H = 768, fp16 branch, dropout mask H/8 bytes):
  forward  H * (4 + 2 + 4 + 4) + 8 + H/8, plus 8H once (weight, bias)
  backward H * (4 + 4 + 4 + 4 + 2) + 8 + H/8, plus 12H once (weight; dW, db)
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _path in (REPO, REPO / "gfx1010-kernels_amd"):
    if str(_path) not in sys.path:
        sys.path.insert(0, str(_path))

HBM_PEAK_GBPS = 8000.0
METRIC = "fwd & fwd+bwd achieved HBM GB/s (% of ~8 TB/s peak), rows/s at H=768"
BATCH, SEQUENCE, HIDDEN = 8, 1024, 768
ROWS = BATCH * SEQUENCE
DROPOUT_P = 0.1
EPS = 1e-5
BRANCH_BYTES = 2
TRAFFIC_FILE = REPO / "profiles" / "rln_backward_c1_traffic.json"


def forward_bytes(rows: int = ROWS, hidden: int = HIDDEN) -> int:
    return rows * (hidden * (4 + BRANCH_BYTES + 4 + 4) + 8 + hidden // 8) + 8 * hidden


def backward_bytes(rows: int = ROWS, hidden: int = HIDDEN) -> int:
    return rows * (hidden * (4 + 4 + 4 + 4 + BRANCH_BYTES) + 8 + hidden // 8) + 12 * hidden


def parse_args():
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=500)
    parser.add_argument("--warmup", type=int, default=50)
    parser.add_argument("--sets", type=int, default=4, help="rotated input sets")
    parser.add_argument("--cpu-seconds", type=float, default=15.0,
                        help="time budget of the CPU baseline sample")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--calibrate-copy-mib", type=int, default=0,
                        help="also launch one device copy of this many MiB (PMC calibration)")
    return parser.parse_args()


def make_set(torch, seed: int):
    """One input/output set on the device, from a seeded CPU generator."""
    generator = torch.Generator().manual_seed(seed)
    shape = (ROWS, HIDDEN)
    host = {
        "x": torch.randn(shape, generator=generator),
        "branch": (0.5 * torch.randn(shape, generator=generator)).half(),
        "grad_updated": torch.randn(shape, generator=generator),
        "grad_normalized": torch.randn(shape, generator=generator),
    }
    tensors = {name: value.cuda() for name, value in host.items()}
    f32 = dict(device="cuda", dtype=torch.float32)
    tensors.update(
        updated=torch.empty(shape, **f32),
        normalized=torch.empty(shape, **f32),
        mean=torch.empty(ROWS, **f32),
        rstd=torch.empty(ROWS, **f32),
        mask=torch.empty(ROWS * HIDDEN // 32, device="cuda", dtype=torch.int32),
        grad_x=torch.empty(shape, **f32),
        grad_branch=torch.empty(shape, device="cuda", dtype=torch.float16),
        grad_weight=torch.zeros(HIDDEN, **f32),
        grad_bias=torch.zeros(HIDDEN, **f32),
    )
    return tensors


def cpu_baseline(torch, budget_seconds: float) -> dict:
    """The reference's CPU path on this host, on a bounded sample of C1 steps."""
    from oracle.torch_path import fwd_bwd_step

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    generator = torch.Generator().manual_seed(1001)
    shape = (ROWS, HIDDEN)
    x = torch.randn(shape, generator=generator).requires_grad_(True)
    branch = (0.5 * torch.randn(shape, generator=generator)).half().requires_grad_(True)
    weight = (1.0 + 0.02 * torch.randn(HIDDEN, generator=generator)).requires_grad_(True)
    bias = (0.02 * torch.randn(HIDDEN, generator=generator)).requires_grad_(True)
    grad_updated = torch.randn(shape, generator=generator)
    grad_normalized = torch.randn(shape, generator=generator)
    for _ in range(2):
        fwd_bwd_step(x, branch, weight, bias, grad_updated, grad_normalized, DROPOUT_P, EPS)
    samples = []
    start = time.perf_counter()
    while len(samples) < 10 or (time.perf_counter() - start < budget_seconds and len(samples) < 1000):
        began = time.perf_counter()
        fwd_bwd_step(x, branch, weight, bias, grad_updated, grad_normalized, DROPOUT_P, EPS)
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
    return {
        "value": round((forward_bytes() + backward_bytes()) / median / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"{len(samples)} fwd+bwd steps of C1 [8,1024,768] (F.dropout + add + "
                   f"F.layer_norm, autograd.grad), median {median * 1e3:.2f} ms/step, "
                   f"torch {torch.__version__} on {model}"),
        "rows_per_s": round(ROWS / median, 1),
        "ms_per_step": round(median * 1e3, 3),
    }


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures a single GPU; --gpus {args.gpus} is not supported "
              "(one MI355X per box; the operator is row-parallel and would shard rows "
              "with no communication besides DDP's all-reduce of dW/db).", file=sys.stderr)
        return 2
    import torch

    from gfx1010_kernels import _cabi, residual_layer_norm_status

    status = residual_layer_norm_status(0)
    if not status.available:
        raise RuntimeError(f"native backend unavailable: {status.reason}")
    library = _cabi.library()

    generator = torch.Generator().manual_seed(1001)
    weight = (1.0 + 0.02 * torch.randn(HIDDEN, generator=generator)).cuda()
    bias = (0.02 * torch.randn(HIDDEN, generator=generator)).cuda()
    sets = [make_set(torch, 1001 + index) for index in range(args.sets)]
    stream = torch.cuda.Stream()
    handle = stream.cuda_stream
    seed = 0x5EED_1001

    def launch_forward(step: int):
        t = sets[step % len(sets)]
        philox = _cabi.RlnPhilox(seed, 4 * step, None, None)
        status_code = library.rln_forward(
            t["x"].data_ptr(), t["branch"].data_ptr(), _cabi.RLN_DTYPE_F16, weight.data_ptr(),
            bias.data_ptr(), t["updated"].data_ptr(), t["normalized"].data_ptr(),
            t["mean"].data_ptr(), t["rstd"].data_ptr(), t["mask"].data_ptr(), ROWS, HIDDEN,
            DROPOUT_P, EPS, 1, philox, handle)
        if status_code:
            raise RuntimeError(_cabi.last_error())

    def launch_backward(step: int):
        t = sets[step % len(sets)]
        status_code = library.rln_backward(
            t["grad_updated"].data_ptr(), t["grad_normalized"].data_ptr(), t["updated"].data_ptr(),
            weight.data_ptr(), t["mean"].data_ptr(), t["rstd"].data_ptr(), t["mask"].data_ptr(),
            t["grad_x"].data_ptr(), t["grad_branch"].data_ptr(), _cabi.RLN_DTYPE_F16,
            t["grad_weight"].data_ptr(), t["grad_bias"].data_ptr(), ROWS, HIDDEN, DROPOUT_P,
            1, 0, 1, None, 0, handle)
        if status_code:
            raise RuntimeError(_cabi.last_error())

    def timed(body, count: int) -> float:
        """Milliseconds per iteration of `body` over `count` iterations, from
        HIP events recorded on the launch stream around the whole batch."""
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record(stream)
        for index in range(count):
            body(index)
        end.record(stream)
        end.synchronize()
        return start.elapsed_time(end) / count

    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        if args.calibrate_copy_mib:
            elements = args.calibrate_copy_mib * (1 << 20) // 4
            source = torch.ones(elements, device="cuda")
            destination = torch.empty_like(source)
            destination.copy_(source)
            torch.cuda.synchronize()
            print(f"[bench] calibration copy of {args.calibrate_copy_mib} MiB done", flush=True)
            del source, destination

        for step in range(args.warmup):
            launch_forward(step)
            launch_backward(step)
        stream.synchronize()
        print(f"[bench] warmup {args.warmup} steps done", flush=True)

        # Timed region: K whole steps, forward then backward of the same batch.
        base = args.warmup

        def step_body(index):
            launch_forward(base + index)
            launch_backward(base + index)

        ms_per_step = timed(step_body, args.steps)
        print(f"[bench] timed {args.steps} steps: {ms_per_step * 1e3:.2f} us/step", flush=True)

        # Per-kernel averages: each kernel alone, back to back over the sets.
        base += args.steps
        forward_ms = timed(lambda index: launch_forward(base + index), args.steps)
        base += args.steps
        # Every set now holds the saved state of a forward; re-running the
        # backward on it is the same work as the step's backward.
        backward_ms = timed(lambda index: launch_backward(base + index), args.steps)
        base += args.steps
        print(f"[bench] kernel averages: forward {forward_ms * 1e3:.2f} us, "
              f"backward {backward_ms * 1e3:.2f} us", flush=True)

        # Cold step: the backward runs on the batch forwarded two steps earlier.
        sets_count = len(sets)

        def cold_body(index):
            launch_forward(base + index)
            launch_backward(base + index - 2 + sets_count)

        cold_ms = timed(cold_body, args.steps)
        print(f"[bench] cold step: {cold_ms * 1e3:.2f} us/step", flush=True)

    total_bytes = forward_bytes() + backward_bytes()
    value = total_bytes / (ms_per_step * 1e-3) / 1e9
    backward_gbps = backward_bytes() / (backward_ms * 1e-3) / 1e9
    forward_gbps = forward_bytes() / (forward_ms * 1e-3) / 1e9
    cold_gbps = total_bytes / (cold_ms * 1e-3) / 1e9

    traffic = None
    if TRAFFIC_FILE.exists():
        traffic = json.loads(TRAFFIC_FILE.read_text()).get("hbm_bytes_per_launch")

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded torch.randn, BASELINE.json config 1 distributions)",
        "config": {
            "workload": "C1 fwd+bwd: x fp32 [8,1024,768], branch fp16, dropout_p=0.1, "
                        "atomic dW/db, 4 rotated input sets",
            "rows": ROWS,
            "hidden": HIDDEN,
            "dropout_p": DROPOUT_P,
            "branch_dtype": "float16",
            "parallelism": "single GPU",
        },
        "pct_of_peak": round(100.0 * value / HBM_PEAK_GBPS, 2),
        "rows_per_s": round(ROWS / (ms_per_step * 1e-3), 1),
        "fwd_gbps": round(forward_gbps, 2),
        "fwd_pct_of_peak": round(100.0 * forward_gbps / HBM_PEAK_GBPS, 2),
        "fwd_us": round(forward_ms * 1e3, 3),
        "bwd_us": round(backward_ms * 1e3, 3),
        "cold_step": {
            "us_per_step": round(cold_ms * 1e3, 3),
            "gbps": round(cold_gbps, 2),
            "pct_of_peak": round(100.0 * cold_gbps / HBM_PEAK_GBPS, 2),
        },
        "algorithmic_bytes_per_step": total_bytes,
        "roofline": {
            "bound": "hbm",
            "kernel": "rln_backward_kernel<768, _Float16, true>",
            "achieved": round(backward_gbps, 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(backward_gbps / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "algorithmic_bytes_per_launch": backward_bytes(),
        },
        "cpu_baseline": None,
        "device": torch.cuda.get_device_name(0),
        "host": platform.node(),
    }
    if not args.no_cpu_baseline:
        print(f"[bench] CPU baseline (~{args.cpu_seconds:.0f} s)", flush=True)
        result["cpu_baseline"] = cpu_baseline(torch, args.cpu_seconds)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
