"""Write tests/golden/hiprand_philox_vectors.json from rocRAND itself.

The reference's dropout values come from hipRAND's Philox4x32-10
(csrc/residual_layer_norm_kernel.hip:449-480), which on ROCm is rocRAND's
engine. This script compiles hiprand_vectors.cpp (host code calling
rocRAND's rocrand_init / rocrand4 from the ROCm headers) with g++, asks it
for raw streams and for the reference kernel's keep masks on small shapes,
and stores the answers as fixtures. The oracle's restatement
(oracle/philox.c) is checked against them by tests/test_oracle.py.

Run here (needs g++ and /opt/rocm/include): python tests/golden/make_hiprand_vectors.py
"""

from __future__ import annotations

import json
import subprocess
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
OUT = HERE / "hiprand_philox_vectors.json"
ROCM_INCLUDE = "/opt/rocm/include"

# (seed, subsequence, offset, calls): both key words, subsequences past 2^32,
# every substate (offset % 4), and counters whose low word carries.
STREAMS = [
    (0, 0, 0, 2),
    (0x1234, 5, 8, 2),
    (0xFFFFFFFFFFFFFFFF, (1 << 32) + 7, 4, 2),
    (42, 3, 1, 3),
    (42, 3, 2, 3),
    (42, 3, 3, 3),
    (9, 0xFFFFFFFF, (1 << 34) + 12, 2),
    (9, 1, 4 * 0xFFFFFFFF, 2),
    (0x2545F4914F6CDD1D, 123456789, 1 << 40, 2),
]


def _threshold(p: float) -> int:
    return int(float(np.float32(p)) * 4294967296.0)


# (first_row, rows, hidden, threads, seed, offset, p): the reference's
# hidden sizes with its own thread counts (gfx1010_kernels/_normalization_native.py:5-12)
# and the other accepted ones (128, 192, 256), ragged last items, one and two
# hiprand4 calls per thread, and a row whose subsequence passes 2^32.
MASKS = [
    (0, 3, 768, 128, 0x2545F4914F6CDD1D, 0, 0.1),
    (0, 2, 1024, 192, 42, 8, 0.1),
    (0, 4, 128, 128, 7, 4, 0.5),
    (0, 2, 128, 256, 7, 12, 0.25),
    (0, 2, 384, 192, 123, 16, 0.1),
    (0, 2, 512, 128, 99, 0, 0.3),
    (0, 2, 256, 192, 1, 4, 0.1),
    (0, 2, 1024, 128, 5, 40, 0.1),
    (0, 2, 768, 256, 77, 24, 0.2),
    (40_000_000, 1, 768, 128, 3, 8, 0.1),
    # Rows on either side of subsequence 2^32 (row * threads + t), a 64-bit
    # seed, an offset past 2^32 * 4, and the rest of the size x threads grid.
    ((1 << 25) - 1, 2, 768, 128, 0xFEDCBA9876543210, 4 * ((1 << 32) + 3), 0.1),
    ((1 << 24) - 1, 2, 1024, 256, 0x0123456789ABCDEF, 4 * 17, 0.3),
    (5, 3, 256, 256, 2024, 4 * 9, 0.1),
    (1, 2, 384, 256, 99, 0, 0.05),
    (0, 2, 512, 192, 1234, 4 * 3, 0.7),
    (0, 1, 512, 256, 5, 4, 0.1),
    (0, 2, 128, 192, 42, 4 * 100, 0.1),
    (0, 2, 768, 192, 42, 4 * 101, 0.1),
    (3, 2, 1024, 192, 0xFFFFFFFFFFFFFFFF, 8, 0.1),
]


def main() -> None:
    with tempfile.TemporaryDirectory() as scratch:
        program = Path(scratch) / "hiprand_vectors"
        subprocess.run(
            ["g++", "-std=c++17", "-O1", "-D__HIP_PLATFORM_AMD__", f"-I{ROCM_INCLUDE}",
             str(HERE / "hiprand_vectors.cpp"), "-o", str(program)],
            check=True)
        requests = [f"stream {s} {q} {o} {c}" for s, q, o, c in STREAMS]
        requests += [f"mask {f} {r} {h} {t} {s} {o} {_threshold(p)}"
                     for f, r, h, t, s, o, p in MASKS]
        result = subprocess.run([str(program)], input="\n".join(requests) + "\n",
                                capture_output=True, text=True, check=True)
    lines = result.stdout.strip().split("\n")
    assert len(lines) == len(requests)
    streams = [
        {"seed": s, "subsequence": q, "offset": o, "calls": c,
         "words": [int(w) for w in line.split()]}
        for (s, q, o, c), line in zip(STREAMS, lines[: len(STREAMS)])
    ]
    masks = [
        {"first_row": f, "rows": r, "hidden": h, "threads": t, "seed": s, "offset": o,
         "dropout_p": p, "threshold": _threshold(p),
         "words": [int(w) for w in line.split()]}
        for (f, r, h, t, s, o, p), line in zip(MASKS, lines[len(STREAMS):])
    ]
    OUT.write_text(json.dumps({
        "source": "rocRAND 4.2.0 (ROCm 7.2.0) rocrand_init / rocrand4 of "
                  "rocrand/rocrand_philox4x32_10.h, the engine behind hipRAND's "
                  "hiprand_init / hiprand4 on ROCm; masks follow the reference kernel's "
                  "per-thread draws (csrc/residual_layer_norm_kernel.hip:449-511)",
        "streams": streams,
        "masks": masks,
    }, indent=1) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
