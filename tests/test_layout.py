"""Repository rules the product must keep (CPU).

* The product (the package under gfx1010-kernels_amd/ and the C ABI headers)
  never references the oracle: the oracle is only the checker, used by the
  tests, smoke() and bench.py's cpu_baseline leg.
* Every HIP build line disables packed fp32 instructions.
* Every entry point declared in include/rln.h carries a reference citation
  (file:line) or says it has no counterpart in the reference.
"""

import re
from pathlib import Path

REPO = Path(__file__).resolve().parents[1]
PRODUCT = REPO / "gfx1010-kernels_amd"


def product_sources():
    for suffix in ("*.py", "*.cpp", "*.hip", "*.h"):
        for path in PRODUCT.rglob(suffix):
            if "_build" not in path.parts:
                yield path
    yield from (REPO / "include").glob("*.h")


def test_product_does_not_reference_the_oracle():
    offenders = [str(p.relative_to(REPO)) for p in product_sources()
                 if re.search(r"\boracle\b", p.read_text())]
    assert offenders == []


def test_bench_uses_the_oracle_only_for_the_cpu_baseline():
    lines = (REPO / "bench.py").read_text().splitlines()
    uses = [i for i, line in enumerate(lines) if re.search(r"\bfrom oracle\b|\bimport oracle\b",
                                                           line)]
    assert uses, "bench.py's CPU baseline imports the oracle's torch path"
    for index in uses:
        enclosing = next(line for line in reversed(lines[:index]) if line.startswith("def "))
        assert enclosing.startswith("def cpu_baseline("), enclosing


def test_hip_flags_disable_packed_fp32():
    build = (PRODUCT / "build.py").read_text()
    assert '"-packed-fp32-ops"' in build and '"-target-feature"' in build


def test_every_entry_point_cites_the_reference_or_says_why_not():
    header = (REPO / "include" / "rln.h").read_text()
    blocks = re.split(r"\n(?=/\*)", header)
    for block in blocks:
        match = re.search(r"^\w[\w\s\*]*?\b(rln_\w+)\(", block, re.M)
        if not match:
            continue
        comment = block.split("*/")[0]
        assert re.search(r"\.(hip|py|cpp|h|md):\d+", comment) or "no counterpart" in comment, (
            match.group(1))
