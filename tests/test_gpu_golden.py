"""Every committed golden fixture (tests/golden/*.npz, written from torch
float64 by tests/golden/make_golden.py) through the gfx950 kernels.

The fixtures hold the reference's contract cases as data: eval and fp16 /
fp32 branches, dropout with a given keep mask, updated-only and
normalized-only upstream gradients, nearly-constant rows at eps 1e-5 and
1e-3 (reference tests/test_residual_layer_norm_edge_cases.py:134-193) and a
large mean offset. The kernels cannot draw a fixture's numpy keep mask, so a
dropout fixture's forward runs on its pre-dropped branch (the same fp32
`updated` bit for bit) and its backward on its keep mask packed into the
reference's words. Checks: `updated` bitwise; every other output within the
fp32 conditioned bounds of tests/parity.py; on rows with kappa <= 2 also the
1e-5 / 1e-4 normwise bars of the other parity tests.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from gfx1010_kernels import _C
from oracle import rln_oracle as oracle
from parity import (
    TOL_FORWARD,
    TOL_INPUT_GRAD,
    TOL_PARAMETER_GRAD,
    assert_bitwise,
    assert_normwise,
    assert_rounded_close,
    assert_within,
    conditioned_bounds,
    half_ulp,
    host,
)

pytestmark = pytest.mark.gpu
GOLDEN = sorted((Path(__file__).parent / "golden").glob("*.npz"))
BRANCH = {np.dtype(np.float32): torch.float32, np.dtype(np.float16): torch.float16}


@pytest.mark.parametrize("path", GOLDEN, ids=lambda p: p.stem)
def test_golden_fixture_through_the_kernels(path):
    d = dict(np.load(path, allow_pickle=False))
    print(f"[golden] {path.stem}", flush=True)
    rows, hidden = d["x"].shape
    eps = float(d["eps"])
    branch_type = BRANCH[d["branch"].dtype]
    kind = "f16" if branch_type == torch.float16 else "f32"
    keep = d.get("keep")
    branch = d["branch"]
    if keep is not None:
        branch = oracle.dropped_branch(branch, keep, d["scale"], kind).astype(d["branch"].dtype)
    device = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    x, weight, bias = device(d["x"]), device(d["weight"]), device(d["bias"])
    updated, normalized, mean, rstd, _ = _C.residual_layer_norm_forward(
        x, device(branch), weight, bias, 0.0, eps, False, 128)
    torch.cuda.synchronize()
    assert_bitwise(host(updated), d["updated"], "updated")

    bounds = conditioned_bounds(d["updated"], d["weight"], eps, d.get("grad_updated"),
                                d.get("grad_normalized"))
    assert_within(host(mean), d["mean"], bounds["mean"], "mean")
    assert_within(host(rstd), d["rstd"], bounds["rstd"], "rstd")
    assert_within(host(normalized), d["normalized"], bounds["normalized"], "normalized")
    tame = bounds["kappa"] <= 2.0
    if tame.any():
        assert_normwise(host(normalized)[tame], d["normalized"][tame], TOL_FORWARD,
                        "normalized (kappa <= 2)")
        assert_normwise(host(rstd)[tame], d["rstd"][tame], TOL_FORWARD, "rstd (kappa <= 2)")

    if "grad_x" not in d:
        return
    grad_updated = device(d["grad_updated"]) if "grad_updated" in d else None
    grad_normalized = device(d["grad_normalized"]) if "grad_normalized" in d else None
    if keep is not None:
        mask = device(oracle.encode_mask(keep).view(np.int32))
        dropout_p, scale = float(d["dropout_p"]), float(d["scale"])
    else:
        mask = torch.empty(0, dtype=torch.int32, device="cuda")
        dropout_p, scale = 0.0, 1.0
    grad_x, grad_branch, grad_weight, grad_bias = _C.residual_layer_norm_backward(
        grad_updated, grad_normalized, updated, weight, mean, rstd, mask, dropout_p, True,
        branch_type == torch.float16, 128, 64, 64, 1, True, branch_type)
    torch.cuda.synchronize()
    assert_within(host(grad_x), d["grad_x"], bounds["grad_x"], "grad_x")
    factor = keep * scale if keep is not None else 1.0
    branch_bound = bounds["grad_x"] * factor
    if branch_type == torch.float16:
        branch_bound = branch_bound + half_ulp(d["grad_branch"], "f16")
    assert_within(host(grad_branch), d["grad_branch"], branch_bound, "grad_branch")
    if tame.any():
        assert_normwise(host(grad_x)[tame], d["grad_x"][tame], TOL_INPUT_GRAD,
                        "grad_x (kappa <= 2)")
        if branch_type == torch.float16:
            assert_rounded_close(host(grad_branch)[tame], d["grad_branch"][tame], "f16",
                                 "grad_branch (kappa <= 2)")
    if "grad_weight" in d:
        assert_within(host(grad_weight), d["grad_weight"], bounds["grad_weight"], "grad_weight")
        assert_within(host(grad_bias), d["grad_bias"], bounds["grad_bias"], "grad_bias")
        if tame.all():
            assert_normwise(host(grad_weight), d["grad_weight"], TOL_PARAMETER_GRAD,
                            "grad_weight")
            assert_normwise(host(grad_bias), d["grad_bias"], TOL_PARAMETER_GRAD, "grad_bias")
