"""Forward parity of the gfx950 kernels against the CPU oracle.

Covers every hidden specialization, the fp16 / bf16 / fp32 branch, eval / train p=0 /
train with dropout, the reference's row-count boundaries
(tests/test_residual_layer_norm_native_matrix.py:171-181) and the misaligned
element-access path (tests/test_residual_layer_norm_vectorized.py:96-164).
"""

import pytest
import torch

from gfx1010_kernels import _C, residual_layer_norm
from parity import (
    REFERENCE_THREADS,
    SPECIALIZED_HIDDEN_SIZES,
    assert_bitwise,
    check_forward,
    generator_state,
    host,
    make_inputs,
)

pytestmark = pytest.mark.gpu

MODES = {
    "eval": (0.8, False),
    "train-p0": (0.0, True),
    "train-p0.15": (0.15, True),
}


@pytest.mark.parametrize("hidden", SPECIALIZED_HIDDEN_SIZES)
@pytest.mark.parametrize("branch_dtype", [torch.float16, torch.bfloat16, torch.float32],
                         ids=["f16", "bf16", "f32"])
@pytest.mark.parametrize("mode", list(MODES))
def test_forward_matches_oracle(hidden, branch_dtype, mode):
    dropout_p, training = MODES[mode]
    inputs = make_inputs((37, hidden), branch_dtype, seed=17 + hidden)
    torch.cuda.manual_seed(2026 + hidden)
    seed, offset = generator_state()
    threads = REFERENCE_THREADS[hidden]  # what the public API passes
    outputs = _C.residual_layer_norm_forward(*inputs, dropout_p, 1e-5, training, threads)
    check_forward(outputs, inputs, dropout_p, training, 1e-5, seed, offset, f"H={hidden} {mode}",
                  threads=threads)

    # The public strict API runs the same computation for the same RNG state.
    torch.cuda.manual_seed(2026 + hidden)
    updated, normalized = residual_layer_norm(
        *inputs, dropout_p=dropout_p, eps=1e-5, training=training, implementation="gfx950")
    assert_bitwise(host(updated), host(outputs[0]), "public updated")
    assert_bitwise(host(normalized), host(outputs[1]), "public normalized")


@pytest.mark.parametrize("hidden", [128, 384, 1024])
@pytest.mark.parametrize("rows", [1, 15, 16, 17, 511, 512, 513, 2047, 2048, 2049])
def test_row_count_boundaries(hidden, rows):
    inputs = make_inputs((rows, hidden), torch.float16, seed=227 + rows)
    torch.cuda.manual_seed(rows)
    seed, offset = generator_state()
    outputs = _C.residual_layer_norm_forward(*inputs, 0.1, 1e-5, True, 128)
    check_forward(outputs, inputs, 0.1, True, 1e-5, seed, offset, f"rows={rows}")


def test_grid_stride_rows_beyond_one_launch_wave():
    # More rows than the launch has waves: every wave walks several rows.
    inputs = make_inputs((3 * 8192 + 5, 256), torch.float16, seed=5)
    torch.cuda.manual_seed(6)
    seed, offset = generator_state()
    outputs = _C.residual_layer_norm_forward(*inputs, 0.2, 1e-5, True, 128)
    check_forward(outputs, inputs, 0.2, True, 1e-5, seed, offset, "grid-stride")


@pytest.mark.parametrize("branch_dtype", [torch.float16, torch.float32], ids=["f16", "f32"])
@pytest.mark.parametrize("dropout_p", [0.0, 0.15])
def test_misaligned_inputs_use_element_access_with_identical_results(branch_dtype, dropout_p):
    rows, hidden = 23, 384
    x, branch, weight, bias = make_inputs((rows, hidden), branch_dtype, seed=409)
    storage = torch.empty(rows * hidden + 1, device=x.device)
    misaligned_x = storage[1:].view(rows, hidden)
    misaligned_x.copy_(x)
    assert misaligned_x.is_contiguous() and misaligned_x.data_ptr() % 16 != 0

    torch.cuda.manual_seed(11)
    aligned = _C.residual_layer_norm_forward(x, branch, weight, bias, dropout_p, 1e-5, True, 128)
    torch.cuda.manual_seed(11)
    scalar = _C.residual_layer_norm_forward(
        misaligned_x, branch, weight, bias, dropout_p, 1e-5, True, 128)
    for name, a, b in zip(("updated", "normalized", "mean", "rstd", "mask"), aligned, scalar):
        assert_bitwise(host(b), host(a), name)


def test_leading_dimensions_are_flattened():
    inputs = make_inputs((2, 3, 5, 512), torch.float16, seed=3)
    torch.cuda.manual_seed(4)
    seed, offset = generator_state()
    outputs = _C.residual_layer_norm_forward(*inputs, 0.1, 1e-5, True, 128)
    assert outputs[0].shape == (2, 3, 5, 512) and outputs[2].shape == (30,)
    check_forward(outputs, inputs, 0.1, True, 1e-5, seed, offset, "4-d")


def test_raw_forward_rejects_invalid_inputs_on_gpu():
    x, branch, weight, bias = make_inputs((4, 768), torch.float16, seed=1)
    with pytest.raises(RuntimeError, match="empty tensors are unsupported"):
        _C.residual_layer_norm_forward(x[:0], branch[:0], weight, bias, 0.0, 1e-5, True, 128)
    for hidden in (96, 640 + 32, 8192 + 64):
        with pytest.raises(RuntimeError, match=f"unsupported native hidden size: {hidden}"):
            big = torch.zeros(4, hidden, device=x.device)
            _C.residual_layer_norm_forward(big, big, big[0], big[0], 0.0, 1e-5, True, 128)
    with pytest.raises(RuntimeError, match="threads must be 128, 192 or 256"):
        _C.residual_layer_norm_forward(x, branch, weight, bias, 0.0, 1e-5, True, 64)
    with pytest.raises(RuntimeError, match="all tensors must be contiguous"):
        strided = x.t().contiguous().t()
        _C.residual_layer_norm_forward(strided, branch, weight, bias, 0.0, 1e-5, True, 128)
    with pytest.raises(RuntimeError, match="x must use float32"):
        _C.residual_layer_norm_forward(x.half(), branch, weight, bias, 0.0, 1e-5, True, 128)


@pytest.mark.parametrize("mode", ["no_grad", "inference_mode", "no_input_requires_grad"])
def test_forward_without_a_graph_equals_the_recorded_forward(mode):
    """A call with nothing to record (grad mode off, or no input requiring
    grad) runs the forward alone, without the autograd node or the gradient
    sums. Its outputs equal the recorded call's bit for bit, it draws the same
    dropout mask from the same generator state and advances the generator by
    the same offset, and its outputs carry no graph."""
    inputs = make_inputs((5, 77, 768), torch.float16, seed=71)
    recorded_leaves = [t.detach().clone().requires_grad_(True) for t in inputs]
    torch.cuda.manual_seed(9)
    recorded = residual_layer_norm(*recorded_leaves, dropout_p=0.1, implementation="gfx950")
    recorded_offset = torch.cuda.default_generators[0].get_offset()
    assert all(t.grad_fn is not None for t in recorded)

    torch.cuda.manual_seed(9)
    if mode == "no_input_requires_grad":
        bare = residual_layer_norm(*inputs, dropout_p=0.1, implementation="gfx950")
    else:
        context = torch.no_grad() if mode == "no_grad" else torch.inference_mode()
        leaves = [t.detach().clone().requires_grad_(True) for t in inputs]
        with context:
            bare = residual_layer_norm(*leaves, dropout_p=0.1, implementation="gfx950")
    assert torch.cuda.default_generators[0].get_offset() == recorded_offset
    for actual, expected in zip(bare, recorded):
        assert actual.grad_fn is None and not actual.requires_grad
        assert_bitwise(host(actual), host(expected.detach()))


def test_auto_fast_check_accepts_exactly_what_the_reasons_accept():
    """implementation="auto" first asks one C++ check (`_C.fused_inputs_supported`)
    and works out the reference's reason (`_input_reason`) only when the check
    declines. The check must accept exactly the inputs with no reason and a
    native hidden size: one case per reason, plus accepted ones. After the fast
    path has served a call, a declined call still warns with its reason and
    falls back."""
    import warnings

    from gfx1010_kernels.normalization import _NATIVE_SIZES, _input_reason

    def inputs(rows=64, hidden=768, branch_dtype=torch.float16):
        generator = torch.Generator(device="cuda").manual_seed(rows + hidden)
        x = torch.randn(rows, hidden, device="cuda", generator=generator)
        return dict(x=x, branch=torch.randn_like(x).to(branch_dtype),
                    weight=torch.ones(hidden, device="cuda"),
                    bias=torch.zeros(hidden, device="cuda"))

    base = inputs()
    transposed = torch.randn(768, 64, device="cuda").t()
    cases = {
        "valid f16": (base, 0.1, 1e-5),
        "valid bf16": (inputs(branch_dtype=torch.bfloat16), 0.0, 1e-5),
        "valid f32 1600": (inputs(7, 1600, torch.float32), 0.5, 1e-6),
        "valid 3-d": ({**base, "x": base["x"].view(4, 16, 768),
                       "branch": base["branch"].view(4, 16, 768)}, 0.1, 1e-5),
        "x on cpu": ({**base, "x": base["x"].cpu()}, 0.1, 1e-5),
        "bias on cpu": ({**base, "bias": base["bias"].cpu()}, 0.1, 1e-5),
        "one dimension": ({**base, "x": base["x"][0], "branch": base["branch"][0]}, 0.1, 1e-5),
        "shape mismatch": ({**base, "branch": base["branch"][:32]}, 0.1, 1e-5),
        "hidden 160": (inputs(hidden=160), 0.1, 1e-5),
        "hidden 96": (inputs(hidden=96), 0.1, 1e-5),
        "hidden 8256": (inputs(2, 8256), 0.1, 1e-5),
        "hidden 772": (inputs(hidden=772), 0.1, 1e-5),
        "weight size": ({**base, "weight": base["weight"][:704]}, 0.1, 1e-5),
        "x float16": ({**base, "x": base["x"].half()}, 0.1, 1e-5),
        "x float64": ({**base, "x": base["x"].double()}, 0.1, 1e-5),
        "branch int32": ({**base, "branch": base["branch"].int()}, 0.1, 1e-5),
        "weight float16": ({**base, "weight": base["weight"].half()}, 0.1, 1e-5),
        "x not contiguous": ({**base, "x": transposed}, 0.1, 1e-5),
        "dropout 1": (base, 1.0, 1e-5),
        "dropout negative": (base, -0.1, 1e-5),
        "eps 0": (base, 0.1, 0.0),
        "dropout nan": (base, float("nan"), 1e-5),
        # No reason in Python (nan <= 0 is false): accepted, and the op itself
        # rejects it ("eps must be positive"), as it did before the check.
        "valid for the reasons, eps nan": (base, 0.1, float("nan")),
        "empty": (inputs(rows=0), 0.1, 1e-5),
    }
    for name, (tensors, dropout_p, eps) in cases.items():
        args = (tensors["x"], tensors["branch"], tensors["weight"], tensors["bias"])
        expected = (_input_reason(*args, dropout_p, eps) is None
                    and args[0].shape[-1] in _NATIVE_SIZES)
        assert _C.fused_inputs_supported(*args, dropout_p, eps) == expected, name
        assert expected == name.startswith("valid"), name
    with pytest.raises(RuntimeError, match="eps must be positive"):
        residual_layer_norm(base["x"], base["branch"], base["weight"], base["bias"],
                            eps=float("nan"))

    served = residual_layer_norm(base["x"], base["branch"], base["weight"], base["bias"])
    strict = residual_layer_norm(base["x"], base["branch"], base["weight"], base["bias"],
                                 implementation="gfx950")
    for actual, wanted in zip(served, strict):
        assert_bitwise(host(actual), host(wanted))
    declined = inputs(hidden=160)
    with warnings.catch_warnings(record=True) as caught:
        warnings.simplefilter("always")
        residual_layer_norm(declined["x"], declined["branch"], declined["weight"],
                            declined["bias"])
    assert any("native hidden size must be one of" in str(w.message) for w in caught)
