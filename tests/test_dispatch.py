"""Public API surface and dispatch rules (CPU only).

Follows the reference's CPU-runnable tests: fallback with a warning on CPU
(tests/test_residual_layer_norm.py:34-44), strict-mode error ordering before
any backend lookup (:47-99), and the public surface (tests/test_api.py:43-48).
"""

import warnings

import pytest
import torch
from torch.nn import functional as F

import gfx1010_kernels
import gfx1010_kernels.normalization as normalization
from gfx1010_kernels import (
    BackendStatus,
    can_use_residual_layer_norm,
    residual_layer_norm,
    residual_layer_norm_status,
)

STRICT = ["gfx950", "gfx1010"]


def _torch_reference(x, branch, weight, bias, dropout_p=0.0, eps=1e-5, training=True):
    if training:
        branch = F.dropout(branch, dropout_p, True)
    updated = x + branch
    return updated, F.layer_norm(updated, (updated.shape[-1],), weight, bias, eps)


def test_public_surface():
    assert gfx1010_kernels.__version__ == "0.4.0"
    assert set(gfx1010_kernels.__all__) == {
        "__version__", "BackendStatus", "can_use_residual_layer_norm",
        "residual_layer_norm", "residual_layer_norm_status",
        "prenorm_forward", "residual_norm",
    }
    assert callable(gfx1010_kernels.residual_layer_norm_status)
    status = BackendStatus(True, "dev", "gfx950", "ready")
    with pytest.raises(Exception):
        status.available = False


def test_cpu_falls_back_to_torch():
    x = torch.randn(2, 4, 16)
    branch = torch.randn_like(x)
    weight = torch.randn(16)
    bias = torch.randn(16)
    with pytest.warns(RuntimeWarning, match="was not used"):
        actual = residual_layer_norm(x, branch, weight, bias)
    expected = _torch_reference(x, branch, weight, bias)
    torch.testing.assert_close(actual[0], expected[0])
    torch.testing.assert_close(actual[1], expected[1])
    assert not can_use_residual_layer_norm(x, branch, weight, bias)


@pytest.mark.parametrize("implementation", STRICT)
def test_forced_kernel_reports_cpu_input_before_backend_lookup(monkeypatch, implementation):
    def fail_if_called(*args, **kwargs):
        raise AssertionError("forced CPU input reached backend lookup")

    monkeypatch.setattr(normalization, "residual_layer_norm_status", fail_if_called)
    x = torch.randn(2, 4, 128)
    with pytest.raises(RuntimeError, match="x must be a HIP tensor"):
        residual_layer_norm(x, x, torch.ones(128), torch.zeros(128), implementation=implementation)


class FakeCudaTensor:
    is_cuda = True
    ndim = 2
    shape = (4, 160)

    def get_device(self):
        return 0


@pytest.mark.parametrize("implementation", STRICT)
def test_forced_kernel_reports_hidden_size_before_backend_lookup(monkeypatch, implementation):
    def fail_if_called(*args, **kwargs):
        raise AssertionError("invalid hidden size reached backend lookup")

    monkeypatch.setattr(normalization, "residual_layer_norm_status", fail_if_called)
    tensor = FakeCudaTensor()
    with pytest.raises(RuntimeError, match="native hidden size must be one of"):
        residual_layer_norm(tensor, tensor, tensor, tensor, implementation=implementation)


@pytest.mark.parametrize("implementation", STRICT)
def test_forced_kernel_reports_unavailable_backend(monkeypatch, implementation):
    class Tensor768(FakeCudaTensor):
        shape = (4, 768)
        device = torch.device("cpu")

    monkeypatch.setattr(
        normalization,
        "residual_layer_norm_status",
        lambda device=None: BackendStatus(False, "x", "gfx942", "the native extension targets gfx950"),
    )
    monkeypatch.setattr(normalization, "_READY_DEVICES", set())
    tensor = Tensor768()
    with pytest.raises(RuntimeError, match="unavailable: the native extension targets gfx950"):
        residual_layer_norm(tensor, tensor, tensor, tensor, implementation=implementation)


def test_invalid_implementation_is_a_value_error():
    x = torch.randn(2, 128)
    with pytest.raises(ValueError, match="implementation must be"):
        residual_layer_norm(x, x, torch.ones(128), torch.zeros(128), implementation="cuda")


def test_triton_is_not_part_of_the_build():
    x = torch.randn(2, 128)
    with pytest.raises(RuntimeError, match="x must be a HIP tensor"):
        residual_layer_norm(x, x, torch.ones(128), torch.zeros(128), implementation="triton")


def test_torch_implementation_runs_the_decomposition():
    torch.manual_seed(3)
    x = torch.randn(3, 128)
    branch = torch.randn(3, 128)
    weight, bias = torch.randn(128), torch.randn(128)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        actual = residual_layer_norm(x, branch, weight, bias, training=False, implementation="torch")
    expected = _torch_reference(x, branch, weight, bias, training=False)
    torch.testing.assert_close(actual[0], expected[0], rtol=0, atol=0)
    torch.testing.assert_close(actual[1], expected[1], rtol=0, atol=0)


@pytest.mark.skipif(torch.cuda.is_available(), reason="CPU-only expectation")
def test_status_without_a_gpu():
    status = residual_layer_norm_status()
    assert status == BackendStatus(False, None, None, "PyTorch CUDA/HIP is unavailable")
    assert residual_layer_norm_status("cpu").reason == "PyTorch CUDA/HIP is unavailable"


def _eligible(monkeypatch, status):
    monkeypatch.setattr(normalization, "_input_reason", lambda *args: None)
    monkeypatch.setattr(normalization, "residual_layer_norm_status", lambda device=None: status)


def test_auto_raises_on_target_hardware_with_a_broken_extension(monkeypatch):
    _eligible(monkeypatch, BackendStatus(False, "MI355X", "gfx950", "cannot import _C"))
    x = torch.randn(2, 768)
    with pytest.raises(RuntimeError, match="unavailable: cannot import _C"):
        residual_layer_norm(x, x, torch.ones(768), torch.zeros(768))


def test_auto_falls_back_on_other_hardware(monkeypatch):
    _eligible(monkeypatch, BackendStatus(False, "other", "gfx1100", "the native extension targets gfx950"))
    x = torch.randn(2, 768)
    with pytest.warns(RuntimeWarning, match="was not used: the native extension targets gfx950"):
        residual_layer_norm(x, x, torch.ones(768), torch.zeros(768))


def test_auto_falls_back_for_non_native_hidden_size(monkeypatch):
    _eligible(monkeypatch, BackendStatus(True, "MI355X", "gfx950", "ready"))
    x = torch.randn(2, 136)
    with pytest.warns(RuntimeWarning, match="native hidden size must be one of"):
        residual_layer_norm(x, x, torch.ones(136), torch.zeros(136))


@pytest.mark.parametrize(
    "mutate,reason",
    [
        (lambda t: t.update(x=t["x"].double()), "requires float32 x"),
        (lambda t: t.update(branch=t["branch"].double()), "float16, bfloat16 or float32"),
        (lambda t: t.update(weight=t["weight"][:-8]), "match the final tensor dimension"),
        (lambda t: t.update(x=t["x"][:, :120].contiguous(), branch=t["branch"][:, :120].contiguous(),
                            weight=t["weight"][:120], bias=t["bias"][:120]), "between 128 and 8192"),
        (lambda t: t.update(x=t["x"].t().contiguous().t()), "contiguous"),
        (lambda t: t.update(dropout_p=1.0), r"\[0, 1\)"),
        (lambda t: t.update(eps=0.0), "eps must be positive"),
    ],
)
def test_input_reasons(mutate, reason):
    class Cuda(torch.Tensor):
        pass

    tensors = dict(x=torch.randn(4, 128), branch=torch.randn(4, 128), weight=torch.ones(128),
                   bias=torch.zeros(128), dropout_p=0.0, eps=1e-5)
    mutate(tensors)
    # Present the CPU tensors as HIP tensors to reach the later checks.
    for key in ("x", "branch", "weight", "bias"):
        tensors[key] = tensors[key].as_subclass(Cuda)
    Cuda.is_cuda = property(lambda self: True)
    try:
        found = normalization._input_reason(
            tensors["x"], tensors["branch"], tensors["weight"], tensors["bias"],
            tensors["dropout_p"], tensors["eps"])
    finally:
        del Cuda.is_cuda
    assert found is not None and __import__("re").search(reason, found), found


@pytest.mark.parametrize("hidden,native", [(128, True), (192, True), (1600, True), (8192, True),
                                           (136, False), (160, False), (1000, False),
                                           (8256, False)])
def test_native_hidden_sizes_are_the_multiples_of_64_up_to_8192(monkeypatch, hidden, native):
    """can_use_residual_layer_norm accepts every multiple of 64 from 128 to
    8192 when the inputs are otherwise eligible and the backend is ready."""
    _eligible(monkeypatch, BackendStatus(True, "MI355X", "gfx950", "ready"))
    x = torch.randn(2, hidden)
    assert can_use_residual_layer_norm(x, x, torch.ones(hidden), torch.zeros(hidden)) is native


def test_auto_eligibility_range_reaches_8192():
    x = torch.zeros(2, 8256)
    reason = normalization._input_reason(x, x, torch.ones(8256), torch.zeros(8256), 0.0, 1e-5)
    assert reason == "x must be a HIP tensor"  # checked before the size on CPU tensors

    class Cuda:
        is_cuda = True
        ndim = 2
        device = torch.device("cpu")

        def __init__(self, shape):
            self.shape = torch.Size(shape)

    wide = Cuda((2, 8256))
    assert "between 128 and 8192" in normalization._input_reason(
        wide, wide, wide, wide, 0.0, 1e-5)
