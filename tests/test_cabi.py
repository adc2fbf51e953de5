"""The C ABI library loads, exports every declared symbol and validates inputs.

No test here launches GPU work: every call below fails argument validation,
which happens before any HIP call.
"""

import ctypes
import re
import threading
from pathlib import Path

import pytest
import torch  # noqa: F401  (binds the library to torch's HIP runtime)

from gfx1010_kernels import _cabi
from gfx1010_kernels._normalization_native import NATIVE_HIDDEN_SIZES

HEADER = Path(__file__).resolve().parents[1] / "include" / "rln.h"


def _declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:[\w\s\*]+?)\b(rln_\w+)\s*\(", text, re.MULTILINE)))


def test_header_declares_the_expected_entry_points():
    assert _declared_functions() == sorted(_cabi.SIGNATURES)


def test_library_exports_every_declared_symbol():
    library = _cabi.library()
    for name in _declared_functions():
        assert hasattr(library, name), name


def test_library_metadata():
    library = _cabi.library()
    assert library.rln_target_arch() == b"gfx950"
    assert re.fullmatch(rb"\d+\.\d+\.\d+", library.rln_version())
    assert _cabi.supported_hidden_sizes() == NATIVE_HIDDEN_SIZES
    for hidden in NATIVE_HIDDEN_SIZES:
        assert library.rln_hidden_supported(hidden) == 1
    for hidden in (0, 32, 64, 100, 160, 1000, 8256, 16384):
        assert library.rln_hidden_supported(hidden) == 0
    assert NATIVE_HIDDEN_SIZES == tuple(range(128, 8193, 64))


def test_philox_struct_layout():
    assert ctypes.sizeof(_cabi.RlnPhilox) == 40
    assert _cabi.RlnPhilox.threads.offset == 32
    assert _cabi.RlnPhilox(1, 2, None, None).threads == 0


@pytest.mark.parametrize("hidden,threads,increment", [
    (768, 0, 4), (1600, 0, 4), (8192, 0, 4),
    # The reference's 4 * ceil(ceil(H / threads) / 4)
    # (csrc/residual_layer_norm_kernel.hip:1766-1770).
    (128, 128, 4), (512, 128, 4), (768, 128, 8), (1024, 128, 8), (1024, 192, 8),
    (1024, 256, 4), (768, 256, 4), (384, 192, 4),
    # No reference layout: other sizes, other widths.
    (1600, 128, 0), (640, 256, 0), (768, 64, 0), (768, 512, 0), (100, 0, 0),
])
def test_philox_increment(hidden, threads, increment):
    assert _cabi.philox_increment(hidden, threads) == increment


def test_size_queries():
    assert _cabi.mask_words(8192, 768) == 8192 * 24
    assert _cabi.mask_words(0, 768) == 0
    assert _cabi.backward_workspace_bytes(8192, 768, False) == 0
    assert _cabi.backward_workspace_bytes(0, 768, True) == 0
    # One partial [2, H] per block; 8 waves per block, one row per wave (two at
    # H=128/384), at most 256 blocks.
    assert _cabi.backward_workspace_bytes(8192, 768, True) == 256 * 2 * 768 * 4
    assert _cabi.backward_workspace_bytes(37, 128, True) == 3 * 2 * 128 * 4
    assert _cabi.backward_workspace_bytes(41, 768, True) == 6 * 2 * 768 * 4
    assert _cabi.backward_workspace_bytes(1 << 20, 1024, True) == 256 * 2 * 1024 * 4
    # The backward of 1024 columns runs 4 waves per row: 2 rows per 8-wave
    # block, and 3 per 12-wave block up to 8192 rows.
    assert _cabi.backward_workspace_bytes(41, 1024, True) == 14 * 2 * 1024 * 4
    assert _cabi.backward_workspace_bytes(8193, 1024, True) == 256 * 2 * 1024 * 4
    assert _cabi.backward_workspace_bytes(600, 1024, True) == 200 * 2 * 1024 * 4
    # Run-time row lengths in the backward: one wave per row up to 768, 4 up to
    # 1024, 2 up to 1216, 4 up to 2432, else 8 waves per row (8, 4, 2 or 1 rows
    # per 8-wave block); four-wave rows of one or two slots (769-1024 and
    # 1217-2048 columns) in 12-wave blocks up to 8192 rows.
    assert _cabi.backward_workspace_bytes(41, 640, True) == 6 * 2 * 640 * 4
    assert _cabi.backward_workspace_bytes(41, 896, True) == 14 * 2 * 896 * 4
    assert _cabi.backward_workspace_bytes(41, 1216, True) == 11 * 2 * 1216 * 4
    assert _cabi.backward_workspace_bytes(41, 1280, True) == 14 * 2 * 1280 * 4
    assert _cabi.backward_workspace_bytes(41, 2048, True) == 14 * 2 * 2048 * 4
    assert _cabi.backward_workspace_bytes(41, 2432, True) == 21 * 2 * 2432 * 4
    assert _cabi.backward_workspace_bytes(41, 2496, True) == 41 * 2 * 2496 * 4
    assert _cabi.backward_workspace_bytes(41, 4096, True) == 41 * 2 * 4096 * 4
    assert _cabi.backward_workspace_bytes(41, 8192, True) == 41 * 2 * 8192 * 4
    assert _cabi.backward_workspace_bytes(8192, 8192, True) == 256 * 2 * 8192 * 4


FAKE = 1 << 20  # a non-null address; validation fails before it is touched


def _forward(**overrides):
    args = dict(
        x=FAKE, branch=FAKE, branch_dtype=_cabi.RLN_DTYPE_F16, weight=FAKE, bias=FAKE,
        updated=FAKE, normalized=FAKE, mean=FAKE, rstd=FAKE, mask=FAKE, rows=4, hidden=768,
        dropout_p=0.1, eps=1e-5, training=True, philox=_cabi.RlnPhilox(1, 0, None, None),
    )
    args.update(overrides)
    _cabi.forward(**args)


@pytest.mark.parametrize(
    "overrides,status,message",
    [
        (dict(rows=0), _cabi.RLN_ERR_INVALID, "empty tensors are unsupported"),
        (dict(hidden=160), _cabi.RLN_ERR_UNSUPPORTED, "unsupported native hidden size: 160"),
        (dict(branch_dtype=7), _cabi.RLN_ERR_INVALID, "branch must use float16, bfloat16 or float32"),
        (dict(normalized_dtype=5), _cabi.RLN_ERR_INVALID, "normalized must use"),
        (dict(dropout_p=1.0), _cabi.RLN_ERR_INVALID, r"dropout_p must be in \[0, 1\)"),
        (dict(dropout_p=-0.1), _cabi.RLN_ERR_INVALID, r"dropout_p must be in \[0, 1\)"),
        (dict(dropout_p=0.999999999), _cabi.RLN_ERR_INVALID, r"dropout_p must be in \[0, 1\)"),
        (dict(eps=0.0), _cabi.RLN_ERR_INVALID, "eps must be positive"),
        (dict(x=None), _cabi.RLN_ERR_INVALID, "forward tensors must not be null"),
        (dict(mask=None), _cabi.RLN_ERR_INVALID, "dropout_mask must not be null"),
        (dict(philox=None), _cabi.RLN_ERR_INVALID, "philox must not be null"),
        (dict(rows=1 << 62), _cabi.RLN_ERR_INVALID, "overflows"),
        (dict(zero_grad_weight=FAKE), _cabi.RLN_ERR_INVALID,
         "zero_grad_weight and zero_grad_bias must both be given or both be null"),
        (dict(philox=_cabi.RlnPhilox(1, 0, None, None, 64)), _cabi.RLN_ERR_INVALID,
         "threads must be 0, 128, 192 or 256"),
        (dict(hidden=1600, philox=_cabi.RlnPhilox(1, 0, None, None, 128)),
         _cabi.RLN_ERR_UNSUPPORTED, "reference's dropout stream exists for hidden sizes"),
        (dict(philox=_cabi.RlnPhilox(1, 6, None, None, 128)), _cabi.RLN_ERR_INVALID,
         "offset that is a multiple of 4"),
    ],
)
def test_forward_rejects_invalid_arguments(overrides, status, message):
    with pytest.raises(_cabi.RlnError, match=message) as error:
        _forward(**overrides)
    assert error.value.status == status


def _backward(**overrides):
    args = dict(
        grad_updated=FAKE, grad_normalized=FAKE, updated=FAKE, weight=FAKE, mean=FAKE, rstd=FAKE,
        mask=FAKE, grad_x=FAKE, grad_branch=FAKE, branch_dtype=_cabi.RLN_DTYPE_F16,
        grad_weight=FAKE, grad_bias=FAKE, rows=4, hidden=768, dropout_p=0.1, training=True,
        deterministic=True, workspace=None, workspace_bytes=0,
    )
    args.update(overrides)
    _cabi.backward(**args)


@pytest.mark.parametrize(
    "overrides,message",
    [
        (dict(rows=-1), "empty tensors are unsupported"),
        (dict(hidden=100), "unsupported native hidden size: 100"),
        (dict(updated=None), "backward tensors must not be null"),
        (dict(grad_bias=None), "both be given or both be null"),
        (dict(mask=None), "dropout_mask must not be null"),
        (dict(), "workspace too small"),
        (dict(workspace=FAKE, workspace_bytes=16), "workspace too small"),
        (dict(workspace=FAKE + 4, workspace_bytes=1 << 30), "16-byte aligned"),
    ],
)
def test_backward_rejects_invalid_arguments(overrides, message):
    with pytest.raises(_cabi.RlnError, match=message):
        _backward(**overrides)


def test_glue_module_imports_and_checks_device_first():
    from gfx1010_kernels import _C

    x = torch.zeros(2, 128)
    with pytest.raises(RuntimeError, match="x must be a HIP tensor"):
        _C.residual_layer_norm_forward(x, x, torch.ones(128), torch.zeros(128), 0.0, 1e-5, True, 128)
    stats = torch.zeros(2)
    with pytest.raises(RuntimeError, match="updated must be a HIP tensor"):
        _C.residual_layer_norm_backward(
            x, x, x, torch.ones(128), stats, stats, torch.empty(0, dtype=torch.int32),
            0.0, True, True, 128, 16, 64, 1, True)
    with pytest.raises(RuntimeError, match="x must be a HIP tensor"):
        _C.residual_layer_norm(x, x, torch.ones(128), torch.zeros(128), 0.0, 1e-5, True, 128, 64, 64, 1)
    assert _C.target_arch() == "gfx950"


def test_glue_auto_check_declines_host_tensors_without_error():
    """The auto path's C++ check answers False for host tensors (the
    reference's first reason, "x must be a HIP tensor"), and the checked entry
    point returns None instead of raising, so the Python path works out the
    reason and falls back."""
    from gfx1010_kernels import _C

    x = torch.zeros(4, 768)
    args = (x, x.half(), torch.ones(768), torch.zeros(768), 0.1, 1e-5)
    assert _C.fused_inputs_supported(*args) is False
    assert _C.residual_layer_norm_if_supported(*args, True, 128, 64, 64, 1, None) is None


def test_noalloc_backward_refuses_partials_above_its_scratch_before_any_gpu_work():
    """rln_backward_noalloc checks its arguments and the size of the weight /
    bias partials on the host, before any HIP call: a shape whose
    deterministic partials exceed RLN_NOALLOC_SCRATCH_BYTES fails with
    RLN_ERR_INVALID and says why; atomic mode needs no scratch at all."""
    rows, hidden = 65536, 4096
    needed = _cabi.backward_workspace_bytes(rows, hidden, True)
    assert needed > _cabi.NOALLOC_SCRATCH_BYTES
    assert _cabi.backward_workspace_bytes(rows, 2048, True) <= _cabi.NOALLOC_SCRATCH_BYTES
    fake = 0x1000  # never dereferenced: the call fails before any GPU work
    with pytest.raises(_cabi.RlnError) as caught:
        _cabi.backward_noalloc(fake, fake, fake, fake, fake, fake, fake, fake, fake,
                               _cabi.RLN_DTYPE_F16, fake, fake, rows, hidden, 0.1, True, True)
    assert caught.value.status == _cabi.RLN_ERR_INVALID
    assert f"need {needed} bytes" in str(caught.value) and "scratch" in str(caught.value)
    with pytest.raises(_cabi.RlnError) as caught:
        _cabi.backward_noalloc(fake, fake, None, fake, fake, fake, fake, fake, fake,
                               _cabi.RLN_DTYPE_F16, fake, fake, rows, hidden, 0.1, True, True)
    assert "backward tensors must not be null" in str(caught.value)


def test_last_error_is_kept_per_thread():
    """rln_last_error() is thread-local (include/rln.h): a failure on one
    thread neither overwrites nor clears the message another thread reads
    afterwards, and a successful call clears only its own thread's message.
    The two threads take turns at barriers, so each reads its message after
    the other thread's failing call."""
    library = _cabi.library()
    barrier = threading.Barrier(2, timeout=30)
    seen = {}

    def first():
        seen["first status"] = library.rln_philox_increment(100, 0)
        barrier.wait()  # the second thread fails now
        barrier.wait()
        seen["first"] = library.rln_last_error().decode()

    def second():
        barrier.wait()
        seen["second status"] = library.rln_philox_increment(768, 64)
        barrier.wait()
        seen["second"] = library.rln_last_error().decode()
        seen["success"] = library.rln_philox_increment(768, 0)
        seen["cleared"] = library.rln_last_error().decode()

    threads = [threading.Thread(target=first), threading.Thread(target=second)]
    for thread in threads:
        thread.start()
    for thread in threads:
        thread.join(timeout=60)
    assert seen == {
        "first status": 0, "first": "unsupported hidden size 100",
        "second status": 0, "second": "threads must be 0, 128, 192 or 256",
        "success": 4, "cleared": "",
    }
