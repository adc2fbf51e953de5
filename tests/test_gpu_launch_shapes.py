"""Both sides of the forward's launch-shape switches, every row class.

Forward launches of one-wave rows below 2^23 elements run 2-5 blocks per CU
whose teams walk several rows (2^24 for the four-slot rows of 512 and 1024
columns); above, one row step per team on up to 65536 blocks, rounded down to
a whole number of blocks per CU, so that some teams take one step more.
Multi-wave rows run a persistent grid of eight waves
per CU (one block per row step when there are fewer) below 2^24 elements, or
below 2^27 for eight-wave rows walked with look-ahead, and the one-step grid
(two steps per team for eight-wave rows) above. Each case runs a forward +
backward just below and just above a switch, with ragged row counts, and
checks every element against the oracle (parity.check_full_tensor): the whole
mask bitwise, `updated` bitwise, the rest against float64 on the device, dW/db
against a float64 reduction.
"""

import pytest
import torch

from gfx1010_kernels import _C, _cabi
from parity import check_full_tensor, generator_state
from test_gpu_configs import check_parameter_gradients, device_inputs

pytestmark = pytest.mark.gpu
EPS = 1e-5
SWITCH = 1 << 23

# (hidden, rows below the switch, rows above it, branch type): one-wave rows of a
# specialized size, four and two rows per wave, and run-time rows of two, four
# and eight waves.
CASES = [
    (1024, 8191, 8193, torch.float16),
    (128, 65535, 65537, torch.float16),
    (384, 21845, 21846, torch.bfloat16),
    (1600, 5242, 5243, torch.float16),
    (4096, 2047, 2049, torch.float16),
    (8192, 1023, 1025, torch.bfloat16),
]


@pytest.mark.parametrize("side", ["below", "above"])
@pytest.mark.parametrize("hidden,below,above,branch_dtype", CASES,
                         ids=[f"H{case[0]}" for case in CASES])
def test_forward_grid_switch(hidden, below, above, branch_dtype, side):
    rows = below if side == "below" else above
    assert (rows * hidden >= SWITCH) == (side == "above")
    print(f"[launch shapes] rows={rows} H={hidden} {branch_dtype}", flush=True)
    inputs, grads = device_inputs(rows, hidden, branch_dtype, seed=hidden + rows)
    torch.cuda.manual_seed(hidden + rows)
    seed, offset = generator_state()
    outputs = _C.residual_layer_norm_forward(*inputs, 0.1, EPS, True, 128)
    gradients = _C.residual_layer_norm_backward(
        grads[0], grads[1], outputs[0], inputs[2], outputs[2], outputs[3], outputs[4], 0.1, True,
        branch_dtype == torch.float16, 128, 64, 64, 1, True, branch_dtype)
    assert gradients[1].dtype == branch_dtype
    check_full_tensor(inputs, grads, outputs, gradients, 0.1, EPS, seed, offset,
                      what=f"{rows} x {hidden}")
    check_parameter_gradients(outputs[0], grads[1], gradients)


# (hidden, rows below, rows above, branch type) around the switches from a
# persistent grid to one step per team: rows of two and four waves at 2^24
# elements (ragged and whole slots), eight waves of three slots where their walk
# turns paced (2^26), eight waves of four slots at 2^27, and the specialized
# four-slot rows (512, 1024 columns) at 2^24.
PERSISTENT_CASES = [
    (2048, 8191, 8192, torch.float16),
    (4096, 4095, 4096, torch.bfloat16),
    (1600, 10485, 10486, torch.float16),
    (6144, 10922, 10923, torch.float16),
    (8192, 16383, 16384, torch.bfloat16),
    # specialized rows of four slots per lane: one round of resident blocks below
    # 2^24 elements, one step per team above
    (1024, 16383, 16385, torch.float16),
    (512, 32767, 32768, torch.bfloat16),
]
PERSISTENT_SWITCH = {2048: 1 << 24, 4096: 1 << 24, 1600: 1 << 24, 6144: 1 << 26, 8192: 1 << 27,
                     1024: 1 << 24, 512: 1 << 24}


@pytest.mark.parametrize("side", ["below", "above"])
@pytest.mark.parametrize("hidden,below,above,branch_dtype", PERSISTENT_CASES,
                         ids=[f"H{case[0]}" for case in PERSISTENT_CASES])
def test_persistent_grid_switch(hidden, below, above, branch_dtype, side):
    rows = below if side == "below" else above
    assert (rows * hidden >= PERSISTENT_SWITCH[hidden]) == (side == "above")
    print(f"[launch shapes] rows={rows} H={hidden} {branch_dtype}", flush=True)
    inputs, grads = device_inputs(rows, hidden, branch_dtype, seed=5 * hidden + rows)
    torch.cuda.manual_seed(5 * hidden + rows)
    seed, offset = generator_state()
    outputs = _C.residual_layer_norm_forward(*inputs, 0.1, EPS, True, 128)
    gradients = _C.residual_layer_norm_backward(
        grads[0], grads[1], outputs[0], inputs[2], outputs[2], outputs[3], outputs[4], 0.1, True,
        branch_dtype == torch.float16, 128, 64, 64, 1, True, branch_dtype)
    check_full_tensor(inputs, grads, outputs, gradients, 0.1, EPS, seed, offset,
                      what=f"{rows} x {hidden}")
    check_parameter_gradients(outputs[0], grads[1], gradients)


@pytest.mark.parametrize("hidden,rows", [(4096, 1), (4096, 64), (2048, 1001), (8192, 3),
                                         (8192, 255), (6144, 257), (1280, 513),
                                         (1280, 3074), (4096, 2048), (2560, 1537), (1600, 4097)])
def test_multi_wave_persistent_grid_row_counts(hidden, rows):
    """Row counts that give the persistent grid fewer row steps than its eight
    waves per CU (one block per step), just past one or two blocks per CU, and
    inside the band of 6-8 row steps per CU that runs twelve waves per CU."""
    print(f"[launch shapes] rows={rows} H={hidden}", flush=True)
    inputs, grads = device_inputs(rows, hidden, torch.float16, seed=7 * hidden + rows)
    torch.cuda.manual_seed(7 * hidden + rows)
    seed, offset = generator_state()
    outputs = _C.residual_layer_norm_forward(*inputs, 0.1, EPS, True, 128)
    gradients = _C.residual_layer_norm_backward(
        grads[0], grads[1], outputs[0], inputs[2], outputs[2], outputs[3], outputs[4], 0.1, True,
        True, 128, 64, 64, 1, True, torch.float16)
    check_full_tensor(inputs, grads, outputs, gradients, 0.1, EPS, seed, offset,
                      what=f"{rows} x {hidden}")
    check_parameter_gradients(outputs[0], grads[1], gradients)


@pytest.mark.parametrize("hidden,rows,branch_dtype", [
    (512, 6144, torch.float16), (256, 10240, torch.bfloat16), (128, 32768, torch.float16),
    (384, 8192, torch.float32), (512, 16383, torch.float16), (640, 8192, torch.float16),
    (960, 8738, torch.bfloat16)], ids=lambda v: str(v).replace("torch.", ""))
def test_small_launches_at_one_round_of_resident_blocks(hidden, rows, branch_dtype):
    """Small forwards whose grid is one round of the blocks a CU holds at once
    (raised to it for rows of two or four per wave, lowered to it from between
    one and two rounds), whole tensors."""
    print(f"[launch shapes] rows={rows} H={hidden} {branch_dtype}", flush=True)
    inputs, grads = device_inputs(rows, hidden, branch_dtype, seed=11 * hidden + rows)
    torch.cuda.manual_seed(11 * hidden + rows)
    seed, offset = generator_state()
    outputs = _C.residual_layer_norm_forward(*inputs, 0.1, EPS, True, 128)
    gradients = _C.residual_layer_norm_backward(
        grads[0], grads[1], outputs[0], inputs[2], outputs[2], outputs[3], outputs[4], 0.1, True,
        branch_dtype == torch.float16, 128, 64, 64, 1, True, branch_dtype)
    check_full_tensor(inputs, grads, outputs, gradients, 0.1, EPS, seed, offset,
                      what=f"{rows} x {hidden}")
    check_parameter_gradients(outputs[0], grads[1], gradients)


@pytest.mark.parametrize("hidden,rows,branch_dtype,normalized_dtype", [
    (768, 10923, torch.bfloat16, torch.bfloat16),
    (256, 32769, torch.float16, torch.float16),
    (2048, 4097, torch.bfloat16, torch.float16),
], ids=["H768-bf16", "H256-f16", "H2048-bf16-f16"])
def test_half_normalized_above_the_switch(hidden, rows, branch_dtype, normalized_dtype):
    """The large-launch grid with a half-precision normalized output and
    upstream gradient (one ulp of its type), whole tensors."""
    assert rows * hidden >= SWITCH
    print(f"[launch shapes] rows={rows} H={hidden} {branch_dtype} -> {normalized_dtype}",
          flush=True)
    inputs, grads = device_inputs(rows, hidden, branch_dtype, seed=3 * hidden + rows)
    grads = (grads[0], grads[1].to(normalized_dtype))
    torch.cuda.manual_seed(3 * hidden + rows)
    seed, offset = generator_state()
    outputs = _C.residual_layer_norm_forward(*inputs, 0.1, EPS, True, 128,
                                             normalized_dtype=normalized_dtype)
    assert outputs[1].dtype == normalized_dtype
    gradients = _C.residual_layer_norm_backward(
        grads[0], grads[1], outputs[0], inputs[2], outputs[2], outputs[3], outputs[4], 0.1, True,
        branch_dtype == torch.float16, 128, 64, 64, 1, True, branch_dtype)
    check_full_tensor(inputs, grads, outputs, gradients, 0.1, EPS, seed, offset,
                      what=f"{rows} x {hidden} {normalized_dtype}")
    check_parameter_gradients(outputs[0], grads[1], gradients)


def _random_large_cases(count=8, seed=2302):
    """Seeded (rows, hidden, branch, normalized, p) above the switch: hidden any
    multiple of 64 up to 8192, 2^23-2^25 elements, every dtype pairing."""
    import random

    rng = random.Random(seed)
    cases = []
    for _ in range(count):
        hidden = 64 * rng.randint(2, 128)
        rows = rng.randint(SWITCH // hidden + 1, (1 << 25) // hidden)
        cases.append((rows, hidden, rng.choice([torch.float16, torch.bfloat16, torch.float32]),
                      rng.choice([None, torch.float16, torch.bfloat16]),
                      rng.choice([0.0, 0.1, 0.15])))
    return cases


@pytest.mark.parametrize("rows,hidden,branch_dtype,normalized_dtype,dropout_p",
                         _random_large_cases(), ids=lambda v: str(v).replace("torch.", ""))
def test_seeded_random_shapes_above_the_switch(rows, hidden, branch_dtype, normalized_dtype,
                                               dropout_p):
    print(f"[launch shapes] rows={rows} H={hidden} {branch_dtype} -> {normalized_dtype} "
          f"p={dropout_p}", flush=True)
    inputs, grads = device_inputs(rows, hidden, branch_dtype, seed=rows + 7 * hidden)
    if normalized_dtype is not None:
        grads = (grads[0], grads[1].to(normalized_dtype))
    torch.cuda.manual_seed(rows)
    seed, offset = generator_state()
    outputs = _C.residual_layer_norm_forward(*inputs, dropout_p, EPS, True, 128,
                                             normalized_dtype=normalized_dtype)
    gradients = _C.residual_layer_norm_backward(
        grads[0], grads[1], outputs[0], inputs[2], outputs[2], outputs[3], outputs[4],
        dropout_p, True, branch_dtype == torch.float16, 128, 64, 64, 1, True, branch_dtype)
    check_full_tensor(inputs, grads, outputs, gradients, dropout_p, EPS, seed, offset,
                      what=f"{rows} x {hidden}")
    check_parameter_gradients(outputs[0], grads[1], gradients)


# (hidden, rows below 2^26 elements, rows at or above, branch type): the
# backward's switch from eight waves of four slots to sixteen waves of two for
# rows of 6657-8192 columns.
SIXTEEN_WAVE_CASES = [
    (8192, 8191, 8192, torch.float16),
    (7168, 9362, 9363, torch.bfloat16),
    (6720, 9986, 9987, torch.float32),
]


@pytest.mark.parametrize("side", ["below", "above"])
@pytest.mark.parametrize("hidden,below,above,branch_dtype", SIXTEEN_WAVE_CASES,
                         ids=[f"H{case[0]}" for case in SIXTEEN_WAVE_CASES])
def test_sixteen_wave_backward_switch(hidden, below, above, branch_dtype, side):
    rows = below if side == "below" else above
    assert (rows * hidden >= 1 << 26) == (side == "above")
    print(f"[launch shapes] rows={rows} H={hidden} {branch_dtype}", flush=True)
    inputs, grads = device_inputs(rows, hidden, branch_dtype, seed=13 * hidden + rows)
    torch.cuda.manual_seed(13 * hidden + rows)
    seed, offset = generator_state()
    outputs = _C.residual_layer_norm_forward(*inputs, 0.1, EPS, True, 128)
    gradients = _C.residual_layer_norm_backward(
        grads[0], grads[1], outputs[0], inputs[2], outputs[2], outputs[3], outputs[4], 0.1, True,
        branch_dtype == torch.float16, 128, 64, 64, 1, True, branch_dtype)
    check_full_tensor(inputs, grads, outputs, gradients, 0.1, EPS, seed, offset,
                      what=f"{rows} x {hidden}")
    check_parameter_gradients(outputs[0], grads[1], gradients)


def test_sixteen_wave_backward_deterministic_and_half_gradient():
    """The sixteen-wave backward's fixed-order weight/bias reduction (bitwise
    equal over three runs) with a bf16 upstream gradient, whole tensors."""
    from test_gpu_backward import deterministic_algorithms

    rows, hidden = 8200, 8192
    print(f"[launch shapes] deterministic rows={rows} H={hidden}", flush=True)
    inputs, grads = device_inputs(rows, hidden, torch.bfloat16, seed=8200)
    grads = (grads[0], grads[1].to(torch.bfloat16))
    torch.cuda.manual_seed(8200)
    seed, offset = generator_state()
    outputs = _C.residual_layer_norm_forward(*inputs, 0.15, EPS, True, 128,
                                             normalized_dtype=torch.bfloat16)
    with deterministic_algorithms(True):
        runs = [_C.residual_layer_norm_backward(
            grads[0], grads[1], outputs[0], inputs[2], outputs[2], outputs[3], outputs[4], 0.15,
            True, False, 128, 64, 64, 1, True, torch.bfloat16) for _ in range(3)]
    for other in runs[1:]:
        for a, b in zip(runs[0], other):
            assert torch.equal(a.view(torch.int32) if a.dtype == torch.float32 else a,
                               b.view(torch.int32) if b.dtype == torch.float32 else b)
    check_full_tensor(inputs, grads, outputs, runs[0], 0.15, EPS, seed, offset,
                      what=f"{rows} x {hidden} deterministic")
    check_parameter_gradients(outputs[0], grads[1], runs[0])


# Row counts of 768 columns around backward_twelve_waves (rln_device.h): the
# backward runs twelve-wave blocks on the copy walk for 2048-9216 rows whose
# last row step keeps at least half of the 256 x 12 waves busy (or all of
# them), and the eight-wave ring otherwise.
TWELVE_WAVE_CASES = [(2047, False), (2048, True), (4096, False), (5120, True), (7168, False),
                     (8192, True), (9216, True), (9217, False)]

# Row counts of 384 columns around backward_nine_waves: nine-wave blocks of
# two-row teams for 11520-13056 rows, eight-wave blocks otherwise; 12291 is
# the C4 tail.
NINE_WAVE_CASES = [(11519, False), (11520, True), (12291, True), (13056, True), (13057, False)]


def _check_staggered_backward(rows, hidden, branch_dtype, mask_threads=128):
    """Whole tensors of the backward against the oracle; deterministic mode
    replays bitwise, and its input gradients equal the atomic mode's.
    `mask_threads`: the dropout layout the forward draws (0 at the hidden
    sizes that only have the library's own)."""
    from test_gpu_backward import deterministic_algorithms

    inputs, grads = device_inputs(rows, hidden, branch_dtype, seed=13 * hidden + rows)
    torch.cuda.manual_seed(13 * hidden + rows)
    seed, offset = generator_state()
    outputs = _C.residual_layer_norm_forward(*inputs, 0.1, EPS, True, 128)

    def backward():
        return _C.residual_layer_norm_backward(
            grads[0], grads[1], outputs[0], inputs[2], outputs[2], outputs[3], outputs[4], 0.1,
            True, True, 128, 64, 64, 1, True, branch_dtype)

    with deterministic_algorithms(False):
        atomic = backward()
    check_full_tensor(inputs, grads, outputs, atomic, 0.1, EPS, seed, offset,
                      threads=mask_threads, what=f"{rows} x {hidden}")
    check_parameter_gradients(outputs[0], grads[1], atomic)
    with deterministic_algorithms(True):
        first, second = backward(), backward()
    for a, b in zip(first, second):
        assert torch.equal(a, b)
    assert torch.equal(first[0], atomic[0]) and torch.equal(first[1], atomic[1])
    check_parameter_gradients(outputs[0], grads[1], first)


@pytest.mark.parametrize("rows,twelve_waves", TWELVE_WAVE_CASES,
                         ids=[f"{rows}-{'twelve' if twelve else 'eight'}"
                              for rows, twelve in TWELVE_WAVE_CASES])
def test_backward_twelve_wave_switch(rows, twelve_waves):
    """Both sides of the switch between eight- and twelve-wave backward blocks
    at 768 columns."""
    hidden = 768
    teams = 256 * 12
    last = rows % teams
    assert (2048 <= rows <= 3 * teams and (last == 0 or 2 * last >= teams)) == twelve_waves
    print(f"[launch shapes] backward rows={rows} H={hidden} twelve={twelve_waves}", flush=True)
    _check_staggered_backward(rows, hidden, torch.float16)


@pytest.mark.parametrize("rows,nine_waves", NINE_WAVE_CASES,
                         ids=[f"{rows}-{'nine' if nine else 'eight'}"
                              for rows, nine in NINE_WAVE_CASES])
def test_backward_nine_wave_switch(rows, nine_waves):
    """Both sides of the switch between eight- and nine-wave backward blocks
    at 384 columns, with the C4 tail's fp32 branch."""
    hidden = 384
    slots = 256 * 9 * 2
    assert (2 * rows >= 5 * slots and 6 * rows <= 17 * slots) == nine_waves
    print(f"[launch shapes] backward rows={rows} H={hidden} nine={nine_waves}", flush=True)
    _check_staggered_backward(rows, hidden, torch.float32)


# Four-wave rows of one or two slots per lane (769-1024 and 1217-2048
# columns) run their backward in twelve-wave blocks (StaggeredWideShape) up
# to 8192 rows; rows of three slots (2049-2432 columns) and of two waves
# (1025-1216) keep eight-wave blocks.
STAGGERED_WIDE_CASES = [(1600, 100, True), (1600, 8192, True), (1600, 8193, False),
                        (1024, 8192, True), (1024, 8193, False), (832, 4096, True),
                        (2432, 4096, False), (1216, 4096, False)]


@pytest.mark.parametrize("hidden,rows,staggered", STAGGERED_WIDE_CASES,
                         ids=[f"{hidden}x{rows}-{'twelve' if staggered else 'eight'}"
                              for hidden, rows, staggered in STAGGERED_WIDE_CASES])
def test_backward_staggered_wide_switch(hidden, rows, staggered):
    """Both sides of the switch between eight- and twelve-wave blocks for the
    backward of four-wave rows: the workspace query counts three rows per
    twelve-wave block, and whole tensors match the oracle either way."""
    per_slot = 4 * 64 * 4
    vectors = -(-hidden // per_slot)
    parts = 4 if (768 < hidden <= 1024 or 1216 < hidden <= 2432) else 2
    assert (parts == 4 and vectors <= 2 and rows <= 8192) == staggered
    rows_per_block = 3 if staggered else 8 // parts
    blocks = min(-(-rows // rows_per_block), 256)
    assert _cabi.backward_workspace_bytes(rows, hidden, True) == blocks * 2 * hidden * 4
    print(f"[launch shapes] backward rows={rows} H={hidden} staggered={staggered}", flush=True)
    _check_staggered_backward(rows, hidden, torch.float16, mask_threads=128 if hidden == 1024 else 0)


# One launch of each staggered backward shape (TwelveWaveShape<768>,
# NineWaveShape<384>, StaggeredWideShape<2> and <1>), with the branch type
# each serves in the sweep.
STAGGERED_SHAPES = [(768, 8192, torch.float16), (384, 12291, torch.float32),
                    (1600, 4096, torch.float16), (1024, 4096, torch.float16)]


@pytest.mark.parametrize("hidden,rows,branch_dtype", STAGGERED_SHAPES,
                         ids=[f"{hidden}x{rows}" for hidden, rows, _ in STAGGERED_SHAPES])
def test_staggered_backward_element_access_matches_vector_access(hidden, rows, branch_dtype):
    """The element-access instance of each staggered backward shape (taken
    when a tensor is not 16-byte aligned) gives the vector instance's bits,
    deterministic mode."""
    from parity import assert_bitwise, host, make_grads, make_inputs
    from test_gpu_backward import deterministic_algorithms, raw_backward

    print(f"[launch shapes] misaligned backward rows={rows} H={hidden}", flush=True)
    inputs = make_inputs((rows, hidden), branch_dtype, seed=hidden + rows)
    torch.cuda.manual_seed(hidden)
    outputs = _C.residual_layer_norm_forward(*inputs, 0.1, EPS, True, 128)
    grad_updated, grad_normalized = make_grads((rows, hidden), seed=hidden + rows + 1)
    storage = torch.empty(rows * hidden + 1, device="cuda")
    misaligned = storage[1:].view(rows, hidden)
    misaligned.copy_(grad_updated)
    assert misaligned.data_ptr() % 16 != 0
    with deterministic_algorithms(True):
        aligned = raw_backward(grad_updated, grad_normalized, outputs, inputs[2], 0.1,
                               branch_dtype)
        element = raw_backward(misaligned, grad_normalized, outputs, inputs[2], 0.1,
                               branch_dtype)
    for a, b, name in zip(aligned, element, ("grad_x", "grad_branch", "grad_weight",
                                             "grad_bias")):
        assert_bitwise(host(b), host(a), f"{rows} x {hidden} {name}")
