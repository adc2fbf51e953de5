"""Pins the CPU oracle (oracle/) before it is trusted as the GPU checker.

Every oracle function is checked against something that does not restate it:
published known-answer vectors, rocRAND's own outputs, PyTorch float64 golden
vectors, closed forms, invariants and finite differences.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import rln_oracle as oracle
from oracle.torch_path import residual_layer_norm_torch

GOLDEN = Path(__file__).resolve().parent / "golden"


def _golden(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as data:
        return {key: data[key] for key in data.files}


def _normwise(actual, expected):
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    return np.max(np.abs(actual - expected)) / max(np.max(np.abs(expected)), 1e-300)


# ---------------------------------------------------------------------------
# Philox4x32-10 and the mask.

def test_philox_matches_random123_known_answers():
    kat = json.loads((GOLDEN / "philox4x32_10_kat.json").read_text())
    for vector in kat["vectors"]:
        counter = [int(word, 16) for word in vector["counter"]]
        key = [int(word, 16) for word in vector["key"]]
        expected = tuple(int(word, 16) for word in vector["expected"])
        assert oracle.philox4x32_10(counter, key) == expected


@pytest.mark.parametrize("rows,hidden", [(3, 128), (2, 384), (1, 1024)])
def test_mask_layout_matches_per_element_restatement(rows, hidden):
    seed, offset = 0x1234_5678_9ABC_DEF0, 4 * 37
    _, _, threshold = oracle.dropout_constants(0.3)
    words = oracle.dropout_mask_words(rows, hidden, seed, offset, threshold)
    expected = [0] * (rows * hidden // 32)
    key = [seed & 0xFFFFFFFF, seed >> 32]
    position = offset // 4
    for row in range(rows):
        for column in range(hidden):
            group = (row * hidden + column) // 4
            draw = oracle.philox4x32_10(
                [position & 0xFFFFFFFF, position >> 32, group & 0xFFFFFFFF, group >> 32], key
            )[column % 4]
            if draw >= threshold:
                word = row * (hidden // 32) + column // 32
                expected[word] |= 1 << (column % 32)
    assert words.tolist() == expected


def test_mask_words_equal_little_endian_u64_layout():
    rows, hidden = 4, 256
    _, _, threshold = oracle.dropout_constants(0.5)
    words = oracle.dropout_mask_words(rows, hidden, 99, 0, threshold)
    keep = oracle.decode_mask(words, rows, hidden)
    as_u64 = words.view("<u8")
    for row in range(rows):
        for column in range(hidden):
            bit = (int(as_u64[row * hidden // 64 + column // 64]) >> (column % 64)) & 1
            assert bit == keep[row, column]
    assert np.array_equal(oracle.encode_mask(keep), words)


def test_uniform_draws_agree_with_mask():
    rows, hidden = 3, 384
    draws = oracle.dropout_uniform(rows, hidden, 7, 8)
    _, _, threshold = oracle.dropout_constants(0.25)
    keep = oracle.decode_mask(oracle.dropout_mask_words(rows, hidden, 7, 8, threshold), rows, hidden)
    assert np.array_equal(keep, draws >= threshold)


@pytest.mark.parametrize("p", [0.1, 0.5, 0.9])
def test_keep_ratio_is_binomial(p):
    rows, hidden = 64, 1024
    _, _, threshold = oracle.dropout_constants(p)
    keep = oracle.decode_mask(oracle.dropout_mask_words(rows, hidden, 2026, 0, threshold), rows, hidden)
    n = keep.size
    sigma = np.sqrt(n * p * (1 - p))
    assert abs(keep.sum() - n * (1 - p)) < 6 * sigma


def test_offsets_select_disjoint_streams():
    a = oracle.dropout_uniform(2, 256, 5, 0)
    b = oracle.dropout_uniform(2, 256, 5, 4)
    c = oracle.dropout_uniform(2, 256, 6, 0)
    assert (a != b).mean() > 0.99 and (a != c).mean() > 0.99


# ---------------------------------------------------------------------------
# The reference's own stream: hipRAND (rocRAND) Philox per (row, thread).

def _hiprand_vectors():
    return json.loads((GOLDEN / "hiprand_philox_vectors.json").read_text())


def test_hiprand_stream_matches_rocrand():
    """rocrand_init / rocrand4 outputs, from rocRAND itself, for both key
    words, subsequences past 2^32, every substate and carrying counters."""
    streams = _hiprand_vectors()["streams"]
    assert {vector["offset"] % 4 for vector in streams} == {0, 1, 2, 3}
    for vector in streams:
        actual = oracle.hiprand_philox4(vector["seed"], vector["subsequence"],
                                        vector["offset"], vector["calls"])
        assert actual == vector["words"], vector


def test_hiprand_stream_with_zero_substate_is_plain_philox():
    """For offset % 4 == 0 the n-th rocrand4 is one Philox block of counter
    (offset/4 + n, subsequence) - the Random123-pinned function."""
    seed, subsequence, offset = 0xDEADBEEF_00C0FFEE, (3 << 32) + 11, 4 * ((1 << 33) + 5)
    words = oracle.hiprand_philox4(seed, subsequence, offset, 2)
    key = [seed & 0xFFFFFFFF, seed >> 32]
    for n in range(2):
        position = offset // 4 + n
        counter = [position & 0xFFFFFFFF, position >> 32, subsequence & 0xFFFFFFFF,
                   subsequence >> 32]
        assert tuple(words[4 * n: 4 * n + 4]) == oracle.philox4x32_10(counter, key)


def test_reference_mask_matches_rocrand():
    """The reference kernel's keep masks, drawn through rocRAND, on its six
    hidden sizes with thread counts 128 / 192 / 256 (ragged last items, one
    and two hiprand4 calls, a subsequence past 2^32)."""
    for vector in _hiprand_vectors()["masks"]:
        words = oracle.reference_mask_rows(
            vector["first_row"], vector["rows"], vector["hidden"], vector["threads"],
            vector["seed"], vector["offset"], vector["threshold"])
        assert words.tolist() == vector["words"], {k: vector[k] for k in vector if k != "words"}
        _, _, threshold = oracle.dropout_constants(vector["dropout_p"])
        assert threshold == vector["threshold"]


@pytest.mark.parametrize("hidden,threads,increment", [
    (128, 128, 4), (256, 128, 4), (384, 128, 4), (512, 128, 4), (768, 128, 8),
    (1024, 128, 8), (1024, 192, 8), (768, 256, 4), (128, 256, 4)])
def test_reference_philox_increment(hidden, threads, increment):
    assert oracle.reference_philox_increment(hidden, threads) == increment


def test_reference_mask_rejects_more_than_eight_values_per_thread():
    with pytest.raises(ValueError, match="at most 8 values"):
        oracle.reference_mask_words(1, 2048, 128, 1, 0, 1 << 30)


@pytest.mark.skipif(not Path("/opt/rocm/include/rocrand/rocrand_philox4x32_10.h").exists(),
                    reason="rocRAND headers are not installed")
def test_hiprand_fixtures_regenerate_from_rocrand(tmp_path, monkeypatch):
    """The committed fixtures are exactly what rocRAND's own engine outputs:
    rebuilding the generator against the installed headers reproduces them."""
    import importlib.util

    spec = importlib.util.spec_from_file_location(
        "make_hiprand_vectors", GOLDEN / "make_hiprand_vectors.py")
    generator = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(generator)
    monkeypatch.setattr(generator, "OUT", tmp_path / "vectors.json")
    generator.main()
    fresh = json.loads((tmp_path / "vectors.json").read_text())
    assert fresh == _hiprand_vectors()


def test_reference_mask_keep_ratio_is_binomial():
    rows, hidden, p = 64, 768, 0.1
    _, _, threshold = oracle.dropout_constants(p)
    keep = oracle.decode_mask(
        oracle.reference_mask_words(rows, hidden, 128, 11, 0, threshold), rows, hidden)
    n = keep.size
    assert abs(keep.sum() - n * (1 - p)) < 6 * np.sqrt(n * p * (1 - p))


def test_dropout_constants_closed_forms():
    assert oracle.dropout_constants(0.0) == (False, np.float32(1.0), 0)
    assert oracle.dropout_constants(0.7, training=False)[0] is False
    assert oracle.dropout_constants(0.5)[1:] == (np.float32(2.0), 1 << 31)
    assert oracle.dropout_constants(0.25)[1:] == (np.float32(4.0 / 3.0), 1 << 30)
    assert oracle.dropout_constants(0.75)[1:] == (np.float32(4.0), 3 << 30)
    # float32(0.1) = 13421773 * 2^-27, so the threshold is 13421773 * 2^5.
    active, scale, threshold = oracle.dropout_constants(0.1)
    assert active and threshold == 13421773 * 32
    assert scale == np.float32(1.1111112)


# ---------------------------------------------------------------------------
# The residual update (bit-exact).

def test_updated_without_dropout_is_torch_fp32_add():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((8, 128)).astype(np.float32)
    for branch in (rng.standard_normal((8, 128)).astype(np.float32),
                   rng.standard_normal((8, 128)).astype(np.float16)):
        expected = (torch.from_numpy(x) + torch.from_numpy(branch).float()).numpy()
        assert np.array_equal(oracle.updated(x, branch).view(np.uint32), expected.view(np.uint32))


def test_dropped_fp16_branch_rounds_fp32_product_once():
    # branch = 1.0, p = 0.1: scale = 1.1111112f and half(1.1111112f) = 1.111328125.
    _, scale, _ = oracle.dropout_constants(0.1)
    branch = np.ones((1, 4), np.float16)
    keep = np.array([[True, False, True, True]])
    dropped = oracle.dropped_branch(branch, keep, scale)
    assert dropped.tolist() == [[1.111328125, 0.0, 1.111328125, 1.111328125]]
    # b = 0.258056640625 (exact fp16): b * 1.1111111640930176f = 0.28672960... lies
    # 1174.44 fp16 steps (2^-12) above 0, so it rounds to 1174 * 2^-12 = 0.28662109375.
    # Multiplying in fp16 instead (b * half(scale) = b * 1.111328125 = 0.286784...,
    # 1174.67 steps) would give 0.286865234375.
    branch = np.full((1, 1), 0.258056640625, np.float16)
    assert float(scale) == 1.1111111640930176
    assert oracle.dropped_branch(branch, np.ones((1, 1), bool), scale)[0, 0] == 0.28662109375
    assert np.float16(branch[0, 0] * np.float16(scale)) == np.float16(0.286865234375)


def test_dropped_fp32_branch_is_single_rounded_product():
    _, scale, _ = oracle.dropout_constants(0.5)
    branch = np.array([[1.5, -3.0, 0.1]], np.float32)
    keep = np.array([[True, True, False]])
    assert oracle.dropped_branch(branch, keep, scale).tolist() == [[3.0, -6.0, 0.0]]


@pytest.mark.parametrize("name", ["forward_eval_f32_h128", "forward_f16_h384", "forward_dropout_f16_h256"])
def test_forward_updated_matches_golden_bitwise(name):
    case = _golden(name)
    keep = case.get("keep")
    result = oracle.forward(case["x"], case["branch"], case["weight"], case["bias"],
                            float(case["eps"]), keep=keep, scale=case["scale"])
    assert np.array_equal(result["updated"].view(np.uint32), case["updated"].view(np.uint32))


# ---------------------------------------------------------------------------
# LayerNorm forward.

FORWARD_CASES = [
    "forward_eval_f32_h128", "forward_f16_h384", "forward_dropout_f16_h256",
    "nearly_constant_rows_eps1e-5", "nearly_constant_rows_eps1e-3", "large_mean_h384",
]


@pytest.mark.parametrize("name", FORWARD_CASES)
def test_forward_statistics_match_torch_float64(name):
    case = _golden(name)
    mean, rstd, normalized = oracle.layer_norm_forward(
        case["updated"], case["weight"], case["bias"], float(case["eps"]))
    assert _normwise(normalized, case["normalized"]) < 1e-12
    assert _normwise(mean, case["mean"]) < 1e-12
    assert _normwise(rstd, case["rstd"]) < 1e-12


def test_forward_linspace_closed_form():
    hidden = 384
    centre, amplitude = 4.0, 2e-3
    t = np.linspace(-1.0, 1.0, hidden)
    row = centre + amplitude * t
    mean, rstd, _ = oracle.layer_norm_forward(row[None, :], np.ones(hidden), np.zeros(hidden), 1e-5)
    variance = amplitude ** 2 * (hidden + 1) / (3.0 * (hidden - 1))
    assert abs(mean[0] - centre) < 1e-12
    assert abs(rstd[0] - 1.0 / np.sqrt(variance + 1e-5)) / rstd[0] < 1e-12


def test_forward_normalized_row_invariants():
    rng = np.random.default_rng(11)
    u = rng.standard_normal((6, 512)) * 3.0 + 1.0
    mean, rstd, y = oracle.layer_norm_forward(u, np.ones(512), np.zeros(512), 1e-5)
    variance = 1.0 / rstd ** 2 - 1e-5
    assert np.allclose(y.mean(axis=-1), 0.0, atol=1e-12)
    assert np.allclose((y ** 2).mean(axis=-1), variance / (variance + 1e-5), rtol=1e-12)


def test_torch_path_matches_oracle_without_dropout():
    case = _golden("forward_f16_h384")
    updated, normalized = residual_layer_norm_torch(
        torch.from_numpy(case["x"]), torch.from_numpy(case["branch"]).float(),
        torch.from_numpy(case["weight"]), torch.from_numpy(case["bias"]),
        0.0, float(case["eps"]), training=False)
    assert np.array_equal(updated.numpy(), case["updated"])
    assert _normwise(normalized.numpy(), case["normalized"]) < 1e-5


# ---------------------------------------------------------------------------
# Backward.

BACKWARD_CASES = [
    "backward_dropout_f16_h384", "backward_f32_h128", "backward_updated_only_h256",
    "backward_normalized_only_h256", "nearly_constant_rows_eps1e-5",
    "nearly_constant_rows_eps1e-3", "large_mean_h384",
]


@pytest.mark.parametrize("name", BACKWARD_CASES)
def test_backward_matches_torch_float64_autograd(name):
    case = _golden(name)
    result = oracle.backward(case.get("grad_updated"), case.get("grad_normalized"), case["updated"],
                             case["weight"], float(case["eps"]), keep=case.get("keep"),
                             scale=case["scale"])
    assert _normwise(result["grad_x"], case["grad_x"]) < 1e-11
    assert _normwise(result["grad_branch"], case["grad_branch"]) < 1e-11
    if "grad_weight" in case:
        assert _normwise(result["grad_weight"], case["grad_weight"]) < 1e-11
        assert _normwise(result["grad_bias"], case["grad_bias"]) < 1e-11


def test_backward_layer_norm_gradient_invariants():
    # sum_i g_LN,i = 0 and sum_i g_LN,i * xhat_i = H * rstd^3 * eps * mean(q * xhat)
    # (zero when eps = 0); a dropped term of the formula breaks one of them.
    rng = np.random.default_rng(5)
    hidden = 768
    u = rng.standard_normal((7, hidden))
    gy = rng.standard_normal((7, hidden))
    weight = rng.standard_normal(hidden)
    for eps in (0.0, 1e-5, 0.5):
        result = oracle.backward(None, gy, u, weight, eps)
        grad_ln, xhat = result["grad_ln"], result["xhat"]
        scale = np.abs(grad_ln).max() * hidden
        centered = u - u.mean(axis=-1, keepdims=True)
        rstd = 1.0 / np.sqrt((centered ** 2).mean(axis=-1) + eps)
        mean_qx = (gy * weight * centered * rstd[:, None]).mean(axis=-1)
        expected = hidden * rstd ** 3 * eps * mean_qx
        assert np.abs(grad_ln.sum(axis=-1)).max() < 1e-12 * scale
        assert np.abs((grad_ln * xhat).sum(axis=-1) - expected).max() < 1e-12 * scale


def test_backward_matches_finite_differences():
    rng = np.random.default_rng(8)
    rows, hidden, eps = 2, 64, 1e-5
    x = rng.standard_normal((rows, hidden))
    d = rng.standard_normal((rows, hidden))
    w = rng.standard_normal(hidden)
    b = rng.standard_normal(hidden)
    gu = rng.standard_normal((rows, hidden))
    gy = rng.standard_normal((rows, hidden))
    keep = rng.random((rows, hidden)) > 0.2
    scale = 1.25

    def loss(xv, dv, wv, bv):
        u = xv + dv * keep * scale
        _, _, y = oracle.layer_norm_forward(u, wv, bv, eps)
        return float((gu * u).sum() + (gy * y).sum())

    u = x + d * keep * scale
    result = oracle.backward(gu, gy, u, w, eps, keep=keep, scale=scale)
    step = 1e-6
    for name, value, expected in (
        ("x", x, result["grad_x"]),
        ("branch", d, result["grad_branch"]),
        ("weight", w, result["grad_weight"]),
        ("bias", b, result["grad_bias"]),
    ):
        flat = value.reshape(-1)
        for index in rng.choice(flat.size, size=6, replace=False):
            original = flat[index]
            flat[index] = original + step
            plus = loss(x, d, w, b)
            flat[index] = original - step
            minus = loss(x, d, w, b)
            flat[index] = original
            numeric = (plus - minus) / (2 * step)
            assert abs(numeric - expected.reshape(-1)[index]) < 1e-5 * max(1.0, abs(numeric)), name


@pytest.mark.parametrize("torch_dtype,rounding", [(torch.bfloat16, oracle.round_to_bfloat16),
                                                  (torch.float16, oracle.round_to_float16)])
def test_half_precision_rounding_matches_torch(torch_dtype, rounding):
    generator = torch.Generator().manual_seed(5)
    random = torch.randn(100000, generator=generator) * torch.logspace(-40, 38, 100000)
    info = torch.finfo(torch_dtype)
    special = torch.tensor([
        0.0, -0.0, 1.0, -1.0, float("inf"), float("-inf"),
        1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, 1.0 + 2.0 ** -12, 1.0 + 3 * 2.0 ** -12,  # ties
        info.max, float(info.max) * 1.0001, float(info.tiny) / 3, 1e-45, 3.4e38,
    ])
    values = torch.cat([random, special]).float()
    expected = values.to(torch_dtype).float().numpy()
    actual = rounding(values.numpy())
    assert np.array_equal(actual.view(np.uint32), expected.view(np.uint32))
    nan = rounding(np.array([np.nan], np.float32))
    assert np.isnan(nan).all()


def test_special_values_follow_the_reference_products():
    """The oracle gives infinities and NaNs the reference's arithmetic gives
    them. The dropped branch has known answers from IEEE 754: inf * 0 is NaN,
    and 65504 (the largest fp16) times 1/(1 - 0.1) rounds to inf in fp16. The
    LayerNorm and its gradient match torch's float64 F.layer_norm and
    autograd: a row holding an inf or a NaN is NaN in every column, an inf or a
    NaN upstream gradient makes every input gradient of its row non-finite, and
    it reaches the weight/bias sums in its own column only."""
    _, scale, _ = oracle.dropout_constants(0.1)
    branch = np.array([np.inf, -np.inf, np.nan, 65504.0, 1.0, np.inf], np.float16)
    keep = np.array([False, True, False, True, False, True])
    with np.errstate(all="ignore"):
        dropped = oracle.dropped_branch(branch, keep, scale, "f16")
    expected = np.array([np.nan, -np.inf, np.nan, np.inf, 0.0, np.inf], np.float32)
    assert np.array_equal(dropped, expected, equal_nan=True)

    generator = torch.Generator().manual_seed(11)
    hidden = 64

    def randn(*shape):
        return torch.randn(*shape, generator=generator, dtype=torch.float64)

    u = randn(3, hidden)
    u[0, 5] = float("inf")
    u[1, 9] = float("nan")
    weight, bias = 1.0 + 0.02 * randn(hidden), 0.02 * randn(hidden)
    with np.errstate(all="ignore"):
        mean, rstd, normalized = oracle.layer_norm_forward(u.numpy(), weight.numpy(),
                                                           bias.numpy(), 1e-5)
    reference = torch.nn.functional.layer_norm(u, (hidden,), weight, bias, 1e-5)
    assert np.isnan(normalized[:2]).all() and torch.isnan(reference[:2]).all()
    assert np.allclose(normalized[2], reference[2].numpy(), rtol=0, atol=1e-12)
    assert mean[0] == np.inf and np.isnan(mean[1]) and np.isnan(rstd[:2]).all()

    u = randn(3, hidden)
    grad_updated, grad_normalized = randn(3, hidden), randn(3, hidden)
    grad_normalized[0, 7] = float("inf")
    grad_normalized[1, 11] = float("nan")
    with np.errstate(all="ignore"):
        got = oracle.backward(grad_updated.numpy(), grad_normalized.numpy(), u.numpy(),
                              weight.numpy(), 1e-5)
    leaves = [t.clone().requires_grad_(True) for t in (u, weight, bias)]
    out = torch.nn.functional.layer_norm(leaves[0], (hidden,), leaves[1], leaves[2], 1e-5)
    torch.autograd.backward((out, leaves[0]), (grad_normalized, grad_updated))
    grad_x, grad_weight, grad_bias = (t.grad.numpy() for t in leaves)
    for row in (0, 1):
        assert not np.isfinite(got["grad_x"][row]).any() and not np.isfinite(grad_x[row]).any()
    assert np.allclose(got["grad_x"][2], grad_x[2], rtol=0, atol=1e-12)
    for mine, torchs in ((got["grad_weight"], grad_weight), (got["grad_bias"], grad_bias)):
        assert np.array_equal(mine[[7, 11]], torchs[[7, 11]], equal_nan=True)
        assert np.isinf(mine[7]) and np.isnan(mine[11])
        others = np.ones(hidden, dtype=bool)
        others[[7, 11]] = False
        assert np.allclose(mine[others], torchs[others], rtol=0, atol=1e-12)
    assert got["grad_bias"][7] == np.inf


def test_dropped_bfloat16_branch_rounds_fp32_product_once():
    branch = oracle.round_to_bfloat16(np.array([1.0, 0.3, -2.7, 1e-3], np.float32))
    keep = np.array([True, True, False, True])
    _, scale, _ = oracle.dropout_constants(0.1)
    product = branch * keep.astype(np.float32) * scale
    expected = torch.from_numpy(product).to(torch.bfloat16).float().numpy()
    got = oracle.dropped_branch(branch, keep, scale, "bf16")
    assert np.array_equal(got, expected)
