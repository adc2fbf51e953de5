// PyTorch glue for the MI355X residual LayerNorm C ABI (include/rln.h).
//
// Module `gfx1010_kernels._C`, with the three entry points of the reference's
// binding (csrc/residual_layer_norm_bindings.cpp:131-141):
//   residual_layer_norm(...)           autograd op returning [updated, normalized]
//   residual_layer_norm_forward(...)   (updated, normalized, mean, rstd, mask)
//   residual_layer_norm_backward(...)  [grad_x, grad_branch, grad_w, grad_b]
// Argument order, return layout and error messages follow
// csrc/residual_layer_norm.h:10-42 and the input checks at
// csrc/residual_layer_norm_kernel.hip:26-166. Two optional trailing keyword
// arguments extend them: `normalized_dtype` (forward; float32, float16 or
// bfloat16 normalized output) and `branch_dtype` (backward; names a bfloat16
// branch, which the reference's `branch_is_half` flag cannot express). The
// reference's launch hints (threads, block_rows, parameter_threads,
// parameter_groups) are validated with the reference's messages; the MI355X
// library picks its own launch shape. `threads` keeps one meaning: on the
// reference's hidden sizes (128-1024) dropout draws the reference's hipRAND
// stream of a `threads`-wide launch, so the masks equal the reference's for
// the same generator state; other hidden sizes, which the reference does not
// run natively, use the library's own stream layout.
//
// This file owns what the C ABI leaves to the caller: tensor allocation on
// the caching allocator, the device guard, the current HIP stream, the
// deterministic-algorithms switch and the Philox (seed, offset) reservation
// from the default HIP generator under its mutex.

#include <torch/extension.h>
#include <torch/csrc/autograd/custom_function.h>

#include <ATen/Context.h>
#include <ATen/core/Generator.h>
#include <ATen/hip/HIPGeneratorImpl.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>

#include <cstring>
#include <mutex>
#include <optional>
#include <tuple>
#include <vector>

#include "rln.h"

namespace {

bool native_hidden(int64_t hidden) {
    return rln_hidden_supported(hidden) != 0;
}

bool supported_dtype(at::ScalarType type) {
    return type == at::kFloat || type == at::kHalf || type == at::kBFloat16;
}

void check_status(int status) {
    TORCH_CHECK(status == RLN_OK, rln_last_error());
}

void check_forward_inputs(
    const at::Tensor& x,
    const at::Tensor& branch,
    const at::Tensor& weight,
    const at::Tensor& bias,
    double dropout_p,
    double eps,
    int64_t threads) {
    TORCH_CHECK(x.is_cuda(), "x must be a HIP tensor");
    TORCH_CHECK(
        branch.is_cuda() && weight.is_cuda() && bias.is_cuda(),
        "branch, weight and bias must be HIP tensors");
    TORCH_CHECK(
        x.device() == branch.device() && x.device() == weight.device()
            && x.device() == bias.device(),
        "all tensors must be on the same HIP device");
    TORCH_CHECK(x.scalar_type() == at::kFloat, "x must use float32");
    TORCH_CHECK(
        branch.scalar_type() == at::kHalf || branch.scalar_type() == at::kBFloat16
            || branch.scalar_type() == at::kFloat,
        "branch must use float16, bfloat16 or float32");
    TORCH_CHECK(
        weight.scalar_type() == at::kFloat && bias.scalar_type() == at::kFloat,
        "weight and bias must use float32");
    TORCH_CHECK(x.dim() >= 2, "x must have at least two dimensions");
    TORCH_CHECK(branch.sizes() == x.sizes(), "branch must match x");
    const int64_t hidden = x.size(-1);
    TORCH_CHECK(
        weight.sizes() == at::IntArrayRef({hidden}) && bias.sizes() == at::IntArrayRef({hidden}),
        "weight and bias must match the hidden size");
    TORCH_CHECK(
        x.is_contiguous() && branch.is_contiguous() && weight.is_contiguous()
            && bias.is_contiguous(),
        "all tensors must be contiguous");
    TORCH_CHECK(x.numel() > 0, "empty tensors are unsupported");
    TORCH_CHECK(native_hidden(hidden), "unsupported native hidden size: ", hidden);
    TORCH_CHECK(
        threads == 128 || threads == 192 || threads == 256,
        "threads must be 128, 192 or 256");
    TORCH_CHECK(dropout_p >= 0.0 && dropout_p < 1.0, "dropout_p must be in [0, 1)");
    TORCH_CHECK(eps > 0.0, "eps must be positive");
}

void check_backward_inputs(
    const std::optional<at::Tensor>& grad_updated,
    const std::optional<at::Tensor>& grad_normalized,
    const at::Tensor& updated,
    const at::Tensor& weight,
    const at::Tensor& mean,
    const at::Tensor& rstd,
    const at::Tensor& dropout_mask,
    double dropout_p,
    bool training,
    int64_t threads,
    int64_t block_rows,
    int64_t parameter_threads,
    int64_t parameter_groups) {
    TORCH_CHECK(updated.is_cuda(), "updated must be a HIP tensor");
    const auto device = updated.device();
    const bool same_device = (!grad_updated || grad_updated->device() == device)
        && (!grad_normalized || grad_normalized->device() == device)
        && weight.device() == device && mean.device() == device && rstd.device() == device;
    TORCH_CHECK(same_device, "all backward tensors must be on the same HIP device");
    const bool float32 = (!grad_updated || grad_updated->scalar_type() == at::kFloat)
        && updated.scalar_type() == at::kFloat && weight.scalar_type() == at::kFloat
        && mean.scalar_type() == at::kFloat && rstd.scalar_type() == at::kFloat;
    TORCH_CHECK(float32, "all backward tensors must use float32");
    TORCH_CHECK(
        !grad_normalized || supported_dtype(grad_normalized->scalar_type()),
        "grad_normalized must use float32, float16 or bfloat16");
    TORCH_CHECK(updated.dim() >= 2, "updated must have at least two dimensions");
    TORCH_CHECK(updated.numel() > 0, "empty tensors are unsupported");
    TORCH_CHECK(
        (!grad_updated || grad_updated->sizes() == updated.sizes())
            && (!grad_normalized || grad_normalized->sizes() == updated.sizes()),
        "output gradients must match updated");
    const int64_t hidden = updated.size(-1);
    TORCH_CHECK(native_hidden(hidden), "unsupported native hidden size: ", hidden);
    const int64_t rows = updated.numel() / hidden;
    TORCH_CHECK(weight.sizes() == at::IntArrayRef({hidden}), "weight must match the hidden size");
    TORCH_CHECK(
        mean.numel() == rows && rstd.numel() == rows,
        "mean and rstd must match the row count");
    TORCH_CHECK(
        (!grad_updated || grad_updated->is_contiguous())
            && (!grad_normalized || grad_normalized->is_contiguous())
            && updated.is_contiguous() && weight.is_contiguous() && mean.is_contiguous()
            && rstd.is_contiguous(),
        "all backward tensors must be contiguous");
    TORCH_CHECK(
        threads == 128 || threads == 192 || threads == 256,
        "threads must be 128, 192 or 256");
    TORCH_CHECK(
        block_rows == 16 || block_rows == 32 || block_rows == 64 || block_rows == 128,
        "block_rows must be 16, 32, 64 or 128");
    TORCH_CHECK(
        parameter_threads == 64 || parameter_threads == 128 || parameter_threads == 256,
        "parameter_threads must be 64, 128 or 256");
    TORCH_CHECK(
        parameter_groups > 0 && parameter_groups <= rows,
        "parameter_groups must be in [1, row_count]");
    TORCH_CHECK(dropout_p >= 0.0 && dropout_p < 1.0, "dropout_p must be in [0, 1)");
    if (training && dropout_p > 0.0) {
        TORCH_CHECK(
            dropout_mask.is_cuda() && dropout_mask.device() == device,
            "dropout_mask must be on the same HIP device");
        TORCH_CHECK(
            dropout_mask.scalar_type() == at::kInt && dropout_mask.is_contiguous(),
            "dropout_mask must be a contiguous int32 tensor");
        TORCH_CHECK(
            dropout_mask.numel() == rln_mask_words(rows, hidden),
            "dropout_mask has the wrong size");
    }
}

// The dropout layout for `threads` (rln_philox_t::threads): the reference's
// where it exists for this hidden size, else the library's own (0).
int64_t layout_threads(int64_t hidden, int64_t threads) {
    return rln_philox_increment(hidden, threads) != 0 ? threads : 0;
}

// Reserves rln_philox_increment() offset units from the device's default
// generator (the reference does the same at
// csrc/residual_layer_norm_kernel.hip:1762-1779). Under HIP graph capture the
// generator hands out device pointers that the kernel reads at replay time,
// so captured graphs draw fresh masks on every replay.
rln_philox_t reserve_philox(const at::Tensor& x, int64_t hidden, int64_t threads) {
    const uint64_t increment = rln_philox_increment(hidden, threads);
    check_status(increment != 0 ? RLN_OK : RLN_ERR_INVALID);
    auto generator = at::cuda::detail::getDefaultCUDAGenerator(x.device().index());
    at::PhiloxCudaState state;
    {
        std::lock_guard<std::mutex> lock(generator.mutex());
        state = generator.get<at::CUDAGeneratorImpl>()->philox_cuda_state(increment);
    }
    rln_philox_t philox{};
    philox.threads = threads;
    if (state.captured_) {
        philox.seed_ptr = state.seed_.ptr;
        philox.offset_ptr = state.offset_.ptr;
        philox.offset = state.offset_intragraph_;
    } else {
        philox.seed = state.seed_.val;
        philox.offset = state.offset_.val;
    }
    return philox;
}

int dtype_of(at::ScalarType type) {
    if (type == at::kHalf) {
        return RLN_DTYPE_F16;
    }
    if (type == at::kBFloat16) {
        return RLN_DTYPE_BF16;
    }
    return RLN_DTYPE_F32;
}

// Row statistics and dropout mask of one forward call kept in a single
// allocation (the autograd path, which never returns them): mean at element 0,
// rstd at `rstd_offset`, the mask words at `mask_offset`, each 256-byte
// aligned. Saves two caching-allocator calls per forward.
struct RowStatsLayout {
    int64_t rows;
    int64_t mask_words;
    int64_t rstd_offset;
    int64_t mask_offset;
    int64_t elements;
};

RowStatsLayout row_stats_layout(int64_t rows, int64_t hidden, bool dropout) {
    const auto aligned = [](int64_t count) { return (count + 63) / 64 * 64; };
    RowStatsLayout layout{};
    layout.rows = rows;
    layout.mask_words = dropout ? rln_mask_words(rows, hidden) : 0;
    layout.rstd_offset = aligned(rows);
    layout.mask_offset = layout.rstd_offset + aligned(rows);
    layout.elements = layout.mask_offset + layout.mask_words;
    return layout;
}

// A contiguous 1-D tensor of `count` elements of `type` at element `offset`
// of `base`'s storage, built without a dispatcher call.
at::Tensor storage_slice(const at::Tensor& base, int64_t offset, int64_t count,
                         caffe2::TypeMeta type) {
    auto slice = at::detail::make_tensor<c10::TensorImpl>(
        c10::Storage(base.storage()), base.key_set(), type);
    slice.unsafeGetTensorImpl()->set_sizes_contiguous({count});
    slice.unsafeGetTensorImpl()->set_storage_offset(offset);
    return slice;
}

// `row_stats`: when given, mean, rstd and mask live in one float32 tensor
// stored there (row_stats_layout) and the returned mean/rstd/mask are
// undefined; otherwise they are three separate tensors.
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor> forward_impl(
    const at::Tensor& x,
    const at::Tensor& branch,
    const at::Tensor& weight,
    const at::Tensor& bias,
    double dropout_p,
    double eps,
    bool training,
    int64_t threads,
    std::optional<at::ScalarType> normalized_dtype,
    at::Tensor* zeroed_grad_weight = nullptr,
    at::Tensor* zeroed_grad_bias = nullptr,
    at::Tensor* row_stats = nullptr) {
    check_forward_inputs(x, branch, weight, bias, dropout_p, eps, threads);
    const at::ScalarType output_type = normalized_dtype.value_or(at::kFloat);
    TORCH_CHECK(supported_dtype(output_type),
                "normalized_dtype must be float32, float16 or bfloat16");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    const int64_t hidden = x.size(-1);
    const int64_t rows = x.numel() / hidden;
    const bool dropout = training && dropout_p > 0.0;
    auto updated = at::empty_like(x);
    auto normalized = at::empty_like(x, x.options().dtype(output_type));
    at::Tensor mean;
    at::Tensor rstd;
    at::Tensor mask;
    float* mean_ptr = nullptr;
    float* rstd_ptr = nullptr;
    uint32_t* mask_ptr = nullptr;
    if (row_stats != nullptr) {
        const RowStatsLayout layout = row_stats_layout(rows, hidden, dropout);
        *row_stats = at::empty({layout.elements}, x.options());
        float* base = row_stats->data_ptr<float>();
        mean_ptr = base;
        rstd_ptr = base + layout.rstd_offset;
        mask_ptr = dropout ? reinterpret_cast<uint32_t*>(base + layout.mask_offset) : nullptr;
    } else {
        mean = at::empty({rows}, x.options());
        rstd = at::empty({rows}, x.options());
        mask = at::empty({dropout ? rln_mask_words(rows, hidden) : 0},
                         x.options().dtype(at::kInt));
        mean_ptr = mean.data_ptr<float>();
        rstd_ptr = rstd.data_ptr<float>();
        mask_ptr = dropout ? reinterpret_cast<uint32_t*>(mask.data_ptr<int32_t>()) : nullptr;
    }
    rln_philox_t philox{};
    if (dropout) {
        philox = reserve_philox(x, hidden, layout_threads(hidden, threads));
    }
    // Optional weight/bias gradient sums for the backward of this call,
    // zeroed by the forward launch itself.
    const bool zero_sums = zeroed_grad_weight != nullptr && zeroed_grad_bias != nullptr;
    if (zero_sums) {
        *zeroed_grad_weight = at::empty({hidden}, x.options());
        *zeroed_grad_bias = at::empty({hidden}, x.options());
    }
    const auto stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(x.device().index()).stream();
    check_status(rln_forward(
        x.data_ptr<float>(),
        branch.data_ptr(),
        dtype_of(branch.scalar_type()),
        weight.data_ptr<float>(),
        bias.data_ptr<float>(),
        updated.data_ptr<float>(),
        normalized.data_ptr(),
        dtype_of(output_type),
        mean_ptr,
        rstd_ptr,
        mask_ptr,
        zero_sums ? zeroed_grad_weight->data_ptr<float>() : nullptr,
        zero_sums ? zeroed_grad_bias->data_ptr<float>() : nullptr,
        rows,
        hidden,
        dropout_p,
        eps,
        training ? 1 : 0,
        dropout ? &philox : nullptr,
        stream));
    return {updated, normalized, mean, rstd, mask};
}

std::vector<at::Tensor> backward_impl(
    const std::optional<at::Tensor>& grad_updated_in,
    const std::optional<at::Tensor>& grad_normalized_in,
    const at::Tensor& updated,
    const at::Tensor& weight,
    const at::Tensor& mean,
    const at::Tensor& rstd,
    const at::Tensor& dropout_mask,
    double dropout_p,
    bool training,
    bool branch_is_half,
    int64_t threads,
    int64_t block_rows,
    int64_t parameter_threads,
    int64_t parameter_groups,
    bool compute_parameter_gradients,
    std::optional<at::ScalarType> branch_dtype,
    const at::Tensor* zeroed_grad_weight = nullptr,
    const at::Tensor* zeroed_grad_bias = nullptr) {
    // Undefined tensors arrive from autograd as nullopt-equivalents.
    std::optional<at::Tensor> grad_updated;
    std::optional<at::Tensor> grad_normalized;
    if (grad_updated_in && grad_updated_in->defined()) {
        grad_updated = grad_updated_in;
    }
    if (grad_normalized_in && grad_normalized_in->defined()) {
        grad_normalized = grad_normalized_in;
    }
    check_backward_inputs(
        grad_updated,
        grad_normalized,
        updated,
        weight,
        mean,
        rstd,
        dropout_mask,
        dropout_p,
        training,
        threads,
        block_rows,
        parameter_threads,
        parameter_groups);
    c10::hip::HIPGuardMasqueradingAsCUDA guard(updated.device());
    const int64_t hidden = updated.size(-1);
    const int64_t rows = updated.numel() / hidden;
    const bool dropout = training && dropout_p > 0.0;
    const bool deterministic = at::globalContext().deterministicAlgorithms();
    // The reference passes only `branch_is_half`; `branch_dtype`, when given,
    // names the branch type exactly (bfloat16 included).
    const at::ScalarType branch_type =
        branch_dtype.value_or(branch_is_half ? at::kHalf : at::kFloat);
    TORCH_CHECK(supported_dtype(branch_type), "branch_dtype must be float32, float16 or bfloat16");
    auto grad_x = at::empty_like(updated);
    auto grad_branch = at::empty(updated.sizes(), updated.options().dtype(branch_type));
    at::Tensor grad_weight;
    at::Tensor grad_bias;
    at::Tensor workspace;
    const bool launch_parameters = compute_parameter_gradients && grad_normalized.has_value();
    // Sums the forward already zeroed: accumulate into them, no zeroing launch.
    const bool zeroed = zeroed_grad_weight != nullptr && zeroed_grad_bias != nullptr
        && zeroed_grad_weight->defined() && zeroed_grad_bias->defined();
    if (compute_parameter_gradients) {
        // Without grad_normalized the parameter gradients are exactly zero.
        // Two separate tensors (not views of one), so that no two returned
        // gradients alias each other.
        if (zeroed) {
            grad_weight = *zeroed_grad_weight;
            grad_bias = *zeroed_grad_bias;
        } else {
            grad_weight = launch_parameters ? at::empty({hidden}, updated.options())
                                            : at::zeros({hidden}, updated.options());
            grad_bias = launch_parameters ? at::empty({hidden}, updated.options())
                                          : at::zeros({hidden}, updated.options());
        }
    }
    if (launch_parameters) {
        const size_t bytes = rln_backward_workspace_bytes(rows, hidden, deterministic ? 1 : 0);
        if (bytes > 0) {
            workspace = at::empty(
                {static_cast<int64_t>(bytes / sizeof(float))},
                updated.options());
        }
    }
    const auto stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(updated.device().index()).stream();
    check_status(rln_backward(
        grad_updated ? grad_updated->data_ptr<float>() : nullptr,
        grad_normalized ? grad_normalized->data_ptr() : nullptr,
        grad_normalized ? dtype_of(grad_normalized->scalar_type()) : RLN_DTYPE_F32,
        updated.data_ptr<float>(),
        weight.data_ptr<float>(),
        mean.data_ptr<float>(),
        rstd.data_ptr<float>(),
        dropout ? reinterpret_cast<const uint32_t*>(dropout_mask.data_ptr<int32_t>()) : nullptr,
        grad_x.data_ptr<float>(),
        grad_branch.data_ptr(),
        dtype_of(branch_type),
        launch_parameters ? grad_weight.data_ptr<float>() : nullptr,
        launch_parameters ? grad_bias.data_ptr<float>() : nullptr,
        rows,
        hidden,
        dropout_p,
        training ? 1 : 0,
        deterministic ? 1 : 0,
        zeroed ? 1 : 0,
        workspace.defined() ? workspace.data_ptr() : nullptr,
        workspace.defined() ? static_cast<size_t>(workspace.numel()) * sizeof(float) : 0,
        stream));
    return {grad_x, grad_branch, grad_weight, grad_bias};
}

// Autograd contract of csrc/residual_layer_norm_bindings.cpp:10-98: saves
// updated, weight, mean, rstd and mask (the last three in one row-statistics
// tensor), does not materialize missing output gradients, and returns
// weight/bias gradients only when `normalized` received a gradient (and, here,
// only when the backward pass needs one of them; the reference computes them
// whenever `normalized` has a gradient). Missing
// gradients are passed to the kernel as null pointers instead of materialized
// zeros. The forward's host cost is kept low on purpose (three allocations
// and two more for the gradient sums, one saved_data entry): small calls are
// bound by it.
class ResidualLayerNormFunction : public torch::autograd::Function<ResidualLayerNormFunction> {
 public:
    static torch::autograd::variable_list forward(
        torch::autograd::AutogradContext* ctx,
        torch::autograd::Variable x,
        torch::autograd::Variable branch,
        torch::autograd::Variable weight,
        torch::autograd::Variable bias,
        double dropout_p,
        double eps,
        bool training,
        int64_t threads,
        int64_t block_rows,
        int64_t parameter_threads,
        int64_t parameter_groups,
        std::optional<at::ScalarType> normalized_dtype) {
        // The first backward of this call accumulates the weight/bias
        // gradients into sums the forward launch zeroes (one launch fewer per
        // training step); a repeated backward (retain_graph) allocates anew.
        at::Tensor grad_weight_sum;
        at::Tensor grad_bias_sum;
        at::Tensor row_stats;
        const bool parameters = weight.requires_grad() || bias.requires_grad();
        auto result = forward_impl(
            x, branch, weight, bias, dropout_p, eps, training, threads, normalized_dtype,
            parameters ? &grad_weight_sum : nullptr, parameters ? &grad_bias_sum : nullptr,
            &row_stats);
        auto updated = std::get<0>(result);
        auto normalized = std::get<1>(result);
        ctx->save_for_backward({updated, weight, row_stats, grad_weight_sum, grad_bias_sum});
        ctx->set_materialize_grads(false);
        // The scalars the backward needs, dropout_p as its bit pattern, in one
        // entry (each saved_data entry costs a hash-map insertion per call).
        int64_t dropout_bits = 0;
        std::memcpy(&dropout_bits, &dropout_p, sizeof(dropout_bits));
        ctx->saved_data["state"] = std::vector<int64_t>{
            training ? 1 : 0, static_cast<int64_t>(branch.scalar_type()), threads, block_rows,
            parameter_threads, parameter_groups, dropout_bits};
        return {updated, normalized};
    }

    static torch::autograd::variable_list backward(
        torch::autograd::AutogradContext* ctx,
        torch::autograd::variable_list grad_outputs) {
        auto saved = ctx->get_saved_variables();
        std::optional<at::Tensor> grad_updated;
        std::optional<at::Tensor> grad_normalized;
        if (grad_outputs[0].defined()) {
            grad_updated = grad_outputs[0].contiguous();
        }
        if (grad_outputs[1].defined()) {
            grad_normalized = grad_outputs[1].contiguous();
        }
        const bool has_grad_normalized = grad_normalized.has_value();
        if (!grad_updated && !has_grad_normalized) {
            return {
                at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor(),
                at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor()};
        }
        // The weight/bias sums only when this backward pass asks for them
        // (edges 2 and 3): frozen parameters, or torch.autograd.grad over the
        // inputs alone, skip their reduction entirely.
        const bool parameter_gradients = has_grad_normalized
            && (ctx->needs_input_grad(2) || ctx->needs_input_grad(3));
        // Sums zeroed by the forward serve the first backward that computes them.
        at::Tensor grad_weight_sum;
        at::Tensor grad_bias_sum;
        if (parameter_gradients && ctx->saved_data.find("sums_used") == ctx->saved_data.end()) {
            grad_weight_sum = saved[3];
            grad_bias_sum = saved[4];
            ctx->saved_data["sums_used"] = true;
        }
        const std::vector<int64_t> state = ctx->saved_data["state"].toIntVector();
        const auto branch_dtype = static_cast<at::ScalarType>(state[1]);
        const bool training = state[0] != 0;
        double dropout_p = 0.0;
        std::memcpy(&dropout_p, &state[6], sizeof(dropout_p));
        const at::Tensor& updated = saved[0];
        const int64_t hidden = updated.size(-1);
        const RowStatsLayout layout =
            row_stats_layout(updated.numel() / hidden, hidden, training && dropout_p > 0.0);
        const auto f32 = caffe2::TypeMeta::Make<float>();
        auto gradients = backward_impl(
            grad_updated,
            grad_normalized,
            updated,
            saved[1],
            storage_slice(saved[2], 0, layout.rows, f32),
            storage_slice(saved[2], layout.rstd_offset, layout.rows, f32),
            storage_slice(saved[2], layout.mask_offset, layout.mask_words,
                          caffe2::TypeMeta::Make<int32_t>()),
            dropout_p,
            training,
            branch_dtype == at::kHalf,
            state[2],
            state[3],
            state[4],
            state[5],
            parameter_gradients,
            branch_dtype,
            &grad_weight_sum,
            &grad_bias_sum);
        return {
            gradients[0],
            gradients[1],
            parameter_gradients ? gradients[2] : at::Tensor(),
            parameter_gradients ? gradients[3] : at::Tensor(),
            at::Tensor(),
            at::Tensor(),
            at::Tensor(),
            at::Tensor(),
            at::Tensor(),
            at::Tensor(),
            at::Tensor(),
            at::Tensor(),
        };
    }
};

torch::autograd::variable_list residual_layer_norm_autograd(
    const at::Tensor& x,
    const at::Tensor& branch,
    const at::Tensor& weight,
    const at::Tensor& bias,
    double dropout_p,
    double eps,
    bool training,
    int64_t threads,
    int64_t block_rows,
    int64_t parameter_threads,
    int64_t parameter_groups,
    std::optional<at::ScalarType> normalized_dtype) {
    // Nothing to record (grad mode off, as under torch.no_grad() and
    // inference_mode, or no input requires grad): the forward alone, without
    // the autograd node, its saved state and the gradient sums. Small calls,
    // such as the decode steps of a served model, are bound by this host cost.
    if (!at::GradMode::is_enabled()
        || !(x.requires_grad() || branch.requires_grad() || weight.requires_grad()
             || bias.requires_grad())) {
        at::Tensor row_stats;
        auto result = forward_impl(x, branch, weight, bias, dropout_p, eps, training, threads,
                                   normalized_dtype, nullptr, nullptr, &row_stats);
        return {std::get<0>(result), std::get<1>(result)};
    }
    return ResidualLayerNormFunction::apply(
        x,
        branch,
        weight,
        bias,
        dropout_p,
        eps,
        training,
        threads,
        block_rows,
        parameter_threads,
        parameter_groups,
        normalized_dtype);
}

// True when the fused kernels serve these inputs: the conditions under which
// the Python `_input_reason` (the reference's gfx1010_kernels/normalization.py:97-132,
// widened to this library's sizes and dtypes) finds no reason and the hidden
// size is native. One C++ call instead of ~20 Python attribute reads; the
// reason itself is only worked out, in Python, when this is false.
bool fused_inputs_supported(const at::Tensor& x, const at::Tensor& branch,
                            const at::Tensor& weight, const at::Tensor& bias, double dropout_p,
                            double eps) {
    if (!x.is_cuda() || !branch.is_cuda() || !weight.is_cuda() || !bias.is_cuda()) {
        return false;
    }
    const auto device = x.device();
    if (branch.device() != device || weight.device() != device || bias.device() != device) {
        return false;
    }
    if (x.dim() < 2 || branch.sizes() != x.sizes()) {
        return false;
    }
    const int64_t hidden = x.size(-1);
    // Native sizes are multiples of 64 from 128 up: within the Python range
    // and divisible by 8.
    if (!native_hidden(hidden) || weight.sizes() != at::IntArrayRef({hidden})
        || bias.sizes() != at::IntArrayRef({hidden})) {
        return false;
    }
    if (x.scalar_type() != at::kFloat || !supported_dtype(branch.scalar_type())
        || weight.scalar_type() != at::kFloat || bias.scalar_type() != at::kFloat) {
        return false;
    }
    if (!(x.is_contiguous() && branch.is_contiguous() && weight.is_contiguous()
          && bias.is_contiguous())) {
        return false;
    }
    // The Python comparisons exactly (`not 0 <= p < 1`, `eps <= 0`), NaN
    // included: a NaN eps has no reason there, and the op itself rejects it.
    return dropout_p >= 0.0 && dropout_p < 1.0 && !(eps <= 0.0) && x.numel() > 0;
}

// `residual_layer_norm` for inputs the fused kernels serve, else None (no
// exception): the auto path's common case in one call.
std::optional<torch::autograd::variable_list> residual_layer_norm_if_supported(
    const at::Tensor& x,
    const at::Tensor& branch,
    const at::Tensor& weight,
    const at::Tensor& bias,
    double dropout_p,
    double eps,
    bool training,
    int64_t threads,
    int64_t block_rows,
    int64_t parameter_threads,
    int64_t parameter_groups,
    std::optional<at::ScalarType> normalized_dtype) {
    if (!fused_inputs_supported(x, branch, weight, bias, dropout_p, eps)) {
        return std::nullopt;
    }
    return residual_layer_norm_autograd(x, branch, weight, bias, dropout_p, eps, training,
                                        threads, block_rows, parameter_threads,
                                        parameter_groups, normalized_dtype);
}

}  // namespace

PYBIND11_MODULE(_C, module) {
    module.doc() = "MI355X (gfx950) fused residual + dropout + LayerNorm";
    module.def(
        "residual_layer_norm",
        &residual_layer_norm_autograd,
        pybind11::arg("x"),
        pybind11::arg("branch"),
        pybind11::arg("weight"),
        pybind11::arg("bias"),
        pybind11::arg("dropout_p"),
        pybind11::arg("eps"),
        pybind11::arg("training"),
        pybind11::arg("threads"),
        pybind11::arg("block_rows"),
        pybind11::arg("parameter_threads"),
        pybind11::arg("parameter_groups"),
        pybind11::arg("normalized_dtype") = pybind11::none());
    module.def("residual_layer_norm_if_supported", &residual_layer_norm_if_supported);
    module.def("fused_inputs_supported", &fused_inputs_supported);
    module.def(
        "residual_layer_norm_forward",
        [](const at::Tensor& x, const at::Tensor& branch, const at::Tensor& weight,
           const at::Tensor& bias, double dropout_p, double eps, bool training, int64_t threads,
           std::optional<at::ScalarType> normalized_dtype) {
            return forward_impl(
                x, branch, weight, bias, dropout_p, eps, training, threads, normalized_dtype);
        },
        pybind11::arg("x"),
        pybind11::arg("branch"),
        pybind11::arg("weight"),
        pybind11::arg("bias"),
        pybind11::arg("dropout_p"),
        pybind11::arg("eps"),
        pybind11::arg("training"),
        pybind11::arg("threads"),
        pybind11::arg("normalized_dtype") = pybind11::none());
    module.def(
        "residual_layer_norm_backward",
        [](const std::optional<at::Tensor>& grad_updated,
           const std::optional<at::Tensor>& grad_normalized, const at::Tensor& updated,
           const at::Tensor& weight, const at::Tensor& mean, const at::Tensor& rstd,
           const at::Tensor& dropout_mask, double dropout_p, bool training, bool branch_is_half,
           int64_t threads, int64_t block_rows, int64_t parameter_threads,
           int64_t parameter_groups, bool compute_parameter_gradients,
           std::optional<at::ScalarType> branch_dtype) {
            return backward_impl(
                grad_updated, grad_normalized, updated, weight, mean, rstd, dropout_mask,
                dropout_p, training, branch_is_half, threads, block_rows, parameter_threads,
                parameter_groups, compute_parameter_gradients, branch_dtype);
        },
        pybind11::arg("grad_updated"),
        pybind11::arg("grad_normalized"),
        pybind11::arg("updated"),
        pybind11::arg("weight"),
        pybind11::arg("mean"),
        pybind11::arg("rstd"),
        pybind11::arg("dropout_mask"),
        pybind11::arg("dropout_p"),
        pybind11::arg("training"),
        pybind11::arg("branch_is_half"),
        pybind11::arg("threads"),
        pybind11::arg("block_rows"),
        pybind11::arg("parameter_threads"),
        pybind11::arg("parameter_groups"),
        pybind11::arg("compute_parameter_gradients"),
        pybind11::arg("branch_dtype") = pybind11::none());
    module.def("target_arch", []() { return std::string(rln_target_arch()); });
    module.def("library_version", []() { return std::string(rln_version()); });
}
