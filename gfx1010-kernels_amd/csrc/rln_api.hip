// C ABI of the MI355X fused residual LayerNorm (include/rln.h): argument
// checks, dropout constants, dispatch to the per-row-shape launchers
// (rln_device.h, instantiated in rln_hidden.hip), and the small kernels that
// zero or reduce the weight/bias gradients.

#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

#include "rln_device.h"

namespace rln {

RLN_FOR_EACH_FIXED(RLN_DECLARE_FIXED)
RLN_DECLARE_STAGGERED_BACKWARD()
RLN_FOR_EACH_WIDE_FORWARD(RLN_DECLARE_WIDE_FORWARD)
RLN_FOR_EACH_WIDE_BACKWARD(RLN_DECLARE_WIDE_BACKWARD)

namespace {

thread_local std::string t_last_error;

}  // namespace

int fail(int code, const char* format, ...) {
    char buffer[512];
    va_list args;
    va_start(args, format);
    vsnprintf(buffer, sizeof(buffer), format, args);
    va_end(args);
    t_last_error = buffer;
    return code;
}

int check_launch(const char* what) {
    const hipError_t status = hipGetLastError();
    if (status != hipSuccess) {
        return fail(
            RLN_ERR_HIP,
            "%s launch failed: %s",
            what,
            hipGetErrorString(status));
    }
    return RLN_OK;
}

namespace {

// Fixed-order reduction of per-block partials [groups][2][H] into
// grad_weight / grad_bias. Block = 16 waves over 64 consecutive entries of the
// flattened [2][H] output; wave k sums its contiguous share of the groups in
// ascending order, then wave sums are added in ascending wave order.
constexpr int kReduceWaves = 16;

__global__ __launch_bounds__(kReduceWaves * kWaveSize)
void rln_parameter_reduce_kernel(
    const float* __restrict__ partials,
    float* __restrict__ grad_weight,
    float* __restrict__ grad_bias,
    int64_t groups,
    int hidden,
    int accumulate) {
    __shared__ float wave_totals[kReduceWaves][kWaveSize];
    const int lane = threadIdx.x & (kWaveSize - 1);
    const int wave = threadIdx.x / kWaveSize;
    const int entry = blockIdx.x * kWaveSize + lane;  // index into [2][H]
    const bool active = entry < 2 * hidden;
    const int64_t share = (groups + kReduceWaves - 1) / kReduceWaves;
    const int64_t begin = wave * share;
    const int64_t end = begin + share < groups ? begin + share : groups;
    const int which = active ? entry / hidden : 0;
    const int column = active ? entry % hidden : 0;
    float total = 0.0f;
    if (active) {
        const float* source = partials + static_cast<int64_t>(which) * hidden + column;
        const int64_t stride = 2 * static_cast<int64_t>(hidden);
#pragma unroll 16
        for (int64_t group = begin; group < end; ++group) {
            total += source[group * stride];
        }
    }
    wave_totals[wave][lane] = total;
    __syncthreads();
    if (wave == 0 && active) {
        float sum = 0.0f;
#pragma unroll
        for (int source = 0; source < kReduceWaves; ++source) {
            sum += wave_totals[source][lane];
        }
        float* target = (which ? grad_bias : grad_weight) + column;
        *target = accumulate ? *target + sum : sum;
    }
}

__global__ __launch_bounds__(256)
void rln_zero_parameters_kernel(float* __restrict__ grad_weight, float* __restrict__ grad_bias, int hidden) {
    const int index = blockIdx.x * blockDim.x + threadIdx.x;
    if (index < hidden) {
        grad_weight[index] = 0.0f;
        grad_bias[index] = 0.0f;
    }
}

// Compute units of the current device, looked up once per device (0 when
// the runtime cannot say; the forward then keeps its device-independent grid).
int compute_units() {
    constexpr int kMaxDevices = 64;
    static std::once_flag once[kMaxDevices];
    static int units[kMaxDevices];
    int device = -1;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) {
        static_cast<void>(hipGetLastError());  // clear the failed call's error
        return 0;
    }
    std::call_once(once[device], [device] {
        int count = 0;
        if (hipDeviceGetAttribute(&count, hipDeviceAttributeMultiprocessorCount, device)
            != hipSuccess) {
            static_cast<void>(hipGetLastError());  // clear the failed call's error
            count = 0;
        }
        units[device] = count;
    });
    return units[device];
}

bool aligned_to(const void* pointer, uintptr_t alignment) {
    return pointer == nullptr || (reinterpret_cast<uintptr_t>(pointer) & (alignment - 1)) == 0;
}

// Mirrors the reference's conversion of the double probability
// (csrc/residual_layer_norm_kernel.hip:893-899, :1883-1886).
struct DropoutConstants {
    bool active;
    float scale;
    uint32_t threshold;
};

int dropout_constants(double dropout_p, int training, DropoutConstants* out) {
    if (!(dropout_p >= 0.0 && dropout_p < 1.0)) {
        return fail(RLN_ERR_INVALID, "dropout_p must be in [0, 1)");
    }
    const float p = static_cast<float>(dropout_p);
    out->active = training && dropout_p > 0.0;
    if (out->active && !(p < 1.0f)) {
        return fail(RLN_ERR_INVALID, "dropout_p must be in [0, 1)");
    }
    out->scale = out->active ? 1.0f / (1.0f - p) : 1.0f;
    out->threshold = out->active
        ? static_cast<uint32_t>(static_cast<double>(p) * 4294967296.0)
        : 0u;
    return RLN_OK;
}

bool valid_dtype(int dtype) {
    return dtype == RLN_DTYPE_F32 || dtype == RLN_DTYPE_F16 || dtype == RLN_DTYPE_BF16;
}

// Alignment of one four-element vector of `dtype`.
uintptr_t vector_alignment(int dtype) {
    return dtype == RLN_DTYPE_F32 ? 16 : 8;
}

int check_common(int64_t rows, int64_t hidden, int branch_dtype) {
    if (rows <= 0) {
        return fail(RLN_ERR_INVALID, "empty tensors are unsupported");
    }
    if (!hidden_supported(hidden)) {
        return fail(
            RLN_ERR_UNSUPPORTED,
            "unsupported native hidden size: %lld",
            static_cast<long long>(hidden));
    }
    if (!valid_dtype(branch_dtype)) {
        return fail(RLN_ERR_INVALID, "branch must use float16, bfloat16 or float32");
    }
    if (rows > (INT64_MAX / hidden)) {
        return fail(RLN_ERR_INVALID, "rows * hidden overflows int64");
    }
    return RLN_OK;
}

// A non-default stream must belong to the calling thread's current device:
// the launch shapes (the forward's CU count) and rln_backward_noalloc's
// scratch are those of the current device, and the pointers are on it.
int check_stream(void* stream) {
    if (stream == nullptr) {
        return RLN_OK;
    }
    int current = -1;
    hipDevice_t owner = -1;
    const hipError_t got_current = hipGetDevice(&current);
    const hipError_t got_owner = hipStreamGetDevice(static_cast<hipStream_t>(stream), &owner);
    if (got_current != hipSuccess || got_owner != hipSuccess) {
        static_cast<void>(hipGetLastError());  // clear the failed call's error
        return fail(RLN_ERR_INVALID, "stream: cannot tell its device (%s)",
                    hipGetErrorString(got_current != hipSuccess ? got_current : got_owner));
    }
    if (owner != current) {
        return fail(RLN_ERR_INVALID,
                    "stream belongs to device %d but the current device is %d", owner, current);
    }
    return RLN_OK;
}

// The dropout layout `threads` selects: 0 for this library's; 128, 192 or
// 256 for the reference's stream of a launch with that many threads per row
// (reference csrc/residual_layer_norm_kernel.hip:68-72 accepts the same three
// values), which exists for the reference's hidden sizes only and draws at
// most 8 values per thread (its two hiprand4 calls, :449-480).
int check_philox_threads(int64_t hidden, int64_t threads) {
    if (threads == 0) {
        return RLN_OK;
    }
    if (threads != 128 && threads != 192 && threads != 256) {
        return fail(RLN_ERR_INVALID, "threads must be 0, 128, 192 or 256");
    }
    if (!specialized_hidden(hidden) || (hidden + threads - 1) / threads > 8) {
        return fail(RLN_ERR_UNSUPPORTED,
                    "the reference's dropout stream exists for hidden sizes 128, 256, 384, "
                    "512, 768 and 1024 only, not %lld",
                    static_cast<long long>(hidden));
    }
    return RLN_OK;
}

// Whether the parameter gradients of this call go through per-block partials
// (and therefore the workspace and the reduce kernel).
bool uses_partials(int deterministic) {
    return deterministic || !RLN_ATOMIC_PARAMETERS;
}

}  // namespace
}  // namespace rln

using namespace rln;

// ----------------------------------------------------------------------------
// C ABI.

extern "C" {

int rln_forward(
    const float* x,
    const void* branch,
    int branch_dtype,
    const float* weight,
    const float* bias,
    float* updated,
    void* normalized,
    int normalized_dtype,
    float* mean,
    float* rstd,
    uint32_t* dropout_mask,
    float* zero_grad_weight,
    float* zero_grad_bias,
    int64_t rows,
    int64_t hidden,
    double dropout_p,
    double eps,
    int training,
    const rln_philox_t* philox,
    void* stream) {
    rln::t_last_error.clear();
    int status = check_common(rows, hidden, branch_dtype);
    if (status != RLN_OK) {
        return status;
    }
    status = check_stream(stream);
    if (status != RLN_OK) {
        return status;
    }
    if (!valid_dtype(normalized_dtype)) {
        return fail(RLN_ERR_INVALID, "normalized must use float16, bfloat16 or float32");
    }
    if (!x || !branch || !weight || !bias || !updated || !normalized || !mean || !rstd) {
        return fail(RLN_ERR_INVALID, "forward tensors must not be null");
    }
    if (!(eps > 0.0)) {
        return fail(RLN_ERR_INVALID, "eps must be positive");
    }
    if ((zero_grad_weight == nullptr) != (zero_grad_bias == nullptr)) {
        return fail(RLN_ERR_INVALID,
                    "zero_grad_weight and zero_grad_bias must both be given or both be null");
    }
    DropoutConstants drop{};
    status = dropout_constants(dropout_p, training, &drop);
    if (status != RLN_OK) {
        return status;
    }
    ForwardArgs a{};
    a.x = x;
    a.branch = branch;
    a.weight = weight;
    a.bias = bias;
    a.updated = updated;
    a.normalized = normalized;
    a.mean = mean;
    a.rstd = rstd;
    a.mask = dropout_mask;
    a.zero_weight = zero_grad_weight;
    a.zero_bias = zero_grad_bias;
    a.rows = rows;
    a.eps = static_cast<float>(eps);
    a.dropout = drop.active ? 1 : 0;
    a.scale = drop.scale;
    a.threshold = drop.threshold;
    a.stream = static_cast<hipStream_t>(stream);
    if (drop.active) {
        if (!dropout_mask) {
            return fail(RLN_ERR_INVALID, "dropout_mask must not be null when dropout is active");
        }
        if (!philox) {
            return fail(RLN_ERR_INVALID, "philox must not be null when dropout is active");
        }
        status = check_philox_threads(hidden, philox->threads);
        if (status != RLN_OK) {
            return status;
        }
        if (philox->threads != 0 && philox->offset % 4 != 0) {
            return fail(RLN_ERR_INVALID,
                        "the reference's dropout stream needs a Philox offset that is a "
                        "multiple of 4");
        }
        a.philox.seed = philox->seed;
        a.philox.offset = philox->offset;
        a.philox.seed_ptr = philox->seed_ptr;
        a.philox.offset_ptr = philox->offset_ptr;
        a.philox.threads = static_cast<int>(philox->threads);
    }
    a.compute_units = compute_units();
    const bool aligned = aligned_to(x, 16) && aligned_to(weight, 16) && aligned_to(bias, 16)
        && aligned_to(updated, 16)
        && aligned_to(normalized, vector_alignment(normalized_dtype))
        && aligned_to(branch, vector_alignment(branch_dtype));
    return with_shape<Pass::kForward>(hidden, rows, [&](auto shape) {
        return launch_forward_shape(a, shape, branch_dtype, normalized_dtype, aligned);
    });
}

size_t rln_backward_workspace_bytes(int64_t rows, int64_t hidden, int deterministic) {
    if (!uses_partials(deterministic) || rows <= 0 || !hidden_supported(hidden)) {
        return 0;
    }
    return static_cast<size_t>(backward_blocks(rows, hidden)) * 2 * static_cast<size_t>(hidden)
        * sizeof(float);
}

}  // extern "C"

// Scratch of rln_backward_noalloc: the deterministic weight/bias partials,
// RLN_NOALLOC_SCRATCH_BYTES on every device the library runs on, held until
// the process ends. Host code never passes `scratch` itself to a kernel (on
// the host the name stands for a host-side stand-in, not the device array):
// it uses the address hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) float scratch[RLN_NOALLOC_SCRATCH_BYTES / sizeof(float)];

namespace rln {
namespace {

// Argument checks shared by rln_backward and rln_backward_noalloc (the C ABI
// names them in include/rln.h); RLN_OK or the failing code.
int check_backward(const float* updated, const float* weight, const float* mean,
                   const float* rstd, float* grad_x, void* grad_branch, int branch_dtype,
                   int grad_normalized_dtype, const float* grad_weight, const float* grad_bias,
                   const uint32_t* dropout_mask, int64_t rows, int64_t hidden, double dropout_p,
                   int training) {
    int status = check_common(rows, hidden, branch_dtype);
    if (status != RLN_OK) {
        return status;
    }
    if (!updated || !weight || !mean || !rstd || !grad_x || !grad_branch) {
        return fail(RLN_ERR_INVALID, "backward tensors must not be null");
    }
    if (!valid_dtype(grad_normalized_dtype)) {
        return fail(RLN_ERR_INVALID, "grad_normalized must use float16, bfloat16 or float32");
    }
    if ((grad_weight == nullptr) != (grad_bias == nullptr)) {
        return fail(RLN_ERR_INVALID, "grad_weight and grad_bias must both be given or both be null");
    }
    DropoutConstants drop{};
    status = dropout_constants(dropout_p, training, &drop);
    if (status != RLN_OK) {
        return status;
    }
    if (drop.active && !dropout_mask) {
        return fail(RLN_ERR_INVALID, "dropout_mask must not be null when dropout is active");
    }
    return RLN_OK;
}

// The backward launch sequence behind both backward entry points, after
// check_backward passed: workspace = the per-block weight/bias partials of
// the deterministic reduction (or NULL when none are needed).
int backward_launches(
    const float* grad_updated,
    const void* grad_normalized,
    int grad_normalized_dtype,
    const float* updated,
    const float* weight,
    const float* mean,
    const float* rstd,
    const uint32_t* dropout_mask,
    float* grad_x,
    void* grad_branch,
    int branch_dtype,
    float* grad_weight,
    float* grad_bias,
    int64_t rows,
    int64_t hidden,
    double dropout_p,
    int training,
    int deterministic,
    int accumulate_parameters,
    void* workspace,
    size_t workspace_bytes,
    void* stream) {
    int status = RLN_OK;
    DropoutConstants drop{};
    dropout_constants(dropout_p, training, &drop);
    const bool parameters = grad_weight != nullptr && grad_normalized != nullptr;
    const bool partials = parameters && uses_partials(deterministic);
    const size_t needed = partials ? rln_backward_workspace_bytes(rows, hidden, deterministic) : 0;
    if (needed > 0) {
        if (workspace == nullptr || workspace_bytes < needed) {
            return fail(
                RLN_ERR_INVALID,
                "workspace too small: need %zu bytes, got %zu",
                needed,
                workspace == nullptr ? static_cast<size_t>(0) : workspace_bytes);
        }
        if (!aligned_to(workspace, 16)) {
            return fail(RLN_ERR_INVALID, "workspace must be 16-byte aligned");
        }
    }

    BackwardArgs a{};
    a.grad_updated = grad_updated;
    a.grad_normalized = grad_normalized;
    a.updated = updated;
    a.weight = weight;
    a.mean = mean;
    a.rstd = rstd;
    a.mask = dropout_mask;
    a.grad_x = grad_x;
    a.grad_branch = grad_branch;
    a.grad_weight = grad_weight;
    a.grad_bias = grad_bias;
    a.partials = static_cast<float*>(workspace);
    a.rows = rows;
    a.scale = drop.scale;
    a.stream = static_cast<hipStream_t>(stream);
    a.flags = (grad_updated ? kHasGradUpdated : 0)
        | (grad_normalized ? kHasGradNormalized : 0)
        | (drop.active ? kDropout : 0)
        | (parameters ? kParameters : 0)
        | (partials ? kPartials : 0);

    if (parameters && !partials && !accumulate_parameters) {
        rln_zero_parameters_kernel<<<dim3(static_cast<unsigned>((hidden + 255) / 256)), 256, 0, a.stream>>>(
            grad_weight, grad_bias, static_cast<int>(hidden));
        status = check_launch("rln_zero_parameters_kernel");
        if (status != RLN_OK) {
            return status;
        }
    }

    const bool aligned = aligned_to(grad_updated, 16)
        && aligned_to(grad_normalized, vector_alignment(grad_normalized_dtype))
        && aligned_to(updated, 16) && aligned_to(weight, 16) && aligned_to(grad_x, 16)
        && aligned_to(grad_branch, vector_alignment(branch_dtype));
    status = with_shape<Pass::kBackward>(hidden, rows, [&](auto shape) {
        return launch_backward_shape(a, shape, branch_dtype, grad_normalized_dtype, aligned);
    });
    if (status != RLN_OK) {
        return status;
    }
    if (partials) {
        const int64_t groups = backward_blocks(rows, hidden);
        const unsigned blocks = static_cast<unsigned>((2 * hidden + kWaveSize - 1) / kWaveSize);
        rln_parameter_reduce_kernel<<<dim3(blocks), kReduceWaves * kWaveSize, 0, a.stream>>>(
            a.partials, grad_weight, grad_bias, groups, static_cast<int>(hidden),
            accumulate_parameters ? 1 : 0);
        status = check_launch("rln_parameter_reduce_kernel");
    }
    return status;
}

// rln_backward_noalloc's per-device addresses of `scratch` (defined at file
// scope below), looked up once per device with that device current.
constexpr int kNoAllocMaxDevices = 64;
std::once_flag g_scratch_once[kNoAllocMaxDevices];
void* g_scratch_address[kNoAllocMaxDevices];
hipError_t g_scratch_status[kNoAllocMaxDevices];

// This device's address of `scratch` (the device is current), or NULL with
// the failure recorded.
void* device_scratch() {
    int device = -1;
    const hipError_t current = hipGetDevice(&device);
    if (current != hipSuccess || device < 0 || device >= kNoAllocMaxDevices) {
        fail(RLN_ERR_HIP, "rln_backward_noalloc: no usable current device (%s, device %d)",
             hipGetErrorString(current), device);
        return nullptr;
    }
    std::call_once(g_scratch_once[device], [device] {
        void* address = nullptr;
        g_scratch_status[device] = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
        g_scratch_address[device] = g_scratch_status[device] == hipSuccess ? address : nullptr;
    });
    if (g_scratch_address[device] == nullptr) {
        fail(RLN_ERR_HIP, "rln_backward_noalloc: hipGetSymbolAddress(scratch) failed on device "
             "%d: %s", device, hipGetErrorString(g_scratch_status[device]));
    }
    return g_scratch_address[device];
}

}  // namespace
}  // namespace rln

extern "C" {

int rln_backward(
    const float* grad_updated,
    const void* grad_normalized,
    int grad_normalized_dtype,
    const float* updated,
    const float* weight,
    const float* mean,
    const float* rstd,
    const uint32_t* dropout_mask,
    float* grad_x,
    void* grad_branch,
    int branch_dtype,
    float* grad_weight,
    float* grad_bias,
    int64_t rows,
    int64_t hidden,
    double dropout_p,
    int training,
    int deterministic,
    int accumulate_parameters,
    void* workspace,
    size_t workspace_bytes,
    void* stream) {
    rln::t_last_error.clear();
    const int status = check_backward(updated, weight, mean, rstd, grad_x, grad_branch,
                                      branch_dtype, grad_normalized_dtype, grad_weight,
                                      grad_bias, dropout_mask, rows, hidden, dropout_p, training);
    if (status != RLN_OK) {
        return status;
    }
    if (check_stream(stream) != RLN_OK) {
        return RLN_ERR_INVALID;
    }
    return backward_launches(grad_updated, grad_normalized, grad_normalized_dtype, updated, weight,
                             mean, rstd, dropout_mask, grad_x, grad_branch, branch_dtype,
                             grad_weight, grad_bias, rows, hidden, dropout_p, training,
                             deterministic, accumulate_parameters, workspace, workspace_bytes,
                             stream);
}

int rln_backward_noalloc(
    const float* grad_updated,
    const void* grad_normalized,
    int grad_normalized_dtype,
    const float* updated,
    const float* weight,
    const float* mean,
    const float* rstd,
    const uint32_t* dropout_mask,
    float* grad_x,
    void* grad_branch,
    int branch_dtype,
    float* grad_weight,
    float* grad_bias,
    int64_t rows,
    int64_t hidden,
    double dropout_p,
    int training,
    int deterministic,
    int accumulate_parameters,
    void* stream) {
    rln::t_last_error.clear();
    const int status = check_backward(updated, weight, mean, rstd, grad_x, grad_branch,
                                      branch_dtype, grad_normalized_dtype, grad_weight,
                                      grad_bias, dropout_mask, rows, hidden, dropout_p, training);
    if (status != RLN_OK) {
        return status;
    }
    if (check_stream(stream) != RLN_OK) {
        return RLN_ERR_INVALID;
    }
    const bool parameters = grad_weight != nullptr && grad_normalized != nullptr;
    const size_t needed = parameters ? rln_backward_workspace_bytes(rows, hidden, deterministic) : 0;
    if (needed > RLN_NOALLOC_SCRATCH_BYTES) {
        return fail(RLN_ERR_INVALID,
                    "rln_backward_noalloc: the weight/bias partials of %lld rows x %lld need "
                    "%zu bytes, above its %zu-byte scratch (use rln_backward with a workspace)",
                    static_cast<long long>(rows), static_cast<long long>(hidden), needed,
                    static_cast<size_t>(RLN_NOALLOC_SCRATCH_BYTES));
    }
    void* workspace = nullptr;
    if (needed > 0) {
        workspace = device_scratch();
        if (workspace == nullptr) {
            return RLN_ERR_HIP;
        }
    }
    return backward_launches(grad_updated, grad_normalized, grad_normalized_dtype, updated, weight,
                             mean, rstd, dropout_mask, grad_x, grad_branch, branch_dtype,
                             grad_weight, grad_bias, rows, hidden, dropout_p, training,
                             deterministic, accumulate_parameters, workspace,
                             RLN_NOALLOC_SCRATCH_BYTES, stream);
}

uint64_t rln_philox_increment(int64_t hidden, int64_t threads) {
    rln::t_last_error.clear();
    if (!hidden_supported(hidden)) {
        fail(RLN_ERR_UNSUPPORTED, "unsupported hidden size %lld", static_cast<long long>(hidden));
        return 0;
    }
    if (check_philox_threads(hidden, threads) != RLN_OK) {
        return 0;
    }
    if (threads == 0) {
        return 4;
    }
    const int64_t items = (hidden + threads - 1) / threads;
    return static_cast<uint64_t>(4 * ((items + 3) / 4));
}

int64_t rln_mask_words(int64_t rows, int64_t hidden) {
    if (rows <= 0 || hidden <= 0 || hidden % 32 != 0) {
        return 0;
    }
    return rows * (hidden / 32);
}

int rln_hidden_supported(int64_t hidden) {
    return hidden_supported(hidden) ? 1 : 0;
}

int rln_supported_hidden_sizes(int64_t* out, int capacity) {
    int count = 0;
    for (int64_t hidden = kHiddenMultiple; hidden <= kMaxHidden; hidden += kHiddenMultiple) {
        if (!hidden_supported(hidden)) {
            continue;
        }
        if (out != nullptr && count < capacity) {
            out[count] = hidden;
        }
        ++count;
    }
    return count;
}

const char* rln_last_error(void) {
    return rln::t_last_error.c_str();
}

const char* rln_target_arch(void) {
    return "gfx950";
}

const char* rln_version(void) {
    return "0.4.0";
}

}  // extern "C"
