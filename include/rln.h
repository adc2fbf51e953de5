/*
 * rln.h - C ABI of the MI355X (gfx950) fused residual-add + dropout + LayerNorm
 * library, librln_gfx950.so.
 *
 * The operator, per row of `hidden` elements (H):
 *
 *   d = branch                                   (eval, or dropout_p == 0)
 *   d = round_to_branch_dtype(float(branch) * keep * 1/(1-p))   (training, p > 0)
 *   updated    = x + d                           (fp32)
 *   mean       = sum(updated) / H
 *   rstd       = 1 / sqrt(sum((updated - mean)^2) / H + eps)
 *   normalized = (updated - mean) * rstd * weight + bias
 *
 * and its first-order backward. This is the contract of the reference's
 * native entry points csrc/residual_layer_norm.h:10-42 and
 * csrc/residual_layer_norm_kernel.hip:425-545 (forward), :548-618 (input
 * gradients), :727-869 (weight/bias gradients).
 *
 * Conventions shared by every entry point:
 *  - All pointers are device pointers on the calling thread's current HIP
 *    device, except `philox` (host pointer to a descriptor).
 *  - Tensors are dense row-major [rows, hidden]; mean/rstd are [rows].
 *  - The dropout mask is `rows * hidden / 32` uint32 words: keep(r, c) is
 *    bit (c % 32) of word r * hidden / 32 + c / 32 - the reference's layout
 *    (csrc/residual_layer_norm_kernel.hip:500-511, :162-164).
 *  - `stream` is a hipStream_t (NULL = the legacy default stream) of the
 *    current device; a stream of another device is rejected with
 *    RLN_ERR_INVALID. Work is enqueued asynchronously; nothing synchronizes
 *    the host.
 *  - No entry point allocates device memory; rln_backward_noalloc also takes
 *    no workspace (it keeps a static per-device scratch instead).
 *  - Return value: RLN_OK, or an RLN_ERR_* code with a message available
 *    from rln_last_error() (thread-local, valid until the next call on the
 *    same thread).
 */
#ifndef RLN_H
#define RLN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types of the branch, grad_branch, normalized and grad_normalized
 * tensors (x, updated, mean, rstd and the other gradients are always fp32). */
enum rln_dtype {
    RLN_DTYPE_F32 = 0,
    RLN_DTYPE_F16 = 1,
    RLN_DTYPE_BF16 = 2
};

enum rln_status {
    RLN_OK = 0,
    RLN_ERR_INVALID = 1,     /* bad argument: shape, range, null pointer */
    RLN_ERR_UNSUPPORTED = 2, /* valid request this build does not serve */
    RLN_ERR_HIP = 3          /* HIP runtime reported an error at launch */
};

/*
 * Philox4x32-10 stream selection for dropout. Mirrors torch's
 * at::PhiloxCudaState: outside graph capture the values are given directly;
 * under HIP graph capture the seed and base offset live in device memory and
 * are read when the kernel runs (effective offset = *offset_ptr + offset).
 * Replaces the seed/offset reservation at
 * csrc/residual_layer_norm_kernel.hip:1755-1780.
 *
 * `threads` selects the layout of the stream over the tensor:
 *  - 128, 192 or 256: the reference's own, the hipRAND Philox stream of its
 *    forward launched with that many threads per row (reference
 *    csrc/residual_layer_norm_kernel.hip:449-511; the reference's Python
 *    passes 128, or 192 for hidden 1024, gfx1010_kernels/_normalization_native.py:5-12).
 *    Same (seed, offset, threads) => the reference's mask, bit for bit.
 *    Hidden sizes 128, 256, 384, 512, 768 and 1024 only, and the offset
 *    (offset, plus *offset_ptr under capture) must be a multiple of 4, as
 *    torch's generator hands out.
 *  - 0: this library's layout, one Philox block per four consecutive columns
 *    (counter = (offset / 4, (row * hidden + column) / 4)); every hidden size.
 */
typedef struct rln_philox {
    uint64_t seed;             /* used when seed_ptr == NULL            */
    uint64_t offset;           /* absolute offset, or intra-graph delta */
    const int64_t* seed_ptr;   /* device pointer or NULL                */
    const int64_t* offset_ptr; /* device pointer or NULL                */
    int64_t threads;           /* 0, or 128 / 192 / 256 (see above)     */
} rln_philox_t;

/*
 * Forward. Replaces residual_layer_norm_forward_hip
 * (csrc/residual_layer_norm.h:10-24; csrc/residual_layer_norm_kernel.hip:1720-1827).
 *
 * x, updated: fp32 [rows, hidden]; branch: [rows, hidden] in `branch_dtype`;
 * normalized: [rows, hidden] in `normalized_dtype` (fp32 in the reference;
 * fp16/bf16 round the fp32 result to nearest even for a consumer that reads
 * half precision); weight, bias: fp32 [hidden]; mean, rstd: fp32 [rows].
 * dropout_mask: rln_mask_words(rows, hidden) uint32 words, written only when
 * training && dropout_p > 0 (may be NULL otherwise). `philox` is read only in
 * that case (may be NULL otherwise). The call consumes
 * rln_philox_increment(hidden, philox->threads) offset units of the Philox
 * stream.
 * zero_grad_weight, zero_grad_bias: both NULL, or fp32 [hidden] each, set to
 * zero by this launch: the weight/bias gradient sums of a later
 * rln_backward(..., accumulate_parameters = 1), which then needs no zeroing
 * launch of its own (the reference memsets them in its backward,
 * csrc/residual_layer_norm_kernel.hip:1895-1901; one launch fewer per
 * training step here).
 */
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
    void* stream);

/*
 * Backward. Replaces residual_layer_norm_backward_hip
 * (csrc/residual_layer_norm.h:27-42; csrc/residual_layer_norm_kernel.hip:1830-2036).
 *
 * grad_updated: fp32 [rows, hidden]; grad_normalized: [rows, hidden] in
 * `grad_normalized_dtype` (the dtype of the forward's normalized output);
 * either upstream gradient may be NULL, meaning zero (the reference
 * materializes zeros instead, csrc/residual_layer_norm_bindings.cpp:62-67).
 * grad_x: fp32 [rows, hidden]; grad_branch: [rows, hidden] in branch_dtype.
 * grad_weight, grad_bias: fp32 [hidden], both NULL to skip the parameter
 * gradients (they are skipped as well when grad_normalized is NULL; the
 * outputs are then left untouched).
 * deterministic != 0 selects the fixed-order two-stage reduction of the
 * parameter gradients (bitwise reproducible); 0 selects grouped fp32 atomics.
 * accumulate_parameters != 0 adds the parameter gradients to the values
 * already in grad_weight / grad_bias (gradient accumulation across calls, one
 * kernel launch in atomic mode); 0 overwrites them.
 * Placement (speed only): in atomic mode every block of the launch adds into
 * both arrays at its end. Measured at hidden = 768 (MI355X): when grad_bias
 * starts within 2 KiB of a multiple of 32 KiB after grad_weight (and at some
 * larger distances: 256 and 384 KiB, 4 MiB), both arrays fall on the same
 * memory channels and those atomics take about 3.7 times as long (6.2 instead
 * of 1.7 us per backward at [8192, 768]); adjacent arrays (two consecutive
 * allocations of `hidden` floats, or one [2, hidden] buffer) are fast.
 * workspace: device scratch of at least
 * rln_backward_workspace_bytes(rows, hidden, deterministic) bytes, 16-byte
 * aligned (may be NULL when that size is 0).
 */
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
    void* stream);

/* Scratch bytes rln_backward_noalloc keeps per device (see below). */
#define RLN_NOALLOC_SCRATCH_BYTES (4u << 20)

/*
 * Backward that allocates nothing and takes no workspace. It has
 * no counterpart in the reference: it is for callers that cannot allocate
 * device memory or pass a workspace (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). Same arguments, checks and
 * results as rln_backward without workspace / workspace_bytes: the
 * deterministic weight/bias partials live in a library-owned static device
 * array of RLN_NOALLOC_SCRATCH_BYTES on each device (held until the process
 * ends; its address is looked up once per device on the first call). A call
 * whose partials need more (rln_backward_workspace_bytes(rows, hidden, 1)
 * above that, e.g. hidden above 2048 once the backward runs its full 256
 * blocks) fails with RLN_ERR_INVALID before any GPU work. Every call on a
 * device shares that device's scratch, and nothing in it needs clearing (each
 * call overwrites what it reads): calls that overlap on one device (different
 * streams, different host threads) race and must be ordered by the caller.
 * Atomic mode uses no scratch.
 */
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
    void* stream);

/* Workspace bytes rln_backward needs (0 in atomic mode): the per-block
 * weight/bias partials of the deterministic reduction, which the reference
 * allocates itself (csrc/residual_layer_norm_kernel.hip:1870-1872). */
size_t rln_backward_workspace_bytes(
    int64_t rows,
    int64_t hidden,
    int deterministic);

/* Philox offset units one dropout forward consumes (torch's `increment`):
 * 4 for threads == 0; for the reference's layout its own
 * 4 * ceil(ceil(hidden / threads) / 4) (csrc/residual_layer_norm_kernel.hip:1766-1770).
 * 0 (with rln_last_error set) for an unsupported hidden / threads pair. */
uint64_t rln_philox_increment(int64_t hidden, int64_t threads);

/* Number of uint32 dropout-mask words for [rows, hidden] (the reference's
 * mask size, csrc/residual_layer_norm_kernel.hip:1750-1753, :162-164). */
int64_t rln_mask_words(int64_t rows, int64_t hidden);

/* 1 if the library serves rows of `hidden` values, else 0: the reference's
 * sizes 128, 256, 384, 512, 768 and 1024 (specialized kernels) and every
 * other multiple of 64 from 128 to 8192 (kernels with a run-time row length;
 * the reference compiles only the six, gfx1010_kernels/normalization.py:12). */
int rln_hidden_supported(int64_t hidden);

/* Writes up to `capacity` supported hidden sizes in ascending order; returns
 * how many exist (the reference's NATIVE_HIDDEN_SIZES,
 * gfx1010_kernels/normalization.py:12). */
int rln_supported_hidden_sizes(int64_t* out, int capacity);

/* Thread-local message for the last failed call on this thread (the text of
 * the reference's TORCH_CHECK messages, csrc/residual_layer_norm_kernel.hip:26-166). */
const char* rln_last_error(void);

/* GPU architecture the device code was built for ("gfx950"; the reference
 * gates on "gfx1010", gfx1010_kernels/normalization.py:57). */
const char* rln_target_arch(void);

/* Library version string (the reference's package version is
 * gfx1010_kernels/__init__.py:22). */
const char* rln_version(void);

#ifdef __cplusplus
}
#endif

#endif /* RLN_H */
