// Streaming-ceiling kernels for the benchmark (librln_ceiling_gfx950.so,
// loaded by bench.py only; the operator never calls them). Each kernel moves
// exactly the bytes of one pass of the fused residual LayerNorm over
// [rows, hidden] - the same streams, element types and per-row / per-word
// side traffic - with no row reductions and no dropout draws, in the plainest
// shape a streaming kernel takes on MI355X: one pass over the data, 256
// threads per block, two 128-bit vectors per thread and stream, every row
// stream loaded and stored non-temporally, blocks replaced by the hardware
// dispatcher as they finish. Its time for a launch is the practical floor the
// operator's kernel of the same pass is measured against.
//
//   forward:  reads x (fp32), branch (2 or 4 bytes); writes updated (fp32),
//             normalized (2 or 4 bytes), one mask word per 32 columns when
//             dropping, mean and rstd per row.
//   backward: reads grad_updated (fp32), grad_normalized (2 or 4 bytes),
//             updated (fp32), the mask word of every column group when
//             dropping, mean and rstd per row; writes grad_x (fp32),
//             grad_branch (2 or 4 bytes).
//
// The arithmetic only combines the loaded values so that no access can be
// dropped by the compiler; its results are meaningless.

#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kVectors = 2;  // 128-bit vectors per thread and stream

// Four elements of a 2- or 4-byte stream, widened to fp32 / narrowed back.
template <int Bytes>
struct Narrow;
template <>
struct Narrow<4> {
    using type = f32x4;
    __device__ static f32x4 widen(type v) { return v; }
    __device__ static type narrow(f32x4 v) { return v; }
};
template <>
struct Narrow<2> {
    using type = f16x4;
    __device__ static f32x4 widen(type v) { return __builtin_convertvector(v, f32x4); }
    __device__ static type narrow(f32x4 v) { return __builtin_convertvector(v, f16x4); }
};

template <int BranchBytes, int NormalizedBytes>
__global__ __launch_bounds__(kThreads)
void ceiling_forward_kernel(const f32x4* __restrict__ x,
                            const typename Narrow<BranchBytes>::type* __restrict__ branch,
                            f32x4* __restrict__ updated,
                            typename Narrow<NormalizedBytes>::type* __restrict__ normalized,
                            uint32_t* __restrict__ mask,
                            float* __restrict__ mean,
                            float* __restrict__ rstd,
                            int64_t vectors,
                            int64_t row_vectors) {
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kThreads * kVectors + threadIdx.x;
    f32x4 xv[kVectors];
    typename Narrow<BranchBytes>::type bv[kVectors];
#pragma unroll
    for (int k = 0; k < kVectors; ++k) {
        const int64_t j = base + k * kThreads;
        if (j < vectors) {
            xv[k] = __builtin_nontemporal_load(x + j);
            bv[k] = __builtin_nontemporal_load(branch + j);
        }
    }
#pragma unroll
    for (int k = 0; k < kVectors; ++k) {
        const int64_t j = base + k * kThreads;
        if (j < vectors) {
            const f32x4 u = xv[k] + Narrow<BranchBytes>::widen(bv[k]);
            __builtin_nontemporal_store(u, updated + j);
            __builtin_nontemporal_store(Narrow<NormalizedBytes>::narrow(u * 0.5f), normalized + j);
            if (mask != nullptr && (j & 7) == 0) {
                __builtin_nontemporal_store(static_cast<uint32_t>(j), mask + j / 8);
            }
            if (j % row_vectors == 0) {
                mean[j / row_vectors] = u.x;
                rstd[j / row_vectors] = u.y;
            }
        }
    }
}

template <int GradNormalizedBytes, int BranchBytes>
__global__ __launch_bounds__(kThreads)
void ceiling_backward_kernel(const f32x4* __restrict__ grad_updated,
                             const typename Narrow<GradNormalizedBytes>::type* __restrict__ grad_normalized,
                             const f32x4* __restrict__ updated,
                             const uint32_t* __restrict__ mask,
                             const float* __restrict__ mean,
                             const float* __restrict__ rstd,
                             f32x4* __restrict__ grad_x,
                             typename Narrow<BranchBytes>::type* __restrict__ grad_branch,
                             int64_t vectors,
                             int64_t row_vectors) {
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kThreads * kVectors + threadIdx.x;
    f32x4 gu[kVectors];
    f32x4 gy[kVectors];
    f32x4 u[kVectors];
    uint32_t word[kVectors];
    float statistic[kVectors];
#pragma unroll
    for (int k = 0; k < kVectors; ++k) {
        const int64_t j = base + k * kThreads;
        if (j < vectors) {
            gu[k] = __builtin_nontemporal_load(grad_updated + j);
            gy[k] = Narrow<GradNormalizedBytes>::widen(__builtin_nontemporal_load(grad_normalized + j));
            u[k] = __builtin_nontemporal_load(updated + j);
            word[k] = mask != nullptr ? mask[j / 8] : 1u;
            statistic[k] = mean[j / row_vectors] * rstd[j / row_vectors];
        }
    }
#pragma unroll
    for (int k = 0; k < kVectors; ++k) {
        const int64_t j = base + k * kThreads;
        if (j < vectors) {
            const f32x4 g = (gu[k] + gy[k] * (u[k] - statistic[k]))
                * static_cast<float>(word[k] & 1u);
            __builtin_nontemporal_store(g, grad_x + j);
            __builtin_nontemporal_store(Narrow<BranchBytes>::narrow(g), grad_branch + j);
        }
    }
}

unsigned grid_for(int64_t vectors) {
    return static_cast<unsigned>((vectors + kThreads * kVectors - 1) / (kThreads * kVectors));
}

bool valid(int64_t rows, int64_t hidden, int first_bytes, int second_bytes) {
    return rows > 0 && hidden > 0 && hidden % 32 == 0
        && (first_bytes == 2 || first_bytes == 4) && (second_bytes == 2 || second_bytes == 4);
}

}  // namespace

extern "C" {

// One forward-shaped streaming pass over [rows, hidden]; `mask` may be NULL
// (no dropout). Returns 0, 1 for bad arguments, or 3 for a launch error.
int rln_ceiling_forward(const float* x, const void* branch, int branch_bytes, float* updated,
                        void* normalized, int normalized_bytes, uint32_t* mask, float* mean,
                        float* rstd, int64_t rows, int64_t hidden, void* stream) {
    if (!valid(rows, hidden, branch_bytes, normalized_bytes)) {
        return 1;
    }
    const int64_t vectors = rows * hidden / 4;
    const int64_t row_vectors = hidden / 4;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const auto* xv = reinterpret_cast<const f32x4*>(x);
    auto* uv = reinterpret_cast<f32x4*>(updated);
#define RLN_CEILING_FORWARD(B, N)                                                              \
    ceiling_forward_kernel<B, N><<<grid_for(vectors), kThreads, 0, s>>>(                       \
        xv, static_cast<const typename Narrow<B>::type*>(branch), uv,                          \
        static_cast<typename Narrow<N>::type*>(normalized), mask, mean, rstd, vectors,         \
        row_vectors)
    if (branch_bytes == 2 && normalized_bytes == 4) {
        RLN_CEILING_FORWARD(2, 4);
    } else if (branch_bytes == 2) {
        RLN_CEILING_FORWARD(2, 2);
    } else if (normalized_bytes == 4) {
        RLN_CEILING_FORWARD(4, 4);
    } else {
        RLN_CEILING_FORWARD(4, 2);
    }
#undef RLN_CEILING_FORWARD
    return hipGetLastError() == hipSuccess ? 0 : 3;
}

// One backward-shaped streaming pass over [rows, hidden]; `mask` may be NULL.
int rln_ceiling_backward(const float* grad_updated, const void* grad_normalized,
                         int grad_normalized_bytes, const float* updated, const uint32_t* mask,
                         const float* mean, const float* rstd, float* grad_x, void* grad_branch,
                         int branch_bytes, int64_t rows, int64_t hidden, void* stream) {
    if (!valid(rows, hidden, grad_normalized_bytes, branch_bytes)) {
        return 1;
    }
    const int64_t vectors = rows * hidden / 4;
    const int64_t row_vectors = hidden / 4;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const auto* guv = reinterpret_cast<const f32x4*>(grad_updated);
    const auto* uv = reinterpret_cast<const f32x4*>(updated);
    auto* gxv = reinterpret_cast<f32x4*>(grad_x);
#define RLN_CEILING_BACKWARD(G, B)                                                             \
    ceiling_backward_kernel<G, B><<<grid_for(vectors), kThreads, 0, s>>>(                      \
        guv, static_cast<const typename Narrow<G>::type*>(grad_normalized), uv, mask, mean,    \
        rstd, gxv, static_cast<typename Narrow<B>::type*>(grad_branch), vectors, row_vectors)
    if (grad_normalized_bytes == 4 && branch_bytes == 2) {
        RLN_CEILING_BACKWARD(4, 2);
    } else if (grad_normalized_bytes == 4) {
        RLN_CEILING_BACKWARD(4, 4);
    } else if (branch_bytes == 2) {
        RLN_CEILING_BACKWARD(2, 2);
    } else {
        RLN_CEILING_BACKWARD(2, 4);
    }
#undef RLN_CEILING_BACKWARD
    return hipGetLastError() == hipSuccess ? 0 : 3;
}

}  // extern "C"
