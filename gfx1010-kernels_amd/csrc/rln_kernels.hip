// Fused residual-add + dropout + LayerNorm for MI355X (gfx950, CDNA4).
//
// Device kernels and the C ABI declared in include/rln.h. The operator is the
// one implemented by the reference's csrc/residual_layer_norm_kernel.hip
// (forward :425-545, input backward :548-618, parameter backward :727-869);
// the kernels here are organised for wave64 CDNA hardware instead:
//
//  * One wavefront owns one row (two rows when H/4 is not a multiple of 64,
//    i.e. H = 128 and 384: each half-wave of 32 lanes owns a row). A lane
//    holds kV four-element vectors of its row in registers, so both row
//    reductions run inside the wave with DPP row operations plus
//    v_readlane - no LDS, no barriers.
//  * Loads and stores are 128-bit (64-bit for four fp16 values) and marked
//    non-temporal: every byte of the op is touched exactly once per kernel,
//    so the accesses stream through the caches instead of displacing lines
//    other work may reuse. A scalar-access variant of every kernel serves
//    misaligned pointers with the identical arithmetic, so both variants are
//    bitwise equal.
//  * Waves walk rows with a grid-stride loop over a grid that depends only on
//    (rows, H), never on the device, so the dropout stream and the
//    deterministic parameter-gradient order are reproducible anywhere.
//  * Dropout draws one Philox4x32-10 block (Salmon et al., SC'11) per four
//    consecutive columns: counter = (offset/4, column-group index), key =
//    seed. The keep mask depends only on (seed, offset, row, column), not on
//    the launch shape. Keep bits are OR-combined across 8 lanes with DPP
//    into the reference's int32 word layout (bit c%32 of word c/32).
//  * The backward kernel produces grad_x and grad_branch AND accumulates
//    the weight/bias gradients from the same registers, so g_y and updated
//    are read once (the reference reads them a second time in its separate
//    parameter kernels, :727-869). Each block combines its waves' sums in a
//    fixed order in LDS and writes one [2, H] partial; a second kernel adds
//    the partials in ascending block order (bitwise reproducible). The
//    non-deterministic mode combines the block partials with hardware fp32
//    atomics instead.
//
// Arithmetic that the tests hold bit-exact follows the reference:
//  * dropped branch = round_to_branch_dtype(float(b) * keep * scale),
//    scale = 1.0f / (1.0f - float(p)), keep = u32 >= uint32(double(float(p)) * 2^32)
//    (reference :492-497, :896-899);
//  * updated = x + dropped, a single fp32 add;
//  * grad_branch = round_to_branch_dtype(g * (keep * scale)) (reference :605-615).
// This file is compiled with -ffp-contract=off so that none of these is
// fused into an FMA; FMAs appear only where written explicitly.

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "rln.h"

// Launch-shape constants. They are part of the deterministic contract: the
// grid is a function of (rows, H) and these values only.
#ifndef RLN_FWD_MAX_BLOCKS
#define RLN_FWD_MAX_BLOCKS 2048
#endif
#ifndef RLN_BWD_MAX_BLOCKS
#define RLN_BWD_MAX_BLOCKS 256
#endif
#ifndef RLN_BWD_THREADS
#define RLN_BWD_THREADS 512
#endif
#ifndef RLN_ATOMIC_PARAMETERS
#define RLN_ATOMIC_PARAMETERS 1
#endif
#ifndef RLN_FWD_PREFETCH
#define RLN_FWD_PREFETCH 1
#endif
#ifndef RLN_BWD_PREFETCH
#define RLN_BWD_PREFETCH 1
#endif
#ifndef RLN_NT_LOADS
#define RLN_NT_LOADS 1
#endif
#ifndef RLN_NT_STORES
#define RLN_NT_STORES 1
#endif

namespace {

constexpr int kWaveSize = 64;
constexpr int kForwardThreads = 256;
constexpr int kBackwardThreads = RLN_BWD_THREADS;
constexpr int64_t kForwardMaxBlocks = RLN_FWD_MAX_BLOCKS;
constexpr int64_t kBackwardMaxBlocks = RLN_BWD_MAX_BLOCKS;
constexpr bool kForwardPrefetch = RLN_FWD_PREFETCH != 0;
constexpr bool kBackwardPrefetch = RLN_BWD_PREFETCH != 0;
static_assert(kBackwardThreads % kWaveSize == 0 && kBackwardThreads <= 1024, "backward block");

constexpr int64_t kSupportedHidden[] = {128, 256, 384, 512, 768, 1024};

using half_t = _Float16;
using bf16_t = __bf16;
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

// ----------------------------------------------------------------------------
// Error reporting.

thread_local std::string t_last_error;

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

// ----------------------------------------------------------------------------
// Row geometry for a hidden size H.

template <int H>
struct Geometry {
    static constexpr int kVectors = H / 4;  // four-element vectors per row
    static constexpr int kLanes = (kVectors % kWaveSize == 0) ? 64 : 32;
    static constexpr int kV = kVectors / kLanes;  // vectors per lane
    static constexpr int kRowsPerWave = kWaveSize / kLanes;
    static constexpr int kMaskWords = H / 32;
    static_assert(H % 64 == 0, "hidden size must be a multiple of 64");
    static_assert(kVectors % kLanes == 0, "row must split evenly over lanes");
};

int64_t rows_per_wave(int64_t hidden) {
    return ((hidden / 4) % kWaveSize == 0) ? 1 : 2;
}

// Blocks for a launch over `rows`: enough for `groups_per_wave` row groups
// per wave (a group = the rows one wave handles at once), capped; a function
// of (rows, hidden) only.
int64_t launch_blocks(int64_t rows, int64_t hidden, int threads, int64_t cap,
                      int64_t groups_per_wave) {
    const int64_t groups = (rows + rows_per_wave(hidden) - 1) / rows_per_wave(hidden);
    const int64_t waves = (groups + groups_per_wave - 1) / groups_per_wave;
    const int64_t waves_per_block = threads / kWaveSize;
    const int64_t blocks = (waves + waves_per_block - 1) / waves_per_block;
    return blocks < cap ? blocks : cap;
}

// The forward gives each wave at least two row groups so that its
// look-ahead load overlaps a row's computation; with 256-thread blocks and
// ~100 VGPRs per lane the cap of 2048 blocks is two waves of residency.
int64_t forward_blocks(int64_t rows, int64_t hidden) {
    return launch_blocks(rows, hidden, kForwardThreads, kForwardMaxBlocks, 2);
}

// The backward's grid is also the number of weight/bias partials: 256
// blocks of 8 waves, one block per CU.
int64_t backward_blocks(int64_t rows, int64_t hidden) {
    return launch_blocks(rows, hidden, kBackwardThreads, kBackwardMaxBlocks, 1);
}

bool hidden_supported(int64_t hidden) {
    for (const int64_t value : kSupportedHidden) {
        if (value == hidden) {
            return true;
        }
    }
    return false;
}

// ----------------------------------------------------------------------------
// Wave-level primitives.

// DPP controls (GFX9 encoding).
constexpr int kDppQuadXor1 = 0xB1;     // quad_perm:[1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;     // quad_perm:[2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

#define RLN_DPP_F32(value, control) \
    __builtin_amdgcn_update_dpp(0.0f, (value), (control), 0xF, 0xF, false)
#define RLN_DPP_I32(value, control) \
    __builtin_amdgcn_update_dpp(0, (value), (control), 0xF, 0xF, false)

// Sum over each 16-lane DPP row; every lane of the row receives the same,
// bitwise identical value (each step adds a pair in commutative order).
__device__ __forceinline__ float row16_sum(float value) {
    value += RLN_DPP_F32(value, kDppQuadXor1);
    value += RLN_DPP_F32(value, kDppQuadXor2);
    value += RLN_DPP_F32(value, kDppRowHalfMirror);
    value += RLN_DPP_F32(value, kDppRowMirror);
    return value;
}

// v_readlane_b32 of an fp32 value. The builtin is declared on int, so the
// value travels as its bit pattern (a plain call would convert to int).
__device__ __forceinline__ float readlane_f32(float value, int lane) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, value), lane));
}

// Sum over the lanes that own one row: 64 lanes, or the 32-lane half of the
// wave that the calling lane belongs to. Must be called by all 64 lanes.
template <int Lanes>
__device__ __forceinline__ float row_sum(float value) {
    value = row16_sum(value);
    const float low = readlane_f32(value, 0) + readlane_f32(value, 16);
    const float high = readlane_f32(value, 32) + readlane_f32(value, 48);
    if constexpr (Lanes == 64) {
        return low + high;
    } else {
        return (threadIdx.x & 32) ? high : low;
    }
}

// OR over each aligned group of 8 lanes; all 8 lanes receive the result.
__device__ __forceinline__ uint32_t or8(uint32_t value) {
    int bits = static_cast<int>(value);
    bits |= RLN_DPP_I32(bits, kDppQuadXor1);
    bits |= RLN_DPP_I32(bits, kDppQuadXor2);
    bits |= RLN_DPP_I32(bits, kDppRowHalfMirror);
    return static_cast<uint32_t>(bits);
}

// ----------------------------------------------------------------------------
// Philox4x32-10, from the published round function (Salmon, Moraes, Dror,
// Shaw, "Parallel random numbers: as easy as 1, 2, 3", SC'11):
//   (hi0, lo0) = M0 * c0; (hi1, lo1) = M1 * c2
//   c' = (hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0);  k += (W0, W1)

__device__ __forceinline__ uint4 philox4x32_10(uint4 counter, uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int round = 0; round < 10; ++round) {
        const uint64_t product0 = static_cast<uint64_t>(0xD2511F53u) * counter.x;
        const uint64_t product1 = static_cast<uint64_t>(0xCD9E8D57u) * counter.z;
        counter = make_uint4(
            static_cast<uint32_t>(product1 >> 32) ^ counter.y ^ k0,
            static_cast<uint32_t>(product1),
            static_cast<uint32_t>(product0 >> 32) ^ counter.w ^ k1,
            static_cast<uint32_t>(product0));
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    return counter;
}

struct PhiloxArgs {
    uint64_t seed;
    uint64_t offset;
    const int64_t* seed_ptr;
    const int64_t* offset_ptr;
};

// ----------------------------------------------------------------------------
// Global memory access. Aligned = one 128-bit access (64-bit for 4 x fp16);
// otherwise element accesses with the same values. Streaming accesses carry
// the non-temporal hint.

template <typename T>
__device__ __forceinline__ T stream_load(const T* pointer) {
#if RLN_NT_LOADS
    return __builtin_nontemporal_load(pointer);
#else
    return *pointer;
#endif
}

template <typename T>
__device__ __forceinline__ void stream_store(T value, T* pointer) {
#if RLN_NT_STORES
    __builtin_nontemporal_store(value, pointer);
#else
    *pointer = value;
#endif
}

template <bool Aligned>
__device__ __forceinline__ f32x4 load4(const float* __restrict__ pointer) {
    if constexpr (Aligned) {
        return stream_load(reinterpret_cast<const f32x4*>(pointer));
    } else {
        return f32x4{stream_load(pointer), stream_load(pointer + 1), stream_load(pointer + 2),
                     stream_load(pointer + 3)};
    }
}

template <bool Aligned>
__device__ __forceinline__ void store4(float* __restrict__ pointer, f32x4 value) {
    if constexpr (Aligned) {
        stream_store(value, reinterpret_cast<f32x4*>(pointer));
    } else {
        stream_store(value.x, pointer);
        stream_store(value.y, pointer + 1);
        stream_store(value.z, pointer + 2);
        stream_store(value.w, pointer + 3);
    }
}

// Parameters (weight, bias): ordinary cached loads, every wave reads them.
template <bool Aligned>
__device__ __forceinline__ f32x4 load_parameter4(const float* __restrict__ pointer) {
    if constexpr (Aligned) {
        return *reinterpret_cast<const f32x4*>(pointer);
    } else {
        return f32x4{pointer[0], pointer[1], pointer[2], pointer[3]};
    }
}

template <typename T>
struct Vector4;
template <>
struct Vector4<float> {
    using type = f32x4;
};
template <>
struct Vector4<half_t> {
    using type = f16x4;
};
template <>
struct Vector4<bf16_t> {
    using type = bf16x4;
};

// Four consecutive elements of type T (fp32, fp16 or bf16), widened to fp32.
template <typename T, bool Aligned>
__device__ __forceinline__ f32x4 load_convert4(const T* __restrict__ pointer) {
    if constexpr (Aligned) {
        return __builtin_convertvector(
            stream_load(reinterpret_cast<const typename Vector4<T>::type*>(pointer)), f32x4);
    } else {
        return f32x4{
            static_cast<float>(stream_load(pointer)),
            static_cast<float>(stream_load(pointer + 1)),
            static_cast<float>(stream_load(pointer + 2)),
            static_cast<float>(stream_load(pointer + 3))};
    }
}

// Stores four fp32 values as type T; narrowing rounds to nearest even.
template <typename T, bool Aligned>
__device__ __forceinline__ void store_convert4(T* __restrict__ pointer, f32x4 value) {
    const typename Vector4<T>::type packed =
        __builtin_convertvector(value, typename Vector4<T>::type);
    if constexpr (Aligned) {
        stream_store(packed, reinterpret_cast<typename Vector4<T>::type*>(pointer));
    } else {
        stream_store(static_cast<T>(packed.x), pointer);
        stream_store(static_cast<T>(packed.y), pointer + 1);
        stream_store(static_cast<T>(packed.z), pointer + 2);
        stream_store(static_cast<T>(packed.w), pointer + 3);
    }
}

// The same with the element type chosen at run time (an rln_dtype value,
// uniform across the launch).
template <bool Aligned>
__device__ __forceinline__ f32x4 load_any4(const void* __restrict__ base, int64_t index,
                                           int dtype) {
    if (dtype == RLN_DTYPE_F16) {
        return load_convert4<half_t, Aligned>(static_cast<const half_t*>(base) + index);
    }
    if (dtype == RLN_DTYPE_BF16) {
        return load_convert4<bf16_t, Aligned>(static_cast<const bf16_t*>(base) + index);
    }
    return load_convert4<float, Aligned>(static_cast<const float*>(base) + index);
}

template <bool Aligned>
__device__ __forceinline__ void store_any4(void* __restrict__ base, int64_t index, f32x4 value,
                                           int dtype) {
    if (dtype == RLN_DTYPE_F16) {
        store_convert4<half_t, Aligned>(static_cast<half_t*>(base) + index, value);
    } else if (dtype == RLN_DTYPE_BF16) {
        store_convert4<bf16_t, Aligned>(static_cast<bf16_t*>(base) + index, value);
    } else {
        store_convert4<float, Aligned>(static_cast<float*>(base) + index, value);
    }
}

// Rounds an fp32 value through the branch dtype (identity for fp32).
template <typename B>
__device__ __forceinline__ float round_to_branch(float value) {
    return static_cast<float>(static_cast<B>(value));
}

__device__ __forceinline__ f32x4 zero4() {
    return f32x4{0.0f, 0.0f, 0.0f, 0.0f};
}

__device__ __forceinline__ float sum4(f32x4 value) {
    return (value.x + value.y) + (value.z + value.w);
}

// ----------------------------------------------------------------------------
// Forward kernel.

// The global values the forward reads for one row, held in registers.
template <int V>
struct ForwardRow {
    f32x4 x[V];
    f32x4 branch[V];
};

template <int H, typename B, bool Aligned>
__global__ __launch_bounds__(kForwardThreads)
void rln_forward_kernel(
    const float* __restrict__ x,
    const B* __restrict__ branch,
    const float* __restrict__ weight,
    const float* __restrict__ bias,
    float* __restrict__ updated,
    void* __restrict__ normalized,
    int normalized_dtype,
    float* __restrict__ mean_out,
    float* __restrict__ rstd_out,
    uint32_t* __restrict__ mask,
    int64_t rows,
    float eps,
    int dropout,
    float scale,
    uint32_t threshold,
    PhiloxArgs philox) {
    using G = Geometry<H>;
    constexpr int L = G::kLanes;
    constexpr int V = G::kV;
    constexpr int kWaves = kForwardThreads / kWaveSize;
    constexpr float kInvHidden = 1.0f / static_cast<float>(H);

    const int lane = threadIdx.x & (kWaveSize - 1);
    const int sub = lane / L;
    const int l = lane % L;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x / kWaveSize);
    const int64_t wave_count = static_cast<int64_t>(gridDim.x) * kWaves;

    f32x4 w[V];
    f32x4 b[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
        w[v] = load_parameter4<Aligned>(weight + (v * L + l) * 4);
        b[v] = load_parameter4<Aligned>(bias + (v * L + l) * 4);
    }

    uint32_t key0 = 0;
    uint32_t key1 = 0;
    uint64_t position = 0;
    if (dropout) {
        const uint64_t seed = philox.seed_ptr
            ? static_cast<uint64_t>(*philox.seed_ptr)
            : philox.seed;
        const uint64_t offset = philox.offset
            + (philox.offset_ptr ? static_cast<uint64_t>(*philox.offset_ptr) : 0);
        key0 = static_cast<uint32_t>(seed);
        key1 = static_cast<uint32_t>(seed >> 32);
        position = offset / 4;
    }

    // Loads x and the branch of one row; rows past the end read nothing.
    auto load_row = [&](ForwardRow<V>& r, int64_t row) {
        const bool valid = row < rows;
        const int64_t base = row * H;
#pragma unroll
        for (int v = 0; v < V; ++v) {
            const int column = (v * L + l) * 4;
            r.x[v] = zero4();
            r.branch[v] = zero4();
            if (valid) {
                r.x[v] = load4<Aligned>(x + base + column);
                r.branch[v] = load_convert4<B, Aligned>(branch + base + column);
            }
        }
    };

    auto process_row = [&](const ForwardRow<V>& r, int64_t row) {
        const bool valid = row < rows;
        const int64_t base = row * H;
        f32x4 u[V];
        uint32_t keep_bits[V];
#pragma unroll
        for (int v = 0; v < V; ++v) {
            f32x4 bv = r.branch[v];
            keep_bits[v] = 0;
            if (dropout) {
                const uint64_t group = static_cast<uint64_t>(row) * (H / 4) + (v * L + l);
                const uint4 random = philox4x32_10(
                    make_uint4(
                        static_cast<uint32_t>(position),
                        static_cast<uint32_t>(position >> 32),
                        static_cast<uint32_t>(group),
                        static_cast<uint32_t>(group >> 32)),
                    key0,
                    key1);
                const uint32_t k0 = random.x >= threshold;
                const uint32_t k1 = random.y >= threshold;
                const uint32_t k2 = random.z >= threshold;
                const uint32_t k3 = random.w >= threshold;
                bv.x = round_to_branch<B>(bv.x * static_cast<float>(k0) * scale);
                bv.y = round_to_branch<B>(bv.y * static_cast<float>(k1) * scale);
                bv.z = round_to_branch<B>(bv.z * static_cast<float>(k2) * scale);
                bv.w = round_to_branch<B>(bv.w * static_cast<float>(k3) * scale);
                keep_bits[v] = k0 | (k1 << 1) | (k2 << 2) | (k3 << 3);
            }
            u[v] = r.x[v] + bv;
            if (valid) {
                store4<Aligned>(updated + base + (v * L + l) * 4, u[v]);
            }
        }

        if (dropout) {
#pragma unroll
            for (int v = 0; v < V; ++v) {
                const uint32_t word = or8(keep_bits[v] << (4 * (l & 7)));
                if (valid && (l & 7) == 0) {
                    stream_store(word, mask + row * G::kMaskWords + (v * L + l) / 8);
                }
            }
        }

        float partial = 0.0f;
#pragma unroll
        for (int v = 0; v < V; ++v) {
            partial += sum4(u[v]);
        }
        const float mean = row_sum<L>(partial) * kInvHidden;

        float square = 0.0f;
#pragma unroll
        for (int v = 0; v < V; ++v) {
            u[v] = u[v] - mean;
            square += (u[v].x * u[v].x + u[v].y * u[v].y)
                + (u[v].z * u[v].z + u[v].w * u[v].w);
        }
        const float variance = row_sum<L>(square) * kInvHidden;
        const float rstd = rsqrtf(variance + eps);

        if (valid) {
            if (l == 0) {
                mean_out[row] = mean;
                rstd_out[row] = rstd;
            }
#pragma unroll
            for (int v = 0; v < V; ++v) {
                const int column = (v * L + l) * 4;
                const f32x4 y = {
                    __builtin_fmaf(u[v].x * rstd, w[v].x, b[v].x),
                    __builtin_fmaf(u[v].y * rstd, w[v].y, b[v].y),
                    __builtin_fmaf(u[v].z * rstd, w[v].z, b[v].z),
                    __builtin_fmaf(u[v].w * rstd, w[v].w, b[v].w)};
                store_any4<Aligned>(normalized, base + column, y, normalized_dtype);
            }
        }
    };

    // One row of look-ahead: the next row's loads are in flight while the
    // current row is computed and stored.
    const int64_t stride = wave_count * G::kRowsPerWave;
    int64_t first = wave * G::kRowsPerWave;
    ForwardRow<V> current;
    if constexpr (kForwardPrefetch) {
        load_row(current, first + sub);
    }
    for (; first < rows; first += stride) {
        if constexpr (kForwardPrefetch) {
            ForwardRow<V> next;
            load_row(next, first + stride + sub);
            process_row(current, first + sub);
            current = next;
        } else {
            load_row(current, first + sub);
            process_row(current, first + sub);
        }
    }
}

// ----------------------------------------------------------------------------
// Backward kernel: input gradients plus per-block weight/bias partial sums.

// Every global value the backward reads for one row, held in registers.
template <int V>
struct BackwardRow {
    f32x4 u[V];
    f32x4 gy[V];
    f32x4 gu[V];
    uint32_t keep_bits[V];
    float mean;
    float rstd;
};

enum BackwardFlags : int {
    kHasGradUpdated = 1,
    kHasGradNormalized = 2,
    kDropout = 4,
    kParameters = 8,
    kPartials = 16,  // write per-block partials (else fp32 atomics)
};

template <int H, typename B, bool Aligned>
__global__ __launch_bounds__(kBackwardThreads)
void rln_backward_kernel(
    const float* __restrict__ grad_updated,
    const void* __restrict__ grad_normalized,
    int grad_normalized_dtype,
    const float* __restrict__ updated,
    const float* __restrict__ weight,
    const float* __restrict__ mean_in,
    const float* __restrict__ rstd_in,
    const uint32_t* __restrict__ mask,
    float* __restrict__ grad_x,
    B* __restrict__ grad_branch,
    float* __restrict__ grad_weight,
    float* __restrict__ grad_bias,
    float* __restrict__ partials,
    int64_t rows,
    int flags,
    float scale) {
    using G = Geometry<H>;
    constexpr int L = G::kLanes;
    constexpr int V = G::kV;
    constexpr int kWaves = kBackwardThreads / kWaveSize;
    constexpr float kInvHidden = 1.0f / static_cast<float>(H);

    const int lane = threadIdx.x & (kWaveSize - 1);
    const int sub = lane / L;
    const int l = lane % L;
    const int wave_in_block = threadIdx.x / kWaveSize;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * kWaves + wave_in_block;
    const int64_t wave_count = static_cast<int64_t>(gridDim.x) * kWaves;

    const bool has_gu = flags & kHasGradUpdated;
    const bool has_gy = flags & kHasGradNormalized;
    const bool dropout = flags & kDropout;
    const bool parameters = flags & kParameters;

    f32x4 w[V];
    f32x4 acc_w[V];
    f32x4 acc_b[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
        w[v] = load_parameter4<Aligned>(weight + (v * L + l) * 4);
        acc_w[v] = zero4();
        acc_b[v] = zero4();
    }

    // Loads every global value of one row into registers; rows past the end
    // read nothing and hold zeros.
    auto load_row = [&](BackwardRow<V>& r, int64_t row) {
        const bool valid = row < rows;
        const int64_t base = row * H;
        r.mean = valid ? mean_in[row] : 0.0f;
        r.rstd = valid ? rstd_in[row] : 0.0f;
#pragma unroll
        for (int v = 0; v < V; ++v) {
            const int column = (v * L + l) * 4;
            r.u[v] = zero4();
            r.gy[v] = zero4();
            r.gu[v] = zero4();
            r.keep_bits[v] = 0;
            if (valid) {
                r.u[v] = load4<Aligned>(updated + base + column);
                if (has_gy) {
                    r.gy[v] = load_any4<Aligned>(grad_normalized, base + column, grad_normalized_dtype);
                }
                if (has_gu) {
                    r.gu[v] = load4<Aligned>(grad_updated + base + column);
                }
                if (dropout) {
                    r.keep_bits[v] =
                        mask[row * G::kMaskWords + (v * L + l) / 8] >> (4 * (l & 7));
                }
            }
        }
    };

    // Input gradients of one row and its contribution to the parameter sums.
    auto process_row = [&](const BackwardRow<V>& r, int64_t row) {
        const bool valid = row < rows;
        const int64_t base = row * H;
        f32x4 xhat[V];
        float sum_q = 0.0f;
        float sum_qx = 0.0f;
#pragma unroll
        for (int v = 0; v < V; ++v) {
            xhat[v] = (r.u[v] - r.mean) * r.rstd;
            const f32x4 q = r.gy[v] * w[v];
            sum_q += sum4(q);
            sum_qx += (q.x * xhat[v].x + q.y * xhat[v].y)
                + (q.z * xhat[v].z + q.w * xhat[v].w);
        }

        float mean_q = 0.0f;
        float mean_qx = 0.0f;
        if (has_gy) {
            mean_q = row_sum<L>(sum_q) * kInvHidden;
            mean_qx = row_sum<L>(sum_qx) * kInvHidden;
        }

        if (valid) {
#pragma unroll
            for (int v = 0; v < V; ++v) {
                const int column = (v * L + l) * 4;
                f32x4 g = r.gu[v];
                if (has_gy) {
                    const f32x4 q = r.gy[v] * w[v];
                    g = g + r.rstd * ((q - mean_q) - xhat[v] * mean_qx);
                }
                store4<Aligned>(grad_x + base + column, g);
                if (dropout) {
                    const uint32_t bits = r.keep_bits[v];
                    g.x = g.x * (static_cast<float>(bits & 1u) * scale);
                    g.y = g.y * (static_cast<float>((bits >> 1) & 1u) * scale);
                    g.z = g.z * (static_cast<float>((bits >> 2) & 1u) * scale);
                    g.w = g.w * (static_cast<float>((bits >> 3) & 1u) * scale);
                }
                store_convert4<B, Aligned>(grad_branch + base + column, g);
            }
        }

        if (parameters) {
#pragma unroll
            for (int v = 0; v < V; ++v) {
                acc_w[v].x = __builtin_fmaf(r.gy[v].x, xhat[v].x, acc_w[v].x);
                acc_w[v].y = __builtin_fmaf(r.gy[v].y, xhat[v].y, acc_w[v].y);
                acc_w[v].z = __builtin_fmaf(r.gy[v].z, xhat[v].z, acc_w[v].z);
                acc_w[v].w = __builtin_fmaf(r.gy[v].w, xhat[v].w, acc_w[v].w);
                acc_b[v] = acc_b[v] + r.gy[v];
            }
        }
    };

    // Each wave walks its rows with the next row's loads in flight while the
    // current row is reduced and stored (one row of look-ahead).
    const int64_t stride = wave_count * G::kRowsPerWave;
    int64_t first = wave * G::kRowsPerWave;
    BackwardRow<V> current;
    if constexpr (kBackwardPrefetch) {
        load_row(current, first + sub);
    }
    for (; first < rows; first += stride) {
        if constexpr (kBackwardPrefetch) {
            BackwardRow<V> next;
            load_row(next, first + stride + sub);
            process_row(current, first + sub);
            current = next;
        } else {
            load_row(current, first + sub);
            process_row(current, first + sub);
        }
    }

    if (!parameters) {
        return;
    }

    // Combine the block's sums in a fixed order: for every column, waves
    // 0..kWaves-1 and, within a wave, row slots 0..kRowsPerWave-1.
    __shared__ f32x4 staging[kWaves][kWaveSize][2];
    const bool write_partials = flags & kPartials;
#pragma unroll
    for (int v = 0; v < V; ++v) {
        staging[wave_in_block][lane][0] = acc_w[v];
        staging[wave_in_block][lane][1] = acc_b[v];
        __syncthreads();
        // L lanes x 8 floats to produce; the block's threads share them.
        for (int entry = threadIdx.x; entry < L * 8; entry += kBackwardThreads) {
            const int slot = entry / 8;
            const int which = (entry / 4) & 1;  // 0 = weight, 1 = bias
            const int component = entry & 3;
            float total = 0.0f;
#pragma unroll
            for (int source_wave = 0; source_wave < kWaves; ++source_wave) {
#pragma unroll
                for (int source_sub = 0; source_sub < G::kRowsPerWave; ++source_sub) {
                    total += staging[source_wave][source_sub * L + slot][which][component];
                }
            }
            const int column = (v * L + slot) * 4 + component;
            if (write_partials) {
                partials[(static_cast<int64_t>(blockIdx.x) * 2 + which) * H + column] = total;
            } else {
                unsafeAtomicAdd((which ? grad_bias : grad_weight) + column, total);
            }
        }
        __syncthreads();
    }
}

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

// ----------------------------------------------------------------------------
// Host-side launch helpers.

struct ForwardArgs {
    const float* x;
    const void* branch;
    const float* weight;
    const float* bias;
    float* updated;
    void* normalized;
    int normalized_dtype;
    float* mean;
    float* rstd;
    uint32_t* mask;
    int64_t rows;
    float eps;
    int dropout;
    float scale;
    uint32_t threshold;
    PhiloxArgs philox;
    hipStream_t stream;
};

template <int H, typename B, bool Aligned>
int launch_forward(const ForwardArgs& a) {
    const dim3 grid(static_cast<unsigned>(forward_blocks(a.rows, H)));
    rln_forward_kernel<H, B, Aligned><<<grid, kForwardThreads, 0, a.stream>>>(
        a.x,
        static_cast<const B*>(a.branch),
        a.weight,
        a.bias,
        a.updated,
        a.normalized,
        a.normalized_dtype,
        a.mean,
        a.rstd,
        a.mask,
        a.rows,
        a.eps,
        a.dropout,
        a.scale,
        a.threshold,
        a.philox);
    return check_launch("rln_forward_kernel");
}

template <int H, typename B>
int launch_forward_branch(const ForwardArgs& a, bool aligned) {
    return aligned ? launch_forward<H, B, true>(a) : launch_forward<H, B, false>(a);
}

template <int H>
int launch_forward_hidden(const ForwardArgs& a, int branch_dtype, bool aligned) {
    if (branch_dtype == RLN_DTYPE_F16) {
        return launch_forward_branch<H, half_t>(a, aligned);
    }
    if (branch_dtype == RLN_DTYPE_BF16) {
        return launch_forward_branch<H, bf16_t>(a, aligned);
    }
    return launch_forward_branch<H, float>(a, aligned);
}

struct BackwardArgs {
    const float* grad_updated;
    const void* grad_normalized;
    int grad_normalized_dtype;
    const float* updated;
    const float* weight;
    const float* mean;
    const float* rstd;
    const uint32_t* mask;
    float* grad_x;
    void* grad_branch;
    float* grad_weight;
    float* grad_bias;
    float* partials;
    int64_t rows;
    int flags;
    float scale;
    hipStream_t stream;
};

template <int H, typename B, bool Aligned>
int launch_backward(const BackwardArgs& a) {
    const dim3 grid(static_cast<unsigned>(backward_blocks(a.rows, H)));
    rln_backward_kernel<H, B, Aligned><<<grid, kBackwardThreads, 0, a.stream>>>(
        a.grad_updated,
        a.grad_normalized,
        a.grad_normalized_dtype,
        a.updated,
        a.weight,
        a.mean,
        a.rstd,
        a.mask,
        a.grad_x,
        static_cast<B*>(a.grad_branch),
        a.grad_weight,
        a.grad_bias,
        a.partials,
        a.rows,
        a.flags,
        a.scale);
    return check_launch("rln_backward_kernel");
}

template <int H, typename B>
int launch_backward_branch(const BackwardArgs& a, bool aligned) {
    return aligned ? launch_backward<H, B, true>(a) : launch_backward<H, B, false>(a);
}

template <int H>
int launch_backward_hidden(const BackwardArgs& a, int branch_dtype, bool aligned) {
    if (branch_dtype == RLN_DTYPE_F16) {
        return launch_backward_branch<H, half_t>(a, aligned);
    }
    if (branch_dtype == RLN_DTYPE_BF16) {
        return launch_backward_branch<H, bf16_t>(a, aligned);
    }
    return launch_backward_branch<H, float>(a, aligned);
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

// Whether the parameter gradients of this call go through per-block partials
// (and therefore the workspace and the reduce kernel).
bool uses_partials(int deterministic) {
    return deterministic || !RLN_ATOMIC_PARAMETERS;
}

}  // namespace

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
    int64_t rows,
    int64_t hidden,
    double dropout_p,
    double eps,
    int training,
    const rln_philox_t* philox,
    void* stream) {
    t_last_error.clear();
    int status = check_common(rows, hidden, branch_dtype);
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
    a.normalized_dtype = normalized_dtype;
    a.mean = mean;
    a.rstd = rstd;
    a.mask = dropout_mask;
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
        a.philox.seed = philox->seed;
        a.philox.offset = philox->offset;
        a.philox.seed_ptr = philox->seed_ptr;
        a.philox.offset_ptr = philox->offset_ptr;
    }
    const bool aligned = aligned_to(x, 16) && aligned_to(weight, 16) && aligned_to(bias, 16)
        && aligned_to(updated, 16)
        && aligned_to(normalized, vector_alignment(normalized_dtype))
        && aligned_to(branch, vector_alignment(branch_dtype));
    switch (hidden) {
        case 128: return launch_forward_hidden<128>(a, branch_dtype, aligned);
        case 256: return launch_forward_hidden<256>(a, branch_dtype, aligned);
        case 384: return launch_forward_hidden<384>(a, branch_dtype, aligned);
        case 512: return launch_forward_hidden<512>(a, branch_dtype, aligned);
        case 768: return launch_forward_hidden<768>(a, branch_dtype, aligned);
        case 1024: return launch_forward_hidden<1024>(a, branch_dtype, aligned);
        default: break;
    }
    return fail(RLN_ERR_UNSUPPORTED, "unsupported native hidden size: %lld", static_cast<long long>(hidden));
}

size_t rln_backward_workspace_bytes(int64_t rows, int64_t hidden, int deterministic) {
    if (!uses_partials(deterministic) || rows <= 0 || !hidden_supported(hidden)) {
        return 0;
    }
    return static_cast<size_t>(backward_blocks(rows, hidden)) * 2 * static_cast<size_t>(hidden)
        * sizeof(float);
}

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
    t_last_error.clear();
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
    a.grad_normalized_dtype = grad_normalized_dtype;
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
    switch (hidden) {
        case 128: status = launch_backward_hidden<128>(a, branch_dtype, aligned); break;
        case 256: status = launch_backward_hidden<256>(a, branch_dtype, aligned); break;
        case 384: status = launch_backward_hidden<384>(a, branch_dtype, aligned); break;
        case 512: status = launch_backward_hidden<512>(a, branch_dtype, aligned); break;
        case 768: status = launch_backward_hidden<768>(a, branch_dtype, aligned); break;
        case 1024: status = launch_backward_hidden<1024>(a, branch_dtype, aligned); break;
        default:
            return fail(RLN_ERR_UNSUPPORTED, "unsupported native hidden size: %lld", static_cast<long long>(hidden));
    }
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

uint64_t rln_philox_increment(int64_t hidden) {
    (void)hidden;
    return 4;
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
    const int count = static_cast<int>(sizeof(kSupportedHidden) / sizeof(kSupportedHidden[0]));
    for (int index = 0; index < count && index < capacity && out != nullptr; ++index) {
        out[index] = kSupportedHidden[index];
    }
    return count;
}

const char* rln_last_error(void) {
    return t_last_error.c_str();
}

const char* rln_target_arch(void) {
    return "gfx950";
}

const char* rln_version(void) {
    return "0.2.0";
}

}  // extern "C"
