// Fused residual-add + dropout + LayerNorm for MI355X (gfx950, CDNA4): the
// device kernels and their launchers, shared by the per-hidden-size
// translation units (rln_hidden.hip) and the C ABI (rln_api.hip, declared in
// include/rln.h). The operator is the
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

#ifndef RLN_DEVICE_H
#define RLN_DEVICE_H

#include <hip/hip_runtime.h>

#include <cstdint>

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
// Launches over at least this many elements, with rows of at least
// RLN_PACED_MIN_HIDDEN, walk their rows paced rather than with look-ahead.
#ifndef RLN_PACED_ELEMENTS
#define RLN_PACED_ELEMENTS (1ll << 23)
#endif
#ifndef RLN_PACED_MIN_HIDDEN
#define RLN_PACED_MIN_HIDDEN 256
#endif
#ifndef RLN_NT_LOADS
#define RLN_NT_LOADS 1
#endif
#ifndef RLN_NT_STORES
#define RLN_NT_STORES 1
#endif

namespace rln {

constexpr int kWaveSize = 64;
constexpr int kForwardThreads = 256;
constexpr int kBackwardThreads = RLN_BWD_THREADS;
constexpr int64_t kForwardMaxBlocks = RLN_FWD_MAX_BLOCKS;
constexpr int64_t kBackwardMaxBlocks = RLN_BWD_MAX_BLOCKS;
constexpr int64_t kPacedElements = RLN_PACED_ELEMENTS;
constexpr int64_t kPacedMinHidden = RLN_PACED_MIN_HIDDEN;
static_assert(kBackwardThreads % kWaveSize == 0 && kBackwardThreads <= 1024, "backward block");

constexpr int64_t kSupportedHidden[] = {128, 256, 384, 512, 768, 1024};

using half_t = _Float16;
using bf16_t = __bf16;
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

// ----------------------------------------------------------------------------
// Error reporting (defined in rln_api.hip): `fail` records a message for
// rln_last_error() and returns `code`; `check_launch` turns a launch error
// into RLN_ERR_HIP.
int fail(int code, const char* format, ...);
int check_launch(const char* what);

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

inline int64_t rows_per_wave(int64_t hidden) {
    return ((hidden / 4) % kWaveSize == 0) ? 1 : 2;
}

// Blocks for a launch over `rows`: enough for `groups_per_wave` row groups
// per wave (a group = the rows one wave handles at once), capped; a function
// of (rows, hidden) only.
inline int64_t launch_blocks(int64_t rows, int64_t hidden, int threads, int64_t cap,
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
inline int64_t forward_blocks(int64_t rows, int64_t hidden) {
    return launch_blocks(rows, hidden, kForwardThreads, kForwardMaxBlocks, 2);
}

// The backward's grid is also the number of weight/bias partials: 256
// blocks of 8 waves, one block per CU.
inline int64_t backward_blocks(int64_t rows, int64_t hidden) {
    return launch_blocks(rows, hidden, kBackwardThreads, kBackwardMaxBlocks, 1);
}

// 1 if a launch over rows x hidden walks its rows paced (measured on MI355X:
// faster from about 8 M elements at hidden >= 256, neutral below, slower at
// C1-sized launches), 0 for look-ahead.
inline int paced_schedule(int64_t rows, int64_t hidden) {
    return hidden >= kPacedMinHidden && rows * hidden >= kPacedElements ? 1 : 0;
}

inline bool hidden_supported(int64_t hidden) {
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

// Four consecutive elements of type T in their storage type, unconverted.
// Row loads keep this form so that no arithmetic (and hence no wait for the
// load) happens until the row is processed.
template <typename T, bool Aligned>
__device__ __forceinline__ typename Vector4<T>::type load_raw4(const T* __restrict__ pointer) {
    using Raw = typename Vector4<T>::type;
    if constexpr (Aligned) {
        return stream_load(reinterpret_cast<const Raw*>(pointer));
    } else {
        Raw raw;
        raw.x = stream_load(pointer);
        raw.y = stream_load(pointer + 1);
        raw.z = stream_load(pointer + 2);
        raw.w = stream_load(pointer + 3);
        return raw;
    }
}

template <typename T>
__device__ __forceinline__ f32x4 widen4(typename Vector4<T>::type raw) {
    return __builtin_convertvector(raw, f32x4);
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

// The global values the forward reads for one row, held in registers in
// their storage types.
template <int V, typename B>
struct ForwardRow {
    f32x4 x[V];
    typename Vector4<B>::type branch[V];
};

template <int H, typename B, typename N, bool Aligned>
__global__ __launch_bounds__(kForwardThreads)
void rln_forward_kernel(
    const float* __restrict__ x,
    const B* __restrict__ branch,
    const float* __restrict__ weight,
    const float* __restrict__ bias,
    float* __restrict__ updated,
    N* __restrict__ normalized,
    float* __restrict__ mean_out,
    float* __restrict__ rstd_out,
    uint32_t* __restrict__ mask,
    int64_t rows,
    float eps,
    int dropout,
    float scale,
    uint32_t threshold,
    PhiloxArgs philox,
    int paced) {
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

    // Loads x and the branch of one row. The loads are unconditional (a
    // half-wave row past the end reads the last row instead and discards it),
    // so the compiler can count them and wait for exactly the ones a
    // computation needs; a load under a branch makes it wait for all.
    auto load_row = [&](ForwardRow<V, B>& r, int64_t row, bool wait_slices) {
        const int64_t source = row < rows ? row : rows - 1;
        const float* x_row = x + source * H;
        const B* branch_row = branch + source * H;
#pragma unroll
        for (int v = 0; v < V; ++v) {
            const int column = (v * L + l) * 4;
            r.x[v] = load4<Aligned>(x_row + column);
            r.branch[v] = load_raw4<B, Aligned>(branch_row + column);
            if (wait_slices) {
                __builtin_amdgcn_s_waitcnt(0);
            }
        }
    };

    auto process_row = [&](const ForwardRow<V, B>& r, int64_t row) {
        const bool valid = row < rows;
        const int64_t base = row * H;
        f32x4 u[V];
        uint32_t keep_bits[V];
#pragma unroll
        for (int v = 0; v < V; ++v) {
            f32x4 bv = widen4<B>(r.branch[v]);
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
                store_convert4<N, Aligned>(normalized + base + column, y);
            }
        }
    };

    // Two schedules. Look-ahead (small launches): the next row's loads are
    // in flight while the current row is computed and stored. Paced (large
    // launches): a row is loaded after the previous one is stored, one
    // 4-column slice at a time, each waited for (with every earlier store of
    // the wave), which keeps fewer reads and writes interleaved per wave and
    // streams large tensors faster. The last row of a wave is peeled off, so
    // no load reaches past the wave's rows.
    const int64_t stride = wave_count * G::kRowsPerWave;
    int64_t first = wave * G::kRowsPerWave;
    if (first >= rows) {
        return;
    }
    ForwardRow<V, B> current;
    load_row(current, first + sub, false);
    if (paced) {
        for (; first + stride < rows; first += stride) {
            process_row(current, first + sub);
            load_row(current, first + stride + sub, true);
        }
    } else {
        for (; first + stride < rows; first += stride) {
            ForwardRow<V, B> next;
            load_row(next, first + stride + sub, false);
            process_row(current, first + sub);
            current = next;
        }
    }
    process_row(current, first + sub);
}

// ----------------------------------------------------------------------------
// Backward kernel: input gradients plus per-block weight/bias partial sums.

// Every global value the backward reads for one row, held in registers.
template <int V, typename GY>
struct BackwardRow {
    f32x4 u[V];
    typename Vector4<GY>::type gy[V];  // storage type, widened when processed
    f32x4 gu[V];
    uint32_t mask_word[V];  // whole word; the lane's nibble is taken when processed
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

template <int H, typename B, typename GY, bool Aligned>
__global__ __launch_bounds__(kBackwardThreads)
void rln_backward_kernel(
    const float* __restrict__ grad_updated,
    const GY* __restrict__ grad_normalized,
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
    float scale,
    int paced) {
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

    // Loads every global value of one row. The loads are unconditional, so
    // the compiler can count them and wait for exactly the ones a computation
    // needs (a load under a branch makes it wait for all): an absent input
    // reads the row of `updated` in its place, and a half-wave row past the
    // end reads the last row; process_row discards what it read.
    auto load_row = [&](BackwardRow<V, GY>& r, int64_t row, bool wait_slices) {
        const int64_t source = row < rows ? row : rows - 1;
        const int64_t base = source * H;
        const float* u_row = updated + base;
        const GY* gy_row = has_gy ? grad_normalized + base : reinterpret_cast<const GY*>(u_row);
        const float* gu_row = has_gu ? grad_updated + base : u_row;
        const uint32_t* mask_row = dropout ? mask + source * G::kMaskWords
                                           : reinterpret_cast<const uint32_t*>(u_row);
        r.mean = mean_in[source];
        r.rstd = rstd_in[source];
#pragma unroll
        for (int v = 0; v < V; ++v) {
            const int column = (v * L + l) * 4;
            r.u[v] = load4<Aligned>(u_row + column);
            r.gy[v] = load_raw4<GY, Aligned>(gy_row + column);
            r.gu[v] = load4<Aligned>(gu_row + column);
            r.mask_word[v] = mask_row[(v * L + l) / 8];
            if (wait_slices) {
                __builtin_amdgcn_s_waitcnt(0);
            }
        }
    };

    // Input gradients of one row and its contribution to the parameter sums.
    auto process_row = [&](const BackwardRow<V, GY>& r, int64_t row) {
        const bool valid = row < rows;
        const int64_t base = row * H;
        f32x4 xhat[V];
        f32x4 gy[V];
        float sum_q = 0.0f;
        float sum_qx = 0.0f;
        // Inputs that were not given, and every input of a row past the end,
        // count as zero.
        const bool use_gy = has_gy && valid;
#pragma unroll
        for (int v = 0; v < V; ++v) {
            gy[v] = use_gy ? widen4<GY>(r.gy[v]) : zero4();
            xhat[v] = (r.u[v] - r.mean) * r.rstd;
            const f32x4 q = gy[v] * w[v];
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
                f32x4 g = has_gu ? r.gu[v] : zero4();
                if (has_gy) {
                    const f32x4 q = gy[v] * w[v];
                    g = g + r.rstd * ((q - mean_q) - xhat[v] * mean_qx);
                }
                store4<Aligned>(grad_x + base + column, g);
                if (dropout) {
                    const uint32_t bits = r.mask_word[v] >> (4 * (l & 7));
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
                acc_w[v].x = __builtin_fmaf(gy[v].x, xhat[v].x, acc_w[v].x);
                acc_w[v].y = __builtin_fmaf(gy[v].y, xhat[v].y, acc_w[v].y);
                acc_w[v].z = __builtin_fmaf(gy[v].z, xhat[v].z, acc_w[v].z);
                acc_w[v].w = __builtin_fmaf(gy[v].w, xhat[v].w, acc_w[v].w);
                acc_b[v] = acc_b[v] + gy[v];
            }
        }
    };

    // Each wave walks its rows under one of two schedules: look-ahead (the
    // next row's loads in flight while the current row is reduced and stored;
    // small launches) or paced (a row loaded after the previous one is
    // stored, one 4-column slice at a time, each waited for; large launches,
    // where fewer interleaved reads and writes per wave stream faster). The
    // last row of a wave is peeled off, so no load reaches past the wave's
    // rows. A wave without rows still takes part in the block's combine.
    const int64_t stride = wave_count * G::kRowsPerWave;
    int64_t first = wave * G::kRowsPerWave;
    if (first < rows) {
        BackwardRow<V, GY> current;
        load_row(current, first + sub, false);
        if (paced) {
            for (; first + stride < rows; first += stride) {
                process_row(current, first + sub);
                load_row(current, first + stride + sub, true);
            }
        } else {
            for (; first + stride < rows; first += stride) {
                BackwardRow<V, GY> next;
                load_row(next, first + stride + sub, false);
                process_row(current, first + sub);
                current = next;
            }
        }
        process_row(current, first + sub);
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

// ----------------------------------------------------------------------------
// Host-side launch helpers.

struct ForwardArgs {
    const float* x;
    const void* branch;
    const float* weight;
    const float* bias;
    float* updated;
    void* normalized;
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

struct BackwardArgs {
    const float* grad_updated;
    const void* grad_normalized;
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

template <int H, typename B, typename N, bool Aligned>
int launch_forward(const ForwardArgs& a) {
    const dim3 grid(static_cast<unsigned>(forward_blocks(a.rows, H)));
    rln_forward_kernel<H, B, N, Aligned><<<grid, kForwardThreads, 0, a.stream>>>(
        a.x,
        static_cast<const B*>(a.branch),
        a.weight,
        a.bias,
        a.updated,
        static_cast<N*>(a.normalized),
        a.mean,
        a.rstd,
        a.mask,
        a.rows,
        a.eps,
        a.dropout,
        a.scale,
        a.threshold,
        a.philox,
        paced_schedule(a.rows, H));
    return check_launch("rln_forward_kernel");
}

template <int H, typename B, typename GY, bool Aligned>
int launch_backward(const BackwardArgs& a) {
    const dim3 grid(static_cast<unsigned>(backward_blocks(a.rows, H)));
    rln_backward_kernel<H, B, GY, Aligned><<<grid, kBackwardThreads, 0, a.stream>>>(
        a.grad_updated,
        static_cast<const GY*>(a.grad_normalized),
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
        a.scale,
        paced_schedule(a.rows, H));
    return check_launch("rln_backward_kernel");
}

// Calls `launch.template operator()<T>()` with T the element type of `dtype`.
template <typename Launch>
int with_dtype(int dtype, Launch&& launch) {
    if (dtype == RLN_DTYPE_F16) {
        return launch.template operator()<half_t>();
    }
    if (dtype == RLN_DTYPE_BF16) {
        return launch.template operator()<bf16_t>();
    }
    return launch.template operator()<float>();
}

// Every (branch, normalized, alignment) instantiation for one hidden size;
// explicitly instantiated once per H in rln_hidden.hip.
template <int H>
int launch_forward_hidden(const ForwardArgs& a, int branch_dtype, int normalized_dtype,
                          bool aligned) {
    return with_dtype(branch_dtype, [&]<typename B>() {
        return with_dtype(normalized_dtype, [&]<typename N>() {
            return aligned ? launch_forward<H, B, N, true>(a) : launch_forward<H, B, N, false>(a);
        });
    });
}

template <int H>
int launch_backward_hidden(const BackwardArgs& a, int branch_dtype, int grad_normalized_dtype,
                           bool aligned) {
    return with_dtype(branch_dtype, [&]<typename B>() {
        return with_dtype(grad_normalized_dtype, [&]<typename GY>() {
            return aligned ? launch_backward<H, B, GY, true>(a)
                           : launch_backward<H, B, GY, false>(a);
        });
    });
}

#define RLN_FOR_EACH_HIDDEN(X) X(128) X(256) X(384) X(512) X(768) X(1024)

#define RLN_DECLARE_HIDDEN(H)                                                            \
    extern template int launch_forward_hidden<H>(const ForwardArgs&, int, int, bool);    \
    extern template int launch_backward_hidden<H>(const BackwardArgs&, int, int, bool);

}  // namespace rln

#endif  // RLN_DEVICE_H
