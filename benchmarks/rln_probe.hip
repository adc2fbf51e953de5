// Streaming probe for the benchmark (benchmarks/librln_probe_gfx950.so,
// loaded by bench.py only; the operator never calls it). Each kernel moves
// exactly the bytes of one pass of the fused residual LayerNorm over
// [rows, hidden], with no row reductions and no dropout draws:
//
//   forward:  reads x (fp32), branch; writes updated (fp32), normalized,
//             one mask word per 32 columns, mean and rstd per row;
//   backward: reads grad_updated (fp32), grad_normalized, updated (fp32),
//             the mask word of each 32 columns, mean and rstd per row;
//             writes grad_x (fp32), grad_branch.
//
// The stream configuration is a template argument (Cfg bits): the branch and
// grad_branch 16-bit (the headline configuration, Cfg 0) or fp32 (bit 0);
// normalized and grad_normalized fp32 or 16-bit (bit 1); the mask written
// and read (training with dropout) or absent (bit 2).
//
// The variants span the launch and access choices a streaming kernel has on
// MI355X, so that the fastest of them is a measured floor for the bytes of
// one pass at a given size, not one untuned shape:
//
//   * block size T (256, 512 or 1024 threads);
//   * U four-column units per lane per step (1-4: bytes in flight per lane
//     and stream, 16 B each for the fp32 streams);
//   * look-ahead (the next step's loads issued before the current step is
//     stored) or not;
//   * "wide" fp16: a lane owns 8 consecutive columns per pair of units, so
//     the fp16 stream moves in 128-bit accesses (the fp32 streams then in two
//     128-bit accesses 32 B apart per lane);
//   * cache policy of the loads and stores: the gfx950 buffer instructions'
//     sc0 / sc1 / nt bits;
//   * backward only: the three fp32 load streams through LDS with gfx950's
//     direct-to-LDS buffer loads (no VGPRs held by loads in flight);
//   * the grid: one step per thread (blocks replaced by the dispatcher as
//     they finish), or a persistent grid of a given number of waves per CU
//     walking the units with a grid stride (set by the caller).
//
// Every access is a buffer instruction whose descriptor covers exactly its
// tensor: a unit past the end reads zeros and its stores are dropped by the
// hardware range check, so a grid may overrun the last step safely. The
// arithmetic only combines the loaded values so that no access can be
// dropped by the compiler; its results are meaningless.

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
using rsrc_t = __amdgpu_buffer_rsrc_t;

// Cache-policy bits of a gfx950 buffer instruction's immediate, the values
// of the variants' LoadAux / StoreAux: sc0 = 1, nt = 2, sc1 = 16. kLds is
// not an instruction bit: the backward's fp32 load streams go through LDS.
constexpr int kLds = 256;

// The descriptor's fourth word for a raw (untyped, unswizzled) buffer on
// gfx9-family parts.
constexpr int kRsrcWord3 = 0x00020000;

__device__ __forceinline__ rsrc_t make_rsrc(const void* pointer, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(pointer), 0, bytes, kRsrcWord3);
}

template <int Aux>
__device__ __forceinline__ f32x4 load128(rsrc_t r, uint32_t offset) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, Aux & 0xFF));
}
template <int Aux>
__device__ __forceinline__ u32x2 load64(rsrc_t r, uint32_t offset) {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, offset, 0, Aux & 0xFF));
}
template <int Aux>
__device__ __forceinline__ u32x4 load128u(rsrc_t r, uint32_t offset) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, Aux & 0xFF);
}
template <int Aux>
__device__ __forceinline__ uint32_t load32(rsrc_t r, uint32_t offset) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, offset, 0, Aux & 0xFF);
}
template <int Aux>
__device__ __forceinline__ void store128(rsrc_t r, uint32_t offset, f32x4 value) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, value), r, offset, 0,
                                           Aux & 0xFF);
}
template <int Aux>
__device__ __forceinline__ void store128u(rsrc_t r, uint32_t offset, u32x4 value) {
    __builtin_amdgcn_raw_buffer_store_b128(value, r, offset, 0, Aux & 0xFF);
}
template <int Aux>
__device__ __forceinline__ void store64(rsrc_t r, uint32_t offset, u32x2 value) {
    __builtin_amdgcn_raw_buffer_store_b64(value, r, offset, 0, Aux & 0xFF);
}
template <int Aux>
__device__ __forceinline__ void store32(rsrc_t r, uint32_t offset, uint32_t value) {
    __builtin_amdgcn_raw_buffer_store_b32(value, r, offset, 0, Aux & 0xFF);
}

__device__ __forceinline__ f32x4 widen(u32x2 raw) {
    return __builtin_convertvector(__builtin_bit_cast(f16x4, raw), f32x4);
}
__device__ __forceinline__ u32x2 narrow(f32x4 value) {
    return __builtin_bit_cast(u32x2, __builtin_convertvector(value, f16x4));
}

struct ProbeBuffers {
    // forward
    const float* x;
    const void* branch;  // fp16
    float* updated_out;
    float* normalized;
    uint32_t* mask_out;
    float* mean_out;
    float* rstd_out;
    // backward
    const float* grad_updated;
    const float* grad_normalized;
    const float* updated;
    const uint32_t* mask;
    const float* mean;
    const float* rstd;
    float* grad_x;
    void* grad_branch;  // fp16
};

struct Geometry {
    uint32_t units;      // four-column units in the tensor
    uint32_t row_units;  // units per row
    uint32_t rows;
};

// The streams of stream configuration Cfg.
template <int Cfg>
struct Streams {
    static constexpr bool kBranch32 = (Cfg & 1) != 0;  // branch, grad_branch fp32
    static constexpr bool kNorm16 = (Cfg & 2) != 0;    // normalized, grad_normalized 16-bit
    static constexpr bool kMask = (Cfg & 4) == 0;      // mask written / read
    static constexpr uint32_t kBranchBytes = kBranch32 ? 16 : 8;  // per four-column unit
    static constexpr uint32_t kNormBytes = kNorm16 ? 8 : 16;
};

// Unit index of slot k of this lane in the step starting at `base`.
template <int T, int U, bool Wide>
__device__ __forceinline__ uint32_t unit_of(uint32_t base, int k) {
    if constexpr (Wide) {
        return base + (k / 2) * 2 * T + 2 * threadIdx.x + (k & 1);
    } else {
        return base + k * T + threadIdx.x;
    }
}

template <int T, int U, int LoadAux, int StoreAux, bool Ahead, bool Wide, int Cfg>
__global__ __launch_bounds__(T) void probe_forward(ProbeBuffers b, Geometry g) {
    using C = Streams<Cfg>;
    static_assert(!Wide || U % 2 == 0, "wide fp16 takes unit pairs");
    static_assert(!Wide || !C::kBranch32, "wide applies to a 16-bit branch");
    const rsrc_t rx = make_rsrc(b.x, g.units * 16);
    const rsrc_t rb = make_rsrc(b.branch, g.units * C::kBranchBytes);
    const rsrc_t ru = make_rsrc(b.updated_out, g.units * 16);
    const rsrc_t rn = make_rsrc(b.normalized, g.units * C::kNormBytes);
    const rsrc_t rm = make_rsrc(b.mask_out, C::kMask ? g.units / 2 : 0);
    const rsrc_t rmean = make_rsrc(b.mean_out, g.rows * 4);
    const rsrc_t rrstd = make_rsrc(b.rstd_out, g.rows * 4);
    struct Regs {
        f32x4 x[U];
        u32x2 br[Wide || C::kBranch32 ? 1 : U];
        u32x4 br32[C::kBranch32 ? U : 1];
        u32x4 wide[Wide ? U / 2 : 1];
    };
    auto load = [&](Regs& r, uint32_t base) {
#pragma unroll
        for (int k = 0; k < U; ++k) {
            const uint32_t j = unit_of<T, U, Wide>(base, k);
            r.x[k] = load128<LoadAux>(rx, j * 16);
            if constexpr (C::kBranch32) {
                r.br32[k] = load128u<LoadAux>(rb, j * 16);
            } else if constexpr (Wide) {
                if ((k & 1) == 0) {
                    r.wide[k / 2] = load128u<LoadAux>(rb, j * 8);
                }
            } else {
                r.br[k] = load64<LoadAux>(rb, j * 8);
            }
        }
    };
    auto process = [&](const Regs& r, uint32_t base) {
#pragma unroll
        for (int k = 0; k < U; ++k) {
            const uint32_t j = unit_of<T, U, Wide>(base, k);
            f32x4 branch;
            if constexpr (C::kBranch32) {
                branch = __builtin_bit_cast(f32x4, r.br32[k]);
            } else if constexpr (Wide) {
                const u32x4 pair = r.wide[k / 2];
                branch = widen((k & 1) ? u32x2{pair.z, pair.w} : u32x2{pair.x, pair.y});
            } else {
                branch = widen(r.br[k]);
            }
            const f32x4 u = r.x[k] + branch;
            store128<StoreAux>(ru, j * 16, u);
            if constexpr (C::kNorm16) {
                store64<StoreAux>(rn, j * 8, narrow(u * 0.5f));
            } else {
                store128<StoreAux>(rn, j * 16, u * 0.5f);
            }
            // (Scalar copies: clang's __builtin_bit_cast of a vector element
            // expression reads element 0.)
            const float u0 = u.x, u1 = u.y, u2 = u.z;
            if (C::kMask && (j & 7) == 0) {
                store32<StoreAux>(rm, (j / 8) * 4, __builtin_bit_cast(uint32_t, u0));
            }
            if (j % g.row_units == 0) {
                const uint32_t row = j / g.row_units;
                store32<StoreAux>(rmean, row * 4, __builtin_bit_cast(uint32_t, u1));
                store32<StoreAux>(rrstd, row * 4, __builtin_bit_cast(uint32_t, u2));
            }
        }
    };
    const uint32_t stride = gridDim.x * T * U;
    uint32_t base = blockIdx.x * T * U;
    if (base >= g.units) {
        return;
    }
    Regs current;
    load(current, base);
    for (; base + stride < g.units; base += stride) {
        if constexpr (Ahead) {
            Regs next;
            load(next, base + stride);
            process(current, base);
            current = next;
        } else {
            process(current, base);
            load(current, base + stride);
        }
    }
    process(current, base);
}

template <int T, int U, int LoadAux, int StoreAux, bool Ahead, bool Wide, int Cfg>
__global__ __launch_bounds__(T) void probe_backward(ProbeBuffers b, Geometry g) {
    using C = Streams<Cfg>;
    static_assert(!Wide || U % 2 == 0, "wide fp16 takes unit pairs");
    static_assert(!Wide || !C::kBranch32, "wide applies to a 16-bit branch");
    constexpr bool kViaLds = (LoadAux & kLds) != 0;
    static_assert(!kViaLds || !C::kNorm16, "the LDS path stages three fp32 streams");
    const rsrc_t rgu = make_rsrc(b.grad_updated, g.units * 16);
    const rsrc_t rgy = make_rsrc(b.grad_normalized, g.units * C::kNormBytes);
    const rsrc_t ru = make_rsrc(b.updated, g.units * 16);
    const rsrc_t rm = make_rsrc(b.mask, C::kMask ? g.units / 2 : 0);
    const rsrc_t rmean = make_rsrc(b.mean, g.rows * 4);
    const rsrc_t rrstd = make_rsrc(b.rstd, g.rows * 4);
    const rsrc_t rgx = make_rsrc(b.grad_x, g.units * 16);
    const rsrc_t rgb = make_rsrc(b.grad_branch, g.units * C::kBranchBytes);
    // LDS staging for the direct-to-LDS variant: per wave, two buffers of
    // three streams x U units x 64 lanes x 16 B.
    constexpr int kWaves = T / 64;
    __shared__ f32x4 stage[kViaLds ? kWaves : 1][kViaLds ? 2 : 1][kViaLds ? 3 * U : 1][64];
    const int wave = threadIdx.x / 64;
    const int lane = threadIdx.x % 64;

    struct Regs {
        f32x4 gu[kViaLds ? 1 : U];
        f32x4 gy[kViaLds || C::kNorm16 ? 1 : U];
        u32x2 gy16[C::kNorm16 ? U : 1];
        f32x4 u[kViaLds ? 1 : U];
        uint32_t word[U];
        float mean[U];
        float rstd[U];
    };
    auto load = [&](Regs& r, uint32_t base, int buffer) {
#pragma unroll
        for (int k = 0; k < U; ++k) {
            const uint32_t j = unit_of<T, U, Wide>(base, k);
            if constexpr (kViaLds) {
                using lds_ptr = __attribute__((address_space(3))) void*;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rgu, (lds_ptr)(&stage[wave][buffer][3 * k + 0][0]), 16, j * 16, 0, 0,
                    LoadAux & 0xFF);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rgy, (lds_ptr)(&stage[wave][buffer][3 * k + 1][0]), 16, j * 16, 0, 0,
                    LoadAux & 0xFF);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    ru, (lds_ptr)(&stage[wave][buffer][3 * k + 2][0]), 16, j * 16, 0, 0,
                    LoadAux & 0xFF);
            } else {
                r.gu[k] = load128<LoadAux>(rgu, j * 16);
                if constexpr (C::kNorm16) {
                    r.gy16[k] = load64<LoadAux>(rgy, j * 8);
                } else {
                    r.gy[k] = load128<LoadAux>(rgy, j * 16);
                }
                r.u[k] = load128<LoadAux>(ru, j * 16);
            }
            r.word[k] = C::kMask ? load32<0>(rm, (j / 8) * 4) : 1u;
            const uint32_t row = j / g.row_units;
            r.mean[k] = __builtin_bit_cast(float, load32<0>(rmean, row * 4));
            r.rstd[k] = __builtin_bit_cast(float, load32<0>(rrstd, row * 4));
        }
    };
    auto process = [&](const Regs& r, uint32_t base, int buffer) {
        f32x4 grad[U];
#pragma unroll
        for (int k = 0; k < U; ++k) {
            f32x4 gu, gy, u;
            if constexpr (kViaLds) {
                gu = stage[wave][buffer][3 * k + 0][lane];
                gy = stage[wave][buffer][3 * k + 1][lane];
                u = stage[wave][buffer][3 * k + 2][lane];
            } else {
                gu = r.gu[k];
                if constexpr (C::kNorm16) {
                    gy = widen(r.gy16[k]);
                } else {
                    gy = r.gy[k];
                }
                u = r.u[k];
            }
            grad[k] = (gu + gy * (u - r.mean[k] * r.rstd[k]))
                * static_cast<float>(r.word[k] & 1u);
        }
#pragma unroll
        for (int k = 0; k < U; ++k) {
            const uint32_t j = unit_of<T, U, Wide>(base, k);
            store128<StoreAux>(rgx, j * 16, grad[k]);
            if constexpr (C::kBranch32) {
                store128<StoreAux>(rgb, j * 16, grad[k]);
            } else if constexpr (Wide) {
                if ((k & 1) == 0) {
                    const u32x2 lo = narrow(grad[k]);
                    const u32x2 hi = narrow(grad[k + 1]);
                    store128u<StoreAux>(rgb, j * 8, u32x4{lo.x, lo.y, hi.x, hi.y});
                }
            } else {
                store64<StoreAux>(rgb, j * 8, narrow(grad[k]));
            }
        }
    };
    // Waits until at most `pending` vector memory operations of this wave
    // are outstanding (the direct-to-LDS loads count there, and the LDS
    // reads must come after them).
    auto wait_vm = [](auto pending) {
        constexpr int n = decltype(pending)::value;
        __builtin_amdgcn_s_waitcnt((n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14));
    };
    const uint32_t stride = gridDim.x * T * U;
    uint32_t base = blockIdx.x * T * U;
    if (base >= g.units) {
        return;
    }
    Regs current;
    int buffer = 0;
    load(current, base, buffer);
    for (; base + stride < g.units; base += stride) {
        if constexpr (Ahead) {
            Regs next;
            load(next, base + stride, buffer ^ 1);
            if constexpr (kViaLds) {
                // The next step's loads (six per unit, five without the
                // mask) may stay in flight.
                wait_vm(std::integral_constant<int, (C::kMask ? 6 : 5) * U>{});
            }
            process(current, base, buffer);
            current = next;
            buffer ^= 1;
        } else {
            if constexpr (kViaLds) {
                wait_vm(std::integral_constant<int, 0>{});
            }
            process(current, base, buffer);
            load(current, base + stride, buffer);
        }
    }
    if constexpr (kViaLds) {
        wait_vm(std::integral_constant<int, 0>{});
    }
    process(current, base, buffer);
}

__global__ __launch_bounds__(256) void probe_empty(ProbeBuffers, Geometry) {}

// The backward's weight/bias combine alone: each of the grid's 512-thread
// blocks adds 2 x hidden floats (weight and bias sums of every column, eight
// floats per lane owner as the operator's combine orders them) with fp32
// atomics into one copy of a [copies, 2, hidden] buffer: copy blockIdx %
// copies (interleaved: consecutive blocks, which the dispatcher spreads over
// the XCDs, add into different copies) or blockIdx * copies / gridDim.x
// (ranges: consecutive blocks share a copy).
__global__ __launch_bounds__(512) void probe_atomic_combine(float* sums, int hidden,
                                                            int copies, int ranges) {
    const int copy = ranges ? static_cast<int>(static_cast<int64_t>(blockIdx.x) * copies
                                               / gridDim.x)
                            : static_cast<int>(blockIdx.x % copies);
    float* target = sums + static_cast<int64_t>(copy) * 2 * hidden;
    for (int entry = threadIdx.x; entry < 2 * hidden; entry += 512) {
        const int owner = entry / 8;
        const int which = (entry / 4) & 1;
        const int column = owner * 4 + (entry & 3);
        unsafeAtomicAdd(target + which * hidden + column, 1.0f);
    }
}

// The same combine through buffer atomics carrying the cache-policy bits
// `Aux` (sc0 = 1 asks for the pre-op value, nt = 2, sc1 = 16), into one copy.
template <int Aux>
__global__ __launch_bounds__(512) void probe_atomic_policy(float* sums, int hidden) {
    const rsrc_t r = make_rsrc(sums, 2 * hidden * 4);
    for (int entry = threadIdx.x; entry < 2 * hidden; entry += 512) {
        const int owner = entry / 8;
        const int which = (entry / 4) & 1;
        const int column = owner * 4 + (entry & 3);
        __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(1.0f, r, (which * hidden + column) * 4, 0,
                                                    Aux);
    }
}

// The combine as a fold inside one launch: each 512-thread block adds its
// 2 x hidden values (1.0 each) with fp32 atomics into copy blockIdx % copies
// of `sums` ([copies, 2, hidden]), makes them visible at agent scope
// (release fence by every wave, then a block barrier) and takes a ticket
// from `counter`; the block that takes the last ticket (acquire fence) swaps
// every copy's values for zeros, adds their total into `out` ([2, hidden])
// and resets the counter, so that `sums` and `counter` are zero again for
// the next launch. After n launches of g blocks, out holds g * n per value.
constexpr int kFoldCopies = 16;

__global__ __launch_bounds__(512) void probe_atomic_fold(float* sums, float* out,
                                                         uint32_t* counter, int hidden,
                                                         int copies) {
    const int copy = static_cast<int>(blockIdx.x % copies);
    float* target = sums + static_cast<int64_t>(copy) * 2 * hidden;
    for (int entry = threadIdx.x; entry < 2 * hidden; entry += 512) {
        const int owner = entry / 8;
        const int which = (entry / 4) & 1;
        const int column = owner * 4 + (entry & 3);
        unsafeAtomicAdd(target + which * hidden + column, 1.0f);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __shared__ uint32_t ticket;
    __syncthreads();
    if (threadIdx.x == 0) {
        ticket = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (ticket != gridDim.x - 1) {
        return;
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    // Every swap of a column is issued before any is waited for (at most
    // kFoldCopies copies).
    for (int i = threadIdx.x; i < 2 * hidden; i += 512) {
        float values[kFoldCopies];
#pragma unroll
        for (int k = 0; k < kFoldCopies; ++k) {
            values[k] = k < copies
                ? __hip_atomic_exchange(sums + static_cast<int64_t>(k) * 2 * hidden + i, 0.0f,
                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                : 0.0f;
        }
        float total = 0.0f;
#pragma unroll
        for (int k = 0; k < kFoldCopies; ++k) {
            total += values[k];
        }
        unsafeAtomicAdd(out + i, total);
    }
    if (threadIdx.x == 0) {
        __hip_atomic_exchange(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// A kernel of `blocks` blocks doing nothing, for the per-launch cost.
__global__ void probe_nothing(int) {}

enum Kind { kForward = 0, kBackward = 1, kEmpty = 2 };

struct Variant {
    const char* name;
    int kind;
    int threads;
    int units_per_lane;
    void (*kernel)(ProbeBuffers, Geometry);
    int config;  // the Cfg bits of its streams
};

#define PROBE_F(T, U, L, S, A, W)                                                      \
    {"fwd t" #T " u" #U " ld" #L " st" #S " ahead" #A " wide" #W, kForward, T, U,      \
     &probe_forward<T, U, L, S, A, W, 0>, 0},
#define PROBE_B(T, U, L, S, A, W)                                                      \
    {"bwd t" #T " u" #U " ld" #L " st" #S " ahead" #A " wide" #W, kBackward, T, U,     \
     &probe_backward<T, U, L, S, A, W, 0>, 0},
// Variants of the other stream configurations: the name carries the
// configuration ("b32": fp32 branch, "n16": 16-bit normalized, "nomask").
#define PROBE_FC(T, U, L, S, A, W, C, SUFFIX)                                          \
    {"fwd t" #T " u" #U " ld" #L " st" #S " ahead" #A " wide" #W SUFFIX, kForward, T, U, \
     &probe_forward<T, U, L, S, A, W, C>, C},
#define PROBE_BC(T, U, L, S, A, W, C, SUFFIX)                                          \
    {"bwd t" #T " u" #U " ld" #L " st" #S " ahead" #A " wide" #W SUFFIX, kBackward, T, U, \
     &probe_backward<T, U, L, S, A, W, C>, C},
// Per other stream configuration: one to four units, with and without
// look-ahead, at 256, 512 and 1024 threads, sc0 | sc1 stores; two shapes
// with non-temporal stores.
#define PROBE_CONFIG_SHAPES_T(X, T, C, SUFFIX)                                         \
    X(T, 1, 2, 17, 0, 0, C, SUFFIX) X(T, 1, 2, 17, 1, 0, C, SUFFIX)                    \
    X(T, 2, 2, 17, 0, 0, C, SUFFIX) X(T, 2, 2, 17, 1, 0, C, SUFFIX)                    \
    X(T, 4, 2, 17, 0, 0, C, SUFFIX) X(T, 4, 2, 17, 1, 0, C, SUFFIX)
#define PROBE_CONFIG_SHAPES(X, C, SUFFIX)                                              \
    PROBE_CONFIG_SHAPES_T(X, 256, C, SUFFIX) PROBE_CONFIG_SHAPES_T(X, 512, C, SUFFIX)  \
    PROBE_CONFIG_SHAPES_T(X, 1024, C, SUFFIX)                                          \
    X(256, 2, 2, 2, 1, 0, C, SUFFIX) X(256, 1, 2, 2, 0, 0, C, SUFFIX)
// The backward's LDS-staged loads where grad_normalized is fp32.
#define PROBE_CONFIG_LDS(C, SUFFIX)                                                    \
    PROBE_BC(256, 1, 258, 17, 0, 0, C, SUFFIX) PROBE_BC(256, 1, 258, 17, 1, 0, C, SUFFIX) \
    PROBE_BC(512, 1, 258, 17, 0, 0, C, SUFFIX)
// Shapes with non-temporal loads and sc0 | sc1 stores (the operator's policy).
#define PROBE_SHAPES(X, T)                                                             \
    X(T, 1, 2, 17, 0, 0) X(T, 1, 2, 17, 1, 0) X(T, 2, 2, 17, 0, 0) X(T, 2, 2, 17, 1, 0)    \
    X(T, 3, 2, 17, 0, 0) X(T, 3, 2, 17, 1, 0) X(T, 4, 2, 17, 0, 0) X(T, 4, 2, 17, 1, 0)    \
    X(T, 2, 2, 17, 0, 1) X(T, 2, 2, 17, 1, 1) X(T, 4, 2, 17, 0, 1) X(T, 4, 2, 17, 1, 1)
// Cache policies at 256 threads, two units, look-ahead: loads plain / nt /
// sc1; stores plain, nt, nt + sc1, sc0 + sc1 + nt (sc0 + sc1 is in the
// shapes above).
#define PROBE_POLICIES(X)                                                              \
    X(256, 2, 0, 0, 1, 0) X(256, 2, 0, 2, 1, 0) X(256, 2, 2, 0, 1, 0)                  \
    X(256, 2, 2, 2, 1, 0) X(256, 2, 2, 18, 1, 0) X(256, 2, 2, 19, 1, 0)                \
    X(256, 2, 0, 18, 1, 0) X(256, 2, 16, 17, 1, 0)

const Variant kVariants[] = {
    {"empty t256", kEmpty, 256, 1, &probe_empty, 0},
    PROBE_SHAPES(PROBE_F, 256) PROBE_SHAPES(PROBE_F, 512) PROBE_SHAPES(PROBE_F, 1024)
    PROBE_POLICIES(PROBE_F)
    PROBE_SHAPES(PROBE_B, 256) PROBE_SHAPES(PROBE_B, 512) PROBE_SHAPES(PROBE_B, 1024)
    PROBE_POLICIES(PROBE_B)
    // Load streams through LDS (nt loads into LDS, sc0 | sc1 stores).
    PROBE_B(256, 1, 258, 17, 0, 0) PROBE_B(256, 1, 258, 17, 1, 0)
    PROBE_B(256, 2, 258, 17, 0, 0) PROBE_B(256, 2, 258, 17, 1, 0)
    PROBE_B(512, 1, 258, 17, 0, 0) PROBE_B(512, 1, 258, 17, 1, 0)
    // fp32 branch with a mask (the C4 tail at p > 0), fp32 branch without a
    // mask (C0, the C4 tail at p = 0), 16-bit normalized with a mask (the
    // bf16-out configurations).
    PROBE_CONFIG_SHAPES(PROBE_FC, 1, " b32") PROBE_CONFIG_SHAPES(PROBE_BC, 1, " b32")
    PROBE_CONFIG_LDS(1, " b32")
    PROBE_CONFIG_SHAPES(PROBE_FC, 5, " b32 nomask") PROBE_CONFIG_SHAPES(PROBE_BC, 5, " b32 nomask")
    PROBE_CONFIG_LDS(5, " b32 nomask")
    PROBE_CONFIG_SHAPES(PROBE_FC, 2, " n16") PROBE_CONFIG_SHAPES(PROBE_BC, 2, " n16")
};

constexpr int kVariantCount = sizeof(kVariants) / sizeof(kVariants[0]);

}  // namespace

extern "C" {

int rln_probe_variant_count(void) { return kVariantCount; }

// Name ("fwd t256 u2 ld2 st2 ahead1 wide0": kind, threads, units per lane,
// load and store cache bits, look-ahead, 128-bit fp16), kind (0 forward, 1
// backward, 2 empty) and threads of variant `index`; NULL / -1 out of range.
const char* rln_probe_variant_name(int index) {
    return index >= 0 && index < kVariantCount ? kVariants[index].name : nullptr;
}
int rln_probe_variant_kind(int index) {
    return index >= 0 && index < kVariantCount ? kVariants[index].kind : -1;
}
int rln_probe_variant_threads(int index) {
    return index >= 0 && index < kVariantCount ? kVariants[index].threads : -1;
}
// Stream configuration of variant `index` (bit 0: fp32 branch and
// grad_branch, else 16-bit; bit 1: 16-bit normalized and grad_normalized,
// else fp32; bit 2: no mask); -1 out of range.
int rln_probe_variant_config(int index) {
    return index >= 0 && index < kVariantCount ? kVariants[index].config : -1;
}

// Blocks that give every thread one step of variant `index` over
// [rows, hidden]; 0 for bad arguments.
int64_t rln_probe_one_step_blocks(int index, int64_t rows, int64_t hidden) {
    if (index < 0 || index >= kVariantCount || rows <= 0 || hidden <= 0 || hidden % 32 != 0) {
        return 0;
    }
    const int64_t units = rows * hidden / 4;
    const int64_t per_block = static_cast<int64_t>(kVariants[index].threads)
        * kVariants[index].units_per_lane;
    return (units + per_block - 1) / per_block;
}

// Launches variant `index` over [rows, hidden] with `blocks` blocks on
// `stream`. The buffers are the fifteen pointers of the forward's and the
// backward's streams, in the order x, branch, updated (forward output),
// normalized, mask (forward output), mean (forward output), rstd (forward
// output), grad_updated, grad_normalized, updated, mask, mean, rstd,
// grad_x, grad_branch; a pass reads and writes only its own (the other
// pass's, and the masks of a configuration without one, may be NULL).
// Returns 0, 1 for bad arguments (the tensor over 2^31 bytes and a NULL
// buffer the pass uses included) or 3 for a launch error.
int rln_probe_launch(int index, const void* const* buffers, int64_t rows, int64_t hidden,
                     int64_t blocks, void* stream) {
    if (index < 0 || index >= kVariantCount || buffers == nullptr || rows <= 0 || hidden <= 0
        || hidden % 32 != 0 || rows * hidden * 4 > (int64_t{1} << 31) || blocks <= 0
        || blocks > (int64_t{1} << 20)) {
        return 1;
    }
    const bool masked = (kVariants[index].config & 4) == 0;
    if (kVariants[index].kind == kForward) {
        for (int i = 0; i < 7; ++i) {
            if (buffers[i] == nullptr && (i != 4 || masked)) {
                return 1;
            }
        }
    } else if (kVariants[index].kind == kBackward) {
        for (int i = 7; i < 15; ++i) {
            if (buffers[i] == nullptr && (i != 10 || masked)) {
                return 1;
            }
        }
    }
    ProbeBuffers b;
    b.x = static_cast<const float*>(buffers[0]);
    b.branch = buffers[1];
    b.updated_out = static_cast<float*>(const_cast<void*>(buffers[2]));
    b.normalized = static_cast<float*>(const_cast<void*>(buffers[3]));
    b.mask_out = static_cast<uint32_t*>(const_cast<void*>(buffers[4]));
    b.mean_out = static_cast<float*>(const_cast<void*>(buffers[5]));
    b.rstd_out = static_cast<float*>(const_cast<void*>(buffers[6]));
    b.grad_updated = static_cast<const float*>(buffers[7]);
    b.grad_normalized = static_cast<const float*>(buffers[8]);
    b.updated = static_cast<const float*>(buffers[9]);
    b.mask = static_cast<const uint32_t*>(buffers[10]);
    b.mean = static_cast<const float*>(buffers[11]);
    b.rstd = static_cast<const float*>(buffers[12]);
    b.grad_x = static_cast<float*>(const_cast<void*>(buffers[13]));
    b.grad_branch = const_cast<void*>(buffers[14]);
    const Geometry g{static_cast<uint32_t>(rows * hidden / 4), static_cast<uint32_t>(hidden / 4),
                     static_cast<uint32_t>(rows)};
    const Variant& v = kVariants[index];
    v.kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(v.threads), 0,
               static_cast<hipStream_t>(stream)>>>(b, g);
    return hipGetLastError() == hipSuccess ? 0 : 3;
}

// `repeats` launches of the atomic-combine kernel over `sums` ([copies, 2,
// hidden] floats) with `blocks` blocks (`ranges` 0: interleaved copies, 1:
// block ranges per copy), back to back on `stream` from this loop (a launch
// from Python costs the host more than the kernel takes).
int rln_probe_atomic_combine(float* sums, int64_t hidden, int copies, int ranges,
                             int64_t blocks, int repeats, void* stream) {
    if (sums == nullptr || hidden <= 0 || hidden > 8192 || hidden % 32 != 0 || copies <= 0
        || blocks <= 0 || blocks > 65536 || repeats <= 0) {
        return 1;
    }
    for (int i = 0; i < repeats; ++i) {
        probe_atomic_combine<<<dim3(static_cast<unsigned>(blocks)), dim3(512), 0,
                               static_cast<hipStream_t>(stream)>>>(
            sums, static_cast<int>(hidden), copies, ranges);
    }
    return hipGetLastError() == hipSuccess ? 0 : 3;
}

// `repeats` launches of the buffer-atomic combine with cache policy `policy`
// (0, nt = 2, sc1 = 16, nt | sc1 = 18) over `sums` ([2, hidden] floats, one
// copy) with `blocks` blocks; every launch adds exactly 1.0 per block to each
// float, so the caller can check the sums after the last launch.
int rln_probe_atomic_policy(float* sums, int64_t hidden, int policy, int64_t blocks,
                            int repeats, void* stream) {
    if (sums == nullptr || hidden <= 0 || hidden > 8192 || hidden % 32 != 0 || blocks <= 0
        || blocks > 65536 || repeats <= 0) {
        return 1;
    }
    const hipStream_t s = static_cast<hipStream_t>(stream);
    for (int i = 0; i < repeats; ++i) {
        const dim3 grid(static_cast<unsigned>(blocks));
        switch (policy) {
            case 0: probe_atomic_policy<0><<<grid, 512, 0, s>>>(sums, static_cast<int>(hidden)); break;
            case 2: probe_atomic_policy<2><<<grid, 512, 0, s>>>(sums, static_cast<int>(hidden)); break;
            case 16: probe_atomic_policy<16><<<grid, 512, 0, s>>>(sums, static_cast<int>(hidden)); break;
            case 18: probe_atomic_policy<18><<<grid, 512, 0, s>>>(sums, static_cast<int>(hidden)); break;
            default: return 1;
        }
    }
    return hipGetLastError() == hipSuccess ? 0 : 3;
}

// `repeats` launches of the in-launch fold combine over `sums` ([copies, 2,
// hidden] floats, zero), `out` ([2, hidden] floats) and `counter` (one
// uint32, zero) with `blocks` blocks, back to back on `stream`; sums and
// counter are zero again after each launch, and out gains blocks per value;
// at most 16 copies.
int rln_probe_atomic_fold(float* sums, float* out, uint32_t* counter, int64_t hidden,
                          int copies, int64_t blocks, int repeats, void* stream) {
    if (sums == nullptr || out == nullptr || counter == nullptr || hidden <= 0 || hidden > 8192
        || hidden % 32 != 0 || copies <= 0 || copies > kFoldCopies || blocks <= 0
        || blocks > 65536 || repeats <= 0) {
        return 1;
    }
    for (int i = 0; i < repeats; ++i) {
        probe_atomic_fold<<<dim3(static_cast<unsigned>(blocks)), dim3(512), 0,
                            static_cast<hipStream_t>(stream)>>>(
            sums, out, counter, static_cast<int>(hidden), copies);
    }
    return hipGetLastError() == hipSuccess ? 0 : 3;
}

// `repeats` launches of an empty kernel of `blocks` blocks of `threads`
// threads, back to back on `stream` from this loop.
int rln_probe_empty_launches(int64_t blocks, int threads, int repeats, void* stream) {
    if (blocks <= 0 || blocks > 65536 || threads <= 0 || threads > 1024 || repeats <= 0) {
        return 1;
    }
    for (int i = 0; i < repeats; ++i) {
        probe_nothing<<<dim3(static_cast<unsigned>(blocks)), dim3(threads), 0,
                        static_cast<hipStream_t>(stream)>>>(0);
    }
    return hipGetLastError() == hipSuccess ? 0 : 3;
}

}  // extern "C"
