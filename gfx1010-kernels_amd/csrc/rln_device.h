// Fused residual-add + dropout + LayerNorm for MI355X (gfx950, CDNA4): the
// device kernels and their launchers, shared by the per-row-shape
// translation units (rln_hidden.hip) and the C ABI (rln_api.hip, declared in
// include/rln.h). The operator is the
// one implemented by the reference's csrc/residual_layer_norm_kernel.hip
// (forward :425-545, input backward :548-618, parameter backward :727-869);
// the kernels here are organised for wave64 CDNA hardware instead:
//
//  * Up to 1024 columns, one wavefront, or a group of 16 or 32 of its lanes,
//    owns a row. A lane holds kV four-element vectors of its row in
//    registers, so both row reductions run inside the wave with DPP row
//    operations plus v_readlane - no LDS, no barriers. Longer rows (up to
//    8192) are split over 2, 4 or 8 waves of a block, which add their
//    per-wave sums through LDS.
//  * Loads and stores are 128-bit (64-bit for four fp16 values) and marked
//    non-temporal: every byte of the op is touched exactly once per kernel,
//    so the accesses stream through the caches instead of displacing lines
//    other work may reuse. A scalar-access variant of every kernel serves
//    misaligned pointers with the identical arithmetic, so both variants are
//    bitwise equal.
//  * Waves walk rows with a grid-stride loop. The backward's grid depends
//    only on (rows, H), never on the device, so its deterministic
//    parameter-gradient order is reproducible anywhere; the forward's may
//    follow the device's CU count (its outputs, the dropout mask included,
//    depend on the row alone).
//  * Dropout draws from Philox4x32-10 (Salmon et al., SC'11) in one of two
//    layouts. The reference's (hidden sizes 128-1024): its hipRAND stream,
//    one Philox state per (row, thread) of a launch with 128, 192 or 256
//    threads per row, so masks equal the reference's bit for bit
//    (reference_keep_bits). This library's own (every hidden size): one
//    Philox block per four consecutive columns, counter = (offset/4,
//    column-group index), key = seed, a quarter of the reference's Philox
//    work at H = 128 and three quarters at H = 768. Either way the mask
//    depends on (seed, offset, row, column) and not on this build's launch
//    shape. Keep bits are OR-combined across 8 lanes with DPP into the
//    reference's int32 word layout (bit c%32 of word c/32).
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
#include <type_traits>

#include "rln.h"

// Launch-shape constants. They are part of the deterministic contract: the
// grid is a function of (rows, H) and these values only.
#ifndef RLN_FWD_MAX_BLOCKS
#define RLN_FWD_MAX_BLOCKS 2048
#endif
#ifndef RLN_FWD_GROUPS_PER_WAVE
#define RLN_FWD_GROUPS_PER_WAVE 2
#endif
// Forward launches over at least this many elements run one row step per
// team (two for eight-wave rows), on up to RLN_FWD_LARGE_MAX_BLOCKS blocks.
#ifndef RLN_FWD_LARGE_ELEMENTS
#define RLN_FWD_LARGE_ELEMENTS (1ll << 23)
#endif
#ifndef RLN_FWD_LARGE_MAX_BLOCKS
#define RLN_FWD_LARGE_MAX_BLOCKS 65536
#endif
// Forward launches of multi-wave rows below these sizes (elements; the first
// for rows of two or four waves, the second for eight) run a persistent grid
// of eight waves per CU instead.
#ifndef RLN_FWD_PERSISTENT_ELEMENTS
#define RLN_FWD_PERSISTENT_ELEMENTS (1ll << 24)
#endif
#ifndef RLN_FWD_PERSISTENT_ELEMENTS_8
#define RLN_FWD_PERSISTENT_ELEMENTS_8 (1ll << 27)
#endif
// Small forward launches of rows owned by one whole wave (768 and 1024
// columns) run at most this many blocks per CU (forward_blocks).
#ifndef RLN_FWD_WAVE_ROW_BLOCKS_PER_CU
#define RLN_FWD_WAVE_ROW_BLOCKS_PER_CU 3
#endif
#ifndef RLN_BWD_MAX_BLOCKS
#define RLN_BWD_MAX_BLOCKS 256
#endif
// The look-ahead backward keeps two rows in flight for one-part rows of at
// most this many slots per lane (kTwoAhead), one row for every other shape.
// Default 1: one-slot rows (128 and 256 columns) are short, so one row ahead
// keeps too few bytes in flight ([262144, 128] backward 108.6 us against
// 97.4 with two ahead); at C1 (three slots) one row ahead measured 22.4 us
// against 22.9 us with two (input gradients alone 19.0 against 20.2 us;
// bench.py --ab, alternated, register rings).
#ifndef RLN_BWD_TWO_AHEAD_MAX_SLOTS
#define RLN_BWD_TWO_AHEAD_MAX_SLOTS 1
#endif
// 1 (default): the look-ahead backward walks one-part rows in a ring of
// register buffers; 0, and rows of several waves: one-ahead walks that copy
// the next row between registers (the copy waits for that row's loads, and
// with them every older access, before the following row's loads issue).
// Measured on MI355X (bench.py --ab, alternated): the ring at C1 backward
// 22.5 against 23.2 us, [262144, 768] 611 against 628 us; the copy walk for
// rows of several waves: [8192, 1600] 43.3 against 49.9 us, [104857, 1280]
// 410 against 462 us, C3 200 against 210 us.
#ifndef RLN_BWD_RING
#define RLN_BWD_RING 1
#endif
// 1 (default): the look-ahead forward keeps two rows in flight for one-part
// rows of up to three slots; 0: one row. Measured on MI355X at C1 (bench.py
// --ab, alternated, register rings): forward 15.0 us against 17.1 us.
#ifndef RLN_FWD_TWO_AHEAD
#define RLN_FWD_TWO_AHEAD 1
#endif
// 1: the atomic-mode backward adds its last rows' weight/bias contributions
// as soon as their loads arrive, combines the block's sums in LDS with LDS
// atomics (no block barrier) and has the block's last wave issue the global
// atomics, to drain while the last rows' gradients are computed and stored;
// 0 (default): the fixed-order block combine after the last row. Measured on
// MI355X at C1 (bench.py --ab, alternated): backward 34.4 us early against
// 22.9 us after the last row - global atomics issued while the other blocks
// still stream stall the memory channels that hold the sums' lines.
#ifndef RLN_BWD_EARLY_PARAMETERS
#define RLN_BWD_EARLY_PARAMETERS 0
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
// The reference dropout stream's draws of a row: 1 (default) unrolled for the
// launch width the public API uses at the row's size (128 threads up to 768
// columns, 192 at 1024: the reference's table) and looped for the other
// widths - except the forward of 768 columns with a 2-byte branch and fp32
// output, which unrolls every width; 2 unrolled for every width; 0 looped
// for every width. Unrolled, a row's Philox chains interleave (C1 forward
// 16.9 against 17.4 us; [262144, 128] 80 against 93 us). Unrolling every
// width takes the forward's ring instance past 168 VGPRs (two waves per SIMD
// instead of three) at every size and type except 768 and 1024 columns with
// a 2-byte branch and fp32 output (165), and where it crosses, it is slower
// ([12291, 384] fp32 branch forward 16.1 against 14.2 us); at 768 it is
// faster (C1 forward 15.2 against 15.9 us, step 39.9 against 40.8 us;
// bench.py --ab, alternated).
#ifndef RLN_REFERENCE_DRAWS_UNROLLED
#define RLN_REFERENCE_DRAWS_UNROLLED 1
#endif
#ifndef RLN_NT_LOADS
#define RLN_NT_LOADS 1
#endif
// Cache policies of the row outputs' stores (every output the kernels write
// per row: updated, normalized, the mask, mean and rstd, grad_x,
// grad_branch), as the cache-policy bits of a gfx950 buffer store: sc0 = 1,
// nt = 2, sc1 = 16. Launches over fewer than RLN_WRITE_THROUGH_ELEMENTS
// elements write through the caches at system scope (sc0 | sc1), so that no
// dirty line is left in L2 for the end-of-kernel release to write back;
// larger launches store non-temporally. Measured on MI355X (bench.py --ab,
// alternated): C1 [8192, 768] step 39.1 us write-through against 40.3 us
// non-temporal (forward 14.8 against 17.0 us); at 2^26+ elements
// non-temporal wins by 1-7 % (C3 358.7 against 371.6 us, [262144, 384]
// 541 against 555 us), and so at [8192, 1600] (83.3 against 85.7 us). The
// streaming probe at C1 (benchmarks/rln_probe.hip): forward-shaped pass 15.2
// us write-through against 15.8 us plain and 18.8 us non-temporal.
#ifndef RLN_SMALL_STORE_POLICY
#define RLN_SMALL_STORE_POLICY 17
#endif
#ifndef RLN_LARGE_STORE_POLICY
#define RLN_LARGE_STORE_POLICY 2
#endif
#ifndef RLN_WRITE_THROUGH_ELEMENTS
#define RLN_WRITE_THROUGH_ELEMENTS (1ll << 23)
#endif
#ifndef RLN_FWD_WRITE_THROUGH_ELEMENTS
#define RLN_FWD_WRITE_THROUGH_ELEMENTS RLN_WRITE_THROUGH_ELEMENTS
#endif
#ifndef RLN_BWD_WRITE_THROUGH_ELEMENTS
#define RLN_BWD_WRITE_THROUGH_ELEMENTS RLN_WRITE_THROUGH_ELEMENTS
#endif
// 1: the backward of rows of four waves of one slot (769-1024 columns) writes
// through at every size. Measured on MI355X (bench.py --ab, five alternated
// rounds): step -0.7 % at [262144, 1024], +2 % at C3 [65536, 1024], +1 % at
// [262144, 1024] p = 0.1; so 0.
#ifndef RLN_BWD_WIDE14_WRITE_THROUGH
#define RLN_BWD_WIDE14_WRITE_THROUGH 0
#endif

namespace rln {

constexpr int kWaveSize = 64;
constexpr int kBackwardThreads = RLN_BWD_THREADS;
constexpr int64_t kForwardMaxBlocks = RLN_FWD_MAX_BLOCKS;
constexpr int64_t kForwardLargeElements = RLN_FWD_LARGE_ELEMENTS;
constexpr int64_t kForwardLargeMaxBlocks = RLN_FWD_LARGE_MAX_BLOCKS;
constexpr int64_t kForwardPersistentElements = RLN_FWD_PERSISTENT_ELEMENTS;
constexpr int64_t kForwardPersistentElements8 = RLN_FWD_PERSISTENT_ELEMENTS_8;
constexpr int kForwardPersistentWavesPerCu = 8;
constexpr int64_t kBackwardMaxBlocks = RLN_BWD_MAX_BLOCKS;
constexpr int64_t kPacedElements = RLN_PACED_ELEMENTS;
constexpr int64_t kPacedMinHidden = RLN_PACED_MIN_HIDDEN;
static_assert(kBackwardThreads % kWaveSize == 0 && kBackwardThreads <= 1024, "backward block");

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
// Row shapes. A row of `hidden` values is split into four-element vectors; a
// team of lanes owns the row, and vector j of the row sits in slot v of lane
// l of part p, with j = (v * kParts + p) * kLanes + l.
//
//  * FixedShape<H, Lanes>: the reference's hidden sizes, known at compile
//    time. A wave owns a row, or 32 or 16 lanes own it (two or four rows per
//    wave); every slot holds columns. The forward may split a row over fewer
//    lanes than the backward (forward_lanes): the layouts in memory do not
//    depend on the split.
//  * WideShape<V, P>: every other multiple of 64 from kMinHidden to
//    kMaxHidden, passed at run time. P waves own a row (P > 1 add their row
//    sums through LDS), V slots per lane; slots past the end of the row
//    stay idle. The forward and the backward choose P separately
//    (wide_parts), and V is then the fewest slots that hold the row.

constexpr int64_t kSpecializedHidden[] = {128, 256, 384, 512, 768, 1024};
constexpr int64_t kMinHidden = 128;
constexpr int64_t kMaxHidden = 8192;
constexpr int64_t kHiddenMultiple = 64;

// Lanes per row of a specialized hidden size in the backward, and in the
// shape the C ABI dispatches on: a whole wave when H/4 is a multiple of 64,
// else half a wave.
// Lanes per row of the 128-column backward: 32 (default) or 16. Measured on
// MI355X (bench.py --ab, four alternated rounds): [262144, 128] step 180.5
// us at 32 lanes against 180.9 us at 16 (184.6 us with two rows ahead).
#ifndef RLN_FIXED_LANES_128
#define RLN_FIXED_LANES_128 32
#endif
constexpr int fixed_lanes(int64_t hidden) {
    return hidden == 128 ? RLN_FIXED_LANES_128 : ((hidden / 4) % kWaveSize == 0) ? 64 : 32;
}

// Lanes per row in the forward, whose normalized output has type N: fewer
// lanes with more slots each where that measured faster on MI355X (H = 128:
// 16 lanes, 12 % faster; H = 256 and 512: 32 lanes, 2-6 %); H = 768 and 1024
// are faster with a whole wave. (H = 768 with an fp32 output was 3 % faster
// with 32 lanes in the library's own dropout layout at [8192, 768], but 2-14 %
// slower drawing the reference's stream, whose extra Philox work then runs
// at half the occupancy.) The backward measured slower with more slots.
template <typename N>
constexpr int forward_lanes(int64_t hidden) {
    if (hidden == 128) {
        return 16;
    }
    if (hidden == 768 || hidden == 1024) {
        return 64;
    }
    return 32;
}

template <int H, int Lanes = fixed_lanes(H)>
struct FixedShape {
    static constexpr int kHidden = H;
    static constexpr int kLanes = Lanes;
    static constexpr int kV = (H / 4) / kLanes;
    static constexpr int kParts = 1;
    static constexpr int kRowsPerWave = kWaveSize / kLanes;
    static constexpr bool kRagged = false;
    static constexpr bool kCopyWalk = false;  // look-ahead backward: ring (false) or copy walk
    static constexpr int kForwardThreads = 256;
    static constexpr int kBackwardBlockThreads = kBackwardThreads;
    static_assert(H % 64 == 0 && (H / 4) % kLanes == 0 && kLanes >= 16,
                  "row must split evenly over lanes");
    __host__ __device__ constexpr int64_t hidden() const { return H; }
    __host__ __device__ constexpr float inv_hidden() const {
        return 1.0f / static_cast<float>(H);
    }
};

template <int V, int P>
struct WideShape {
    static constexpr int kHidden = 0;  // run-time
    static constexpr int kLanes = kWaveSize;
    static constexpr int kV = V;
    static constexpr int kParts = P;
    static constexpr int kRowsPerWave = 1;
    static constexpr bool kRagged = true;
    static constexpr bool kCopyWalk = false;
    // Three-wave rows (the backward of large 768-column launches) run in
    // 12-wave blocks and sixteen-wave rows (the backward of large launches of
    // 6657-8192 columns) in 16-wave blocks, so that a block still holds whole
    // rows and the grid keeps one weight/bias partial per CU.
    static constexpr int kForwardThreads = P == 3 ? 6 * kWaveSize : P > 4 ? P * kWaveSize : 256;
    static constexpr int kBackwardBlockThreads =
        P == 3 ? 12 * kWaveSize : P == 16 ? 16 * kWaveSize : kBackwardThreads;
    static_assert(P == 1 || P == 2 || P == 3 || P == 4 || P == 8 || P == 16, "parts per row");
    int64_t hidden_;
    float inv_hidden_;  // 1.0f / hidden, rounded once on the host
    __host__ __device__ int64_t hidden() const { return hidden_; }
    __host__ __device__ float inv_hidden() const { return inv_hidden_; }
};

// The backward of rows of four waves and one or two slots per lane (769-1024
// and 1217-2048 columns) in twelve-wave blocks, three rows per block step:
// the launches of at most kStaggeredWideMaxRows rows (shape_info).
template <int V>
struct StaggeredWideShape : WideShape<V, 4> {
    static constexpr int kBackwardBlockThreads = 12 * kWaveSize;
};

// The backward of a specialized size in twelve-wave blocks (one row per
// wave, one block per CU) walking its rows with the copy walk: the ring walk
// needs ~200 VGPRs at 768 columns and spills at the 168 a twelve-wave block
// allows. Used for the launches backward_twelve_waves selects.
template <int H>
struct TwelveWaveShape : FixedShape<H> {
    static constexpr int kBackwardBlockThreads = 12 * kWaveSize;
    static constexpr bool kCopyWalk = true;
};

// The same for rows of two per wave (384 columns): nine-wave blocks, 165
// VGPRs on the copy walk. Used for the launches backward_nine_waves selects.
template <int H>
struct NineWaveShape : FixedShape<H> {
    static constexpr int kBackwardBlockThreads = 9 * kWaveSize;
    static constexpr bool kCopyWalk = true;
};

inline bool specialized_hidden(int64_t hidden) {
    for (const int64_t value : kSpecializedHidden) {
        if (value == hidden) {
            return true;
        }
    }
    return false;
}

inline bool hidden_supported(int64_t hidden) {
    return specialized_hidden(hidden)
        || (hidden >= kMinHidden && hidden <= kMaxHidden && hidden % kHiddenMultiple == 0);
}

// The shape parameters a supported hidden size runs with (host side; the
// kernels' template parameters must match them).
struct ShapeInfo {
    int rows_per_wave;
    int parts;
    int vectors;  // slots per lane
    int forward_threads;
    int backward_threads;
};

// The forward's shape for dispatch shape S and normalized type N (the
// specialized sizes' forward may use fewer lanes per row, forward_lanes).
template <typename S, typename N>
struct ForwardShape {
    using type = S;
};
template <int H, int Lanes, typename N>
struct ForwardShape<FixedShape<H, Lanes>, N> {
    using type = FixedShape<H, forward_lanes<N>(H)>;
};

template <typename S>
constexpr ShapeInfo info_of() {
    return {S::kRowsPerWave, S::kParts, S::kV, S::kForwardThreads, S::kBackwardBlockThreads};
}

enum class Pass { kForward, kBackward };

// Waves per row of a run-time row length. Measured on MI355X, the backward
// is faster on more waves with fewer slots as long as about as many slots
// hold columns, or at least ~60 % of them: 4 waves x 1 slot against 1 x 4
// for 769-1024 columns (6-7 % at 832 and 896, 2.5 % at 960, 3-4 % at 1024;
// no gain at 8 M elements; at 768 the split, a quarter of its slots idle
// against none for one wave of three, is 2-13 % slower); 4 x 2 against
// 2 x 3-4 (1.5 % at 1280 columns, 4 % at 1536, 5-7 % at 1600 and 2048);
// 8 x 2 against 4 x 3-4 (2 % at 2560, 6-8 % from 3072 to 4096); at 1088 and
// 2112, where half the slots would idle, 4 x 2 is 3-5 % slower. The forward
// is faster on fewer waves with more slots (2 x 4 against 4 x 2: 3-8 % at
// 1600 to 2048).
inline int wide_parts(int64_t hidden, Pass pass) {
    if (pass == Pass::kForward) {
        return hidden <= 1024 ? 1 : hidden <= 2048 ? 2 : hidden <= 4096 ? 4 : 8;
    }
    return hidden <= 704 ? 1 : hidden <= 768 ? 3 : hidden <= 1024 ? 4 : hidden <= 1216 ? 2
        : hidden <= 2432 ? 4 : 8;
}

// Launches of at least this many rows run the backward of 768 columns on
// three waves of one slot (wide_parts): measured 2-4 % faster than one wave
// of three slots from 65536 rows (50 M elements), and 5 % slower at 8192.
constexpr int64_t kWide768BackwardRows = 65536;

// A specialized size whose backward runs the run-time-length kernel for a
// launch over `rows`: 1024 columns always (4 waves of one slot, as every row
// of 769-1024 columns), 768 from kWide768BackwardRows.
inline bool backward_runs_wide(int64_t hidden, int64_t rows) {
    return hidden == 1024 || (hidden == 768 && rows >= kWide768BackwardRows);
}

// The backward of 768 columns over 2048-9216 rows runs twelve-wave blocks
// (TwelveWaveShape) when the last of its at most three row steps per wave
// keeps at least half of the 256 x 12 waves busy, or all of them: then the
// blocks whose waves have a step fewer finish earlier and add their
// weight/bias sums while the others still stream, and the others' twelve
// waves per CU keep the HBM busy meanwhile, so the adds at the end of the
// kernel contend less (at C1 the time the sums add to the backward falls
// from 3.5 to 1.6 us). With fewer rows busy in the last step, the few CUs
// left streaming cannot keep the HBM busy. Measured on MI355X (fwd+bwd step,
// us, eight-wave ring against twelve-wave copy walk, five alternated rounds):
// 2048 rows 19.6 -> 17.9, 2560 23.2 -> 22.5, 5120 29.5 -> 29.1, 6144 32.8 ->
// 32.6, 8192 40.0 -> 39.2 (C1; bf16 output 38.2 -> 36.8); and slower at 4096
// (26.0 -> 26.7) and 7168 (34.3 -> 35.8), where a third of the waves is busy
// in the last step, equal at 10240 and 12288, 1-3 % slower from 16384 rows.
// RLN_BWD_TWELVE_WAVE_768=0 keeps the eight-wave ring everywhere.
#ifndef RLN_BWD_TWELVE_WAVE_768
#define RLN_BWD_TWELVE_WAVE_768 1
#endif
inline bool backward_twelve_waves(int64_t hidden, int64_t rows) {
    constexpr int64_t kTeams = RLN_BWD_MAX_BLOCKS * 12;
    if (!RLN_BWD_TWELVE_WAVE_768 || hidden != 768 || rows < 2048 || rows > 3 * kTeams) {
        return false;
    }
    const int64_t last = rows % kTeams;
    return last == 0 || 2 * last >= kTeams;
}

// The backward of 384 columns (two rows per wave) over 11520-13056 rows runs
// nine-wave blocks: 2304 teams of two rows, two full row steps and a third
// one-half to five-sixths full, so that, as with the twelve-wave blocks of
// 768 columns, some of the blocks end a step early and add their weight/bias
// sums while the others stream. Measured alternated (bench.py --ab
// eight=RLN_BWD_NINE_WAVE_384=0, backward with the sums, against eight-wave
// blocks): the C4 tail [12291, 384] fp32 branch 20.05 -> 19.47 us at p = 0,
// 20.80 -> 20.00 at p = 0.1; fp16 branch 11520 rows 18.93 -> 18.63, 12291
// 20.28 -> 19.13, 13000 21.79 -> 20.11. With the third step (nearly) full
// the blocks end together and the copy walk only costs: 13823 rows 20.68 ->
// 21.46, 13824 20.70 -> 21.43; with two steps, 7168 rows 13.58 -> 14.11.
#ifndef RLN_BWD_NINE_WAVE_384
#define RLN_BWD_NINE_WAVE_384 1
#endif
inline bool backward_nine_waves(int64_t hidden, int64_t rows) {
    constexpr int64_t kRowSlots = RLN_BWD_MAX_BLOCKS * 9 * 2;
    return RLN_BWD_NINE_WAVE_384 && hidden == 384 && 2 * rows >= 5 * kRowSlots
        && 6 * rows <= 17 * kRowSlots;
}

// Backward launches of at most 8192 rows of four waves and one or two slots
// (769-1024 and 1217-2048 columns) run twelve-wave blocks instead of eight:
// their waves already walk with the copy walk (multi-wave rows), in the 162-
// 166 VGPRs that three waves per SIMD allow, so the larger blocks cost the
// input gradients little and give the grid a last row step a third or two
// thirds full where eight-wave blocks end together. Measured alternated
// (bench.py --ab eight=RLN_BWD_STAGGERED_WIDE=0 --ab-rows ... --ab-hidden H,
// backward with the sums): 1600 columns 1024 rows 14.61 -> 12.70 us, 2048
// 17.08 -> 15.16, 4096 24.85 -> 23.45, 6144 36.82 -> 33.81, 8192 45.23 ->
// 42.02; 1024 columns 2048 rows 13.68 -> 12.37, 4096 19.38 -> 18.01, 6144
// 24.47 -> 23.36, 8192 30.10 -> 29.33; 832 columns 4096 rows 18.48 -> 16.47,
// 8192 27.74 -> 24.56; 2048 columns 4096 rows 30.20 -> 29.58, 8192 52.07 ->
// 52.65. Larger launches lose (1024 columns: 12288 rows +0.7 %, 16384
// +1.6 %; [262144, 1600] +5.7 %), and so do rows of three slots (2432
// columns, 4096 rows 35.4 -> 41.9 us).
#ifndef RLN_BWD_STAGGERED_WIDE
#define RLN_BWD_STAGGERED_WIDE 1
#endif
constexpr int64_t kStaggeredWideMaxRows = 8192;

// Backward launches of at least this many elements run rows of 6657-8192
// columns on sixteen waves of two slots (1024-thread blocks) instead of eight
// of four: measured 2-4.5 % faster from 2^26 elements ([16384, 8192] 416
// against 424-436 us, [18724, 7168] 425-427 against 437-441 us, [8192, 8192]
// 209 against 212-214 us, alternated in one run), and 1-4.5 % slower at
// 2^24-2^25; equal at 6656 columns.
#ifndef RLN_BWD_SIXTEEN_WAVE_ELEMENTS
#define RLN_BWD_SIXTEEN_WAVE_ELEMENTS (1ll << 26)
#endif
constexpr int64_t kSixteenWaveBackwardElements = RLN_BWD_SIXTEEN_WAVE_ELEMENTS;
constexpr int64_t kSixteenWaveBackwardMinHidden = 6657;

// The shape of a supported hidden size in one pass over `rows`.
inline ShapeInfo shape_info(int64_t hidden, Pass pass, int64_t rows) {
    if (specialized_hidden(hidden)
        && !(pass == Pass::kBackward && backward_runs_wide(hidden, rows))) {
        const int lanes = fixed_lanes(hidden);
        return {kWaveSize / lanes, 1, static_cast<int>(hidden / 4 / lanes), 256,
                pass != Pass::kBackward                 ? kBackwardThreads
                : backward_twelve_waves(hidden, rows) ? 12 * kWaveSize
                : backward_nine_waves(hidden, rows)   ? 9 * kWaveSize
                                                      : kBackwardThreads};
    }
    int parts = wide_parts(hidden, pass);
    if (pass == Pass::kBackward && parts == 8 && hidden >= kSixteenWaveBackwardMinHidden
        && rows * hidden >= kSixteenWaveBackwardElements) {
        parts = 16;
    }
    const int64_t per_slot = 4 * kWaveSize * parts;
    const int vectors = static_cast<int>((hidden + per_slot - 1) / per_slot);
    const bool staggered = pass == Pass::kBackward && RLN_BWD_STAGGERED_WIDE && parts == 4
        && vectors <= 2 && rows <= kStaggeredWideMaxRows;
    return {1, parts, vectors, parts == 3 ? 6 * kWaveSize : parts > 4 ? parts * kWaveSize : 256,
            parts == 3 || staggered ? 12 * kWaveSize
            : parts == 16           ? 16 * kWaveSize
                                    : kBackwardThreads};
}


// Blocks for a launch over `rows`: each block works on
// (threads / 64) * rows_per_wave / parts rows at a time, and gets enough
// blocks for `iterations` such steps, capped; a function of (rows, hidden)
// only.
inline int64_t launch_blocks(int64_t rows, const ShapeInfo& info, int threads, int64_t cap,
                             int64_t iterations) {
    const int64_t rows_per_block = (threads / kWaveSize) * info.rows_per_wave / info.parts;
    const int64_t steps = (rows + rows_per_block - 1) / rows_per_block;
    const int64_t blocks = (steps + iterations - 1) / iterations;
    return blocks < cap ? blocks : cap;
}

// 1 if a launch over rows x hidden walks its rows paced, 0 for look-ahead.
// Measured on MI355X: paced is faster from about 8 M elements for one-wave
// rows of 256 or more columns (backward up to 12 % at 200 M elements), and
// slower at C1-sized launches. Multi-wave rows gain from it only in the
// forward, from about 64 M elements, and not with 8 waves of 4 slots (one
// block per CU, where look-ahead is up to 19 % faster); their backward is
// faster with look-ahead at every size measured (up to 24 %).
inline int forward_paced(int64_t rows, int64_t hidden) {
    const ShapeInfo info = shape_info(hidden, Pass::kForward, rows);
    const int64_t elements = rows * hidden;
    if (hidden < kPacedMinHidden || elements < kPacedElements) {
        return 0;
    }
    if (info.parts == 1) {
        return 1;
    }
    return elements >= 8 * kPacedElements && !(info.parts == 8 && info.vectors == 4) ? 1 : 0;
}

inline int backward_paced(int64_t rows, int64_t hidden) {
    return hidden >= kPacedMinHidden && rows * hidden >= kPacedElements
        && shape_info(hidden, Pass::kBackward, rows).parts == 1 ? 1 : 0;
}

// Small forward launches give each team at least two row steps so that its
// look-ahead load overlaps a row's computation, with at most 2048 blocks,
// and then a whole number of blocks per CU (`cus`, the device's compute
// units; 0 = unknown): a launch whose block count is not a multiple of the
// CU count leaves some CUs one block more, which then run alone at the end
// (measured on MI355X: the C4 tail, [12291, 384], forward 14.8 us at 769
// blocks, 14.1 us at 768). Rows owned by one whole wave of a specialized size
// (768 and 1024 columns) run at most three blocks per CU: C1 [8192, 768]
// 17.1 us against 17.4 us at four and 17.8 us at 2048 (one step per team);
// the narrower shapes, two or four rows per wave, measured best at their own
// count. A count between one and two rounds of the blocks a CU holds at once
// (`resident`, asked of the runtime for the kernel instance) becomes one
// round, so that no part-full second round runs after the first: measured
// (us, alternated in one run) [16383, 512] 25.3 -> 21.8, [8192, 640] 17.0 ->
// 14.3, [24576, 256] 19.8 -> 17.4, [21845, 384] 25.7 -> 23.9, [8738, 960]
// 26.5 -> 24.6, [49152, 128] 21.6 -> 20.8, and [65535, 128] 26.9 -> 27.6.
// Rows of two or four per wave (128-512 columns) also run one round when
// they have at least a round of row steps, where two steps per team and the
// rounding to whole blocks per CU left fewer blocks: [6144, 512] 13.0 ->
// 8.4, [8192, 512] 12.3 -> 10.7, [10240, 256] 10.9 -> 7.6, [16384, 256] 13.6
// -> 11.6, [32768, 128] 16.2 -> 13.1, [8192, 384] 10.4 -> 8.3; [12291, 384]
// 13.6 -> 13.0 (fp16 branch, p = 0.1), and with an fp32 branch (the C4 tail)
// 14.0 -> 14.3 at p = 0 (step 34.8 -> 35.0) and 14.8 -> 14.6 at p = 0.1
// (step 35.2 -> 35.0). Rows of one wave stay at their count: [4096, 768] at
// one round was 7 % slower, and [8192, 768] at four blocks per CU runs its
// forward 0.4 us faster but the forward + backward step 0.3 us slower.
// Large launches (2^23 elements and up) instead run one row step per
// team (two for eight-wave rows), up to 65536 blocks, again a whole number per
// CU: the hardware keeps as many of them resident as registers allow and
// starts the next as one ends, which streams faster than fewer teams walking
// many rows. A cap of 65536 instead of 24576 blocks, so that 262144 rows of
// one wave take one step each: forward 660 -> 614 us at [262144, 1024], 499
// -> 487 at [262144, 768] (bf16 out 396 -> 385), 324 -> 307 at [209715,
// 640], 324 -> 311 at [104857, 1280], 330 -> 320 at [83886, 1600]; the same
// at [262144, 384] and at rows of 2048 and 4096 columns (bench.py --ab
// fwd64k=RLN_FWD_LARGE_MAX_BLOCKS=65536, three alternated rounds). Measured
// at 262144 rows (forward, us, the small-launch grid
// against one step per team, alternated in one run where marked *): H = 128
// 99 -> 92, 256 179 -> 159, 384 258 -> 238, 512 352 -> 317, 768 541-550 ->
// 491-495 *, 1024 681-758 -> 652-653 *; [65536, 1024] 166-169 -> 159 *,
// [65536, 256] 44.7 -> 40.2, [16384, 768] 32.4 -> 31.9; run-time rows of
// 640-4096 columns 3-6 % faster. Eight-wave rows (4097-8192 columns, one row
// per 512-thread block and few blocks per CU) need the look-ahead of a second
// step: one step per team took 387 us at [16384, 8192] against 321-342 us for
// the small-launch grid, two steps 331-334 us against 338-341 us alternated in
// one run ([26214, 5120]: 328 us against 335 us).
//
// Multi-wave rows (1025-8192 columns) below 2^24 elements (2^27 for eight-wave
// rows walked with look-ahead) run neither grid but a persistent one of eight
// waves per CU - two blocks of four waves, or one of eight - each team
// walking its rows with look-ahead, or one block per row step when there are
// fewer steps. The small-launch grid puts up to 2048 blocks of rows whose
// kernels hold 124-163 VGPRs (3-4 resident blocks per CU, one for eight-wave
// rows of four slots), so a few blocks run in a second round after the rest;
// one step per team leaves the last round part-full. Measured on MI355X
// (forward, us, the two grids above against the persistent one, alternated
// in one run): [2048, 4096] 24.0 -> 22.5, [2730, 3072] 25.9 -> 22.1,
// [4096, 2048] 23.6 -> 22.2, [4096, 1600] 21.6 -> 18.2, [5242, 1600] 26.2 ->
// 23.3, [8192, 1600] 34.7 -> 33.6, [6553, 1280] 25.7 -> 22.9, [64, 4096] 6.2
// -> 4.4; eight-wave rows [256, 8192] 9.0 -> 7.1, [4096, 8192] 84.5 -> 80.5,
// [8192, 8192] 167.9 -> 161.5, [8192, 6144] 124.9 -> 120.0; within +-1.5 % at
// most other sizes; slower by 2-3 % just below 2^24 for rows of 4096 and 2048
// columns ([4095, 4096] 42.6 -> 43.4, [8191, 2048] 42.0 -> 43.1) and at
// [3072, 2048] (16.5 -> 16.8), by 6 % at [1024, 6144] (17.5 -> 18.5); 2^24
// elements and up one step per team is as fast or faster (2-6 % at 2^24 -
// 2^25 for rows of 2048 and 4096 columns), and so are eight-wave rows walked
// paced (4097-6144 columns from 2^26) and [16384, 8192] (332 against 340).
// Twelve waves per CU were faster at a few sizes (2048 row steps) and slower
// at most. Every output of the forward is a function of its row alone (the
// dropout mask of (seed, offset, row, column)), so its grid may depend on
// the device.
template <typename S>
int64_t forward_blocks(int64_t rows, int64_t hidden, int cus, int resident) {
    const int64_t elements = rows * hidden;
    if (S::kParts > 1 && cus > 0
        && (S::kParts < 8 ? elements < kForwardPersistentElements
                          : elements < kForwardPersistentElements8
                                && forward_paced(rows, hidden) == 0)) {
        const int64_t steps = launch_blocks(rows, info_of<S>(), S::kForwardThreads, INT64_MAX, 1);
        int64_t per_cu = kForwardPersistentWavesPerCu * kWaveSize / S::kForwardThreads;
        // Rows of two or four waves with more than 6 and at most 8 row steps
        // per CU: twelve waves per CU (three blocks, when they fit). Measured
        // (forward us, alternated in one run): [4096, 1280] 15.3 -> 14.0,
        // [2048, 2560] 15.5 -> 14.3, [2048, 4096] 22.3 -> 21.6, [4096, 2048]
        // 22.1 -> 21.2, [4096, 1600] 18.3 -> 18.0; at 9 steps per CU 2.5-3.5 %
        // slower ([4608, 2048], [2304, 4096]) and at 6 mixed (+-2.7 %).
        if (S::kParts < 8 && steps > 6 * static_cast<int64_t>(cus)
            && steps <= 8 * static_cast<int64_t>(cus) && resident >= 3) {
            per_cu = 3;
        }
        const int64_t persistent = static_cast<int64_t>(cus) * per_cu;
        return steps < persistent ? steps : persistent;
    }
    // Specialized rows of four slots per lane (512 and 1024 columns) keep one
    // round of resident blocks (three per CU) up to 2^24 elements instead of
    // one step per team. Measured (forward us, alternated in one run):
    // [8192, 1024] 24.3 -> 23.1 (step 54.6 -> 53.4), [12288, 1024] 33.5 ->
    // 32.6, [16383, 1024] 42.8 -> 41.9, [16384, 512] 23.3 -> 22.4, [24576, 512]
    // 32.4 -> 32.0, [32767, 512] 41.6 -> 41.0; from 2^24 one step per team is
    // as fast, and rows of ragged four-slot (769-1023 columns) or three-slot
    // rows slower at one round (2-4 %).
    if (S::kHidden > 0 && S::kV == 4 && cus > 0 && resident > 0
        && elements >= kForwardLargeElements && elements < kForwardPersistentElements) {
        const int64_t steps = launch_blocks(rows, info_of<S>(), S::kForwardThreads, INT64_MAX, 1);
        const int64_t round = static_cast<int64_t>(resident) * cus;
        return steps < round ? steps : round;
    }
    int64_t blocks;
    if (elements >= kForwardLargeElements) {
        blocks = launch_blocks(rows, info_of<S>(), S::kForwardThreads, kForwardLargeMaxBlocks,
                               S::kParts < 8 ? 1 : 2);
    } else {
        blocks = launch_blocks(rows, info_of<S>(), S::kForwardThreads, kForwardMaxBlocks,
                               RLN_FWD_GROUPS_PER_WAVE);
        constexpr int64_t kPerCu = RLN_FWD_WAVE_ROW_BLOCKS_PER_CU;
        if (cus > 0 && S::kHidden > 0 && S::kLanes == kWaveSize && blocks > kPerCu * cus) {
            blocks = kPerCu * cus;
        }
        // No part-full second round: between one and two rounds of resident
        // blocks, one round.
        const int64_t round = static_cast<int64_t>(resident) * cus;
        if (round > 0 && blocks > round && blocks < 2 * round) {
            blocks = round;
        }
        // Rows of two or four per wave with a round's worth of row steps: one
        // round.
        if (round > 0 && S::kRowsPerWave > 1 && blocks < round
            && launch_blocks(rows, info_of<S>(), S::kForwardThreads, INT64_MAX, 1) >= round) {
            blocks = round;
        }
    }
    if (cus > 0 && blocks > cus) {
        blocks -= blocks % cus;
    }
    return blocks;
}

// The backward's grid is also the number of weight/bias partials: at most
// 256 blocks of 8 waves (12 for three-wave rows), one block per CU.
inline int64_t backward_blocks(int64_t rows, int64_t hidden) {
    const ShapeInfo info = shape_info(hidden, Pass::kBackward, rows);
    return launch_blocks(rows, info, info.backward_threads, kBackwardMaxBlocks, 1);
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

// Sum over the lanes that own one row: 64 lanes, the 32-lane half of the
// wave that the calling lane belongs to, or its 16-lane DPP row. Must be
// called by all 64 lanes.
template <int Lanes>
__device__ __forceinline__ float row_sum(float value) {
    value = row16_sum(value);
    if constexpr (Lanes == 16) {
        return value;
    }
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
// A round is two v_mad_u64_u32 (quarter rate) and two three-input XORs, each
// one gfx950 v_bitop3_b32 (truth table 0x96) instead of two v_xor_b32; the
// compiler does not form it from the XOR chain itself.

__device__ __forceinline__ uint32_t xor3(uint32_t a, uint32_t b, uint32_t c) {
    return __builtin_amdgcn_bitop3_b32(a, b, c, 0x96);
}

__device__ __forceinline__ uint4 philox4x32_10(uint4 counter, uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int round = 0; round < 10; ++round) {
        const uint64_t product0 = static_cast<uint64_t>(0xD2511F53u) * counter.x;
        const uint64_t product1 = static_cast<uint64_t>(0xCD9E8D57u) * counter.z;
        counter = make_uint4(
            xor3(static_cast<uint32_t>(product1 >> 32), counter.y, k0),
            static_cast<uint32_t>(product1),
            xor3(static_cast<uint32_t>(product0 >> 32), counter.w, k1),
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
    int threads;  // 0: this library's layout; else the reference's, per rln_philox_t
};

// ----------------------------------------------------------------------------
// Global memory loads. Aligned = one 128-bit access (64-bit for 4 x fp16);
// otherwise element accesses with the same values. Row loads carry the
// non-temporal hint (RLN_NT_LOADS); stores are the row outputs below.

template <typename T>
__device__ __forceinline__ T stream_load(const T* pointer) {
#if RLN_NT_LOADS
    return __builtin_nontemporal_load(pointer);
#else
    return *pointer;
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

// ----------------------------------------------------------------------------
// Row outputs. Every per-row output goes out through buffer stores with the
// launch's cache policy (a global store cannot carry its sc bits from HIP
// source): write-through, or non-temporal (`wt` false), a wave-uniform kernel
// argument, so each store site is a scalar branch between the two
// instructions. A wave's stores of one row step go through one descriptor
// per output over exactly the rows the wave writes in that step: its base
// and extent are wave-uniform (scalar registers), every lane stores at a
// byte offset into it, and the hardware's range check drops any store
// outside the wave's rows.

using rsrc_t = __amdgpu_buffer_rsrc_t;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// The descriptor's fourth word for a raw (untyped, unswizzled) buffer.
constexpr int kRawBufferWord3 = 0x00020000;
constexpr int64_t kForwardWriteThroughElements = RLN_FWD_WRITE_THROUGH_ELEMENTS;
constexpr int64_t kBackwardWriteThroughElements = RLN_BWD_WRITE_THROUGH_ELEMENTS;

// `value` of the wave's first active lane, in scalar registers.
__device__ __forceinline__ int64_t wave_uniform(int64_t value) {
    const uint64_t bits = static_cast<uint64_t>(value);
    const uint32_t low = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(bits));
    const uint32_t high = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(bits >> 32));
    return static_cast<int64_t>((static_cast<uint64_t>(high) << 32) | low);
}

// A descriptor over `count` elements of `tensor` from element `first`
// (wave-uniform arguments; count * sizeof(T) < 2^31).
template <typename T>
__device__ __forceinline__ rsrc_t output_range(T* tensor, int64_t first, int64_t count) {
    return __builtin_amdgcn_make_buffer_rsrc(
        static_cast<void*>(tensor + first), 0,
        static_cast<int>(count * static_cast<int64_t>(sizeof(T))), kRawBufferWord3);
}

__device__ __forceinline__ void output_b32(rsrc_t r, uint32_t offset, uint32_t value, bool wt) {
    if (wt) {
        __builtin_amdgcn_raw_buffer_store_b32(value, r, offset, 0, RLN_SMALL_STORE_POLICY);
    } else {
        __builtin_amdgcn_raw_buffer_store_b32(value, r, offset, 0, RLN_LARGE_STORE_POLICY);
    }
}

__device__ __forceinline__ void output_b128(rsrc_t r, uint32_t offset, u32x4 value, bool wt) {
    if (wt) {
        __builtin_amdgcn_raw_buffer_store_b128(value, r, offset, 0, RLN_SMALL_STORE_POLICY);
    } else {
        __builtin_amdgcn_raw_buffer_store_b128(value, r, offset, 0, RLN_LARGE_STORE_POLICY);
    }
}

__device__ __forceinline__ void output_b64(rsrc_t r, uint32_t offset, u32x2 value, bool wt) {
    if (wt) {
        __builtin_amdgcn_raw_buffer_store_b64(value, r, offset, 0, RLN_SMALL_STORE_POLICY);
    } else {
        __builtin_amdgcn_raw_buffer_store_b64(value, r, offset, 0, RLN_LARGE_STORE_POLICY);
    }
}

__device__ __forceinline__ void output_b16(rsrc_t r, uint32_t offset, uint16_t value, bool wt) {
    if (wt) {
        __builtin_amdgcn_raw_buffer_store_b16(value, r, offset, 0, RLN_SMALL_STORE_POLICY);
    } else {
        __builtin_amdgcn_raw_buffer_store_b16(value, r, offset, 0, RLN_LARGE_STORE_POLICY);
    }
}

// Four fp32 values at byte `offset`: one 128-bit store, or four element
// stores with the same values when the tensor is not 16-byte aligned.
template <bool Aligned>
__device__ __forceinline__ void output4(rsrc_t r, uint32_t offset, f32x4 value, bool wt) {
    if constexpr (Aligned) {
        output_b128(r, offset, __builtin_bit_cast(u32x4, value), wt);
    } else {
        // Element by element through a scalar copy: clang's __builtin_bit_cast
        // of a vector element expression (value.y) reads element 0.
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float element = value[e];
            output_b32(r, offset + 4 * e, __builtin_bit_cast(uint32_t, element), wt);
        }
    }
}

// Parameters (weight, bias): ordinary cached loads, every wave reads them.// Parameters (weight, bias): ordinary cached loads, every wave reads them.
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

// Stores four fp32 values as type T at byte `offset` (the offset of the
// first element); narrowing rounds to nearest even.
template <typename T, bool Aligned>
__device__ __forceinline__ void output_convert4(rsrc_t r, uint32_t offset, f32x4 value,
                                                bool wt) {
    if constexpr (std::is_same_v<T, float>) {
        output4<Aligned>(r, offset, value, wt);
    } else {
        const typename Vector4<T>::type packed =
            __builtin_convertvector(value, typename Vector4<T>::type);
        if constexpr (Aligned) {
            output_b64(r, offset, __builtin_bit_cast(u32x2, packed), wt);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                output_b16(r, offset + 2 * e, __builtin_bit_cast(uint16_t, static_cast<T>(packed[e])),
                           wt);
            }
        }
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

// Where a lane's slots sit in its row, for shape S: vector index of slot v,
// whether the slot holds columns, and the first column to access (slot 0's
// column for an idle slot, so that its accesses stay inside the row).
template <typename S>
struct Slots {
    int part;
    int lane;  // lane within the part's lanes
    int64_t hidden;

    __device__ __forceinline__ int vector(int v) const {
        return (v * S::kParts + part) * S::kLanes + lane;
    }
    __device__ __forceinline__ bool active(int v) const {
        return !S::kRagged || static_cast<int64_t>(vector(v)) * 4 < hidden;
    }
    __device__ __forceinline__ int column(int v) const {
        return active(v) ? vector(v) * 4 : 0;
    }
};

// Sum of `value` over a row's lanes (all lanes receive the same bits). With
// P > 1 parts, each wave's total goes through `exchange[group][part]` in
// LDS and the parts are added in ascending order; every wave of the block
// must call it (it holds a block barrier).
template <typename S>
__device__ __forceinline__ float team_sum(float value, float (*exchange)[S::kParts], int group,
                                          int part) {
    const float wave_total = row_sum<S::kLanes>(value);
    if constexpr (S::kParts == 1) {
        return wave_total;
    } else {
        if ((threadIdx.x & (kWaveSize - 1)) == 0) {
            exchange[group][part] = wave_total;
        }
        __syncthreads();
        float total = exchange[group][0];
#pragma unroll
        for (int other = 1; other < S::kParts; ++other) {
            total += exchange[group][other];
        }
        return total;
    }
}

// Orders the LDS accesses of the wave's lanes before this point ahead of
// those after it, as a memory handoff between lanes of one wave: the release
// and acquire fences at wavefront scope stop the compiler from moving memory
// accesses across (a bare wave barrier only constrains instruction
// scheduling), and a wave's LDS operations complete in issue order, so no
// instruction is needed for the hardware.
__device__ __forceinline__ void wave_handoff() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Keep bits of the reference's own dropout stream for one row of a fixed
// shape (reference csrc/residual_layer_norm_kernel.hip:449-511). The
// reference launches `threads` threads per row; thread t of row r seeds
// hipRAND's Philox with hiprand_init(seed, r * threads + t, offset) - key =
// seed, 128-bit counter = (r * threads + t) * 2^64 + offset / 4, plus n for
// its n-th hiprand4 - and draws items = ceil(H / threads) values, four per
// call; column t + item * threads keeps iff value[item] >= threshold.
//
// Here the row's L lanes stand in for those threads, L at a time
// (t = k * L + l), and compute the same ceil(items / 4) Philox blocks per
// thread. Item `item` of threads k * L .. k * L + L - 1 covers the L
// consecutive columns of chunk item * (threads / L) + k; one ballot
// collects their keep flags, which the row's first L / 16 lanes stage in
// LDS as 16-bit pieces (a ballot carries the chunks of all rows of the
// wave). Each lane then reads the 4 bits of each of its slots and returns
// them packed, slot v in bits 4v .. 4v + 3. `stage` is the row's H / 16
// pieces, used by this wave only: LDS accesses of one wave complete in
// order, so no block barrier is needed; two wave-level handoffs
// (wave_handoff: wavefront-scope release and acquire fences around a wave
// barrier) order the cross-lane exchange for the compiler: the writes after
// the previous row's reads, the reads after the writes.
// Requires offset % 4 == 0 and at most 8
// items (the reference's two hiprand4 calls), checked on the host.
template <typename S, int Threads>
__device__ __forceinline__ uint32_t reference_keep_bits_of(
    uint16_t* stage, int64_t row, int lane, int group, uint64_t position, uint32_t key0,
    uint32_t key1, uint32_t threshold) {
    constexpr int L = S::kLanes;
    constexpr int kChunks = S::kHidden / L;
    static_assert(S::kParts == 1 && S::kHidden > 0 && L % 16 == 0 && S::kV <= 8,
                  "fixed one-part rows of at most 8 slots");
    static_assert(Threads % L == 0, "stand-in lanes divide the threads");
    constexpr int kPerItem = Threads / L;
    constexpr int kItems = (S::kHidden + Threads - 1) / Threads;
    constexpr int kCalls = (kItems + 3) / 4;
    static_assert(kItems <= 8, "at most the reference's two hiprand4 calls");
    // Threads k * L + l with k >= H / L own no column (item 0 is already past
    // the row), so their draws are skipped.
    constexpr int kEnd = kPerItem < kChunks ? kPerItem : kChunks;
    // Every Philox block of the row first - independent chains of quarter-rate
    // multiplies the compiler interleaves - then the ballots.
    uint4 random[kEnd][kCalls];
#pragma unroll
    for (int k = 0; k < kEnd; ++k) {
        const uint64_t subsequence = static_cast<uint64_t>(row) * Threads + k * L + lane;
#pragma unroll
        for (int n = 0; n < kCalls; ++n) {
            const uint64_t low = position + n;
            const uint64_t high = subsequence + (low < position ? 1 : 0);
            random[k][n] = philox4x32_10(
                make_uint4(static_cast<uint32_t>(low), static_cast<uint32_t>(low >> 32),
                           static_cast<uint32_t>(high), static_cast<uint32_t>(high >> 32)),
                key0, key1);
        }
    }
    // The previous row's reads of `stage` (other lanes of this wave) come
    // before this row's writes.
    wave_handoff();
#pragma unroll
    for (int k = 0; k < kEnd; ++k) {
#pragma unroll
        for (int n = 0; n < kCalls; ++n) {
            const uint32_t draws[4] = {random[k][n].x, random[k][n].y, random[k][n].z,
                                       random[k][n].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                constexpr int kUnused = -1;
                const int item = 4 * n + e;
                const int chunk = item < kItems ? item * kPerItem + k : kUnused;
                if (chunk != kUnused && chunk < kChunks) {
                    const uint64_t ballot = __ballot(draws[e] >= threshold);
                    if (lane < L / 16) {
                        stage[chunk * (L / 16) + lane] =
                            static_cast<uint16_t>(ballot >> (group * L + 16 * lane));
                    }
                }
            }
        }
    }
    // The staging writes of lanes < L / 16 come before every lane's reads.
    wave_handoff();
    uint32_t keep = 0;
#pragma unroll
    for (int v = 0; v < S::kV; ++v) {
        const int vector = v * L + lane;
        keep |= ((static_cast<uint32_t>(stage[vector / 4]) >> (4 * (vector % 4))) & 0xFu)
            << (4 * v);
    }
    return keep;
}

// The same draws with run-time loop bounds (one Philox chain after another,
// each followed by its ballots): RLN_REFERENCE_DRAWS_UNROLLED=0.
template <typename S>
__device__ __forceinline__ uint32_t reference_keep_bits_looped(
    uint16_t* stage, int64_t row, int lane, int group, int threads, uint64_t position,
    uint32_t key0, uint32_t key1, uint32_t threshold) {
    constexpr int L = S::kLanes;
    constexpr int kChunks = S::kHidden / L;
    const int per_item = threads / L;
    const int items = (S::kHidden + threads - 1) / threads;
    const int calls = (items + 3) / 4;
    const int k_end = per_item < kChunks ? per_item : kChunks;
    wave_handoff();
    for (int k = 0; k < k_end; ++k) {
        const uint64_t subsequence = static_cast<uint64_t>(row) * threads + k * L + lane;
        for (int n = 0; n < calls; ++n) {
            const uint64_t low = position + n;
            const uint64_t high = subsequence + (low < position ? 1 : 0);
            const uint4 random = philox4x32_10(
                make_uint4(static_cast<uint32_t>(low), static_cast<uint32_t>(low >> 32),
                           static_cast<uint32_t>(high), static_cast<uint32_t>(high >> 32)),
                key0, key1);
            const uint32_t draws[4] = {random.x, random.y, random.z, random.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int item = 4 * n + e;
                const int chunk = item * per_item + k;
                if (item < items && chunk < kChunks) {
                    const uint64_t ballot = __ballot(draws[e] >= threshold);
                    if (lane < L / 16) {
                        stage[chunk * (L / 16) + lane] =
                            static_cast<uint16_t>(ballot >> (group * L + 16 * lane));
                    }
                }
            }
        }
    }
    wave_handoff();
    uint32_t keep = 0;
#pragma unroll
    for (int v = 0; v < S::kV; ++v) {
        const int vector = v * L + lane;
        keep |= ((static_cast<uint32_t>(stage[vector / 4]) >> (4 * (vector % 4))) & 0xFu)
            << (4 * v);
    }
    return keep;
}

// The reference stream's keep bits for a launch of `threads` (128, 192 or
// 256) threads per row: unrolled for the widths RLN_REFERENCE_DRAWS_UNROLLED
// selects (a wave-uniform switch), else the looped draws.
template <typename S, bool AllWidths = false>
__device__ __forceinline__ uint32_t reference_keep_bits(
    uint16_t* stage, int64_t row, int lane, int group, int threads, uint64_t position,
    uint32_t key0, uint32_t key1, uint32_t threshold) {
    constexpr int kApiThreads = S::kHidden == 1024 ? 192 : 128;
    if constexpr (RLN_REFERENCE_DRAWS_UNROLLED == 0) {
        return reference_keep_bits_looped<S>(stage, row, lane, group, threads, position, key0,
                                             key1, threshold);
    } else if constexpr (RLN_REFERENCE_DRAWS_UNROLLED == 1 && !AllWidths) {
        if (threads == kApiThreads) {
            return reference_keep_bits_of<S, kApiThreads>(stage, row, lane, group, position, key0,
                                                          key1, threshold);
        }
        return reference_keep_bits_looped<S>(stage, row, lane, group, threads, position, key0,
                                             key1, threshold);
    }
    switch (threads) {
        case 128:
            return reference_keep_bits_of<S, 128>(stage, row, lane, group, position, key0, key1,
                                                   threshold);
        case 192:
            return reference_keep_bits_of<S, 192>(stage, row, lane, group, position, key0, key1,
                                                   threshold);
        default:
            return reference_keep_bits_of<S, 256>(stage, row, lane, group, position, key0, key1,
                                                   threshold);
    }
}

// Rows are walked by teams: a wave (one or two rows at a time) when a row
// fits one wave, else the whole block (kWaves / P rows at a time), so that
// every wave of a block meets the same barriers.
template <typename S, int Threads>
struct Teams {
    static constexpr int kWaves = Threads / kWaveSize;
    static constexpr int kGroups = S::kParts == 1 ? kWaves : kWaves / S::kParts;
    static constexpr int kRowsPerTeam = S::kParts == 1 ? S::kRowsPerWave : kGroups;
    static_assert(kWaves % S::kParts == 0, "a block holds whole rows");

    int64_t first;   // first row of this thread's team
    int64_t stride;  // rows between a team's consecutive steps
    int offset;      // this thread's row within the team's step
    int group;       // row slot within the block for the LDS exchange
    int part;

    __device__ __forceinline__ Teams() {
        const int lane = threadIdx.x & (kWaveSize - 1);
        const int wave = threadIdx.x / kWaveSize;
        if constexpr (S::kParts == 1) {
            const int64_t team = static_cast<int64_t>(blockIdx.x) * kWaves + wave;
            first = team * kRowsPerTeam;
            stride = static_cast<int64_t>(gridDim.x) * kWaves * kRowsPerTeam;
            offset = lane / S::kLanes;
            group = wave;
            part = 0;
        } else {
            first = static_cast<int64_t>(blockIdx.x) * kRowsPerTeam;
            stride = static_cast<int64_t>(gridDim.x) * kRowsPerTeam;
            offset = wave / S::kParts;
            group = offset;
            part = wave % S::kParts;
        }
    }
};

// `Ring`: the kernel instance walks its rows with look-ahead in a ring of
// register buffers (two rows ahead for one-part rows of up to three slots):
// launches whose teams walk several rows. The other instance - paced walks
// and one-ahead walks that copy rows between registers - serves the large
// launches whose teams take one or two row steps, where the ring's registers
// would only lower occupancy (measured: [262144, 128] forward 117 us with
// the ring's 171+ VGPRs against 80 us).
template <typename S, typename B, typename N, bool Aligned, bool Ring>
__global__ __launch_bounds__(S::kForwardThreads)
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
    float* __restrict__ zero_weight,
    float* __restrict__ zero_bias,
    int64_t rows,
    S shape,
    float eps,
    int dropout,
    float scale,
    uint32_t threshold,
    PhiloxArgs philox,
    int paced,
    int write_through) {
    constexpr int V = S::kV;
    using T = Teams<S, S::kForwardThreads>;
    const bool wt = write_through != 0;
    const int64_t hidden = shape.hidden();
    const float inv_hidden = shape.inv_hidden();
    const T team;
    const Slots<S> slots{team.part, static_cast<int>(threadIdx.x & (kWaveSize - 1)) % S::kLanes,
                         hidden};
    const int l = slots.lane;
    // Row sums of multi-wave rows: [0] the mean's, [1] the variance's. Two
    // arrays and a barrier per sum keep a wave that runs ahead from
    // overwriting a value another wave has yet to read.
    __shared__ float exchange[2][T::kGroups][S::kParts];
    // Keep bits of the reference's stream, staged per row (fixed shapes).
    constexpr bool kReferenceStream = S::kHidden > 0;
    constexpr int kStagePieces = kReferenceStream ? S::kHidden / 16 : 1;
    __shared__ uint16_t stage[kReferenceStream ? T::kWaves * S::kRowsPerWave : 1][kStagePieces];

    f32x4 w[V];
    f32x4 b[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
        w[v] = load_parameter4<Aligned>(weight + slots.column(v));
        b[v] = load_parameter4<Aligned>(bias + slots.column(v));
    }

    // Zero the weight/bias gradient sums a later backward accumulates into.
    if (zero_weight != nullptr) {
        const int64_t threads = static_cast<int64_t>(gridDim.x) * S::kForwardThreads;
        for (int64_t i = static_cast<int64_t>(blockIdx.x) * S::kForwardThreads + threadIdx.x;
             i < hidden; i += threads) {
            zero_weight[i] = 0.0f;
            zero_bias[i] = 0.0f;
        }
    }

    // The Philox key and position of this call (from the generator's device
    // state under graph capture). Read after the team's first row loads are
    // issued, so those loads do not wait behind them (C1 forward 0.1 us).
    uint32_t key0 = 0;
    uint32_t key1 = 0;
    uint64_t position = 0;
    auto read_philox_state = [&]() {
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
    };
    const bool reference_stream = kReferenceStream && dropout && philox.threads != 0;

    // Loads x and the branch of one row. The loads are unconditional (a row
    // past the end reads the last row instead, an idle slot its row's first
    // columns, and both are discarded), so the compiler can count them and
    // wait for exactly the ones a computation needs; a load under a branch
    // makes it wait for all. Paced loads wait slice by slice anyway, so they
    // skip idle slots (10 % faster at H = 896).
    auto load_row = [&](ForwardRow<V, B>& r, int64_t row, bool wait_slices) {
        const int64_t source = row < rows ? row : rows - 1;
        const float* x_row = x + source * hidden;
        const B* branch_row = branch + source * hidden;
#pragma unroll
        for (int v = 0; v < V; ++v) {
            if (wait_slices && !slots.active(v)) {
                r.x[v] = zero4();
                r.branch[v] = typename Vector4<B>::type{};
                continue;
            }
            const int column = slots.column(v);
            r.x[v] = load4<Aligned>(x_row + column);
            r.branch[v] = load_raw4<B, Aligned>(branch_row + column);
            if (wait_slices) {
                __builtin_amdgcn_s_waitcnt(0);
            }
        }
    };

    // The reference stream's keep bits of a row (0 in the library's layout,
    // whose draws happen slot by slot in process_row). They depend on the
    // row index only, so the loops below compute them a row ahead, while
    // that row's loads or the previous row's stores are in flight. (Drawing
    // the library's layout a row ahead too measured within +-2 %, either
    // way, by hidden size.)
    auto reference_keep = [&](int64_t row) -> uint32_t {
        if constexpr (kReferenceStream) {
            if (reference_stream) {
                const int wave = threadIdx.x / kWaveSize;
                constexpr bool kAllWidths =
                    S::kHidden == 768 && sizeof(B) == 2 && std::is_same_v<N, float>;
                return reference_keep_bits<S, kAllWidths>(
                    stage[wave * S::kRowsPerWave + team.offset], row, l, team.offset,
                    philox.threads, position, key0, key1, threshold);
            }
        }
        return 0u;
    };

    auto process_row = [&](const ForwardRow<V, B>& r, int64_t row, uint32_t reference_bits) {
        const bool valid = row < rows;
        // The wave's rows of this step (consecutive; wave-uniform first row
        // and count) and this lane's row among them; the outputs' stores go
        // through descriptors over exactly those rows.
        const int64_t wave_row = wave_uniform(row - (S::kParts == 1 ? team.offset : 0));
        const int64_t left = rows - wave_row;
        const int64_t wave_rows =
            left <= 0 ? 0 : left < S::kRowsPerWave ? left : S::kRowsPerWave;
        const uint32_t row_in_wave = static_cast<uint32_t>(row - wave_row);
        const uint32_t element = row_in_wave * static_cast<uint32_t>(hidden);
        const rsrc_t updated_out = output_range(updated, wave_row * hidden, wave_rows * hidden);
        const rsrc_t normalized_out =
            output_range(normalized, wave_row * hidden, wave_rows * hidden);
        f32x4 u[V];
        uint32_t keep_bits[V];
#pragma unroll
        for (int v = 0; v < V; ++v) {
            f32x4 bv = widen4<B>(r.branch[v]);
            if (dropout) {
                uint32_t k0, k1, k2, k3;
                if (reference_stream) {
                    const uint32_t bits = reference_bits >> (4 * v);
                    k0 = bits & 1u;
                    k1 = (bits >> 1) & 1u;
                    k2 = (bits >> 2) & 1u;
                    k3 = (bits >> 3) & 1u;
                } else {
                    const uint64_t group =
                        static_cast<uint64_t>(row) * (hidden / 4) + slots.vector(v);
                    const uint4 random = philox4x32_10(
                        make_uint4(
                            static_cast<uint32_t>(position),
                            static_cast<uint32_t>(position >> 32),
                            static_cast<uint32_t>(group),
                            static_cast<uint32_t>(group >> 32)),
                        key0,
                        key1);
                    k0 = random.x >= threshold;
                    k1 = random.y >= threshold;
                    k2 = random.z >= threshold;
                    k3 = random.w >= threshold;
                }
                bv.x = round_to_branch<B>(bv.x * static_cast<float>(k0) * scale);
                bv.y = round_to_branch<B>(bv.y * static_cast<float>(k1) * scale);
                bv.z = round_to_branch<B>(bv.z * static_cast<float>(k2) * scale);
                bv.w = round_to_branch<B>(bv.w * static_cast<float>(k3) * scale);
                keep_bits[v] = k0 | (k1 << 1) | (k2 << 2) | (k3 << 3);
            } else {
                keep_bits[v] = 0;
            }
            u[v] = r.x[v] + bv;
            if (valid && slots.active(v)) {
                output4<Aligned>(updated_out, (element + slots.column(v)) * 4, u[v], wt);
            }
            if (!slots.active(v)) {
                u[v] = zero4();
            }
        }

        if (dropout) {
            const int64_t words = hidden / 32;
            const rsrc_t mask_out = output_range(mask, wave_row * words, wave_rows * words);
#pragma unroll
            for (int v = 0; v < V; ++v) {
                // A word's 32 columns belong to 8 lanes of one slot, all
                // active or all idle (hidden is a multiple of 32).
                const uint32_t word = or8(keep_bits[v] << (4 * (l & 7)));
                if (valid && slots.active(v) && (l & 7) == 0) {
                    output_b32(mask_out,
                               (row_in_wave * static_cast<uint32_t>(words) + slots.vector(v) / 8)
                                   * 4,
                               word, wt);
                }
            }
        }

        float partial = 0.0f;
#pragma unroll
        for (int v = 0; v < V; ++v) {
            partial += sum4(u[v]);
        }
        const float mean = team_sum<S>(partial, exchange[0], team.group, team.part) * inv_hidden;

        float square = 0.0f;
#pragma unroll
        for (int v = 0; v < V; ++v) {
            u[v] = slots.active(v) ? u[v] - mean : zero4();
            square += (u[v].x * u[v].x + u[v].y * u[v].y)
                + (u[v].z * u[v].z + u[v].w * u[v].w);
        }
        const float variance =
            team_sum<S>(square, exchange[1], team.group, team.part) * inv_hidden;
        const float rstd = rsqrtf(variance + eps);

        if (valid) {
            if (l == 0 && team.part == 0) {
                output_b32(output_range(mean_out, wave_row, wave_rows), row_in_wave * 4,
                           __builtin_bit_cast(uint32_t, mean), wt);
                output_b32(output_range(rstd_out, wave_row, wave_rows), row_in_wave * 4,
                           __builtin_bit_cast(uint32_t, rstd), wt);
            }
#pragma unroll
            for (int v = 0; v < V; ++v) {
                const f32x4 y = {
                    __builtin_fmaf(u[v].x * rstd, w[v].x, b[v].x),
                    __builtin_fmaf(u[v].y * rstd, w[v].y, b[v].y),
                    __builtin_fmaf(u[v].z * rstd, w[v].z, b[v].z),
                    __builtin_fmaf(u[v].w * rstd, w[v].w, b[v].w)};
                if (slots.active(v)) {
                    output_convert4<N, Aligned>(normalized_out,
                                                (element + slots.column(v)) * sizeof(N), y, wt);
                }
            }
        }
    };

    // Two schedules. Look-ahead (small launches): the next row's loads (the
    // next two rows' for one-part rows of up to three slots) are in flight
    // while the current row is computed and stored. Paced (large launches):
    // a row is loaded after the previous one is stored, one 4-column slice
    // at a time, each waited for (with every earlier store of the wave),
    // which keeps fewer reads and writes interleaved per wave and streams
    // large tensors faster. The team's rows are first + i * stride, i <
    // count (uniform over a team, so a multi-wave team meets its barriers
    // together); no load reaches past them. The look-ahead walks keep their
    // rows in a ring of two or three register buffers whose roles rotate by
    // unrolling: a row copied between registers would wait for its loads,
    // and with them for every older access, before the next loads issue.
    const int64_t stride = team.stride;
    const int64_t first = team.first;
    if (first >= rows) {
        return;
    }
    const int64_t count = (rows - first + stride - 1) / stride;
    auto row_of = [&](int64_t i) { return first + i * stride + team.offset; };
    ForwardRow<V, B> ra;
    load_row(ra, row_of(0), false);
    read_philox_state();
    uint32_t keep_a = reference_keep(row_of(0));
    if constexpr (!Ring) {
        if (paced) {
            for (int64_t i = 0; i + 1 < count; ++i) {
                process_row(ra, row_of(i), keep_a);
                keep_a = reference_keep(row_of(i + 1));
                load_row(ra, row_of(i + 1), true);
            }
        } else {
            for (int64_t i = 0; i + 1 < count; ++i) {
                ForwardRow<V, B> next;
                load_row(next, row_of(i + 1), false);
                process_row(ra, row_of(i), keep_a);
                keep_a = reference_keep(row_of(i + 1));
                ra = next;
            }
        }
        process_row(ra, row_of(count - 1), keep_a);
    } else if constexpr (RLN_FWD_TWO_AHEAD && S::kParts == 1 && V <= 3) {
        ForwardRow<V, B> rb;
        ForwardRow<V, B> rc;
        uint32_t keep_b = 0;
        uint32_t keep_c = 0;
        if (count > 1) {
            load_row(rb, row_of(1), false);
        }
        int64_t i = 0;
        for (; i + 3 <= count; i += 3) {
            load_row(rc, row_of(i + 2), false);
            process_row(ra, row_of(i), keep_a);
            keep_b = reference_keep(row_of(i + 1));
            if (i + 3 < count) {
                load_row(ra, row_of(i + 3), false);
            }
            process_row(rb, row_of(i + 1), keep_b);
            keep_c = reference_keep(row_of(i + 2));
            if (i + 4 < count) {
                load_row(rb, row_of(i + 4), false);
            }
            process_row(rc, row_of(i + 2), keep_c);
            if (i + 3 < count) {
                keep_a = reference_keep(row_of(i + 3));
            }
        }
        if (i < count) {
            process_row(ra, row_of(i), keep_a);
            if (i + 1 < count) {
                keep_b = reference_keep(row_of(i + 1));
                process_row(rb, row_of(i + 1), keep_b);
            }
        }
    } else {
        ForwardRow<V, B> rb;
        uint32_t keep_b = 0;
        int64_t i = 0;
        for (; i + 2 <= count; i += 2) {
            load_row(rb, row_of(i + 1), false);
            process_row(ra, row_of(i), keep_a);
            keep_b = reference_keep(row_of(i + 1));
            if (i + 2 < count) {
                load_row(ra, row_of(i + 2), false);
            }
            process_row(rb, row_of(i + 1), keep_b);
            if (i + 2 < count) {
                keep_a = reference_keep(row_of(i + 2));
            }
        }
        if (i < count) {
            process_row(ra, row_of(i), keep_a);
        }
    }
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

template <typename S, typename B, typename GY, bool Aligned>
__global__ __launch_bounds__(S::kBackwardBlockThreads)
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
    S shape,
    int flags,
    float scale,
    int paced,
    int write_through) {
    constexpr int L = S::kLanes;
    const bool wt = write_through != 0;
    constexpr int V = S::kV;
    constexpr int P = S::kParts;
    using T = Teams<S, S::kBackwardBlockThreads>;
    constexpr int kWaves = T::kWaves;
    constexpr bool kTwoAhead = P == 1 && V <= RLN_BWD_TWO_AHEAD_MAX_SLOTS;
    const int64_t hidden = shape.hidden();
    const float inv_hidden = shape.inv_hidden();
    const int lane = threadIdx.x & (kWaveSize - 1);
    const int wave_in_block = threadIdx.x / kWaveSize;
    const T team;
    const Slots<S> slots{team.part, lane % L, hidden};
    const int l = slots.lane;
    // Row sums of multi-wave rows: [0] Σq, [1] Σq·x̂. Two arrays and a
    // barrier per sum keep a wave that runs ahead from overwriting a value
    // another wave has yet to read.
    __shared__ float exchange[2][T::kGroups][P];

    const bool has_gu = flags & kHasGradUpdated;
    const bool has_gy = flags & kHasGradNormalized;
    const bool dropout = flags & kDropout;
    const bool parameters = flags & kParameters;

    // Sixteen-wave blocks (128 VGPRs) read the weight per row instead of
    // holding it: 4 VGPRs spilled instead of 15.
    constexpr bool kWeightPerRow = P == 16;
    f32x4 held_weight[kWeightPerRow ? 1 : V];
    f32x4 acc_w[V];
    f32x4 acc_b[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
        if constexpr (!kWeightPerRow) {
            held_weight[v] = load_parameter4<Aligned>(weight + slots.column(v));
        }
        acc_w[v] = zero4();
        acc_b[v] = zero4();
    }

    // Loads every global value of one row. The loads are unconditional, so
    // the compiler can count them and wait for exactly the ones a computation
    // needs (a load under a branch makes it wait for all): an absent input
    // reads the row of `updated` in its place, a row past the end reads the
    // last row, an idle slot its row's first columns; process_row discards
    // what it read. (Unlike the forward, skipping idle slots in paced loads
    // measured slower here: 9 % at H = 640 and 896.)
    auto load_row = [&](BackwardRow<V, GY>& r, int64_t row, bool wait_slices) {
        const int64_t source = row < rows ? row : rows - 1;
        const int64_t base = source * hidden;
        const float* u_row = updated + base;
        const GY* gy_row = has_gy ? grad_normalized + base : reinterpret_cast<const GY*>(u_row);
        const float* gu_row = has_gu ? grad_updated + base : u_row;
        const uint32_t* mask_row = dropout ? mask + source * (hidden / 32)
                                           : reinterpret_cast<const uint32_t*>(u_row);
        r.mean = mean_in[source];
        r.rstd = rstd_in[source];
#pragma unroll
        for (int v = 0; v < V; ++v) {
            const int column = slots.column(v);
            r.u[v] = load4<Aligned>(u_row + column);
            r.gy[v] = load_raw4<GY, Aligned>(gy_row + column);
            r.gu[v] = load4<Aligned>(gu_row + column);
            r.mask_word[v] = mask_row[column / 32];
            if (wait_slices) {
                __builtin_amdgcn_s_waitcnt(0);
            }
        }
    };

    // Input gradients of one row and, with `accumulate`, its contribution to
    // the parameter sums.
    auto process_row = [&](const BackwardRow<V, GY>& r, int64_t row, bool accumulate) {
        f32x4 w[V];
#pragma unroll
        for (int v = 0; v < V; ++v) {
            if constexpr (kWeightPerRow) {
                w[v] = load_parameter4<Aligned>(weight + slots.column(v));
            } else {
                w[v] = held_weight[v];
            }
        }
        const bool valid = row < rows;
        // The wave's rows of this step and this lane's row among them (as in
        // the forward); the input gradients go out through descriptors over
        // exactly those rows.
        const int64_t wave_row = wave_uniform(row - (P == 1 ? team.offset : 0));
        const int64_t left = rows - wave_row;
        const int64_t wave_rows =
            left <= 0 ? 0 : left < S::kRowsPerWave ? left : S::kRowsPerWave;
        const uint32_t element =
            static_cast<uint32_t>(row - wave_row) * static_cast<uint32_t>(hidden);
        const rsrc_t grad_x_out = output_range(grad_x, wave_row * hidden, wave_rows * hidden);
        const rsrc_t grad_branch_out =
            output_range(grad_branch, wave_row * hidden, wave_rows * hidden);
        f32x4 xhat[V];
        f32x4 gy[V];
        float sum_q = 0.0f;
        float sum_qx = 0.0f;
        // Inputs that were not given, every input of a row past the end and
        // idle slots count as zero.
        const bool use_gy = has_gy && valid;
#pragma unroll
        for (int v = 0; v < V; ++v) {
            const bool live = use_gy && slots.active(v);
            gy[v] = live ? widen4<GY>(r.gy[v]) : zero4();
            xhat[v] = slots.active(v) ? (r.u[v] - r.mean) * r.rstd : zero4();
            const f32x4 q = gy[v] * w[v];
            sum_q += sum4(q);
            sum_qx += (q.x * xhat[v].x + q.y * xhat[v].y)
                + (q.z * xhat[v].z + q.w * xhat[v].w);
        }

        float mean_q = 0.0f;
        float mean_qx = 0.0f;
        if (has_gy) {
            mean_q = team_sum<S>(sum_q, exchange[0], team.group, team.part) * inv_hidden;
            mean_qx = team_sum<S>(sum_qx, exchange[1], team.group, team.part) * inv_hidden;
        }

        if (valid) {
#pragma unroll
            for (int v = 0; v < V; ++v) {
                if (!slots.active(v)) {
                    continue;
                }
                const int column = slots.column(v);
                f32x4 g = has_gu ? r.gu[v] : zero4();
                if (has_gy) {
                    const f32x4 q = gy[v] * w[v];
                    g = g + r.rstd * ((q - mean_q) - xhat[v] * mean_qx);
                }
                output4<Aligned>(grad_x_out, (element + column) * 4, g, wt);
                if (dropout) {
                    const uint32_t bits = r.mask_word[v] >> (4 * (l & 7));
                    g.x = g.x * (static_cast<float>(bits & 1u) * scale);
                    g.y = g.y * (static_cast<float>((bits >> 1) & 1u) * scale);
                    g.z = g.z * (static_cast<float>((bits >> 2) & 1u) * scale);
                    g.w = g.w * (static_cast<float>((bits >> 3) & 1u) * scale);
                }
                output_convert4<B, Aligned>(grad_branch_out, (element + column) * sizeof(B), g,
                                            wt);
            }
        }

        if (parameters && accumulate) {
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

    // A row's contribution to the parameter sums alone, with the arithmetic
    // process_row uses (the lane's sums come out bitwise the same).
    auto accumulate_row = [&](const BackwardRow<V, GY>& r, int64_t row) {
        if (!(has_gy && row < rows)) {
            return;
        }
#pragma unroll
        for (int v = 0; v < V; ++v) {
            if (!slots.active(v)) {
                continue;
            }
            const f32x4 gy = widen4<GY>(r.gy[v]);
            const f32x4 xhat = (r.u[v] - r.mean) * r.rstd;
            acc_w[v].x = __builtin_fmaf(gy.x, xhat.x, acc_w[v].x);
            acc_w[v].y = __builtin_fmaf(gy.y, xhat.y, acc_w[v].y);
            acc_w[v].z = __builtin_fmaf(gy.z, xhat.z, acc_w[v].z);
            acc_w[v].w = __builtin_fmaf(gy.w, xhat.w, acc_w[v].w);
            acc_b[v] = acc_b[v] + gy;
        }
    };

    // The block's parameter sums: staged per wave for the fixed-order combine,
    // or (early mode) added up in LDS as [2, hidden] floats in the same space.
    __shared__ f32x4 staging[V][kWaves][kWaveSize][2];
    __shared__ int arrivals;
    static_assert(sizeof(staging) >= 2 * sizeof(float) * V * P * L * 4, "LDS sums fit");
    float* const block_sums = reinterpret_cast<float*>(&staging[0][0][0][0]);
    const bool early = RLN_BWD_EARLY_PARAMETERS && parameters && !(flags & kPartials);
    if (early) {
        for (int i = threadIdx.x; i < 2 * hidden; i += S::kBackwardBlockThreads) {
            block_sums[i] = 0.0f;
        }
        if (threadIdx.x == 0) {
            arrivals = 0;
        }
        __syncthreads();
    }

    // Early mode: adds this wave's sums into the block's LDS sums (LDS
    // atomics), then counts the wave in; the block's last wave to arrive
    // adds the block's sums into grad_weight / grad_bias with fp32 atomics.
    // Every wave of the block calls it once, rows or not.
    auto deposit_parameters = [&]() {
#pragma unroll
        for (int v = 0; v < V; ++v) {
            if (!slots.active(v)) {
                continue;
            }
            const int column = slots.column(v);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                atomicAdd(block_sums + column + e, acc_w[v][e]);
                atomicAdd(block_sums + hidden + column + e, acc_b[v][e]);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        int arrived = 0;
        if (lane == 0) {
            arrived = atomicAdd(&arrivals, 1);
        }
        arrived = __builtin_amdgcn_readfirstlane(arrived);
        if (arrived == kWaves - 1) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
            for (int i = lane; i < 2 * hidden; i += kWaveSize) {
                const bool bias_sum = i >= hidden;
                unsafeAtomicAdd((bias_sum ? grad_bias : grad_weight) + (i - (bias_sum ? hidden : 0)),
                                block_sums[i]);
            }
        }
    };

    // Each team walks its rows under one of two schedules: look-ahead (the
    // next row's loads - the next two rows' for one-wave rows of up to three
    // slots, which still fit the two waves per SIMD this kernel runs at - in
    // flight while the current row is reduced and stored; small launches;
    // the second row measured 3 % faster at C1) or paced (a row loaded after the previous one is
    // stored, one 4-column slice at a time, each waited for; large launches,
    // where fewer interleaved reads and writes per wave stream faster). The
    // last row of a team is peeled off, so no load reaches past the team's
    // rows. `first` is uniform over a team, so a multi-wave team meets its
    // barriers together; a team without rows still takes part in the block's
    // combine below.
    // The team's rows are first + i * stride, i < count (this lane's row is
    // offset by team.offset). Look-ahead walks keep their rows in a ring of
    // two (one row ahead) or three (two rows ahead) register buffers whose
    // roles rotate by unrolling, so no row is ever copied between registers:
    // a copy would wait for the copied row's loads (and with them for every
    // older access, stores included) before the next row's loads are issued.
    // In early mode the rows still held when a team's walk ends (its last
    // one or two) add their contributions first, the wave deposits its sums,
    // and only then are those rows' gradients computed and stored, so that
    // the block's global atomics drain under that work instead of after it.
    const int64_t stride = team.stride;
    const int64_t first = team.first;
    const int64_t count = first < rows ? (rows - first + stride - 1) / stride : 0;
    auto row_of = [&](int64_t i) { return first + i * stride + team.offset; };
    // Finishes the walk on the held rows `a` (row i) and, when present, `b`
    // (row i + 1).
    auto finish = [&](const BackwardRow<V, GY>& a, const BackwardRow<V, GY>& b, int64_t i) {
        const bool second = i + 1 < count;
        if (early) {
            accumulate_row(a, row_of(i));
            if (second) {
                accumulate_row(b, row_of(i + 1));
            }
            deposit_parameters();
        }
        process_row(a, row_of(i), !early);
        if (second) {
            process_row(b, row_of(i + 1), !early);
        }
    };
    if (count > 0) {
        BackwardRow<V, GY> ra;
        BackwardRow<V, GY> rb;
        load_row(ra, row_of(0), false);
        if (paced) {
            int64_t i = 0;
            for (; i + 1 < count; ++i) {
                process_row(ra, row_of(i), true);
                load_row(ra, row_of(i + 1), true);
            }
            finish(ra, rb, i);
        } else if constexpr (!RLN_BWD_RING || P > 1 || S::kCopyWalk) {
            int64_t i = 0;
            for (; i + 1 < count; ++i) {
                BackwardRow<V, GY> next;
                load_row(next, row_of(i + 1), false);
                process_row(ra, row_of(i), true);
                ra = next;
            }
            finish(ra, rb, i);
        } else if constexpr (kTwoAhead) {
            BackwardRow<V, GY> rc;
            if (count > 1) {
                load_row(rb, row_of(1), false);
            }
            int64_t i = 0;
            for (; i + 3 <= count; i += 3) {
                load_row(rc, row_of(i + 2), false);
                process_row(ra, row_of(i), true);
                if (i + 3 < count) {
                    load_row(ra, row_of(i + 3), false);
                }
                process_row(rb, row_of(i + 1), true);
                if (i + 4 < count) {
                    load_row(rb, row_of(i + 4), false);
                }
                process_row(rc, row_of(i + 2), true);
            }
            if (i < count) {
                finish(ra, rb, i);
            } else if (early) {
                deposit_parameters();
            }
        } else {
            int64_t i = 0;
            for (; i + 2 <= count; i += 2) {
                load_row(rb, row_of(i + 1), false);
                process_row(ra, row_of(i), true);
                if (i + 2 < count) {
                    load_row(ra, row_of(i + 2), false);
                }
                process_row(rb, row_of(i + 1), true);
            }
            if (i < count) {
                finish(ra, rb, i);
            } else if (early) {
                deposit_parameters();
            }
        }
    } else if (early) {
        deposit_parameters();
    }

    if (!parameters || early) {
        return;
    }

    // Combine the block's sums in a fixed order. A column is owned by one
    // (part, lane) pair; for each, the block adds groups 0..kGroups-1 and,
    // within a wave, row slots 0..kRowsPerWave-1. All slots are staged at
    // once (16 KiB of LDS per slot), so one barrier serves the whole combine.
    const bool write_partials = flags & kPartials;
#pragma unroll
    for (int v = 0; v < V; ++v) {
        staging[v][wave_in_block][lane][0] = acc_w[v];
        staging[v][wave_in_block][lane][1] = acc_b[v];
    }
    __syncthreads();
    // V x P x L owners x 8 floats to produce; the block's threads share them.
    constexpr int kPerSlot = P * L * 8;
    for (int entry = threadIdx.x; entry < V * kPerSlot; entry += S::kBackwardBlockThreads) {
        const int v = entry / kPerSlot;
        const int owner = (entry % kPerSlot) / 8;
        const int owner_part = owner / L;
        const int slot = owner % L;
        const int which = (entry / 4) & 1;  // 0 = weight, 1 = bias
        const int component = entry & 3;
        const int64_t column = static_cast<int64_t>((v * P + owner_part) * L + slot) * 4
            + component;
        if (S::kRagged && column >= hidden) {
            continue;
        }
        float total = 0.0f;
#pragma unroll
        for (int group = 0; group < T::kGroups; ++group) {
#pragma unroll
            for (int source_sub = 0; source_sub < S::kRowsPerWave; ++source_sub) {
                total += staging[v][group * P + owner_part][source_sub * L + slot][which]
                                [component];
            }
        }
        if (write_partials) {
            partials[(static_cast<int64_t>(blockIdx.x) * 2 + which) * hidden + column] = total;
        } else {
            unsafeAtomicAdd((which ? grad_bias : grad_weight) + column, total);
        }
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
    float* zero_weight;  // optional: zeroed by the launch (hidden floats each)
    float* zero_bias;
    int64_t rows;
    float eps;
    int dropout;
    float scale;
    uint32_t threshold;
    PhiloxArgs philox;
    int compute_units;  // of the launch device; 0 = unknown (forward_blocks)
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

// The dispatch shape must be the one shape_info() describes for the hidden
// size, pass and rows, since the backward's grid (and so the deterministic
// order and the workspace size) is computed from the latter.
template <typename S>
int check_shape(const S& shape, Pass pass, int64_t rows) {
    const ShapeInfo info = shape_info(shape.hidden(), pass, rows);
    if (info.parts != S::kParts || info.rows_per_wave != S::kRowsPerWave
        || info.vectors != S::kV || info.forward_threads != S::kForwardThreads
        || info.backward_threads != S::kBackwardBlockThreads) {
        return fail(RLN_ERR_UNSUPPORTED, "shape mismatch for hidden size %lld",
                    static_cast<long long>(shape.hidden()));
    }
    return RLN_OK;
}

// Blocks of one forward kernel instance a CU holds at once (registers and
// LDS permitting), asked of the runtime once per instance; 0 if it cannot say.
template <typename S, typename B, typename N, bool Aligned, bool Ring>
int forward_resident_blocks() {
    static const int resident = [] {
        int blocks = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &blocks,
                reinterpret_cast<const void*>(&rln_forward_kernel<S, B, N, Aligned, Ring>),
                S::kForwardThreads, 0) != hipSuccess) {
            static_cast<void>(hipGetLastError());  // clear the failed call's error
            return 0;
        }
        return blocks;
    }();
    return resident;
}

// Whether a forward launch runs the ring-walk kernel instance: launches that
// are not paced and whose grid gives teams several rows - the small-launch
// grid, the one-round grid of four-slot rows and the persistent grid of
// multi-wave rows (forward_blocks).
template <typename S>
bool forward_ring(int64_t rows, int64_t hidden) {
    if (forward_paced(rows, hidden)) {
        return false;
    }
    const int64_t elements = rows * hidden;
    if (S::kParts > 1) {
        return elements < (S::kParts < 8 ? kForwardPersistentElements
                                         : kForwardPersistentElements8);
    }
    if (S::kHidden > 0 && S::kV == 4 && elements < kForwardPersistentElements) {
        return true;
    }
    return elements < kForwardLargeElements;
}

template <typename S, typename B, typename N, bool Aligned, bool Ring>
int launch_forward_walk(const ForwardArgs& a, S shape) {
    const dim3 grid(static_cast<unsigned>(forward_blocks<S>(
        a.rows, shape.hidden(), a.compute_units,
        forward_resident_blocks<S, B, N, Aligned, Ring>())));
    rln_forward_kernel<S, B, N, Aligned, Ring><<<grid, S::kForwardThreads, 0, a.stream>>>(
        a.x,
        static_cast<const B*>(a.branch),
        a.weight,
        a.bias,
        a.updated,
        static_cast<N*>(a.normalized),
        a.mean,
        a.rstd,
        a.mask,
        a.zero_weight,
        a.zero_bias,
        a.rows,
        shape,
        a.eps,
        a.dropout,
        a.scale,
        a.threshold,
        a.philox,
        forward_paced(a.rows, shape.hidden()),
        a.rows * shape.hidden() < kForwardWriteThroughElements ? 1 : 0);
    return check_launch("rln_forward_kernel");
}

template <typename S, typename B, typename N, bool Aligned>
int launch_forward(const ForwardArgs& a, S shape) {
    return forward_ring<S>(a.rows, shape.hidden())
        ? launch_forward_walk<S, B, N, Aligned, true>(a, shape)
        : launch_forward_walk<S, B, N, Aligned, false>(a, shape);
}

template <typename S, typename B, typename GY, bool Aligned>
int launch_backward(const BackwardArgs& a, S shape) {
    const dim3 grid(static_cast<unsigned>(backward_blocks(a.rows, shape.hidden())));
    rln_backward_kernel<S, B, GY, Aligned><<<grid, S::kBackwardBlockThreads, 0, a.stream>>>(
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
        shape,
        a.flags,
        a.scale,
        backward_paced(a.rows, shape.hidden()),
        a.rows * shape.hidden() < kBackwardWriteThroughElements
                || (RLN_BWD_WIDE14_WRITE_THROUGH && S::kHidden == 0 && S::kParts == 4
                    && S::kV == 1)
            ? 1
            : 0);
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

// Every (branch, normalized, alignment) instantiation for one row shape;
// explicitly instantiated once per shape in rln_hidden.hip.
template <typename S>
int launch_forward_shape(const ForwardArgs& a, S shape, int branch_dtype, int normalized_dtype,
                         bool aligned) {
    const int status = check_shape(shape, Pass::kForward, a.rows);
    if (status != RLN_OK) {
        return status;
    }
    return with_dtype(branch_dtype, [&]<typename B>() {
        return with_dtype(normalized_dtype, [&]<typename N>() {
            using F = typename ForwardShape<S, N>::type;
            F forward_shape{};
            if constexpr (std::is_same_v<F, S>) {
                forward_shape = shape;
            }
            return aligned ? launch_forward<F, B, N, true>(a, forward_shape)
                           : launch_forward<F, B, N, false>(a, forward_shape);
        });
    });
}

template <typename S>
int launch_backward_shape(const BackwardArgs& a, S shape, int branch_dtype,
                          int grad_normalized_dtype, bool aligned) {
    const int status = check_shape(shape, Pass::kBackward, a.rows);
    if (status != RLN_OK) {
        return status;
    }
    return with_dtype(branch_dtype, [&]<typename B>() {
        return with_dtype(grad_normalized_dtype, [&]<typename GY>() {
            return aligned ? launch_backward<S, B, GY, true>(a, shape)
                           : launch_backward<S, B, GY, false>(a, shape);
        });
    });
}

// The row shapes, one translation unit each (rln_hidden.hip): the
// specialized sizes (1024's backward excepted, backward_runs_wide),
// and the (slots per lane, waves per row) pairs of the run-time lengths each
// pass runs (wide_parts).
#define RLN_FOR_EACH_FIXED(X) X(128) X(256) X(384) X(512) X(768) X(1024)
#define RLN_FOR_EACH_WIDE_FORWARD(X) \
    X(1, 1) X(2, 1) X(3, 1) X(4, 1) X(3, 2) X(4, 2) X(3, 4) X(4, 4) X(3, 8) X(4, 8)
#define RLN_FOR_EACH_WIDE_BACKWARD(X) \
    X(1, 1) X(2, 1) X(3, 1) X(1, 3) X(1, 4) X(3, 2) X(2, 4) X(3, 4) X(2, 8) X(3, 8) X(4, 8) \
    X(2, 16)

#define RLN_WIDE_CASE(V, P) \
    case P * 16 + V: return launch(WideShape<V, P>{hidden, inv_hidden});

// Calls `launch(shape)` with the shape a supported hidden size runs in
// `kPass` over `rows`.
template <Pass kPass, typename Launch>
int with_shape(int64_t hidden, int64_t rows, Launch&& launch) {
    switch (hidden) {
        case 128: return launch(FixedShape<128>{});
        case 256: return launch(FixedShape<256>{});
        case 384:
            if constexpr (kPass == Pass::kBackward) {
                if (backward_nine_waves(hidden, rows)) {
                    return launch(NineWaveShape<384>{});
                }
            }
            return launch(FixedShape<384>{});
        case 512: return launch(FixedShape<512>{});
        case 768:
            if constexpr (kPass == Pass::kBackward) {
                if (backward_twelve_waves(hidden, rows)) {
                    return launch(TwelveWaveShape<768>{});
                }
            }
            if (kPass == Pass::kForward || !backward_runs_wide(hidden, rows)) {
                return launch(FixedShape<768>{});
            }
            break;
        case 1024:
            if constexpr (kPass == Pass::kForward) {
                return launch(FixedShape<1024>{});
            }
            break;
        default: break;
    }
    if (!hidden_supported(hidden)) {
        return fail(RLN_ERR_UNSUPPORTED, "unsupported native hidden size: %lld",
                    static_cast<long long>(hidden));
    }
    const ShapeInfo info = shape_info(hidden, kPass, rows);
    const float inv_hidden = 1.0f / static_cast<float>(hidden);
    if constexpr (kPass == Pass::kForward) {
        switch (info.parts * 16 + info.vectors) {
            RLN_FOR_EACH_WIDE_FORWARD(RLN_WIDE_CASE)
            default: break;
        }
    } else {
        if (info.parts == 4 && info.backward_threads == 12 * kWaveSize) {
            if (info.vectors == 1) {
                return launch(StaggeredWideShape<1>{{hidden, inv_hidden}});
            }
            if (info.vectors == 2) {
                return launch(StaggeredWideShape<2>{{hidden, inv_hidden}});
            }
        }
        switch (info.parts * 16 + info.vectors) {
            RLN_FOR_EACH_WIDE_BACKWARD(RLN_WIDE_CASE)
            default: break;
        }
    }
    return fail(RLN_ERR_UNSUPPORTED, "no row shape for hidden size %lld",
                static_cast<long long>(hidden));
}

#define RLN_DECLARE_FIXED(H)                                                              \
    extern template int launch_forward_shape<FixedShape<H>>(                             \
        const ForwardArgs&, FixedShape<H>, int, int, bool);                               \
    extern template int launch_backward_shape<FixedShape<H>>(                            \
        const BackwardArgs&, FixedShape<H>, int, int, bool);
#define RLN_DECLARE_STAGGERED_BACKWARD()                                                  \
    extern template int launch_backward_shape<TwelveWaveShape<768>>(                     \
        const BackwardArgs&, TwelveWaveShape<768>, int, int, bool);                        \
    extern template int launch_backward_shape<NineWaveShape<384>>(                       \
        const BackwardArgs&, NineWaveShape<384>, int, int, bool);                          \
    extern template int launch_backward_shape<StaggeredWideShape<1>>(                    \
        const BackwardArgs&, StaggeredWideShape<1>, int, int, bool);                       \
    extern template int launch_backward_shape<StaggeredWideShape<2>>(                    \
        const BackwardArgs&, StaggeredWideShape<2>, int, int, bool);
#define RLN_DECLARE_WIDE_FORWARD(V, P)                                                    \
    extern template int launch_forward_shape<WideShape<V, P>>(                           \
        const ForwardArgs&, WideShape<V, P>, int, int, bool);
#define RLN_DECLARE_WIDE_BACKWARD(V, P)                                                   \
    extern template int launch_backward_shape<WideShape<V, P>>(                          \
        const BackwardArgs&, WideShape<V, P>, int, int, bool);

}  // namespace rln

#endif  // RLN_DEVICE_H
