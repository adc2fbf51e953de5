/*
 * CPU oracle - TEST INFRASTRUCTURE ONLY. Used by tests/, the smoke check in
 * __graft_entry__.py and the cpu_baseline leg of bench.py, only as the checker.
 * The product (gfx1010-kernels_amd/) never links, loads or calls it.
 *
 * Restates the dropout keep decision and mask layout of the fused residual
 * LayerNorm in plain C:
 *
 *  - keep(r, c) = u32 >= threshold, threshold = uint32(double(float(p)) * 2^32)
 *    (reference csrc/residual_layer_norm_kernel.hip:492 and :893-897);
 *  - mask word layout: bit (c % 32) of int32 word r * H / 32 + c / 32
 *    (reference csrc/residual_layer_norm_kernel.hip:500-511, :162-164);
 *  - u32 stream: Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random
 *    numbers: as easy as 1, 2, 3", SC'11), one block per four consecutive
 *    columns, counter = (offset/4 low, offset/4 high, g low, g high) with
 *    g = (r * H + c) / 4, key = (seed low, seed high); output word c % 4.
 *    This counter assignment is the MI355X build's own layout; the
 *    reference's hipRAND layout (csrc/residual_layer_norm_kernel.hip:449-480)
 *    is restated at the end of this file (oracle_reference_mask_rows).
 *
 * Pinned by: the Random123 known-answer vectors for philox4x32_10
 * (tests/golden/philox4x32_10_kat.json, tests/test_oracle.py) and a
 * per-element Python restatement of the layout on small shapes.
 */
#include <stdint.h>
#include <string.h>

#define PHILOX_M0 0xD2511F53u
#define PHILOX_M1 0xCD9E8D57u
#define PHILOX_W0 0x9E3779B9u
#define PHILOX_W1 0xBB67AE85u

void oracle_philox4x32_10(const uint32_t counter[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t c0 = counter[0], c1 = counter[1], c2 = counter[2], c3 = counter[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int round = 0; round < 10; ++round) {
        const uint64_t p0 = (uint64_t)PHILOX_M0 * c0;
        const uint64_t p1 = (uint64_t)PHILOX_M1 * c2;
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
        const uint32_t n1 = (uint32_t)p1;
        const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        const uint32_t n3 = (uint32_t)p0;
        c0 = n0;
        c1 = n1;
        c2 = n2;
        c3 = n3;
        k0 += PHILOX_W0;
        k1 += PHILOX_W1;
    }
    out[0] = c0;
    out[1] = c1;
    out[2] = c2;
    out[3] = c3;
}

/* Raw u32 draws for every element of a [rows, hidden] tensor. */
void oracle_dropout_uniform(
    int64_t rows, int64_t hidden, uint64_t seed, uint64_t offset, uint32_t* draws) {
    const uint64_t position = offset / 4;
    const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    const int64_t groups = rows * hidden / 4;
    for (int64_t g = 0; g < groups; ++g) {
        const uint32_t counter[4] = {
            (uint32_t)position, (uint32_t)(position >> 32),
            (uint32_t)(uint64_t)g, (uint32_t)((uint64_t)g >> 32)};
        oracle_philox4x32_10(counter, key, draws + 4 * g);
    }
}

/* Packed keep mask for rows [first_row, first_row + rows) of a tensor with
 * `hidden` columns (hidden % 32 == 0); words[0] is the first word of first_row. */
void oracle_dropout_mask_rows(
    int64_t first_row, int64_t rows, int64_t hidden, uint64_t seed, uint64_t offset,
    uint32_t threshold, uint32_t* words) {
    const uint64_t position = offset / 4;
    const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    const int64_t begin = first_row * hidden;
    const int64_t total = rows * hidden;
    memset(words, 0, (size_t)(total / 32) * sizeof(uint32_t));
    for (int64_t local = 0; local < total; local += 4) {
        const uint64_t g = (uint64_t)(begin + local) / 4;
        const uint32_t counter[4] = {
            (uint32_t)position, (uint32_t)(position >> 32), (uint32_t)g, (uint32_t)(g >> 32)};
        uint32_t draw[4];
        oracle_philox4x32_10(counter, key, draw);
        for (int j = 0; j < 4; ++j) {
            const int64_t element = local + j; /* = (r - first_row) * hidden + c */
            if (draw[j] >= threshold) {
                words[element / 32] |= 1u << (element % 32);
            }
        }
    }
}

/* Packed keep mask for a whole [rows, hidden] tensor. */
void oracle_dropout_mask(
    int64_t rows, int64_t hidden, uint64_t seed, uint64_t offset, uint32_t threshold,
    uint32_t* words) {
    oracle_dropout_mask_rows(0, rows, hidden, seed, offset, threshold, words);
}

/* ------------------------------------------------------------------------
 * The reference's own dropout stream: hipRAND's Philox4x32-10, which on ROCm
 * is rocRAND's engine (third-party dependency of the reference, not vendored
 * in it: rocRAND 4.2.0 of ROCm 7.2.0, rocrand/rocrand_philox4x32_10.h;
 * hiprand_init / hiprand4 forward to rocrand_init / rocrand4,
 * hiprand/hiprand_kernel_rocm.h:201-222, :377-380). Restated from its
 * published behaviour:
 *
 *  - rocrand_init(seed, subsequence, offset): key = (seed low, seed high);
 *    128-bit counter = subsequence * 2^64 + offset / 4; substate = offset % 4;
 *  - the n-th rocrand4 call (n = 0, 1, ...) returns words substate ..
 *    substate + 3 of the 8-word sequence philox(counter + n) ||
 *    philox(counter + n + 1) (for substate 0 that is philox(counter + n)).
 *
 * Pinned by vectors that tests/golden/make_hiprand_vectors.py writes by
 * calling rocRAND's rocrand_init / rocrand4 themselves
 * (tests/golden/hiprand_philox_vectors.json, tests/test_oracle.py).
 */

/* Philox block of the 128-bit counter (high:low) + n. */
static void philox_at(uint64_t low, uint64_t high, uint64_t n, const uint32_t key[2],
                      uint32_t out[4]) {
    const uint64_t sum = low + n;
    const uint64_t carry = sum < low ? 1u : 0u;
    const uint64_t top = high + carry;
    const uint32_t counter[4] = {(uint32_t)sum, (uint32_t)(sum >> 32), (uint32_t)top,
                                 (uint32_t)(top >> 32)};
    oracle_philox4x32_10(counter, key, out);
}

/* `calls` consecutive rocrand4 results after rocrand_init(seed, subsequence,
 * offset); out holds 4 * calls words. */
void oracle_hiprand_philox4(uint64_t seed, uint64_t subsequence, uint64_t offset, int calls,
                            uint32_t* out) {
    const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    const unsigned substate = (unsigned)(offset % 4);
    uint32_t current[4];
    philox_at(offset / 4, subsequence, 0, key, current);
    for (int n = 0; n < calls; ++n) {
        uint32_t next[4];
        philox_at(offset / 4, subsequence, (uint64_t)n + 1, key, next);
        for (unsigned j = 0; j < 4; ++j) {
            const unsigned word = substate + j;
            out[4 * n + j] = word < 4 ? current[word] : next[word - 4];
        }
        memcpy(current, next, sizeof(current));
    }
}

/* The reference's keep mask for rows [first_row, first_row + rows) of a
 * [*, hidden] tensor launched with `threads` threads per row
 * (csrc/residual_layer_norm_kernel.hip:449-511): thread t of row r draws
 * items = ceil(hidden / threads) values, random_values[0..3] from the first
 * hiprand4 of hiprand_init(seed, r * threads + t, offset) and [4..7] from the
 * second; column c = t + item * threads (< hidden) keeps iff
 * random_values[item] >= threshold; bit c % 32 of word c / 32. Returns 0, or
 * -1 when a thread would need more than the reference's 8 values. */
int oracle_reference_mask_rows(int64_t first_row, int64_t rows, int64_t hidden, int64_t threads,
                               uint64_t seed, uint64_t offset, uint32_t threshold,
                               uint32_t* words) {
    const int64_t items = (hidden + threads - 1) / threads;
    if (threads <= 0 || items > 8 || hidden % 32 != 0) {
        return -1;
    }
    const int calls = (int)((items + 3) / 4);
    memset(words, 0, (size_t)(rows * hidden / 32) * sizeof(uint32_t));
    for (int64_t local = 0; local < rows; ++local) {
        const uint64_t row = (uint64_t)(first_row + local);
        for (int64_t t = 0; t < threads; ++t) {
            uint32_t values[8];
            oracle_hiprand_philox4(seed, row * (uint64_t)threads + (uint64_t)t, offset, calls,
                                   values);
            for (int64_t item = 0; item < items; ++item) {
                const int64_t column = t + item * threads;
                if (column < hidden && values[item] >= threshold) {
                    words[local * (hidden / 32) + column / 32] |= 1u << (column % 32);
                }
            }
        }
    }
    return 0;
}
