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
 *    This counter assignment is the MI355X build's own: the reference draws
 *    from hipRAND's Philox with a launch-shape-dependent subsequence
 *    (csrc/residual_layer_norm_kernel.hip:449-480), which no test of the
 *    reference pins bit for bit.
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
