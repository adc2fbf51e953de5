// Golden-vector generator for the reference's dropout stream (test
// infrastructure; built and run on the host by make_hiprand_vectors.py).
//
// The reference draws its dropout values with hipRAND's Philox4x32-10
// (csrc/residual_layer_norm_kernel.hip:13, :449-480). On ROCm, hiprand_init
// and hiprand4 forward to rocRAND's rocrand_init and rocrand4
// (hiprand/hiprand_kernel_rocm.h:201-222, :377-380), which are host-callable
// in rocrand/rocrand_philox4x32_10.h; this program calls those, so the
// numbers below come from the engine the reference links, not from a
// restatement of it.
//
// Input (stdin), one request per line:
//   stream <seed> <subsequence> <offset> <calls>
//       -> the uint4 results of <calls> rocrand4 calls after
//          rocrand_init(seed, subsequence, offset)
//   mask <first_row> <rows> <hidden> <threads> <seed> <offset> <threshold>
//       -> the reference kernel's keep-mask words for those rows: thread t of
//          row r draws from rocrand_init(seed, r * threads + t, offset),
//          random_values[0..3] from the first rocrand4 and [4..7] from the
//          second; column t + item * threads keeps iff
//          random_values[item] >= threshold; bit c % 32 of word c / 32
//          (reference :449-511, word layout :500-511).
// Output: one line per request, the uint32 words in decimal.
#include <rocrand/rocrand_philox4x32_10.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

static void stream(unsigned long long seed, unsigned long long subsequence,
                   unsigned long long offset, int calls) {
    rocrand_state_philox4x32_10 state;
    rocrand_init(seed, subsequence, offset, &state);
    for (int call = 0; call < calls; ++call) {
        const uint4 value = rocrand4(&state);
        std::printf("%s%u %u %u %u", call ? " " : "", value.x, value.y, value.z, value.w);
    }
    std::printf("\n");
}

static int mask(long long first_row, long long rows, int hidden, int threads,
                unsigned long long seed, unsigned long long offset, unsigned threshold) {
    const int items = (hidden + threads - 1) / threads;
    if (items > 8) {
        std::fprintf(stderr, "the reference draws at most 8 values per thread\n");
        return 1;
    }
    std::vector<uint32_t> words(static_cast<size_t>(rows) * (hidden / 32), 0u);
    for (long long local = 0; local < rows; ++local) {
        const unsigned long long row = static_cast<unsigned long long>(first_row + local);
        for (int t = 0; t < threads; ++t) {
            rocrand_state_philox4x32_10 state;
            rocrand_init(seed, row * threads + t, offset, &state);
            uint32_t values[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            const uint4 first = rocrand4(&state);
            values[0] = first.x;
            values[1] = first.y;
            values[2] = first.z;
            values[3] = first.w;
            if (items > 4) {
                const uint4 second = rocrand4(&state);
                values[4] = second.x;
                values[5] = second.y;
                values[6] = second.z;
                values[7] = second.w;
            }
            for (int item = 0; item < items; ++item) {
                const int column = t + item * threads;
                if (column < hidden && values[item] >= threshold) {
                    words[static_cast<size_t>(local) * (hidden / 32) + column / 32] |=
                        1u << (column % 32);
                }
            }
        }
    }
    for (size_t i = 0; i < words.size(); ++i) {
        std::printf("%s%u", i ? " " : "", words[i]);
    }
    std::printf("\n");
    return 0;
}

int main() {
    char kind[16];
    while (std::scanf("%15s", kind) == 1) {
        if (std::strcmp(kind, "stream") == 0) {
            unsigned long long seed, subsequence, offset;
            int calls;
            if (std::scanf("%llu %llu %llu %d", &seed, &subsequence, &offset, &calls) != 4) {
                return 2;
            }
            stream(seed, subsequence, offset, calls);
        } else if (std::strcmp(kind, "mask") == 0) {
            long long first_row, rows;
            int hidden, threads;
            unsigned long long seed, offset;
            unsigned threshold;
            if (std::scanf("%lld %lld %d %d %llu %llu %u", &first_row, &rows, &hidden, &threads,
                           &seed, &offset, &threshold) != 7) {
                return 2;
            }
            if (mask(first_row, rows, hidden, threads, seed, offset, threshold) != 0) {
                return 3;
            }
        } else {
            return 2;
        }
    }
    return 0;
}
