/*
 * A plain C host for the C ABI (test infrastructure): allocates device memory
 * with the HIP runtime alone (no torch), runs one rln_forward + rln_backward
 * through include/rln.h and writes every output, so that
 * tests/test_gpu_cabi_host.py can check them against the oracle. It shows
 * the library needs nothing from PyTorch.
 *
 * Usage: rln_host <input file> <output file>
 * Input: int64 rows, hidden, threads, seed, offset, deterministic; double
 * dropout_p, eps; then x (fp32 [rows, hidden]), branch (fp16 bits), weight,
 * bias (fp32 [hidden]), grad_updated, grad_normalized (fp32 [rows, hidden]).
 * Output: updated, normalized (fp32), mean, rstd (fp32 [rows]), mask
 * (uint32 [rows * hidden / 32]), grad_x (fp32), grad_branch (fp16 bits),
 * grad_weight, grad_bias (fp32 [hidden]).
 */
#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "rln.h"

#define CHECK_HIP(call)                                                              \
    do {                                                                             \
        hipError_t status_ = (call);                                                 \
        if (status_ != hipSuccess) {                                                 \
            fprintf(stderr, "%s:%d: %s\n", __FILE__, __LINE__, hipGetErrorString(status_)); \
            exit(3);                                                                 \
        }                                                                            \
    } while (0)

#define CHECK_RLN(call)                                                              \
    do {                                                                             \
        int status_ = (call);                                                        \
        if (status_ != RLN_OK) {                                                     \
            fprintf(stderr, "%s:%d: rln status %d: %s\n", __FILE__, __LINE__, status_, \
                    rln_last_error());                                               \
            exit(4);                                                                 \
        }                                                                            \
    } while (0)

static void* read_block(FILE* file, size_t bytes) {
    void* data = malloc(bytes);
    if (data == NULL || fread(data, 1, bytes, file) != bytes) {
        fprintf(stderr, "short input\n");
        exit(2);
    }
    return data;
}

static void* to_device(const void* host, size_t bytes) {
    void* device = NULL;
    CHECK_HIP(hipMalloc(&device, bytes));
    CHECK_HIP(hipMemcpy(device, host, bytes, hipMemcpyHostToDevice));
    return device;
}

static void* device_buffer(size_t bytes) {
    void* device = NULL;
    CHECK_HIP(hipMalloc(&device, bytes > 0 ? bytes : 4));
    return device;
}

static void write_back(FILE* file, const void* device, size_t bytes) {
    void* host = malloc(bytes);
    if (host == NULL) {
        exit(2);
    }
    CHECK_HIP(hipMemcpy(host, device, bytes, hipMemcpyDeviceToHost));
    if (fwrite(host, 1, bytes, file) != bytes) {
        exit(2);
    }
    free(host);
}

int main(int argc, char** argv) {
    if (argc != 3) {
        fprintf(stderr, "usage: %s <input> <output>\n", argv[0]);
        return 1;
    }
    FILE* in = fopen(argv[1], "rb");
    if (in == NULL) {
        return 2;
    }
    int64_t header[6];
    double scalars[2];
    if (fread(header, sizeof(int64_t), 6, in) != 6 || fread(scalars, sizeof(double), 2, in) != 2) {
        return 2;
    }
    const int64_t rows = header[0], hidden = header[1];
    const int deterministic = (int)header[5];
    const size_t n = (size_t)(rows * hidden);
    const size_t words = (size_t)rln_mask_words(rows, hidden);

    void* x = read_block(in, n * 4);
    void* branch = read_block(in, n * 2);
    void* weight = read_block(in, (size_t)hidden * 4);
    void* bias = read_block(in, (size_t)hidden * 4);
    void* grad_updated = read_block(in, n * 4);
    void* grad_normalized = read_block(in, n * 4);
    fclose(in);

    hipStream_t stream;
    CHECK_HIP(hipStreamCreate(&stream));
    float* d_x = to_device(x, n * 4);
    void* d_branch = to_device(branch, n * 2);
    float* d_weight = to_device(weight, (size_t)hidden * 4);
    float* d_bias = to_device(bias, (size_t)hidden * 4);
    float* d_grad_updated = to_device(grad_updated, n * 4);
    float* d_grad_normalized = to_device(grad_normalized, n * 4);
    float* d_updated = device_buffer(n * 4);
    float* d_normalized = device_buffer(n * 4);
    float* d_mean = device_buffer((size_t)rows * 4);
    float* d_rstd = device_buffer((size_t)rows * 4);
    uint32_t* d_mask = device_buffer(words * 4);
    float* d_grad_x = device_buffer(n * 4);
    void* d_grad_branch = device_buffer(n * 2);
    float* d_grad_weight = device_buffer((size_t)hidden * 4);
    float* d_grad_bias = device_buffer((size_t)hidden * 4);
    const size_t workspace_bytes = rln_backward_workspace_bytes(rows, hidden, deterministic);
    void* workspace = workspace_bytes ? device_buffer(workspace_bytes) : NULL;

    rln_philox_t philox = {0};
    philox.seed = (uint64_t)header[3];
    philox.offset = (uint64_t)header[4];
    philox.threads = header[2];

    /* The forward zeroes the parameter sums the backward accumulates into. */
    CHECK_RLN(rln_forward(d_x, d_branch, RLN_DTYPE_F16, d_weight, d_bias, d_updated,
                          d_normalized, RLN_DTYPE_F32, d_mean, d_rstd, d_mask, d_grad_weight,
                          d_grad_bias, rows, hidden, scalars[0], scalars[1], 1, &philox,
                          stream));
    CHECK_RLN(rln_backward(d_grad_updated, d_grad_normalized, RLN_DTYPE_F32, d_updated, d_weight,
                           d_mean, d_rstd, d_mask, d_grad_x, d_grad_branch, RLN_DTYPE_F16,
                           d_grad_weight, d_grad_bias, rows, hidden, scalars[0], 1,
                           deterministic, 1, workspace, workspace_bytes, stream));
    CHECK_HIP(hipStreamSynchronize(stream));

    FILE* out = fopen(argv[2], "wb");
    if (out == NULL) {
        return 2;
    }
    write_back(out, d_updated, n * 4);
    write_back(out, d_normalized, n * 4);
    write_back(out, d_mean, (size_t)rows * 4);
    write_back(out, d_rstd, (size_t)rows * 4);
    write_back(out, d_mask, words * 4);
    write_back(out, d_grad_x, n * 4);
    write_back(out, d_grad_branch, n * 2);
    write_back(out, d_grad_weight, (size_t)hidden * 4);
    write_back(out, d_grad_bias, (size_t)hidden * 4);
    fclose(out);
    printf("rln_host: %s rows=%lld hidden=%lld threads=%lld ok\n", rln_version(),
           (long long)rows, (long long)hidden, (long long)header[2]);
    return 0;
}
