/*
 * Drives the C ABI's argument validation (include/rln.h) under the host-side
 * address and undefined-behaviour sanitizers (test infrastructure,
 * tests/test_sanitize_host.py). Every call below is rejected, or is a pure
 * size / metadata query, before the library touches a device: the checks
 * run on a CPU-only machine. Pointers are non-null placeholders that
 * validation must never dereference.
 *
 * Prints "ok" and exits 0 when every call returns the expected status and
 * message; a sanitizer report aborts the run with a non-zero status.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "rln.h"

static int failures = 0;

static void expect(int status, int expected, const char* message, const char* what) {
    const char* error = rln_last_error();
    if (status != expected || error == NULL || strstr(error, message) == NULL) {
        fprintf(stderr, "%s: status %d (expected %d), message \"%s\" (expected \"%s\")\n", what,
                status, expected, error ? error : "(null)", message);
        ++failures;
    }
}

static void check(int condition, const char* what) {
    if (!condition) {
        fprintf(stderr, "%s: failed\n", what);
        ++failures;
    }
}

#define FAKE ((void*)(uintptr_t)(1u << 20))

struct forward_args {
    const float* x;
    const void* branch;
    int branch_dtype;
    const float* weight;
    const float* bias;
    float* updated;
    void* normalized;
    int normalized_dtype;
    float* mean;
    float* rstd;
    uint32_t* mask;
    float* zero_weight;
    float* zero_bias;
    int64_t rows;
    int64_t hidden;
    double dropout_p;
    double eps;
    int training;
    const rln_philox_t* philox;
};

static int call_forward(struct forward_args a) {
    return rln_forward(a.x, a.branch, a.branch_dtype, a.weight, a.bias, a.updated, a.normalized,
                       a.normalized_dtype, a.mean, a.rstd, a.mask, a.zero_weight, a.zero_bias,
                       a.rows, a.hidden, a.dropout_p, a.eps, a.training, a.philox, NULL);
}

static struct forward_args forward_defaults(const rln_philox_t* philox) {
    struct forward_args a = {FAKE, FAKE, RLN_DTYPE_F16, FAKE, FAKE, FAKE, FAKE, RLN_DTYPE_F32,
                             FAKE, FAKE, FAKE, NULL, NULL, 4, 768, 0.1, 1e-5, 1, philox};
    return a;
}

struct backward_args {
    const float* grad_updated;
    const void* grad_normalized;
    const float* updated;
    const float* weight;
    const float* mean;
    const float* rstd;
    const uint32_t* mask;
    float* grad_x;
    void* grad_branch;
    int branch_dtype;
    float* grad_weight;
    float* grad_bias;
    int64_t rows;
    int64_t hidden;
    double dropout_p;
    int training;
    int deterministic;
    void* workspace;
    size_t workspace_bytes;
};

static int call_backward(struct backward_args a, int noalloc) {
    if (noalloc) {
        return rln_backward_noalloc(a.grad_updated, a.grad_normalized, RLN_DTYPE_F32, a.updated,
                                    a.weight, a.mean, a.rstd, a.mask, a.grad_x, a.grad_branch,
                                    a.branch_dtype, a.grad_weight, a.grad_bias, a.rows, a.hidden,
                                    a.dropout_p, a.training, a.deterministic, 0, NULL);
    }
    return rln_backward(a.grad_updated, a.grad_normalized, RLN_DTYPE_F32, a.updated, a.weight,
                        a.mean, a.rstd, a.mask, a.grad_x, a.grad_branch, a.branch_dtype,
                        a.grad_weight, a.grad_bias, a.rows, a.hidden, a.dropout_p, a.training,
                        a.deterministic, 0, a.workspace, a.workspace_bytes, NULL);
}

static struct backward_args backward_defaults(void) {
    struct backward_args a = {FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                              RLN_DTYPE_F16, FAKE, FAKE, 4, 768, 0.1, 1, 1, NULL, 0};
    return a;
}

int main(void) {
    rln_philox_t philox = {1, 0, NULL, NULL, 0};
    struct forward_args f;

    f = forward_defaults(&philox); f.rows = 0;
    expect(call_forward(f), RLN_ERR_INVALID, "empty tensors are unsupported", "forward rows=0");
    f = forward_defaults(&philox); f.hidden = 160;
    expect(call_forward(f), RLN_ERR_UNSUPPORTED, "unsupported native hidden size: 160",
           "forward hidden=160");
    f = forward_defaults(&philox); f.branch_dtype = 7;
    expect(call_forward(f), RLN_ERR_INVALID, "branch must use", "forward branch dtype");
    f = forward_defaults(&philox); f.normalized_dtype = 5;
    expect(call_forward(f), RLN_ERR_INVALID, "normalized must use", "forward normalized dtype");
    f = forward_defaults(&philox); f.dropout_p = 1.0;
    expect(call_forward(f), RLN_ERR_INVALID, "dropout_p must be in [0, 1)", "forward p=1");
    f = forward_defaults(&philox); f.dropout_p = NAN;
    expect(call_forward(f), RLN_ERR_INVALID, "dropout_p must be in [0, 1)", "forward p=nan");
    f = forward_defaults(&philox); f.eps = 0.0;
    expect(call_forward(f), RLN_ERR_INVALID, "eps must be positive", "forward eps=0");
    f = forward_defaults(&philox); f.eps = NAN;
    expect(call_forward(f), RLN_ERR_INVALID, "eps must be positive", "forward eps=nan");
    f = forward_defaults(&philox); f.x = NULL;
    expect(call_forward(f), RLN_ERR_INVALID, "forward tensors must not be null", "forward x=NULL");
    f = forward_defaults(&philox); f.mask = NULL;
    expect(call_forward(f), RLN_ERR_INVALID, "dropout_mask must not be null", "forward mask=NULL");
    f = forward_defaults(NULL);
    expect(call_forward(f), RLN_ERR_INVALID, "philox must not be null", "forward philox=NULL");
    f = forward_defaults(&philox); f.rows = (int64_t)1 << 62;
    expect(call_forward(f), RLN_ERR_INVALID, "overflows", "forward rows overflow");
    f = forward_defaults(&philox); f.rows = INT64_MAX;
    expect(call_forward(f), RLN_ERR_INVALID, "overflows", "forward rows=INT64_MAX");
    f = forward_defaults(&philox); f.hidden = INT64_MAX;
    expect(call_forward(f), RLN_ERR_UNSUPPORTED, "unsupported native hidden size",
           "forward hidden=INT64_MAX");
    f = forward_defaults(&philox); f.zero_weight = FAKE;
    expect(call_forward(f), RLN_ERR_INVALID, "both be given or both be null",
           "forward zero_grad_weight alone");
    rln_philox_t narrow = {1, 0, NULL, NULL, 64};
    f = forward_defaults(&narrow);
    expect(call_forward(f), RLN_ERR_INVALID, "threads must be 0, 128, 192 or 256",
           "forward threads=64");
    rln_philox_t reference = {1, 0, NULL, NULL, 128};
    f = forward_defaults(&reference); f.hidden = 1600;
    expect(call_forward(f), RLN_ERR_UNSUPPORTED, "reference's dropout stream exists",
           "forward reference stream at 1600");
    rln_philox_t odd = {1, 6, NULL, NULL, 128};
    f = forward_defaults(&odd);
    expect(call_forward(f), RLN_ERR_INVALID, "offset that is a multiple of 4",
           "forward offset 6");

    struct backward_args b;
    for (int noalloc = 0; noalloc < 2; ++noalloc) {
        b = backward_defaults(); b.rows = -1;
        expect(call_backward(b, noalloc), RLN_ERR_INVALID, "empty tensors are unsupported",
               "backward rows=-1");
        b = backward_defaults(); b.hidden = 100;
        expect(call_backward(b, noalloc), RLN_ERR_UNSUPPORTED,
               "unsupported native hidden size: 100", "backward hidden=100");
        b = backward_defaults(); b.updated = NULL;
        expect(call_backward(b, noalloc), RLN_ERR_INVALID, "backward tensors must not be null",
               "backward updated=NULL");
        b = backward_defaults(); b.grad_bias = NULL;
        expect(call_backward(b, noalloc), RLN_ERR_INVALID, "both be given or both be null",
               "backward grad_bias=NULL");
        b = backward_defaults(); b.mask = NULL;
        expect(call_backward(b, noalloc), RLN_ERR_INVALID, "dropout_mask must not be null",
               "backward mask=NULL");
        b = backward_defaults(); b.branch_dtype = -3;
        expect(call_backward(b, noalloc), RLN_ERR_INVALID, "branch must use",
               "backward branch dtype");
        b = backward_defaults(); b.dropout_p = -0.5;
        expect(call_backward(b, noalloc), RLN_ERR_INVALID, "dropout_p", "backward p<0");
    }
    b = backward_defaults();
    expect(call_backward(b, 0), RLN_ERR_INVALID, "workspace too small", "backward no workspace");
    b = backward_defaults(); b.workspace = FAKE; b.workspace_bytes = 16;
    expect(call_backward(b, 0), RLN_ERR_INVALID, "workspace too small",
           "backward workspace 16 bytes");
    b = backward_defaults(); b.workspace = (char*)FAKE + 4; b.workspace_bytes = (size_t)1 << 30;
    expect(call_backward(b, 0), RLN_ERR_INVALID, "16-byte aligned", "backward workspace align");
    b = backward_defaults(); b.rows = 1 << 20; b.hidden = 8192;
    expect(call_backward(b, 1), RLN_ERR_INVALID, "above its", "noalloc partials above scratch");

    check(rln_mask_words(8192, 768) == 8192 * 24, "mask words");
    check(rln_mask_words(0, 768) == 0, "mask words of no rows");
    check(rln_backward_workspace_bytes(8192, 768, 1) == (size_t)256 * 2 * 768 * 4,
          "workspace bytes");
    check(rln_backward_workspace_bytes(8192, 768, 0) == 0, "atomic mode needs no workspace");
    check(rln_philox_increment(768, 128) == 8, "reference increment at 768");
    check(rln_philox_increment(1600, 128) == 0, "no reference stream at 1600");
    check(rln_hidden_supported(768) == 1 && rln_hidden_supported(160) == 0, "hidden supported");
    int count = rln_supported_hidden_sizes(NULL, 0);
    int64_t sizes[256];
    check(count > 6 && count <= 256, "supported hidden size count");
    check(rln_supported_hidden_sizes(sizes, 3) == count, "partial size list keeps its count");
    check(rln_supported_hidden_sizes(sizes, count) == count && sizes[0] == 128,
          "supported sizes start at 128");
    check(strcmp(rln_target_arch(), "gfx950") == 0, "target arch");
    check(rln_version() != NULL && strlen(rln_version()) > 0, "version");

    if (failures != 0) {
        fprintf(stderr, "%d checks failed\n", failures);
        return 1;
    }
    printf("ok\n");
    return 0;
}
