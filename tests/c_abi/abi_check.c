/*
 * abi_check.c -- a plain C99 caller of include/acfun/acfun.h linked against
 * libacfun_amd.so, as a user of the reference's C API would build it.
 *
 *   abi_check nogpu   : no device present: entry points must fail loudly
 *                       (backend 0, an error string, outputs left untouched)
 *   abi_check gpu     : one GEMM (integer-valued operands, exact in fp32) and
 *                       one fused conv+ReLU (checked against a double loop),
 *                       through the host-pointer API; prints "abi ok".
 * Exit status 0 on success.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "acfun/acfun.h"

static int fail(const char* what) {
    fprintf(stderr, "abi_check: %s (last error: %s)\n", what, acfun_last_error());
    return 1;
}

static int check_nogpu(void) {
    float a[16], c[16];
    for (int i = 0; i < 16; ++i) { a[i] = 1.0f; c[i] = 7.0f; }
    if (acfun_backend() != 0) return fail("backend should be 0 without a device");
    if (strcmp(acfun_backend_name(), "none") != 0) return fail("backend name");
    acfun_gemm(4, 4, 4, a, a, c);
    for (int i = 0; i < 16; ++i)
        if (c[i] != 7.0f) return fail("acfun_gemm wrote without a device");
    if (acfun_last_error()[0] == '\0') return fail("no error string");
    if (acfun_model_load("/nonexistent.acfun") != NULL) return fail("model load");
    puts("abi ok (no device)");
    return 0;
}

static int check_gpu(void) {
    enum { M = 70, N = 52, K = 44 };
    float* A = malloc(sizeof(float) * M * K);
    float* B = malloc(sizeof(float) * K * N);
    float* C = malloc(sizeof(float) * M * N);
    if (!A || !B || !C) return fail("malloc");
    if (acfun_backend() != 4) return fail("no gfx950 device");
    for (int i = 0; i < M * K; ++i) A[i] = (float)(i % 7 - 3);
    for (int i = 0; i < K * N; ++i) B[i] = (float)(i % 5 - 2);
    acfun_gemm(M, N, K, A, B, C);
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j) {
            long s = 0;
            for (int k = 0; k < K; ++k) s += (long)A[i * K + k] * (long)B[k * N + j];
            if (C[i * N + j] != (float)s) return fail("acfun_gemm result");
        }
    /* 3x3/s1/p1 conv + ReLU, 2 x 9 x 11 x 8 -> 12 (the Winograd F(2,3) route) */
    enum { Nn = 2, H = 9, W = 11, Ci = 8, Co = 12 };
    float* x = malloc(sizeof(float) * Nn * H * W * Ci);
    float* w = malloc(sizeof(float) * 9 * Ci * Co);
    float b[Co];
    float* y = malloc(sizeof(float) * Nn * H * W * Co);
    if (!x || !w || !y) return fail("malloc");
    for (int i = 0; i < Nn * H * W * Ci; ++i) x[i] = (float)((i * 37) % 101) / 101.0f - 0.5f;
    for (int i = 0; i < 9 * Ci * Co; ++i) w[i] = (float)((i * 53) % 89) / 89.0f - 0.5f;
    for (int j = 0; j < Co; ++j) b[j] = 0.01f * (float)(j - 6);
    acfun_conv2d_relu(x, Nn, H, W, Ci, w, b, 3, 3, Co, 1, 1, y);
    double maxd = 0.0, maxr = 0.0;
    for (int n = 0; n < Nn; ++n)
        for (int oh = 0; oh < H; ++oh)
            for (int ow = 0; ow < W; ++ow)
                for (int o = 0; o < Co; ++o) {
                    double s = b[o];
                    for (int kh = 0; kh < 3; ++kh)
                        for (int kw = 0; kw < 3; ++kw) {
                            int ih = oh - 1 + kh, iw = ow - 1 + kw;
                            if (ih < 0 || ih >= H || iw < 0 || iw >= W) continue;
                            for (int c = 0; c < Ci; ++c)
                                s += (double)x[((n * H + ih) * W + iw) * Ci + c] *
                                     (double)w[((kh * 3 + kw) * Ci + c) * Co + o];
                        }
                    if (s < 0) s = 0;
                    double d = fabs(s - y[((n * H + oh) * W + ow) * Co + o]);
                    if (d > maxd) maxd = d;
                    if (fabs(s) > maxr) maxr = fabs(s);
                }
    if (!(maxd <= 1e-3 * maxr)) return fail("acfun_conv2d_relu result");
    free(A); free(B); free(C); free(x); free(w); free(y);
    printf("abi ok (%s): gemm exact, conv2d_relu rel err %.2e\n", acfun_backend_name(),
           maxd / maxr);
    return 0;
}

int main(int argc, char** argv) {
    if (argc > 1 && strcmp(argv[1], "gpu") == 0) return check_gpu();
    return check_nogpu();
}
