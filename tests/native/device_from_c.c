/*
 * A plain C11 program that runs the LayerAdam step on the GPU through
 * include/layer_adam.h alone (HIP runtime API for memory, no torch):
 *   device_from_c IN OUT
 * IN : uint64 n, then p[n] float, g[n] bf16 bits, m[n] float, v[n] float.
 * It computes the grad norm and clip coefficient (max norm 0.5) with
 * la_grad_norm_clip, then runs three la_adam_update steps (AdamW, lr 1e-3,
 * betas 0.9/0.999, eps 1e-8, wd 0.01) with that coefficient and the bf16
 * copy, on one stream of its own.
 * OUT: float coef, float norm, then p[n], m[n], v[n] float, out[n] bf16 bits.
 */
#include <hip/hip_runtime_api.h>
#include <stdio.h>
#include <stdlib.h>

#include "layer_adam.h"

#define CHECK_HIP(x)                                                        \
    do {                                                                    \
        hipError_t e_ = (x);                                                \
        if (e_ != hipSuccess) {                                             \
            fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_)); \
            return 20;                                                      \
        }                                                                   \
    } while (0)
#define CHECK_LA(x)                                                      \
    do {                                                                 \
        int r_ = (x);                                                    \
        if (r_ != LA_OK) {                                               \
            fprintf(stderr, "%s failed: %s\n", #x, la_strerror(r_));     \
            return 21;                                                   \
        }                                                                \
    } while (0)

static int read_all(FILE* f, void* dst, size_t bytes) { return fread(dst, 1, bytes, f) == bytes; }

int main(int argc, char** argv)
{
    if (argc != 3) return 2;
    FILE* in = fopen(argv[1], "rb");
    if (!in) return 3;
    uint64_t n = 0;
    if (!read_all(in, &n, sizeof(n)) || n == 0 || n > (1u << 26)) return 4;
    float* p = malloc(n * 4);
    uint16_t* g = malloc(n * 2);
    float* m = malloc(n * 4);
    float* v = malloc(n * 4);
    uint16_t* out = malloc(n * 2);
    if (!p || !g || !m || !v || !out) return 5;
    if (!read_all(in, p, n * 4) || !read_all(in, g, n * 2) || !read_all(in, m, n * 4) || !read_all(in, v, n * 4))
        return 6;
    fclose(in);

    hipStream_t st;
    CHECK_HIP(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    void *dp, *dg, *dm, *dv, *dout, *dws, *dsq, *dcoef, *dnorm;
    const uint64_t ws_bytes = la_grad_sqnorm_workspace(n);
    CHECK_HIP(hipMalloc(&dp, n * 4));
    CHECK_HIP(hipMalloc(&dg, n * 2));
    CHECK_HIP(hipMalloc(&dm, n * 4));
    CHECK_HIP(hipMalloc(&dv, n * 4));
    CHECK_HIP(hipMalloc(&dout, n * 2));
    CHECK_HIP(hipMalloc(&dws, ws_bytes));
    CHECK_HIP(hipMalloc(&dsq, 8));
    CHECK_HIP(hipMalloc(&dcoef, 4));
    CHECK_HIP(hipMalloc(&dnorm, 4));
    CHECK_HIP(hipMemcpy(dp, p, n * 4, hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(dg, g, n * 2, hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(dm, m, n * 4, hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(dv, v, n * 4, hipMemcpyHostToDevice));

    CHECK_LA(la_create(7070, 1e-3f, 0.9f, 0.999f, 1e-8f, 0.01f, 1, 0));
    CHECK_LA(la_grad_norm_clip(LA_BF16, dg, n, dws, ws_bytes, (double*)dsq, 0, 0.5f, (float*)dcoef, (float*)dnorm,
                               (la_stream_t)st));
    for (uint64_t step = 1; step <= 3; ++step)
        CHECK_LA(la_adam_update(7070, step, 1e-3f, 0.9f, 0.999f, 1e-8f, 0.01f, 1, LA_F32, dp, LA_BF16, dg, LA_F32,
                                dm, dv, n, (uint16_t*)dout, (const float*)dcoef, (la_stream_t)st));
    CHECK_HIP(hipStreamSynchronize(st));
    CHECK_LA(la_destroy(7070));

    float coef = 0, norm = 0;
    CHECK_HIP(hipMemcpy(&coef, dcoef, 4, hipMemcpyDeviceToHost));
    CHECK_HIP(hipMemcpy(&norm, dnorm, 4, hipMemcpyDeviceToHost));
    CHECK_HIP(hipMemcpy(p, dp, n * 4, hipMemcpyDeviceToHost));
    CHECK_HIP(hipMemcpy(m, dm, n * 4, hipMemcpyDeviceToHost));
    CHECK_HIP(hipMemcpy(v, dv, n * 4, hipMemcpyDeviceToHost));
    CHECK_HIP(hipMemcpy(out, dout, n * 2, hipMemcpyDeviceToHost));
    FILE* o = fopen(argv[2], "wb");
    if (!o) return 7;
    int ok = fwrite(&coef, 4, 1, o) == 1 && fwrite(&norm, 4, 1, o) == 1 && fwrite(p, 4, n, o) == n &&
             fwrite(m, 4, n, o) == n && fwrite(v, 4, n, o) == n && fwrite(out, 2, n, o) == n;
    fclose(o);
    if (!ok) return 8;
    void* bufs[] = {dp, dg, dm, dv, dout, dws, dsq, dcoef, dnorm};
    for (unsigned i = 0; i < sizeof(bufs) / sizeof(bufs[0]); ++i) CHECK_HIP(hipFree(bufs[i]));
    CHECK_HIP(hipStreamDestroy(st));
    free(p);
    free(g);
    free(m);
    free(v);
    free(out);
    printf("device_from_c: n=%llu done\n", (unsigned long long)n);
    return 0;
}
