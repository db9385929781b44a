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
 *   device_from_c IN OUT vmm
 * does the same with every device array in HIP virtual memory: an address
 * range reserved with hipMemAddressReserve, backed by hipMemCreate and mapped
 * with hipMemMap / hipMemSetAccess (the kind of memory a caching allocator
 * with expandable segments hands out).  Exit status 30 when the device does
 * not support it.
 */
#include <hip/hip_runtime_api.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

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

/* One device array: hipMalloc, or a mapping of HIP virtual memory. */
typedef struct {
    void* ptr;
    size_t mapped;                          /* bytes mapped; 0 for hipMalloc */
    hipMemGenericAllocationHandle_t handle;
} dev_array;

static hipError_t dev_alloc(dev_array* a, size_t bytes, int vmm)
{
    a->ptr = NULL;
    a->mapped = 0;
    if (!vmm) return hipMalloc(&a->ptr, bytes);
    hipMemAllocationProp prop;
    memset(&prop, 0, sizeof(prop));
    prop.type = hipMemAllocationTypePinned;
    prop.location.type = hipMemLocationTypeDevice;
    prop.location.id = 0;
    size_t gran = 0;
    hipError_t e = hipMemGetAllocationGranularity(&gran, &prop, hipMemAllocationGranularityMinimum);
    if (e != hipSuccess) return e;
    const size_t size = (bytes + gran - 1) / gran * gran;
    e = hipMemAddressReserve(&a->ptr, size, 0, NULL, 0);
    if (e != hipSuccess) return e;
    e = hipMemCreate(&a->handle, size, &prop, 0);
    if (e != hipSuccess) return e;
    e = hipMemMap(a->ptr, size, 0, a->handle, 0);
    if (e != hipSuccess) return e;
    hipMemAccessDesc desc;
    memset(&desc, 0, sizeof(desc));
    desc.location.type = hipMemLocationTypeDevice;
    desc.location.id = 0;
    desc.flags = hipMemAccessFlagsProtReadWrite;
    e = hipMemSetAccess(a->ptr, size, &desc, 1);
    if (e == hipSuccess) a->mapped = size;
    return e;
}

static hipError_t dev_free(dev_array* a)
{
    if (!a->mapped) return hipFree(a->ptr);
    hipError_t e = hipMemUnmap(a->ptr, a->mapped);
    if (e == hipSuccess) e = hipMemRelease(a->handle);
    if (e == hipSuccess) e = hipMemAddressFree(a->ptr, a->mapped);
    return e;
}

int main(int argc, char** argv)
{
    if (argc != 3 && !(argc == 4 && strcmp(argv[3], "vmm") == 0)) return 2;
    const int vmm = argc == 4;
    if (vmm) {
        int supported = 0;
        CHECK_HIP(hipDeviceGetAttribute(&supported, hipDeviceAttributeVirtualMemoryManagementSupported, 0));
        if (!supported) return 30;
    }
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
    const uint64_t ws_bytes = la_grad_sqnorm_workspace(n);
    dev_array arr[9];
    const size_t sizes[9] = {n * 4, n * 2, n * 4, n * 4, n * 2, ws_bytes, 8, 4, 4};
    for (int i = 0; i < 9; ++i) CHECK_HIP(dev_alloc(&arr[i], sizes[i], vmm));
    void *dp = arr[0].ptr, *dg = arr[1].ptr, *dm = arr[2].ptr, *dv = arr[3].ptr, *dout = arr[4].ptr;
    void *dws = arr[5].ptr, *dsq = arr[6].ptr, *dcoef = arr[7].ptr, *dnorm = arr[8].ptr;
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
    for (int i = 0; i < 9; ++i) CHECK_HIP(dev_free(&arr[i]));
    CHECK_HIP(hipStreamDestroy(st));
    free(p);
    free(g);
    free(m);
    free(v);
    free(out);
    printf("device_from_c: n=%llu, %s arrays, done\n", (unsigned long long)n, vmm ? "virtual-memory" : "hipMalloc");
    return 0;
}
