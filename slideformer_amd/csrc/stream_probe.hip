// slideformer_amd: memory-ceiling probes of the update kernel (measurement only).
//
// Built into its own library, libslideformer_amd_probe.so, which only
// `bench.py --update-ceiling` loads; nothing of the product calls it.
//
// Each probe kernel keeps the update kernel's memory side for the hot triple
// (fp32 p/m/v, bf16 g, bf16 copy) exactly: one wave per workgroup, one run of
// 256 elements per wave in a one-shot grid, one raw buffer descriptor per
// stream per wave in scalar registers, the same access widths and cache-policy
// bits (wave_io.h), s_setprio 3 while the loads issue, and the same dynamic
// LDS reservation that caps resident waves per CU (passed per launch).  Only
// the arithmetic between the loads and the stores differs:
//   LA_PROBE_COPY   loads p, g, m, v; stores p, m, v unchanged and the bf16
//                   copy of p: the update's 28 B/param with no AdamW math;
//   LA_PROBE_READ   loads p, g, m, v and stores nothing: 14 B/param;
//   LA_PROBE_WRITE  stores p, m, v and the bf16 copy, values made from the
//                   element index, loads nothing: 14 B/param.
// An empty asm takes every loaded register as an input, so each load is
// issued and waited for although nothing else uses its value.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "wave_io.h"

#define LA_PROBE_COPY 0
#define LA_PROBE_READ 1
#define LA_PROBE_WRITE 2

namespace {

struct ProbeArgs {
    float* p;
    const uint16_t* g;
    float* m;
    float* v;
    uint16_t* out;
    uint64_t nvec;  // groups of 4 elements
};

template <int MODE>
__global__ __launch_bounds__(64) void la_probe_kernel(ProbeArgs a)
{
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t w = wave_uniform((static_cast<uint64_t>(blockIdx.x) * 64 + threadIdx.x) >> 6);
    if (w * 64 >= a.nvec) return;
    const uint64_t left = a.nvec - w * 64;
    const uint32_t nel = (left < 64 ? static_cast<uint32_t>(left) : 64u) * kVec;
    const uint64_t e0 = w * 64 * kVec;
    const rsrc_t rg = WaveIo<bf16_t>::rsrc(a.g, e0, nel);
    const rsrc_t rp = WaveIo<float>::rsrc(a.p, e0, nel);
    const rsrc_t rm = WaveIo<float>::rsrc(a.m, e0, nel);
    const rsrc_t rv = WaveIo<float>::rsrc(a.v, e0, nel);
    float p[kVec], g[kVec], m[kVec], v[kVec];
    if constexpr (MODE != LA_PROBE_WRITE) {
#if LA_SETPRIO
        __builtin_amdgcn_s_setprio(3);
#endif
        WaveIo<bf16_t>::load4(rg, lane, g);
        WaveIo<float>::load4(rp, lane, p);
        WaveIo<float>::load4(rm, lane, m);
        WaveIo<float>::load4(rv, lane, v);
#if LA_SETPRIO
        __builtin_amdgcn_s_setprio(0);
#endif
#pragma unroll
        for (int j = 0; j < kVec; ++j) asm volatile("" ::"v"(g[j]), "v"(p[j]), "v"(m[j]), "v"(v[j]));
    } else {
#pragma unroll
        for (int j = 0; j < kVec; ++j) {
            const float x = static_cast<float>(static_cast<uint32_t>(e0) + lane * kVec + j);
            p[j] = x;
            m[j] = x * 0.5f;
            v[j] = x * 0.25f;
        }
    }
    if constexpr (MODE != LA_PROBE_READ) {
        WaveIo<float>::store4(rp, lane, p);
        WaveIo<float>::store4(rm, lane, m);
        WaveIo<float>::store4(rv, lane, v);
        WaveIo<bf16_t>::store4(WaveIo<bf16_t>::rsrc(a.out, e0, nel), lane, p);
    }
}

}  // namespace

extern "C" {

// One launch of probe `mode` over n elements (a multiple of 4; every pointer
// 16-byte aligned) with `lds_bytes` of dynamic LDS reserved per workgroup, on
// `stream`.  Returns 0, -22 for bad arguments, or a hipError_t.
int la_probe_stream(int mode, float* p, const uint16_t* g, float* m, float* v, uint16_t* out, uint64_t n,
                    uint32_t lds_bytes, void* stream)
{
    if (!p || !g || !m || !v || !out || n % kVec != 0 || n == 0) return -22;
    const uintptr_t ptrs[5] = {reinterpret_cast<uintptr_t>(p), reinterpret_cast<uintptr_t>(g),
                               reinterpret_cast<uintptr_t>(m), reinterpret_cast<uintptr_t>(v),
                               reinterpret_cast<uintptr_t>(out)};
    for (uintptr_t q : ptrs)
        if (q % 16) return -22;
    ProbeArgs a{p, g, m, v, out, n / kVec};
    const uint64_t waves = (a.nvec + 63) / 64;
    if (waves > 0xffffffffull / 64 || lds_bytes > 65536) return -22;
    void (*k)(ProbeArgs) = mode == LA_PROBE_COPY ? la_probe_kernel<LA_PROBE_COPY>
                         : mode == LA_PROBE_READ ? la_probe_kernel<LA_PROBE_READ>
                         : mode == LA_PROBE_WRITE ? la_probe_kernel<LA_PROBE_WRITE> : nullptr;
    if (!k) return -22;
    void* argv[1] = {&a};
    const hipError_t e = hipLaunchKernel(reinterpret_cast<const void*>(k), dim3(static_cast<uint32_t>(waves)),
                                         dim3(64), argv, lds_bytes, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? 0 : static_cast<int>(e);
}

}  // extern "C"
