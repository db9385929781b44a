// slideformer_amd: fused LayerAdam step for MI355X (gfx950, wave64).
//
// One pass over a layer's flat buffers reads p, g, m, v and writes p, m, v and
// the bf16 compute copy of p: 28 algorithmic bytes per element for the hot
// triple (fp32 p/m/v, bf16 g).  Nothing here is a contraction, so there is no
// MFMA; the kernel is bound by HBM bandwidth.
//
// Memory layout of a launch: lane L of a wave owns 4 consecutive elements, so
// one wave instruction covers 256 consecutive elements of every stream
// (16-byte fp32 accesses, 8-byte 16-bit accesses, all lane-contiguous).  The
// grid is one-shot (one group of 4 per lane, one wave per workgroup) up to
// 2^26 - 1 workgroups, 2^34 - 256 elements: on gfx950 the vector memory counter covers
// loads and stores alike, so a grid-stride loop would make each trip wait for
// the previous trip's store acknowledgements.
// Loads and stores carry the nontemporal hint (every byte is touched once), and
// the stores are device-scope, so they are written through the L2.
//
// Arithmetic follows the reference CPU Adam op for op (cpu_adam.h:159-192),
// with explicit fmaf() and this file compiled with -ffp-contract=off; fp32
// division and sqrt stay correctly rounded (no fast-math flags), denormals are
// kept.  The last n % 16 elements of a call follow the reference's scalar tail
// (cpu_adam_impl.cpp:46-67) as its GCC build contracts it.
//
// The grad norm is two launches: stage 1 keeps per-lane float64 sums, reduces
// them across the wave64 with DPP and across the 8 waves of a workgroup in
// LDS, and writes one partial per workgroup to the caller's workspace; stage 2
// (one workgroup) folds the partials in a fixed order and, optionally, writes
// the clip coefficient.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <tuple>
#include <type_traits>
#include <unordered_map>
#include <utility>
#include <vector>

#include "../../include/layer_adam.h"
#include "hip_ptr.h"
#include "wave_io.h"

// Update workgroup size.  One wave per workgroup: in a one-shot grid a
// finished wave is replaced at once instead of waiting for its siblings
// (measured on MI355X, C2 layer: 64 -> 6.17 TB/s, 128 -> 6.02, 256 -> 5.94).
#ifndef LA_BLOCK
#define LA_BLOCK 64
#endif
// Grad-norm workgroup size (8 waves; partials are folded in LDS first).
#ifndef LA_NORM_BLOCK
#define LA_NORM_BLOCK 512
#endif
// Upper bound on update workgroups per launch (grid-stride beyond it).  The
// dispatch packet holds the grid size in work-items as a 32-bit number, so
// workgroups x LA_BLOCK must stay below 2^32.
#ifndef LA_MAX_GRID
#define LA_MAX_GRID ((1 << 26) - 1)
#endif
// Upper bound on grad-norm stage-1 workgroups (= partials folded by stage 2).
// Measured on MI355X over a 218M-element bf16 buffer (workgroup size x
// workgroups x groups of 4 per lane per trip): 512 x 256 x 8 reads in
// 62.5-62.7 us (7.0 TB/s, 87 %), 256 x 512 x 8 in 63-64, 256 x 256 x 16 in
// 63, 256 x 1024 x 4 in 67-68, 256 x 2048 x 2 in 70, 256 x 2048 x 4 in 83.
// About 8 waves per CU, each with 4 KB in flight per trip, read best.
#ifndef LA_NORM_MAX_GRID
#define LA_NORM_MAX_GRID 256
#endif
// Groups of 4 each lane of the grad-norm kernel loads per loop trip.
#ifndef LA_NORM_UNROLL
#define LA_NORM_UNROLL 8
#endif
// The grad-norm kernel's loads.  A call that also writes the clip coefficient
// (la_grad_norm_clip) is the last read of these grads before the update that
// uses the coefficient: its loads are plain (no nontemporal hint), so the
// grads it reads stay in the 256 MB memory-side cache (MALL) for that update,
// whose own nontemporal traffic does not displace them.  The grid walks the
// buffer from the top down, so the front of the buffer, which the update's
// first waves read, is the part read last.  Measured on MI355X, C2 layer
// (436 MB of bf16 grads), norm then update, per step: nontemporal ascending
// 0.986 ms (update 0.919), nontemporal descending 0.987 (0.920), plain
// ascending 0.958 (0.886), plain descending 0.957 (0.885); the norm pass
// itself takes ~4 us longer with plain loads.  Loading only the front 160-320
// MiB plain and the rest nontemporal, or folding the partials with one wave
// instead of eight, changed the step by less than 1 us.
// A call that only accumulates (la_grad_sqnorm: one layer of a global norm,
// whose update waits for every other layer's norm) keeps the nontemporal
// hint: there the grads would not stay cached until their update, and the
// plain loads only cost time (whole resident models, 34-48 layers: 219
// instead of 222 Gparams/s with plain loads everywhere).
#ifndef LA_NORM_CLIP_PLAIN
#define LA_NORM_CLIP_PLAIN 1
#endif
#ifndef LA_NORM_DESCENDING
#define LA_NORM_DESCENDING 1
#endif
// Dynamic LDS reserved per update workgroup, unused by the kernel: it caps the
// workgroups (= waves) resident per CU at 160 KiB / (reserved bytes), 12 for
// 13 KiB.  Fewer streams in flight at once keep the HBM row buffers busier.
// Measured on MI355X, C2 layer, (f32, bf16, f32), same box, update kernel:
// 16 waves per CU 0.918 ms, 14 0.918, 13 0.910, 12 0.906, 11 0.909, 10 0.927;
// the same kernel with the wave index left in vector registers (descriptors
// built there, every access in a readfirstlane loop) was best at 16 waves,
// 0.917 ms.  Wave priority and the write-through stores still add 1-3 % on
// top of the cap.
// The best cap differs by triple: bytes per element and conversion work
// differ, and so do the waves needed to hide them.  At the C2 shape, one box,
// reserved 10 / 12 / 13 / 14 / 15 / 16 KiB, two runs each (ms per launch):
// (f32, f32, f32) 0.996 / 0.979 / 0.977 / 0.975 / 0.975 / 0.986, kept 14 KiB;
// (f16, f16, f32) 0.812 / 0.789 / 0.786 / 0.802 / 0.803 / 0.835 and every
// other triple of this layout best at 13 KiB (12 waves).  A previous build,
// with the wave index in vector registers, was best at 16 KiB for
// (f32, f32, f32) and at 10 KiB for (f16, f16, f32).  The all-16-bit triples
// normally run la_adamw16_kernel (own cap below); with LA_WIDE16=0 they take
// this kernel, best there at 8 KiB (bf16) and 10 KiB (f16) on the previous
// build.  LA_UPDATE_LDS_BYTES, when defined, overrides the table for every
// triple.
#ifdef LA_UPDATE_LDS_BYTES
#define LA_UPDATE_LDS_OVERRIDE 1
#else
#define LA_UPDATE_LDS_OVERRIDE 0
#define LA_UPDATE_LDS_BYTES 13312
#endif
static_assert(LA_BLOCK % 64 == 0, "workgroups are whole waves");
static_assert(static_cast<unsigned long long>(LA_MAX_GRID) * LA_BLOCK <= 0xffffffffull,
              "the grid size in work-items must fit the dispatch packet's 32 bits");

namespace {

// ---------------------------------------------------------------------------
// the element update
// ---------------------------------------------------------------------------
struct Coeffs {
    float b1, b2, omb1, omb2, bc2, eps, step_size, w_decay, wd;
    int32_t mode;  // 0 none, 1 L2, 2 decoupled
};

// SIMD body order of the reference, cpu_adam.h:159-192.
__device__ __forceinline__ void adam_body(float& p, float g, float& m, float& v, const Coeffs& k)
{
    if (k.mode == 1) g = __builtin_fmaf(p, k.wd, g);          // :171-173
    m = m * k.b1;                                            // :175
    m = __builtin_fmaf(g, k.omb1, m);                        // :176
    v = v * k.b2;                                            // :177
    const float gg = g * g;                                  // :178
    v = __builtin_fmaf(gg, k.omb2, v);                       // :179
    float d = __builtin_sqrtf(v);                            // :180
    d = __builtin_fmaf(d, k.bc2, k.eps);                     // :181
    const float u = m / d;                                   // :182
    if (k.mode == 2) p = __builtin_fmaf(p, k.w_decay, p);    // :184-186
    p = __builtin_fmaf(u, k.step_size, p);                   // :188
}

// Scalar tail of the reference, cpu_adam_impl.cpp:46-67, as GCC -O3 with an
// FMA ISA contracts it: the m*b1 and v*b2 products are the fused ones.
__device__ __forceinline__ void adam_tail(float& p, float g, float& m, float& v, const Coeffs& k)
{
    if (k.mode == 1) g = __builtin_fmaf(p, k.wd, g);
    const float gm = g * k.omb1;
    m = __builtin_fmaf(m, k.b1, gm);
    float gg = g * g;
    gg = gg * k.omb2;
    v = __builtin_fmaf(v, k.b2, gg);
    float d = __builtin_sqrtf(v);
    d = __builtin_fmaf(d, k.bc2, k.eps);
    const float u = m / d;
    if (k.mode == 2) p = __builtin_fmaf(p, k.w_decay, p);
    p = __builtin_fmaf(u, k.step_size, p);
}

struct StepArgs {
    void* p;
    const void* g;
    void* m;
    void* v;
    uint16_t* out;       // bf16 compute copy, may be null
    const float* coef;   // clip coefficient (device), may be null
    uint64_t n;
    uint64_t head;       // elements before the first aligned group
    uint64_t nvec;       // aligned groups of 4, starting at `head`
    uint64_t tail_start; // n - n % 16: first element of the reference's scalar tail
    Coeffs k;
};

// One wave's run of 64 aligned groups (256 elements) of every stream, run w of
// the call: loads, update, stores.  Each stream is addressed through a raw
// buffer descriptor whose base is the run's first element (scalar registers)
// and whose size covers only the run's valid groups, so the lanes of a partial
// last run need no branch: their loads return 0 and their stores are dropped
// by the hardware range check.
template <typename TP, typename TG, typename TS>
__device__ __forceinline__ void update_run(const StepArgs& a, uint64_t w, uint32_t lane, bool has_coef, float coef)
{
    const uint64_t left = a.nvec - w * 64;
    const uint32_t nel = (left < 64 ? static_cast<uint32_t>(left) : 64u) * kVec;
    const uint64_t e0 = a.head + w * 64 * kVec;
    const rsrc_t rg = WaveIo<TG>::rsrc(a.g, e0, nel);
    const rsrc_t rp = WaveIo<TP>::rsrc(a.p, e0, nel);
    const rsrc_t rm = WaveIo<TS>::rsrc(a.m, e0, nel);
    const rsrc_t rv = WaveIo<TS>::rsrc(a.v, e0, nel);
    float p[kVec], g[kVec], m[kVec], v[kVec];
#if LA_SETPRIO
    __builtin_amdgcn_s_setprio(3);
#endif
    WaveIo<TG>::load4(rg, lane, g);
    WaveIo<TP>::load4(rp, lane, p);
    WaveIo<TS>::load4(rm, lane, m);
    WaveIo<TS>::load4(rv, lane, v);
#if LA_SETPRIO
    __builtin_amdgcn_s_setprio(0);
#endif
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
        const float gj = has_coef ? g[j] * coef : g[j];
        adam_body(p[j], gj, m[j], v[j], a.k);
    }
    WaveIo<TP>::store4(rp, lane, p);
    WaveIo<TS>::store4(rm, lane, m);
    WaveIo<TS>::store4(rv, lane, v);
    if (a.out) WaveIo<bf16_t>::store4(WaveIo<bf16_t>::rsrc(a.out, e0, nel), lane, p);
}

// One element outside the aligned groups; the reference's scalar tail from
// a.tail_start on, its SIMD body order before.
template <typename TP, typename TG, typename TS>
__device__ __forceinline__ void update_one(const StepArgs& a, uint64_t e, bool has_coef, float coef)
{
    float g = Io<TG>::load1(a.g, e);
    if (has_coef) g = g * coef;
    float p = Io<TP>::load1(a.p, e);
    float m = Io<TS>::load1(a.m, e);
    float v = Io<TS>::load1(a.v, e);
    if (e >= a.tail_start) adam_tail(p, g, m, v, a.k);
    else adam_body(p, g, m, v, a.k);
    Io<TP>::store1(a.p, e, p);
    Io<TS>::store1(a.m, e, m);
    Io<TS>::store1(a.v, e, v);
    if (a.out) a.out[e] = static_cast<uint16_t>(f32_to_bf16_bits(p));
}

template <typename TP, typename TG, typename TS>
__global__ __launch_bounds__(LA_BLOCK) void la_adamw_kernel(StepArgs a)
{
    const bool has_coef = a.coef != nullptr;
    const float coef = has_coef ? *a.coef : 1.0f;
    const uint64_t tid = static_cast<uint64_t>(blockIdx.x) * LA_BLOCK + threadIdx.x;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * LA_BLOCK;

    // Wave w owns run w: groups [64w, 64w + 64), 256 lane-contiguous elements
    // per stream.  The grid is one-shot unless n exceeds LA_MAX_GRID runs.
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t nwaves = stride >> 6;
    for (uint64_t w = wave_uniform(tid >> 6); w * 64 < a.nvec; w += nwaves)
        update_run<TP, TG, TS>(a, w, lane, has_coef, coef);

    // Elements outside the aligned groups: [0, head) and [head + 4*nvec, n).
    const uint64_t vec_end = a.head + a.nvec * kVec;
    const uint64_t nscalar = a.head + (a.n - vec_end);
    for (uint64_t s = tid; s < nscalar; s += stride) {
        const uint64_t e = s < a.head ? s : vec_end + (s - a.head);
        update_one<TP, TG, TS>(a, e, has_coef, coef);
    }
}

// All-16-bit triples ((bf16, bf16, bf16), (f16, f16, f16)): every stream, the
// bf16 copy included, has 2-byte elements, so a lane owns 8 consecutive
// elements and moves each stream with one 16-byte access; one wave
// instruction covers 512 elements (1 KiB) of a stream, and a launch needs
// half the waves of the 4-element layout.  The per-element arithmetic and the
// scalar path are the same as la_adamw_kernel's.  `head` and `nvec` of the
// arguments count 8-element groups here.
constexpr int kVec16 = 8;

template <typename Conv> struct WaveIo16x8 {
    __device__ __forceinline__ static rsrc_t rsrc(const void* base, uint64_t e0, uint32_t nel)
    {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(static_cast<const uint16_t*>(base) + e0), 0,
                                                 static_cast<int>(nel * 2), kRsrcFlags);
    }
    __device__ __forceinline__ static void load8(rsrc_t r, uint32_t lane, float (&x)[kVec16])
    {
        const u32x4 u = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(lane * 16), 0, kAux);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            x[2 * k] = Conv::to_f32(w[k] & 0xffffu);
            x[2 * k + 1] = Conv::to_f32(w[k] >> 16);
        }
    }
    __device__ __forceinline__ static void store8(rsrc_t r, uint32_t lane, const float (&x)[kVec16])
    {
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) w[k] = Conv::from_f32x2(x[2 * k], x[2 * k + 1]);
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{w[0], w[1], w[2], w[3]}, r, static_cast<int>(lane * 16), 0,
                                               kAuxSt);
    }
};
template <typename T> struct Conv16;
template <> struct Conv16<bf16_t> { using type = ConvBf16; };
template <> struct Conv16<f16_t> { using type = ConvF16; };

template <typename T16, typename TG16>
__device__ __forceinline__ void update_run16(const StepArgs& a, uint64_t w, uint32_t lane, bool has_coef, float coef)
{
    using IoS = WaveIo16x8<typename Conv16<T16>::type>;
    using IoG = WaveIo16x8<typename Conv16<TG16>::type>;
    const uint64_t left = a.nvec - w * 64;
    const uint32_t nel = (left < 64 ? static_cast<uint32_t>(left) : 64u) * kVec16;
    const uint64_t e0 = a.head + w * 64 * kVec16;
    const rsrc_t rg = IoG::rsrc(a.g, e0, nel);
    const rsrc_t rp = IoS::rsrc(a.p, e0, nel);
    const rsrc_t rm = IoS::rsrc(a.m, e0, nel);
    const rsrc_t rv = IoS::rsrc(a.v, e0, nel);
    float p[kVec16], g[kVec16], m[kVec16], v[kVec16];
#if LA_SETPRIO
    __builtin_amdgcn_s_setprio(3);
#endif
    IoG::load8(rg, lane, g);
    IoS::load8(rp, lane, p);
    IoS::load8(rm, lane, m);
    IoS::load8(rv, lane, v);
#if LA_SETPRIO
    __builtin_amdgcn_s_setprio(0);
#endif
#pragma unroll
    for (int j = 0; j < kVec16; ++j) {
        const float gj = has_coef ? g[j] * coef : g[j];
        adam_body(p[j], gj, m[j], v[j], a.k);
    }
    IoS::store8(rp, lane, p);
    IoS::store8(rm, lane, m);
    IoS::store8(rv, lane, v);
    if (a.out) WaveIo16x8<ConvBf16>::store8(WaveIo16x8<ConvBf16>::rsrc(a.out, e0, nel), lane, p);
}

template <typename TP, typename TG, typename TS>
__global__ __launch_bounds__(LA_BLOCK) void la_adamw16_kernel(StepArgs a)
{
    static_assert(std::is_same<TP, TS>::value && std::is_same<TP, TG>::value, "all-16-bit triples only");
    const bool has_coef = a.coef != nullptr;
    const float coef = has_coef ? *a.coef : 1.0f;
    const uint64_t tid = static_cast<uint64_t>(blockIdx.x) * LA_BLOCK + threadIdx.x;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * LA_BLOCK;
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t nwaves = stride >> 6;
    for (uint64_t w = wave_uniform(tid >> 6); w * 64 < a.nvec; w += nwaves)
        update_run16<TP, TG>(a, w, lane, has_coef, coef);
    const uint64_t vec_end = a.head + a.nvec * kVec16;
    const uint64_t nscalar = a.head + (a.n - vec_end);
    for (uint64_t s = tid; s < nscalar; s += stride) {
        const uint64_t e = s < a.head ? s : vec_end + (s - a.head);
        update_one<TP, TG, TS>(a, e, has_coef, coef);
    }
}

// Several calls of one step in one launch: the tensors of a layer, each its
// own reference adam_update call with its own scalars (the beta-power state
// advances once per call) and its own scalar tail.  Waves [run_begin[s],
// run_begin[s+1]) take the runs of segment s; then one wave per segment takes
// its at most 21 elements outside the aligned groups.  Segments must not
// overlap in memory.
constexpr int kMaxSegs = 16;
constexpr uint64_t kMaxSegScalars = 64;  // one wave's lanes
// Segments of any size go in a batch: with the wave index and the segment
// arguments in scalar registers, a Llama-3.1-8B layer's nine tensors (16-58 Mi
// elements) batched run 1.1-1.7 % faster than separate launches of the big
// ones (step_with_grad_views 840-845 against 851-853 us, step(layer) 911-912
// against 925-929 us, MI355X), also against batches that large at the
// single-call kernel's residency (936 / 848 us).  The kernel has no
// grid-stride loop, one wave per run, so a batch holds at most LA_MAX_GRID / 2
// runs; a segment of more runs than that takes la_adamw_kernel's grid-stride
// launch of its own (above 2^33 elements in the product build; the small-grid
// test build, LA_MAX_GRID 64, takes it from 32 runs).

struct MultiArgs {
    const float* coef;
    uint32_t count;
    uint64_t run_begin[kMaxSegs + 1];
    StepArgs seg[kMaxSegs];
};

template <typename TP, typename TG, typename TS>
__global__ __launch_bounds__(LA_BLOCK) void la_adamw_multi_kernel(MultiArgs a)
{
    const bool has_coef = a.coef != nullptr;
    const float coef = has_coef ? *a.coef : 1.0f;
    const uint64_t w = wave_uniform((static_cast<uint64_t>(blockIdx.x) * LA_BLOCK + threadIdx.x) >> 6);
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t runs = a.run_begin[a.count];
    if (w < runs) {
        uint32_t s = 0;
        while (w >= a.run_begin[s + 1]) ++s;
        update_run<TP, TG, TS>(a.seg[s], w - a.run_begin[s], lane, has_coef, coef);
        return;
    }
    const uint64_t s = w - runs;
    if (s >= a.count) return;
    const StepArgs& sa = a.seg[s];
    const uint64_t vec_end = sa.head + sa.nvec * kVec;
    const uint64_t nscalar = sa.head + (sa.n - vec_end);
    if (lane < nscalar) {
        const uint64_t e = lane < sa.head ? lane : vec_end + (lane - sa.head);
        update_one<TP, TG, TS>(sa, e, has_coef, coef);
    }
}

// ---------------------------------------------------------------------------
// grad norm
// ---------------------------------------------------------------------------

// Move a float64 across lanes with one DPP control on both 32-bit halves.
// Rows disabled by ROW_MASK read 0.0.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ double dpp_f64(double x)
{
    const uint64_t u = __builtin_bit_cast(uint64_t, x);
    const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(u)), CTRL,
                                               ROW_MASK, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(u >> 32)),
                                               CTRL, ROW_MASK, 0xf, false);
    return __builtin_bit_cast(double, (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) |
                                          static_cast<uint32_t>(lo));
}

// wave64 sum; the total lands in lane 63.  Fixed order, so deterministic.
__device__ __forceinline__ double wave_sum_f64(double x)
{
    x += dpp_f64<0xb1>(x);        // quad_perm [1,0,3,2]
    x += dpp_f64<0x4e>(x);        // quad_perm [2,3,0,1]
    x += dpp_f64<0x141>(x);       // row_half_mirror: 8-lane sums
    x += dpp_f64<0x140>(x);       // row_mirror: 16-lane (row) sums
    x += dpp_f64<0x142, 0xa>(x);  // row_bcast15 into rows 1 and 3
    x += dpp_f64<0x143, 0xc>(x);  // row_bcast31 into rows 2 and 3
    return x;
}

// Sum over the workgroup; valid in thread 0.  Ends with every wave past the
// barrier, so it may be called again in the same kernel.
__device__ __forceinline__ double block_sum_f64(double x)
{
    __shared__ double part[LA_NORM_BLOCK / 64];
    x = wave_sum_f64(x);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 63) part[wave] = x;
    __syncthreads();
    double t = 0.0;
    if (threadIdx.x == 0) {
#pragma unroll
        for (int w = 0; w < LA_NORM_BLOCK / 64; ++w) t += part[w];
    }
    __syncthreads();
    return t;
}

// torch.nn.utils.clip_grad_norm_: coef = min(1, max_norm / (norm + 1e-6)) in fp32.
__device__ __forceinline__ void write_clip(double sq, float max_norm, float* coef, float* norm_out)
{
    const float norm = static_cast<float>(__builtin_sqrt(sq));
    const float c = max_norm / (norm + 1e-6f);
    *coef = (c < 1.0f || c != c) ? c : 1.0f;
    if (norm_out) *norm_out = norm;
}

struct NormArgs {
    const void* g;
    uint64_t n, head, nvec;
    double* partials;     // one slot per stage-1 workgroup
    double* sqnorm;
    int32_t accumulate;
    float max_norm;
    float* coef;          // may be null: then only *sqnorm is written
    float* norm_out;      // may be null
};

// One buffer's share of stage 1 for thread `tid` of `stride`: its aligned
// groups of 4, walked from the top of the buffer down, then its scalar head
// and remainder, added into `acc` in a fixed order.
template <typename TG, bool NT>
__device__ __forceinline__ void sqnorm_buffer(const void* g, uint64_t n, uint64_t head, uint64_t nvec, uint64_t tid,
                                              uint64_t stride, double& acc)
{
    // aligned group i of the walk -> group index in the buffer
    auto group = [nvec](uint64_t i) { return LA_NORM_DESCENDING ? nvec - 1 - i : i; };
    auto load = [g, head](uint64_t gidx, float (&x)[kVec]) { Io<TG>::template load4<NT>(g, head + gidx * kVec, x); };
    uint64_t gi = tid;
    for (; gi + (LA_NORM_UNROLL - 1) * stride < nvec; gi += LA_NORM_UNROLL * stride) {
        float x[LA_NORM_UNROLL][kVec];
#pragma unroll
        for (int u = 0; u < LA_NORM_UNROLL; ++u) load(group(gi + u * stride), x[u]);
#pragma unroll
        for (int u = 0; u < LA_NORM_UNROLL; ++u)
#pragma unroll
            for (int j = 0; j < kVec; ++j) {
                const double d = static_cast<double>(x[u][j]);
                acc = __builtin_fma(d, d, acc);
            }
    }
    for (; gi < nvec; gi += stride) {
        float x[kVec];
        load(group(gi), x);
#pragma unroll
        for (int j = 0; j < kVec; ++j) {
            const double d = static_cast<double>(x[j]);
            acc = __builtin_fma(d, d, acc);
        }
    }
    const uint64_t vec_end = head + nvec * kVec;
    const uint64_t nscalar = head + (n - vec_end);
    for (uint64_t s = tid; s < nscalar; s += stride) {
        const uint64_t e = s < head ? s : vec_end + (s - head);
        const double d = static_cast<double>(Io<TG>::load1(g, e));
        acc = __builtin_fma(d, d, acc);
    }
}

template <typename TG, bool NT>
__global__ __launch_bounds__(LA_NORM_BLOCK) void la_sqnorm_kernel(NormArgs a)
{
    const uint64_t tid = static_cast<uint64_t>(blockIdx.x) * LA_NORM_BLOCK + threadIdx.x;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * LA_NORM_BLOCK;
    double acc = 0.0;
    sqnorm_buffer<TG, NT>(a.g, a.n, a.head, a.nvec, tid, stride, acc);
    const double t = block_sum_f64(acc);
    if (threadIdx.x == 0) a.partials[blockIdx.x] = t;
}

// Stage 1 over up to LA_NORM_MULTI_MAX buffers of one element type in one
// launch: every thread takes its share of each buffer in turn, so a buffer of
// any size is spread over the whole grid, and the partials hold the sum over
// all of them.
struct NormMultiArgs {
    const void* g[LA_NORM_MULTI_MAX];
    uint64_t n[LA_NORM_MULTI_MAX], head[LA_NORM_MULTI_MAX], nvec[LA_NORM_MULTI_MAX];
    int32_t count;
    double* partials;
};

template <typename TG, bool NT>
__global__ __launch_bounds__(LA_NORM_BLOCK) void la_sqnorm_multi_kernel(NormMultiArgs a)
{
    const uint64_t tid = static_cast<uint64_t>(blockIdx.x) * LA_NORM_BLOCK + threadIdx.x;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * LA_NORM_BLOCK;
    double acc = 0.0;
    for (int b = 0; b < a.count; ++b) sqnorm_buffer<TG, NT>(a.g[b], a.n[b], a.head[b], a.nvec[b], tid, stride, acc);
    const double t = block_sum_f64(acc);
    if (threadIdx.x == 0) a.partials[blockIdx.x] = t;
}

// Stage 2, one workgroup: fold the stage-1 partials in a fixed order.  The
// kernel boundary makes every partial visible: a single-launch "last
// workgroup" fold would need an agent-scope release per workgroup, which on
// gfx950 writes back the whole per-XCD L2 each time.
__global__ __launch_bounds__(LA_NORM_BLOCK) void la_sqnorm_finish(NormArgs a, uint32_t nparts)
{
    double s = 0.0;
    for (uint32_t i = threadIdx.x; i < nparts; i += LA_NORM_BLOCK) s += a.partials[i];
    const double total = block_sum_f64(s);
    if (threadIdx.x == 0) {
        const double sq = a.accumulate ? *a.sqnorm + total : total;
        *a.sqnorm = sq;
        if (a.coef) write_clip(sq, a.max_norm, a.coef, a.norm_out);
    }
}

__global__ void la_clip_coef_kernel(const double* sqnorm, float max_norm, float* coef, float* norm_out)
{
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    write_clip(*sqnorm, max_norm, coef, norm_out);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

// Scalar state of one optimizer id, Adam_Optimizer members cpu_adam.h:91-105.
struct HostState {
    float alpha, betta1, betta2, eps, weight_decay;
    float betta1_t = 1.0f, betta2_t = 1.0f;
    uint64_t step = 0;
    float bias_correction1 = 1.0f, bias_correction2 = 1.0f;
    bool adamw_mode = true;
};

std::mutex g_mu;
std::unordered_map<int, HostState> g_states;

int elem_bytes(int dt) { return dt == LA_F32 ? 4 : 2; }
bool dt_valid(int dt) { return dt == LA_F32 || dt == LA_BF16 || dt == LA_F16; }

// First element index h in [0, vec) at which every pointer is aligned to a
// full group of `vec` elements (4 elements: 16 bytes for fp32, 8 bytes for
// 16-bit types), or -1 when the pointers disagree in phase.
int common_head(const uintptr_t* addr, const int* bytes, int count, int vec = kVec)
{
    for (int h = 0; h < vec; ++h) {
        bool ok = true;
        for (int i = 0; i < count && ok; ++i) {
            const uintptr_t align = static_cast<uintptr_t>(vec * bytes[i]);
            ok = ((addr[i] + static_cast<uintptr_t>(h) * bytes[i]) % align) == 0;
        }
        if (ok) return h;
    }
    return -1;
}

uint32_t grid_for(uint64_t work, uint64_t block, uint64_t cap)
{
    uint64_t blocks = (work + block - 1) / block;
    if (blocks < 1) blocks = 1;
    if (blocks > cap) blocks = cap;
    return static_cast<uint32_t>(blocks);
}

uint32_t norm_grid(uint64_t n)
{
    const uint64_t groups = (n + kVec - 1) / kVec;
    return grid_for((groups + LA_NORM_UNROLL - 1) / LA_NORM_UNROLL, LA_NORM_BLOCK, LA_NORM_MAX_GRID);
}

// workspace: norm_grid(n) doubles of stage-1 partials
uint64_t norm_workspace_bytes(uint64_t n) { return static_cast<uint64_t>(norm_grid(n)) * sizeof(double); }

int hip_rc(hipError_t e) { return e == hipSuccess ? LA_OK : static_cast<int>(e); }

// Whether the kernels may touch `ptr`: device (or managed / unified) memory.
// A host address handed to a kernel faults the GPU: pageable and page-locked
// host memory are both refused (host arrays go through la_pipeline_step).
using la_ptr::device_accessible;

// Launch `kernel` and return the status of this launch itself.  Arguments are
// converted to the kernel's own parameter types and handed over by address;
// unlike a check of hipGetLastError() after the launch, an error left behind
// by an unrelated earlier call cannot be mistaken for a failure here.
template <typename... KArgs, typename... Args>
int launch(void (*kernel)(KArgs...), dim3 grid, dim3 block, uint32_t lds_bytes, hipStream_t stream,
           Args&&... args)
{
    static_assert(sizeof...(KArgs) == sizeof...(Args), "argument count must match the kernel");
    std::tuple<std::decay_t<KArgs>...> held(std::forward<Args>(args)...);
    void* argv[sizeof...(KArgs)];
    std::apply([&argv](auto&... x) {
        int i = 0;
        ((argv[i++] = static_cast<void*>(&x)), ...);
    }, held);
    return hip_rc(hipLaunchKernel(reinterpret_cast<const void*>(kernel), grid, block, argv, lds_bytes, stream));
}

// LDS reserved per update workgroup for one (param, grad, state) triple (see
// LA_UPDATE_LDS_BYTES); 0 = no cap below the register limit.
template <typename TP, typename TG, typename TS> constexpr uint32_t update_lds_bytes()
{
    if (LA_UPDATE_LDS_OVERRIDE) return LA_UPDATE_LDS_BYTES;
    if (std::is_same<TP, bf16_t>::value && std::is_same<TS, bf16_t>::value) return 8192;       // (bf16, bf16, bf16)
    if (std::is_same<TP, f16_t>::value && std::is_same<TS, f16_t>::value) return 10240;       // (f16, f16, f16)
    if (std::is_same<TP, float>::value && std::is_same<TG, float>::value) return 14336;       // (f32, f32, f32)
    return LA_UPDATE_LDS_BYTES;
}

// The all-16-bit path moves twice the bytes per wave, so it wants fewer
// resident waves than the 4-element layout of the same triple.  Measured on
// MI355X, C2 shape, 100 launches, three runs, ms per launch (4-element layout
// at its own best cap / 8-element layout at 10, 11, 12, 13, 14 KiB reserved):
// (bf16, bf16, bf16) 0.571-0.574 / 0.549-0.553, 0.547-0.551, 0.546-0.550,
// 0.550-0.553, 0.560-0.561; (f16, f16, f16) 0.539-0.541 / 0.534-0.536,
// 0.532-0.534, 0.531, 0.524-0.525, 0.524-0.526.  Kept: 12 KiB (13 waves per
// CU) and 13 KiB (12).  LA_UPDATE16_LDS_BYTES, when defined, overrides both;
// LA_WIDE16=0 restores the 4-element layout for these triples.
#ifndef LA_WIDE16
#define LA_WIDE16 1
#endif
template <typename T> constexpr uint32_t update16_lds_bytes()
{
#ifdef LA_UPDATE16_LDS_BYTES
    return LA_UPDATE16_LDS_BYTES;
#else
    return std::is_same<T, bf16_t>::value ? 12288u : 13312u;
#endif
}

// The multi kernel's waves first look up their segment and its arguments, a
// latency that more resident waves hide better: at most 10 KiB (16 waves per
// CU).  Measured on MI355X, a GPT-2 block's twelve tensors in one launch,
// (f32, bf16, f32), step_with_grad_views: 30.4 us at 16 waves, 31.2 at 20,
// 32.1 at 12, 31.3 uncapped.  LA_MULTI_LDS_BYTES, when defined, overrides it
// for every triple.
template <typename TP, typename TG, typename TS> constexpr uint32_t multi_lds_bytes()
{
#ifdef LA_MULTI_LDS_BYTES
    return LA_MULTI_LDS_BYTES;
#else
    return update_lds_bytes<TP, TG, TS>() < 10240u ? update_lds_bytes<TP, TG, TS>() : 10240u;
#endif
}

// Launch of la_adamw_kernel for the 4-element layout of `a`.
template <typename TP, typename TG, typename TS> int launch4(const StepArgs& a, hipStream_t stream)
{
    const uint64_t nscalar = a.head + (a.n - (a.head + a.nvec * kVec));
    // lanes needed: every wave takes one run of 64 groups
    const uint64_t vec_lanes = (a.nvec + 63) / 64 * 64;
    const uint64_t work = vec_lanes > nscalar ? vec_lanes : nscalar;
    return launch(la_adamw_kernel<TP, TG, TS>, dim3(grid_for(work, LA_BLOCK, LA_MAX_GRID)), dim3(LA_BLOCK),
                  update_lds_bytes<TP, TG, TS>(), stream, a);
}

// The all-16-bit path: the call's groups are re-laid out as 8-element groups.
// Pointers that share a 4-element phase but not an 8-element one (16-byte
// alignment) keep the 4-element layout of la_adamw_kernel rather than the
// all-scalar path.
template <typename T> int launch16(const StepArgs& a4, hipStream_t stream)
{
    StepArgs a = a4;
    const uintptr_t addr[5] = {reinterpret_cast<uintptr_t>(a.p), reinterpret_cast<uintptr_t>(a.g),
                               reinterpret_cast<uintptr_t>(a.m), reinterpret_cast<uintptr_t>(a.v),
                               reinterpret_cast<uintptr_t>(a.out)};
    const int bytes[5] = {2, 2, 2, 2, 2};
    const int h = common_head(addr, bytes, a.out ? 5 : 4, kVec16);
    if (h < 0 || static_cast<uint64_t>(h) >= a.tail_start) {
        if (a4.nvec > 0) return launch4<T, T, T>(a4, stream);
        a.head = 0;
        a.nvec = 0;
    } else {
        a.head = static_cast<uint64_t>(h);
        a.nvec = (a.tail_start - a.head) / kVec16;
    }
    const uint64_t nscalar = a.head + (a.n - (a.head + a.nvec * kVec16));
    const uint64_t vec_lanes = (a.nvec + 63) / 64 * 64;
    const uint64_t work = vec_lanes > nscalar ? vec_lanes : nscalar;
    return launch(la_adamw16_kernel<T, T, T>, dim3(grid_for(work, LA_BLOCK, LA_MAX_GRID)), dim3(LA_BLOCK),
                  update16_lds_bytes<T>(), stream, a);
}

template <typename TP, typename TG, typename TS> struct StepLauncher {
    static int run(const StepArgs& a, hipStream_t stream)
    {
        if constexpr (LA_WIDE16 && std::is_same<TP, TG>::value && std::is_same<TP, TS>::value &&
                      !std::is_same<TP, float>::value)
            return launch16<TP>(a, stream);
        return launch4<TP, TG, TS>(a, stream);
    }
};

template <typename TP, typename TG, typename TS> struct MultiLauncher {
    // waves: runs of every segment + one scalar wave per segment
    static int run(const MultiArgs& a, uint64_t waves, hipStream_t stream)
    {
        return launch(la_adamw_multi_kernel<TP, TG, TS>, dim3(static_cast<uint32_t>(waves * 64 / LA_BLOCK)),
                      dim3(LA_BLOCK), multi_lds_bytes<TP, TG, TS>(), stream, a);
    }
};

// The nine (param, grad, state) triples the reference registers,
// cpu_adam_impl.cpp:181-189; nothing else is instantiated.
template <template <typename, typename, typename> class L, typename... Args>
int dispatch_triple(int p, int g, int s, Args&&... args)
{
    if (p == LA_F32 && s == LA_F32) {
        if (g == LA_BF16) return L<float, bf16_t, float>::run(args...);
        if (g == LA_F32) return L<float, float, float>::run(args...);
        if (g == LA_F16) return L<float, f16_t, float>::run(args...);
    } else if (p == LA_BF16) {
        if (g == LA_BF16 && s == LA_F32) return L<bf16_t, bf16_t, float>::run(args...);
        if (g == LA_F32 && s == LA_F32) return L<bf16_t, float, float>::run(args...);
        if (g == LA_BF16 && s == LA_BF16) return L<bf16_t, bf16_t, bf16_t>::run(args...);
    } else if (p == LA_F16) {
        if (g == LA_F16 && s == LA_F32) return L<f16_t, f16_t, float>::run(args...);
        if (g == LA_F32 && s == LA_F32) return L<f16_t, float, float>::run(args...);
        if (g == LA_F16 && s == LA_F16) return L<f16_t, f16_t, f16_t>::run(args...);
    }
    return LA_EDTYPE;
}

// Check the pointers of one call and lay out its elements (everything of
// StepArgs but the coefficients).  n > 0.
int prepare_step(int p_dtype, void* p, int g_dtype, const void* g, int s_dtype, void* m, void* v, uint64_t n,
                 uint16_t* p_bf16_out, const float* clip_coef, StepArgs& a)
{
    if (!p || !g || !m || !v) return LA_EINVAL;
    const uintptr_t addr[5] = {reinterpret_cast<uintptr_t>(p), reinterpret_cast<uintptr_t>(g),
                               reinterpret_cast<uintptr_t>(m), reinterpret_cast<uintptr_t>(v),
                               reinterpret_cast<uintptr_t>(p_bf16_out)};
    const int bytes[5] = {elem_bytes(p_dtype), elem_bytes(g_dtype), elem_bytes(s_dtype), elem_bytes(s_dtype), 2};
    const int count = p_bf16_out ? 5 : 4;
    for (int i = 0; i < count; ++i)
        if (addr[i] % static_cast<uintptr_t>(bytes[i]) != 0) return LA_EINVAL;
    if (clip_coef && (reinterpret_cast<uintptr_t>(clip_coef) & 3u)) return LA_EINVAL;
    for (int i = 0; i < count; ++i)
        if (!device_accessible(reinterpret_cast<const void*>(addr[i]))) return LA_EFAULT;
    if (clip_coef && !device_accessible(clip_coef)) return LA_EFAULT;
    a.p = p;
    a.g = g;
    a.m = m;
    a.v = v;
    a.out = p_bf16_out;
    a.coef = clip_coef;
    a.n = n;
    a.tail_start = n - n % 16;
    const int h = common_head(addr, bytes, count);
    if (h < 0 || static_cast<uint64_t>(h) >= a.tail_start) {
        a.head = 0;
        a.nvec = 0;
    } else {
        a.head = static_cast<uint64_t>(h);
        a.nvec = (a.tail_start - a.head) / kVec;
    }
    return LA_OK;
}

void set_coeffs(const la_scalars_t& sc, Coeffs& k)
{
    k.b1 = sc.beta1;
    k.b2 = sc.beta2;
    k.omb1 = sc.one_minus_beta1;
    k.omb2 = sc.one_minus_beta2;
    k.bc2 = sc.bias_correction2;
    k.eps = sc.eps;
    k.step_size = sc.step_size;
    k.w_decay = sc.w_decay;
    k.wd = sc.weight_decay;
    k.mode = sc.decay_mode;
}

bool triple_registered(int p, int g, int s)
{
    if (p == LA_F32) return s == LA_F32;
    if (p == LA_BF16) return g != LA_F16 && (s == LA_F32 || (s == LA_BF16 && g == LA_BF16));
    return g != LA_BF16 && (s == LA_F32 || (s == LA_F16 && g == LA_F16));
}

void derive_scalars(HostState& s, uint64_t step, float lr, float b1, float b2, float eps, float wd,
                    int bias_correction, la_scalars_t* out)
{
    // IncrementStep, cpu_adam.h:57-76; std::pow(float, size_t) is a double pow.
    if (b1 != s.betta1 || b2 != s.betta2) {
        s.step = step;
        s.betta1 = b1;
        s.betta2 = b2;
        s.betta1_t = static_cast<float>(std::pow(static_cast<double>(s.betta1), static_cast<double>(step)));
        s.betta2_t = static_cast<float>(std::pow(static_cast<double>(s.betta2), static_cast<double>(step)));
    } else {
        s.step++;
        if (s.step != step) {
            s.betta1_t = static_cast<float>(std::pow(static_cast<double>(s.betta1), static_cast<double>(step)));
            s.betta2_t = static_cast<float>(std::pow(static_cast<double>(s.betta2), static_cast<double>(step)));
            s.step = step;
        } else {
            s.betta1_t *= s.betta1;
            s.betta2_t *= s.betta2;
        }
    }
    // update_state, cpu_adam.h:77-89 (float sqrt and float divide).
    s.alpha = lr;
    s.eps = eps;
    s.weight_decay = wd;
    s.bias_correction1 = 1.0f;
    s.bias_correction2 = 1.0f;
    if (bias_correction) {
        s.bias_correction1 = 1.0f - s.betta1_t;
        s.bias_correction2 = 1.0f / std::sqrt(1.0f - s.betta2_t);
    }
    // Step_AVX prologue, cpu_adam.h:131-148.
    out->beta1 = s.betta1;
    out->beta2 = s.betta2;
    out->one_minus_beta1 = 1.0f - s.betta1;
    out->one_minus_beta2 = 1.0f - s.betta2;
    out->bias_correction2 = s.bias_correction2;
    out->eps = s.eps;
    out->step_size = -1.0f * s.alpha / s.bias_correction1;
    out->w_decay = -1.0f * s.alpha * s.weight_decay;
    out->weight_decay = s.weight_decay;
    out->decay_mode = s.weight_decay > 0.0f ? (s.adamw_mode ? 2 : 1) : 0;
    out->beta1_t = s.betta1_t;
    out->beta2_t = s.betta2_t;
    out->bias_correction1 = s.bias_correction1;
    out->step = s.step;
}

int launch_norm(int g_dtype, const void* g, uint64_t n, void* workspace, uint64_t workspace_bytes,
                double* sqnorm, int accumulate, float max_norm, float* coef, float* norm_out, hipStream_t st)
{
    if (!dt_valid(g_dtype)) return LA_EDTYPE;
    if (!sqnorm || !workspace) return LA_EINVAL;
    if ((reinterpret_cast<uintptr_t>(sqnorm) & 7u) || (reinterpret_cast<uintptr_t>(workspace) & 7u)) return LA_EINVAL;
    if (coef && (reinterpret_cast<uintptr_t>(coef) & 3u)) return LA_EINVAL;
    if (norm_out && (reinterpret_cast<uintptr_t>(norm_out) & 3u)) return LA_EINVAL;
    if (n > 0 && !g) return LA_EINVAL;
    const int gb = elem_bytes(g_dtype);
    if (reinterpret_cast<uintptr_t>(g) % static_cast<uintptr_t>(gb)) return LA_EINVAL;
    if (workspace_bytes < norm_workspace_bytes(n)) return LA_EINVAL;
    if ((n > 0 && !device_accessible(g)) || !device_accessible(workspace) || !device_accessible(sqnorm) ||
        (coef && !device_accessible(coef)) || (norm_out && !device_accessible(norm_out)))
        return LA_EFAULT;

    NormArgs a;
    const uint32_t grid = norm_grid(n);
    a.g = g;
    a.n = n;
    a.head = 0;
    a.nvec = 0;
    const uintptr_t addr = reinterpret_cast<uintptr_t>(g);
    const int h = n > 0 ? common_head(&addr, &gb, 1) : -1;
    if (h >= 0 && static_cast<uint64_t>(h) < n) {
        a.head = static_cast<uint64_t>(h);
        a.nvec = (n - a.head) / kVec;
    }
    a.partials = static_cast<double*>(workspace);
    a.sqnorm = sqnorm;
    a.accumulate = accumulate ? 1 : 0;
    a.max_norm = max_norm;
    a.coef = coef;
    a.norm_out = norm_out;
    // plain loads for the read that produces the coefficient, nontemporal otherwise
    const bool nt = !(coef && LA_NORM_CLIP_PLAIN);
    int rc;
    switch (g_dtype) {
    case LA_F32:
        rc = launch(nt ? la_sqnorm_kernel<float, true> : la_sqnorm_kernel<float, false>, dim3(grid),
                    dim3(LA_NORM_BLOCK), 0, st, a);
        break;
    case LA_BF16:
        rc = launch(nt ? la_sqnorm_kernel<bf16_t, true> : la_sqnorm_kernel<bf16_t, false>, dim3(grid),
                    dim3(LA_NORM_BLOCK), 0, st, a);
        break;
    default:
        rc = launch(nt ? la_sqnorm_kernel<f16_t, true> : la_sqnorm_kernel<f16_t, false>, dim3(grid),
                    dim3(LA_NORM_BLOCK), 0, st, a);
        break;
    }
    if (rc != LA_OK) return rc;
    return launch(la_sqnorm_finish, dim3(1), dim3(LA_NORM_BLOCK), 0, st, a, grid);
}

int launch_norm_multi(int g_dtype, const la_grad_buffer_t* bufs, int count, void* workspace,
                      uint64_t workspace_bytes, double* sqnorm, int accumulate, float max_norm, float* coef,
                      float* norm_out, hipStream_t st)
{
    if (!dt_valid(g_dtype)) return LA_EDTYPE;
    if (!bufs || count < 1 || count > LA_NORM_MULTI_MAX || !sqnorm || !workspace) return LA_EINVAL;
    if ((reinterpret_cast<uintptr_t>(sqnorm) & 7u) || (reinterpret_cast<uintptr_t>(workspace) & 7u)) return LA_EINVAL;
    if (coef && (reinterpret_cast<uintptr_t>(coef) & 3u)) return LA_EINVAL;
    if (norm_out && (reinterpret_cast<uintptr_t>(norm_out) & 3u)) return LA_EINVAL;
    const int gb = elem_bytes(g_dtype);
    uint64_t total = 0;
    for (int b = 0; b < count; ++b) {
        const la_grad_buffer_t& q = bufs[b];
        if (q.n > 0 && (!q.g || reinterpret_cast<uintptr_t>(q.g) % static_cast<uintptr_t>(gb))) return LA_EINVAL;
        if (q.n > UINT64_MAX - total) return LA_EINVAL;
        total += q.n;
    }
    if (workspace_bytes < norm_workspace_bytes(total)) return LA_EINVAL;
    if (!device_accessible(workspace) || !device_accessible(sqnorm) || (coef && !device_accessible(coef)) ||
        (norm_out && !device_accessible(norm_out)))
        return LA_EFAULT;
    for (int b = 0; b < count; ++b)
        if (bufs[b].n > 0 && !device_accessible(bufs[b].g)) return LA_EFAULT;

    NormMultiArgs m;
    m.count = count;
    m.partials = static_cast<double*>(workspace);
    for (int b = 0; b < LA_NORM_MULTI_MAX; ++b) {
        m.g[b] = nullptr;
        m.n[b] = m.head[b] = m.nvec[b] = 0;
    }
    for (int b = 0; b < count; ++b) {
        const uint64_t n = bufs[b].n;
        m.g[b] = bufs[b].g;
        m.n[b] = n;
        const uintptr_t addr = reinterpret_cast<uintptr_t>(bufs[b].g);
        const int h = n > 0 ? common_head(&addr, &gb, 1) : -1;
        if (h >= 0 && static_cast<uint64_t>(h) < n) {
            m.head[b] = static_cast<uint64_t>(h);
            m.nvec[b] = (n - m.head[b]) / kVec;
        }
    }
    const uint32_t grid = norm_grid(total);
    // plain loads for the read that produces the coefficient, nontemporal otherwise
    const bool nt = !(coef && LA_NORM_CLIP_PLAIN);
    int rc;
    switch (g_dtype) {
    case LA_F32:
        rc = launch(nt ? la_sqnorm_multi_kernel<float, true> : la_sqnorm_multi_kernel<float, false>, dim3(grid),
                    dim3(LA_NORM_BLOCK), 0, st, m);
        break;
    case LA_BF16:
        rc = launch(nt ? la_sqnorm_multi_kernel<bf16_t, true> : la_sqnorm_multi_kernel<bf16_t, false>, dim3(grid),
                    dim3(LA_NORM_BLOCK), 0, st, m);
        break;
    default:
        rc = launch(nt ? la_sqnorm_multi_kernel<f16_t, true> : la_sqnorm_multi_kernel<f16_t, false>, dim3(grid),
                    dim3(LA_NORM_BLOCK), 0, st, m);
        break;
    }
    if (rc != LA_OK) return rc;
    NormArgs a{};
    a.partials = m.partials;
    a.sqnorm = sqnorm;
    a.accumulate = accumulate ? 1 : 0;
    a.max_norm = max_norm;
    a.coef = coef;
    a.norm_out = norm_out;
    return launch(la_sqnorm_finish, dim3(1), dim3(LA_NORM_BLOCK), 0, st, a, grid);
}

}  // namespace

// Fixed device scratch of la_grad_norm_clip_noalloc: the grad norm's stage-1
// partials (one float64 per stage-1 workgroup), for callers that cannot
// allocate device memory.  Every GPU the library runs on holds its own copy
// until the process ends.  Host code never uses this name as an address: on
// the host it is only a stand-in, and the device address comes from
// hipGetSymbolAddress (scratch_on_current_device below).
static __device__ __align__(256) double scratch[LA_NORM_SCRATCH_PARTIALS];

namespace {

constexpr uint64_t kScratchBytes = static_cast<uint64_t>(LA_NORM_SCRATCH_PARTIALS) * sizeof(double);

// Device ordinals the address table covers; a fixed table, so that not even
// the first call on a device allocates host memory.
constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
double* g_scratch_ptr[kScratchDevices] = {};  // device ordinal -> that device's copy of `scratch`

// The address of `scratch` on device `dev`, which is the current device,
// looked up once per device with that device current.
int scratch_on_current_device(int dev, double** out)
{
    if (dev < 0 || dev >= kScratchDevices) return LA_EINVAL;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_rc(e);
        if (!ptr) return LA_EINVAL;
        g_scratch_ptr[dev] = static_cast<double*>(ptr);
    }
    *out = g_scratch_ptr[dev];
    return LA_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" {

int la_abi_version(void) { return LA_ABI_VERSION; }

const char* la_strerror(int code)
{
    if (code == LA_OK) return "ok";
    if (code == LA_EINVAL) return "invalid argument (null/misaligned pointer, unknown id or bad size)";
    if (code == LA_EDTYPE) return "dtype triple not supported";
    if (code == LA_ENOMEM) return "out of host memory or host threads";
    if (code == LA_ERANGE) return "size beyond the fixed device scratch of a no-allocation entry point";
    if (code == LA_EFAULT) return "a pointer that a kernel would touch is not device memory (host arrays go through la_pipeline_step)";
    if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
    return "unknown error";
}

int la_create(int id, float lr, float beta1, float beta2, float eps, float weight_decay, int adamw_mode,
              int should_log)
try {
    HostState s;
    s.alpha = lr;
    s.betta1 = beta1;
    s.betta2 = beta2;
    s.eps = eps;
    s.weight_decay = weight_decay;
    s.adamw_mode = adamw_mode != 0;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        g_states[id] = s;
    }
    if (should_log) {
        // the reference's creation log (cpu_adam_impl.cpp:108-126), on stderr so
        // that a caller's stdout stays its own
        std::fprintf(stderr, "Adam Optimizer #%d is created with MI355X (gfx950 HIP) arithmetic capability.\n", id);
        std::fprintf(stderr, "Config: alpha=%f, betas=(%f, %f), weight_decay=%f, adam_w=%d\n", lr, beta1, beta2,
                    weight_decay, adamw_mode ? 1 : 0);
    }
    return LA_OK;
} catch (...) {
    return LA_ENOMEM;
}

int la_destroy(int id)
{
    std::lock_guard<std::mutex> lk(g_mu);
    g_states.erase(id);
    return LA_OK;
}

int la_scalars(int id, uint64_t step, float lr, float beta1, float beta2, float eps, float weight_decay,
               int bias_correction, la_scalars_t* out)
{
    if (!out) return LA_EINVAL;
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_states.find(id);
    if (it == g_states.end()) return LA_EINVAL;
    derive_scalars(it->second, step, lr, beta1, beta2, eps, weight_decay, bias_correction, out);
    return LA_OK;
}

int la_adamw_step(const la_scalars_t* sc, int p_dtype, void* p, int g_dtype, const void* g, int s_dtype,
                  void* m, void* v, uint64_t n, uint16_t* p_bf16_out, const float* clip_coef,
                  la_stream_t stream)
{
    if (!sc) return LA_EINVAL;
    if (!dt_valid(p_dtype) || !dt_valid(g_dtype) || !dt_valid(s_dtype)) return LA_EDTYPE;
    if (!triple_registered(p_dtype, g_dtype, s_dtype)) return LA_EDTYPE;
    if (n == 0) return LA_OK;

    StepArgs a;
    const int rc = prepare_step(p_dtype, p, g_dtype, g, s_dtype, m, v, n, p_bf16_out, clip_coef, a);
    if (rc != LA_OK) return rc;
    set_coeffs(*sc, a.k);
    return dispatch_triple<StepLauncher>(p_dtype, g_dtype, s_dtype, a, static_cast<hipStream_t>(stream));
}

int la_adam_update(int id, uint64_t step, float lr, float beta1, float beta2, float eps, float weight_decay,
                   int bias_correction, int p_dtype, void* p, int g_dtype, const void* g, int s_dtype, void* m,
                   void* v, uint64_t n, uint16_t* p_bf16_out, const float* clip_coef, la_stream_t stream)
{
    // ds_adam_step checks the dtype triple only after IncrementStep/update_state
    // (cpu_adam_impl.cpp:241-261), so the state machine advances either way.
    la_scalars_t sc;
    int rc = la_scalars(id, step, lr, beta1, beta2, eps, weight_decay, bias_correction, &sc);
    if (rc != LA_OK) return rc;
    return la_adamw_step(&sc, p_dtype, p, g_dtype, g, s_dtype, m, v, n, p_bf16_out, clip_coef, stream);
}

int la_adam_update_multi(int id, uint64_t step, float lr, float beta1, float beta2, float eps, float weight_decay,
                         int bias_correction, int p_dtype, int g_dtype, int s_dtype, const la_segment_t* segs,
                         int count, const float* clip_coef, la_stream_t stream)
try {
    if (count < 0 || (count > 0 && !segs)) return LA_EINVAL;
    if (clip_coef && (reinterpret_cast<uintptr_t>(clip_coef) & 3u)) return LA_EINVAL;
    const bool registered = dt_valid(p_dtype) && dt_valid(g_dtype) && dt_valid(s_dtype) &&
                            triple_registered(p_dtype, g_dtype, s_dtype);
    std::vector<StepArgs> args(registered ? static_cast<size_t>(count) : 0);
    if (registered) {
        // every pointer is checked before anything changes
        for (int k = 0; k < count; ++k) {
            const la_segment_t& q = segs[k];
            if (q.n == 0) {
                args[k].n = 0;
                continue;
            }
            const int rc = prepare_step(p_dtype, q.p, g_dtype, q.g, s_dtype, q.m, q.v, q.n, q.p_bf16_out,
                                        clip_coef, args[k]);
            if (rc != LA_OK) return rc;
        }
    }
    {
        // the beta-power state advances once per segment, as separate calls would
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_states.find(id);
        if (it == g_states.end()) return LA_EINVAL;
        if (!registered) {
            // the first call of the sequence would advance the state, then fail
            // on the triple (cpu_adam_impl.cpp:241-261)
            la_scalars_t sc;
            if (count > 0) derive_scalars(it->second, step, lr, beta1, beta2, eps, weight_decay, bias_correction, &sc);
            return LA_EDTYPE;
        }
        for (int k = 0; k < count; ++k) {
            la_scalars_t sc;
            derive_scalars(it->second, step, lr, beta1, beta2, eps, weight_decay, bias_correction, &sc);
            set_coeffs(sc, args[k].k);
        }
    }
    const hipStream_t st = static_cast<hipStream_t>(stream);
    MultiArgs batch;
    std::memset(&batch, 0, sizeof(batch));
    batch.coef = clip_coef;
    uint64_t runs = 0;
    auto flush = [&]() -> int {
        if (batch.count == 0) return LA_OK;
        // one wave per run and per segment: the grid must fit the dispatch packet
        // (holds by construction: a batch takes at most LA_MAX_GRID / 2 runs and
        // kMaxSegs segments)
        if (runs + batch.count > static_cast<uint64_t>(LA_MAX_GRID)) return LA_EINVAL;
        batch.run_begin[batch.count] = runs;
        const int rc = dispatch_triple<MultiLauncher>(p_dtype, g_dtype, s_dtype, batch, runs + batch.count, st);
        std::memset(&batch, 0, sizeof(batch));
        batch.coef = clip_coef;
        runs = 0;
        return rc;
    };
    for (int k = 0; k < count; ++k) {
        const StepArgs& a = args[k];
        if (a.n == 0) continue;
        const uint64_t seg_runs = (a.nvec + 63) / 64;
        const uint64_t nscalar = a.head + (a.n - (a.head + a.nvec * kVec));
        if (nscalar > kMaxSegScalars || seg_runs > LA_MAX_GRID / 2) {
            // pointers out of phase (all elements scalar), or more runs than one
            // batch holds: its own launch, which grid-strides
            const int rc = dispatch_triple<StepLauncher>(p_dtype, g_dtype, s_dtype, a, st);
            if (rc != LA_OK) return rc;
            continue;
        }
        if (batch.count == static_cast<uint32_t>(kMaxSegs) || runs + seg_runs > LA_MAX_GRID / 2) {
            const int rc = flush();
            if (rc != LA_OK) return rc;
        }
        batch.run_begin[batch.count] = runs;
        batch.seg[batch.count] = a;
        batch.count++;
        runs += seg_runs;
    }
    return flush();
} catch (...) {
    return LA_ENOMEM;
}

uint64_t la_grad_sqnorm_workspace(uint64_t n) { return norm_workspace_bytes(n); }

int la_grad_sqnorm(int g_dtype, const void* g, uint64_t n, void* workspace, uint64_t workspace_bytes,
                   double* sqnorm, int accumulate, la_stream_t stream)
{
    return launch_norm(g_dtype, g, n, workspace, workspace_bytes, sqnorm, accumulate, 0.0f, nullptr, nullptr,
                       static_cast<hipStream_t>(stream));
}

int la_grad_norm_clip(int g_dtype, const void* g, uint64_t n, void* workspace, uint64_t workspace_bytes,
                      double* sqnorm, int accumulate, float max_norm, float* coef, float* norm_out,
                      la_stream_t stream)
{
    if (!coef) return LA_EINVAL;
    return launch_norm(g_dtype, g, n, workspace, workspace_bytes, sqnorm, accumulate, max_norm, coef, norm_out,
                       static_cast<hipStream_t>(stream));
}

int la_grad_norm_multi(int g_dtype, const la_grad_buffer_t* bufs, int count, void* workspace,
                       uint64_t workspace_bytes, double* sqnorm, int accumulate, float max_norm, float* coef,
                       float* norm_out, la_stream_t stream)
{
    return launch_norm_multi(g_dtype, bufs, count, workspace, workspace_bytes, sqnorm, accumulate, max_norm, coef,
                             norm_out, static_cast<hipStream_t>(stream));
}

int la_grad_norm_clip_noalloc(int g_dtype, const void* g, uint64_t n, double* sqnorm, int accumulate,
                              float max_norm, float* coef, float* norm_out, la_stream_t stream)
try {
    if (!coef) return LA_EINVAL;
    // stage 1 writes one partial per workgroup into the fixed array
    if (norm_workspace_bytes(n) > kScratchBytes) return LA_ERANGE;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_rc(e);
    // the scratch address is the current device's: a stream of another device
    // would run the kernels there, on that device's memory
    // NULL, the legacy and the per-thread default stream are the current device's
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (st != nullptr && st != hipStreamPerThread && st != hipStreamLegacy) {
        hipDevice_t stream_dev = -1;
        e = hipStreamGetDevice(st, &stream_dev);
        if (e != hipSuccess) return hip_rc(e);
        if (stream_dev != dev) return LA_EINVAL;
    }
    double* ptr = nullptr;
    const int rc = scratch_on_current_device(dev, &ptr);
    if (rc != LA_OK) return rc;
    return launch_norm(g_dtype, g, n, ptr, kScratchBytes, sqnorm, accumulate, max_norm, coef, norm_out,
                       static_cast<hipStream_t>(stream));
} catch (...) {
    return LA_ENOMEM;
}

int la_clip_coef(const double* sqnorm, float max_norm, float* coef, float* norm_out, la_stream_t stream)
{
    if (!sqnorm || !coef) return LA_EINVAL;
    if ((reinterpret_cast<uintptr_t>(sqnorm) & 7u) || (reinterpret_cast<uintptr_t>(coef) & 3u)) return LA_EINVAL;
    if (norm_out && (reinterpret_cast<uintptr_t>(norm_out) & 3u)) return LA_EINVAL;
    if (!device_accessible(sqnorm) || !device_accessible(coef) || (norm_out && !device_accessible(norm_out)))
        return LA_EFAULT;
    return launch(la_clip_coef_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), sqnorm, max_norm,
                  coef, norm_out);
}

}  // extern "C"
