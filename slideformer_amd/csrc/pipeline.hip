// slideformer_amd: host <-> HBM streaming of the LayerAdam step.
//
// For optimizer state that lives in host RAM (the reference runtime's layout:
// fp32 master and moments on the CPU, transformer_layer.py:192-196 and
// layer_adam.py:161-173), one call streams the state through HBM in chunks:
//
//   h2d stream :  copy p, m, v (and g when it is on the host) of chunk i into slot i % S
//   compute    :  wait for that copy, run the fused update on the slot
//   d2h stream :  wait for the update, copy p, m, v (and the bf16 copy when it goes
//                 to the host) back, then free the slot for chunk i + S
//
// The reference does the same split with threads and a queue of per-chunk
// events (transformer_layer.py:297-305 H2D, :343-422 D2H, :453-493 update);
// here three HIP streams at default priority and per-slot events chain the
// stages, so copies in both directions overlap the update of other chunks.
// Chunks are multiples of 16 elements, so only the last chunk of a call holds
// the reference's scalar tail.  The caller owns the device staging memory.

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <new>
#include <vector>

#include "../../include/layer_adam.h"

struct la_pipeline {
    int device = 0;
    uint64_t chunk = 0;
    int slots = 0;
    hipStream_t h2d = nullptr, comp = nullptr, d2h = nullptr;
    std::vector<hipEvent_t> ev_h2d, ev_comp, ev_d2h;
    hipEvent_t t_begin = nullptr, t_h2d_end = nullptr, t_comp_end = nullptr, t_end = nullptr, t_comp_begin = nullptr,
               t_d2h_begin = nullptr;
};

namespace {

constexpr uint64_t kAlign = 256;

uint64_t round_up(uint64_t x, uint64_t a) { return (x + a - 1) / a * a; }
int esize(int dt) { return dt == LA_F32 ? 4 : 2; }

struct SlotLayout {
    uint64_t p, m, v, g, out, slot_bytes;
};

SlotLayout slot_layout(uint64_t chunk, int p_dt, int g_dt, int s_dt, int g_on_host, int out_on_host)
{
    SlotLayout L{};
    uint64_t off = 0;
    L.p = off;
    off += round_up(chunk * esize(p_dt), kAlign);
    L.m = off;
    off += round_up(chunk * esize(s_dt), kAlign);
    L.v = off;
    off += round_up(chunk * esize(s_dt), kAlign);
    L.g = off;
    if (g_on_host) off += round_up(chunk * esize(g_dt), kAlign);
    L.out = off;
    if (out_on_host) off += round_up(chunk * 2, kAlign);
    L.slot_bytes = off;
    return L;
}

int rc_of(hipError_t e) { return e == hipSuccess ? LA_OK : static_cast<int>(e); }

#define LA_TRY(expr)                           \
    do {                                       \
        const hipError_t e_ = (expr);          \
        if (e_ != hipSuccess) return rc_of(e_); \
    } while (0)

void destroy_events(la_pipeline* pl)
{
    for (auto* v : {&pl->ev_h2d, &pl->ev_comp, &pl->ev_d2h})
        for (hipEvent_t e : *v)
            if (e) (void)hipEventDestroy(e);
    for (hipEvent_t e : {pl->t_begin, pl->t_h2d_end, pl->t_comp_end, pl->t_end, pl->t_comp_begin, pl->t_d2h_begin})
        if (e) (void)hipEventDestroy(e);
}

}  // namespace

extern "C" {

uint64_t la_pipeline_workspace_bytes(uint64_t chunk_elems, int slots, int p_dtype, int g_dtype, int s_dtype,
                                     int g_on_host, int out_on_host)
{
    chunk_elems = chunk_elems / 16 * 16;
    if (chunk_elems == 0 || slots <= 0) return 0;
    return slot_layout(chunk_elems, p_dtype, g_dtype, s_dtype, g_on_host, out_on_host).slot_bytes *
           static_cast<uint64_t>(slots);
}

int la_pipeline_create(uint64_t chunk_elems, int slots, la_pipeline_t** out)
{
    if (!out) return LA_EINVAL;
    *out = nullptr;
    chunk_elems = chunk_elems / 16 * 16;
    if (chunk_elems == 0 || slots < 1 || slots > 16) return LA_EINVAL;
    la_pipeline* pl = new (std::nothrow) la_pipeline();
    if (!pl) return LA_EINVAL;
    pl->chunk = chunk_elems;
    pl->slots = slots;
    hipError_t e = hipGetDevice(&pl->device);
    // default priority everywhere (hipStreamCreateWithFlags, no priority argument)
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&pl->h2d, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&pl->comp, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&pl->d2h, hipStreamNonBlocking);
    for (int i = 0; i < slots && e == hipSuccess; ++i) {
        hipEvent_t a = nullptr, b = nullptr, c = nullptr;
        e = hipEventCreateWithFlags(&a, hipEventDisableTiming);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&b, hipEventDisableTiming);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&c, hipEventDisableTiming);
        pl->ev_h2d.push_back(a);
        pl->ev_comp.push_back(b);
        pl->ev_d2h.push_back(c);
    }
    for (hipEvent_t* t : {&pl->t_begin, &pl->t_h2d_end, &pl->t_comp_end, &pl->t_end, &pl->t_comp_begin, &pl->t_d2h_begin})
        if (e == hipSuccess) e = hipEventCreate(t);
    if (e != hipSuccess) {
        la_pipeline_destroy(pl);
        return rc_of(e);
    }
    *out = pl;
    return LA_OK;
}

int la_pipeline_destroy(la_pipeline_t* pl)
{
    if (!pl) return LA_OK;
    if (pl->h2d) (void)hipStreamSynchronize(pl->h2d);
    if (pl->comp) (void)hipStreamSynchronize(pl->comp);
    if (pl->d2h) (void)hipStreamSynchronize(pl->d2h);
    destroy_events(pl);
    if (pl->h2d) (void)hipStreamDestroy(pl->h2d);
    if (pl->comp) (void)hipStreamDestroy(pl->comp);
    if (pl->d2h) (void)hipStreamDestroy(pl->d2h);
    delete pl;
    return LA_OK;
}

int la_pipeline_step(la_pipeline_t* pl, const la_scalars_t* sc, int p_dtype, void* p_host, int g_dtype, const void* g,
                     int g_on_host, int s_dtype, void* m_host, void* v_host, uint64_t n, uint16_t* out,
                     int out_on_host, const float* clip_coef, void* workspace, uint64_t workspace_bytes,
                     la_stream_t after, int synchronize, la_pipeline_stats_t* stats)
{
    if (stats) std::memset(stats, 0, sizeof(*stats));
    if (!pl || !sc) return LA_EINVAL;
    if (p_dtype < LA_F32 || p_dtype > LA_F16 || g_dtype < LA_F32 || g_dtype > LA_F16 || s_dtype < LA_F32 ||
        s_dtype > LA_F16)
        return LA_EDTYPE;
    // the dtype triple is checked up front (an n = 0 call validates without launching),
    // so a bad triple cannot stop the chunk loop half-way
    {
        const int rc = la_adamw_step(sc, p_dtype, nullptr, g_dtype, nullptr, s_dtype, nullptr, nullptr, 0, nullptr,
                                     nullptr, nullptr);
        if (rc != LA_OK) return rc;
    }
    if (n == 0) return LA_OK;
    if (!p_host || !g || !m_host || !v_host || !workspace) return LA_EINVAL;
    if (!g_on_host && reinterpret_cast<uintptr_t>(g) % static_cast<uintptr_t>(esize(g_dtype))) return LA_EINVAL;
    if (out && !out_on_host && (reinterpret_cast<uintptr_t>(out) & 1u)) return LA_EINVAL;
    if (clip_coef && (reinterpret_cast<uintptr_t>(clip_coef) & 3u)) return LA_EINVAL;
    if (out_on_host && !out) return LA_EINVAL;
    if (reinterpret_cast<uintptr_t>(workspace) % kAlign) return LA_EINVAL;
    const SlotLayout L = slot_layout(pl->chunk, p_dtype, g_dtype, s_dtype, g_on_host, out_on_host && out);
    if (workspace_bytes < L.slot_bytes * static_cast<uint64_t>(pl->slots)) return LA_EINVAL;

    const int pb = esize(p_dtype), gb = esize(g_dtype), sb = esize(s_dtype);
    char* ws = static_cast<char*>(workspace);
    char* ph = static_cast<char*>(p_host);
    char* mh = static_cast<char*>(m_host);
    char* vh = static_cast<char*>(v_host);
    const char* gp = static_cast<const char*>(g);
    char* op = reinterpret_cast<char*>(out);
    const uint64_t nchunks = (n + pl->chunk - 1) / pl->chunk;
    hipStream_t caller = static_cast<hipStream_t>(after);
    uint64_t h2d_bytes = 0, d2h_bytes = 0;

    // the slots are free once the previous call's last copy-back is done
    LA_TRY(hipStreamWaitEvent(pl->h2d, pl->t_end, 0));
    // everything the caller queued before (e.g. the backward that produced g) comes first
    LA_TRY(hipEventRecord(pl->t_begin, caller));
    LA_TRY(hipStreamWaitEvent(pl->h2d, pl->t_begin, 0));
    LA_TRY(hipStreamWaitEvent(pl->comp, pl->t_begin, 0));
    LA_TRY(hipStreamWaitEvent(pl->d2h, pl->t_begin, 0));
    LA_TRY(hipEventRecord(pl->t_comp_begin, pl->comp));
    LA_TRY(hipEventRecord(pl->t_d2h_begin, pl->d2h));

    for (uint64_t i = 0; i < nchunks; ++i) {
        const int s = static_cast<int>(i % static_cast<uint64_t>(pl->slots));
        const uint64_t off = i * pl->chunk;
        const uint64_t k = (n - off) < pl->chunk ? (n - off) : pl->chunk;
        char* slot = ws + static_cast<uint64_t>(s) * L.slot_bytes;
        if (i >= static_cast<uint64_t>(pl->slots)) LA_TRY(hipStreamWaitEvent(pl->h2d, pl->ev_d2h[s], 0));
        LA_TRY(hipMemcpyAsync(slot + L.p, ph + off * pb, k * pb, hipMemcpyHostToDevice, pl->h2d));
        LA_TRY(hipMemcpyAsync(slot + L.m, mh + off * sb, k * sb, hipMemcpyHostToDevice, pl->h2d));
        LA_TRY(hipMemcpyAsync(slot + L.v, vh + off * sb, k * sb, hipMemcpyHostToDevice, pl->h2d));
        h2d_bytes += k * (pb + 2 * sb);
        const void* gdev = gp + off * gb;
        if (g_on_host) {
            LA_TRY(hipMemcpyAsync(slot + L.g, gp + off * gb, k * gb, hipMemcpyHostToDevice, pl->h2d));
            h2d_bytes += k * gb;
            gdev = slot + L.g;
        }
        LA_TRY(hipEventRecord(pl->ev_h2d[s], pl->h2d));

        LA_TRY(hipStreamWaitEvent(pl->comp, pl->ev_h2d[s], 0));
        uint16_t* odev = nullptr;
        if (out) odev = out_on_host ? reinterpret_cast<uint16_t*>(slot + L.out) : out + off;
        const int rc = la_adamw_step(sc, p_dtype, slot + L.p, g_dtype, gdev, s_dtype, slot + L.m, slot + L.v, k,
                                     odev, clip_coef, pl->comp);
        if (rc != LA_OK) return rc;
        LA_TRY(hipEventRecord(pl->ev_comp[s], pl->comp));

        LA_TRY(hipStreamWaitEvent(pl->d2h, pl->ev_comp[s], 0));
        LA_TRY(hipMemcpyAsync(ph + off * pb, slot + L.p, k * pb, hipMemcpyDeviceToHost, pl->d2h));
        LA_TRY(hipMemcpyAsync(mh + off * sb, slot + L.m, k * sb, hipMemcpyDeviceToHost, pl->d2h));
        LA_TRY(hipMemcpyAsync(vh + off * sb, slot + L.v, k * sb, hipMemcpyDeviceToHost, pl->d2h));
        d2h_bytes += k * (pb + 2 * sb);
        if (out && out_on_host) {
            LA_TRY(hipMemcpyAsync(op + off * 2, slot + L.out, k * 2, hipMemcpyDeviceToHost, pl->d2h));
            d2h_bytes += k * 2;
        }
        LA_TRY(hipEventRecord(pl->ev_d2h[s], pl->d2h));
    }
    LA_TRY(hipEventRecord(pl->t_h2d_end, pl->h2d));
    LA_TRY(hipEventRecord(pl->t_comp_end, pl->comp));
    LA_TRY(hipEventRecord(pl->t_end, pl->d2h));
    // later work on the caller's stream sees the updated state
    LA_TRY(hipStreamWaitEvent(caller, pl->t_end, 0));
    if (synchronize || stats) LA_TRY(hipEventSynchronize(pl->t_end));
    if (stats) {
        stats->h2d_bytes = h2d_bytes;
        stats->d2h_bytes = d2h_bytes;
        stats->chunks = static_cast<uint32_t>(nchunks);
        (void)hipEventElapsedTime(&stats->wall_ms, pl->t_begin, pl->t_end);
        (void)hipEventElapsedTime(&stats->h2d_ms, pl->t_begin, pl->t_h2d_end);
        (void)hipEventElapsedTime(&stats->compute_ms, pl->t_comp_begin, pl->t_comp_end);
        (void)hipEventElapsedTime(&stats->d2h_ms, pl->t_d2h_begin, pl->t_end);
    }
    return LA_OK;
}

}  // extern "C"
