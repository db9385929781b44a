// slideformer_amd: host <-> HBM streaming of the LayerAdam step.
//
// For optimizer state that lives in host RAM (the reference runtime's layout:
// fp32 master and moments on the CPU, transformer_layer.py:192-196 and
// layer_adam.py:161-173), one call streams the state through HBM in chunks:
//
//   h2d stream :  copy the host-resident arrays among p, m, v, g of chunk i into
//                 slot i % S
//   compute    :  wait for that copy, run the fused update on the slot (arrays
//                 that live in device memory are read and written in place)
//   d2h stream :  wait for the update, copy the host-resident p, m, v (and the
//                 bf16 copy when it goes to the host) back, then free the slot
//                 for chunk i + S
//
// The reference does the same split with threads and a queue of per-chunk
// events (transformer_layer.py:297-305 H2D, :343-422 D2H, :453-493 update);
// here three HIP streams at default priority and per-slot events chain the
// stages, so copies in both directions overlap the update of other chunks.
// Chunks are multiples of 16 elements, so only the last chunk of a call holds
// the reference's scalar tail.  The caller owns the device staging memory.
//
// Pageable host arrays (the reference allocates its moments with plain
// torch.zeros, layer_adam.py:161-173) cannot be reached by the copy engines
// directly; the runtime would bounce them through small internal buffers at a
// fraction of the link rate.  With page-locked host staging attached
// (la_pipeline_set_host_staging), each slot gets a page-locked twin: a pool of
// host threads copies chunk i of every pageable array into the twin, the copy
// engines move the twin, and after the copy-back the threads copy the results
// out of the twin before chunk i + S reuses it.
//
// Calls need not drain the pipeline.  The slot ring carries over from call to
// call, so the runtime's one-call-per-chunk protocol (transformer_layer.py:
// 470-476) keeps both copy directions busy across its calls.  A call with
// synchronize == 0 returns once its work is queued; a staged chunk's copy-out
// is then owed until its slot is reused, a call touches the same host bytes,
// or la_pipeline_sync runs.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <memory>
#include <new>
#include <thread>
#include <vector>

#include "../../include/layer_adam.h"
#include "copy_pool.h"
#include "hip_ptr.h"

using la_host::CopyPool;
using la_host::Piece;

// Host-side trace of the pipeline's HIP calls, off in the product build:
// with LA_PIPELINE_TRACE defined to 1, every call of la_pipeline_step that
// holds the calling thread for LA_PIPELINE_TRACE_MS or longer is printed to
// stderr with its pipeline call, chunk, slot and text.
#ifndef LA_PIPELINE_TRACE
#define LA_PIPELINE_TRACE 0
#endif
#ifndef LA_PIPELINE_TRACE_MS
#define LA_PIPELINE_TRACE_MS 0.5
#endif

struct la_pipeline {
    int device = 0;
    uint64_t chunk = 0;
    int slots = 0;
    hipStream_t h2d = nullptr, comp = nullptr, d2h = nullptr;
    std::vector<hipEvent_t> ev_h2d, ev_comp, ev_d2h;
    hipEvent_t t_begin = nullptr, t_h2d_end = nullptr, t_comp_end = nullptr, t_end = nullptr, t_comp_begin = nullptr,
               t_d2h_begin = nullptr;
    // page-locked host staging for pageable arrays (caller-owned; null = none)
    char* host_staging = nullptr;
    uint64_t host_staging_bytes = 0;
    std::unique_ptr<CopyPool> pool;
    // the slot ring across calls: chunks issued so far; slot_used[s] once
    // ev_d2h[s] has been recorded
    uint64_t issued = 0;
    std::vector<char> slot_used;
    // copy-outs owed per slot (staged arrays of a chunk whose call returned
    // before its results left the page-locked twin)
    std::vector<std::vector<Piece>> owed;
    // host byte ranges [lo, hi) touched by calls since the last full sync
    std::vector<std::pair<uintptr_t, uintptr_t>> touched;
    // device workspace and slot size of the last call: slot s of another
    // layout can overlap slot s + 1 of this one
    const char* last_ws = nullptr;
    uint64_t last_slot_bytes = 0;
    uint64_t calls = 0;  // la_pipeline_step calls so far (the trace's call numbers)
};

namespace {

constexpr uint64_t kAlign = 256;

uint64_t round_up(uint64_t x, uint64_t a) { return (x + a - 1) / a * a; }
int esize(int dt) { return dt == LA_F32 ? 4 : 2; }

struct SlotLayout {
    uint64_t p, m, v, g, out, slot_bytes;
};

// A slot holds one chunk of every host-resident array (on_host bits).
SlotLayout slot_layout(uint64_t chunk, int p_dt, int g_dt, int s_dt, unsigned on_host)
{
    SlotLayout L{};
    uint64_t off = 0;
    L.p = off;
    if (on_host & LA_ON_HOST_P) off += round_up(chunk * esize(p_dt), kAlign);
    L.m = off;
    if (on_host & LA_ON_HOST_M) off += round_up(chunk * esize(s_dt), kAlign);
    L.v = off;
    if (on_host & LA_ON_HOST_V) off += round_up(chunk * esize(s_dt), kAlign);
    L.g = off;
    if (on_host & LA_ON_HOST_G) off += round_up(chunk * esize(g_dt), kAlign);
    L.out = off;
    if (on_host & LA_ON_HOST_OUT) off += round_up(chunk * 2, kAlign);
    L.slot_bytes = off;
    return L;
}

bool misaligned(const void* ptr, int bytes) { return reinterpret_cast<uintptr_t>(ptr) % static_cast<uintptr_t>(bytes); }

int rc_of(hipError_t e) { return e == hipSuccess ? LA_OK : static_cast<int>(e); }

// Host memory the copy engines can read and write directly: page-locked
// (hipHostMalloc, torch pin_memory) or registered.  Anything else is pageable.
using la_ptr::page_locked;
// Device (or managed / unified) memory, which the update may read and write in place.
inline bool device_memory(const void* ptr) { return la_ptr::device_accessible(ptr); }

// Host copies are split into pieces of at most this many bytes for the pool.
constexpr uint64_t kPieceBytes = 1ull << 20;

void add_pieces(std::vector<Piece>& out, void* dst, const void* src, uint64_t bytes)
{
    char* d = static_cast<char*>(dst);
    const char* s = static_cast<const char*>(src);
    for (uint64_t o = 0; o < bytes; o += kPieceBytes)
        out.push_back(Piece{d + o, s + o, std::min(kPieceBytes, bytes - o)});
}

// Copy the results of slot s out of its page-locked twin once its copy-back
// has landed (nothing to do when no copy-out is owed).
int settle_slot(la_pipeline* pl, uint64_t s)
{
    if (pl->owed[s].empty()) return LA_OK;
    const hipError_t e = hipEventSynchronize(pl->ev_d2h[s]);
    if (e != hipSuccess) return rc_of(e);
    pl->pool->run(pl->owed[s]);
    pl->owed[s].clear();
    return LA_OK;
}

// Everything queued so far has landed in host memory: owed copy-outs in slot
// order of issue, then the copy streams.
int settle_all(la_pipeline* pl)
{
    const uint64_t S = static_cast<uint64_t>(pl->slots);
    for (uint64_t j = 0; j < S; ++j) {
        const int rc = settle_slot(pl, (pl->issued + j) % S);
        if (rc != LA_OK) return rc;
    }
    hipError_t e = hipStreamSynchronize(pl->h2d);
    if (e == hipSuccess) e = hipStreamSynchronize(pl->comp);
    if (e == hipSuccess) e = hipStreamSynchronize(pl->d2h);
    pl->touched.clear();
    return rc_of(e);
}

// After a failure part-way through a call, let the queued copies finish before
// returning, so that nothing still writes the caller's memory afterwards, and
// deliver the copy-outs of every chunk whose copy-back was queued.
int drain_streams(la_pipeline* pl, int rc)
{
    (void)hipStreamSynchronize(pl->h2d);
    (void)hipStreamSynchronize(pl->comp);
    (void)hipStreamSynchronize(pl->d2h);
    const uint64_t S = static_cast<uint64_t>(pl->slots);
    for (uint64_t j = 0; j < S; ++j) {
        std::vector<Piece>& o = pl->owed[(pl->issued + j) % S];
        if (!o.empty() && pl->pool) pl->pool->run(o);
        o.clear();
    }
    pl->touched.clear();
    return rc;
}

bool overlaps(const std::vector<std::pair<uintptr_t, uintptr_t>>& a, uintptr_t lo, uintptr_t hi)
{
    for (const auto& r : a)
        if (lo < r.second && r.first < hi) return true;
    return false;
}

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
                                     unsigned on_host)
{
    chunk_elems = chunk_elems / 16 * 16;
    if (chunk_elems == 0 || slots <= 0 || (on_host & ~LA_ON_HOST_ALL)) return 0;
    return slot_layout(chunk_elems, p_dtype, g_dtype, s_dtype, on_host).slot_bytes * static_cast<uint64_t>(slots);
}

int la_pipeline_create(uint64_t chunk_elems, int slots, la_pipeline_t** out)
try {
    if (!out) return LA_EINVAL;
    *out = nullptr;
    chunk_elems = chunk_elems / 16 * 16;
    if (chunk_elems == 0 || slots < 1 || slots > 16) return LA_EINVAL;
    la_pipeline* pl = new (std::nothrow) la_pipeline();
    if (!pl) return LA_EINVAL;
    pl->chunk = chunk_elems;
    pl->slots = slots;
    pl->slot_used.assign(static_cast<size_t>(slots), 0);
    pl->owed.resize(static_cast<size_t>(slots));
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
} catch (...) {
    return LA_ENOMEM;
}

int la_pipeline_destroy(la_pipeline_t* pl)
{
    if (!pl) return LA_OK;
    // copy-outs still owed are completed: the host arrays must still be valid
    if (pl->pool && pl->h2d && pl->comp && pl->d2h) (void)settle_all(pl);
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

int la_pipeline_sync(la_pipeline_t* pl)
try {
    if (!pl) return LA_EINVAL;
    return settle_all(pl);
} catch (...) {
    return LA_ENOMEM;
}

int la_pipeline_set_host_staging(la_pipeline_t* pl, void* pinned, uint64_t bytes, int threads)
{
    if (!pl) return LA_EINVAL;
    if (threads == 0) threads = static_cast<int>(std::min(16u, std::max(1u, std::thread::hardware_concurrency())));
    if (static_cast<char*>(pinned) == pl->host_staging && (!pinned || (bytes == pl->host_staging_bytes && pl->pool &&
                                                                       pl->pool->threads() == threads)))
        return LA_OK;  // unchanged
    // owed copy-outs read the current twins: settle them before the staging changes
    {
        const int rc = settle_all(pl);
        if (rc != LA_OK) return rc;
    }
    if (!pinned) {
        pl->host_staging = nullptr;
        pl->host_staging_bytes = 0;
        return LA_OK;
    }
    if (bytes == 0 || reinterpret_cast<uintptr_t>(pinned) % kAlign || threads < 0 || threads > 64) return LA_EINVAL;
    char* base = static_cast<char*>(pinned);
    if (!page_locked(base) || !page_locked(base + bytes - 1)) return LA_EINVAL;
    if (!pl->pool || pl->pool->threads() != threads) {
        pl->pool.reset();
        try {
            pl->pool.reset(new CopyPool(threads));
        } catch (...) {
            return LA_EINVAL;
        }
    }
    pl->host_staging = base;
    pl->host_staging_bytes = bytes;
    return LA_OK;
}

int la_pipeline_step(la_pipeline_t* pl, const la_scalars_t* sc, int p_dtype, void* p, int g_dtype, const void* g,
                     int s_dtype, void* m, void* v, uint64_t n, uint16_t* out, unsigned on_host,
                     const float* clip_coef, void* workspace, uint64_t workspace_bytes, la_stream_t after,
                     int synchronize, la_pipeline_stats_t* stats)
try {
    const auto t0 = std::chrono::steady_clock::now();
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
    if (on_host & ~LA_ON_HOST_ALL) return LA_EINVAL;
    if (n == 0) return LA_OK;
    if (!p || !g || !m || !v || !workspace) return LA_EINVAL;
    {
        // the pipeline's streams belong to the device current at creation, and so
        // must the update it launches there and the device arrays it touches
        int cur = -1;
        const hipError_t e = hipGetDevice(&cur);
        if (e != hipSuccess) return rc_of(e);
        if (cur != pl->device) return LA_EINVAL;
    }
    const bool hp = on_host & LA_ON_HOST_P, hm = on_host & LA_ON_HOST_M, hv = on_host & LA_ON_HOST_V;
    const bool hg = on_host & LA_ON_HOST_G, ho = on_host & LA_ON_HOST_OUT;
    if (ho && !out) return LA_EINVAL;
    const int pb = esize(p_dtype), gb = esize(g_dtype), sb = esize(s_dtype);
    // device-resident arrays are used in place: whole elements only
    if ((!hp && misaligned(p, pb)) || (!hm && misaligned(m, sb)) || (!hv && misaligned(v, sb)) ||
        (!hg && misaligned(g, gb)) || (out && !ho && misaligned(out, 2)))
        return LA_EINVAL;
    if (clip_coef && misaligned(clip_coef, 4)) return LA_EINVAL;
    if (misaligned(workspace, static_cast<int>(kAlign))) return LA_EINVAL;
    // arrays the update reads and writes in place must be device memory; refuse
    // them here, before any transfer starts, rather than in the first chunk
    if ((!hp && !device_memory(p)) || (!hm && !device_memory(m)) || (!hv && !device_memory(v)) ||
        (!hg && !device_memory(g)) || (out && !ho && !device_memory(out)) || !device_memory(workspace) ||
        (clip_coef && !device_memory(clip_coef)))
        return LA_EFAULT;
    const SlotLayout L = slot_layout(pl->chunk, p_dtype, g_dtype, s_dtype, on_host);
    const uint64_t ws_need = L.slot_bytes * static_cast<uint64_t>(pl->slots);
    if (workspace_bytes < ws_need) return LA_EINVAL;

    // which host arrays go through the page-locked staging (pageable ones, when it is attached)
    bool st_p = false, st_m = false, st_v = false, st_g = false, st_o = false;
    if (pl->host_staging) {
        st_p = hp && !page_locked(p);
        st_m = hm && !page_locked(m);
        st_v = hv && !page_locked(v);
        st_g = hg && !page_locked(g);
        st_o = ho && !page_locked(out);
    }
    const bool staged = st_p || st_m || st_v || st_g || st_o;
    if (staged && pl->host_staging_bytes < ws_need) return LA_EINVAL;

    char* ws = static_cast<char*>(workspace);
    char* pp = static_cast<char*>(p);
    char* mp = static_cast<char*>(m);
    char* vp = static_cast<char*>(v);
    const char* gp = static_cast<const char*>(g);
    char* op = reinterpret_cast<char*>(out);
    const uint64_t nchunks = (n + pl->chunk - 1) / pl->chunk;
    const uint64_t S = static_cast<uint64_t>(pl->slots);
    hipStream_t caller = static_cast<hipStream_t>(after);
    uint64_t h2d_bytes = 0, d2h_bytes = 0, staged_bytes = 0;
    double host_copy_ms = 0.0;
    std::vector<Piece> pieces;

    // Host bytes this call reads or writes.  If an earlier call that has not
    // been settled touched any of them (the same layer stepped again), settle
    // everything first; otherwise this call streams on behind the earlier ones.
    std::pair<uintptr_t, uintptr_t> ranges[5];
    int nranges = 0;
    auto add_range = [&](bool host, const void* ptr, uint64_t bytes) {
        if (!host) return;
        const uintptr_t lo = reinterpret_cast<uintptr_t>(ptr);
        ranges[nranges++] = {lo, lo + bytes};
    };
    add_range(hp, pp, n * pb);
    add_range(hm, mp, n * sb);
    add_range(hv, vp, n * sb);
    add_range(hg, gp, n * gb);
    add_range(ho, op, n * 2);
    bool clash = pl->touched.size() > 4096;
    // another workspace or slot layout than the previous call's: the slots of
    // the two layouts overlap, so earlier work must be finished first
    if (pl->issued > 0 && (ws != pl->last_ws || L.slot_bytes != pl->last_slot_bytes)) clash = true;
    for (int r = 0; r < nranges && !clash; ++r) clash = overlaps(pl->touched, ranges[r].first, ranges[r].second);
    if (clash) {
        const int rc = settle_all(pl);
        if (rc != LA_OK) return rc;
    }
    for (int r = 0; r < nranges; ++r) pl->touched.push_back(ranges[r]);
    pl->last_ws = ws;
    pl->last_slot_bytes = L.slot_bytes;

    auto host_copy = [&]() {
        const auto a = std::chrono::steady_clock::now();
        pl->pool->run(pieces);
        host_copy_ms += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - a).count();
        for (const Piece& q : pieces) staged_bytes += q.bytes;
        pieces.clear();
    };
    // settle a slot's owed copy-out, counting it in this call's statistics
    auto settle = [&](uint64_t s) -> int {
        if (pl->owed[s].empty()) return LA_OK;
        const hipError_t e = hipEventSynchronize(pl->ev_d2h[s]);
        if (e != hipSuccess) return rc_of(e);
        pieces.swap(pl->owed[s]);
        host_copy();
        return LA_OK;
    };

    uint64_t trace_chunk = 0, trace_slot = 0;
    const uint64_t trace_call = pl->calls++;
    (void)trace_chunk;
    (void)trace_slot;
    (void)trace_call;
#if LA_PIPELINE_TRACE
#define LA_STEP_TRY(expr)                                                                                        \
    do {                                                                                                         \
        const auto a_ = std::chrono::steady_clock::now();                                                        \
        const hipError_t e_ = (expr);                                                                            \
        const double ms_ = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - a_).count(); \
        if (ms_ >= LA_PIPELINE_TRACE_MS)                                                                         \
            std::fprintf(stderr, "[la_pipeline] call %llu chunk %llu slot %llu: %.3f ms in %s\n",                \
                         (unsigned long long)trace_call, (unsigned long long)trace_chunk,                         \
                         (unsigned long long)trace_slot, ms_, #expr);                                            \
        if (e_ != hipSuccess) return drain_streams(pl, rc_of(e_));                                                \
    } while (0)
#else
#define LA_STEP_TRY(expr)                                         \
    do {                                                          \
        const hipError_t e_ = (expr);                             \
        if (e_ != hipSuccess) return drain_streams(pl, rc_of(e_)); \
    } while (0)
#endif

    // Everything the caller queued before (e.g. the backward that produced g)
    // comes first.  A call that stages pageable arrays waits for it on the host
    // anyway, since its host threads read the host arrays directly; that work
    // is then complete, and the pipeline's streams need no wait of their own.
    // Measured on MI355X: with such device-side waits, one per call, a series
    // of staged calls that return once queued (one per 32 Mi elements) stalled
    // the copy streams for ~3.5 ms per Llama-3.1-8B layer, twice; without
    // them the series runs at the single-call rate.
    // Otherwise only the H2D stream waits: the update of chunk i waits for
    // ev_h2d of chunk i and the copy-back for ev_comp, so the other two streams
    // follow the caller's work through those events.
    LA_STEP_TRY(hipEventRecord(pl->t_begin, caller));
    if (staged) {
        LA_STEP_TRY(hipEventSynchronize(pl->t_begin));
    } else {
        LA_STEP_TRY(hipStreamWaitEvent(pl->h2d, pl->t_begin, 0));
    }
    LA_STEP_TRY(hipEventRecord(pl->t_comp_begin, pl->comp));
    LA_STEP_TRY(hipEventRecord(pl->t_d2h_begin, pl->d2h));

    for (uint64_t i = 0; i < nchunks; ++i) {
        const uint64_t s = pl->issued % S;
        trace_chunk = i;
        trace_slot = s;
        const uint64_t off = i * pl->chunk;
        const uint64_t k = (n - off) < pl->chunk ? (n - off) : pl->chunk;
        char* slot = ws + s * L.slot_bytes;
        char* hs = staged ? pl->host_staging + s * L.slot_bytes : nullptr;
        {
            // the twin of slot s still holds the results of chunk issued - S
            const int rc = settle(s);
            if (rc != LA_OK) return drain_streams(pl, rc);
        }
        if (staged) {
            // The twin may still be the source of the previous chunk of slot s:
            // its H2D waits behind that slot's earlier copy-back and can be
            // queued well after this point.  When copy-outs were owed, settle()
            // already waited for the copy-back, which follows the H2D; when only
            // inputs were staged (pageable grads beside pinned or device state),
            // nothing else holds the host back from overwriting the twin.
            if (pl->slot_used[s]) LA_STEP_TRY(hipEventSynchronize(pl->ev_h2d[s]));
            if (st_p) add_pieces(pieces, hs + L.p, pp + off * pb, k * pb);
            if (st_m) add_pieces(pieces, hs + L.m, mp + off * sb, k * sb);
            if (st_v) add_pieces(pieces, hs + L.v, vp + off * sb, k * sb);
            if (st_g) add_pieces(pieces, hs + L.g, gp + off * gb, k * gb);
            host_copy();
        }
        // the addresses the update uses: a slot region for host arrays, the array itself otherwise
        char* pd = hp ? slot + L.p : pp + off * pb;
        char* md = hm ? slot + L.m : mp + off * sb;
        char* vd = hv ? slot + L.v : vp + off * sb;
        const void* gd = hg ? static_cast<const void*>(slot + L.g) : static_cast<const void*>(gp + off * gb);
        uint16_t* od = nullptr;
        if (out) od = ho ? reinterpret_cast<uint16_t*>(slot + L.out) : out + off;

        if (pl->slot_used[s]) LA_STEP_TRY(hipStreamWaitEvent(pl->h2d, pl->ev_d2h[s], 0));
        auto copy_in = [&](bool host, bool st, char* dst, uint64_t region, const char* src, uint64_t bytes) {
            if (!host) return hipSuccess;
            h2d_bytes += bytes;
            return hipMemcpyAsync(dst, st ? hs + region : src, bytes, hipMemcpyHostToDevice, pl->h2d);
        };
        LA_STEP_TRY(copy_in(hp, st_p, pd, L.p, pp + off * pb, k * pb));
        LA_STEP_TRY(copy_in(hm, st_m, md, L.m, mp + off * sb, k * sb));
        LA_STEP_TRY(copy_in(hv, st_v, vd, L.v, vp + off * sb, k * sb));
        LA_STEP_TRY(copy_in(hg, st_g, slot + L.g, L.g, gp + off * gb, k * gb));
        LA_STEP_TRY(hipEventRecord(pl->ev_h2d[s], pl->h2d));

        LA_STEP_TRY(hipStreamWaitEvent(pl->comp, pl->ev_h2d[s], 0));
        const int rc = la_adamw_step(sc, p_dtype, pd, g_dtype, gd, s_dtype, md, vd, k, od, clip_coef, pl->comp);
        if (rc != LA_OK) return drain_streams(pl, rc);
        LA_STEP_TRY(hipEventRecord(pl->ev_comp[s], pl->comp));

        LA_STEP_TRY(hipStreamWaitEvent(pl->d2h, pl->ev_comp[s], 0));
        auto copy_out = [&](bool host, bool st, char* dst, uint64_t region, const char* src, uint64_t bytes) {
            if (!host) return hipSuccess;
            d2h_bytes += bytes;
            return hipMemcpyAsync(st ? hs + region : dst, src, bytes, hipMemcpyDeviceToHost, pl->d2h);
        };
        LA_STEP_TRY(copy_out(hp, st_p, pp + off * pb, L.p, pd, k * pb));
        LA_STEP_TRY(copy_out(hm, st_m, mp + off * sb, L.m, md, k * sb));
        LA_STEP_TRY(copy_out(hv, st_v, vp + off * sb, L.v, vd, k * sb));
        LA_STEP_TRY(copy_out(ho, st_o, op + off * 2, L.out, reinterpret_cast<const char*>(od), k * 2));
        LA_STEP_TRY(hipEventRecord(pl->ev_d2h[s], pl->d2h));
        pl->slot_used[s] = 1;
        pl->issued++;
        // the results of staged arrays are owed until they leave the twin
        if (st_p) add_pieces(pl->owed[s], pp + off * pb, hs + L.p, k * pb);
        if (st_m) add_pieces(pl->owed[s], mp + off * sb, hs + L.m, k * sb);
        if (st_v) add_pieces(pl->owed[s], vp + off * sb, hs + L.v, k * sb);
        if (st_o) add_pieces(pl->owed[s], op + off * 2, hs + L.out, k * 2);
    }
    LA_STEP_TRY(hipEventRecord(pl->t_h2d_end, pl->h2d));
    LA_STEP_TRY(hipEventRecord(pl->t_comp_end, pl->comp));
    LA_STEP_TRY(hipEventRecord(pl->t_end, pl->d2h));
    // later work on the caller's stream sees the updated state.  Not for a call
    // that returns once queued: the next call records its start on the caller's
    // stream, and that wait would make it start only after this call's last
    // copy-back; such calls are completed by la_pipeline_sync instead.
    if (synchronize || stats) LA_STEP_TRY(hipStreamWaitEvent(caller, pl->t_end, 0));
#undef LA_STEP_TRY
    if (synchronize || stats) {
        // every copy-out owed, this call's and earlier ones, in order of issue
        for (uint64_t j = 0; j < S; ++j) {
            const int rc = settle((pl->issued + j) % S);
            if (rc != LA_OK) return drain_streams(pl, rc);
        }
        const hipError_t e = hipEventSynchronize(pl->t_end);
        if (e != hipSuccess) return rc_of(e);
        // t_end follows every earlier call's copy-backs on the same stream
        pl->touched.clear();
    }
    if (stats) {
        stats->h2d_bytes = h2d_bytes;
        stats->d2h_bytes = d2h_bytes;
        stats->chunks = static_cast<uint32_t>(nchunks);
        (void)hipEventElapsedTime(&stats->wall_ms, pl->t_begin, pl->t_end);
        (void)hipEventElapsedTime(&stats->h2d_ms, pl->t_begin, pl->t_h2d_end);
        (void)hipEventElapsedTime(&stats->compute_ms, pl->t_comp_begin, pl->t_comp_end);
        (void)hipEventElapsedTime(&stats->d2h_ms, pl->t_d2h_begin, pl->t_end);
        stats->staged_bytes = staged_bytes;
        stats->host_copy_ms = static_cast<float>(host_copy_ms);
        if (staged)
            stats->wall_ms = static_cast<float>(
                std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count());
    }
    return LA_OK;
} catch (...) {
    // host allocation failed part-way: let the queued work land first
    if (pl) (void)drain_streams(pl, LA_OK);
    return LA_ENOMEM;
}

}  // extern "C"
