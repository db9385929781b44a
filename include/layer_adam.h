/*
 * slideformer_amd -- C-ABI of the MI355X (gfx950) LayerAdam step.
 *
 * Replaces the reference's pybind module `cpu_adam`
 * (optimizer/layer_adam/csrc/cpu_adam.cpp:8-13, declarations cpu_adam.h:199-221).
 * Plain pointers and sizes only; no torch types.  The caller owns every buffer;
 * the library keeps only per-id scalar state (the beta-power state machine).
 *
 * Return codes: 0 on success; LA_EINVAL for a null/misaligned pointer, an
 * unknown id or a bad size; LA_EDTYPE for a dtype triple the reference does
 * not register; LA_ENOMEM when host memory or a host thread cannot be had;
 * LA_ERANGE for a size beyond the fixed scratch of la_grad_norm_clip_noalloc;
 * LA_EFAULT when an array a kernel would read or write (p, g, m, v, the bf16
 * copy, the clip coefficient, the norm's scalars and workspace) is not device
 * memory: host arrays, pageable or page-locked, are refused before any launch
 * (la_pipeline_step streams them);
 * a positive hipError_t value when a HIP call fails.  No C++ exception
 * leaves the library.
 * All device entry points are asynchronous on the stream passed in.
 */
#ifndef SLIDEFORMER_AMD_LAYER_ADAM_H
#define SLIDEFORMER_AMD_LAYER_ADAM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LA_ABI_VERSION 9

#define LA_OK 0
#define LA_EINVAL (-22)
#define LA_EDTYPE (-95)
#define LA_ENOMEM (-12)
#define LA_ERANGE (-34)
#define LA_EFAULT (-14)

/* element types of p / g / m,v */
#define LA_F32 0
#define LA_BF16 1
#define LA_F16 2

/* opaque HIP stream (hipStream_t); NULL = the default stream */
typedef void* la_stream_t;

/*
 * Scalars of one adam_update call, derived on the host by la_scalars()
 * exactly as Adam_Optimizer::IncrementStep + update_state + Step_AVX do
 * (cpu_adam.h:57-89, :131-148).
 */
typedef struct {
    float beta1, beta2;              /* _betta1, _betta2 */
    float one_minus_beta1;           /* 1 - b1            cpu_adam.h:131 */
    float one_minus_beta2;           /* 1 - b2            cpu_adam.h:132 */
    float bias_correction2;          /* 1/sqrtf(1-b2^t) or 1 (cpu_adam.h:87) */
    float eps;                       /* _eps */
    float step_size;                 /* -lr / bc1         cpu_adam.h:142 */
    float w_decay;                   /* -lr * wd          cpu_adam.h:146 */
    float weight_decay;              /* wd (L2 mode)      cpu_adam.h:148 */
    int32_t decay_mode;              /* 0 none, 1 L2 into the grad, 2 decoupled (AdamW) */
    float beta1_t, beta2_t;          /* _betta1_t, _betta2_t after IncrementStep */
    float bias_correction1;          /* 1 - b1^t or 1 */
    uint64_t step;                   /* _step after IncrementStep */
} la_scalars_t;

/* ABI version (LA_ABI_VERSION) */
int la_abi_version(void);

/* Human-readable text for a return code. */
const char* la_strerror(int code);

/*
 * Create / reset scalar state for `id`.
 * Replaces create_adam_optimizer, cpu_adam_impl.cpp:91-129 (pybind create_adam).
 * adamw_mode is fixed here, as in the reference; lr/eps/wd/betas are per call.
 */
int la_create(int id, float lr, float beta1, float beta2, float eps, float weight_decay,
              int adamw_mode, int should_log);

/* Replaces destroy_adam_optimizer, cpu_adam_impl.cpp:272-277 (pybind destroy_adam). */
int la_destroy(int id);

/*
 * Advance the beta-power state machine of `id` for one adam_update call and
 * return the derived scalars (cpu_adam.h:57-89; called at cpu_adam_impl.cpp:241-242).
 * Mutates the per-id state exactly like one reference call.
 */
int la_scalars(int id, uint64_t step, float lr, float beta1, float beta2, float eps,
               float weight_decay, int bias_correction, la_scalars_t* out);

/*
 * The fused elementwise update on device buffers, in place:
 *   p, m, v updated (Step_AVX body, cpu_adam.h:159-192; the last n % 16
 *   elements follow the reference's scalar tail, cpu_adam_impl.cpp:46-67),
 *   p_bf16_out[i] = RNE bf16 of the new p (nullable; transformer_layer.py:302-305),
 *   grads scaled by *clip_coef before use (nullable device pointer).
 * Elementwise body of ds_adam_step, cpu_adam_impl.cpp:255-267 (Step_8 cascade).
 */
int la_adamw_step(const la_scalars_t* sc, int p_dtype, void* p, int g_dtype, const void* g,
                  int s_dtype, void* m, void* v, uint64_t n, uint16_t* p_bf16_out,
                  const float* clip_coef, la_stream_t stream);

/*
 * One whole reference call: la_scalars + la_adamw_step.
 * Replaces ds_adam_step, cpu_adam_impl.cpp:220-270 (pybind adam_update).
 */
int la_adam_update(int id, uint64_t step, float lr, float beta1, float beta2, float eps,
                   float weight_decay, int bias_correction, int p_dtype, void* p, int g_dtype,
                   const void* g, int s_dtype, void* m, void* v, uint64_t n,
                   uint16_t* p_bf16_out, const float* clip_coef, la_stream_t stream);

/*
 * Several reference adam_update calls of one step in one go: segment k is the
 * call on (p, g, m, v, n) of tensor k, in order, with the same hyper-parameters
 * and element types, as LayerAdam.step(layer) and step_with_grad_views make
 * them (layer_adam.py:299-327, 391-422).  Exactly equivalent to count
 * la_adam_update calls: the beta-power state advances once per segment (also
 * for n = 0), and each segment keeps its own scalar tail.  Segments are
 * launched together (one launch per 16 segments; a segment of more than
 * 2^33 elements gets a grid-stride launch of its own), so the segments must
 * not overlap in memory.  Every pointer is checked before anything changes; an
 * unregistered dtype triple advances the state once and returns LA_EDTYPE,
 * as the first of the separate calls would.
 */
typedef struct {
    void* p;               /* params, p_dtype */
    const void* g;         /* grads, g_dtype */
    void* m;               /* exp_avg, s_dtype */
    void* v;               /* exp_avg_sq, s_dtype */
    uint16_t* p_bf16_out;  /* bf16 copy of the new params, nullable */
    uint64_t n;
} la_segment_t;

int la_adam_update_multi(int id, uint64_t step, float lr, float beta1, float beta2, float eps,
                         float weight_decay, int bias_correction, int p_dtype, int g_dtype,
                         int s_dtype, const la_segment_t* segs, int count, const float* clip_coef,
                         la_stream_t stream);

/*
 * Grad norm (no counterpart in the reference, which has no clipping;
 * SlideFormer's update sits at transformer_layer.py:453-493): sum of squares
 * of g[0..n) in float64 into *sqnorm (device), added to the old value when
 * accumulate != 0.  Two kernels on `stream`: per-workgroup partials, then one
 * workgroup folds them.
 * `workspace` is caller-owned device memory of at least
 * la_grad_sqnorm_workspace(n) bytes, 8-byte aligned, holding the partials.
 * Calls that share a workspace must be ordered (same stream); overlapping
 * calls race.  Deterministic for a given n and pointer alignment.
 */
uint64_t la_grad_sqnorm_workspace(uint64_t n);
int la_grad_sqnorm(int g_dtype, const void* g, uint64_t n, void* workspace,
                   uint64_t workspace_bytes, double* sqnorm, int accumulate, la_stream_t stream);

/*
 * la_grad_sqnorm whose folding kernel also writes the clip coefficient of the
 * (accumulated) *sqnorm, as la_clip_coef computes it.  coef must not be NULL.
 */
int la_grad_norm_clip(int g_dtype, const void* g, uint64_t n, void* workspace,
                      uint64_t workspace_bytes, double* sqnorm, int accumulate, float max_norm,
                      float* coef, float* norm_out, la_stream_t stream);

/*
 * The grad norm over several buffers of one element type in two launches
 * (one stage-1 launch that reads every buffer, one fold), where
 * la_grad_sqnorm would take two per buffer: for grads held per tensor, as
 * step(layer) and step_with_grad_views take them (layer_adam.py:299-327,
 * 391-422).  No counterpart in the reference, which has no clipping.
 * bufs[0..count) with 1 <= count <= LA_NORM_MULTI_MAX; a buffer may be empty
 * (g may then be NULL).  The sum of squares of all of them goes into *sqnorm,
 * added to the old value when accumulate != 0; with coef != NULL the fold
 * also writes the clip coefficient (and *norm_out when not NULL), as
 * la_grad_norm_clip does.  `workspace`: at least la_grad_sqnorm_workspace(N)
 * bytes for N the buffers' total element count.  Deterministic for given
 * sizes and pointer alignments; with one buffer the result is bit-identical
 * to la_grad_sqnorm's / la_grad_norm_clip's.  Every pointer is checked before
 * the first launch.
 */
#define LA_NORM_MULTI_MAX 32
typedef struct {
    const void* g;  /* grads, g_dtype */
    uint64_t n;
} la_grad_buffer_t;

int la_grad_norm_multi(int g_dtype, const la_grad_buffer_t* bufs, int count, void* workspace,
                       uint64_t workspace_bytes, double* sqnorm, int accumulate, float max_norm,
                       float* coef, float* norm_out, la_stream_t stream);

/*
 * la_grad_norm_clip without a workspace: for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference.  The stage-1
 * partials go to a fixed device array inside the library of
 * LA_NORM_SCRATCH_PARTIALS float64 (2 KiB), one copy per GPU, held until the
 * process ends; its address is looked up once per device and kept in a fixed
 * table of device ordinals 0-63 (a higher ordinal gives LA_EINVAL).  The call
 * itself allocates nothing (no hipMalloc, no hipFree, no allocating library
 * call, no host heap).
 * Stage 1 of this build never uses more than 256 workgroups, so every n fits;
 * a build whose stage-1 grid could outgrow the array returns LA_ERANGE for
 * such n.  Runs on the current device; `stream` must belong to it (NULL and
 * the legacy and per-thread default streams do): a stream of another device is refused
 * with LA_EINVAL before any launch.  Every
 * call on one GPU shares that GPU's array, which keeps the last call's
 * partials: calls that overlap on one GPU (streams not ordered with each
 * other) race.  The results are bit-identical to la_grad_norm_clip's for the
 * same arguments.
 */
#define LA_NORM_SCRATCH_PARTIALS 256
int la_grad_norm_clip_noalloc(int g_dtype, const void* g, uint64_t n, double* sqnorm, int accumulate,
                              float max_norm, float* coef, float* norm_out, la_stream_t stream);

/*
 * Clip coefficient on device, torch.nn.utils.clip_grad_norm_ convention:
 * norm = (float)sqrt(*sqnorm); *coef = min(1, max_norm / (norm + 1e-6)) in fp32;
 * *norm_out = norm (nullable).  No host synchronisation.
 */
int la_clip_coef(const double* sqnorm, float max_norm, float* coef, float* norm_out,
                 la_stream_t stream);

/*
 * Host <-> HBM streaming of the step, for state that lives in host RAM.
 * Replaces the runtime's chunk pipeline around the update: CPU fp32->bf16
 * cast + H2D (transformer_layer.py:297-305), grad D2H in chunks with
 * per-chunk events (:343-422) and the update thread consuming them (:453-493).
 * Here the host-resident arrays are copied in, updated on the GPU and copied
 * back, chunk by chunk, on three HIP streams (H2D, compute, D2H) so that
 * transfers in both directions overlap the update of other chunks.
 *
 * Placement: `on_host` has one bit per array.  A set bit means the array is
 * in host memory and streams through the device slots; a clear bit means it
 * is in device memory and the update reads and writes it in place.  The
 * reference runtime keeps everything on the host (LA_ON_HOST_P|M|V|G, plus
 * OUT when the bf16 copy goes to host staging); keeping the moments in HBM
 * (LA_ON_HOST_P | LA_ON_HOST_G) moves 6 B/param in and 4 B/param out instead
 * of 14 and 12.
 *
 * la_pipeline_create: chunk_elems is rounded down to a multiple of 16 (only
 *   the last chunk of a call then holds the reference's scalar tail); 1..16
 *   staging slots.  Creates the streams and events on the current device,
 *   which the pipeline then belongs to; allocates no memory.
 * la_pipeline_workspace_bytes: device staging bytes the caller must provide
 *   (256-byte aligned) for the given element types and placement.
 * la_pipeline_step: one reference adam_update over n elements (p, m, v, g
 *   and the nullable bf16 copy `out` placed as `on_host` says; host arrays
 *   page-locked for full speed).  Work queued on `after` before the call
 *   runs first; work queued on `after` later sees the result.  A call that
 *   copies pageable arrays through the host staging first waits on the host
 *   for that earlier work, since its threads read host memory directly.
 *   synchronize != 0 (or stats != NULL) waits for completion of this call
 *   and of every earlier one.  With synchronize == 0 the call returns once
 *   its work is queued, and work queued on `after` later is not ordered
 *   after it; its arrays, workspace and staging must then stay valid, and
 *   must not be read or written by the caller, until a synchronizing call or
 *   la_pipeline_sync.  The slot ring carries over from call to call, so
 *   consecutive calls on disjoint host ranges (the runtime's one call per
 *   chunk) keep both copy directions busy; a call touching host bytes of an
 *   earlier unsettled call, or using another workspace or slot layout
 *   (element types, placement) than the previous call, settles everything
 *   first.  Device-resident arrays are updated in call order on one stream.
 *   One pipeline object must not be used by two threads at once.  The call
 *   needs the pipeline's device current (LA_EINVAL otherwise), with the
 *   workspace and the device-resident arrays on that device.
 * la_pipeline_sync: wait until every queued call is complete in host memory.
 * la_pipeline_set_host_staging: attach caller-owned page-locked host memory
 *   (256-byte aligned, at least la_pipeline_workspace_bytes() for the call's
 *   types and placement) and the number of host copy threads (0 = up to 16),
 *   or detach it with pinned = NULL.  While attached, la_pipeline_step copies
 *   every pageable host array through it: `threads` host threads copy each
 *   chunk into the page-locked twin of its slot and the results back out, and
 *   the copy engines only ever see page-locked memory.  Without it pageable
 *   arrays go through the HIP runtime's own bounce buffers.  Changing the
 *   attachment settles every queued call first.  No
 *   reference counterpart: the reference updates pageable state on the CPU.
 */
#define LA_ON_HOST_P 1u
#define LA_ON_HOST_M 2u
#define LA_ON_HOST_V 4u
#define LA_ON_HOST_G 8u
#define LA_ON_HOST_OUT 16u
#define LA_ON_HOST_ALL 31u

typedef struct la_pipeline la_pipeline_t;

typedef struct {
    float wall_ms;      /* first H2D start .. last D2H end; with staging, the whole call (host clock) */
    float h2d_ms;       /* span of the H2D stream (includes waits for free slots) */
    float compute_ms;   /* span of the compute stream */
    float d2h_ms;       /* span of the D2H stream */
    uint64_t h2d_bytes;
    uint64_t d2h_bytes;
    uint32_t chunks;
    float host_copy_ms;     /* time the host threads spent copying through the staging */
    uint64_t staged_bytes;  /* bytes they copied (both directions) */
} la_pipeline_stats_t;

uint64_t la_pipeline_workspace_bytes(uint64_t chunk_elems, int slots, int p_dtype, int g_dtype,
                                     int s_dtype, unsigned on_host);
int la_pipeline_create(uint64_t chunk_elems, int slots, la_pipeline_t** out);
int la_pipeline_destroy(la_pipeline_t* pl);
int la_pipeline_sync(la_pipeline_t* pl);
int la_pipeline_set_host_staging(la_pipeline_t* pl, void* pinned, uint64_t bytes, int threads);
int la_pipeline_step(la_pipeline_t* pl, const la_scalars_t* sc, int p_dtype, void* p, int g_dtype,
                     const void* g, int s_dtype, void* m, void* v, uint64_t n, uint16_t* out,
                     unsigned on_host, const float* clip_coef, void* workspace,
                     uint64_t workspace_bytes, la_stream_t after, int synchronize,
                     la_pipeline_stats_t* stats);

/*
 * Asynchronous file offload of host state buffers (the NVMe moment offload).
 * Replaces tensornvme's DiskOffloader as LayerAdam uses it
 * (layer_adam.py:92-106 construction, :200-247 async_read / async_write /
 * sync_read_events / sync_write_events).  A pool of `threads` workers does
 * positioned reads/writes in 64 MiB pieces; one file per key,
 * "<dir>/offload-<pid>-<key>", removed by la_disk_destroy.
 *   la_disk_write_async / la_disk_read_async: queue the transfer of `bytes`
 *     from / into host memory that must stay valid until the matching sync.
 *     A read of a key never written returns -ENOENT.
 *   la_disk_sync_writes / la_disk_sync_reads: wait for every queued write /
 *     read; return 0 or the first failure as a negative errno.
 *   la_disk_create_ex with LA_DISK_DIRECT: the files are opened with O_DIRECT
 *     (no page-cache copies; the device's rates).  Buffers need no alignment:
 *     pieces of 16 MiB, unaligned ones through an aligned bounce buffer per
 *     worker, the last piece padded with zeros to a 4 KiB block.  Returns
 *     the open() error (e.g. -EINVAL) when the directory's file system does
 *     not take O_DIRECT.  la_disk_create is la_disk_create_ex with flags 0.
 */
typedef struct la_disk la_disk_t;

#define LA_DISK_DIRECT 1u

int la_disk_create(const char* dir, int threads, la_disk_t** out);
int la_disk_create_ex(const char* dir, int threads, unsigned flags, la_disk_t** out);
int la_disk_destroy(la_disk_t* d);
int la_disk_write_async(la_disk_t* d, uint64_t key, const void* src, uint64_t bytes);
int la_disk_read_async(la_disk_t* d, uint64_t key, void* dst, uint64_t bytes);
int la_disk_sync_writes(la_disk_t* d);
int la_disk_sync_reads(la_disk_t* d);

#ifdef __cplusplus
}
#endif
#endif /* SLIDEFORMER_AMD_LAYER_ADAM_H */
