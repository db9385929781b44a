/*
 * TEST INFRASTRUCTURE ONLY -- CPU restatement of the reference LayerAdam step.
 *
 * Follows, op for op:
 *   - Adam_Optimizer state + IncrementStep/update_state   cpu_adam.h:24-89
 *   - the SIMD element body (Step_AVX<span>)              cpu_adam.h:108-196
 *   - the scalar tail (Step_1 after the SIMD prefix)      cpu_adam_impl.cpp:23-70
 *   - the span cascade 8 -> 4 -> 1 -> scalar              cpu_adam_impl.cpp:72-89,131-148
 *   - dtype triples and the call sequence of ds_adam_step cpu_adam_impl.cpp:178-191,220-270
 *   - bf16 load/store helpers                             simd.h:47-88
 * and adds what the MI355X build fuses into the same pass: the bf16 compute
 * copy (transformer_layer.py:302-305 casts the master with torch copy_) and a
 * clip coefficient applied to the gradient (torch clip_grad_norm_ convention).
 *
 * Compiled with -ffp-contract=off: every fused multiply-add below is an
 * explicit fmaf(); every other * + / sqrtf is a separately rounded IEEE op.
 *
 * Parity pins (tests/test_oracle.py): bit-exact against the reference compiled
 * from its own sources (oracle/_ref) for every dtype triple, body and tail,
 * both state-machine paths; against the committed fixtures in tests/golden/;
 * against torch.optim.AdamW within rtol 1e-6 / atol 1e-7
 * (test_shared_data_parallel.py:89); conversions against torch / numpy.
 */
#include "layer_adam_oracle.h"

#include <math.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* conversions                                                         */
/* ------------------------------------------------------------------ */

static inline uint32_t f2u(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float u2f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* simd.h:56-86: u + ((u >> 16) & 1) + 0x7FFF, >> 16; NaN -> 0x7FC0 */
uint16_t orc_f32_to_bf16(float x)
{
    uint32_t u = f2u(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    return (uint16_t)((u + ((u >> 16) & 1u) + 0x7fffu) >> 16);
}

/* simd.h:47-54: zero-extend then shift left by 16 */
float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* IEEE binary16, round to nearest even (the rounding of c10::Half(float) and
 * of _mm512_cvtps_ph(.., _MM_FROUND_TO_NEAREST_INT)). */
uint16_t orc_f32_to_f16(float x)
{
    uint32_t u = f2u(x);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return sign | 0x7e00u;          /* NaN */
    if (a >= 0x477ff000u) return sign | 0x7c00u;         /* >= 65520 -> inf */
    if (a >= 0x38800000u) {                               /* normal half */
        uint32_t r = a - 0x38000000u;                     /* rebias 127 -> 15 */
        return sign | (uint16_t)((r + 0xfffu + ((r >> 13) & 1u)) >> 13);
    }
    uint32_t e = a >> 23;
    if (e < 102) return sign;                             /* < 2^-25 -> 0 */
    uint32_t mant = (a & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126 - e;                             /* 14 .. 24 */
    uint32_t q = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return sign | (uint16_t)q;
}

float orc_f16_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0) {
        float mag = (float)m * 0x1p-24f;                  /* exact */
        return u2f(f2u(mag) | sign);
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

void orc_f32_to_bf16_array(const float* x, uint16_t* y, uint64_t n)
{
    for (uint64_t i = 0; i < n; ++i) y[i] = orc_f32_to_bf16(x[i]);
}

static inline float load_as_f32(int dt, const void* base, uint64_t i)
{
    switch (dt) {
    case ORC_F32: return ((const float*)base)[i];
    case ORC_BF16: return orc_bf16_to_f32(((const uint16_t*)base)[i]);
    default: return orc_f16_to_f32(((const uint16_t*)base)[i]);
    }
}

static inline void store_from_f32(int dt, void* base, uint64_t i, float x)
{
    switch (dt) {
    case ORC_F32: ((float*)base)[i] = x; break;
    case ORC_BF16: ((uint16_t*)base)[i] = orc_f32_to_bf16(x); break;
    default: ((uint16_t*)base)[i] = orc_f32_to_f16(x); break;
    }
}

/* ------------------------------------------------------------------ */
/* scalar state machine                                                */
/* ------------------------------------------------------------------ */

void orc_create(orc_adam_t* s, float alpha, float b1, float b2, float eps, float wd,
                int adamw_mode)
{
    memset(s, 0, sizeof(*s));
    s->alpha = alpha;
    s->betta1 = b1;
    s->betta2 = b2;
    s->eps = eps;
    s->weight_decay = wd;
    s->betta1_t = 1.0f;
    s->betta2_t = 1.0f;
    s->step = 0;
    s->adamw_mode = adamw_mode;
}

/* cpu_adam.h:57-76.  std::pow(float, size_t) promotes both to double; the
 * result is rounded to float on assignment. */
void orc_increment_step(orc_adam_t* s, uint64_t step, float b1, float b2)
{
    if (b1 != s->betta1 || b2 != s->betta2) {
        s->step = step;
        s->betta1 = b1;
        s->betta2 = b2;
        s->betta1_t = (float)pow((double)s->betta1, (double)step);
        s->betta2_t = (float)pow((double)s->betta2, (double)step);
    } else {
        s->step++;
        if (s->step != step) {
            s->betta1_t = (float)pow((double)s->betta1, (double)step);
            s->betta2_t = (float)pow((double)s->betta2, (double)step);
            s->step = step;
        } else {
            s->betta1_t *= s->betta1;
            s->betta2_t *= s->betta2;
        }
    }
}

/* cpu_adam.h:77-89; the reference build computes bc2 as 1.0f / sqrtf(float). */
void orc_update_state(orc_adam_t* s, float lr, float eps, float wd, int bias_correction)
{
    s->alpha = lr;
    s->eps = eps;
    s->weight_decay = wd;
    s->bias_correction1 = 1.0f;
    s->bias_correction2 = 1.0f;
    if (bias_correction) {
        s->bias_correction1 = 1.0f - s->betta1_t;
        s->bias_correction2 = 1.0f / sqrtf(1.0f - s->betta2_t);
    }
}

void orc_scalars(const orc_adam_t* s, float out[8])
{
    out[0] = s->betta1_t;
    out[1] = s->betta2_t;
    out[2] = s->bias_correction1;
    out[3] = s->bias_correction2;
    out[4] = -1.0f * s->alpha / s->bias_correction1;   /* cpu_adam.h:142 */
    out[5] = -1.0f * s->alpha * s->weight_decay;       /* cpu_adam.h:146 */
    out[6] = 1.0f - s->betta1;                          /* cpu_adam.h:131 */
    out[7] = 1.0f - s->betta2;                          /* cpu_adam.h:132 */
}

/* ------------------------------------------------------------------ */
/* element loop                                                        */
/* ------------------------------------------------------------------ */

typedef struct {
    float b1, b2, omb1, omb2, bc2, eps, step_size, w_decay, wd;
    int l2, decoupled;
} orc_k_t;

/* One element.  tail == 0: SIMD body order, cpu_adam.h:159-192.
 * tail == 1: the plain-C loop cpu_adam_impl.cpp:46-67 as GCC -O3 (FMA ISA)
 * contracts it: the products m*b1 and v*b2 become the fused terms
 * (m = fma(m, b1, g*(1-b1)), v = fma(v, b2, (g*g)*(1-b2))); every other
 * contraction coincides with the body's explicit FMAs. */
static inline void orc_elem(float* pp, float g, float* mm, float* vv, const orc_k_t* k, int tail)
{
    float p = *pp, m = *mm, v = *vv;
    if (k->l2) g = fmaf(p, k->wd, g);
    if (!tail) {
        m = m * k->b1;
        m = fmaf(g, k->omb1, m);
        v = v * k->b2;
        float gg = g * g;
        v = fmaf(gg, k->omb2, v);
    } else {
        float gm = g * k->omb1;
        m = fmaf(m, k->b1, gm);
        float gg = g * g;
        gg = gg * k->omb2;
        v = fmaf(v, k->b2, gg);
    }
    float d = sqrtf(v);
    d = fmaf(d, k->bc2, k->eps);
    float u = m / d;
    if (k->decoupled) p = fmaf(p, k->w_decay, p);
    p = fmaf(u, k->step_size, p);
    *pp = p;
    *mm = m;
    *vv = v;
}

static int dt_ok(int dt) { return dt == ORC_F32 || dt == ORC_BF16 || dt == ORC_F16; }

int orc_adam_update(orc_adam_t* s, uint64_t step, float lr, float b1, float b2, float eps,
                    float wd, int bias_correction, int p_dtype, void* p, int g_dtype,
                    const void* g, int s_dtype, void* m, void* v, uint64_t n,
                    uint16_t* p_bf16_out, const float* clip_coef, int body_width)
{
    if (!dt_ok(p_dtype) || !dt_ok(g_dtype) || !dt_ok(s_dtype)) return -22;
    orc_increment_step(s, step, b1, b2);
    orc_update_state(s, lr, eps, wd, bias_correction);

    float sc[8];
    orc_scalars(s, sc);
    orc_k_t k;
    k.b1 = s->betta1;
    k.b2 = s->betta2;
    k.omb1 = sc[6];
    k.omb2 = sc[7];
    k.bc2 = s->bias_correction2;
    k.eps = s->eps;
    k.step_size = sc[4];
    k.w_decay = sc[5];
    k.wd = s->weight_decay;
    k.l2 = (s->weight_decay > 0.0f) && !s->adamw_mode;
    k.decoupled = (s->weight_decay > 0.0f) && s->adamw_mode;

    uint64_t body_end;
    if (body_width <= 0) body_end = 0;
    else body_end = n - n % (uint64_t)body_width;

    const int has_clip = clip_coef != NULL;
    const float coef = has_clip ? *clip_coef : 1.0f;

#pragma omp parallel for schedule(static) if (n > (1u << 16))
    for (uint64_t i = 0; i < n; ++i) {
        float gi = load_as_f32(g_dtype, g, i);
        if (has_clip) gi = gi * coef;
        float pi = load_as_f32(p_dtype, p, i);
        float mi = load_as_f32(s_dtype, m, i);
        float vi = load_as_f32(s_dtype, v, i);
        orc_elem(&pi, gi, &mi, &vi, &k, i >= body_end);
        store_from_f32(p_dtype, p, i, pi);
        store_from_f32(s_dtype, m, i, mi);
        store_from_f32(s_dtype, v, i, vi);
        if (p_bf16_out) p_bf16_out[i] = orc_f32_to_bf16(pi);
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* grad norm + clip coefficient                                        */
/* ------------------------------------------------------------------ */

/* Compensated (Neumaier) float64 sum of the exact squares, so that the result
 * is the true sum to about one ulp of binary64 whatever the length; any
 * summation order (the GPU's tree) is then compared against the exact value. */
/* Neumaier's compensated addition of y into the running pair (s, c). */
static void neumaier_add(double* s, double* c, double y)
{
    const double t = *s + y;
    if (fabs(*s) >= fabs(y)) *c += (*s - t) + y;
    else *c += (y - t) + *s;
    *s = t;
}

/* Compensated float64 sum of g[i]^2 over [lo, hi) as the pair (s, c). */
static void sqnorm_block(int g_dtype, const void* g, uint64_t lo, uint64_t hi, double* s_out, double* c_out)
{
    double s = 0.0, c = 0.0;
    for (uint64_t i = lo; i < hi; ++i) {
        const double x = (double)load_as_f32(g_dtype, g, i);
        neumaier_add(&s, &c, x * x);  /* x * x is exact in binary64 for any binary32 x */
    }
    *s_out = s;
    *c_out = isfinite(s) ? c : 0.0;  /* an inf term (or overflow) leaves inf - inf = NaN in c */
}

/* Sum of squares, compensated.  Large inputs are cut into a fixed number of
 * blocks summed in parallel; the blocks' pairs are then added, compensated, in
 * block order, so the result does not depend on the thread count. */
#define ORC_SQNORM_BLOCKS 64
double orc_grad_sqnorm(int g_dtype, const void* g, uint64_t n)
{
    double s, c;
    if (n < (1u << 20)) {
        sqnorm_block(g_dtype, g, 0, n, &s, &c);
        return s + c;  /* c is 0 when s is inf or NaN */
    }
    double bs[ORC_SQNORM_BLOCKS], bc[ORC_SQNORM_BLOCKS];
#pragma omp parallel for schedule(static)
    for (int b = 0; b < ORC_SQNORM_BLOCKS; ++b)
        sqnorm_block(g_dtype, g, n / ORC_SQNORM_BLOCKS * (uint64_t)b,
                     b == ORC_SQNORM_BLOCKS - 1 ? n : n / ORC_SQNORM_BLOCKS * (uint64_t)(b + 1), &bs[b], &bc[b]);
    s = 0.0;
    c = 0.0;
    for (int b = 0; b < ORC_SQNORM_BLOCKS; ++b) {
        neumaier_add(&s, &c, bs[b]);
        neumaier_add(&s, &c, bc[b]);
    }
    return isfinite(s) ? s + c : s;
}

/* torch.nn.utils.clip_grad_norm_: clip_coef = max_norm / (total_norm + 1e-6),
 * clamped to at most 1.0, evaluated in fp32. */
float orc_clip_coef(double sqnorm, float max_norm, float* norm_out)
{
    float norm = (float)sqrt(sqnorm);
    if (norm_out) *norm_out = norm;
    float c = max_norm / (norm + 1e-6f);
    return (c < 1.0f || c != c) ? c : 1.0f;
}
