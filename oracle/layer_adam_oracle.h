/*
 * TEST INFRASTRUCTURE ONLY -- the CPU checker for the LayerAdam step.
 *
 * A plain-C restatement of the reference's CPU Adam (DeepSpeed-derived
 * cpu_adam in optimizer/layer_adam/csrc/), plus the two things the MI355X
 * build adds on top of it (the bf16 compute copy and the grad-norm clip).
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it, and only as the checker.  The shipped library never calls it.
 */
#ifndef LAYER_ADAM_ORACLE_H
#define LAYER_ADAM_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types, same codes as the product C-ABI (include/layer_adam.h) */
enum { ORC_F32 = 0, ORC_BF16 = 1, ORC_F16 = 2 };

/* Scalar state of one optimizer id: mirrors class Adam_Optimizer,
 * cpu_adam.h:24-106 (members cpu_adam.h:91-105). */
typedef struct {
    float alpha, betta1, betta2, eps, weight_decay;
    float betta1_t, betta2_t;
    uint64_t step;
    float bias_correction1, bias_correction2;
    int adamw_mode;
} orc_adam_t;

/* constructor defaults, cpu_adam.h:26-42 */
void orc_create(orc_adam_t* s, float alpha, float b1, float b2, float eps, float wd,
                int adamw_mode);
/* IncrementStep, cpu_adam.h:57-76 */
void orc_increment_step(orc_adam_t* s, uint64_t step, float b1, float b2);
/* update_state, cpu_adam.h:77-89 */
void orc_update_state(orc_adam_t* s, float lr, float eps, float wd, int bias_correction);
/* Per-call derived scalars used by the element loop (cpu_adam.h:131-148):
 * out = {betta1_t, betta2_t, bc1, bc2, step_size, w_decay, 1-b1, 1-b2} */
void orc_scalars(const orc_adam_t* s, float out[8]);

/*
 * ds_adam_step, cpu_adam_impl.cpp:220-270: IncrementStep + update_state,
 * then the element loop over n elements in place.
 *   body_width : elements [0, n - n % body_width) follow the SIMD body op
 *                order (cpu_adam.h:159-192); the rest follow the scalar tail
 *                (cpu_adam_impl.cpp:46-67) as GCC -O3 contracts it.
 *                16 = the reference's AVX-512 build, 8 = its AVX2 build for
 *                all-fp32 triples, 0 = scalar tail everywhere (AVX2 build with
 *                a 16-bit type), 1 = body order everywhere.
 *   p_bf16_out : optional, receives RNE bf16 of the updated param.
 *   clip_coef  : optional, grads are fl32(f32(g) * *clip_coef) before use.
 * Returns 0, or -22 for an unknown dtype code.
 */
int orc_adam_update(orc_adam_t* s, uint64_t step, float lr, float b1, float b2, float eps,
                    float wd, int bias_correction, int p_dtype, void* p, int g_dtype,
                    const void* g, int s_dtype, void* m, void* v, uint64_t n,
                    uint16_t* p_bf16_out, const float* clip_coef, int body_width);

/* sum of squares of the grads in float64, sequential order */
double orc_grad_sqnorm(int g_dtype, const void* g, uint64_t n);
/* torch.nn.utils.clip_grad_norm_ coefficient: min(1, max_norm / (norm + 1e-6)) in fp32,
 * norm = (float)sqrt(sqnorm) */
float orc_clip_coef(double sqnorm, float max_norm, float* norm_out);

/* conversions */
uint16_t orc_f32_to_bf16(float x);   /* RNE, NaN -> 0x7FC0 (simd.h:56-86) */
float orc_bf16_to_f32(uint16_t h);   /* exact widening (simd.h:47-54) */
uint16_t orc_f32_to_f16(float x);    /* IEEE binary16 RNE, NaN -> sign|0x7E00 */
float orc_f16_to_f32(uint16_t h);    /* exact */
void orc_f32_to_bf16_array(const float* x, uint16_t* y, uint64_t n);

#ifdef __cplusplus
}
#endif
#endif
