/*
 * A plain C11 caller of include/layer_adam.h: the boundary must be usable from
 * C, not only through ctypes.  Only host-side entry points are called (no GPU
 * is needed): version, error strings, the optimizer registry, the beta-power
 * state machine and the workspace sizes.  Prints one line per scalar set for
 * the calling test to check against the CPU checker.
 */
#include <stdio.h>
#include <string.h>

#include "layer_adam.h"

int main(void)
{
    if (la_abi_version() != LA_ABI_VERSION) return 10;
    if (la_strerror(LA_EINVAL) == NULL || strlen(la_strerror(LA_EDTYPE)) == 0) return 11;
    if (la_create(4242, 1e-3f, 0.9f, 0.999f, 1e-8f, 0.01f, 1, 0) != LA_OK) return 12;
    la_scalars_t sc;
    /* steps 1..5, then a second call of step 5 (pow path), then a jump to step 9 */
    const uint64_t steps[] = {1, 2, 3, 4, 5, 5, 9};
    for (unsigned i = 0; i < sizeof(steps) / sizeof(steps[0]); ++i) {
        memset(&sc, 0, sizeof(sc));
        if (la_scalars(4242, steps[i], 1e-3f, 0.9f, 0.999f, 1e-8f, 0.01f, 1, &sc) != LA_OK) return 13;
        printf("%llu %a %a %a %a %a %a %d\n", (unsigned long long)sc.step, sc.beta1_t, sc.beta2_t,
               sc.bias_correction1, sc.bias_correction2, sc.step_size, sc.w_decay, (int)sc.decay_mode);
    }
    if (la_scalars(4243, 1, 1e-3f, 0.9f, 0.999f, 1e-8f, 0.01f, 1, &sc) != LA_EINVAL) return 14;  /* unknown id */
    if (la_destroy(4242) != LA_OK) return 15;
    if (la_pipeline_workspace_bytes(1000, 2, LA_F32, LA_BF16, LA_F32, LA_ON_HOST_P | LA_ON_HOST_G) != 2 * (4096 + 2048))
        return 16;
    if (la_grad_sqnorm_workspace(1) == 0) return 17;
    /* argument checks that fail before touching a device */
    if (la_adamw_step(NULL, LA_F32, NULL, LA_BF16, NULL, LA_F32, NULL, NULL, 1, NULL, NULL, NULL) != LA_EINVAL)
        return 18;
    return 0;
}
