/* Exhaustive check of the few-token quantiser's division-free scale and
 * reciprocal (act_scale_reciprocal_fast in fp8_gemm_h20/csrc/fp8bg.hip) on its
 * domain, x a finite bf16 value in [2^-100, 0x1.fep127] (the kernel takes
 * them for an amax of at least eps >= 1e-30):
 *   s = fma(fma(-q0, 448, x), RN(1/448), q0), q0 = RN(x * RN(1/448)),
 *       equals RN(x / 448) for every positive finite bf16 x;
 *   r = fma(fma(-s, r0, 1), r0, r0) equals RN(1 / s) for every s of the
 *       domain and every start value r0 within 2 ulp of RN(1 / s) (the
 *       hardware reciprocal is documented within 1 ulp).
 * Also counts how often the plain product x * RN(1/448) is wrong, so a
 * check that skipped the correction would be seen to fail.
 * Built with -ffp-contract=off; prints "ok <n> <m> <plain_bad>" or the
 * first failures. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float f32(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }
static uint32_t bits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }

int main(void) {
    const float inv448 = 1.0f / 448.0f;
    unsigned long n_div = 0, n_rcp = 0, bad = 0, plain_bad = 0;
    for (uint32_t h = 1; h < 0x7f80u; ++h) {          /* every positive finite bf16 */
        const float x = f32(h << 16);
        const float q0 = x * inv448;
        const float s = fmaf(fmaf(-q0, 448.0f, x), inv448, q0);
        const float s_ref = x / 448.0f;
        ++n_div;
        if (bits(q0) != bits(s_ref)) ++plain_bad;
        if (bits(s) != bits(s_ref)) {
            if (bad++ < 5) printf("quotient x=%a: %a, expected %a\n", x, s, s_ref);
            continue;
        }
        if (x < 0x1p-100f) continue;                  /* outside the fast domain */
        const float r_ref = 1.0f / s;
        for (int d = -2; d <= 2; ++d) {
            const float r0 = f32(bits(r_ref) + d);
            const float r = fmaf(fmaf(-s, r0, 1.0f), r0, r0);
            ++n_rcp;
            if (bits(r) != bits(r_ref) && bad++ < 5)
                printf("reciprocal s=%a from %a: %a, expected %a\n", s, r0, r, r_ref);
        }
    }
    if (bad) {
        printf("FAILED %lu\n", bad);
        return 1;
    }
    printf("ok %lu %lu %lu\n", n_div, n_rcp, plain_bad);
    return 0;
}
