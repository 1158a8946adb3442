/* Exhaustive check of the activation quantiser's per-value division
 * (div_by_scale in fp8_gemm_h20/csrc/fp8bg.hip): for r = RN(1 / s),
 *     q1 = fma(fma(-q0, s, v), r, q0),  q0 = RN(v * r),
 * equals RN(v / s) for every bf16 v in [1, 4) and every fp32 s in [1, 2)
 * (2^31 pairs: every scale mantissa against every bf16 mantissa, quotients
 * on both sides of 1).  Multiplying v and s by powers of two scales every
 * step exactly, so this covers all bf16 v and all s the kernel takes.
 * Also counts the pairs where the plain product q0 is wrong, so a check that
 * skipped the correction would be seen to fail.  Built with
 * -ffp-contract=off; prints "ok <pairs> <plain_bad>" or the first failures. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float f32(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }
static uint32_t bits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }

int main(void) {
    unsigned long n = 0, bad = 0, plain_bad = 0;
#pragma omp parallel for reduction(+ : n, bad, plain_bad) schedule(static)
    for (int sm = 0; sm < (1 << 23); ++sm) {
        const float s = f32(0x3f800000u | (uint32_t)sm);
        const float r = 1.0f / s;
        for (uint32_t h = 0x3f80u; h < 0x4080u; ++h) {
            const float v = f32(h << 16);
            const float q0 = v * r;
            const float q1 = fmaf(fmaf(-q0, s, v), r, q0);
            const uint32_t want = bits(v / s);
            ++n;
            plain_bad += bits(q0) != want;
            bad += bits(q1) != want;
        }
    }
    if (bad) {
        printf("FAILED %lu of %lu\n", bad, n);
        return 1;
    }
    printf("ok %lu %lu\n", n, plain_bad);
    return 0;
}
