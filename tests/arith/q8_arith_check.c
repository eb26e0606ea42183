/* Exhaustive checks of the two short arithmetic sequences the q8_1 activation prologue of the
 * streaming kernels uses in place of an IEEE division and roundf (kernels.hip, quant_store). Each
 * must give exactly the IEEE result the reference's q8_1 quantizer computes:
 *   1. d = amax / 127:  q = amax * c (c = RN(1/127)), r = fma(-q, 127, amax), d = fma(r, c, q)
 *      (Markstein's correction step), for every normal amax whose quotient is normal;
 *   2. roundf(v) (half away from zero) = trunc(v + copysign(0.49999997f, v)) for |v| <= 2^23.
 * Check 1 depends only on the significand (scaling by powers of two is exact in the normal
 * range), so all 2^23 significands at a few exponents cover the normal range. (The reciprocal
 * 1/d stays an IEEE division: one or two Newton steps from a 1-ulp seed miss the rounding for
 * some d.)
 * Prints "ok" and exits 0, or prints the first counterexample and exits 1. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float f_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t u_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

int main(void) {
    const float c = 1.0f / 127.0f;
    for (uint32_t m = 0; m < (1u << 23); m++) {
        for (int e = 0; e < 3; e++) {   /* three exponents around 1 (the significand decides) */
            const float a = f_of(((uint32_t)(126 + e) << 23) | m);
            const float q = a * c;
            const float r = fmaf(-q, 127.0f, a);
            const float d = fmaf(r, c, q);
            if (u_of(d) != u_of(a / 127.0f)) { printf("div127 fails at %a\n", a); return 1; }
        }
    }
    for (uint32_t u = 0; u <= 0x4b000000u; u++) {   /* 0 .. 2^23, both signs */
        const float v = f_of(u);
        for (int s = 0; s < 2; s++) {
            const float x = s ? -v : v;
            const float t = truncf(x + copysignf(0.49999997f, x));
            if (u_of(t) != u_of(roundf(x)) && !(t == 0.0f && roundf(x) == 0.0f)) {
                printf("round fails at %a\n", x);
                return 1;
            }
        }
    }
    printf("ok\n");
    return 0;
}
