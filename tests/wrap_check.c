/* CPU check of the binade-at-a-time angle wrap used by the device sin/cos
 * (rac_amd/csrc/rac_math.hpp wrap_binades) against the step-by-step loop of
 * rac_cpu.c:92-94: every float in (pi, 2^lim) with the given stride, both
 * signs, and the no-tie condition the method relies on (2 pi / u never has
 * fractional part 1/2 for binades 4..26).  Exit status 1 on any mismatch. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#define PI_F 3.14159265358979f
#define TAU_F 6.28318530717958f
static uint32_t as_u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float seq_wrap(float t) {
    while (t > PI_F) t -= TAU_F;
    while (t <= -PI_F) t += TAU_F;
    return t;
}
/* theta > 0 side: while (theta > pi) theta -= tau, in O(binades) */
static float fast_pos(float th) {
    while (th >= 16.0f) {
        const int e = (int)((as_u(th) >> 23) & 0xFF) - 127;       /* th in [2^e, 2^(e+1)) */
        const int m = (int)(as_u(th) & 0x7FFFFF);
        const float ulp = ldexpf(1.0f, e - 23);
        const float tq = TAU_F * ldexpf(1.0f, 23 - e);            /* tau in units of ulp (exact) */
        const int t = (int)rintf(tq), c = (int)ceilf(tq);
        if (m >= c) {
            const int k = (m - c) / t + 1;                         /* steps that stay in [2^e, 2^(e+1)) */
            th = fmaf(-(float)k, (float)t * ulp, th);              /* exact */
        }
        th = th - TAU_F;                                           /* the step that leaves the binade */
    }
    while (th > PI_F) th -= TAU_F;
    return th;
}
static float fast_neg(float th) {   /* th <= -pi side, mirrored: while (th <= -pi) th += tau */
    float a = -th;
    while (a >= 16.0f) {
        const int e = (int)((as_u(a) >> 23) & 0xFF) - 127;
        const int m = (int)(as_u(a) & 0x7FFFFF);
        const float ulp = ldexpf(1.0f, e - 23);
        const float tq = TAU_F * ldexpf(1.0f, 23 - e);
        const int t = (int)rintf(tq), c = (int)ceilf(tq);
        if (m >= c) {
            const int k = (m - c) / t + 1;
            a = fmaf(-(float)k, (float)t * ulp, a);
        }
        a = a - TAU_F;
    }
    th = -a;
    while (th <= -PI_F) th += TAU_F;
    return th;
}
static float fast_wrap(float t) {
    if (t > PI_F) return fast_pos(t);
    if (t <= -PI_F) return fast_neg(t);
    return t;
}
int main(int argc, char** argv) {
    /* ties: tau/ulp has fractional part exactly 1/2 for which binade? */
    for (int e = 4; e <= 26; e++) {
        float tq = TAU_F * ldexpf(1.0f, 23 - e);
        if (tq - floorf(tq) == 0.5f) { printf("TIE at e=%d\n", e); return 1; }
    }
    long bad = 0, n = 0;
    /* every float in (pi, 2^lim) with stride S, both signs */
    const int lim = argc > 1 ? atoi(argv[1]) : 16;
    const uint32_t stride = argc > 2 ? (uint32_t)atoi(argv[2]) : 1;
    const uint32_t lo = as_u(PI_F), hi = as_u(ldexpf(1.0f, lim));
    for (uint32_t u = lo; u < hi; u += stride) {
        float th; memcpy(&th, &u, 4);
        for (int sgn = 0; sgn < 2; sgn++) {
            float x = sgn ? -th : th;
            float a = seq_wrap(x), b = fast_wrap(x);
            n++;
            if (as_u(a) != as_u(b)) { if (bad < 10) printf("MISMATCH %a: %a vs %a\n", x, a, b); bad++; }
        }
    }
    printf("lim 2^%d stride %u: %ld checked, %ld mismatches\n", lim, stride, n, bad);
    return bad != 0;
}
