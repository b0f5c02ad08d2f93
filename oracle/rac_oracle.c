/*
 * rac_oracle.c — CPU restatement of the RAC rotation-accumulate hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py load this library, and only as the checker.
 * The product (rac_amd/librac_amd.so) never links, loads or calls it.
 *
 * Build: oracle/Makefile -> oracle/liboracle.so (gcc -O2 -ffp-contract=off,
 * no fast-math: every rounding below is the one written, so the results are
 * reproducible bit for bit by the gfx950 kernels, which are compiled with
 * -ffp-contract=off as well).
 *
 * Each function cites the reference file:line it restates.  How each one is
 * pinned (golden vectors from the compiled reference, closed forms,
 * exhaustive or brute-force checks) is listed in tests/test_oracle.py.
 * Functions that are the product's own algorithm choice where the reference
 * has none (hyperbolic CORDIC exp in product-register form, CORDIC-vectoring
 * rsqrt) are pinned against the reference spec they generalise and against
 * libm within their analytic error bound.
 *
 * Signed zeros: results are compared with IEEE equality (-0 == +0) where the
 * only possible difference is the sign of an exact zero.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define ORC_API __attribute__((visibility("default")))

/* ── Constants ──────────────────────────────────────────────────────────── */

static const float ORC_PI = 3.14159265358979f;        /* RAC_PI, rac_cpu.h:43 */
static const float ORC_TAU = 6.28318530717958f;       /* rac_kernels.hip:143; == 2.0f*RAC_PI */
static const float ORC_K_INV = 0.60725f;              /* RAC_K_INV, rac_cpu.h:39 */
static const float ORC_LN2 = 0.69314718056f;          /* rac_alu.c:558 */
static const float ORC_INV_LN2 = 1.44269504089f;      /* rac_alu.c:559 */

/* K-hat(n): the reference's circular-gain table, value for value
 * (rac_kernels.hip:42-50 == rac_cpu.c:44-52).  It is NOT the textbook
 * prod sqrt(1+4^-i) beyond n=2 (e.g. K-hat(16) = 1.64675049 vs
 * 1.64676026), and CORDIC-mode matmul results depend on it, so it is data. */
static const float ORC_KHAT[25] = {
    1.00000000f, 1.41421356f, 1.58113883f, 1.62979295f,
    1.64248460f, 1.64568447f, 1.64648404f, 1.64668388f,
    1.64673383f, 1.64674632f, 1.64674944f, 1.64675022f,
    1.64675042f, 1.64675047f, 1.64675048f, 1.64675049f,
    1.64675049f, 1.64675049f, 1.64675049f, 1.64675049f,
    1.64675049f, 1.64675049f, 1.64675049f, 1.64675049f,
    1.64675049f,
};

/* atan(2^-i), i = 0..23: the reference table (rac_cpu.c:20-40,
 * rac_kernels.hip:32-39) is each value printed to 8 decimals; the same
 * construction is applied here ("%.8f" then strtof) and
 * tests/test_oracle.py checks it against the compiled reference's table. */
static float orc_atan[24];

/* atanh(2^-s), s = 1..16: the reference's values (rac_cpu.c:27-32), kept as
 * data because they are not one rounding rule (s = 5, 7, 8 are truncated to
 * 8 decimals, s = 9 is rounded) and CORDIC exp results depend on them.
 * s = 17..24 have no reference counterpart (its table stops at 16); those
 * entries are the correctly rounded float atanh(2^-s), filled at init. */
static float orc_atanh[25] = {
    0.0f,
    0.54930614f, 0.25541281f, 0.12565721f, 0.06258157f,
    0.03126017f, 0.01562627f, 0.00781265f, 0.00390626f,
    0.00195313f, 0.00097656f, 0.00048828f, 0.00024414f,
    0.00012207f, 0.00006104f, 0.00003052f, 0.00001526f,
};
static int orc_tables_ready = 0;

static float eight_decimals(double v)
{
    char buf[64];
    snprintf(buf, sizeof buf, "%.8f", v);
    return strtof(buf, NULL);
}

static void orc_init(void)
{
    if (orc_tables_ready) return;
    for (int i = 0; i < 24; i++) orc_atan[i] = eight_decimals(atan(ldexp(1.0, -i)));
    for (int s = 17; s <= 24; s++) orc_atanh[s] = (float)atanh(ldexp(1.0, -s));
    orc_tables_ready = 1;
}

ORC_API void orc_tables(float *atan24, float *atanh24, float *khat25)
{
    orc_init();
    for (int i = 0; i < 24; i++) atan24[i] = orc_atan[i];
    for (int s = 1; s <= 24; s++) atanh24[s - 1] = orc_atanh[s];
    for (int i = 0; i < 25; i++) khat25[i] = ORC_KHAT[i];
}

static int clamp_iters_launch(int iters)      /* rac_kernels.hip:816-820 */
{
    if (iters < 1) return 1;
    if (iters > 24) return 24;
    return iters;
}

/* ── Circular CORDIC ────────────────────────────────────────────────────── */

/* rac_cordic_rotate_n, rac_kernels.hip:140-165 (same steps as _cordic_rotate,
 * rac_cpu.c:90-118): sequential float wrap into (-pi, pi], pre-rotation by
 * +-pi for |theta| > pi/2, then `iters` micro-rotations whose direction is
 * the sign of the residual angle. */
ORC_API void orc_cordic_rotate(float vx, float vy, float theta, int iters,
                               float *ox, float *oy)
{
    orc_init();
    /* The reference loop below never terminates for |theta| >= 2^27 or
     * +-inf (theta - TAU rounds back to theta); both sides return NaN. */
    if (!(fabsf(theta) < 134217728.0f)) { *ox = *oy = NAN; return; }
    while (theta > ORC_PI) theta -= ORC_TAU;
    while (theta <= -ORC_PI) theta += ORC_TAU;
    float x = vx, y = vy;
    if (theta > ORC_PI * 0.5f) { x = -x; y = -y; theta -= ORC_PI; }
    else if (theta < -ORC_PI * 0.5f) { x = -x; y = -y; theta += ORC_PI; }
    float angle = theta, scale = 1.0f;
    int lim = clamp_iters_launch(iters);
    for (int i = 0; i < lim; i++) {
        float d = (angle >= 0.0f) ? 1.0f : -1.0f;
        float xn = x - d * y * scale;
        float yn = y + d * x * scale;
        angle -= d * orc_atan[i];
        x = xn;
        y = yn;
        scale *= 0.5f;
    }
    *ox = x;
    *oy = y;
}

/* Direction sequence of a rotation that starts at angle 0 (the only angle
 * CORDIC-mode matmul ever uses after its +-pi pre-rotation): the "angle-index"
 * stage, data independent.  d[i] = +1 / -1.  rac_kernels.hip:152-159. */
ORC_API void orc_cordic_dirs(int iters, int *d)
{
    orc_init();
    float angle = 0.0f;
    int lim = clamp_iters_launch(iters);
    for (int i = 0; i < lim; i++) {
        float di = (angle >= 0.0f) ? 1.0f : -1.0f;
        d[i] = (di > 0.0f) ? 1 : -1;
        angle -= di * orc_atan[i];
    }
}

/* ── Matmul MAC semantics (A3-A5) ───────────────────────────────────────── */

/* 1.0f / K-hat(n), the gain compensation of rac_fma_cordic
 * (rac_kernels.hip:182-183), correctly rounded. */
ORC_API float orc_cordic_kinv(int iters)
{
    return 1.0f / ORC_KHAT[clamp_iters_launch(iters)];
}

/* rac_fma_cordic, rac_kernels.hip:177-185, literally: b is encoded as the
 * angle 0 (b >= +0) or pi (sign bit set) and |b|; (a, 0) is rotated by that
 * angle with `iters` micro-rotations; the x output, gain compensated, is
 * projected onto |b| and accumulated with one fused multiply-add. */
ORC_API float orc_fma_cordic(float a, float b, float acc, int iters)
{
    uint32_t bi;
    memcpy(&bi, &b, 4);
    uint32_t mi = bi & 0x7FFFFFFFu;
    float mag_b;
    memcpy(&mag_b, &mi, 4);
    float angle_b = (bi & 0x80000000u) ? 3.14159265358979f : 0.0f;
    float rx, ry;
    orc_cordic_rotate(a, 0.0f, angle_b, iters, &rx, &ry);
    return fmaf(rx * orc_cordic_kinv(iters), mag_b, acc);
}

/* Projection P_n(a) = R_n(a) * (1/K-hat(n)) of one A element: the x output of
 * `iters` micro-rotations of (a, 0) at angle 0, gain compensated.  Because
 * IEEE round-to-nearest is odd-symmetric, rotating (-a, -0) gives exactly
 * -R_n(a), so rac_fma_cordic(a, b, acc) == fmaf(P_n(a), b, acc) up to the
 * sign of an exact zero; tests/test_oracle.py checks this identity
 * exhaustively over the float mantissas. */
ORC_API float orc_cordic_project(float a, int iters)
{
    float rx, ry;
    orc_cordic_rotate(a, 0.0f, 0.0f, iters, &rx, &ry);
    return rx * orc_cordic_kinv(iters);
}

/* The micro-rotation chain as the gfx950 kernel evaluates it (strength
 * reduced but bit-identical for every finite a whose intermediate products
 * stay normal): micro-rotation 0 maps (a, 0) to (a, a); micro-rotation 1
 * gives x = fl(1.5 a) and y = a/2 exactly, so y is carried as yh = 2y = a;
 * every later micro-rotation is two FMAs on (x, yh) with the power-of-two
 * constants rescaled by the carried factor 2.  The last y update is unused.
 * tests/test_oracle.py compares this with orc_cordic_rotate for all 2^23
 * mantissas at iters 1..24. */
ORC_API float orc_cordic_chain_fast(float a, int iters)
{
    int lim = clamp_iters_launch(iters);
    int d[24];
    orc_cordic_dirs(lim, d);
    if (lim == 1) return a;
    float x = a * 1.5f;           /* fl(a + a/2): micro-rotation 1, d1 = -1 */
    float yh = a;                 /* 2 * (a - a/2) */
    for (int i = 2; i < lim; i++) {
        float s = ldexpf(1.0f, -i);
        float cx = -(float)d[i] * s * 0.5f;   /* -d_i 2^-i applied to y = yh/2 */
        float cy = (float)d[i] * s * 2.0f;    /* 2 * d_i 2^-i */
        float xn = fmaf(cx, yh, x);
        float yn = fmaf(cy, x, yh);
        x = xn;
        yh = yn;
    }
    return x;
}

/* rac_shiftadd_mul, rac_kernels.hip:85-122, literally (integer shift-add
 * product of the top `iters` bits of |b|'s mantissa with |a|'s mantissa,
 * truncating normalisation, sub-/super-normal results flushed to 0). */
ORC_API float orc_shiftadd_mul(float a, float b, int iters)
{
    if (a == 0.0f || b == 0.0f) return 0.0f;
    uint32_t ai, bi;
    memcpy(&ai, &a, 4);
    memcpy(&bi, &b, 4);
    uint32_t sign = (ai ^ bi) & 0x80000000u;
    int exp_a = (int)((ai >> 23) & 0xFFu) - 127;
    int exp_b = (int)((bi >> 23) & 0xFFu) - 127;
    uint32_t ma = 0x00800000u | (ai & 0x007FFFFFu);
    uint32_t mb = 0x00800000u | (bi & 0x007FFFFFu);
    uint64_t prod = 0;
    int lim = iters < 1 ? 1 : (iters > 24 ? 24 : iters);
    for (int i = 0; i < lim; i++) {
        uint32_t bit = (mb >> (23 - i)) & 1u;
        if (bit) prod += ((uint64_t)ma) << (23 - i);
    }
    if (prod == 0) return 0.0f;
    int top = 63 - __builtin_clzll(prod);
    int shift_r = top - 23;
    uint32_t mantissa;
    if (shift_r > 0) mantissa = (uint32_t)(prod >> shift_r) & 0x007FFFFFu;
    else if (shift_r < 0) mantissa = (uint32_t)(prod << -shift_r) & 0x007FFFFFu;
    else mantissa = (uint32_t)prod & 0x007FFFFFu;
    int rexp = exp_a + exp_b + (top - 46) + 127;
    if (rexp <= 0 || rexp >= 0xFF) return 0.0f;
    uint32_t bits = sign | ((uint32_t)(rexp & 0xFF) << 23) | mantissa;
    float r;
    memcpy(&r, &bits, 4);
    return r;
}

/* rac_fma_iters, rac_kernels.hip:204-219: mode 0 FAST (sign-XOR FMA, equal to
 * fmaf(a, b, acc)), 1 CORDIC, 2 SHIFTADD. */
ORC_API float orc_fma_iters(float a, float b, float acc, int iters, int mode)
{
    if (mode == 0) {
        uint32_t ai, bi;
        memcpy(&ai, &a, 4);
        memcpy(&bi, &b, 4);
        uint32_t pi = ai ^ (bi & 0x80000000u), mi = bi & 0x7FFFFFFFu;
        float proj, mag;
        memcpy(&proj, &pi, 4);
        memcpy(&mag, &mi, 4);
        return fmaf(proj, mag, acc);
    }
    if (mode == 1) return orc_fma_cordic(a, b, acc, iters);
    return acc + orc_shiftadd_mul(a, b, iters);
}

static inline float mat_at(const float *X, int trans, int rows, int cols,
                           int r, int c)
{
    /* logical X[r][c] of a rows x cols operand; trans: stored as [cols][rows] */
    return trans ? X[(size_t)c * rows + r] : X[(size_t)r * cols + c];
}

/* One output of rac_launch_{nn,nt,tn}_iters (rac_kernels.hip:822-883):
 * acc accumulates over k = 0..K-1 in order (every reference tile shape keeps
 * one accumulator per output over the whole K), then
 * C = alpha*acc (beta == 0) or fmaf(alpha, acc, beta*C) (:267-272).
 * `literal` = 1 runs orc_fma_iters per MAC; 0 uses the projection identity
 * (CORDIC: fmaf(P_n(a), b, acc)), which is bit-identical and fast. */
static float mm_entry(int ta, int tb, const float *A, const float *B,
                      const float *C, int M, int N, int K, int i, int j,
                      float alpha, float beta, int iters, int mode,
                      const float *projA, int literal)
{
    float acc = 0.0f;
    for (int k = 0; k < K; k++) {
        float a = mat_at(A, ta, M, K, i, k);
        float b = mat_at(B, tb, K, N, k, j);
        if (literal || mode != 1) acc = orc_fma_iters(a, b, acc, iters, mode);
        else {
            float p = projA ? projA[ta ? (size_t)k * M + i : (size_t)i * K + k]
                            : orc_cordic_project(a, iters);
            acc = fmaf(p, b, acc);
        }
    }
    float c0 = C ? C[(size_t)i * N + j] : 0.0f;
    return (beta != 0.0f) ? fmaf(alpha, acc, beta * c0) : alpha * acc;
}

/* Full product.  ta: A stored [K,M] (the TN launcher), tb: B stored [N,K]
 * (the NT launcher).  C is read when beta != 0. */
ORC_API int orc_matmul(int ta, int tb, const float *A, const float *B, float *C,
                       int M, int N, int K, float alpha, float beta,
                       int iters, int mode, int literal)
{
    if (!A || !B || !C) return -1;
    if (M <= 0 || N <= 0 || K <= 0) return -2;
    iters = clamp_iters_launch(iters);
    float *projA = NULL;
    if (mode == 1 && !literal) {
        projA = (float *)malloc((size_t)M * K * sizeof(float));
        if (!projA) return -3;
        for (size_t t = 0; t < (size_t)M * K; t++) projA[t] = orc_cordic_project(A[t], iters);
    }
    float *out = (float *)malloc((size_t)M * N * sizeof(float));
    if (!out) { free(projA); return -3; }
    #pragma omp parallel for schedule(dynamic)
    for (int i = 0; i < M; i++)
        for (int j = 0; j < N; j++)
            out[(size_t)i * N + j] = mm_entry(ta, tb, A, B, C, M, N, K, i, j,
                                              alpha, beta, iters, mode, projA, literal);
    memcpy(C, out, (size_t)M * N * sizeof(float));
    free(out);
    free(projA);
    return 0;
}

/* Selected outputs only (rows[t], cols[t]) — for large shapes. */
ORC_API int orc_matmul_entries(int ta, int tb, const float *A, const float *B,
                               int M, int N, int K, int iters, int mode,
                               const int *rows, const int *cols, int count,
                               float *out)
{
    iters = clamp_iters_launch(iters);
    #pragma omp parallel for schedule(dynamic)
    for (int t = 0; t < count; t++)
        out[t] = mm_entry(ta, tb, A, B, NULL, M, N, K, rows[t], cols[t],
                          1.0f, 0.0f, iters, mode, NULL, 0);
    return 0;
}

/* ── RoPE (A6, A9, A10) ─────────────────────────────────────────────────── */

/* inv_freq[i] = 1.0f / powf(base, (2.0f*i)/head_dim), rac_cpu.c:588-589. */
ORC_API void orc_rope_inv_freq(float *inv_freq, int head_dim, float base)
{
    int half = head_dim / 2;
    for (int i = 0; i < half; i++) {
        float exponent = (2.0f * (float)i) / (float)head_dim;
        inv_freq[i] = 1.0f / powf(base, exponent);
    }
}

/* rac_sincos, rac_cpu.c:322-328: one 16-iteration rotation of (K_INV, 0). */
ORC_API void orc_sincos(float theta, float *s, float *c)
{
    float x, y;
    orc_cordic_rotate(ORC_K_INV, 0.0f, theta, 16, &x, &y);
    *c = x;
    *s = y;
}

/* orc_sincos over an array (test sweeps). */
ORC_API void orc_sincos_batch(const float *theta, float *s, float *c, long count)
{
    #pragma omp parallel for schedule(dynamic, 4096)
    for (long i = 0; i < count; i++) orc_sincos(theta[i], &s[i], &c[i]);
}

/* rac_rope_cache, rac_cpu.c:576-598 (angle = (float)p * inv_freq[i]). */
ORC_API int orc_rope_cache(float *cos_out, float *sin_out, int max_seq,
                           int head_dim, float base)
{
    if (!cos_out || !sin_out) return -1;
    if (max_seq <= 0 || head_dim <= 0 || (head_dim & 1)) return -2;
    int half = head_dim / 2;
    float *inv = (float *)malloc((size_t)half * sizeof(float));
    if (!inv) return -3;
    orc_rope_inv_freq(inv, head_dim, base);
    #pragma omp parallel for schedule(static)
    for (int p = 0; p < max_seq; p++)
        for (int i = 0; i < half; i++) {
            float s, c;
            orc_sincos((float)p * inv[i], &s, &c);
            cos_out[(size_t)p * half + i] = c;
            sin_out[(size_t)p * half + i] = s;
        }
    free(inv);
    return 0;
}

/* rac_rope_apply, rac_cpu.c:600-635, generalised to element strides so the
 * [B,T,H,D] view used by attention is covered too (contiguous [B,H,T,D]:
 * sb = H*T*D, sh = T*D, st = D). */
ORC_API int orc_rope_apply_strided(float *x, const float *cos_tab, const float *sin_tab,
                                   int batch, int n_heads, int seq, int head_dim,
                                   long sb, long sh, long st)
{
    if (!x || !cos_tab || !sin_tab) return -1;
    if (batch <= 0 || n_heads <= 0 || seq <= 0 || head_dim <= 0 || (head_dim & 1))
        return -2;
    int half = head_dim / 2;
    #pragma omp parallel for collapse(3) schedule(static)
    for (int b = 0; b < batch; b++)
        for (int h = 0; h < n_heads; h++)
            for (int t = 0; t < seq; t++) {
                float *row = x + b * sb + h * sh + t * st;
                const float *cr = cos_tab + (size_t)t * half;
                const float *sr = sin_tab + (size_t)t * half;
                for (int i = 0; i < half; i++) {
                    float a = row[2 * i], b2 = row[2 * i + 1];
                    float c = cr[i], s = sr[i];
                    row[2 * i] = fmaf(a, c, -b2 * s);
                    row[2 * i + 1] = fmaf(a, s, b2 * c);
                }
            }
    return 0;
}

ORC_API int orc_rope_apply(float *x, const float *cos_tab, const float *sin_tab,
                           int batch, int n_heads, int seq, int head_dim)
{
    long st = head_dim, sh = (long)seq * head_dim, sb = (long)n_heads * sh;
    return orc_rope_apply_strided(x, cos_tab, sin_tab, batch, n_heads, seq,
                                  head_dim, sb, sh, st);
}

/* ── Hyperbolic CORDIC (A7) ─────────────────────────────────────────────── */

/* Walther shift schedule: 1, 2, 3, 4, 4, 5, ..., 13, 13, 14, ..., 40, 40, ...
 * (the repeats keep the non-restoring iteration convergent), first n shifts.
 * For n = 16 this is rac_hip.cpp:168 / rac_alu.c:57-59. */
ORC_API int orc_hyp_schedule(int n, int *shifts)
{
    int s = 1, j = 0, next_repeat = 4;
    while (j < n) {
        shifts[j++] = s;
        if (s == next_repeat && j < n) {
            shifts[j++] = s;
            next_repeat = 3 * next_repeat + 1;
        }
        s++;
    }
    return n;
}

/* 1 / K_h(n), K_h(n) = prod_j sqrt(1 - 4^-s_j), rounded once to float.
 * (rac_alu.c:572 uses RAC_K_HYP_INV = 1.2074970f for n = 16; the exact
 * product rounds to 1.2074971f — one ulp apart; orc_exp_xy takes the
 * constant as a parameter so both are reproducible.) */
ORC_API float orc_hyp_kinv(int n)
{
    int sh[64];
    if (n > 64) n = 64;
    orc_hyp_schedule(n, sh);
    double k = 1.0;
    for (int j = 0; j < n; j++) k *= sqrt(1.0 - ldexp(1.0, -2 * sh[j]));
    return (float)(1.0 / k);
}

static int clamp_iters_hyp(int n)
{
    if (n < 1) return 1;
    if (n > 24) return 24;
    return n;
}

/* Range reduction of rac_alu_exp, rac_alu.c:560-561, in the fused form the
 * reference's own build produces (gcc contracts both lines to FMAs):
 * k = trunc(fma(x, 1/ln2, +-0.5)), r = fma(-k, ln2, x).  The truncation
 * argument is clamped to +-2^30 so huge |x| saturate instead of wrapping. */
static void exp_reduce(float x, int *k_out, float *r_out)
{
    float t = fmaf(x, ORC_INV_LN2, (x >= 0.0f) ? 0.5f : -0.5f);
    if (t > 1073741824.0f) t = 1073741824.0f;
    if (t < -1073741824.0f) t = -1073741824.0f;
    int k = (int)t;
    *k_out = k;
    *r_out = fmaf(-(float)k, ORC_LN2, x);
}

/* 2^k applied through the exponent field, rac_alu.c:576-581. */
static float exp_scale(float er, int k)
{
    int bias_k = k + 127;
    if (bias_k < 0) return 0.0f;
    if (bias_k > 254) return er * INFINITY;
    uint32_t u = (uint32_t)bias_k << 23;
    float f;
    memcpy(&f, &u, 4);
    return er * f;
}

/* Hyperbolic CORDIC e^x in x/y-register form: rac_alu_exp (rac_alu.c:550-582,
 * rotation core rac_alu.c:256-270 with d = copysign(1, z)), generalised from
 * 16 to n steps of the Walther schedule. */
ORC_API float orc_exp_xy(float xin, int n, float khinv)
{
    orc_init();
    if (xin != xin) return xin;
    n = clamp_iters_hyp(n);
    int sh[24];
    orc_hyp_schedule(n, sh);
    int k;
    float r;
    exp_reduce(xin, &k, &r);
    float x = 1.0f, y = 0.0f, z = r;
    for (int j = 0; j < n; j++) {
        float d = copysignf(1.0f, z);
        float ds = d * ldexpf(1.0f, -sh[j]);
        float xn = x + ds * y;
        float yn = y + ds * x;
        z -= d * orc_atanh[sh[j]];
        x = xn;
        y = yn;
    }
    return exp_scale((x + y) * khinv, k);
}

/* Hyperbolic CORDIC e^x as the gfx950 kernels compute it: the sum register
 * p = x + y of the same rotation, which evolves on its own as
 * p <- p * (1 + d_j 2^-s_j) (x' + y' = (x + y)(1 + d s) for the hyperbolic
 * step), one fused multiply-add per micro-rotation; the residual angle is
 * updated as z <- fma(-d 2^-s, atanh(2^-s) 2^s, z), which equals
 * z - d*atanh(2^-s) exactly.  Directions d = copysign(1, z) as in
 * rac_alu.c:246; output (p / K_h(n)) * 2^k as rac_alu.c:572-581. */
ORC_API float orc_exp_n(float xin, int n)
{
    orc_init();
    if (xin != xin) return xin;
    n = clamp_iters_hyp(n);
    int sh[24];
    orc_hyp_schedule(n, sh);
    int k;
    float r;
    exp_reduce(xin, &k, &r);
    float p = 1.0f, z = r;
    for (int j = 0; j < n; j++) {
        float s = ldexpf(1.0f, -sh[j]);
        float ds = copysignf(s, z);
        float c = ldexpf(orc_atanh[sh[j]], sh[j]);
        p = fmaf(ds, p, p);
        z = fmaf(-ds, c, z);
    }
    return exp_scale(p * orc_hyp_kinv(n), k);
}

ORC_API void orc_exp_batch(const float *x, float *y, long count, int n)
{
    #pragma omp parallel for schedule(static)
    for (long i = 0; i < count; i++) y[i] = orc_exp_n(x[i], n);
}

/* Row softmax, rac_cpu.c:258-271 (max; e = exp(x - max) with a sequential
 * float sum; multiply by 1.0f/sum), with exp = orc_exp_n(., iters), or libm
 * expf when iters <= 0 (then it is rac_softmax_batch exactly). */
ORC_API void orc_softmax_rows(const float *x, float *out, int rows, int n, int iters)
{
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (size_t)r * n;
        float *o = out + (size_t)r * n;
        float m = xr[0];
        for (int i = 1; i < n; i++) if (xr[i] > m) m = xr[i];
        float sum = 0.0f;
        for (int i = 0; i < n; i++) {
            o[i] = (iters > 0) ? orc_exp_n(xr[i] - m, iters) : expf(xr[i] - m);
            sum += o[i];
        }
        float inv = 1.0f / sum;
        for (int i = 0; i < n; i++) o[i] *= inv;
    }
}

/* ── rsqrt by hyperbolic vectoring (A11) ────────────────────────────────── */

/* rac_rsqrt's contract (rac_cpu.c:330-335: x <= 0 -> 0, NaN -> NaN,
 * +inf -> 0) computed the way rac_cpu.h:123-130 describes it: v = m 4^e with
 * m in [0.5, 2) from the exponent field; hyperbolic vectoring of
 * (m + 1/4, m - 1/4) drives y to 0 and leaves x = K_h sqrt(m) (since
 * (m+1/4)^2 - (m-1/4)^2 = m); sqrt(m) = x / K_h; 1/sqrt(m) by one IEEE
 * division; 2^-e by the exponent.  The vectoring magnitude converges
 * quadratically in the residual angle, so the fixed 16-step Walther
 * schedule (last shift 14) is at float precision. */
#define ORC_RSQRT_STEPS 16
ORC_API float orc_rsqrt(float v)
{
    if (v != v) return v;
    if (!(v > 0.0f)) return 0.0f;
    if (isinf(v)) return 0.0f;
    int ex;
    float mant = frexpf(v, &ex);          /* v = mant 2^ex, mant in [0.5, 1) */
    float m;
    int e;
    if (ex & 1) { m = mant * 2.0f; e = (ex - 1) / 2; }
    else { m = mant; e = ex / 2; }
    int sh[ORC_RSQRT_STEPS];
    orc_hyp_schedule(ORC_RSQRT_STEPS, sh);
    float X = m + 0.25f, Y = m - 0.25f;
    for (int j = 0; j < ORC_RSQRT_STEPS; j++) {
        float ds = copysignf(ldexpf(1.0f, -sh[j]), Y);   /* d = -sign(Y) */
        float Xn = fmaf(-ds, Y, X);
        float Yn = fmaf(-ds, X, Y);
        X = Xn;
        Y = Yn;
    }
    float root = X * orc_hyp_kinv(ORC_RSQRT_STEPS);
    float r = 1.0f / root;
    return ldexpf(r, -e);
}

/* orc_rsqrt over an array (test sweeps). */
ORC_API void orc_rsqrt_batch(const float *x, float *y, long count)
{
    #pragma omp parallel for schedule(static)
    for (long i = 0; i < count; i++) y[i] = orc_rsqrt(x[i]);
}

/* rac_rmsnorm, rac_cpu.c:548-574: ms = sequential fmaf(x,x,ms), ms /= d,
 * inv = rsqrt(ms + eps), y = (x*inv)*g.  use_cordic selects orc_rsqrt
 * (product semantics) or 1.0f/sqrtf (the reference's libm rsqrt). */
static float rsqrt_sel(float v, int use_cordic)
{
    if (use_cordic) return orc_rsqrt(v);
    if (v <= 0.0f) return 0.0f;
    return 1.0f / sqrtf(v);
}

ORC_API int orc_rmsnorm(const float *x, float *y, const float *gamma, float eps,
                        int rows, int d, int use_cordic)
{
    if (!x || !y) return -1;
    if (rows <= 0 || d <= 0) return -2;
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (size_t)r * d;
        float *yr = y + (size_t)r * d;
        float ms = 0.0f;
        for (int i = 0; i < d; i++) ms = fmaf(xr[i], xr[i], ms);
        ms /= (float)d;
        float inv = rsqrt_sel(ms + eps, use_cordic);
        for (int i = 0; i < d; i++) {
            float g = gamma ? gamma[i] : 1.0f;
            yr[i] = xr[i] * inv * g;
        }
    }
    return 0;
}

/* rac_layernorm, rac_cpu.c:507-546. */
ORC_API int orc_layernorm(const float *x, float *y, const float *gamma,
                          const float *beta, float eps, int rows, int d,
                          int use_cordic)
{
    if (!x || !y) return -1;
    if (rows <= 0 || d <= 0) return -2;
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (size_t)r * d;
        float *yr = y + (size_t)r * d;
        float mean = 0.0f;
        for (int i = 0; i < d; i++) mean += xr[i];
        mean /= (float)d;
        float var = 0.0f;
        for (int i = 0; i < d; i++) {
            float z = xr[i] - mean;
            var = fmaf(z, z, var);
        }
        var /= (float)d;
        float inv = rsqrt_sel(var + eps, use_cordic);
        for (int i = 0; i < d; i++) {
            float z = (xr[i] - mean) * inv;
            float g = gamma ? gamma[i] : 1.0f;
            float b = beta ? beta[i] : 0.0f;
            yr[i] = fmaf(g, z, b);
        }
    }
    return 0;
}

/* ── Row sums in the gfx950 row kernels' order ────────────────────────────
 * orc_rmsnorm, orc_layernorm and orc_softmax_rows add a row left to right,
 * as rac_cpu.c does.  The device row kernels add it as a tree: 256 lanes,
 * lane l owning the float4 groups l, l + 256, l + 512, ... (VPT groups, VPT
 * the smallest of 1, 2, 4, 8, 16 with n/4 <= 256 VPT; rows with n % 4 != 0
 * or n/4 > 4096 are owned element-wise, lane l taking elements l, l + 256,
 * ...), each lane adding its own elements in that order; then the 64 lanes
 * of each wave combine by a butterfly (lane l adds lane l ^ 32, then l ^ 16,
 * ..., l ^ 1; IEEE addition commutes, so both partners hold the same sum)
 * and the four wave sums are added in wave order.  The *_lanes functions
 * below are the same computations as their left-to-right counterparts with
 * only the row sums regrouped that way, so the GPU kernels can be checked
 * bit for bit instead of within a reordering bound.  Every other rounding
 * (max, CORDIC exp, rsqrt, the output products) is the one of the
 * counterpart.  Pinned in tests/test_oracle.py: equal to the left-to-right
 * versions where every partial sum is exact, and within the reordering
 * bound of them otherwise. */

#define ORC_ROW_LANES 256

/* Number of elements (slots) each lane owns in a row of n (the owner map
 * above). */
static int row_slots(int n)
{
    int n4 = n / 4;
    if (n % 4 == 0) {
        for (int vpt = 1; vpt <= 16; vpt *= 2)
            if (n4 <= ORC_ROW_LANES * vpt) return 4 * vpt;
    }
    return (n + ORC_ROW_LANES - 1) / ORC_ROW_LANES;
}

/* Butterfly within each wave of 64 lanes, then the 4 wave sums in order. */
static float lanes_combine(const float *lane)
{
    float red[ORC_ROW_LANES / 64];
    for (int w = 0; w < ORC_ROW_LANES / 64; w++) {
        float v[64], t[64];
        memcpy(v, lane + 64 * w, sizeof v);
        for (int off = 32; off > 0; off >>= 1) {
            for (int l = 0; l < 64; l++) t[l] = v[l] + v[l ^ off];
            memcpy(v, t, sizeof v);
        }
        red[w] = v[0];
    }
    float r = red[0];
    for (int w = 1; w < ORC_ROW_LANES / 64; w++) r += red[w];
    return r;
}

/* The element index held in (lane, slot), or -1 past the row end. */
static int row_elem(int n, int lane, int slot)
{
    int n4 = n / 4;
    if (n % 4 == 0 && n4 <= ORC_ROW_LANES * 16) {
        int g = lane + ORC_ROW_LANES * (slot / 4);
        return g < n4 ? 4 * g + slot % 4 : -1;
    }
    int i = lane + ORC_ROW_LANES * slot;
    return i < n ? i : -1;
}

/* sum over the row of f(i) in lane order; f(i) of a missing element
 * contributes nothing (the kernels' padding adds +0 or is skipped). */
#define ROW_LANE_SUM(n, result, ACC_INIT, ACC_STEP)                           \
    do {                                                                      \
        float lane_[ORC_ROW_LANES];                                           \
        int slots_ = row_slots(n);                                            \
        for (int l_ = 0; l_ < ORC_ROW_LANES; l_++) {                          \
            float acc = ACC_INIT;                                             \
            for (int s_ = 0; s_ < slots_; s_++) {                             \
                int i = row_elem(n, l_, s_);                                  \
                if (i >= 0) { ACC_STEP; }                                     \
            }                                                                 \
            lane_[l_] = acc;                                                  \
        }                                                                     \
        result = lanes_combine(lane_);                                        \
    } while (0)

/* rac_rmsnorm (rac_cpu.c:548-574) with the lane-order sum of squares. */
ORC_API int orc_rmsnorm_lanes(const float *x, float *y, const float *gamma, float eps, int rows, int d)
{
    if (!x || !y) return -1;
    if (rows <= 0 || d <= 0) return -2;
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (size_t)r * d;
        float *yr = y + (size_t)r * d;
        float ss;
        ROW_LANE_SUM(d, ss, 0.0f, acc = fmaf(xr[i], xr[i], acc));
        float inv = rsqrt_sel(ss / (float)d + eps, 1);
        for (int i = 0; i < d; i++) {
            float g = gamma ? gamma[i] : 1.0f;
            yr[i] = xr[i] * inv * g;
        }
    }
    return 0;
}

/* rac_layernorm (rac_cpu.c:507-546) with lane-order sums. */
ORC_API int orc_layernorm_lanes(const float *x, float *y, const float *gamma, const float *beta, float eps,
                                int rows, int d)
{
    if (!x || !y) return -1;
    if (rows <= 0 || d <= 0) return -2;
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (size_t)r * d;
        float *yr = y + (size_t)r * d;
        float sm, sv;
        ROW_LANE_SUM(d, sm, 0.0f, acc += xr[i]);
        float mean = sm / (float)d;
        ROW_LANE_SUM(d, sv, 0.0f, { float z = xr[i] - mean; acc = fmaf(z, z, acc); });
        float inv = rsqrt_sel(sv / (float)d + eps, 1);
        for (int i = 0; i < d; i++) {
            float z = (xr[i] - mean) * inv;
            float g = gamma ? gamma[i] : 1.0f;
            float b = beta ? beta[i] : 0.0f;
            yr[i] = fmaf(g, z, b);
        }
    }
    return 0;
}

/* Row softmax (rac_cpu.c:258-271; CORDIC exp of `iters` steps) with the
 * lane-order row sum.  With masking on (causal, an additive [seq, seq] mask
 * or the zero-sum guard, the attention form of rac_cpu.c:668-689), row r is
 * query position t = r % seq: causal sets -inf above the diagonal, then the
 * mask is added, and a non-positive sum gives inv = 0 when zero_guard. */
ORC_API int orc_softmax_lanes(const float *x, float *out, int rows, int n, int iters, int causal,
                              const float *mask, int zero_guard)
{
    if (!x || !out) return -1;
    if (rows <= 0 || n <= 0) return -2;
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (size_t)r * n;
        float *o = out + (size_t)r * n;
        int t = r % n;
        for (int i = 0; i < n; i++) {
            float v = xr[i];
            if (causal && i > t) v = -INFINITY;
            if (mask) v += mask[(size_t)t * n + i];
            o[i] = v;
        }
        float m = o[0];
        for (int i = 1; i < n; i++) if (o[i] > m) m = o[i];
        for (int i = 0; i < n; i++) o[i] = orc_exp_n(o[i] - m, iters);
        float s;
        ROW_LANE_SUM(n, s, 0.0f, acc += o[i]);
        float inv = (zero_guard && !(s > 0.0f)) ? 0.0f : 1.0f / s;
        for (int i = 0; i < n; i++) o[i] *= inv;
    }
    return 0;
}

/* ── Activations (A12) ──────────────────────────────────────────────────── */

/* rac_silu, rac_cpu.c:453-457: x / (1 + e^-x), with e^-x from the n-step
 * CORDIC (iters <= 0: libm expf, i.e. the reference exactly). */
ORC_API void orc_silu(const float *x, float *y, long count, int iters)
{
    #pragma omp parallel for schedule(static)
    for (long i = 0; i < count; i++) {
        float e = (iters > 0) ? orc_exp_n(-x[i], iters) : expf(-x[i]);
        y[i] = x[i] / (1.0f + e);
    }
}

/* rac_sigmoid's value 1 / (1 + e^-x) (rac_cpu.c:337-340 computes it as
 * 0.5*(1 + tanh(x/2)), the same function). */
ORC_API void orc_sigmoid(const float *x, float *y, long count, int iters)
{
    #pragma omp parallel for schedule(static)
    for (long i = 0; i < count; i++) {
        float e = (iters > 0) ? orc_exp_n(-x[i], iters) : expf(-x[i]);
        y[i] = 1.0f / (1.0f + e);
    }
}

/* rac_gelu, rac_cpu.c:447-451: x * 0.5 * (1 + erf(x / sqrt 2)). */
ORC_API void orc_gelu(const float *x, float *y, long count)
{
    #pragma omp parallel for schedule(static)
    for (long i = 0; i < count; i++)
        y[i] = x[i] * 0.5f * (1.0f + erff(x[i] * 0.7071067811865f));
}

/* tanh(x) = sign(x) (1 - e) / (1 + e), e = e^{-2|x|} from the n-step CORDIC
 * (iters <= 0: libm tanhf, rac_cpu.c:254-256). */
ORC_API void orc_tanh(const float *x, float *y, long count, int iters)
{
    #pragma omp parallel for schedule(static)
    for (long i = 0; i < count; i++) {
        if (iters <= 0) { y[i] = tanhf(x[i]); continue; }
        float e = orc_exp_n(-2.0f * fabsf(x[i]), iters);
        y[i] = copysignf((1.0f - e) / (1.0f + e), x[i]);
    }
}

/* ── Exhaustive checks used by tests/test_oracle.py ─────────────────────── */

static float lit_rotate_x(float a, float angle, int iters)
{
    float x, y;
    orc_cordic_rotate(a, 0.0f, angle, iters, &x, &y);
    return x;
}

/* For every float a = (1 + m 2^-23) 2^e, m = 0 .. 2^23-1: counts the a where
 * (i) the strength-reduced chain differs from the literal rotation, or
 * (ii) rotating by pi (rac_fma_cordic's encoding of a negative b) is not
 * exactly the negation of rotating by 0. */
ORC_API long orc_check_chain_all_mantissas(int iters, int e)
{
    long bad = 0;
    #pragma omp parallel for reduction(+:bad) schedule(static)
    for (long m = 0; m < (1L << 23); m++) {
        uint32_t u = ((uint32_t)(e + 127) << 23) | (uint32_t)m;
        float a;
        memcpy(&a, &u, 4);
        float lit = lit_rotate_x(a, 0.0f, iters);
        float fast = orc_cordic_chain_fast(a, iters);
        float neg = lit_rotate_x(a, 3.14159265358979f, iters);
        if (lit != fast || neg != -lit) bad++;
    }
    return bad;
}

/* rac_fma_cordic(a, b, acc) == fmaf(P(a), b, acc) on `count` random triples
 * (xorshift from `seed`; a, b spread over 2^-20 .. 2^20, acc over +-2^10). */
ORC_API long orc_check_projection_identity(int iters, long count, uint64_t seed)
{
    long bad = 0;
    for (long t = 0; t < count; t++) {
        float v[3];
        for (int j = 0; j < 3; j++) {
            seed ^= seed << 13; seed ^= seed >> 7; seed ^= seed << 17;
            uint32_t mant = (uint32_t)(seed & 0x7FFFFFu);
            int ex = (int)((seed >> 23) % 41) - 20;
            if (j == 2) ex = (int)((seed >> 23) % 21) - 10;
            uint32_t u = ((seed >> 40) & 1u ? 0x80000000u : 0u) | ((uint32_t)(ex + 127) << 23) | mant;
            memcpy(&v[j], &u, 4);
        }
        float lit = orc_fma_cordic(v[0], v[1], v[2], iters);
        float fast = fmaf(orc_cordic_project(v[0], iters), v[1], v[2]);
        if (lit != fast) bad++;
    }
    return bad;
}

/* ── Vector primitives of rac.h (rac.h:101-250, 345-346) ─────────────────
 * Restated from the CPU library's definitions (rac_cpu.c:136-228, 275-288,
 * 351-371), which reduce the angle to (-pi, pi] and pre-rotate left-half-
 * plane vectors, so they hold over the whole plane.  cosf/sinf/powf are
 * glibc's here and the device's own on the GPU (a few ulp apart); every
 * CORDIC step is exact in either. */

/* rac_polar, rac_cpu.c:158-180 (16 vectoring steps). */
ORC_API void orc_polar(float vx, float vy, float *mag, float *angle)
{
    orc_init();
    float pre = 0.0f;
    if (vx < 0.0f) {
        pre = (vy >= 0.0f) ? ORC_PI : -ORC_PI;
        vx = -vx;
        vy = -vy;
    }
    float x = vx, y = vy, z = 0.0f, scale = 1.0f;
    for (int i = 0; i < 16; i++) {
        float d = (y < 0.0f) ? 1.0f : -1.0f;
        float xn = x - d * y * scale;
        float yn = y + d * x * scale;
        z += d * orc_atan[i];
        x = xn;
        y = yn;
        scale *= 0.5f;
    }
    *mag = x * ORC_K_INV;
    *angle = pre - z;
}

/* rac_project, rac_cpu.c:150-154. */
ORC_API float orc_project(float vx, float vy, float theta)
{
    return fmaf(vx, cosf(theta), vy * sinf(theta));
}

static int clamp_prec(int iters)                 /* _clamp_iters, rac_cpu.c:54-58 */
{
    return iters < 4 ? 4 : (iters > 24 ? 24 : iters);
}

/* Elementwise primitive `op` over n items (the device library's op codes):
 *  0 rac_rotate        (rac_cpu.c:136-139)   a, th -> o2
 *  1 rac_rotate_raw    (:141-143)            a, th -> o2
 *  2 rac_compensate    (:145-148)            a, iarg -> o2
 *  3 rac_project       (:150-154)            a, th -> o1
 *  4 rac_polar         (:158-180)            a -> o2 = (mag, angle)
 *  5 rac_normalize     (:188-192)            a -> o2
 *  6 rac_dot           (:196-201)            a, b -> o1
 *  7 rac_coherence     (:203-208)            a, b -> o1
 *  8 rac_complex_mul   (:212-217)            a, b -> o2
 *  9 rac_rotate_n      (:275-280)            a, th, iarg -> o2
 * 10 rac_project_n     (:282-288)            a, th, iarg -> o1
 * 11 rac_inner's term  (:355-357)            a, b -> o1
 * a, b, o2 are interleaved (x, y) pairs. */
ORC_API void orc_prim(int op, long n, const float *a, const float *b, const float *th,
                      int iarg, float *o2, float *o1)
{
    orc_init();
    for (long i = 0; i < n; i++) {
        const float ax = a[2 * i], ay = a[2 * i + 1];
        float x = 0, y = 0, m, ang, mb, ab;
        switch (op) {
        case 0:
            orc_cordic_rotate(ax * ORC_K_INV, ay * ORC_K_INV, th[i], 16, &x, &y);
            o2[2 * i] = x; o2[2 * i + 1] = y;
            break;
        case 1:
            orc_cordic_rotate(ax, ay, th[i], 16, &x, &y);
            o2[2 * i] = x; o2[2 * i + 1] = y;
            break;
        case 2: {
            const float c = powf(ORC_K_INV, (float)iarg);
            o2[2 * i] = ax * c; o2[2 * i + 1] = ay * c;
            break;
        }
        case 3:
            o1[i] = orc_project(ax, ay, th[i]);
            break;
        case 4:
            orc_polar(ax, ay, &m, &ang);
            o2[2 * i] = m; o2[2 * i + 1] = ang;
            break;
        case 5:
            orc_polar(ax, ay, &m, &ang);
            o2[2 * i] = cosf(ang); o2[2 * i + 1] = sinf(ang);
            break;
        case 6:
            orc_polar(ax, ay, &m, &ang);
            orc_polar(b[2 * i], b[2 * i + 1], &mb, &ab);
            o1[i] = m * mb * cosf(ang - ab);
            break;
        case 7:
            orc_polar(ax, ay, &m, &ang);
            orc_polar(b[2 * i], b[2 * i + 1], &mb, &ab);
            o1[i] = cosf(ang - ab);
            break;
        case 8:
            orc_polar(b[2 * i], b[2 * i + 1], &mb, &ab);
            orc_cordic_rotate(ax * ORC_K_INV, ay * ORC_K_INV, ab, 16, &x, &y);
            o2[2 * i] = x * mb; o2[2 * i + 1] = y * mb;
            break;
        case 9: {
            const int it = clamp_prec(iarg);
            const float kinv = 1.0f / ORC_KHAT[it];
            orc_cordic_rotate(ax * kinv, ay * kinv, th[i], it, &x, &y);
            o2[2 * i] = x; o2[2 * i + 1] = y;
            break;
        }
        case 10: {
            const int it = clamp_prec(iarg);
            orc_cordic_rotate(1.0f / ORC_KHAT[it], 0.0f, th[i], it, &x, &y);
            o1[i] = fmaf(ax, x, ay * y);
            break;
        }
        case 11:
            orc_polar(b[2 * i], b[2 * i + 1], &mb, &ab);
            o1[i] = orc_project(ax, ay, ab) * mb;
            break;
        default:
            break;
        }
    }
}

/* rac_outer, rac_cpu.c:362-371. */
ORC_API void orc_outer(const float *a, const float *b, float *C, int m, int n)
{
    for (int i = 0; i < m; i++)
        for (int j = 0; j < n; j++) {
            float mb, ab;
            orc_polar(b[2 * j], b[2 * j + 1], &mb, &ab);
            C[(size_t)i * n + j] = orc_project(a[2 * i], a[2 * i + 1], ab) * mb;
        }
}

/* rac_dct, rac_cpu.c:219-228 (sum in order i = 0..n-1). */
ORC_API void orc_dct(const float *x, float *X, int n)
{
    for (int k = 0; k < n; k++) {
        float sum = 0.0f;
        for (int i = 0; i < n; i++) {
            float theta = ORC_PI * (float)(2 * i + 1) * (float)k / (float)(2 * n);
            sum += orc_project(x[i], 0.0f, theta);
        }
        X[k] = sum;
    }
}

/* ── Scaled dot-product attention (rac.h:323-335) ──────────────────────────
 * The reference CPU definition (rac_cpu.c:637-703) per (batch, head):
 * scores[t,s] = (sum_d fmaf q.k) * (1/sqrtf(D)); causal -> -inf for s > t;
 * then += mask[t*T+s]; row softmax with inv = sum > 0 ? 1/sum : 0; then
 * out[t,d] = sum_s fmaf(p, v).  rac.h asks for every stage through the RAC
 * primitives: the two products are rac_matmul (orc_matmul with `mode`,
 * `iters`) and exp is the CORDIC exp of `iters` steps; iters <= 0 selects
 * expf, which with mode 0 (FAST == fmaf) reproduces rac_cpu.c exactly. */
ORC_API int orc_attention(const float *q, const float *k, const float *v, const float *mask,
                          int is_causal, float *out, int batch, int heads, int seq, int dim,
                          int iters, int mode)
{
    if (!q || !k || !v || !out) return -1;
    if (batch <= 0 || heads <= 0 || seq <= 0 || dim <= 0) return -2;
    const float scale = 1.0f / sqrtf((float)dim);
    const size_t tt = (size_t)seq * seq, td = (size_t)seq * dim;
    float *sc = (float *)malloc(tt * sizeof(float));
    if (!sc) return -3;
    const int mm_iters = iters > 0 ? iters : 24;
    for (int bh = 0; bh < batch * heads; bh++) {
        orc_matmul(0, 1, q + bh * td, k + bh * td, sc, seq, seq, dim, scale, 0.0f,
                   mm_iters, mode, 0);
        for (int t = 0; t < seq; t++) {
            float *row = sc + (size_t)t * seq;
            for (int s = 0; s < seq; s++) {
                if (is_causal && s > t) row[s] = -INFINITY;
                if (mask) row[s] += mask[(size_t)t * seq + s];
            }
            float m = row[0];
            for (int s = 1; s < seq; s++) if (row[s] > m) m = row[s];
            float sum = 0.0f;
            for (int s = 0; s < seq; s++) {
                row[s] = (iters > 0) ? orc_exp_n(row[s] - m, iters) : expf(row[s] - m);
                sum += row[s];
            }
            float inv = (sum > 0.0f) ? 1.0f / sum : 0.0f;
            for (int s = 0; s < seq; s++) row[s] *= inv;
        }
        orc_matmul(0, 0, sc, v + bh * td, out + bh * td, seq, dim, seq, 1.0f, 0.0f,
                   mm_iters, mode, 0);
    }
    free(sc);
    return 0;
}

/* ── Q8_0 weights and the decode GEMV (lib/c/rac_q8_0.h:35-100) ──────────
 * Block: uint16 fp16 scale d, then 32 int8 q (34 bytes, packed, little
 * endian); value = fp16_to_fp32(d) * q. */

#define ORC_Q8_BLOCK 32
#define ORC_Q8_BYTES 34

/* rac_fp16_to_fp32, rac_q8_0.c:21-45 (exact; subnormal halves normalised). */
ORC_API float orc_fp16_to_fp32(uint16_t h)
{
    uint32_t sign = (h >> 15) & 1u, ex = (h >> 10) & 0x1fu, mant = h & 0x3ffu, bits;
    if (ex == 0) {
        if (mant == 0) {
            bits = sign << 31;
        } else {
            int e = -14;
            while ((mant & 0x400u) == 0) { mant <<= 1; e--; }
            mant &= 0x3ffu;
            bits = (sign << 31) | ((uint32_t)(e + 127) << 23) | (mant << 13);
        }
    } else if (ex == 31) {
        bits = (sign << 31) | (0xffu << 23) | (mant << 13);
    } else {
        bits = (sign << 31) | ((ex - 15 + 127) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* rac_fp32_to_fp16, rac_q8_0.c:47-64: mantissa TRUNCATED (no rounding),
 * exponents below the half range flush to signed zero, above to inf. */
ORC_API uint16_t orc_fp32_to_fp16(float f)
{
    uint32_t b;
    memcpy(&b, &f, 4);
    uint32_t sign = (b >> 16) & 0x8000u;
    int32_t ex = (int32_t)((b >> 23) & 0xffu) - 127 + 15;
    uint32_t mant = b & 0x7fffffu;
    if (ex <= 0) {
        if (ex < -10) return (uint16_t)sign;
        mant = (mant | 0x800000u) >> (1 - ex);
        return (uint16_t)(sign | (mant >> 13));
    }
    if (ex >= 31) return (uint16_t)(sign | 0x7c00u | (mant ? 0x200u : 0u));
    return (uint16_t)(sign | ((uint32_t)ex << 10) | (mant >> 13));
}

/* rac_q8_0_quantize_row / _matrix, rac_q8_0.c:68-100: per block amax,
 * d = amax / 127, id = 1/d (0 when d == 0), q = lrintf(x * id) clamped to
 * [-127, 127]; d stored through orc_fp32_to_fp16. */
ORC_API void orc_q8_0_quantize(const float *src, uint8_t *dst, long rows, int K)
{
    const int nb = K / ORC_Q8_BLOCK;
    for (long r = 0; r < rows; r++)
        for (int b = 0; b < nb; b++) {
            const float *blk = src + (size_t)r * K + (size_t)b * ORC_Q8_BLOCK;
            uint8_t *o = dst + ((size_t)r * nb + b) * ORC_Q8_BYTES;
            float amax = 0.0f;
            for (int i = 0; i < ORC_Q8_BLOCK; i++) {
                float a = fabsf(blk[i]);
                if (a > amax) amax = a;
            }
            float d = amax / 127.0f;
            float id = (d > 0.0f) ? 1.0f / d : 0.0f;
            uint16_t h = orc_fp32_to_fp16(d);
            o[0] = (uint8_t)(h & 0xff);
            o[1] = (uint8_t)(h >> 8);
            for (int i = 0; i < ORC_Q8_BLOCK; i++) {
                int q = (int)lrintf(blk[i] * id);
                if (q < -127) q = -127;
                if (q > 127) q = 127;
                o[2 + i] = (uint8_t)(int8_t)q;
            }
        }
}

/* rac_q8_0_dequantize_row, rac_q8_0.c:102-111. */
ORC_API void orc_q8_0_dequantize(const uint8_t *src, float *dst, long rows, int K)
{
    const long nblk = rows * (long)(K / ORC_Q8_BLOCK);
    for (long b = 0; b < nblk; b++) {
        const uint8_t *blk = src + (size_t)b * ORC_Q8_BYTES;
        float d = orc_fp16_to_fp32((uint16_t)(blk[0] | (blk[1] << 8)));
        for (int i = 0; i < ORC_Q8_BLOCK; i++)
            dst[(size_t)b * ORC_Q8_BLOCK + i] = d * (float)(int8_t)blk[2 + i];
    }
}

/* One block's dot product in the order of the AVX2 kernel
 * (rac_q8_0.c:128-165): lane l of 8 accumulates q[l] x[l] (a product),
 * then fma with q[8+l] x[8+l], q[16+l] x[16+l], q[24+l] x[24+l]; the 8 lane
 * sums combine as ((a0+a4) + (a1+a5)) + ((a2+a6) + (a3+a7)). */
ORC_API float orc_q8_0_block_dot(const uint8_t *blk, const float *x)
{
    const int8_t *q = (const int8_t *)(blk + 2);
    float a[8];
    for (int l = 0; l < 8; l++) {
        float s = (float)q[l] * x[l];
        s = fmaf((float)q[8 + l], x[8 + l], s);
        s = fmaf((float)q[16 + l], x[16 + l], s);
        s = fmaf((float)q[24 + l], x[24 + l], s);
        a[l] = s;
    }
    float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
    return (s0 + s1) + (s2 + s3);
}

/* rac_q8_0_gemv, rac_q8_0.c:178-211, for M input rows: out[m][j] =
 * act(sum_b d_b dot_b + bias[j]) with the block terms accumulated in block
 * order as acc = fmaf(d_b, dot_b, acc) (the reference build contracts
 * `acc += d * dot`; contract = 0 gives the unfused form).  act: 0 none,
 * 1 ReLU, 2 GELU (erff), 3 SiLU (expf), as rac_q8_0.c:167-174. */
ORC_API int orc_q8_0_gemv(const float *x, const uint8_t *w, const float *bias, float *out,
                          int M, int N, int K, int act, int contract)
{
    if (!x || !w || !out) return -1;
    if (M <= 0 || N <= 0 || K <= 0 || K % ORC_Q8_BLOCK) return -2;
    const int nb = K / ORC_Q8_BLOCK;
    #pragma omp parallel for schedule(static)
    for (long t = 0; t < (long)M * N; t++) {
        const int m = (int)(t / N), j = (int)(t % N);
        const uint8_t *row = w + (size_t)j * nb * ORC_Q8_BYTES;
        float acc = 0.0f;
        for (int b = 0; b < nb; b++) {
            const uint8_t *blk = row + (size_t)b * ORC_Q8_BYTES;
            float dot = orc_q8_0_block_dot(blk, x + (size_t)m * K + (size_t)b * ORC_Q8_BLOCK);
            float d = orc_fp16_to_fp32((uint16_t)(blk[0] | (blk[1] << 8)));
            acc = contract ? fmaf(d, dot, acc) : acc + d * dot;
        }
        if (bias) acc += bias[j];
        float s = acc;
        switch (act) {
        case 1: s = s > 0.0f ? s : 0.0f; break;
        case 2: s = 0.5f * s * (1.0f + erff(s * 0.7071067811865f)); break;
        case 3: s = s / (1.0f + expf(-s)); break;
        default: break;
        }
        out[t] = s;
    }
    return 0;
}

/* ── RAC-DSP fixed-point CORDIC engine (sim/rac_dsp_core.c) ──────────────
 * Integer model of the RTL datapath: x, y in Q32.32, z in Q0.63 fractions
 * of pi; 64-bit two's-complement arithmetic (computed here in uint64_t so
 * overflow wraps as the hardware does).  ROMs: a 1024-entry coarse LUT of
 * 10-bit direction words, atan(2^-i) for i = 0..16 and atanh(2^-s) for
 * s = 8..16, both in Q0.63 fractions of pi. */

#define ORC_DSP_LUT_BITS 10
#define ORC_DSP_LUT 1024
#define ORC_DSP_RES 9
#define ORC_DSP_RES_START 8
#define ORC_DSP_ATAN (ORC_DSP_RES_START + ORC_DSP_RES)

static uint64_t orc_dsp_lut[ORC_DSP_LUT];
static int64_t orc_dsp_atan[ORC_DSP_ATAN];
static int64_t orc_dsp_atanh[ORC_DSP_RES];
static int orc_dsp_ready = 0;

/* round(v / pi * 2^63) as rtl/gen_coarse_lut.py computes it in doubles
 * (round half to even), as a 64-bit pattern. */
static int64_t q063_frac_pi(double v)
{
    double s = nearbyint(v / M_PI * 9223372036854775808.0);
    return (int64_t)s;
}

/* The ROMs by the generation rule of rtl/gen_coarse_lut.py:27-123: LUT
 * entry k holds the direction bits of a double-precision circular CORDIC
 * driving z = (k - 512 + 0.5) pi / 1024 to zero over 10 steps (bit i set
 * for d_i = +1). */
ORC_API void orc_dsp_gen_roms(uint64_t *lut, int64_t *atan_rom, int64_t *atanh_rom)
{
    for (int k = 0; k < ORC_DSP_LUT; k++) {
        double z = (k - ORC_DSP_LUT / 2 + 0.5) * M_PI / ORC_DSP_LUT;
        uint64_t bits = 0;
        for (int i = 0; i < ORC_DSP_LUT_BITS; i++) {
            double step = atan(ldexp(1.0, -i));
            if (z >= 0.0) { z -= step; bits |= (uint64_t)1 << i; }
            else z += step;
        }
        lut[k] = bits;
    }
    for (int i = 0; i < ORC_DSP_ATAN; i++) atan_rom[i] = q063_frac_pi(atan(ldexp(1.0, -i)));
    for (int i = 0; i < ORC_DSP_RES; i++)
        atanh_rom[i] = q063_frac_pi(atanh(ldexp(1.0, -(ORC_DSP_RES_START + i))));
}

static void dsp_init(void)
{
    if (!orc_dsp_ready) {
        orc_dsp_gen_roms(orc_dsp_lut, orc_dsp_atan, orc_dsp_atanh);
        orc_dsp_ready = 1;
    }
}

/* Use the given ROM contents instead of the generated ones. */
ORC_API void orc_dsp_set_roms(const uint64_t *lut, const int64_t *atan_rom, const int64_t *atanh_rom)
{
    memcpy(orc_dsp_lut, lut, sizeof(orc_dsp_lut));
    memcpy(orc_dsp_atan, atan_rom, sizeof(orc_dsp_atan));
    memcpy(orc_dsp_atanh, atanh_rom, sizeof(orc_dsp_atanh));
    orc_dsp_ready = 1;
}

static inline uint64_t dsp_asr(uint64_t v, int n)          /* arithmetic shift right */
{
    return (uint64_t)((int64_t)v >> n);
}

/* rac_dsp_eval, sim/rac_dsp_core.c:95-149: quadrant fold (|z| >= pi/2 ->
 * z + pi, (x, y) negated), then for op != 2 (vectoring) a coarse stage of
 * 10 circular micro-rotations whose directions come from the LUT indexed by
 * the top bits of 2z, then 9 residual micro-rotations at shifts 8..16
 * (hyperbolic for op 3; vectoring directions from sign(y) for op 2). */
ORC_API void orc_dsp_eval(int64_t xi, int64_t yi, int64_t zi, int op, int64_t *xo, int64_t *yo, int64_t *zo)
{
    dsp_init();
    uint64_t x = (uint64_t)xi, y = (uint64_t)yi, z = (uint64_t)zi;
    if (((z >> 63) ^ (z >> 62)) & 1u) {
        z ^= (uint64_t)1 << 63;
        x = (uint64_t)0 - x;
        y = (uint64_t)0 - y;
    }
    const int hyper = (op == 3), vect = (op == 2);
    if (!vect) {
        const int idx = (int)(((int64_t)(z << 1) >> (64 - ORC_DSP_LUT_BITS)) + ORC_DSP_LUT / 2) & (ORC_DSP_LUT - 1);
        const uint64_t dv = orc_dsp_lut[idx];
        uint64_t za = 0;
        for (int i = 0; i < ORC_DSP_LUT_BITS; i++) {
            const uint64_t ys = dsp_asr(y, i), xs = dsp_asr(x, i);
            if ((dv >> i) & 1u) { x = x - ys; y = y + xs; za += (uint64_t)orc_dsp_atan[i]; }
            else { x = x + ys; y = y - xs; za -= (uint64_t)orc_dsp_atan[i]; }
        }
        z = z - za;
    }
    for (int i = 0; i < ORC_DSP_RES; i++) {
        const int ph = ORC_DSP_RES_START + i;
        const int dpos = vect ? ((int64_t)y < 0) : ((int64_t)z >= 0);
        const uint64_t xs = dsp_asr(x, ph), ys = dsp_asr(y, ph);
        const uint64_t c = (uint64_t)(hyper ? orc_dsp_atanh[i] : orc_dsp_atan[ph]);
        uint64_t xn;
        if (hyper) xn = dpos ? x + ys : x - ys;
        else xn = dpos ? x - ys : x + ys;
        const uint64_t yn = dpos ? y + xs : y - xs;
        const uint64_t zn = dpos ? z - c : z + c;
        x = xn; y = yn; z = zn;
    }
    *xo = (int64_t)x; *yo = (int64_t)y; *zo = (int64_t)z;
}

ORC_API void orc_dsp_eval_batch(int op, long n, const int64_t *x, const int64_t *y, const int64_t *z,
                                int64_t *xo, int64_t *yo, int64_t *zo)
{
    for (long i = 0; i < n; i++) orc_dsp_eval(x[i], y[i], z[i], op, &xo[i], &yo[i], &zo[i]);
}

/* sim/rac_systolic_ref.c:40-55: Y[k][c] = sum_r project(X[k][r], 0,
 * W[r][c]).x over a weight-stationary N x N array, for K input vectors. */
ORC_API void orc_dsp_systolic(int N, int K, const int64_t *W, const int64_t *X, int64_t *Y)
{
    for (int k = 0; k < K; k++)
        for (int c = 0; c < N; c++) {
            uint64_t sum = 0;
            for (int r = 0; r < N; r++) {
                int64_t xo, yo, zo;
                orc_dsp_eval(X[(size_t)k * N + r], 0, W[(size_t)r * N + c], 1, &xo, &yo, &zo);
                sum += (uint64_t)xo;
            }
            Y[(size_t)k * N + c] = (int64_t)sum;
        }
}

/* ── safetensors element conversion (bench/safetensors_reader.c:375-425) ──
 * dtype codes of safetensors_reader.h:37-49: 1 F32 (copy), 2 F16 (the same
 * exact widening as rac_fp16_to_fp32, safetensors_reader.c:375-397),
 * 3 BF16 (bits << 16), 4 F64 ((float) cast on this x86-64 host).  Returns
 * -1 for any other dtype, as st_to_f32 does. */
ORC_API int orc_st_to_f32(int dtype, const void *raw, long n, float *out)
{
    switch (dtype) {
    case 1:
        memcpy(out, raw, (size_t)n * sizeof(float));
        return 0;
    case 2: {
        const uint16_t *h = (const uint16_t *)raw;
        for (long i = 0; i < n; i++) out[i] = orc_fp16_to_fp32(h[i]);
        return 0;
    }
    case 3: {
        const uint16_t *h = (const uint16_t *)raw;
        for (long i = 0; i < n; i++) {
            uint32_t b = (uint32_t)h[i] << 16;
            memcpy(&out[i], &b, 4);
        }
        return 0;
    }
    case 4: {
        const double *d = (const double *)raw;
        for (long i = 0; i < n; i++) out[i] = (float)d[i];
        return 0;
    }
    default:
        return -1;
    }
}
