/*
 * rac.h — C ABI of librac_amd.so, the MI355X (gfx950) implementation of the
 * RAC rotation-accumulate hot path.  Drop-in for the reference rac.h
 * (rac.h:85-346): same function names, argument lists and return types for
 * the entry points below, compilable as plain C (the reference header needs
 * HIP/CUDA to define __device__/__host__; this one does not).
 *
 * Contract (same as the reference): the caller owns every buffer; calls are
 * synchronous and return void/float.  Each pointer may be host memory or
 * device memory (hipMalloc); the library classifies it per call, stages host
 * buffers through device memory and returns once results are in the
 * caller's buffers.  Errors (NULL pointers, bad dimensions, HIP failures)
 * leave outputs untouched and are readable through rac_last_error()
 * (rac_ext.h).  Iteration count and matmul mode come from the process knobs
 * of rac_ext.h (environment RAC_CORDIC_ITERS, default 16 = RAC_ITERS, and
 * RAC_CORDIC_MODE, default "cordic").
 */
#ifndef RAC_H
#define RAC_H

#ifdef __cplusplus
extern "C" {
#endif

/* The reference's pair type (rac.h:25-33): HIP's float2 in HIP code, the
 * same two-float struct for C and C++ hosts. */
#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#else
typedef struct {
    float x;
    float y;
} float2;
#endif

#define RAC_K_INV 0.60725f /* rac.h:39 */
#define RAC_K 1.64676f     /* rac.h:40 */
#define RAC_ITERS 16       /* rac.h:41 */

/* ── context (rac.h:45-88) ───────────────────────────────────────────────── */

typedef struct rac_context_t *rac_context;

typedef enum {
    RAC_BACKEND_CUDA = 0,
    RAC_BACKEND_HIP = 1,
    RAC_BACKEND_CPU = 2,
    RAC_BACKEND_FIL = 3
} rac_backend;

typedef enum {
    RAC_OP_ROTATE = 0, RAC_OP_ROTATE_RAW = 1, RAC_OP_PROJECT = 2, RAC_OP_POLAR = 3,
    RAC_OP_NORM = 4, RAC_OP_NORMALIZE = 5, RAC_OP_DOT = 6, RAC_OP_COHERENCE = 7,
    RAC_OP_COMPLEX_MUL = 8, RAC_OP_DCT = 9, RAC_OP_EXP = 10, RAC_OP_TANH = 11,
    RAC_OP_SOFTMAX = 12, RAC_OP_ROTATE_BATCH = 13, RAC_OP_INNER = 14, RAC_OP_OUTER = 15,
    RAC_OP_MATMUL = 16, RAC_OP_RSQRT = 17, RAC_OP_SIGMOID = 18, RAC_OP_SINCOS = 19,
    RAC_OP_LAYERNORM = 20, RAC_OP_RMSNORM = 21, RAC_OP_ROPE_CACHE = 22,
    RAC_OP_ROPE_APPLY = 23, RAC_OP_ATTENTION = 24, RAC_OP_EXTENDED = 0xFF
} rac_op_type;

/* rac.h:85-88; replaces the stub of rac_hip.cpp:416-435 (same answers:
 * every op except RAC_OP_EXTENDED is supported; rac_execute returns 0). */
rac_context rac_create_context(rac_backend backend);
void rac_destroy_context(rac_context ctx);
int rac_query_capability(rac_context ctx, rac_op_type op);
int rac_execute(rac_context ctx, rac_op_type op, void *desc);

/* ── core rotation, polar, similarity, complex (rac.h:101-189) ─────────────
 * Semantics of the reference CPU library (rac_cpu.c:136-228): angles are
 * reduced to (-pi, pi] and vectors with x < 0 are pre-rotated by pi, so
 * every call holds over the whole plane; 16 CORDIC steps; projections use
 * cosf/sinf of the angle.  Angles with |theta| >= 2^27 or +-inf give NaN
 * (the reference's reduction loop does not end there). */
float2 rac_rotate(float2 v, float theta);          /* (v * K_INV) rotated by theta */
float2 rac_rotate_raw(float2 v, float theta);      /* no gain compensation */
float2 rac_compensate(float2 v, int chain_length); /* v * K_INV^chain_length */
float rac_project(float2 v, float theta);          /* v.x cos(theta) + v.y sin(theta) */
void rac_polar(float2 v, float *mag, float *angle);
float rac_norm(float2 v);
float2 rac_normalize(float2 v);
float rac_dot(float2 a, float2 b);
float rac_coherence(float2 a, float2 b);
float2 rac_complex_mul(float2 a, float2 b);
/* DCT-II: X[k] = sum_i x[i] cos(pi (2i+1) k / 2n).  rac.h:189. */
void rac_dct(float *x, float *X, int n);

/* ── hyperbolic / activations (rac.h:198-214) ────────────────────────────── */

/* e^x by hyperbolic CORDIC (RAC_CORDIC_ITERS Walther steps, ln2 range
 * reduction).  Replaces rac.h:198 / rac_hip.cpp:302-306. */
float rac_exp(float x);
/* tanh(x) = sign(x)(1-e)/(1+e), e = CORDIC e^{-2|x|}.  rac.h:205. */
float rac_tanh(float x);
/* Row softmax of n floats (max, CORDIC exp, sum, multiply by 1/sum).
 * Replaces rac.h:214 / rac_hip.cpp:315-329. */
void rac_softmax(float *x, float *out, int n);

/* ── batch vector operations (rac.h:223-240) ─────────────────────────────── */

void rac_rotate_batch(float2 *v, float *theta, float2 *out, int n);
/* sum_i rac_project(a[i], angle(b[i])) * |b[i]| */
float rac_inner(float2 *a, float2 *b, int n);
/* C[i*n + j] = rac_project(a[i], angle(b[j])) * |b[j]| */
void rac_outer(float2 *a, float2 *b, float *C, int m, int n);

/* ── matmul (rac.h:249) ──────────────────────────────────────────────────── */

/* C[M,N] = A[M,K] @ B[K,N], row-major, by rotate-project-accumulate
 * (mode and iteration count from the process knobs; default CORDIC, 16).
 * Replaces rac.h:249 / rac_hip.cpp:364-379. */
void rac_matmul(float *A, float *B, float *C, int M, int N, int K);

/* ── transformer primitives (rac.h:274-320) ──────────────────────────────── */

/* 1/sqrt(x) by hyperbolic CORDIC vectoring; x <= 0 -> 0.  rac.h:274. */
float rac_rsqrt(float x);
/* 1/(1 + e^-x) with the CORDIC e^x.  rac.h:280. */
float rac_sigmoid(float x);
/* (sin, cos) of theta by one 16-step circular CORDIC rotation of
 * (RAC_K_INV, 0).  rac.h:286 (semantics of rac_cpu.c:322-328). */
void rac_sincos(float theta, float *s, float *c);
/* Per-row LayerNorm / RMSNorm over [rows, d]; gamma/beta may be NULL.
 * rac.h:294-300 (semantics of rac_cpu.c:507-574). */
void rac_layernorm(const float *x, float *y, const float *gamma, const float *beta,
                   float eps, int rows, int d);
void rac_rmsnorm(const float *x, float *y, const float *gamma, float eps, int rows, int d);
/* cos/sin tables [max_seq, head_dim/2] by circular CORDIC; bit-identical to
 * the reference table.  rac.h:307 (semantics of rac_cpu.c:576-598). */
void rac_rope_cache(float *cos_out, float *sin_out, int max_seq, int head_dim, float base);
/* In-place RoPE on x[batch, n_heads, seq, head_dim].  rac.h:316
 * (semantics of rac_cpu.c:600-635). */
void rac_rope_apply(float *x, const float *cos_tab, const float *sin_tab, int batch,
                    int n_heads, int seq, int head_dim);

/* Scaled dot-product attention on [batch, n_heads, seq, head_dim] tensors,
 * composed of RAC stages (rac.h:323-335): scores = Q K^T / sqrt(head_dim)
 * by rac_matmul, is_causal -> -inf above the diagonal, plus the optional
 * additive [seq, seq] mask, row softmax with the CORDIC exp, out = P V by
 * rac_matmul.  Mode and iteration count from the process knobs. */
void rac_attention(const float *q, const float *k, const float *v, const float *mask,
                   int is_causal, float *out, int batch, int n_heads, int seq, int head_dim);

/* ── tunable precision (rac.h:345-346; semantics of rac_cpu.c:275-288) ────── */

/* rac_rotate with iters (clamped to [4, 24]) steps and gain 1/K(iters). */
float2 rac_rotate_precision(float2 v, float theta, int iters);
/* v . (cos, sin)(theta), the pair from one iters-step CORDIC rotation. */
float rac_project_precision(float2 v, float theta, int iters);

/* ── batch activations with the rac_cpu.h signatures (rac_cpu.h:169-172) ── */

void rac_relu(const float *x, float *out, int n);
void rac_gelu(const float *x, float *out, int n);
void rac_silu(const float *x, float *out, int n);
void rac_softmax_batch(const float *x, float *out, int batch, int n);

#ifdef __cplusplus
}
#endif

#endif /* RAC_H */
