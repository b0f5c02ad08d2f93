/*
 * rac_ext.h — device-pointer, stream-ordered entry points of librac_amd.so,
 * the process knobs, and the reference kernel-library launcher ABI.
 *
 * Device API (rac_*_dev): every buffer is device memory; the work is
 * enqueued on `stream` (a hipStream_t, 0 = null stream) and the call
 * returns without synchronising.  Return value: 0 on success, or
 *   -1 RAC_ERR_NULL_PTR, -2 RAC_ERR_INVALID_DIM, -3 RAC_ERR_ALLOC
 *   (same codes as the reference rac_cpu.h:54-59), -4 HIP error;
 * the message is in rac_last_error().  Arguments are validated before any
 * HIP call.  These are the calls the Python layer makes (with torch's
 * current stream); they have no counterpart in rac.h, whose entry points
 * are synchronous.
 */
#ifndef RAC_EXT_H
#define RAC_EXT_H

#ifdef __cplusplus
extern "C" {
#endif

#define RAC_MODE_FAST 0     /* rac_kernels.hip:23-25 */
#define RAC_MODE_CORDIC 1
#define RAC_MODE_SHIFTADD 2

/* ── errors, knobs, info ─────────────────────────────────────────────────── */

const char *rac_last_error(void);   /* thread-local message of the last failure */
void rac_clear_error(void);
/* Process knobs of the synchronous rac.h API, seeded from RAC_CORDIC_ITERS
 * (default 16) and RAC_CORDIC_MODE (fast|cordic|shiftadd, default cordic).
 * Clamping follows rac_torch_bind.cpp:205-219 (iters <= 0 -> default,
 * clamp to [1, 24]; an unknown mode selects FAST). */
void rac_set_cordic_iters(int iters);
int rac_get_cordic_iters(void);
void rac_set_cordic_mode(int mode);
int rac_get_cordic_mode(void);
/* Stream used by the synchronous rac.h calls (default 0). */
void rac_set_stream(void *stream);
void *rac_get_stream(void);
int rac_version(void);
/* The synchronous rac.h calls stage host buffers through device buffers
 * that stay cached per GPU (at most RAC_STAGE_CACHE_MB MiB each, 512 by
 * default, 0 = no caching).  This frees every cached buffer on every GPU and
 * returns the bytes released, for processes whose other allocator (torch's)
 * needs the memory.  No counterpart in the reference, which has no device
 * staging (rac_hip.cpp:364-379 allocates per call). */
long rac_release_cached_memory(void);
/* Host-side queries of the constants the kernels use (no GPU needed):
 * the circular direction sequence of CORDIC-mode matmul (d[i] = +1/-1 for
 * i < iters; returns the clamped count), 1/K_h of the n-step exp, and 1/K_h
 * of the 16-step rsqrt. */
int rac_cordic_direction_bits(int iters, int *d);
float rac_exp_gain_inverse(int iters);
float rac_rsqrt_gain_inverse(void);

/* ── device API ──────────────────────────────────────────────────────────── */

/* C[M,N] = alpha * op(A) op(B) (+ beta * C); op(A) = A [M,K] or, with
 * trans_a, A stored [K,M]; op(B) = B [K,N] or, with trans_b, B stored [N,K].
 * mode 0 FAST / 1 CORDIC / 2 SHIFTADD, iters clamped to [1, 24].
 * Replaces rac_kernels.hip:822-883 (same semantics, explicit status). */
int rac_gemm_dev(const float *A, const float *B, float *C, int M, int N, int K,
                 int trans_a, int trans_b, float alpha, float beta, int iters, int mode,
                 void *stream);
/* `batch` independent products (batch <= 65535): C_z = alpha op(A_z) op(B_z)
 * (+ beta C_z) with A_z = A + z*stride_a etc. (element strides). */
int rac_gemm_batched_dev(const float *A, const float *B, float *C, int M, int N, int K,
                         int trans_a, int trans_b, float alpha, float beta, int iters, int mode,
                         int batch, long stride_a, long stride_b, long stride_c, void *stream);
/* Fused linear layer (rac_torch.cu:705-780): out[M,N] = act(input[M,K]
 * weight[N,K]^T + bias[N]) with the RAC MAC of `mode`; act 0 none, 1 ReLU,
 * 2 GELU (erf), 3 SiLU (CORDIC exp of `iters` steps); bias and pre may be
 * NULL; pre receives the pre-activation values when given. */
int rac_fused_linear_dev(const float *input, const float *weight, const float *bias, float *out,
                         float *pre, int M, int N, int K, int act, int iters, int mode, void *stream);
/* d[i] = g[i] * act'(pre[i]) (rac_torch.cu:680-694), same activation ids. */
int rac_act_grad_dev(const float *g, const float *pre, float *d, long count, int act, int iters,
                     void *stream);
/* Attention softmax of rows that form [.., seq, seq] score blocks: row r is
 * query position t = r % seq; is_causal sets -inf for columns > t, then the
 * optional additive mask[t*seq + col] is added; 1/sum is 0 for a sum that is
 * not > 0 (rac_cpu.c:664-687).  x == y is allowed. */
int rac_softmax_masked_dev(const float *x, float *y, long rows, long seq, const float *mask,
                           int is_causal, int iters, void *stream);
/* Softmax of each of `rows` rows of n floats (rac_cpu.c:258-271 with the
 * n-step CORDIC exp). */
int rac_softmax_dev(const float *x, float *y, long rows, long n, int iters, void *stream);
/* Elementwise: CORDIC e^x, SiLU x/(1+e^-x), sigmoid 1/(1+e^-x), tanh;
 * GELU x/2(1+erf(x/sqrt2)) and ReLU (rac_cpu.c:441-457). */
int rac_exp_dev(const float *x, float *y, long count, int iters, void *stream);
int rac_silu_dev(const float *x, float *y, long count, int iters, void *stream);
int rac_sigmoid_dev(const float *x, float *y, long count, int iters, void *stream);
int rac_tanh_dev(const float *x, float *y, long count, int iters, void *stream);
int rac_gelu_dev(const float *x, float *y, long count, void *stream);
int rac_relu_dev(const float *x, float *y, long count, void *stream);
/* Batch CORDIC rsqrt and circular sin/cos (the scalar rac.h calls use these). */
int rac_rsqrt_dev(const float *x, float *y, long count, void *stream);
int rac_sincos_dev(const float *theta, float *s, float *c, long count, void *stream);
/* RMSNorm / LayerNorm over rows of d floats; gamma/beta may be NULL
 * (rac_cpu.c:507-574 with the CORDIC rsqrt). */
int rac_rmsnorm_dev(const float *x, float *y, const float *gamma, float eps, long rows, long d,
                    void *stream);
int rac_layernorm_dev(const float *x, float *y, const float *gamma, const float *beta, float eps,
                      long rows, long d, void *stream);
/* RoPE table on the device.  inv_freq_dev holds head_dim/2 floats produced
 * by rac_rope_inv_freq (host) and copied by the caller, so the call itself
 * allocates nothing.  `base` is informational (inv_freq carries it). */
int rac_rope_inv_freq(float *inv_freq_host, int head_dim, float base);
int rac_rope_cache_dev(float *cos_out, float *sin_out, int max_seq, int head_dim, float base,
                       const float *inv_freq_dev, void *stream);
/* In-place RoPE on rows (b, h, t) at x + b*stride_b + h*stride_h + t*stride_t
 * (element strides; head_dim contiguous).  Contiguous [B,H,T,D]:
 * stride_b = H*T*D, stride_h = T*D, stride_t = D; the [B,T,H,D] storage of
 * attention projections: stride_b = T*H*D, stride_h = D, stride_t = H*D. */
int rac_rope_apply_dev(float *x, const float *cos_tab, const float *sin_tab, int batch,
                       int n_heads, int seq, int head_dim, long stride_b, long stride_h,
                       long stride_t, void *stream);
/* The same rotation out of place (rac_cpu.c:600-635 on a copy): rows read
 * at x with strides (stride_b, stride_h, stride_t), written at y with
 * (out_b, out_h, out_t); x and y must not overlap.  One read and one write
 * per element. */
int rac_rope_apply_out_dev(const float *x, float *y, const float *cos_tab, const float *sin_tab,
                           int batch, int n_heads, int seq, int head_dim, long stride_b,
                           long stride_h, long stride_t, long out_b, long out_h, long out_t,
                           void *stream);

/* Vector primitives over n items of interleaved (x, y) pairs.  `op` selects
 * the rac.h primitive evaluated per item i (rac.h:101-250, 345-346, with the
 * semantics of rac_cpu.c:136-288):
 *   RAC_V2_ROTATE      out2[i] = rac_rotate(a[i], theta[i])
 *   RAC_V2_ROTATE_RAW  out2[i] = rac_rotate_raw(a[i], theta[i])
 *   RAC_V2_COMPENSATE  out2[i] = rac_compensate(a[i], iarg)
 *   RAC_V2_PROJECT     out1[i] = rac_project(a[i], theta[i])
 *   RAC_V2_POLAR       out2[i] = (mag, angle) of rac_polar(a[i])
 *   RAC_V2_NORMALIZE   out2[i] = rac_normalize(a[i])
 *   RAC_V2_DOT         out1[i] = rac_dot(a[i], b[i])
 *   RAC_V2_COHERENCE   out1[i] = rac_coherence(a[i], b[i])
 *   RAC_V2_COMPLEX_MUL out2[i] = rac_complex_mul(a[i], b[i])
 *   RAC_V2_ROTATE_N    out2[i] = rac_rotate_precision(a[i], theta[i], iarg)
 *   RAC_V2_PROJECT_N   out1[i] = rac_project_precision(a[i], theta[i], iarg)
 *   RAC_V2_INNER_TERM  out1[i] = rac_project(a[i], angle(b[i])) * |b[i]|
 * Operands an op does not use may be NULL. */
#define RAC_V2_ROTATE 0
#define RAC_V2_ROTATE_RAW 1
#define RAC_V2_COMPENSATE 2
#define RAC_V2_PROJECT 3
#define RAC_V2_POLAR 4
#define RAC_V2_NORMALIZE 5
#define RAC_V2_DOT 6
#define RAC_V2_COHERENCE 7
#define RAC_V2_COMPLEX_MUL 8
#define RAC_V2_ROTATE_N 9
#define RAC_V2_PROJECT_N 10
#define RAC_V2_INNER_TERM 11
int rac_vec2_dev(int op, long n, const float *a, const float *b, const float *theta, int iarg,
                 float *out2, float *out1, void *stream);
/* *out = rac_inner(a, b, n) (rac.h:233), one workgroup, fixed-order tree sum. */
int rac_inner_dev(const float *a, const float *b, long n, float *out, void *stream);
/* C[m,n] = rac_outer(a, b) (rac.h:240). */
int rac_outer_dev(const float *a, const float *b, float *C, int m, int n, void *stream);
/* X = rac_dct(x) (rac.h:189), one lane per output k. */
int rac_dct_dev(const float *x, float *X, int n, void *stream);
/* rac_attention (rac.h:330; CPU definition rac_cpu.c:637-703) on device
 * buffers [batch, n_heads, seq, head_dim]: scores = Q K^T / sqrt(head_dim) by
 * the RAC matmul (mode, iters), causal and additive [seq, seq] mask, CORDIC
 * softmax, out = P V by the RAC matmul.  The core runs over chunks of query
 * rows, so the workspace holds the scores of one chunk (at most 128 MiB, or
 * 64 query rows of every head when one row of every head needs more than
 * 2 MiB), not the [batch*n_heads, seq, seq] matrix the reference
 * materialises; results do not depend on the chunk.  workspace:
 * rac_attention_workspace_bytes(batch, n_heads, seq) bytes of device memory
 * owned by the caller. */
long rac_attention_workspace_bytes(int batch, int n_heads, int seq);
int rac_attention_dev(const float *q, const float *k, const float *v, const float *mask,
                      int is_causal, float *out, int batch, int n_heads, int seq, int head_dim,
                      float *workspace, int iters, int mode, void *stream);
/* rac_attention_dev with the workspace's size in bytes: the chunk is the
 * largest that workspace_bytes holds (at least one query row of every head,
 * 4*batch*n_heads*seq + 256 bytes).  Same output bits for every size. */
int rac_attention_ws_dev(const float *q, const float *k, const float *v, const float *mask,
                         int is_causal, float *out, int batch, int n_heads, int seq, int head_dim,
                         float *workspace, long workspace_bytes, int iters, int mode, void *stream);
/* rac_attention_dev for callers that cannot allocate device memory (code
 * under stream or graph capture, serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  It allocates nothing: its
 * chunk workspace is a 64 MiB (+ 256 B) device array inside the library, one
 * per GPU, held until the process ends.  Limit: batch*n_heads*seq <=
 * 16777215 (one query row of every head must fit the array); larger shapes
 * are refused with -2 before any device work.  Every call on one GPU shares
 * that GPU's array, so calls that overlap on one GPU race: serialise them.
 * Same output bits as rac_attention_dev. */
int rac_attention_noalloc_dev(const float *q, const float *k, const float *v, const float *mask,
                              int is_causal, float *out, int batch, int n_heads, int seq, int head_dim,
                              int iters, int mode, void *stream);
/* The same attention in one chunk, keeping every probability: on return the
 * first batch*n_heads*seq*seq floats of the workspace (of
 * rac_attention_probs_workspace_bytes bytes) hold P, what the backward pass
 * (dV = P^T dO, dS = P (dP - rowsum(dP P))) reads.  Same output bits as
 * rac_attention_dev. */
long rac_attention_probs_workspace_bytes(int batch, int n_heads, int seq);
int rac_attention_probs_dev(const float *q, const float *k, const float *v, const float *mask,
                            int is_causal, float *out, int batch, int n_heads, int seq, int head_dim,
                            float *workspace, int iters, int mode, void *stream);

/* The probabilities of query rows row0 .. row0+rows-1 of every head into P
 * [batch*n_heads, rows, seq], equal bit for bit to those rows of the P that
 * rac_attention_probs_dev leaves in its workspace (the attention core's
 * scores and masked CORDIC softmax, rac_cpu.c:651-690).  For a backward
 * pass that recomputes P one chunk of query rows at a time instead of
 * keeping the [batch*n_heads, seq, seq] matrix (what the reference's
 * autograd of its composition keeps, rac_torch.py:1327-1337).  Same
 * argument checks as rac_attention_dev, plus 0 <= row0 < row0 + rows <= seq. */
int rac_attention_probs_rows_dev(const float *q, const float *k, const float *mask, int is_causal,
                                 float *P, int batch, int n_heads, int seq, int head_dim, int row0,
                                 int rows, int iters, int mode, void *stream);

/* ── reference launcher ABI (rac_kernels.hip:822-909; bound by
 *    rac_torch_bind.cpp:16-45 with the stream as void*) ──────────────────── */

void rac_launch_nn_iters(const float *A, const float *B, float *C, int M, int N, int K,
                         float alpha, float beta, int iters, int mode, void *stream);
void rac_launch_nt_iters(const float *A, const float *B, float *C, int M, int N, int K,
                         float alpha, float beta, int iters, int mode, void *stream);
void rac_launch_tn_iters(const float *A, const float *B, float *C, int M, int N, int K,
                         float alpha, float beta, int iters, int mode, void *stream);
void rac_launch_nn(const float *A, const float *B, float *C, int M, int N, int K, float alpha,
                   float beta, void *stream);
void rac_launch_nt(const float *A, const float *B, float *C, int M, int N, int K, float alpha,
                   float beta, void *stream);
void rac_launch_tn(const float *A, const float *B, float *C, int M, int N, int K, float alpha,
                   float beta, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* RAC_EXT_H */
