/*
 * rac_decode.h — the per-token pieces of a decoder layer's decode step in
 * librac_amd.so (MI355X, gfx950): the reference's full-model decode
 * (bench/bench_rac_transformer.c decoder_forward_kv :557-616 and
 * full_model_forward :618-625 with T_new = 1), whose GEMVs and norms are
 * rac_q8_0_gemv_dev and rac_rmsnorm_dev.
 *
 * Conventions of rac_ext.h: device buffers, work enqueued on `stream`, 0 or
 * a negative RAC_ERR_* code (message in rac_last_error()).
 *
 * The cache position is an int in device memory, read by the kernels when
 * they run: the launches of a decode step then have fixed arguments, and a
 * caller may record the step once as a HIP graph and replay it per token,
 * rac_position_advance_dev moving the position inside the graph.
 *
 * Cache layout: k_cache and v_cache are [n_kv_heads, t_cap, d_head] fp32
 * (each head's positions a row-major matrix); the reference keeps
 * [T_max, n_kv_heads * d_head] (kv_alloc :476-490).
 */
#ifndef RAC_DECODE_H
#define RAC_DECODE_H

#ifdef __cplusplus
extern "C" {
#endif

/* Largest d_head and cache length of rac_decode_attention_dev. */
#define RAC_DECODE_MAX_HEAD 256
#define RAC_DECODE_MAX_LEN 8192

/* out[h * d_head + c] = sum_j p_hj v[g][j][c] over positions j = 0 .. *pos,
 * p_h = softmax_j(scale * q_h . k[g][j]), g = h / (n_heads / n_kv_heads):
 * attention_head_causal (:508-548) for the last query row, with the RAC
 * softmax at `iters` CORDIC steps and FAST (fp32 fma) dot products.  q and
 * out are [n_heads * d_head].  Bit-identical to rac_gemm_batched_dev
 * (scores, alpha = scale) -> rac_softmax_dev on the scores padded with
 * -inf to a multiple of 4 -> rac_gemm_batched_dev (P V).  A position
 * outside [0, t_cap) gives NaN outputs and reads nothing. */
int rac_decode_attention_dev(const float *q, const float *k_cache, const float *v_cache, float *out,
                             int n_heads, int n_kv_heads, int d_head, long t_cap, const int *pos,
                             float scale, int iters, void *stream);

/* kv = [k (n_kv_heads * d_head) | v (n_kv_heads * d_head)] of the new token
 * written at position *pos of every head (:569-574); nothing is written
 * for a position outside [0, t_cap). */
int rac_kv_append_dev(const float *kv, float *k_cache, float *v_cache, int n_kv_heads, int d_head,
                      long t_cap, const int *pos, void *stream);

/* *pos += by (kv->cur_len += T_new, :624). */
int rac_position_advance_dev(int *pos, int by, void *stream);

/* out[i] = silu(gu[i]) * gu[n + i], i < n: the SwiGLU product of gate and
 * up stacked in one vector (:607-611), SiLU by the n-step CORDIC exp as
 * rac_silu_dev. */
int rac_swiglu_dev(const float *gu, float *out, long n, int iters, void *stream);

/* One-row Q8_0 GEMVs with the RMSNorm fused in: h = rmsnorm(x) *
 * norm_weight computed as rac_rmsnorm_dev does (same bits), then the GEMV
 * of rac_q8_0_gemv_dev over h (same bits).  K % 256 == 0, K <= 16384; x,
 * norm_weight and weight 16-byte aligned.  No counterpart entry point in
 * the reference, whose decoder_forward_kv calls rmsnorm (:316-332) and
 * bench_fused_linear_q8 (:301-312) one after the other. */
int rac_q8_0_gemv_rmsnorm_dev(const float *x, const float *norm_weight, float eps, const void *weight,
                              const float *bias, float *out, int N, int K, int act, void *stream);

/* The Q, K, V projection of one token (:565-574): weight holds the
 * (n_heads + 2 n_kv_heads) * d_head rows W_q, W_k, W_v over K = d_model;
 * queries to q_out [n_heads * d_head], keys and values into the caches at
 * position *pos (nothing for a position outside [0, t_cap)). */
int rac_decode_qkv_dev(const float *x, const float *norm_weight, float eps, const void *weight, float *q_out,
                       float *k_cache, float *v_cache, int n_heads, int n_kv_heads, int d_head, int K,
                       long t_cap, const int *pos, void *stream);

/* Gate and up of the SwiGLU feed-forward (:605-611): weight holds 2 n_ff
 * rows interleaved gate_0, up_0, gate_1, up_1, ...; out[i] = silu(gate_i .
 * h) * (up_i . h), SiLU by the CORDIC exp at `iters` steps. */
int rac_decode_swiglu_gemv_dev(const float *x, const float *norm_weight, float eps, const void *weight,
                               float *out, int n_ff, int K, int iters, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* RAC_DECODE_H */
