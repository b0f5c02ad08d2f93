/*
 * rac_q8_0.h — Q8_0 weight blocks and the decode GEMV of librac_amd.so on
 * MI355X (gfx950).  Drop-in for the reference lib/c/rac_q8_0.h:35-100:
 * same block layout, names, argument lists and status codes; the work runs
 * on the GPU.  Buffers may be host or device memory (classified per call,
 * like rac.h); calls are synchronous.  rac_fp16_to_fp32 / rac_fp32_to_fp16
 * are the scalar format helpers and run on the host.
 *
 * Results are bit-identical to the reference's AVX2 build for activation
 * NONE and RELU, and within the device erff/expf rounding for GELU and SiLU.
 */
#ifndef RAC_Q8_0_H
#define RAC_Q8_0_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RAC_Q8_0_BLOCK_SIZE 32

/* rac_q8_0.h:35-38: one fp16 scale, 32 int8 weights; 34 bytes, packed. */
typedef struct {
    uint16_t d;
    int8_t qs[RAC_Q8_0_BLOCK_SIZE];
} rac_q8_0_block;

/* activation ids (rac_cpu.h:176-181) */
#define RAC_Q8_ACT_NONE 0
#define RAC_Q8_ACT_RELU 1
#define RAC_Q8_ACT_GELU 2
#define RAC_Q8_ACT_SILU 3

/* rac_q8_0.h:47-48 (host, IEEE half; fp32 -> fp16 truncates the mantissa) */
float rac_fp16_to_fp32(uint16_t h);
uint16_t rac_fp32_to_fp16(float f);

/* rac_q8_0.h:56-68: per-block amax / 127 scale, q = lrintf(x / d) clamped
 * to [-127, 127].  N, K multiples of 32. */
void rac_q8_0_quantize_row(const float *src, rac_q8_0_block *dst, int N);
void rac_q8_0_quantize_matrix(const float *src, rac_q8_0_block *dst, int rows, int K);
/* rac_q8_0.h:72 */
void rac_q8_0_dequantize_row(const rac_q8_0_block *src, float *dst, int N);

/* rac_q8_0.h:94-100: output[N] = act(weight[N, K/32] @ input[K] + bias);
 * returns 0 (RAC_OK) or -1 null pointer / -2 bad dimension / -3 allocation
 * / -4 HIP error; act as above. */
int rac_q8_0_gemv(const float *input, const rac_q8_0_block *weight, const float *bias,
                  float *output, int N, int K, int act);

/* Device-buffer, stream-ordered forms (same conventions as rac_ext.h).
 * gemv_dev takes M input rows x[M, K] (batched decode; the weights stream
 * from HBM once per 8 rows) and writes out[M, N]. */
int rac_q8_0_gemv_dev(const float *x, const void *weight, const float *bias, float *out, int M,
                      int N, int K, int act, void *stream);
int rac_q8_0_quantize_dev(const float *src, void *dst, long rows, int K, void *stream);
int rac_q8_0_dequantize_dev(const void *src, float *dst, long rows, int K, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* RAC_Q8_0_H */
