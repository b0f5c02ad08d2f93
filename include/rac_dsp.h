/*
 * rac_dsp.h — the RAC-DSP fixed-point CORDIC engine on MI355X.
 *
 * Same entry points as the reference's bit-exact RTL model
 * (sim/rac_dsp_core.h:32-58), evaluated by gfx950 kernels of librac_amd.so,
 * plus asynchronous device-memory forms.  Operands: x, y in Q32.32, z in
 * Q0.63 fractions of pi, all int64 with wrapping arithmetic.  op: 0 rotate,
 * 1 project, 2 vectoring, 3 hyperbolic (any other value evaluates as a
 * circular rotation, as the reference does).
 *
 * ROMs: the library generates the coarse-LUT, atan and atanh contents by the
 * rule of rtl/gen_coarse_lut.py (identical to rtl/cordic_*.mem); the
 * loaders below replace them for every later call.  Replacing ROMs while
 * RAC-DSP kernels are still running on another stream races with them.
 */
#ifndef RAC_AMD_RAC_DSP_H
#define RAC_AMD_RAC_DSP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RAC_DSP_WIDTH           64
#define RAC_DSP_LUT_BITS        10
#define RAC_DSP_RESIDUAL        9
#define RAC_DSP_RESIDUAL_START  8
#define RAC_DSP_LUT_SIZE        (1 << RAC_DSP_LUT_BITS)
#define RAC_DSP_ATAN_ROM_SIZE   (RAC_DSP_RESIDUAL_START + RAC_DSP_RESIDUAL)

typedef int64_t rac_q_t;

/* Replaces sim/rac_dsp_core.h:32 — parse a $readmemh-style hex file (blank
 * lines and // comments skipped); returns the count parsed, -1 on error. */
int rac_load_hex_lut(const char *path, uint64_t *out, int expected);

/* Replaces sim/rac_dsp_core.h:36-38 — load the three ROM files; 0 on
 * success, 1 / 2 / 3 when the LUT / atan / atanh file cannot be read (the
 * ROMs in use are then unchanged). */
int rac_load_all_roms(const char *coarse_lut_path, const char *atan_path, const char *atanh_path);

/* Replaces direct assignment to the reference's ROM globals
 * (sim/rac_dsp_core.h:23-27); a null pointer keeps that ROM. */
void rac_dsp_set_roms(const uint64_t *lut, const rac_q_t *atan_rom, const rac_q_t *atanh_rom);

/* Host copy of the ROMs in use (RAC_DSP_LUT_SIZE, RAC_DSP_ATAN_ROM_SIZE and
 * RAC_DSP_RESIDUAL entries; null pointers skipped). */
void rac_dsp_get_roms(uint64_t *lut, rac_q_t *atan_rom, rac_q_t *atanh_rom);

/* Replaces sim/rac_dsp_core.h:42-43 — one evaluation (synchronous). */
void rac_dsp_eval(rac_q_t x_in, rac_q_t y_in, rac_q_t z_in, int op, rac_q_t *x_out, rac_q_t *y_out,
                  rac_q_t *z_out);

/* Replaces sim/rac_dsp_core.h:48-50 — x_out[i] = project(xs[i], 0, zs[i]).x.
 * Host or device pointers; synchronous. */
void rac_dsp_project_batch(int n, const rac_q_t *xs, const rac_q_t *zs, rac_q_t *x_out);

/* Replaces sim/rac_dsp_core.h:56-58 — the wrapping sum of those n
 * projections (one systolic column). */
rac_q_t rac_dsp_project_sum(int n, const rac_q_t *xs, const rac_q_t *zs);

/* Device-memory batch evaluation on `stream` (hipStream_t; null = default):
 * (xo, yo, zo)[i] = eval(x[i], y ? y[i] : 0, z[i], op).  x, z, xo are
 * required; yo, zo may be null.  Returns 0 or a RAC_ERR_* code
 * (rac_last_error() has the message). */
int rac_dsp_eval_dev(int op, long n, const rac_q_t *x, const rac_q_t *y, const rac_q_t *z, rac_q_t *xo,
                     rac_q_t *yo, rac_q_t *zo, void *stream);

/* Device-memory weight-stationary systolic product, the computation of
 * sim/rac_systolic_ref.c:40-55 for a batch of K activation vectors:
 * Y[k][c] = sum_r project(X[k][r], 0, W[r][c]).x  (W: N x N angles,
 * X, Y: K x N, row-major, wrapping sums). */
int rac_dsp_systolic_dev(int N, int K, const rac_q_t *W, const rac_q_t *X, rac_q_t *Y, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* RAC_AMD_RAC_DSP_H */
