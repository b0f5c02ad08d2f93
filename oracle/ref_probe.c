/*
 * ref_probe.c — accessor shim compiled together with the reference lib/c.
 *
 * TEST INFRASTRUCTURE ONLY.  Built by oracle/Makefile into oracle/_ref/
 * from the reference sources where they lie (/root/reference/lib/c); the
 * reference text is never copied into this repository.  The shim exposes
 * the reference's file-static CORDIC tables and its static rotation /
 * hyperbolic cores so the clean-room oracle (rac_oracle.c) can be pinned
 * against the compiled reference bit for bit:
 *
 *   ref_tables            -> rac_cpu.c:20-52   (atan, atanh, K-hat tables)
 *   ref_cordic_rotate     -> rac_cpu.c:90-118  (_cordic_rotate)
 *   ref_cordic_hyperbolic -> rac_cpu.c:120-132 (_cordic_hyperbolic)
 *
 * Every other reference entry point (rac_matmul, rac_softmax_batch,
 * rac_rope_cache, rac_rope_apply, rac_rmsnorm, rac_layernorm, rac_silu,
 * rac_hal_matmul, rac_alu_exp, ...) is exported by the library itself.
 */
#include "rac_cpu.c"

void ref_tables(float *atan16, float *atan_ext8, float *atanh16, float *ktab25)
{
    for (int i = 0; i < 16; i++) atan16[i] = rac_atan_table[i];
    for (int i = 0; i < 8; i++) atan_ext8[i] = rac_atan_table_ext[i];
    for (int i = 0; i < 16; i++) atanh16[i] = rac_atanh_table[i];
    for (int i = 0; i < 25; i++) ktab25[i] = rac_k_table[i];
}

void ref_cordic_rotate(float vx, float vy, float theta, int iters,
                       float *ox, float *oy)
{
    rac_vec2 v = {vx, vy};
    rac_vec2 r = _cordic_rotate(v, theta, iters);
    *ox = r.x;
    *oy = r.y;
}

void ref_cordic_hyperbolic(float x, float y, float z, float *ox, float *oy)
{
    rac_vec2 r = _cordic_hyperbolic(x, y, z);
    *ox = r.x;
    *oy = r.y;
}
