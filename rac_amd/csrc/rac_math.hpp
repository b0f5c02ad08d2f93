// rac_math.hpp — per-element CORDIC arithmetic of the gfx950 kernels.
//
// Every function here is written so that each IEEE rounding is explicit
// (sources are compiled with -ffp-contract=off; fused steps are spelled
// __builtin_fmaf).  The CPU checker in oracle/rac_oracle.c evaluates the
// same roundings, so results agree bit for bit.
#pragma once
#include <hip/hip_runtime.h>
#include "rac_tables.hpp"

namespace rac {

__device__ __forceinline__ float as_f(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t as_u(float f) { return __float_as_uint(f); }

// 16-byte streaming (non-temporal) global load/store: data touched once.
typedef float v4f __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld4_stream(const float4* p) {
    const v4f v = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st4_stream(float4* p, float4 v) {
    const v4f w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, reinterpret_cast<v4f*>(p));
}

// ── CORDIC-mode MAC (rac_kernels.hip:140-185) ────────────────────────────
//
// R_n(x0): x output of n circular micro-rotations of (x0, 0) starting at
// angle 0 (directions cordic_dir(i)).  Micro-rotation 0 maps (x0, 0) to
// (x0, x0); micro-rotation 1 gives (fl(1.5 x0), x0/2), the latter exact, so
// y is carried doubled (yh = x0); each later micro-rotation is two FMAs with
// power-of-two constants; the final y update is never needed.  Bit-identical
// to the literal chain for all finite x0 whose products stay normal.
// Micro-rotation i >= 2 of the chain, constants forced to compile time.
template <int N, int I>
struct ChainStep {
    __device__ __forceinline__ static void run(float& x, float& yh) {
        constexpr float cx = chain_cx(I);
        constexpr float cy = chain_cy(I);
        const float xn = __builtin_fmaf(cx, yh, x);
        if constexpr (I + 1 < N) {
            yh = __builtin_fmaf(cy, x, yh);
            x = xn;
            ChainStep<N, I + 1>::run(x, yh);
        } else {
            x = xn;
        }
    }
};

template <int N>
__device__ __forceinline__ float cordic_rot_x(float x0) {
    static_assert(N >= 1 && N <= kMaxIters, "iteration count");
    if constexpr (N == 1) {
        return x0;
    } else {
        float x = x0 * 1.5f;
        float yh = x0;
        if constexpr (N > 2) ChainStep<N, 2>::run(x, yh);
        return x;
    }
}

// E independent rotations advanced step-major (micro-rotation i of every
// chain before micro-rotation i+1 of any): the chains interleave in the
// instruction stream, so even a SIMD holding a single wave has independent
// FMAs to issue back to back.  Bit-identical to E calls of cordic_rot_x<N>.
template <int N, int I, int E>
struct ChainStepV {
    __device__ __forceinline__ static void run(float* x, float* yh) {
        constexpr float cx = chain_cx(I);
        constexpr float cy = chain_cy(I);
        if constexpr (I + 1 < N) {
#pragma unroll
            for (int e = 0; e < E; e++) {
                const float xn = __builtin_fmaf(cx, yh[e], x[e]);
                yh[e] = __builtin_fmaf(cy, x[e], yh[e]);
                x[e] = xn;
            }
            ChainStepV<N, I + 1, E>::run(x, yh);
        } else {
#pragma unroll
            for (int e = 0; e < E; e++) x[e] = __builtin_fmaf(cx, yh[e], x[e]);
        }
    }
};

// x[e] <- R_N(x[e]) for E values at once.
template <int N, int E>
__device__ __forceinline__ void cordic_rot_x_vec(float* x) {
    static_assert(N >= 1 && N <= kMaxIters, "iteration count");
    if constexpr (N > 1) {
        float yh[E];
#pragma unroll
        for (int e = 0; e < E; e++) {
            yh[e] = x[e];
            x[e] = x[e] * 1.5f;
        }
        if constexpr (N > 2) ChainStepV<N, 2, E>::run(x, yh);
    }
}

// Constant tables for the run-time iteration count paths (wave-uniform
// indices -> scalar loads).  Built from the same constexpr definitions.
struct StepTables {
    float cx[kMaxIters];
    float cy[kMaxIters];
    float dir[kMaxIters];
    float hS[kMaxIters];
    float hC[kMaxIters];
};
constexpr StepTables make_step_tables() {
    StepTables t{};
    for (int i = 0; i < kMaxIters; i++) {
        t.cx[i] = chain_cx(i);
        t.cy[i] = chain_cy(i);
        t.dir[i] = (float)cordic_dir(i);
        t.hS[i] = hyp_S(i);
        t.hC[i] = hyp_C(i);
    }
    return t;
}
static __constant__ StepTables g_steps = make_step_tables();

// The same chain with a run-time iteration count; used for n outside the
// specialised set.
__device__ __forceinline__ float cordic_rot_x_rt(float x0, int n) {
    if (n == 1) return x0;
    float x = x0 * 1.5f;
    float yh = x0;
    for (int i = 2; i < n; i++) {
        const float xn = __builtin_fmaf(g_steps.cx[i], yh, x);
        yh = __builtin_fmaf(g_steps.cy[i], x, yh);
        x = xn;
    }
    return x;
}

// The micro-rotation chain exactly as rac_kernels.hip:152-163 writes it:
// x' = x - d*y*scale, y' = y + d*x*scale, every product and sum rounded on
// its own (d*y is exact, (d*y)*scale may round once it is subnormal).  The
// strength-reduced chain above equals it bit for bit whenever
// 2^-105 <= |x0| < 2^127 (exhaustive over every float in that range, n = 1..24);
// outside it (subnormal and tiny inputs, the top binade, inf, NaN) the GEMM
// runs this form instead.  Here on E values one after the other (the GEMM
// takes it only for rare tiles, so it is written for few live registers, not
// for speed): x[e] <- x output of rotating (x[e], 0).
template <int N, int E>
__device__ __forceinline__ void cordic_rot_x_literal_vec(float* x) {
#pragma unroll
    for (int e = 0; e < E; e++) {
        float xv = x[e], y = 0.0f, scale = 1.0f;
#pragma unroll
        for (int i = 0; i < N; i++) {
            const float d = (float)cordic_dir(i);
            const float xn = xv - (d * y) * scale;
            const float yn = y + (d * xv) * scale;
            xv = xn;
            y = yn;
            scale *= 0.5f;
        }
        x[e] = xv;
        __builtin_amdgcn_sched_barrier(0);   // keep the chains apart: no interleaving
    }
}

__device__ __forceinline__ float cordic_rot_x_literal_rt(float x0, int n) {
    float x = x0, y = 0.0f, scale = 1.0f;
    for (int i = 0; i < n; i++) {
        const float d = g_steps.dir[i];
        const float xn = x - (d * y) * scale;
        const float yn = y + (d * x) * scale;
        x = xn;
        y = yn;
        scale *= 0.5f;
    }
    return x;
}

// The inputs whose rotation must take the literal chain: nonzero with
// |x0| < 2^-105 or |x0| >= 2^127 (inf and NaN included).  For a set of
// inputs given by lo_m1 = min(|x|bits - 1) (unsigned: zeros wrap to the
// top) and hi = max(|x|bits): true when any member needs it.
__device__ __forceinline__ bool cordic_range_needs_literal(uint32_t lo_m1, uint32_t hi) {
    return lo_m1 < (22u << 23) - 1u || hi >= (254u << 23);
}
__device__ __forceinline__ bool cordic_needs_literal(float x0) {
    const uint32_t u = as_u(x0) & 0x7fffffffu;
    return cordic_range_needs_literal(u - 1u, u);
}

// One CORDIC-mode multiply-accumulate: b is the angle index (sign -> 0 or pi,
// applied as a negation of (a, 0)) and magnitude |b|; the rotated x, gain
// compensated by kinv, is projected on |b| and accumulated by one FMA.
// `bsign` is b's sign bit, extracted once per B element by the caller.
template <int N>
__device__ __forceinline__ float mac_cordic(float a, float b, uint32_t bsign, float acc) {
    const float x0 = as_f(as_u(a) ^ bsign);
    const float xr = cordic_rot_x<N>(x0);
    return __builtin_fmaf(xr * cordic_kinv(N), __builtin_fabsf(b), acc);
}

// ── SHIFTADD-mode product (rac_kernels.hip:85-122) ───────────────────────
__device__ __forceinline__ float shiftadd_mul(float a, float b, int iters) {
    if (a == 0.0f || b == 0.0f) return 0.0f;
    const uint32_t ai = as_u(a), bi = as_u(b);
    const uint32_t sign = (ai ^ bi) & 0x80000000u;
    const int exp_a = (int)((ai >> 23) & 0xFFu) - 127;
    const int exp_b = (int)((bi >> 23) & 0xFFu) - 127;
    const uint64_t ma = 0x00800000u | (ai & 0x007FFFFFu);
    const uint32_t mb = 0x00800000u | (bi & 0x007FFFFFu);
    // top `lim` bits of mb, each adding ma at its weight: the bit-serial sum
    // equals ma * (mb with the low 24-lim bits cleared); written as a loop of
    // shifts and masked adds (no multiplier), as the reference does.
    uint64_t prod = 0;
    const int lim = iters < 1 ? 1 : (iters > 24 ? 24 : iters);
    for (int i = 0; i < lim; i++) {
        const uint64_t bit = (mb >> (23 - i)) & 1u;
        prod += (ma << (23 - i)) & (0ull - bit);
    }
    if (prod == 0) return 0.0f;
    const int top = 63 - __clzll((long long)prod);
    const int shift_r = top - 23;
    uint32_t mantissa;
    if (shift_r > 0) mantissa = (uint32_t)(prod >> shift_r) & 0x007FFFFFu;
    else if (shift_r < 0) mantissa = (uint32_t)(prod << -shift_r) & 0x007FFFFFu;
    else mantissa = (uint32_t)prod & 0x007FFFFFu;
    const int rexp = exp_a + exp_b + (top - 46) + 127;
    if (rexp <= 0 || rexp >= 0xFF) return 0.0f;
    return as_f(sign | ((uint32_t)(rexp & 0xFF) << 23) | mantissa);
}

// ── Hyperbolic CORDIC e^x (product-register form) ────────────────────────
//
// Range reduction k = trunc(fma(x, 1/ln2, +-0.5)), r = fma(-k, ln2, x)
// (rac_alu.c:560-561 as its build contracts them); then n Walther steps on
// the sum register p = x + y of the hyperbolic rotation of (1, 0) by r:
// p <- p (1 + d 2^-s) as one FMA, z <- z - d atanh(2^-s) as one FMA with
// the constant atanh(2^-s) 2^s, d = copysign(1, z) (rac_alu.c:246).  Output
// (p / K_h(n)) 2^k through the exponent field (rac_alu.c:572-581).
// t = fma(x, 1/ln2, +-0.5) truncated; (x >= 0 ? 0.5 : -0.5) is written as
// copysign(0.5, x): they differ only at x = -0, where both truncate to 0.

// float -> int32 by v_cvt_i32_f32: truncation toward zero, out-of-range
// values saturate to INT32_MIN / INT32_MAX, NaN gives 0.  C's (int) cast of
// such values is undefined, so the instruction is named directly.  For the
// exp this is exact: |t| >= 2^31 means |x| > 1.4e9, where the result is
// inf or 0 (k far outside -149..127) whatever the saturated k and r are.
__device__ __forceinline__ int cvt_i32_sat(float t) {
    int r;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(t));
    return r;
}

__device__ __forceinline__ void exp_reduce(float x, int& k, float& r) {
    const float t = __builtin_fmaf(x, kInvLn2, __builtin_copysignf(0.5f, x));
    k = cvt_i32_sat(t);
    r = __builtin_fmaf(-(float)k, kLn2, x);
}

// er * 2^k with the reference's exponent-field semantics (k + 127 <= 0 ->
// 0; k + 127 > 254 -> er * inf = +inf, er being positive; otherwise the
// product er * 2^k, rounded once).  v_ldexp_f32 computes er * 2^k with one
// rounding for every k; the two ends need selects: k <= -127 flushes, and
// k = 128 with er < 1 (x in [127.5 ln2, 88.72)) would still be finite.
__device__ __forceinline__ float exp_scale(float er, int k) {
    const float res = __builtin_ldexpf(er, k);
    return (k <= -127) ? 0.0f : (k > 127 ? __builtin_inff() : res);
}

// Step J of the product-register exp, constants forced to compile time.
template <int N, int J>
struct HypStep {
    __device__ __forceinline__ static void run(float& p, float& z) {
        constexpr float S = hyp_S(J);
        constexpr float C = hyp_C(J);
        const float ds = __builtin_copysignf(S, z);
        p = __builtin_fmaf(ds, p, p);
        if constexpr (J + 1 < N) {
            z = __builtin_fmaf(-ds, C, z);
            HypStep<N, J + 1>::run(p, z);
        }
    }
};

template <int N>
__device__ __forceinline__ float exp_cordic(float x, float khinv) {
    static_assert(N >= 1 && N <= kMaxIters, "iteration count");
    int k;
    float r;
    exp_reduce(x, k, r);
    float p = 1.0f, z = r;
    HypStep<N, 0>::run(p, z);
    const float res = exp_scale(p * khinv, k);
    return (x != x) ? x : res;
}

// The same exp on E independent arguments, step-major: step J is applied to
// all E registers before step J+1, so the E dependency chains interleave
// and each step's constants are materialised once.  Bit-identical to E
// calls of exp_cordic<N>.
template <int N, int J, int E>
struct HypStepV {
    __device__ __forceinline__ static void run(float* p, float* z) {
        constexpr float S = hyp_S(J);
        constexpr float C = hyp_C(J);
#pragma unroll
        for (int e = 0; e < E; e++) {
            const float ds = __builtin_copysignf(S, z[e]);
            p[e] = __builtin_fmaf(ds, p[e], p[e]);
            if constexpr (J + 1 < N) z[e] = __builtin_fmaf(-ds, C, z[e]);
        }
        if constexpr (J + 1 < N) HypStepV<N, J + 1, E>::run(p, z);
    }
};

//
// OPT drops stages a caller makes redundant (each saves VALU issue slots;
// none changes a result the caller keeps):
//   kExpNan    NaN arguments return themselves.  Without it a NaN argument
//              gives an unspecified finite value or inf: fine for x / (1 + e)
//              (SiLU), whose result is NaN through x.
//   kExpFlush  k <= -127 gives +0 as the reference's exponent field does.
//              Without it those k give er * 2^k (a subnormal or 0): fine
//              wherever the exp only enters 1 + e or 1 - e, which round to
//              1 alike for any e < 2^-24.
//   kExpNonPos every argument is <= 0 or NaN (softmax's x - max), so the
//              rounding bias copysign(0.5, x) is the constant -0.5: at x = +0
//              both biases truncate to k = 0, below 0 they are equal; and
//              k <= 0, so the overflow select (k > 127 -> inf) is dropped.
//   kExpNoOvf  every argument is below 88 (k <= 127), so the overflow
//              select is dropped; the rounding bias keeps its sign.
//   kExpNegArg x holds v and the exp is of -v, with exp_reduce(-v)'s
//              operands: copysign(0.5, -v) by one v_bitop3 (mask ? 0.5 :
//              ~v) and -v as source modifiers of the two FMAs, instead of
//              a v_xor that materialises -v (1 VALU per element fewer).
constexpr int kExpNan = 1, kExpFlush = 2, kExpNonPos = 4, kExpNoOvf = 8, kExpNegArg = 16;
constexpr int kExpFull = kExpNan | kExpFlush;

template <int N, int E, int OPT = kExpFull>
__device__ __forceinline__ void exp_cordic_vec(float* x, float khinv) {
    static_assert(N >= 1 && N <= kMaxIters, "iteration count");
    int k[E];
    float p[E], z[E];
#pragma unroll
    for (int e = 0; e < E; e++) {
        if constexpr ((OPT & kExpNonPos) != 0) {
            k[e] = cvt_i32_sat(__builtin_fmaf(x[e], kInvLn2, -0.5f));
            z[e] = __builtin_fmaf(-(float)k[e], kLn2, x[e]);
        } else if constexpr ((OPT & kExpNegArg) != 0) {
            const float b = as_f(__builtin_amdgcn_bitop3_b32(0x7fffffffu, 0x3f000000u, as_u(x[e]), 0xC5));
            k[e] = cvt_i32_sat(__builtin_fmaf(-x[e], kInvLn2, b));
            z[e] = __builtin_fmaf(-(float)k[e], kLn2, -x[e]);
        } else {
            exp_reduce(x[e], k[e], z[e]);
        }
        p[e] = 1.0f;
    }
    HypStepV<N, 0, E>::run(p, z);
#pragma unroll
    for (int e = 0; e < E; e++) {
        const float er = p[e] * khinv;
        float res = __builtin_ldexpf(er, k[e]);
        if constexpr ((OPT & kExpFlush) != 0) res = (k[e] <= -127) ? 0.0f : res;
        if constexpr ((OPT & (kExpNonPos | kExpNoOvf)) == 0) res = (k[e] > 127) ? __builtin_inff() : res;
        if constexpr ((OPT & kExpNan) != 0) x[e] = (x[e] != x[e]) ? x[e] : res;
        else x[e] = res;
    }
}

__device__ __forceinline__ float exp_cordic_rt(float x, int n, float khinv) {
    int k;
    float r;
    exp_reduce(x, k, r);
    float p = 1.0f, z = r;
    for (int j = 0; j < n; j++) {
        const float ds = __builtin_copysignf(g_steps.hS[j], z);
        p = __builtin_fmaf(ds, p, p);
        z = __builtin_fmaf(-ds, g_steps.hC[j], z);
    }
    const float res = exp_scale(p * khinv, k);
    return (x != x) ? x : res;
}

// ── rsqrt by hyperbolic vectoring ────────────────────────────────────────

// Vectoring step J (d = -sign(Y)), constants forced to compile time.
template <int N, int J>
struct VecStep {
    __device__ __forceinline__ static void run(float& X, float& Y) {
        constexpr float S = hyp_S(J);
        const float ds = __builtin_copysignf(S, Y);
        const float Xn = __builtin_fmaf(-ds, Y, X);
        const float Yn = __builtin_fmaf(-ds, X, Y);
        X = Xn;
        Y = Yn;
        if constexpr (J + 1 < N) VecStep<N, J + 1>::run(X, Y);
    }
};
//
// rac_rsqrt's contract (rac_cpu.c:330-335): v <= 0 -> 0, NaN -> NaN,
// +inf -> 0.  v = m 4^e, m in [0.5, 2); vectoring (m + 1/4, m - 1/4) to
// y = 0 leaves x = K_h sqrt(m); 1/sqrt(v) = (1 / (x / K_h)) 2^-e.
// khinv16 = 1/K_h over the 16-step schedule (host computed).
__device__ __forceinline__ float rsqrt_cordic(float v, float khinv16) {
    if (v != v) return v;
    if (!(v > 0.0f) || v == __builtin_inff()) return 0.0f;
    int ex = __builtin_amdgcn_frexp_expf(v);
    float mant = __builtin_amdgcn_frexp_mantf(v);   // v = mant 2^ex, mant in [0.5, 1)
    float m;
    int e;
    if (ex & 1) { m = mant * 2.0f; e = (ex - 1) / 2; }
    else { m = mant; e = ex / 2; }
    float X = m + 0.25f, Y = m - 0.25f;
    VecStep<kRsqrtSteps, 0>::run(X, Y);
    const float root = X * khinv16;
    const float r = 1.0f / root;
    return __builtin_ldexpf(r, -e);
}

// ── Circular CORDIC sin/cos (rac_cpu.c:90-118, 322-328) ──────────────────

// Rotation step I: d from the residual angle (angle >= 0 -> +1), x/y moved by
// d*y*2^-I exactly as written in the reference (the products are exact).
template <int N, int I>
struct CircStep {
    __device__ __forceinline__ static void run(float& x, float& y, float& angle) {
        constexpr float scale = pow2(-I);
        constexpr float at = kAtan[I];
        const float d = (angle >= 0.0f) ? 1.0f : -1.0f;
        const float xn = x - d * y * scale;
        const float yn = y + d * x * scale;
        angle -= d * at;
        x = xn;
        y = yn;
        if constexpr (I + 1 < N) CircStep<N, I + 1>::run(x, y, angle);
    }
};
// One 16-step rotation of (K_INV, 0) by theta, with the reference's
// sequential float wrap of theta into (-pi, pi] (rac_cpu.c:92-94: a loop of
// rounded subtractions, not a remainder: its drift at large angles is part
// of the table's values).  The reference's wrap loop never terminates for
// |theta| >= 2^27 or +-inf (theta - 2pi rounds back to theta); such angles
// return NaN here instead.
constexpr float kWrapLimit = 134217728.0f;   // 2^27

// The reference's subtractions a <- fl(a - tau) while a >= 16, done a
// binade at a time (a = |theta|, a in [2^e, 2^(e+1)), 4 <= e <= 26).  On
// the binade's grid (spacing u = 2^(e-23)) let T be tau rounded to a
// multiple of u: tau / u never has fractional part 1/2 for these e, so
// |T - tau| < u / 2, and every step whose exact result a - tau stays >= 2^e
// rounds to exactly a - T.  Those are the steps i = 1 .. k with
// k = floor((m - c) / t) + 1 (m the mantissa field of a, t = T / u, c =
// ceil(tau / u): all in units of u), taken at once by one exact fma; the
// step that leaves the binade is then taken as the reference takes it.  So
// the result is the loop's, bit for bit, in at most ~23 passes instead of
// up to a / 2pi subtractions.
__device__ __forceinline__ float wrap_binades(float a) {
    while (a >= 16.0f) {
        const uint32_t bits = __builtin_bit_cast(uint32_t, a);
        const int e = (int)(bits >> 23) - 127;
        const int m = (int)(bits & 0x7FFFFFu);
        const float u = __builtin_ldexpf(1.0f, e - 23);
        const float tq = kTau * __builtin_ldexpf(1.0f, 23 - e);    // tau / u, exact
        const int t = (int)__builtin_rintf(tq), c = (int)__builtin_ceilf(tq);
        if (m >= c) {
            const int k = (m - c) / t + 1;
            a = __builtin_fmaf(-(float)k, (float)t * u, a);          // a - k T, exact
        }
        a = a - kTau;
    }
    return a;
}

__device__ __forceinline__ void sincos_cordic(float theta, float& s, float& c) {
    if (!(__builtin_fabsf(theta) < kWrapLimit)) {
        s = c = __builtin_nanf("");
        return;
    }
    // fl(theta + tau) = -fl(-theta - tau) (round to nearest is odd), so the
    // negative side runs the same subtractions on |theta|
    if (theta > kPi) theta = wrap_binades(theta);
    else if (theta <= -kPi) theta = -wrap_binades(-theta);
    while (theta > kPi) theta -= kTau;
    while (theta <= -kPi) theta += kTau;
    float x = kKInv, y = 0.0f;
    if (theta > kPi * 0.5f) { x = -x; y = -y; theta -= kPi; }
    else if (theta < -kPi * 0.5f) { x = -x; y = -y; theta += kPi; }
    float angle = theta;
    CircStep<16, 0>::run(x, y, angle);
    c = x;
    s = y;
}

}  // namespace rac
