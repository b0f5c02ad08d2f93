// rac_act.hpp — the activation functions shared by the elementwise kernels
// and the fused GEMM epilogue, so both produce the same bits.
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>
#include "rac_internal.hpp"
#include "rac_math.hpp"

namespace rac {

template <int OP, int NITER>
__device__ __forceinline__ float elt(float x, int iters, float khinv) {
    if constexpr (OP == kEltRelu) {
        return (x > 0.0f) ? x : 0.0f;                           // rac_cpu.c:441-445
    } else if constexpr (OP == kEltGelu) {
        return x * 0.5f * (1.0f + erff(x * 0.7071067811865f));  // rac_cpu.c:447-451
    } else {
        auto ex = [&](float v) {
            if constexpr (NITER > 0) return exp_cordic<NITER>(v, khinv);
            else return exp_cordic_rt(v, iters, khinv);
        };
        if constexpr (OP == kEltExp) {
            return ex(x);
        } else if constexpr (OP == kEltSilu) {
            return x / (1.0f + ex(-x));                         // rac_cpu.c:453-457
        } else if constexpr (OP == kEltSigmoid) {
            return 1.0f / (1.0f + ex(-x));
        } else {                                                // tanh
            const float e = ex(-2.0f * __builtin_fabsf(x));
            return __builtin_copysignf((1.0f - e) / (1.0f + e), x);
        }
    }
}

// num / den rounded to nearest, without the scale / fixup stages of the
// compiler's IEEE division: v_rcp_f32 (1 ulp), one Newton step that makes
// the reciprocal y correctly rounded, then q = num y and one remainder
// correction q + (num - den q) y (Markstein's sequence; the remainder is
// exact once q is faithful).  Used only where the scale / fixup stages are
// identities: den in [1, 2^64], num = 0 or in [2^-100, 2^100] in magnitude,
// so no operand, remainder or quotient is subnormal, infinite or NaN (a
// zero num gives +0 at every step, as the IEEE quotient does).  On that
// domain, for the activations' own denominators 1 + e, it equals the
// IEEE quotient for every float32 argument at n = 8, 16 and 24 (checked
// exhaustively on the device by tests/test_gpu_parity.py).  Without the
// Newton step one argument in 2^32 (SiLU, n = 16) rounds the other way.
__device__ __forceinline__ float div_rn_normal(float num, float den) {
    float y = __builtin_amdgcn_rcpf(den);
    y = __builtin_fmaf(__builtin_fmaf(-den, y, 1.0f), y, y);
    const float q = num * y;
    return __builtin_fmaf(__builtin_fmaf(-den, q, num), y, q);
}

// elt<OP, NITER> on E values at once: for the exp-based ops with a
// compile-time step count the E exps run step-major (exp_cordic_vec);
// bit-identical to E calls of elt<OP, NITER> (up to NaN payloads).  The
// activations only use e in 1 + e / 1 - e, so the k <= -127 flush is
// skipped, and SiLU's x / (1 + e) is NaN through x, so its exp skips the
// NaN pass-through as well.  SiLU and sigmoid divide by div_rn_normal when
// all E arguments of the lane keep it in its domain (|x| in [2^-100, 44]
// for SiLU: then 1 + e^-x < 2^64 and the quotient is normal; x >= -44 for
// sigmoid, NaN included, which propagates through the reciprocal), and by
// the IEEE division otherwise; the two give the same bits.  tanh always
// takes it: (1 - e) / (1 + e) with e = e^-2|x| in [0, 1.01) (the CORDIC
// error at n >= 8 is below 2^-7) has a numerator 0 or of magnitude >= 2^-24
// (1 - e is exact for e in [0.5, 2)) and a denominator in [1, 2.01].
template <int OP, int NITER, int E>
__device__ __forceinline__ void elt_vec(float* v, int iters, float khinv) {
    if constexpr (NITER > 0 && (OP == kEltExp || OP == kEltSilu || OP == kEltSigmoid || OP == kEltTanh)) {
        float a[E];
#pragma unroll
        for (int e = 0; e < E; e++) {
            if constexpr (OP == kEltExp) a[e] = v[e];
            else if constexpr (OP == kEltTanh) a[e] = -2.0f * __builtin_fabsf(v[e]);
            else a[e] = -v[e];
        }
        constexpr int kOpt = OP == kEltExp ? kExpFull : (OP == kEltSilu ? 0 : kExpNan);
        if constexpr (OP == kEltSilu) {
            // |x| in [2^-100, 44] on every argument of the lane: the exp of -x
            // cannot overflow (so it drops that select) and the quotient
            // x / (1 + e) is in div_rn_normal's domain; else the full exp
            // and the IEEE division.
            float mx = __builtin_fabsf(v[0]), mn = mx;
#pragma unroll
            for (int e = 1; e < E; e++) {
                mx = __builtin_fmaxf(mx, __builtin_fabsf(v[e]));
                mn = __builtin_fminf(mn, __builtin_fabsf(v[e]));
            }
            if (mx <= 44.0f && mn >= 0x1p-100f) {
#pragma unroll
                for (int e = 0; e < E; e++) a[e] = v[e];   // exp of -v (kExpNegArg)
                exp_cordic_vec<NITER, E, kExpNoOvf | kExpNegArg>(a, khinv);
#pragma unroll
                for (int e = 0; e < E; e++) v[e] = div_rn_normal(v[e], 1.0f + a[e]);
            } else {
                exp_cordic_vec<NITER, E, kOpt>(a, khinv);
#pragma unroll
                for (int e = 0; e < E; e++) v[e] = v[e] / (1.0f + a[e]);
            }
            return;
        }
        exp_cordic_vec<NITER, E, kOpt>(a, khinv);
        if constexpr (OP == kEltSigmoid) {
            float mn = v[0];
#pragma unroll
            for (int e = 1; e < E; e++) mn = __builtin_fminf(mn, v[e]);   // drops NaN: NaN lanes stay fast
            if (mn >= -44.0f) {
#pragma unroll
                for (int e = 0; e < E; e++) v[e] = div_rn_normal(1.0f, 1.0f + a[e]);
            } else {
#pragma unroll
                for (int e = 0; e < E; e++) v[e] = 1.0f / (1.0f + a[e]);
            }
            return;
        }
#pragma unroll
        for (int e = 0; e < E; e++) {
            if constexpr (OP == kEltExp) v[e] = a[e];
            else v[e] = __builtin_copysignf(div_rn_normal(1.0f - a[e], 1.0f + a[e]), v[e]);   // tanh
        }
    } else {
#pragma unroll
        for (int e = 0; e < E; e++) v[e] = elt<OP, NITER>(v[e], iters, khinv);
    }
}

// Activation ids of the fused linear path (rac_torch.cu:669-675):
// 0 identity, 1 ReLU, 2 GELU (exact erf), 3 SiLU (CORDIC exp).
constexpr int kActNone = 0, kActRelu = 1, kActGelu = 2, kActSilu = 3;

__device__ __forceinline__ float act_rt(float x, int act, int iters, float khinv) {
    switch (act) {
    case kActRelu: return elt<kEltRelu, 0>(x, iters, khinv);
    case kActGelu: return elt<kEltGelu, 0>(x, iters, khinv);
    case kActSilu: return elt<kEltSilu, 0>(x, iters, khinv);
    default: return x;
    }
}

// d act / dx at the pre-activation x, times the incoming gradient g
// (derivative formulas of rac_torch.cu:680-694; the SiLU sigmoid uses the
// same CORDIC exp as the forward pass).
__device__ __forceinline__ float act_grad(float g, float x, int act, int iters, float khinv) {
    switch (act) {
    case kActRelu: return g * ((x > 0.0f) ? 1.0f : 0.0f);
    case kActGelu: {
        const float cdf = 0.5f * (1.0f + erff(x * 0.7071067811865f));
        const float pdf = 0.3989422804f * expf(-0.5f * x * x);
        return g * (cdf + x * pdf);
    }
    case kActSilu: {
        const float sig = elt<kEltSigmoid, 0>(x, iters, khinv);
        return g * (sig * (1.0f + x * (1.0f - sig)));
    }
    default: return g;
    }
}

}  // namespace rac
