// rac_tables.hpp — CORDIC constants shared by the gfx950 kernels and the
// host shim.  All values are compile-time; the direction sequences and the
// per-step constants are derived here with constexpr float arithmetic, which
// clang evaluates with IEEE single-precision round-to-nearest — the same
// rounding the kernels and the CPU checker use at run time.
#pragma once
#include <stdint.h>

namespace rac {

// atan(2^-i), i = 0..23, each value printed to 8 decimals: the circular
// table of rac_kernels.hip:32-39 (== rac_cpu.c:20-40).  Results of
// rac_rope_cache are bit-exact only with these exact floats.
constexpr float kAtan[24] = {
    0.78539816f, 0.46364761f, 0.24497866f, 0.12435499f,
    0.06241881f, 0.03123983f, 0.01562373f, 0.00781234f,
    0.00390623f, 0.00195312f, 0.00097656f, 0.00048828f,
    0.00024414f, 0.00012207f, 0.00006104f, 0.00003052f,
    0.00001526f, 0.00000763f, 0.00000381f, 0.00000191f,
    0.00000095f, 0.00000048f, 0.00000024f, 0.00000012f,
};

// atanh(2^-s), s = 1..16: the hyperbolic table of rac_cpu.c:27-32 (its
// entries are not one rounding rule, so they are carried as data).  s > 16
// are exactly 2^-s in float (atanh(2^-s) = 2^-s (1 + 4^-s/3 + ...)).
constexpr float kAtanh16[17] = {
    0.0f,
    0.54930614f, 0.25541281f, 0.12565721f, 0.06258157f,
    0.03126017f, 0.01562627f, 0.00781265f, 0.00390626f,
    0.00195313f, 0.00097656f, 0.00048828f, 0.00024414f,
    0.00012207f, 0.00006104f, 0.00003052f, 0.00001526f,
};

// K-hat(n), the circular gain table of rac_kernels.hip:42-50, value for
// value (it departs from prod sqrt(1 + 4^-i) beyond n = 2, and CORDIC-mode
// matmul results depend on it).
constexpr float kKhat[25] = {
    1.00000000f, 1.41421356f, 1.58113883f, 1.62979295f,
    1.64248460f, 1.64568447f, 1.64648404f, 1.64668388f,
    1.64673383f, 1.64674632f, 1.64674944f, 1.64675022f,
    1.64675042f, 1.64675047f, 1.64675048f, 1.64675049f,
    1.64675049f, 1.64675049f, 1.64675049f, 1.64675049f,
    1.64675049f, 1.64675049f, 1.64675049f, 1.64675049f,
    1.64675049f,
};

constexpr float kPi = 3.14159265358979f;    // RAC_PI
constexpr float kTau = 6.28318530717958f;   // == 2.0f * RAC_PI
constexpr float kKInv = 0.60725f;           // RAC_K_INV
constexpr float kLn2 = 0.69314718056f;      // rac_alu.c:558
constexpr float kInvLn2 = 1.44269504089f;   // rac_alu.c:559

constexpr int kMaxIters = 24;

constexpr float pow2(int e) {
    float r = 1.0f;
    if (e >= 0) for (int i = 0; i < e; i++) r *= 2.0f;
    else for (int i = 0; i < -e; i++) r *= 0.5f;
    return r;
}

// Direction of micro-rotation i of a circular rotation that starts at angle
// 0 — the angle-index stage of CORDIC-mode matmul, data independent
// (rac_kernels.hip:152-159 with theta = 0 after the +-pi pre-rotation).
constexpr int cordic_dir(int i) {
    float angle = 0.0f;
    int d = 1;
    for (int j = 0; j <= i; j++) {
        d = (angle >= 0.0f) ? 1 : -1;
        angle -= (float)d * kAtan[j];
    }
    return d;
}

// +---+-++----++--++--+--+ : the sequence the reference's kernel walks for
// every MAC.  Checked here at compile time.
constexpr bool dirs_match(const char* s) {
    for (int i = 0; i < 24; i++)
        if ((s[i] == '+' ? 1 : -1) != cordic_dir(i)) return false;
    return true;
}
static_assert(dirs_match("+---+-++----++--++--+--+"), "CORDIC direction table");

// Strength-reduced micro-rotation constants.  After micro-rotations 0 and 1
// (which map (a, 0) to (fl(1.5a), a/2) exactly), y is carried as yh = 2y so
// step i (i >= 2) is x += kCx[i]*yh ; yh += kCy[i]*x(old).
constexpr float chain_cx(int i) { return -(float)cordic_dir(i) * pow2(-i - 1); }
constexpr float chain_cy(int i) { return (float)cordic_dir(i) * pow2(1 - i); }

// 1.0f / K-hat(n) (rac_kernels.hip:183), correctly rounded at compile time.
constexpr float cordic_kinv(int n) { return 1.0f / kKhat[n]; }

// Walther hyperbolic shift schedule: 1,2,3,4,4,5,...,13,13,14,...,40,40,...
constexpr int hyp_shift(int j) {
    int s = 1, idx = 0, next_repeat = 4;
    while (true) {
        if (idx == j) return s;
        idx++;
        if (s == next_repeat) {
            if (idx == j) return s;
            idx++;
            next_repeat = 3 * next_repeat + 1;
        }
        s++;
    }
}

constexpr float atanh_pow2(int s) { return s <= 16 ? kAtanh16[s] : pow2(-s); }
// Per-step constants of the product-register exp: S = 2^-s, C = atanh(2^-s) 2^s
constexpr float hyp_S(int j) { return pow2(-hyp_shift(j)); }
constexpr float hyp_C(int j) { return atanh_pow2(hyp_shift(j)) * pow2(hyp_shift(j)); }

constexpr int kRsqrtSteps = 16;   // hyperbolic-vectoring steps of rac_rsqrt

}  // namespace rac
