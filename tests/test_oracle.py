"""Pins of the CPU checker (oracle/rac_oracle.c) — CPU only.

Each oracle function is checked against something it was not derived from:
golden vectors written by the compiled reference (tests/golden/), the
compiled reference itself where it is built here (oracle/_ref), closed forms,
exhaustive enumeration, or libm within an analytic bound.  Map:

  tables                  golden tables.json (reference rac_cpu.c:20-52)
  orc_cordic_rotate       golden rotate.npz; compiled _cordic_rotate
  orc_cordic_chain_fast   exhaustive over all mantissas vs the literal chain
  orc_fma_cordic /
  orc_cordic_project      odd-symmetry + projection identity (exhaustive /
                          random); closed form |P(a)/a - 1| = bias of K-hat
  orc_shiftadd_mul        integer closed form ma * (mb with low bits cleared)
  orc_matmul (FAST)       2x2 known answer; golden 1024^3 samples (tolerance,
                          the reference groups k in 64-tiles)
  orc_matmul (CORDIC)     per-element bound 1e-4*|a_i|*|b_j| vs golden C
  orc_rope_cache/apply    golden rope.npz, bit-exact (incl. 4096x64 digest)
  orc_exp_xy              golden alu_exp.npz (rac_alu_exp), bit-exact
  orc_exp_n               libm within the CORDIC bound; vs orc_exp_xy
  orc_softmax_rows        iters=0: golden softmax.npz bit-exact; CORDIC: bound
  orc_rsqrt               libm 1/sqrt within 1e-6; guard cases; golden KATs
  orc_rmsnorm/layernorm   libm variant bit-exact vs golden; CORDIC within 1e-6
  orc_silu/gelu/sigmoid   libm variant vs golden; CORDIC within bound
  orc_prim/outer/dct      golden prims.npz (compiled rac_cpu.c primitives),
                          bit-exact; rac_inner within its summation-order
                          bound; closed forms (hypot/atan2, exact rotation,
                          complex product, float64 DCT-II)
  orc_fp16/fp32 convert   golden q8.npz (compiled rac_q8_0.c) bit-exact;
                          every half round-trips; IEEE closed forms
  orc_q8_0_quantize/gemv  golden q8.npz bit-exact (quantized blocks, GEMV
                          outputs for each activation); dequantize error
                          <= d/2 per weight; GEMV = float64 dot of the
                          dequantized weights within the summation bound
  orc_attention           golden attention.npz (compiled
                          rac_scaled_dot_attention) bit-exact with expf and
                          FAST products; float64 softmax attention within the
                          CORDIC bound
  orc_rmsnorm_lanes /     the left-to-right functions above with the row
  orc_layernorm_lanes /   sums regrouped: equal to them where every partial
  orc_softmax_lanes       sum is exact (integer-valued rows, rows of <= 4
                          live elements), within the reordering bound
                          otherwise; a row where the order decides the sum
                          (the lane map, butterfly and wave order of the
                          row kernels) against its hand-derived value
"""
import json
import math
import os

import numpy as np
import pytest

import raclib as rl

G = rl.GOLDEN


def npz(name):
    return np.load(os.path.join(G, name))


@pytest.fixture(scope="module")
def o():
    return rl.oracle()


def tables(o):
    a24 = np.zeros(24, np.float32)
    h24 = np.zeros(24, np.float32)
    k25 = np.zeros(25, np.float32)
    o.orc_tables(rl.p(a24), rl.p(h24), rl.p(k25))
    return a24, h24, k25


def test_tables_match_reference(o):
    a24, h24, k25 = tables(o)
    t = json.load(open(os.path.join(G, "tables.json")))
    assert np.array_equal(a24[:16], np.float32(t["atan16"]))
    assert np.array_equal(a24[16:], np.float32(t["atan_ext8"]))
    assert np.array_equal(h24[:16], np.float32(t["atanh16"]))
    assert np.array_equal(k25, np.float32(t["khat25"]))
    # extension entries s = 17..24 are exactly 2^-s
    assert np.array_equal(h24[16:], np.float32([2.0 ** -s for s in range(17, 25)]))
    # K-hat departs from the textbook gain (documented property of the data)
    true16 = np.prod([math.sqrt(1 + 4.0 ** -i) for i in range(16)])
    assert abs(k25[16] / true16 - 1 + 5.9e-6) < 2e-7


def test_rotate_matches_reference_golden(o):
    d = npz("rotate.npz")
    import ctypes as C
    bad = 0
    for vx, vy, th, it, x, y in zip(d["vx"], d["vy"], d["theta"], d["iters"], d["x"], d["y"]):
        ox, oy = C.c_float(), C.c_float()
        o.orc_cordic_rotate(float(vx), float(vy), float(th), int(it), C.byref(ox), C.byref(oy))
        bad += (np.float32(ox.value) != x) or (np.float32(oy.value) != y)
    assert bad == 0


@pytest.mark.skipif(not rl.have_ref(), reason="oracle/_ref not built")
def test_rotate_matches_compiled_reference(o):
    import ctypes as C
    r = rl.ref()
    rng = np.random.default_rng(5)
    for _ in range(5000):
        vx, vy = rng.uniform(-3, 3, 2)
        th = rng.uniform(-10000, 10000)
        it = int(rng.integers(4, 25))
        a, b, c, d = C.c_float(), C.c_float(), C.c_float(), C.c_float()
        o.orc_cordic_rotate(vx, vy, th, it, C.byref(a), C.byref(b))
        r.ref_cordic_rotate(vx, vy, th, it, C.byref(c), C.byref(d))
        assert (a.value, b.value) == (c.value, d.value)


def test_direction_sequence(o):
    d = (np.zeros(24, np.int32))
    o.orc_cordic_dirs(24, rl.p(d))
    assert "".join("+" if v > 0 else "-" for v in d) == "+---+-++----++--++--+--+"


@pytest.mark.parametrize("iters", [1, 2, 3, 4, 8, 12, 16, 20, 24])
def test_fast_chain_exhaustive(o, iters):
    # all 2^23 mantissas at exponent 0 and at spot exponents inside the
    # range where every intermediate of both chains stays normal
    for e in (0, -60, 60):
        assert o.orc_check_chain_all_mantissas(iters, e) == 0


def test_fast_chain_range_boundary(o):
    """The GEMM runs the strength-reduced chain only for 2^-105 <= |a| < 2^127
    and the literal one elsewhere.  Both edge binades of that range agree
    for every mantissa and step count; the binades just outside it do not
    (subnormal products round differently from the fused form below, the
    doubled y overflows above), which is why the range ends there."""
    for e in (-105, 126):
        for n in range(1, 25):
            assert o.orc_check_chain_all_mantissas(n, e) == 0, (e, n)
    assert o.orc_check_chain_all_mantissas(24, -106) > 0
    assert o.orc_check_chain_all_mantissas(24, 127) > 0


@pytest.mark.parametrize("iters", [1, 5, 8, 16, 24])
def test_projection_identity(o, iters):
    assert o.orc_check_projection_identity(iters, 300000, 0xC0FFEE + iters) == 0


def test_projection_gain_bias(o):
    # P_n(a)/a - 1 is the reference's K-hat bias: -1.9e-5 at n=8,
    # +5.8e-6 at n=16 and n=24 (independent of a up to rounding)
    exp = {8: -1.9e-5, 16: 5.8e-6, 24: 5.8e-6}
    for n, b in exp.items():
        r = o.orc_cordic_project(1.0, n) - 1.0
        assert abs(r - b) < 0.1e-5 * (1 if n == 8 else 0.2) + 1e-7, (n, r)


def _shiftadd_closed_form(a, b, iters):
    a, b = np.float32(a), np.float32(b)
    if a == 0 or b == 0:
        return np.float32(0)
    ai = int(a.view(np.uint32))
    bi = int(b.view(np.uint32))
    ma = 0x800000 | (ai & 0x7FFFFF)
    mb = 0x800000 | (bi & 0x7FFFFF)
    lim = max(1, min(24, iters))
    mb_t = mb & ~((1 << (24 - lim)) - 1)
    prod = ma * mb_t
    top = prod.bit_length() - 1
    mant = (prod >> (top - 23)) & 0x7FFFFF if top >= 23 else (prod << (23 - top)) & 0x7FFFFF
    rexp = ((ai >> 23) & 0xFF) - 127 + ((bi >> 23) & 0xFF) - 127 + (top - 46) + 127
    if rexp <= 0 or rexp >= 255:
        return np.float32(0)
    sign = (ai ^ bi) & 0x80000000
    return np.uint32(sign | (rexp << 23) | mant).view(np.float32)


def test_shiftadd_closed_form(o):
    rng = np.random.default_rng(9)
    xs = np.concatenate([rng.standard_normal(3000), rng.uniform(-1e30, 1e30, 200),
                         rng.uniform(-1e-30, 1e-30, 200), [0.0, -0.0, 1.0, -1.0]]).astype(np.float32)
    for i in range(0, len(xs) - 1):
        a, b = xs[i], xs[(i * 7919 + 13) % len(xs)]
        for it in (1, 4, 8, 16, 24):
            assert np.float32(o.orc_shiftadd_mul(float(a), float(b), it)) == _shiftadd_closed_form(a, b, it)
    # at 24 bits the product is the exact product truncated toward zero
    a, b = np.float32(1.1), np.float32(3.3)
    exact = float(a) * float(b)
    got = o.orc_shiftadd_mul(float(a), float(b), 24)
    assert got <= exact and exact - got < 2 * np.spacing(np.float32(got))


def test_matmul_known_answers(o):
    A = np.array([[1, 2], [3, 4]], np.float32)
    B = np.array([[5, 6], [7, 8]], np.float32)
    d = npz("matmul.npz")
    C = rl.orc_matmul(A, B, 2, 2, 2, 24, 0)
    assert np.array_equal(C, d["kat_C"])
    assert np.array_equal(C, np.float32([[19, 22], [43, 50]]))
    # alpha/beta known answer of the reference DVT (C[0]=7, C[3]=28)
    I2 = np.eye(2, dtype=np.float32)
    C0 = np.array([[1, 2], [3, 4]], np.float32)
    Cb = rl.orc_matmul(I2, np.float32([[5, 6], [7, 8]]), 2, 2, 2, 24, 0, alpha=1.0, beta=2.0, C0=C0)
    assert Cb[0, 0] == 7 and Cb[1, 1] == 16
    for mode in (1, 2):
        Cm = rl.orc_matmul(A, B, 2, 2, 2, 16, mode)
        assert np.allclose(Cm, [[19, 22], [43, 50]], rtol=1e-4)


def test_matmul_1024_vs_reference_golden(o):
    d = npz("matmul.npz")
    M = N = K = 1024
    A = rl.gen_uniform((M, K), seed=0)
    B = rl.gen_uniform((K, N), seed=1)
    assert rl.sha256(A) == str(d["A_sha"]) and rl.sha256(B) == str(d["B_sha"])
    idx = d["idx"][::4]
    rows, cols = (idx // N).astype(np.int32), (idx % N).astype(np.int32)
    ref = d["C_samples"][::4]
    na = np.linalg.norm(A.astype(np.float64), axis=1)[rows]
    nb = np.linalg.norm(B.astype(np.float64), axis=0)[cols]
    for mode, iters in ((0, 24), (1, 8), (1, 16), (1, 24)):
        got = rl.orc_matmul_entries(A, B, M, N, K, iters, mode, rows, cols)
        err = np.abs(got.astype(np.float64) - ref)
        assert np.all(err <= 1e-4 * na * nb), (mode, iters, float((err / (na * nb)).max()))
    # the FAST-mode oracle differs from lib/c only by k-grouping
    got = rl.orc_matmul_entries(A, B, M, N, K, 24, 0, rows, cols)
    assert np.max(np.abs(got - ref)) < 1e-4


def test_matmul_literal_equals_projection_form(o):
    rng = np.random.default_rng(3)
    M, N, K = 9, 7, 13
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    for ta, tb in ((0, 0), (0, 1), (1, 0)):
        Aa = np.ascontiguousarray(A.T) if ta else A
        Bb = np.ascontiguousarray(B.T) if tb else B
        for it in (1, 8, 16, 24):
            c1 = rl.orc_matmul(Aa, Bb, M, N, K, it, 1, ta=ta, tb=tb, literal=1)
            c2 = rl.orc_matmul(Aa, Bb, M, N, K, it, 1, ta=ta, tb=tb, literal=0)
            assert np.array_equal(c1, c2)
        c3 = rl.orc_matmul(Aa, Bb, M, N, K, 24, 0, ta=ta, tb=tb)
        assert np.allclose(c3, A.astype(np.float64) @ B, rtol=1e-5, atol=1e-5)


def test_rope_cache_bit_exact_vs_golden(o):
    d = npz("rope.npz")
    c, s = rl.orc_rope_cache(4096, 128)
    assert rl.sha256(c) == str(d["big_cos_sha"]) and rl.sha256(s) == str(d["big_sin_sha"])
    c2, s2 = rl.orc_rope_cache(64, 32)
    assert np.array_equal(c2, d["small_cos"]) and np.array_equal(s2, d["small_sin"])
    # invariants (reference BVT-14 tolerance 0.001): p=0 gives (1, 0) up to
    # the 16-step residual angle; |(c,s)| ~ 1
    assert np.all(np.abs(c[0] - 1) < 1e-3) and np.all(np.abs(s[0]) < 1e-3)
    assert np.all(np.abs(c.astype(np.float64) ** 2 + s.astype(np.float64) ** 2 - 1) < 1e-2)


def test_rope_apply_bit_exact_vs_golden(o):
    d = npz("rope.npz")
    out = rl.orc_rope_apply(d["apply_x"], d["apply_cos"], d["apply_sin"])
    assert np.array_equal(out, d["apply_out"])


def test_rope_apply_strided_matches_contiguous(o):
    x = rl.gen_normal((2, 3, 5, 8), seed=4)
    c, s = rl.orc_rope_cache(5, 8)
    ref = rl.orc_rope_apply(x, c, s)
    xt = np.ascontiguousarray(x.transpose(0, 2, 1, 3))  # [B, T, H, D] storage
    B, T, H, D = xt.shape
    assert o.orc_rope_apply_strided(rl.p(xt), rl.p(c), rl.p(s), 2, 3, 5, 8, T * H * D, D, H * D) == 0
    assert np.array_equal(xt.transpose(0, 2, 1, 3), ref)


def test_exp_xy_bit_exact_vs_rac_alu_exp(o):
    d = npz("alu_exp.npz")
    got = np.array([o.orc_exp_xy(float(v), 16, 1.2074970) for v in d["x"]], np.float32)
    assert np.array_equal(got, d["y"])


def _hyp_last_shift(n):
    sh = np.zeros(64, np.int32)
    rl.oracle().orc_hyp_schedule(n, rl.p(sh))
    return int(sh[n - 1]), sh[:n]


def test_hyperbolic_schedule():
    _, s16 = _hyp_last_shift(16)
    assert list(s16) == [1, 2, 3, 4, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 13, 14]
    _, s24 = _hyp_last_shift(24)
    assert list(s24) == [1, 2, 3, 4, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 13, 14, 15, 16, 17, 18, 19, 20, 21, 22]
    assert abs(rl.oracle().orc_hyp_kinv(16) - 1.2074970) < 2e-7


@pytest.mark.parametrize("n", [8, 16, 24])
def test_exp_cordic_error_bound(o, n):
    x = np.concatenate([np.linspace(-87, 88, 20001), rl.gen_normal((5000,), 3, std=2.0)]).astype(np.float32)
    y = rl.orc_unary("orc_exp_batch", x, n)
    true = np.exp(x.astype(np.float64))
    rel = np.abs(y - true) / true
    last, _ = _hyp_last_shift(n)
    # residual angle <= atanh(2^-s) ~ 2^-s, plus ~n roundings
    assert rel.max() <= 1.05 * 2.0 ** -last + n * 6e-8, rel.max()
    xy = np.array([o.orc_exp_xy(float(v), n, o.orc_hyp_kinv(n)) for v in x[::7]], np.float32)
    assert rl.max_rel(y[::7], xy) < 1e-6


def test_exp_special_values(o):
    assert o.orc_exp_n(0.0, 16) == pytest.approx(1.0, rel=7e-5)
    assert o.orc_exp_n(-200.0, 16) == 0.0
    assert math.isinf(o.orc_exp_n(200.0, 16))
    assert math.isnan(o.orc_exp_n(float("nan"), 16))
    assert o.orc_exp_n(float("-inf"), 16) == 0.0


def test_softmax_libm_bit_exact_and_cordic_bound(o):
    d = npz("softmax.npz")
    assert np.array_equal(rl.orc_softmax(d["x"], 0), d["y"])
    for n in (8, 16, 24):
        last, _ = _hyp_last_shift(n)
        y = rl.orc_softmax(d["x"], n)
        assert np.allclose(y.sum(1), 1.0, atol=1e-5)
        assert rl.max_rel(y, d["y"]) <= 2.2 * 2.0 ** -last + 1e-6


def test_rsqrt_against_libm_and_guards(o):
    x = np.exp(np.random.default_rng(1).uniform(-85, 85, 50000)).astype(np.float32)
    got = np.array([o.orc_rsqrt(float(v)) for v in x])
    assert rl.max_rel(got, 1 / np.sqrt(x.astype(np.float64))) < 1e-6
    assert abs(o.orc_rsqrt(4.0) - 0.5) < 1e-6
    assert o.orc_rsqrt(0.0) == 0.0 and o.orc_rsqrt(-1.0) == 0.0 and o.orc_rsqrt(float("inf")) == 0.0
    assert math.isnan(o.orc_rsqrt(float("nan")))
    d = npz("activations.npz")
    got = np.array([o.orc_rsqrt(float(v)) for v in d["xq"]], np.float32)
    assert rl.max_rel(got, d["rsqrt"], floor=1e-30) < 1e-6
    # subnormal input
    assert rl.max_rel([o.orc_rsqrt(1e-40)], [1 / math.sqrt(np.float32(1e-40))]) < 1e-6


def test_norms(o):
    d = npz("norms.npz")
    assert np.array_equal(rl.orc_rmsnorm(d["x"], d["gamma"], 1e-6, 0), d["rms"])
    assert np.array_equal(rl.orc_layernorm(d["x"], d["gamma"], d["beta"], 1e-5, 0), d["ln"])
    assert np.array_equal(rl.orc_rmsnorm(d["xw"], d["gw"], 1e-6, 0), d["rmsw"])
    assert rl.max_rel(rl.orc_rmsnorm(d["x"], d["gamma"], 1e-6, 1), d["rms"], 1e-6) < 1e-6
    assert rl.max_rel(rl.orc_layernorm(d["x"], d["gamma"], d["beta"], 1e-5, 1), d["ln"], 1e-3) < 1e-5
    kat = rl.orc_rmsnorm(d["kat"], None, 1e-6, 1)
    assert np.allclose(kat, [[1.2, 1.6, 0, 0]], atol=1e-6)


def test_activations(o):
    d = npz("activations.npz")
    x = d["x"]
    assert np.array_equal(rl.orc_unary("orc_silu", x, 0), d["silu"])
    assert np.array_equal(rl.orc_unary("orc_gelu", x), d["gelu"])
    sig0 = rl.orc_unary("orc_sigmoid", x, 0)
    # reference form 0.5(1+tanh(x/2)) cancels to 0 for x << 0, so an absolute
    # floor: both are the same function to ~1 ulp of 0.5
    assert np.max(np.abs(sig0 - d["sigmoid"]) / np.maximum(np.abs(d["sigmoid"]), 0.1)) < 1e-6
    for n in (8, 16, 24):
        last, _ = _hyp_last_shift(n)
        s = rl.orc_unary("orc_silu", x, n)
        assert np.max(np.abs(s - d["silu"]) / np.maximum(np.abs(d["silu"]), 1e-3)) < 1.1 * 2.0 ** -last + 1e-6
        t = rl.orc_unary("orc_tanh", x, n)
        assert np.max(np.abs(t - np.tanh(x.astype(np.float64)))) < 2 * 2.0 ** -last + 1e-6


# ── vector primitives (rac.h:101-250, 345-346) ─────────────────────────────

_PAIR_ARG = {"compensate": "chain", "rotate_n": "iters", "project_n": "iters"}


def _prim_from_golden(d, name):
    code, pair, nb, nt = rl.PRIM_OPS[name]
    a, b, th = d["a"], d["b"], d["theta"]
    if name in _PAIR_ARG:
        arg = d[_PAIR_ARG[name]]
        return np.stack([rl.orc_prim(name, a[i:i + 1], None, th[i:i + 1], int(arg[i]))[0]
                         for i in range(len(a))])
    return rl.orc_prim(name, a, b if nb else None, th if nt else None)


@pytest.mark.parametrize("name", ["rotate", "rotate_raw", "compensate", "project", "polar", "normalize",
                                  "dot", "coherence", "complex_mul", "rotate_n", "project_n"])
def test_prims_bit_exact_vs_reference_golden(o, name):
    d = npz("prims.npz")
    assert np.array_equal(_prim_from_golden(d, name), d[name], equal_nan=True)


def test_prims_batch_forms_vs_reference_golden(o):
    d = npz("prims.npz")
    a, b = d["a"], d["b"]
    pol = rl.orc_prim("polar", a)
    assert np.array_equal(pol[:, 0], d["norm"])
    outer = np.zeros((24, 40), np.float32)
    o.orc_outer(rl.p(np.ascontiguousarray(a[:24])), rl.p(np.ascontiguousarray(b[:40])), rl.p(outer), 24, 40)
    assert np.array_equal(outer, d["outer"])
    X = np.zeros(64, np.float32)
    dct_x = d["dct_x"]
    o.orc_dct(rl.p(dct_x), rl.p(X), 64)
    assert np.array_equal(X, d["dct"])
    # rac_inner sums with an OpenMP reduction (order not fixed): bound by
    # n * 2^-24 * sum |term|
    terms = rl.orc_prim("inner_term", a[:64], b[:64]).astype(np.float64)
    assert abs(terms.sum() - float(d["inner"])) <= 64 * 2.0 ** -24 * np.abs(terms).sum()


def test_prims_closed_forms(o):
    rng = np.random.default_rng(7)
    n = 2000
    a = rng.uniform(-5, 5, (n, 2)).astype(np.float32)
    b = rng.uniform(-5, 5, (n, 2)).astype(np.float32)
    th = rng.uniform(-20, 20, n).astype(np.float32)
    a64, b64, th64 = a.astype(np.float64), b.astype(np.float64), th.astype(np.float64)
    r = np.hypot(a64[:, 0], a64[:, 1])
    # polar: 16 vectoring steps leave an angle residual <= atan(2^-15) and
    # the magnitude carries K_INV = 0.60725 against K_16 (|bias| < 2e-5)
    pol = rl.orc_prim("polar", a).astype(np.float64)
    ang_err = np.angle(np.exp(1j * (pol[:, 1] - np.arctan2(a64[:, 1], a64[:, 0]))))
    assert np.max(np.abs(ang_err)) < 4e-5
    assert np.max(np.abs(pol[:, 0] / r - 1)) < 5e-5
    # rotate: exact rotation to the 16-step residual (plus the sequential
    # float reduction of theta, whose drift grows with |theta|)
    rot = rl.orc_prim("rotate", a, None, th).astype(np.float64)
    c, s_ = np.cos(th64), np.sin(th64)
    ex = np.stack([a64[:, 0] * c - a64[:, 1] * s_, a64[:, 0] * s_ + a64[:, 1] * c], 1)
    assert np.max(np.hypot(*(rot - ex).T) / r) < 1e-4
    # complex_mul: the complex product a*b
    cm = rl.orc_prim("complex_mul", a, b).astype(np.float64)
    prod = (a64[:, 0] + 1j * a64[:, 1]) * (b64[:, 0] + 1j * b64[:, 1])
    assert np.max(np.abs(cm[:, 0] + 1j * cm[:, 1] - prod) / np.abs(prod)) < 2e-4
    # dot / coherence: the Euclidean dot product and cosine similarity
    dot = rl.orc_prim("dot", a, b).astype(np.float64)
    rb = np.hypot(b64[:, 0], b64[:, 1])
    assert np.max(np.abs(dot - (a64 * b64).sum(1)) / (r * rb)) < 2e-4
    coh = rl.orc_prim("coherence", a, b).astype(np.float64)
    assert np.max(np.abs(coh - (a64 * b64).sum(1) / (r * rb))) < 1e-4
    # rotate_n at 24 steps: residual angle ~2^-23, but the gain 1/K-hat(24)
    # of the reference table is 5.93e-6 above 1/K_24, so |error| / |v| is
    # that bias plus rounding
    rn = rl.orc_prim("rotate_n", a[:200], None, th[:200] * np.float32(0.1), 24).astype(np.float64)
    th2 = (th[:200] * np.float32(0.1)).astype(np.float64)
    ex2 = np.stack([a64[:200, 0] * np.cos(th2) - a64[:200, 1] * np.sin(th2),
                    a64[:200, 0] * np.sin(th2) + a64[:200, 1] * np.cos(th2)], 1)
    assert np.max(np.hypot(*(rn - ex2).T) / r[:200]) < 5.93e-6 + 1e-6
    # DCT-II of a constant and of a cosine basis vector
    X = np.zeros(32, np.float32)
    one = np.ones(32, np.float32)
    o.orc_dct(rl.p(one), rl.p(X), 32)
    assert abs(X[0] - 32) < 1e-4 and np.max(np.abs(X[1:])) < 1e-4
    x5 = np.cos(np.pi * (2 * np.arange(32) + 1) * 5 / 64).astype(np.float32)
    o.orc_dct(rl.p(x5), rl.p(X), 32)
    expect = np.zeros(32)
    expect[5] = 16.0
    assert np.max(np.abs(X - expect)) < 1e-4


# ── attention (rac.h:323-335) ───────────────────────────────────────────────

@pytest.mark.parametrize("case", ["plain", "causal", "mask", "causal_mask"])
def test_attention_bit_exact_vs_reference_golden(o, case):
    d = npz("attention.npz")
    mask = d["mask"] if "mask" in case else None
    causal = "causal" in case
    out = rl.orc_attention(d["q"], d["k"], d["v"], mask, causal, 0, 0)
    assert np.array_equal(out, d["out_" + case])


def _attention64(q, k, v, mask, causal):
    q, k, v = (t.astype(np.float64) for t in (q, k, v))
    T, D = q.shape[2], q.shape[3]
    s = q @ np.swapaxes(k, 2, 3) / math.sqrt(D)
    if causal:
        s = np.where(np.triu(np.ones((T, T), bool), 1), -np.inf, s)
    if mask is not None:
        s = s + mask.astype(np.float64)
    s = s - s.max(-1, keepdims=True)
    p_ = np.exp(s)
    p_ /= p_.sum(-1, keepdims=True)
    return p_ @ v


@pytest.mark.parametrize("iters,mode", [(16, 1), (24, 1), (16, 0), (8, 1)])
def test_attention_cordic_bound(o, iters, mode):
    d = npz("attention.npz")
    for mask, causal in ((None, 0), (d["mask"], 1)):
        ref = _attention64(d["q"], d["k"], d["v"], mask, causal)
        out = rl.orc_attention(d["q"], d["k"], d["v"], mask, causal, iters, mode)
        last, _ = _hyp_last_shift(iters)
        # CORDIC exp relative error ~2^-last moves each probability by that
        # fraction; the CORDIC products add ~2e-5 (n >= 16) relative
        bound = 4 * (2.0 ** -last + (2e-5 if iters >= 16 else 2e-4)) * np.abs(d["v"]).max()
        assert np.max(np.abs(out - ref)) < bound


# ── Q8_0 (lib/c/rac_q8_0.h) ─────────────────────────────────────────────────

def test_fp16_conversions_vs_reference_golden(o):
    d = npz("q8.npz")
    h2f = np.array([o.orc_fp16_to_fp32(int(h)) for h in d["halves"]], np.float32)
    assert np.array_equal(h2f.view(np.uint32), d["h2f"].view(np.uint32))
    f2h = np.array([o.orc_fp32_to_fp16(float(v)) for v in d["floats"]], np.uint16)
    assert np.array_equal(f2h, d["f2h"])
    # closed forms: every finite half is exactly representable, so fp16 ->
    # fp32 -> fp16 is the identity; fp16 -> fp32 equals numpy's conversion
    hs = np.arange(65536, dtype=np.uint16)
    fin = (hs & 0x7c00) != 0x7c00
    f = np.array([o.orc_fp16_to_fp32(int(h)) for h in hs[fin]], np.float32)
    assert np.array_equal(f, hs[fin].view(np.float16).astype(np.float32))
    back = np.array([o.orc_fp32_to_fp16(float(v)) for v in f], np.uint16)
    assert np.array_equal(back, hs[fin])


def test_q8_quantize_and_gemv_vs_reference_golden(o):
    d = npz("q8.npz")
    wq = rl.orc_q8_quantize(d["W"])
    assert np.array_equal(wq, d["wq"])
    for act in range(4):
        for with_bias in (0, 1):
            out = rl.orc_q8_gemv(d["x"], wq, d["bias"] if with_bias else None, act)[0]
            assert np.array_equal(out, d[f"out_a{act}_b{with_bias}"]), (act, with_bias)


def test_q8_closed_forms(o):
    rng = np.random.default_rng(5)
    N, K = 37, 320
    W = rng.normal(0, 1, (N, K)).astype(np.float32)
    wq = rl.orc_q8_quantize(W)
    deq = np.zeros((N, K), np.float32)
    o.orc_q8_0_dequantize(rl.p(wq), rl.p(deq), N, K)
    scale = np.array([[o.orc_fp16_to_fp32(int(b[0]) | int(b[1]) << 8) for b in row] for row in wq], np.float32)
    # |x - d q| <= d/2 (+ the scale's truncation to fp16, < 2^-10 relative)
    err = np.abs(W - deq).reshape(N, K // 32, 32)
    amax = np.abs(W).reshape(N, K // 32, 32).max(-1)
    assert np.all(err <= (0.5 * amax / 127 + amax * 2.0 ** -10)[..., None] * 1.0001)
    assert np.array_equal(np.abs(wq[..., 2:].view(np.int8)).max(-1), np.full((N, K // 32), 127))
    # GEMV = float64 dot of the dequantized weights, within the summation bound
    x = rng.normal(0, 1, (3, K)).astype(np.float32)
    out = rl.orc_q8_gemv(x, wq, None, 0)
    ref = x.astype(np.float64) @ deq.astype(np.float64).T
    bound = (K + 8) * 2.0 ** -24 * (np.abs(x).astype(np.float64) @ np.abs(deq).astype(np.float64).T)
    assert np.all(np.abs(out - ref) <= bound)
    # a zero block quantizes to d = 0, q = 0
    Z = np.zeros((1, 64), np.float32)
    zq = rl.orc_q8_quantize(Z)
    assert not zq.any()


# ── RAC-DSP fixed-point engine (sim/rac_dsp_core.c) ──────────────────────

DSP_UNIT = 2.0 ** 63 / math.pi          # Q0.63 fraction-of-pi units per radian
K_COARSE = math.prod(math.sqrt(1 + 4.0 ** -i) for i in range(10))
K_RES = math.prod(math.sqrt(1 + 4.0 ** -s) for s in range(8, 17))
K_HRES = math.prod(math.sqrt(1 - 4.0 ** -s) for s in range(8, 17))


def _coarse_angle(word):
    """Angle (rad) applied by the 10 coarse micro-rotations of one LUT word."""
    return sum((1 if (int(word) >> i) & 1 else -1) * math.atan(2.0 ** -i) for i in range(10))


def _fold(x, y, theta):
    """The quadrant fold as geometry: an angle outside [-pi/2, pi/2) is moved
    by pi and the vector negated (the rotation the pair describes is kept)."""
    if theta >= math.pi / 2 or theta < -math.pi / 2:
        theta = theta - math.pi if theta > 0 else theta + math.pi
        return -x, -y, theta
    return x, y, theta


def test_dsp_roms_vs_rtl_mem_golden(o):
    d = npz("dsp.npz")
    lut, at, ath = np.zeros(1024, np.uint64), np.zeros(17, np.int64), np.zeros(9, np.int64)
    o.orc_dsp_gen_roms(rl.p(lut), rl.p(at), rl.p(ath))
    assert np.array_equal(lut, d["lut"]) and np.array_equal(at, d["atan"]) and np.array_equal(ath, d["atanh"])
    # every LUT word steers its bin centre to within the last coarse step
    for k in range(1024):
        centre = (k - 512 + 0.5) * math.pi / 1024
        assert abs(_coarse_angle(d["lut"][k]) - centre) <= math.atan(2.0 ** -9) + 1e-12, k


@pytest.mark.parametrize("op", [0, 1, 2, 3])
def test_dsp_eval_bit_exact_vs_reference_golden(o, op):
    d = npz("dsp.npz")
    x, y, z = d["x"], d["y"], d["z"]
    xo, yo, zo = rl.orc_dsp_batch(op, x, y, z)
    assert np.array_equal(np.stack([xo, yo, zo], 1), d[f"op{op}"])


def test_dsp_systolic_vs_reference_golden(o):
    d = npz("dsp.npz")
    W, X = np.ascontiguousarray(d["W"]), np.ascontiguousarray(d["X"])
    K, N = X.shape
    Y = np.zeros((K, N), np.int64)
    o.orc_dsp_systolic(N, K, rl.p(W), rl.p(X), rl.p(Y))
    assert np.array_equal(Y, d["Y"])
    # each column sum is K_cordic * sum_r x_r cos(w_rc) up to the residual angle error
    th = W.astype(np.float64) / DSP_UNIT
    ref = K_COARSE * K_RES * (X.astype(np.float64) @ np.cos(th))
    tol = 3e-5 * (np.abs(X).astype(np.float64) @ np.ones_like(th)) + 64 * N
    assert np.all(np.abs(Y - ref) <= tol)


def test_dsp_closed_forms(o):
    rng = np.random.default_rng(77)
    n = 3000
    x = rng.integers(-2 ** 40, 2 ** 40, n, dtype=np.int64)
    y = rng.integers(-2 ** 40, 2 ** 40, n, dtype=np.int64)
    z = rng.integers(-2 ** 63, 2 ** 63 - 1, n, dtype=np.int64)
    xf, yf = x.astype(np.float64), y.astype(np.float64)
    th = z.astype(np.float64) / DSP_UNIT
    mag = np.hypot(xf, yf)
    # rotate / project: K * R(theta) (x, y); z driven to within the last step
    r0 = rl.orc_dsp_batch(0, x, y, z)
    r1 = rl.orc_dsp_batch(1, x, y, z)
    assert all(np.array_equal(a, b) for a, b in zip(r0, r1))
    K = K_COARSE * K_RES
    ex, ey = K * (xf * np.cos(th) - yf * np.sin(th)), K * (xf * np.sin(th) + yf * np.cos(th))
    tol = 3e-5 * mag + 64
    assert np.all(np.abs(r0[0] - ex) <= tol) and np.all(np.abs(r0[1] - ey) <= tol)
    assert np.all(np.abs(r0[2] / DSP_UNIT) <= 2 * math.atan(2.0 ** -16))
    # vectoring (no coarse stage): a vector within the residual range of the
    # x axis is rotated onto it; z accumulates its angle
    phi = rng.uniform(-0.007, 0.007, n)
    xv = rng.integers(2 ** 36, 2 ** 40, n, dtype=np.int64)
    yv = np.round(xv * np.tan(phi)).astype(np.int64)
    zv = rng.integers(-2 ** 61, 2 ** 61, n, dtype=np.int64)       # |angle| < pi/4: no fold
    v = rl.orc_dsp_batch(2, xv, yv, zv)
    mv = np.hypot(xv.astype(np.float64), yv.astype(np.float64))
    assert np.all(np.abs(v[0] - K_RES * mv) <= 3e-5 * mv + 64)
    assert np.all(np.abs(v[1]) <= 3e-5 * mv + 64)
    assert np.all(np.abs((v[2] - zv) / DSP_UNIT - np.arctan2(yv, xv)) <= 2 * math.atan(2.0 ** -16))
    # hyperbolic: circular coarse rotation by the LUT angle of the folded z,
    # then a hyperbolic rotation by the rest of the angle
    lut = npz("dsp.npz")["lut"]
    h = rl.orc_dsp_batch(3, x, y, z)
    for i in range(0, n, 7):
        a, b, t = _fold(xf[i], yf[i], th[i])
        k = min(int(math.floor((t + math.pi / 2) / (math.pi / 1024))), 1023)
        tc = _coarse_angle(lut[k])
        a, b = K_COARSE * (a * math.cos(tc) - b * math.sin(tc)), K_COARSE * (a * math.sin(tc) + b * math.cos(tc))
        phi_h = t - tc
        hx = K_HRES * (a * math.cosh(phi_h) + b * math.sinh(phi_h))
        hy = K_HRES * (b * math.cosh(phi_h) + a * math.sinh(phi_h))
        bound = 6e-5 * mag[i] + 64
        assert abs(h[0][i] - hx) <= bound and abs(h[1][i] - hy) <= bound, i


# ── safetensors element conversion (bench/safetensors_reader.c:375-425) ──

ST_GOLDEN_FLOAT = {"f32": 1, "f16": 2, "bf16": 3, "f64": 4, "model.layers.0.mlp.up_proj.weight": 3, "scalar": 1,
                   "empty": 2}


def _st_raw(d, rec):
    blob = d["sample"].tobytes()
    hl = int.from_bytes(blob[:8], "little")
    return blob[8 + hl + rec["offset"]: 8 + hl + rec["offset"] + rec["nbytes"]]


def test_st_to_f32_bit_exact_vs_reference_golden(o):
    d = npz("st.npz")
    recs = {r["name"]: r for r in json.loads(str(d["parse"]))}
    for name, dt in ST_GOLDEN_FLOAT.items():
        rec = recs[name]
        n = int(np.prod(rec["shape"])) if rec["shape"] else 1
        got = rl.orc_st_to_f32(dt, _st_raw(d, rec), n)
        assert np.array_equal(got.view(np.uint32), d[f"f32_{name}"].view(np.uint32)), name
        if f"q8_{name}" in d:
            assert np.array_equal(rl.orc_q8_quantize(got.reshape(-1, rec["shape"][-1])), d[f"q8_{name}"]), name
    raw = np.zeros(8, np.uint8)
    out = np.zeros(2, np.float32)
    assert o.orc_st_to_f32(5, rl.p(raw), 2, rl.p(out)) == -1          # I8: refused, as st_to_f32 does
    assert int(d["rc_i8"]) == -1


def test_st_conversions_closed_forms(o):
    rng = np.random.default_rng(8)
    # every half: the IEEE widening (numpy's, which keeps NaN payloads)
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got = rl.orc_st_to_f32(2, h.tobytes(), h.size)
    assert np.array_equal(got.view(np.uint32), h.view(np.float16).astype(np.float32).view(np.uint32))
    # bf16 is the top half of an fp32 word
    b = rng.integers(0, 1 << 16, 4096, dtype=np.uint32).astype(np.uint16)
    got = rl.orc_st_to_f32(3, b.tobytes(), b.size)
    assert np.array_equal(got.view(np.uint32), b.astype(np.uint32) << 16)
    # f64 -> f32 rounds to nearest even (numpy's cast), finite and infinite inputs
    v = rng.normal(0, 1, 4096) * np.exp(rng.uniform(-120, 120, 4096))
    v[:6] = [np.inf, -np.inf, 0.0, -0.0, 1.0 + 2.0 ** -24, 1.0 + 3 * 2.0 ** -24]
    with np.errstate(over="ignore"):
        want = v.astype(np.float32)
    got = rl.orc_st_to_f32(4, v.tobytes(), v.size)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert got[4] == 1.0 and got[5] == np.float32(1.0 + 2.0 ** -22)


def test_lane_order_row_sums_pinned():
    """orc_*_lanes regroup only the row sums of orc_rmsnorm / orc_layernorm /
    orc_softmax_rows."""
    rng = np.random.default_rng(11)
    g = rl.gen_normal((4096,), 4, 1.0, 0.02)
    b = rl.gen_normal((4096,), 5, std=0.1)
    # integer-valued rows of zero sum (+-v pairs): every partial sum, the mean
    # (0) and every partial sum of squares are exact, so any order gives the
    # same bits
    for d in (4096, 1000, 4099, 64):
        half = rng.integers(-8, 9, (6, d // 2))
        xi = np.concatenate([half, -half, np.zeros((6, d % 2), half.dtype)], axis=1)
        xi = rng.permuted(xi, axis=1).astype(np.float32)
        assert np.array_equal(rl.orc_rmsnorm_lanes(xi, g[:d], 1e-6), rl.orc_rmsnorm(xi, g[:d], 1e-6)), d
        assert np.array_equal(rl.orc_layernorm_lanes(xi, g[:d], b[:d], 1e-5),
                              rl.orc_layernorm(xi, g[:d], b[:d], 1e-5, use_cordic=1)), d
    # random rows: within the reordering bound of the left-to-right sums
    x = rl.gen_normal((32, 4096), 6)
    assert rl.max_rel(rl.orc_rmsnorm_lanes(x, g, 1e-6), rl.orc_rmsnorm(x, g, 1e-6), 1e-6) < 4e-6
    s = rl.gen_normal((32, 4096), 7, std=2.0)
    for iters in (8, 16, 24):
        assert rl.max_rel(rl.orc_softmax_lanes(s, iters), rl.orc_softmax(s, iters), 1e-37) < 4e-6
    # causal rows with at most 4 live elements sit in lane 0's first float4,
    # summed left to right: equal to the left-to-right softmax of the prefix
    sc = rl.gen_normal((16, 16), 8)
    pl = rl.orc_softmax_lanes(sc, 16, causal=True, zero_guard=True)
    for t_ in range(4):
        assert np.array_equal(pl[t_, :t_ + 1], rl.orc_softmax(sc[t_:t_ + 1, :t_ + 1], 16)[0])
        assert not pl[t_, t_ + 1:].any()
    # the order itself: a row of 1024 (256 lanes x one float4) with 2^24 in
    # element 0 and 1.0 everywhere else.  Left to right every 1.0 is lost
    # (2^24 + 1 rounds to 2^24), sum = 2^24.  In lane order lane 0 holds
    # ((2^24 + 1) + 1) + 1 = 2^24 and lanes 1..63 hold 4; the butterfly adds
    # lane 0's 2^24 to partial sums 4, 8, 16, ..., 128 of the other lanes in
    # turn (each exactly representable above 2^24 at spacing 2), giving
    # 2^24 + 252 for wave 0, and waves 1..3 hold 256 each: total
    # 2^24 + 252 + 768 = 2^24 + 1020.  mean square = that / 1024 exactly.
    row = np.ones((1, 1024), np.float32)
    row[0, 0] = np.float32(4096.0)                     # 4096^2 = 2^24 as the square
    ms_lanes = np.float32(2 ** 24 + 1020) / np.float32(1024)
    ms_seq = np.float32(2 ** 24) / np.float32(1024)
    got_l = rl.orc_rmsnorm_lanes(row, None, 0.0)
    got_s = rl.orc_rmsnorm(row, None, 0.0)
    inv_l = rl.orc_unary("orc_rsqrt_batch", np.array([ms_lanes], np.float32))[0]
    inv_s = rl.orc_unary("orc_rsqrt_batch", np.array([ms_seq], np.float32))[0]
    assert got_l[0, 1] == np.float32(1.0) * inv_l and got_s[0, 1] == np.float32(1.0) * inv_s
    assert inv_l != inv_s
