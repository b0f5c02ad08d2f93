"""Write the golden vectors of the hot path from the compiled reference.

Runs in the build container, where /root/reference exists and
oracle/Makefile has built oracle/_ref/librac_ref.so from the reference lib/c
sources (rac_cpu.c, rac_avx2.c, rac_hal.c, rac_alu.c, the .S kernels) plus
oracle/ref_probe.c.  Every value below is produced by reference code; the
inputs come from tests/raclib.py's seeded generator and are stored too, so
the fixtures are self-contained data (nothing of the reference's source).

    python tests/golden/make_golden.py [core] [prims] [attention] [q8] [dsp]

Outputs (tests/golden/):
  tables.json            reference CORDIC tables (rac_cpu.c:20-52)
  rotate.npz             _cordic_rotate samples (rac_cpu.c:90-118)
  rope.npz               rac_rope_cache 4096x64 digest + samples,
                         a full 64x16 table, rac_rope_apply on [2,2,16,64]
  norms.npz              rac_rmsnorm / rac_layernorm on 8x64 and a 3x4096 row set
  softmax.npz            rac_softmax_batch on 4x256 ~ N(0, 2)
  activations.npz        rac_silu / rac_gelu / rac_sigmoid / rac_rsqrt samples
  alu_exp.npz            rac_alu_exp (16-step hyperbolic CORDIC exp) samples
  matmul.npz             rac_matmul 1024^3, U[-1,1] seeds 0/1: digest + samples;
                         the 2x2 known answer
  prims.npz              rac_rotate/_raw/_n, rac_compensate, rac_project/_n,
                         rac_polar, rac_norm, rac_normalize, rac_dot,
                         rac_coherence, rac_complex_mul on 512 pairs;
                         rac_inner, rac_outer, rac_dct
  attention.npz          rac_scaled_dot_attention on [2,3,16,8], with and
                         without causal / additive mask
  dsp.npz                RAC-DSP integer CORDIC (sim/rac_dsp_core.c with the
                         rtl/*.mem ROMs): ROM contents, rac_dsp_eval for
                         ops 0-3, a 16x16 systolic product
  q8.npz                 rac_fp16_to_fp32 / rac_fp32_to_fp16 samples,
                         rac_q8_0_quantize_matrix of a 40x512 matrix, and
                         rac_q8_0_gemv with each activation, +- bias
"""
from __future__ import annotations

import ctypes as C
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import raclib as rl  # noqa: E402


def main(sections) -> None:
    if not rl.have_ref():
        raise SystemExit("oracle/_ref/librac_ref.so is not built (make -C oracle ref)")
    r = rl.ref()
    if "core" in sections:
        write_core(r)
    if "prims" in sections:
        write_prims(r)
    if "attention" in sections:
        write_attention(r)
    if "q8" in sections:
        write_q8(r)
    if "dsp" in sections:
        write_dsp(r)
    if "st" in sections:
        write_st(r)
    print("golden fixtures written to", HERE)


def write_core(r) -> None:
    rng = np.random.default_rng(20261201)

    # tables
    at, ext, ath, kt = (np.zeros(16, np.float32), np.zeros(8, np.float32),
                        np.zeros(16, np.float32), np.zeros(25, np.float32))
    r.ref_tables(rl.p(at), rl.p(ext), rl.p(ath), rl.p(kt))
    with open(os.path.join(HERE, "tables.json"), "w") as f:
        json.dump({"atan16": at.tolist(), "atan_ext8": ext.tolist(),
                   "atanh16": ath.tolist(), "khat25": kt.tolist()}, f, indent=1)

    # rotate samples (small and large angles, all iteration counts 4..24)
    n = 3000
    vx = rng.uniform(-2, 2, n).astype(np.float32)
    vy = rng.uniform(-2, 2, n).astype(np.float32)
    th = np.where(np.arange(n) % 2 == 0, rng.uniform(-4, 4, n), rng.uniform(-5000, 5000, n)).astype(np.float32)
    it = rng.integers(4, 25, n).astype(np.int32)
    ox = np.zeros(n, np.float32)
    oy = np.zeros(n, np.float32)
    for i in range(n):
        a, b = C.c_float(), C.c_float()
        r.ref_cordic_rotate(float(vx[i]), float(vy[i]), float(th[i]), int(it[i]), C.byref(a), C.byref(b))
        ox[i], oy[i] = a.value, b.value
    np.savez_compressed(os.path.join(HERE, "rotate.npz"), vx=vx, vy=vy, theta=th, iters=it, x=ox, y=oy)

    # RoPE
    cos_big = np.zeros((4096, 64), np.float32)
    sin_big = np.zeros((4096, 64), np.float32)
    assert r.rac_rope_cache(rl.p(cos_big), rl.p(sin_big), 4096, 128, 10000.0) == 0
    sample_idx = np.arange(0, cos_big.size, 97, dtype=np.int64)
    cos_small = np.zeros((64, 16), np.float32)
    sin_small = np.zeros((64, 16), np.float32)
    assert r.rac_rope_cache(rl.p(cos_small), rl.p(sin_small), 64, 32, 10000.0) == 0
    xr = rl.gen_normal((2, 2, 16, 64), seed=7)
    ct = np.zeros((16, 32), np.float32)
    st = np.zeros((16, 32), np.float32)
    assert r.rac_rope_cache(rl.p(ct), rl.p(st), 16, 64, 10000.0) == 0
    xo = xr.copy()
    assert r.rac_rope_apply(rl.p(xo), rl.p(ct), rl.p(st), 2, 2, 16, 64, None) == 0
    np.savez_compressed(os.path.join(HERE, "rope.npz"),
                        big_cos_sha=rl.sha256(cos_big), big_sin_sha=rl.sha256(sin_big),
                        big_idx=sample_idx, big_cos=cos_big.ravel()[sample_idx],
                        big_sin=sin_big.ravel()[sample_idx],
                        small_cos=cos_small, small_sin=sin_small,
                        apply_x=xr, apply_cos=ct, apply_sin=st, apply_out=xo)

    # norms
    xn = rl.gen_normal((8, 64), seed=11)
    g = rl.gen_normal((64,), seed=12, mean=1.0, std=0.02)
    b = rl.gen_normal((64,), seed=13, std=0.1)
    rms = np.zeros_like(xn)
    ln = np.zeros_like(xn)
    assert r.rac_rmsnorm(rl.p(xn), rl.p(rms), rl.p(g), 1e-6, 8, 64, None) == 0
    assert r.rac_layernorm(rl.p(xn), rl.p(ln), rl.p(g), rl.p(b), 1e-5, 8, 64, None) == 0
    xw = rl.gen_normal((3, 4096), seed=14)
    gw = rl.gen_normal((4096,), seed=15, mean=1.0, std=0.02)
    rmsw = np.zeros_like(xw)
    assert r.rac_rmsnorm(rl.p(xw), rl.p(rmsw), rl.p(gw), 1e-6, 3, 4096, None) == 0
    kat = np.array([[3, 4, 0, 0]], np.float32)
    kat_out = np.zeros_like(kat)
    assert r.rac_rmsnorm(rl.p(kat), rl.p(kat_out), None, 1e-6, 1, 4, None) == 0
    np.savez_compressed(os.path.join(HERE, "norms.npz"), x=xn, gamma=g, beta=b, rms=rms, ln=ln,
                        xw=xw, gw=gw, rmsw=rmsw, kat=kat, kat_out=kat_out)

    # softmax (libm expf), N(0, std 2)
    xs = rl.gen_normal((4, 256), seed=21, std=2.0)
    ys = np.zeros_like(xs)
    r.rac_softmax_batch(rl.p(xs), rl.p(ys), 4, 256)
    np.savez_compressed(os.path.join(HERE, "softmax.npz"), x=xs, y=ys)

    # activations
    xa = np.concatenate([rl.gen_normal((2000,), seed=31, std=3.0),
                         np.array([0.0, -0.0, 1.0, -1.0, 10.0, -10.0, 50.0, -50.0, 88.0, -88.0], np.float32)])
    silu = np.zeros_like(xa)
    gelu = np.zeros_like(xa)
    r.rac_silu(rl.p(xa), rl.p(silu), xa.size)
    r.rac_gelu(rl.p(xa), rl.p(gelu), xa.size)
    sig = np.array([r.rac_sigmoid(float(v)) for v in xa], np.float32)
    xq = np.concatenate([np.exp(rng.uniform(-80, 80, 2000)).astype(np.float32),
                         np.array([4.0, 1.0, 0.25, 0.0, -1.0, 1e-30, 3e38], np.float32)])
    rsq = np.array([r.rac_rsqrt(float(v)) for v in xq], np.float32)
    np.savez_compressed(os.path.join(HERE, "activations.npz"), x=xa, silu=silu, gelu=gelu,
                        sigmoid=sig, xq=xq, rsqrt=rsq)

    # hyperbolic CORDIC exp of the reference's ALU model
    xe = np.concatenate([rng.uniform(-87, 88, 4000), rng.uniform(-1, 1, 1000)]).astype(np.float32)
    ye = np.array([r.rac_alu_exp(float(v)) for v in xe], np.float32)
    np.savez_compressed(os.path.join(HERE, "alu_exp.npz"), x=xe, y=ye)

    # matmul 1024^3 (scalar lib/c path, deterministic per element)
    M = N = K = 1024
    A = rl.gen_uniform((M, K), seed=0)
    B = rl.gen_uniform((K, N), seed=1)
    Cm = np.zeros((M, N), np.float32)
    assert r.rac_matmul(rl.p(A), rl.p(B), rl.p(Cm), M, N, K, None) == 0
    idx = np.arange(0, M * N, 251, dtype=np.int64)
    A2 = np.array([[1, 2], [3, 4]], np.float32)
    B2 = np.array([[5, 6], [7, 8]], np.float32)
    C2 = np.zeros((2, 2), np.float32)
    assert r.rac_matmul(rl.p(A2), rl.p(B2), rl.p(C2), 2, 2, 2, None) == 0
    np.savez_compressed(os.path.join(HERE, "matmul.npz"), A_sha=rl.sha256(A), B_sha=rl.sha256(B),
                        C_sha=rl.sha256(Cm), idx=idx, C_samples=Cm.ravel()[idx], kat_C=C2)


def _v(x, y):
    return rl.Vec2(float(x), float(y))


def write_prims(r) -> None:
    """rac.h vector primitives from the reference CPU library (rac_cpu.c:136-371)."""
    rng = np.random.default_rng(20261202)
    n = 512
    # pairs over all four quadrants, the axes, zero, and a wide magnitude range
    a = rng.uniform(-3, 3, (n, 2)).astype(np.float32)
    b = rng.uniform(-3, 3, (n, 2)).astype(np.float32)
    a[:8] = [[0, 0], [1, 0], [-1, 0], [0, 1], [0, -1], [-2, 1e-3], [-2, -1e-3], [1e-20, -1e-20]]
    a[8:16] *= np.float32(1e4)
    b[:4] = [[0, 0], [-1, 0], [0, -2], [-3, 3]]
    th = rng.uniform(-4, 4, n).astype(np.float32)
    th[:8] = [0.0, np.pi / 2, -np.pi / 2, np.pi, -np.pi, 3.0, -3.0, 1e-7]
    th[16:32] = rng.uniform(-5000, 5000, 16).astype(np.float32)
    it = rng.integers(1, 30, n).astype(np.int32)   # includes out-of-range counts (clamped to [4, 24])
    chain = rng.integers(0, 40, n).astype(np.int32)
    out = {k: np.zeros((n, 2), np.float32) for k in ("rotate", "rotate_raw", "compensate", "polar",
                                                     "normalize", "complex_mul", "rotate_n")}
    out.update({k: np.zeros(n, np.float32) for k in ("project", "norm", "dot", "coherence", "project_n")})
    m, ang = C.c_float(), C.c_float()
    for i in range(n):
        va, vb = _v(*a[i]), _v(*b[i])
        for key, res in (("rotate", r.rac_rotate(va, th[i])), ("rotate_raw", r.rac_rotate_raw(va, th[i])),
                         ("compensate", r.rac_compensate(va, int(chain[i]))),
                         ("normalize", r.rac_normalize(va)), ("complex_mul", r.rac_complex_mul(va, vb)),
                         ("rotate_n", r.rac_rotate_n(va, th[i], int(it[i])))):
            out[key][i] = (res.x, res.y)
        r.rac_polar(va, C.byref(m), C.byref(ang))
        out["polar"][i] = (m.value, ang.value)
        out["project"][i] = r.rac_project(va, th[i])
        out["norm"][i] = r.rac_norm(va)
        out["dot"][i] = r.rac_dot(va, vb)
        out["coherence"][i] = r.rac_coherence(va, vb)
        out["project_n"][i] = r.rac_project_n(va, th[i], int(it[i]))
    # batch forms
    rb = np.zeros((n, 2), np.float32)
    r.rac_rotate_batch(rl.p(a), rl.p(th), rl.p(rb), n)
    assert np.array_equal(rb, out["rotate"])
    inner = np.float32(r.rac_inner(rl.p(a[:64]), rl.p(b[:64]), 64))
    outer = np.zeros((24, 40), np.float32)
    r.rac_outer(rl.p(a[:24]), rl.p(b[:40]), rl.p(outer), 24, 40)
    dct_x = rng.normal(0, 1, 64).astype(np.float32)
    dct = np.zeros(64, np.float32)
    r.rac_dct(rl.p(dct_x), rl.p(dct), 64)
    np.savez_compressed(os.path.join(HERE, "prims.npz"), a=a, b=b, theta=th, iters=it, chain=chain,
                        inner=inner, outer=outer, dct_x=dct_x, dct=dct, **out)


def write_attention(r) -> None:
    """rac_scaled_dot_attention (rac_cpu.c:637-703) on [2, 3, 16, 8]: plain,
    causal, additive mask, and causal + mask."""
    B, H, T, D = 2, 3, 16, 8
    q = rl.gen_normal((B, H, T, D), seed=11)
    k = rl.gen_normal((B, H, T, D), seed=12)
    v = rl.gen_normal((B, H, T, D), seed=13)
    mask = (rl.gen_normal((T, T), seed=14) * np.float32(0.5)).astype(np.float32)
    mask[3, 5] = -np.inf
    res = {}
    for name, mk, causal in (("out_plain", None, 0), ("out_causal", None, 1), ("out_mask", mask, 0),
                             ("out_causal_mask", mask, 1)):
        o = np.zeros_like(q)
        assert r.rac_scaled_dot_attention(rl.p(q), rl.p(k), rl.p(v), rl.p(mk) if mk is not None else None,
                                          causal, rl.p(o), B, H, T, D, None) == 0
        res[name] = o
    np.savez_compressed(os.path.join(HERE, "attention.npz"), q=q, k=k, v=v, mask=mask, **res)


def write_q8(r) -> None:
    """Q8_0 format and decode GEMV (rac_q8_0.c): fp16 conversions, quantize,
    and rac_q8_0_gemv with each activation, bias and no bias."""
    rng = np.random.default_rng(20261203)
    halves = np.concatenate([np.arange(0, 65536, 7), [0x0000, 0x8000, 0x0001, 0x03ff, 0x0400, 0x7bff, 0x7c00,
                                                       0xfc00, 0x7e00, 0x7c01]]).astype(np.uint16)
    h2f = np.array([r.rac_fp16_to_fp32(int(h)) for h in halves], np.float32)
    fl = np.concatenate([rng.normal(0, 1, 4000), rng.normal(0, 1e-5, 2000), rng.normal(0, 3e4, 2000),
                         [0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e-8, 6e-8, 5.96e-8, np.inf, -np.inf,
                          np.nan]]).astype(np.float32)
    f2h = np.array([r.rac_fp32_to_fp16(float(v)) for v in fl], np.uint16)
    N, K = 40, 512
    W = rng.normal(0, 0.05, (N, K)).astype(np.float32)
    W[2, :32] = 0.0              # all-zero block (d = 0)
    W[7, 100] = 40.0             # outlier
    W[9, 64:96] = 1e-30          # underflowing scale
    wq = np.zeros((N, K // 32, 34), np.uint8)
    r.rac_q8_0_quantize_matrix(rl.p(W), rl.p(wq), N, K)
    x = rng.normal(0, 1, K).astype(np.float32)
    bias = rng.normal(0, 1, N).astype(np.float32)
    outs = {}
    for act in range(4):
        for with_bias in (0, 1):
            o = np.zeros(N, np.float32)
            assert r.rac_q8_0_gemv(rl.p(x), rl.p(wq), rl.p(bias) if with_bias else None, rl.p(o), N, K, act) == 0
            outs[f"out_a{act}_b{with_bias}"] = o
    np.savez_compressed(os.path.join(HERE, "q8.npz"), halves=halves, h2f=h2f, floats=fl, f2h=f2h, W=W, wq=wq,
                        x=x, bias=bias, **outs)


def write_dsp(r) -> None:
    """RAC-DSP integer CORDIC model (sim/rac_dsp_core.c) with the ROMs of
    rtl/*.mem: the ROM contents, rac_dsp_eval on 1500 vectors per op, and a
    16 x 16 weight-stationary systolic product (sim/rac_systolic_ref.c) of
    3 input vectors through rac_dsp_project_sum."""
    rtl = "/root/reference/rtl"
    assert r.rac_load_all_roms(*(os.path.join(rtl, f).encode() for f in
                                 ("cordic_coarse_lut.mem", "cordic_atan.mem", "cordic_atanh.mem"))) == 0
    lib = C.CDLL(rl.REF_SO)
    lut = np.ctypeslib.as_array((C.c_uint64 * 1024).in_dll(lib, "rac_coarse_lut")).copy()
    atan_rom = np.ctypeslib.as_array((C.c_int64 * 17).in_dll(lib, "rac_atan_rom")).copy()
    atanh_rom = np.ctypeslib.as_array((C.c_int64 * 9).in_dll(lib, "rac_atanh_tab")).copy()
    rng = np.random.default_rng(20261204)
    n = 1500
    x = rng.integers(-2 ** 40, 2 ** 40, n, dtype=np.int64)
    y = rng.integers(-2 ** 40, 2 ** 40, n, dtype=np.int64)
    z = rng.integers(-2 ** 63, 2 ** 63 - 1, n, dtype=np.int64)
    # quadrant boundaries, zero, and extreme magnitudes
    z[:8] = [0, 2 ** 62, -2 ** 62, 2 ** 62 - 1, -2 ** 62 - 1, -2 ** 63, 2 ** 63 - 1, 1]
    x[8:16] = [2 ** 62, -2 ** 62, 2 ** 63 - 1, -2 ** 63, 0, 1, -1, 2 ** 32]
    y[8:16] = [0, 2 ** 61, -2 ** 63, 2 ** 63 - 1, 0, -1, 1, 0]
    outs = {}
    a, b, c = C.c_int64(), C.c_int64(), C.c_int64()
    for op in range(4):
        res = np.zeros((n, 3), np.int64)
        for i in range(n):
            r.rac_dsp_eval(int(x[i]), int(y[i]), int(z[i]), op, C.byref(a), C.byref(b), C.byref(c))
            res[i] = (a.value, b.value, c.value)
        outs[f"op{op}"] = res
    N, K = 16, 3
    W = rng.integers(-2 ** 63, 2 ** 63 - 1, (N, N), dtype=np.int64)
    X = rng.integers(-2 ** 34, 2 ** 34, (K, N), dtype=np.int64)
    Y = np.zeros((K, N), np.int64)
    for k in range(K):
        for col in range(N):
            zc = np.ascontiguousarray(W[:, col])
            xk = np.ascontiguousarray(X[k])
            Y[k, col] = r.rac_dsp_project_sum(N, rl.p(xk), rl.p(zc))
    np.savez_compressed(os.path.join(HERE, "dsp.npz"), lut=lut, atan=atan_rom, atanh=atanh_rom, x=x, y=y, z=z,
                        W=W, X=X, Y=Y, **outs)


def st_sample():
    """The sample safetensors file: every dtype the reader converts (with
    subnormals, infinities, NaN payloads, -0), an integer tensor it refuses,
    a 0-d and an empty tensor, metadata and an unknown per-tensor field."""
    rng = np.random.default_rng(20261207)
    f32 = np.array([1.0, -2.5, 0.0, 0.0, np.inf, 0.0], np.float32)
    f32.view(np.uint32)[2] = 0x7FA00001            # signalling NaN with payload
    f32.view(np.uint32)[3] = 0x80000000            # -0
    f32.view(np.uint32)[5] = 0x00000001            # smallest subnormal
    h = rng.integers(0, 1 << 16, 64, dtype=np.uint64).astype(np.uint16)
    h[:12] = [0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x7BFF, 0x7C00, 0xFC00, 0x7C01, 0x7E00, 0xFE55, 0x3C00]
    bf = rng.integers(0, 1 << 16, 64, dtype=np.uint64).astype(np.uint16)
    bf[:8] = [0x0000, 0x8000, 0x0001, 0x7F80, 0xFF80, 0x7F81, 0x7FC0, 0x3F80]
    d = rng.normal(0, 1, 64) * np.exp(rng.uniform(-30, 30, 64))
    d[:14] = [0.0, -0.0, np.inf, -np.inf, 1e300, -1e300, 1e-40, -1e-45, 1e-50, 3.4028235677973366e38,
              1.0000000596046448, 1.0000001788139343, 0.0, 0.0]
    dv = d.view(np.uint64)
    dv[12] = 0x7FF0000000000001                     # signalling NaN, low payload
    dv[13] = 0xFFF8DEADBEEF1234                     # quiet NaN, high payload, negative
    i8 = np.array([1, -2, 3, -4], np.int8)
    w = (rng.normal(0, 0.02, (8, 64)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    scalar = np.array(3.0, np.float32)
    parts = [("f32", "F32", [6], f32.tobytes()), ("f16", "F16", [64], h.tobytes()),
             ("bf16", "BF16", [2, 32], bf.tobytes()), ("f64", "F64", [2, 32], d.tobytes()),
             ("i8", "I8", [4], i8.tobytes()), ("model.layers.0.mlp.up_proj.weight", "BF16", [8, 64], w.tobytes()),
             ("scalar", "F32", [], scalar.tobytes()), ("empty", "F16", [0, 32], b"")]
    header = {"__metadata__": {"format": "pt", "note": "keys are not tensors {x: [1]}"}}
    data = b""
    for name, dt, shape, raw in parts:
        header[name] = {"dtype": dt, "shape": shape, "data_offsets": [len(data), len(data) + len(raw)]}
        data += raw
    header["f32"]["extra"] = [1, [2, 3], {"a": 4}]
    return rl.st_bytes(header, data), parts


def st_malformed():
    """(name, file bytes) of headers every reader must refuse."""
    ok_body = '{"dtype":"F32","shape":[1],"data_offsets":[0,4]}'
    four = b"\0\0\0\0"
    return [
        ("not_an_object", rl.st_bytes("[1,2]", four)),
        ("missing_offsets", rl.st_bytes('{"a":{"dtype":"F32","shape":[1]}}', four)),
        ("unterminated_key", rl.st_bytes('{"a', four)),
        ("garbage_after_body", rl.st_bytes('{"a":' + ok_body + ' x}', four)),
        ("body_not_object", rl.st_bytes('{"a":[1]}', four)),
        ("header_too_long", (1000).to_bytes(8, "little") + b"{}"),
        ("too_small", b"\x02\0\0"),
    ]


def write_st(r) -> None:
    """The compiled reference reader (bench/safetensors_reader.c) on the
    sample file: its parse of every tensor, st_to_f32 of each (or its -1),
    rac_q8_0_quantize_matrix of those with a last dimension that is a
    multiple of 32, and its verdict on each malformed header."""
    import tempfile
    blob, parts = st_sample()
    out = {"sample": np.frombuffer(blob, np.uint8)}
    recs = []
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "sample.safetensors")
        with open(path, "wb") as fh:
            fh.write(blob)
        err = C.create_string_buffer(256)
        f = r.st_open(path.encode(), err)
        assert f, err.value
        for i in range(f.contents.n_tensors):
            t = f.contents.tensors[i]
            recs.append({"name": t.name.decode(), "dtype": t.dtype, "ndim": t.ndim,
                         "shape": [t.shape[k] for k in range(t.ndim)], "offset": t.offset, "nbytes": t.nbytes})
        for name, dt, shape, raw in parts:
            t = r.st_find(f, name.encode())
            n = int(r.st_numel(t))
            buf = np.zeros(max(n, 1), np.float32)
            rc = r.st_to_f32(f, t, rl.p(buf))
            out[f"rc_{name}"] = np.array(rc)
            if rc == 0:
                out[f"f32_{name}"] = buf[:n].copy()
                if shape and n and shape[-1] % 32 == 0:
                    K = shape[-1]
                    q = np.zeros((n // K, K // 32, 34), np.uint8)
                    src = np.ascontiguousarray(buf[:n])
                    r.rac_q8_0_quantize_matrix(rl.p(src), rl.p(q), n // K, K)
                    out[f"q8_{name}"] = q
        r.st_close(f)
        bad = st_malformed()
        verdict = []
        for i, (name, b) in enumerate(bad):
            bp = os.path.join(tmp, f"bad{i}.safetensors")
            with open(bp, "wb") as fh:
                fh.write(b)
            g = r.st_open(bp.encode(), err)
            verdict.append(bool(g))
            if g:
                r.st_close(g)
            out[f"bad_{i}"] = np.frombuffer(b, np.uint8)
        out["bad_names"] = np.array(json.dumps([n for n, _ in bad]))
        out["bad_opened"] = np.array(verdict)
    out["parse"] = np.array(json.dumps(recs))
    np.savez_compressed(os.path.join(HERE, "st.npz"), **out)


if __name__ == "__main__":
    main(sys.argv[1:] or ["core", "prims", "attention", "q8", "dsp", "st"])
