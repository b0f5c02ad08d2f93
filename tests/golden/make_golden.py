"""Write the golden vectors of the hot path from the compiled reference.

Runs in the build container, where /root/reference exists and
oracle/Makefile has built oracle/_ref/librac_ref.so from the reference lib/c
sources (rac_cpu.c, rac_avx2.c, rac_hal.c, rac_alu.c, the .S kernels) plus
oracle/ref_probe.c.  Every value below is produced by reference code; the
inputs come from tests/raclib.py's seeded generator and are stored too, so
the fixtures are self-contained data (nothing of the reference's source).

    python tests/golden/make_golden.py

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


def main() -> None:
    if not rl.have_ref():
        raise SystemExit("oracle/_ref/librac_ref.so is not built (make -C oracle ref)")
    r = rl.ref()
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
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
