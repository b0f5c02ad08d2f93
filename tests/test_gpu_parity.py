"""GPU parity: the gfx950 kernels (through librac_amd.so) vs the CPU checker.

Bars: bit-exact wherever the kernel and the checker evaluate the same
roundings (CORDIC/FAST/SHIFTADD matmul, exp, SiLU, sigmoid, tanh, rsqrt,
sin/cos, RoPE table and apply); elementwise relative error <= 1e-5 where a
row sum is reduced in a different order (softmax, RMSNorm, LayerNorm); matmul
vs the reference lib/c within 1e-4*|a_i|*|b_j| per element.  Full benchmark
sizes are covered through sampled entries and digests.
"""
import ctypes
import math
import os

import numpy as np
import pytest

import raclib as rl

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    import rac_amd
    rac_amd.load()
    yield
    torch.cuda.synchronize()


def T(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def H(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def ext():
    from rac_amd import ext as e
    return e


def lib():
    import rac_amd
    return rac_amd.load()


def gemm(A, B, M, N, K, ta, tb, iters, mode, alpha=1.0, beta=0.0, C0=None):
    Ad, Bd = T(A), T(B)
    Cd = T(C0) if C0 is not None else torch.zeros((M, N), device=DEV)
    rc = lib().rac_gemm_dev(Ad.data_ptr(), Bd.data_ptr(), Cd.data_ptr(), M, N, K, ta, tb, alpha,
                            beta, iters, mode, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib().rac_last_error()
    return H(Cd)


# ── matmul ─────────────────────────────────────────────────────────────────

SHAPES = [(1, 1, 1), (3, 5, 7), (64, 64, 16), (67, 45, 83), (128, 130, 129), (200, 96, 300)]


@pytest.mark.parametrize("iters", [8, 16, 24, 5, 1])
@pytest.mark.parametrize("layout", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_cordic_matmul_bit_exact(iters, layout):
    ta, tb = layout
    for (M, N, K) in SHAPES:
        print(f"cordic iters={iters} layout={layout} shape={(M, N, K)}", flush=True)
        A = rl.gen_uniform((M, K), seed=M * 7 + K)
        B = rl.gen_uniform((K, N), seed=N * 3 + K)
        As = np.ascontiguousarray(A.T) if ta else A
        Bs = np.ascontiguousarray(B.T) if tb else B
        got = gemm(As, Bs, M, N, K, ta, tb, iters, 1)
        ref = rl.orc_matmul(As, Bs, M, N, K, iters, 1, ta=ta, tb=tb)
        assert np.array_equal(got, ref), (M, N, K, float(np.max(np.abs(got - ref))))


SPECIALS = np.array([0.0, -0.0, 1e-45, -3e-39, 2.0 ** -126, -(2.0 ** -110), 1.5 * 2.0 ** -106, 2.0 ** -105,
                     -(2.0 ** -104), 1.9 * 2.0 ** 126, -(2.0 ** 127), 3e38, np.inf, -np.inf, np.nan, 1.0, -0.75],
                    np.float32)


def _sprinkle(A, B, seed):
    """Special values in a few rows of A (their tiles take the literal
    rotation chain, the others stay on the strength-reduced one) and a few
    finite ones in B."""
    rng = np.random.default_rng(seed)
    M, K = A.shape
    for r in rng.integers(0, M, 6):
        A[r, rng.integers(0, K, 5)] = rng.choice(SPECIALS, 5)
    B[rng.integers(0, B.shape[0], 4), rng.integers(0, B.shape[1], 4)] = rng.choice(SPECIALS[:12], 4)
    return A, B


@pytest.mark.parametrize("iters", [8, 16, 24, 5])
@pytest.mark.parametrize("layout", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_cordic_matmul_special_values(iters, layout):
    """Subnormal, tiny (< 2^-105), top-binade, infinite and NaN operands:
    bit-exact with the literal rotation chain of the reference, NaN exactly
    where the checker has NaN; 2x2 tiles (small shapes) and 4x4 tiles."""
    ta, tb = layout
    for (M, N, K) in [(67, 45, 83), (130, 129, 64), (2100, 2100, 20)]:
        print(f"cordic specials iters={iters} layout={layout} shape={(M, N, K)}", flush=True)
        A, B = _sprinkle(rl.gen_uniform((M, K), seed=M + 11 * K), rl.gen_uniform((K, N), seed=N + K), M + iters)
        As = np.ascontiguousarray(A.T) if ta else A
        Bs = np.ascontiguousarray(B.T) if tb else B
        got = gemm(As, Bs, M, N, K, ta, tb, iters, 1)
        ref = rl.orc_matmul(As, Bs, M, N, K, iters, 1, ta=ta, tb=tb)
        assert np.array_equal(got, ref, equal_nan=True), (M, N, K)
        assert np.isnan(ref).any() and np.isfinite(ref).sum() > ref.size // 2


@pytest.mark.parametrize("mode,iters", [(0, 24), (2, 8), (2, 24)])
def test_fast_shiftadd_special_values(mode, iters):
    """The same special operands through the FAST and SHIFTADD MACs."""
    for (M, N, K) in [(67, 45, 83), (130, 129, 64)]:
        for ta, tb in [(0, 0), (1, 1)]:
            print(f"mode={mode} specials iters={iters} shape={(M, N, K)} layout={(ta, tb)}", flush=True)
            A, B = _sprinkle(rl.gen_uniform((M, K), seed=M), rl.gen_uniform((K, N), seed=N), M + mode)
            As = np.ascontiguousarray(A.T) if ta else A
            Bs = np.ascontiguousarray(B.T) if tb else B
            got = gemm(As, Bs, M, N, K, ta, tb, iters, mode)
            ref = rl.orc_matmul(As, Bs, M, N, K, iters, mode, ta=ta, tb=tb, literal=1)
            assert np.array_equal(got, ref, equal_nan=True), (mode, iters, (M, N, K))


@pytest.mark.parametrize("mode", [0, 2])
def test_fast_and_shiftadd_bit_exact(mode):
    for (M, N, K) in [(3, 5, 7), (67, 45, 83), (130, 129, 40)]:
        for ta, tb in [(0, 0), (0, 1), (1, 0)]:
            print(f"mode={mode} shape={(M, N, K)} layout={(ta, tb)}", flush=True)
            A = rl.gen_normal((M, K), seed=1)
            B = rl.gen_normal((K, N), seed=2)
            As = np.ascontiguousarray(A.T) if ta else A
            Bs = np.ascontiguousarray(B.T) if tb else B
            for iters in ((24,) if mode == 0 else (4, 8, 16, 24)):
                got = gemm(As, Bs, M, N, K, ta, tb, iters, mode)
                ref = rl.orc_matmul(As, Bs, M, N, K, iters, mode, ta=ta, tb=tb, literal=1)
                assert np.array_equal(got, ref), (mode, iters, (M, N, K))


def test_alpha_beta_epilogue():
    M, N, K = 70, 33, 20
    A = rl.gen_normal((M, K), 3)
    B = rl.gen_normal((K, N), 4)
    C0 = rl.gen_normal((M, N), 5)
    for mode in (0, 1):
        got = gemm(A, B, M, N, K, 0, 0, 16, mode, alpha=0.5, beta=-2.0, C0=C0)
        ref = rl.orc_matmul(A, B, M, N, K, 16, mode, alpha=0.5, beta=-2.0, C0=C0)
        assert np.array_equal(got, ref)
    # reference DVT known answer: I*B with alpha=1, beta=2 over C0
    got = gemm(np.eye(2, dtype=np.float32), np.float32([[5, 6], [7, 8]]), 2, 2, 2, 0, 0, 24, 0,
               alpha=1.0, beta=2.0, C0=np.float32([[1, 2], [3, 4]]))
    assert got[0, 0] == 7 and got[1, 1] == 16


def test_rac_h_matmul_1024_config1_host_pointers():
    """Benchmark config 1: rac_matmul 1024^3, U[-1,1] seeds 0/1, n=16, through
    the synchronous rac.h entry point with host buffers."""
    M = N = K = 1024
    A = rl.gen_uniform((M, K), seed=0)
    B = rl.gen_uniform((K, N), seed=1)
    C = np.zeros((M, N), np.float32)
    L = lib()
    L.rac_set_cordic_iters(16)
    L.rac_set_cordic_mode(1)
    L.rac_clear_error()
    L.rac_matmul(rl.p(A), rl.p(B), rl.p(C), M, N, K)
    assert L.rac_last_error() == b"", L.rac_last_error()
    d = np.load(os.path.join(rl.GOLDEN, "matmul.npz"))
    idx = d["idx"]
    rows, cols = idx // N, idx % N
    na = np.linalg.norm(A.astype(np.float64), axis=1)[rows]
    nb = np.linalg.norm(B.astype(np.float64), axis=0)[cols]
    err = np.abs(C.ravel()[idx].astype(np.float64) - d["C_samples"])
    assert np.all(err <= 1e-4 * na * nb), float((err / (na * nb)).max())
    ref = rl.orc_matmul_entries(A, B, M, N, K, 16, 1, rows, cols)
    assert np.array_equal(C.ravel()[idx], ref)



def test_rac_h_staging_cache_release():
    """The synchronous rac.h calls stage host buffers through cached device
    buffers; rac_release_cached_memory frees them (returning the bytes) and
    later calls stage afresh with the same results."""
    M, N, K = 256, 192, 320
    A = rl.gen_uniform((M, K), seed=11)
    B = rl.gen_uniform((K, N), seed=12)
    L = lib()
    L.rac_set_cordic_iters(16)
    L.rac_set_cordic_mode(1)
    ref = rl.orc_matmul(A, B, M, N, K, 16, 1)
    C1 = np.zeros((M, N), np.float32)
    L.rac_clear_error()
    L.rac_matmul(rl.p(A), rl.p(B), rl.p(C1), M, N, K)
    assert L.rac_last_error() == b"", L.rac_last_error()
    assert np.array_equal(C1, ref)
    freed = L.rac_release_cached_memory()
    assert freed >= 4 * (M * K + K * N + M * N), freed
    assert L.rac_release_cached_memory() == 0
    C2 = np.zeros((M, N), np.float32)
    L.rac_matmul(rl.p(A), rl.p(B), rl.p(C2), M, N, K)
    assert L.rac_last_error() == b"", L.rac_last_error()
    assert np.array_equal(C2, ref)
    import rac_amd
    assert rac_amd.release_cached_memory() >= 4 * (M * K + K * N + M * N)

@pytest.mark.parametrize("iters", [8, 16, 24])
def test_cordic_matmul_4096_sampled(iters):
    """The metric shape, 4096^3: sampled entries bit-exact vs the checker."""
    M = N = K = 4096
    A = rl.gen_uniform((M, K), seed=0)
    B = rl.gen_uniform((K, N), seed=1)
    got = gemm(A, B, M, N, K, 0, 0, iters, 1)
    rng = np.random.default_rng(iters)
    rows = rng.integers(0, M, 600)
    cols = rng.integers(0, N, 600)
    rows[:4] = [0, 0, M - 1, M - 1]
    cols[:4] = [0, N - 1, 0, N - 1]
    ref = rl.orc_matmul_entries(A, B, M, N, K, iters, 1, rows, cols)
    assert np.array_equal(got[rows, cols], ref)


# Launches pick their register tile from the block count: (3996, 4000) fills
# whole rounds of 256x128 blocks on 256 CUs (FAST 16x8 per lane), (4100,
# 4097) has >= 1024 128x128 blocks (FAST 8x8, CORDIC / SHIFTADD 4x4), (2050,
# 2049) >= 1024 64x64 blocks but fewer 128x128 ones (4x4 for every mode),
# (1500, 1400) 528 64x64 blocks (CORDIC / SHIFTADD 4x4, FAST 2x2), and
# small shapes take 2x2.  Each is ragged on both edges; K < 128 keeps FAST
# on the VALU tiles.
TILE_SHAPES = [(3996, 4000, 19), (4100, 4097, 21), (2050, 2049, 37), (1500, 1400, 45), (90, 70, 50)]


@pytest.mark.parametrize("mode,iters", [(1, 16), (0, 24), (2, 8), (1, 5)])
@pytest.mark.parametrize("layout", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_every_tile_size_ragged(mode, iters, layout):
    """Sampled entries (every corner and the last partial tile rows/columns
    included) bit-exact vs the checker for each register-tile size."""
    ta, tb = layout
    rng = np.random.default_rng(mode * 10 + iters)
    for (M, N, K) in TILE_SHAPES:
        print(f"tile shapes mode={mode} iters={iters} layout={layout} shape={(M, N, K)}", flush=True)
        A = rl.gen_uniform((M, K), seed=M + K)
        B = rl.gen_uniform((K, N), seed=N + 3 * K)
        As = np.ascontiguousarray(A.T) if ta else A
        Bs = np.ascontiguousarray(B.T) if tb else B
        got = gemm(As, Bs, M, N, K, ta, tb, iters, mode)
        rows = np.concatenate([rng.integers(0, M, 300), rng.integers(max(0, M - 70), M, 100), [0, 0, M - 1, M - 1]])
        cols = np.concatenate([rng.integers(0, N, 300), rng.integers(max(0, N - 70), N, 100), [0, N - 1, 0, N - 1]])
        ref = rl.orc_matmul_entries(As, Bs, M, N, K, iters, mode, rows, cols, ta=ta, tb=tb)
        assert np.array_equal(got[rows, cols], ref), (M, N, K)


@pytest.mark.parametrize("mode,shape", [(1, (2050, 2049, 37)), (0, (3996, 4000, 19)), (0, (4100, 4097, 21))])
def test_fused_linear_on_large_tiles(mode, shape):
    """The fused bias + SiLU epilogue on the large register tiles (the
    small-shape fused tests run on the 2x2 tile): CORDIC on 4x4, FAST on
    16x8 and 8x8.  Equal to the unfused GEMM + activation, sampled
    pre-activations bit-exact vs the checker."""
    e = ext()
    M, N, K = shape
    iters = 16 if mode == 1 else 24
    x = rl.gen_normal((M, K), seed=3)
    w = rl.gen_normal((N, K), seed=4, std=0.2)
    b = rl.gen_normal(N, seed=5)
    out, pre = e.fused_linear_forward(T(x), T(w), T(b), 3, iters=iters, mode=mode, return_pre=True)
    lin = e.linear_forward(T(x), T(w), T(b), iters=iters, mode=mode)
    assert torch.equal(pre, lin)
    assert torch.equal(out, e.silu(lin, iters))
    rng = np.random.default_rng(7)
    rows = np.concatenate([rng.integers(0, M, 400), [0, M - 1]])
    cols = np.concatenate([rng.integers(0, N, 400), [N - 1, 0]])
    ref = rl.orc_matmul_entries(x, w, M, N, K, iters, mode, rows, cols, tb=1) + b[cols]
    assert np.array_equal(H(pre)[rows, cols], ref.astype(np.float32))


def test_reference_launcher_abi():
    M, N, K = 48, 40, 56
    A = rl.gen_normal((M, K), 8)
    Bt = rl.gen_normal((N, K), 9)
    Ad, Bd = T(A), T(Bt)
    Cd = torch.zeros((M, N), device=DEV)
    s = torch.cuda.current_stream().cuda_stream
    lib().rac_launch_nt_iters(Ad.data_ptr(), Bd.data_ptr(), Cd.data_ptr(), M, N, K, 1.0, 0.0, 16, 1, s)
    assert np.array_equal(H(Cd), rl.orc_matmul(A, Bt, M, N, K, 16, 1, tb=1))
    lib().rac_launch_nt(Ad.data_ptr(), Bd.data_ptr(), Cd.data_ptr(), M, N, K, 1.0, 0.0, s)
    assert np.array_equal(H(Cd), rl.orc_matmul(A, Bt, M, N, K, 24, 0, tb=1))


# ── exp / activations ──────────────────────────────────────────────────────

SPECIAL = np.float32([0.0, -0.0, 1.0, -1.0, 0.5, 88.0, 88.8, 89.0, -87.0, -88.0, -103.0, -104.0,
                      200.0, -200.0, np.inf, -np.inf, np.nan, 1e-30, -1e-30, 0.34657359, -0.34657359,
                      # |x| / ln2 >= 2^30 and >= 2^31: the range reduction's integer k saturates
                      7.5e8, -7.5e8, 1.5e9, -1.5e9, 3e38, -3e38, 1e-45, -1e-45,
                      # k = 128 with a reduced factor below 1: the exponent field
                      # overflows (inf) although er * 2^128 would still be finite
                      88.38, 88.5, 88.7, -88.38, -88.5, -88.7, 88.376, 88.721])


@pytest.mark.parametrize("iters", [1, 5, 8, 16, 24])
def test_exp_and_activations_bit_exact(iters):
    x = np.concatenate([rl.gen_normal((100003,), 11, std=4.0), SPECIAL]).astype(np.float32)
    e = ext()
    xd = T(x)
    for name, oname in (("exp", "orc_exp_batch"), ("silu", "orc_silu"),
                        ("sigmoid", "orc_sigmoid"), ("tanh", "orc_tanh")):
        print(f"{name} iters={iters}", flush=True)
        got = H(getattr(e, name)(xd, iters=iters))
        ref = rl.orc_unary(oname, x, iters)
        assert np.array_equal(got, ref, equal_nan=True), (name, iters)


@pytest.mark.parametrize("iters", [8, 16, 24])
def test_exp_family_over_all_float_classes(iters):
    """Every 1009th 32-bit pattern (4.26 M floats: both signs, subnormals,
    every exponent, inf and NaN payloads): exp, SiLU, sigmoid and tanh
    bit-exact with the checker."""
    x = (np.arange(0, 2 ** 32, 1009, dtype=np.uint64) & 0xFFFFFFFF).astype(np.uint32).view(np.float32)
    e = ext()
    xd = T(x)
    for name, oname in (("exp", "orc_exp_batch"), ("silu", "orc_silu"),
                        ("sigmoid", "orc_sigmoid"), ("tanh", "orc_tanh")):
        print(f"{name} all float classes iters={iters}", flush=True)
        got = H(getattr(e, name)(xd, iters=iters))
        ref = rl.orc_unary(oname, x, iters)
        assert np.array_equal(got, ref, equal_nan=True), (name, iters)


@pytest.mark.parametrize("iters", [8, 16, 24])
def test_activation_division_every_float(iters):
    """SiLU, sigmoid and tanh on all 2^32 bit patterns against x / (1 + e),
    1 / (1 + e) and copysign((1 - e2) / (1 + e2), x) formed with torch's IEEE
    division on the device from the library's own e = exp(-x) and
    e2 = exp(-2|x|) (the exps the activations use, pinned to the checker by
    the tests above; the activations skip its k <= -127 flush, which 1 + e
    and 1 - e cannot see).  Pins the kernels' shortened division
    (reciprocal, Newton step, one remainder correction, taken when a lane's
    arguments stay in its range) to the IEEE quotient on every input.
    torch's device division is itself checked against numpy's float32
    division on a sample of each chunk."""
    e = ext()
    CH = 1 << 28
    rng = np.random.default_rng(iters)
    for c in range(16):
        lo = -(1 << 31) + c * CH
        print(f"silu/sigmoid/tanh every float iters={iters} chunk {c}", flush=True)
        x = torch.arange(lo, lo + CH, dtype=torch.int32, device=DEV).view(torch.float32)
        d = 1.0 + e.exp(-x, iters=iters)
        e2 = e.exp(-2.0 * x.abs(), iters=iters)
        for name in ("silu", "sigmoid", "tanh"):
            if name == "tanh":
                num, d = 1.0 - e2, 1.0 + e2
            else:
                num = x if name == "silu" else torch.ones_like(x)
            got = getattr(e, name)(x, iters=iters)
            ref = torch.div(num, d)
            if name == "tanh":
                ref = torch.copysign(ref, x)
            bad = (got.view(torch.int32) != ref.view(torch.int32)) & ~(torch.isnan(got) & torch.isnan(ref))
            n_bad = int(bad.sum())
            if n_bad:
                i = int(torch.nonzero(bad)[0, 0])
                pytest.fail(f"{name} iters={iters}: {n_bad} mismatches, first x bits "
                            f"{int(x.view(torch.int32)[i]) & 0xFFFFFFFF:#010x}: {float(got[i])!r} vs {float(ref[i])!r}")
            idx = torch.from_numpy(rng.integers(0, CH, 4096)).to(DEV)
            q = H(torch.div(num, d)[idx])
            with np.errstate(all="ignore"):
                assert np.array_equal(q, H(num[idx]) / H(d[idx]), equal_nan=True), name
            del got, ref, bad, num
        del x, d, e2


def test_elementwise_odd_length_and_offsets():
    e = ext()
    x = rl.gen_normal((1031,), 12, std=3.0)
    full = T(x)
    sub = full[1:]                                   # misaligned, odd length -> scalar path
    got = H(e.silu(sub, iters=16))
    assert np.array_equal(got, rl.orc_unary("orc_silu", x[1:], 16))


def test_gelu_relu_vs_reference():
    d = np.load(os.path.join(rl.GOLDEN, "activations.npz"))
    e = ext()
    g = H(e.gelu(T(d["x"])))
    # erf has no CORDIC mode: device erff vs glibc erff differ by ~1 ulp of
    # erf, which 1 + erf(x) amplifies for x << 0 -> absolute floor 1e-7
    ref = d["gelu"].astype(np.float64)
    assert np.all(np.abs(g - ref) <= 2e-6 * np.abs(ref) + 1e-7)
    r = H(e.relu(T(d["x"])))
    assert np.array_equal(r, np.maximum(d["x"], 0))


def test_rsqrt_sincos_bit_exact():
    rng = np.random.default_rng(2)
    x = np.concatenate([np.exp(rng.uniform(-87, 88, 50000)).astype(np.float32),
                        np.float32([4.0, 1.0, 0.0, -1.0, np.inf, np.nan, 1e-40, 3e38])])
    got = H(ext().rsqrt(T(x)))
    ref = np.array([rl.oracle().orc_rsqrt(float(v)) for v in x], np.float32)
    assert np.array_equal(got, ref, equal_nan=True)
    th = np.concatenate([rng.uniform(-7000, 7000, 20000), [0.0, math.pi / 2, 1e9, np.inf, np.nan]]).astype(np.float32)
    s, c = ext().sincos(T(th))
    s, c = H(s), H(c)
    for i in range(0, len(th), 97):
        so, co = ctypes.c_float(), ctypes.c_float()
        rl.oracle().orc_sincos(float(th[i]), ctypes.byref(so), ctypes.byref(co))
        assert (np.float32(so.value) == s[i] or (np.isnan(s[i]) and math.isnan(so.value)))
        assert (np.float32(co.value) == c[i] or (np.isnan(c[i]) and math.isnan(co.value)))
    assert np.isnan(s[-3]) and np.isnan(s[-2])   # wrap-loop guard


def _float_sweep(stride):
    """Every stride-th 32-bit pattern as float32 (both signs, subnormals,
    every exponent, infinities, NaN payloads)."""
    return (np.arange(0, 2 ** 32, stride, dtype=np.uint64) & 0xFFFFFFFF).astype(np.uint32).view(np.float32)


def test_rsqrt_sincos_over_float_classes():
    """rsqrt on every 1009th bit pattern; sin/cos on every 1009th pattern
    with |theta| < 2^14 (the reference's wrap loop runs |theta| / 2 pi
    times), plus the NaN/inf angles: bit-exact with the checker."""
    x = _float_sweep(1009)
    got = H(ext().rsqrt(T(x)))
    ref = np.empty_like(x)
    rl.oracle().orc_rsqrt_batch(rl.p(x), rl.p(ref), x.size)
    assert np.array_equal(got, ref, equal_nan=True)
    th = x[~(np.abs(x) >= 16384.0)]              # keeps NaN
    th = np.concatenate([th, np.float32([np.inf, -np.inf])])
    s, c = ext().sincos(T(th))
    so, co = np.empty_like(th), np.empty_like(th)
    rl.oracle().orc_sincos_batch(rl.p(th), rl.p(so), rl.p(co), th.size)
    assert np.array_equal(H(s), so, equal_nan=True) and np.array_equal(H(c), co, equal_nan=True)


@pytest.mark.parametrize("mode,iters", [(1, 8), (1, 16), (1, 24), (1, 5), (2, 8), (2, 24), (0, 24)])
def test_mac_over_float_classes(mode, iters):
    """The GEMM's MAC on every 65521st bit pattern of a against 40 values
    of b (a K = 1 product C = A B: one MAC per output), literal per-MAC
    checker; the CORDIC tiles holding out-of-range a take the literal
    rotation chain."""
    a = _float_sweep(65521).reshape(-1, 1)
    b = np.concatenate([rl.gen_normal(28, seed=9, std=3.0),
                        np.float32([0.0, -0.0, 1.0, -1.0, 1e-40, -2.0 ** -120, 3e38, -1.7e38, np.inf, -np.inf,
                                    np.nan, 2.0 ** -100])]).astype(np.float32).reshape(1, -1)
    M, N = a.shape[0], b.shape[1]
    print(f"mac sweep mode={mode} iters={iters} M={M} N={N}", flush=True)
    got = gemm(a, b, M, N, 1, 0, 0, iters, mode)
    ref = rl.orc_matmul(a, b, M, N, 1, iters, mode, literal=1)
    assert np.array_equal(got, ref, equal_nan=True)


def test_scalar_rac_h_entry_points():
    L = lib()
    L.rac_set_cordic_iters(16)
    assert abs(L.rac_rsqrt(4.0) - 0.5) < 1e-6                       # BVT-12
    assert L.rac_rsqrt(0.0) == 0.0 and L.rac_rsqrt(-1.0) == 0.0
    assert abs(L.rac_sigmoid(0.0) - 0.5) < 1e-5
    assert L.rac_sigmoid(10.0) > 0.999 and L.rac_sigmoid(-10.0) < 0.001
    assert np.float32(L.rac_exp(0.75)) == np.float32(rl.oracle().orc_exp_n(0.75, 16))
    s, c = ctypes.c_float(), ctypes.c_float()
    L.rac_sincos(np.float32(math.pi / 2), ctypes.byref(s), ctypes.byref(c))
    assert abs(s.value - 1) < 0.01 and abs(c.value) < 0.01          # BVT-12
    x = rl.gen_normal((300,), 4, std=2.0)
    y = np.zeros_like(x)
    L.rac_softmax(rl.p(x), rl.p(y), 300)
    assert abs(float(y.sum()) - 1) < 1e-5
    assert rl.max_rel(y, rl.orc_softmax(x[None], 16)[0]) < 1e-5
    kat = np.float32([3, 4, 0, 0])
    ko = np.zeros(4, np.float32)
    L.rac_rmsnorm(rl.p(kat), rl.p(ko), None, 1e-6, 1, 4)                # BVT-13
    assert np.allclose(ko, [1.2, 1.6, 0, 0], atol=1e-6)
    xs = rl.gen_normal((257,), 5)
    so = np.zeros_like(xs)
    L.rac_silu(rl.p(xs), rl.p(so), 257)
    assert np.array_equal(so, rl.orc_unary("orc_silu", xs, 16))


@pytest.mark.parametrize("iters", [8, 16, 24])
def test_silu_config4b_full_size(iters):
    """Benchmark config 4b: SiLU over [16384 x 11008] N(0, 1) (44 M float4
    groups, 176 k workgroups), bit-exact with the checker's CORDIC SiLU on
    every element; plus counts that end inside a workgroup's groups and
    inside a float4 (the scalar path)."""
    x = np.random.default_rng(31).standard_normal((16384, 11008), dtype=np.float32)
    got = H(ext().silu(T(x), iters=iters))
    assert np.array_equal(got, rl.orc_unary("orc_silu", x, iters))
    for count in (4 * 256 * 7 + 4 * 129, 4 * 256 + 4, 4 * 3, 4099, 1):
        xs = rl.gen_normal((count,), 32 + count % 7, std=3.0)
        assert np.array_equal(H(ext().silu(T(xs), iters=iters)), rl.orc_unary("orc_silu", xs, iters)), count


# ── softmax / norms ────────────────────────────────────────────────────────

@pytest.mark.parametrize("iters", [8, 16, 24])
def test_softmax_config2(iters):
    """Benchmark config 2: 4096 x 4096, N(0, std 2)."""
    x = rl.gen_normal((4096, 4096), 0, std=2.0)
    got = H(ext().softmax(T(x), iters=iters))
    ref = rl.orc_softmax(x, iters)
    assert rl.max_rel(got, ref, 1e-37) <= 1e-5
    assert np.array_equal(got, rl.orc_softmax_lanes(x, iters))     # the kernel's row-sum order
    assert np.allclose(got.sum(1), 1.0, atol=2e-5)


@pytest.mark.parametrize("shape", [(1, 1), (3, 3), (5, 257), (2, 1024), (7, 16384), (3, 20000), (2, 4099)])
def test_softmax_shapes(shape):
    x = rl.gen_normal(shape, 6, std=2.0)
    if shape[1] > 1:
        x[0, 0] = -np.inf        # masked entry (causal attention): e^-inf = 0
    got = H(ext().softmax(T(x), iters=16))
    ref = rl.orc_softmax(x, 16)
    assert rl.max_rel(got, ref, 1e-37) <= 1e-5
    assert np.array_equal(got, rl.orc_softmax_lanes(x, 16))


@pytest.mark.parametrize("iters", [8, 16, 24, 5])
@pytest.mark.parametrize("cols", [4096, 4000])
def test_softmax_special_rows(iters, cols):
    """Rows holding NaN, +-inf, only -inf, huge offsets and arguments whose
    range reduction saturates: NaN exactly where the checker has NaN (a NaN
    anywhere makes the reference's whole row NaN).  Finite rows are compared
    with the checker's own exps over their float64 sum: rows of equal values
    drive the reference's left-to-right float sum to ~4e-5 relative error,
    which is the checker's rounding, not the kernel's."""
    x = rl.gen_normal((14, cols), 21, std=3.0)
    x[0, 5] = np.nan
    x[1, 0] = np.nan
    x[2, 77] = np.inf
    x[3, :] = -np.inf
    x[4, :100] = -np.inf
    x[5] -= 200.0
    x[5, 3] = 0.0
    x[6] = -np.abs(x[6]) * 40.0
    x[7] = 0.0
    x[8] = -1e30
    x[9] = -np.inf
    x[9, 4] = 1.0
    x[10] = -np.inf
    x[10, 4] = np.nan
    x[11] = 3e38
    x[12, ::2] = -2e9
    x[13] = np.float32(-1e-45)
    x[13, 7] = 0.0
    got = H(ext().softmax(T(x), iters=iters))
    ref = rl.orc_softmax(x, iters)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    nan_rows = np.isnan(ref).any(axis=1)
    assert nan_rows.tolist() == [True] * 4 + [False] * 6 + [True] + [False] * 3
    for r in np.flatnonzero(~nan_rows):
        xm = x[r] - np.max(x[r])                      # float32 subtraction, as the kernel
        e = rl.orc_unary("orc_exp_batch", xm, iters).astype(np.float64)
        assert rl.max_rel(got[r], e / e.sum(), 1e-37) <= 1e-5, r
    # bit for bit against the checker's lane-order model: the rows whose
    # x - max falls below -86 (-inf entries, offsets of -200, -1e30, -2e9)
    # take the ldexp-and-flush scale, the others the exponent-field one, and
    # NaN or an infinite maximum makes the whole row NaN
    lanes = rl.orc_softmax_lanes(x, iters)
    assert np.array_equal(np.isnan(got), np.isnan(lanes))
    fin = ~np.isnan(lanes)
    assert np.array_equal(got[fin], lanes[fin])



def _zero_max_rows(rows, cols, seed):
    """Rows of negative values whose maximum is a zero of mixed signs:
    first zero -0 or +0, all -0, a random sign per element (a zero query
    row's scores), the first zero in another lane's group than a later
    one; plus rows whose maximum is not zero."""
    x = -np.abs(rl.gen_normal((rows, cols), seed, std=2.0)) - np.float32(0.001)
    z = np.float32(0.0)
    nz = np.float32(-0.0)
    plant = [
        lambda r: (r.__setitem__(10, nz), r.__setitem__(cols // 2, z)),
        lambda r: (r.__setitem__(10, z), r.__setitem__(cols // 2, nz)),
        lambda r: r.__setitem__(slice(None), nz),
        lambda r: (r.__setitem__(slice(None), z), r.__setitem__(0, nz)),
        lambda r: r.__setitem__(slice(None), np.where(rl.gen_uniform((cols,), seed + 1) < 0, nz, z)),
        lambda r: (r.__setitem__(min(12, cols - 1), z), r.__setitem__(min(1025, cols - 1), nz)),
        lambda r: (r.__setitem__(min(12, cols - 1), nz), r.__setitem__(min(1025, cols - 1), z)),
        lambda r: None,
    ]
    for i in range(rows):
        plant[i % len(plant)](x[i])
    return x.astype(np.float32)


@pytest.mark.parametrize("iters", [8, 16, 24, 5])
@pytest.mark.parametrize("cols", [4096, 1000, 20000])
def test_softmax_zero_max_takes_first_zero_sign(iters, cols):
    """A zero row maximum carries the sign of the row's first zero, as the
    reference's scan leaves it (rac_cpu.c:258-262: m = x[0], replaced only by
    a strictly greater value); x - max is then +0 or -0 exactly as there,
    which the CORDIC exp's first direction sees.  Bit-exact with the
    checker's lane-order model on the register path (4096 columns, the lean
    unmasked form; 1000, a ragged row), the strided loop (20000) and the
    run-time step count (n = 5)."""
    x = _zero_max_rows(16, cols, 57)
    got = H(ext().softmax(T(x), iters=iters))
    ref = rl.orc_softmax_lanes(x, iters)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_softmax_zero_max_prefetch_and_masked_paths():
    """The same rows through the persistent prefetching kernel (n = 8,
    enough rows for it) and the masked attention softmax (additive mask of
    -0: x + -0 keeps each zero's sign)."""
    x = _zero_max_rows(3072, 4096, 61)
    got = H(ext().softmax(T(x), iters=8))
    ref = rl.orc_softmax_lanes(x, 8)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    Tn = 256
    xs = _zero_max_rows(Tn, Tn, 63)
    mask = np.full((Tn, Tn), -0.0, np.float32)
    for iters in (8, 16):
        sc = T(xs)
        ext().softmax_masked_(sc, T(mask), False, iters=iters)
        ref = rl.orc_softmax_lanes(xs, iters, mask=mask)
        assert np.array_equal(H(sc).view(np.uint32), ref.view(np.uint32))

def test_softmax_vs_libm_reference_reported():
    d = np.load(os.path.join(rl.GOLDEN, "softmax.npz"))
    for iters, bound in ((8, 2 * 2.0 ** -7), (16, 2 * 2.0 ** -14), (24, 3e-6)):
        got = H(ext().softmax(T(d["x"]), iters=iters))
        assert rl.max_rel(got, d["y"]) < bound + 1e-6


@pytest.mark.parametrize("shape", [(16384, 4096), (5, 64), (3, 4099), (4, 1), (2, 40000)])
def test_rmsnorm_layernorm(shape):
    """Benchmark config 4 (16384 x 4096, gamma ~ N(1, 0.02), eps 1e-6) and edge shapes."""
    x = rl.gen_normal(shape, 1)
    g = rl.gen_normal((shape[1],), 2, mean=1.0, std=0.02)
    b = rl.gen_normal((shape[1],), 3, std=0.1)
    e = ext()
    y = H(e.rmsnorm(T(x), T(g), 1e-6))
    assert rl.max_rel(y, rl.orc_rmsnorm(x, g, 1e-6), 1e-30) <= 1e-5
    assert np.array_equal(y, rl.orc_rmsnorm_lanes(x, g, 1e-6))     # the kernel's row-sum order
    y0 = H(e.rmsnorm(T(x), None, 1e-6))
    assert rl.max_rel(y0, rl.orc_rmsnorm(x, None, 1e-6), 1e-30) <= 1e-5
    assert np.array_equal(y0, rl.orc_rmsnorm_lanes(x, None, 1e-6))
    if shape[0] <= 16:
        z = H(e.layernorm(T(x), T(g), T(b), 1e-5))
        assert np.array_equal(z, rl.orc_layernorm_lanes(x, g, b, 1e-5))
        zr = rl.orc_layernorm(x, g, b, 1e-5)
        # LayerNorm outputs are unit-scale; a different order of the mean's
        # sum moves every output by the same ~1e-7, so the bar is relative
        # to max(|z|, 1) (the reference DVT-29 uses atol 1e-5)
        assert np.max(np.abs(z - zr) / np.maximum(np.abs(zr), 1.0)) <= 1e-5


@pytest.mark.parametrize("cols", [4096, 1000])
def test_norm_special_rows(cols):
    """Rows holding NaN, +-inf, all zeros, only subnormals, huge values whose
    squares overflow, tiny and mixed magnitudes: NaN exactly where the
    checker has NaN, zeros where it has zeros, the rest within the row-sum
    bar."""
    x = rl.gen_normal((12, cols), 31)
    x[0, 7] = np.nan
    x[1, 3] = np.inf
    x[2, 5] = -np.inf
    x[3] = 0.0
    x[4] = np.float32(1e-41) * np.sign(x[4])
    x[5] = x[5] * np.float32(3e19)                # squares overflow: mean square = inf
    x[6] = x[6] * np.float32(1e-20)               # squares underflow to ~0: eps dominates
    x[7, ::3] = np.float32(1e18)
    x[8] = x[8] * np.float32(1e15)
    x[9, 0] = np.float32(3e38)
    g = rl.gen_normal((cols,), 32, mean=1.0, std=0.02)
    b = rl.gen_normal((cols,), 33, std=0.1)
    e = ext()
    for eps in (1e-6, 0.0):
        y = H(e.rmsnorm(T(x), T(g), eps))
        r = rl.orc_rmsnorm(x, g, eps)
        assert np.array_equal(np.isnan(y), np.isnan(r)), eps
        assert np.array_equal(y == 0, r == 0), eps
        fin = np.isfinite(r) & (r != 0)
        assert np.all(np.abs(y[fin] - r[fin]) <= 1e-5 * np.abs(r[fin])), eps
        z = H(e.layernorm(T(x), T(g), T(b), eps))
        zr = rl.orc_layernorm(x, g, b, eps)
        assert np.array_equal(np.isnan(z), np.isnan(zr)), eps
        fin = np.isfinite(zr)
        assert np.max(np.abs(z[fin] - zr[fin]) / np.maximum(np.abs(zr[fin]), 1.0)) <= 1e-5, eps


def test_norms_vs_reference_golden():
    d = np.load(os.path.join(rl.GOLDEN, "norms.npz"))
    e = ext()
    assert rl.max_rel(H(e.rmsnorm(T(d["x"]), T(d["gamma"]), 1e-6)), d["rms"], 1e-30) <= 1e-5
    assert rl.max_rel(H(e.rmsnorm(T(d["xw"]), T(d["gw"]), 1e-6)), d["rmsw"], 1e-30) <= 1e-5
    ln = H(e.layernorm(T(d["x"]), T(d["gamma"]), T(d["beta"]), 1e-5))
    assert np.max(np.abs(ln - d["ln"]) / np.maximum(np.abs(d["ln"]), 1.0)) <= 1e-5


# ── RoPE ───────────────────────────────────────────────────────────────────

def test_rope_cache_bit_exact_vs_reference_digest():
    d = np.load(os.path.join(rl.GOLDEN, "rope.npz"))
    c, s = ext().rope_cache(4096, 128, 10000.0, device=DEV)
    c, s = H(c), H(s)
    assert rl.sha256(c) == str(d["big_cos_sha"]) and rl.sha256(s) == str(d["big_sin_sha"])
    c2 = np.zeros((64, 16), np.float32)
    s2 = np.zeros((64, 16), np.float32)
    lib().rac_rope_cache(rl.p(c2), rl.p(s2), 64, 32, 10000.0)
    assert np.array_equal(c2, d["small_cos"]) and np.array_equal(s2, d["small_sin"])


@pytest.mark.parametrize("shape", [(2, 2, 16, 64), (1, 3, 37, 6), (2, 1, 9, 2), (1, 2, 40, 1024), (3, 5, 33, 128)])
def test_rope_apply_bit_exact(shape):
    B, Hh, Tt, D = shape
    x = rl.gen_normal(shape, 17)
    c, s = rl.orc_rope_cache(Tt, D)
    ref = rl.orc_rope_apply(x, c, s)
    xd = T(x)
    ext().rope_apply_(xd, T(c), T(s))
    assert np.array_equal(H(xd), ref)
    # the [B, T, H, D] storage used by attention projections
    xt = T(np.ascontiguousarray(x.transpose(0, 2, 1, 3)))
    view = xt.transpose(1, 2)
    # out of place first (reads the view, leaves it untouched), then in place
    y = ext().rope_apply(view, T(c), T(s))
    assert y.is_contiguous() and np.array_equal(H(y), ref)
    assert np.array_equal(H(view), x)
    ext().rope_apply_(view, T(c), T(s))
    assert np.array_equal(H(view), ref)
    assert np.array_equal(H(ext().rope_apply(T(x), T(c), T(s))), ref)


def test_rope_apply_golden_and_rac_h():
    d = np.load(os.path.join(rl.GOLDEN, "rope.npz"))
    x = np.array(d["apply_x"], copy=True)
    c, s = d["apply_cos"], d["apply_sin"]     # keep the arrays alive across the call
    lib().rac_rope_apply(rl.p(x), rl.p(c), rl.p(s), 2, 2, 16, 64)
    assert np.array_equal(x, d["apply_out"])


def test_rope_config3_full_size():
    """Benchmark config 3: Q and K [8, 32, 4096, 128] (B,H,T,D), tables from
    rac_rope_cache(4096, 128, 10000): bit-exact over the full tensors."""
    shape = (8, 32, 4096, 128)
    c, s = ext().rope_cache(4096, 128, device=DEV)
    ch, sh = H(c), H(s)
    gen = torch.Generator(device=DEV)
    for seed in (0, 1):
        gen.manual_seed(seed)
        xd = torch.randn(shape, device=DEV, generator=gen)
        x = H(xd)
        ref = rl.orc_rope_apply(x, ch, sh)
        if seed == 1:        # out of place, through the module's path
            got = H(ext().rope_apply(xd, c, s))
        else:
            ext().rope_apply_(xd, c, s)
            got = H(xd)
        assert np.array_equal(got, ref)
        del xd, got, ref, x


# ── torch surface ──────────────────────────────────────────────────────────

def test_rac_linear_forward_backward():
    from rac_amd import rac_torch as rt
    rt.rac_set_mode('cordic')
    rt.rac_set_precision(16)
    try:
        torch.manual_seed(0)
        lin = rt.RACLinear(96, 80).to(DEV)
        x = torch.randn(3, 7, 96, device=DEV, requires_grad=True)
        y = lin(x)
        W = H(lin.weight)
        xin = H(x).reshape(-1, 96)
        ref = rl.orc_matmul(xin, W, 21, 80, 96, 16, 1, tb=1) + H(lin.bias)[None]
        assert np.array_equal(H(y).reshape(21, 80), ref.astype(np.float32))
        g = torch.randn_like(y)
        y.backward(g)
        go = H(g).reshape(21, 80)
        gi_ref = rl.orc_matmul(go, W, 21, 96, 80, 16, 1)
        gw_ref = rl.orc_matmul(go, xin, 80, 96, 21, 16, 1, ta=1)
        assert np.array_equal(H(x.grad).reshape(21, 96), gi_ref)
        assert np.array_equal(H(lin.weight.grad), gw_ref)
        assert np.allclose(H(lin.bias.grad), go.sum(0), rtol=1e-5, atol=1e-5)
    finally:
        rt.rac_set_mode('fast')
        rt.rac_set_precision(24)


def test_rac_matmul_fast_mode_matches_torch():
    from rac_amd import rac_torch as rt
    A = torch.randn(70, 50, device=DEV)
    B = torch.randn(50, 30, device=DEV)
    C = rt.rac_matmul(A, B)
    assert torch.allclose(C, A.double().matmul(B.double()).float(), rtol=1e-4, atol=1e-4)


def test_reference_dvt_properties():
    from rac_amd import rac_torch as rt
    torch.manual_seed(42)
    rope = rt.RACRoPE(head_dim=16, max_seq_len=32)
    q = torch.randn(2, 4, 8, 16, device=DEV)
    k = torch.randn_like(q)
    q2, k2 = rope(q, k)
    m0 = q.view(2, 4, 8, 8, 2).pow(2).sum(-1).sqrt()
    m1 = q2.view(2, 4, 8, 8, 2).pow(2).sum(-1).sqrt()
    assert torch.allclose(m0, m1, atol=1e-4)                          # DVT-27
    assert torch.allclose(q[:, :, 0], q2[:, :, 0], atol=1e-4)
    q3, _ = rope(q, k, positions=torch.arange(8))
    assert torch.allclose(q3, q2, atol=1e-4)
    ql = torch.randn(1, 1, 4, 16, device=DEV, requires_grad=True)
    kl = torch.randn(1, 1, 4, 16, device=DEV, requires_grad=True)
    qo, ko = rope(ql, kl)
    (qo.sum() + ko.sum()).backward()
    assert ql.grad is not None and kl.grad is not None
    # RMSNorm vs formula (DVT-28, atol 1e-5)
    rms = rt.RACRMSNorm(64, eps=1e-6).to(DEV)
    x = torch.randn(8, 64, device=DEV)
    yref = (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)) * rms.weight
    assert torch.allclose(rms(x), yref, atol=1e-5)
    # LayerNorm vs nn.LayerNorm (DVT-29, atol 1e-5)
    ln = rt.RACLayerNorm(48, eps=1e-5).to(DEV)
    tn = torch.nn.LayerNorm(48, eps=1e-5).to(DEV)
    x = torch.randn(4, 7, 48, device=DEV)
    assert torch.allclose(ln(x), tn(x), atol=1e-5)


def test_llama_block_small_forward_backward_and_causality():
    from rac_amd import rac_torch as rt
    torch.manual_seed(0)
    blk = rt.RACLlamaBlock(64, 4, ff_dim=176, max_seq_len=32).to(DEV)
    x = torch.randn(2, 16, 64, device=DEV, requires_grad=True)
    y = blk(x, is_causal=True)
    assert y.shape == x.shape and torch.isfinite(y).all()
    y.sum().backward()
    assert x.grad is not None and all(p.grad is not None for p in blk.parameters())
    blk.eval()
    xa = torch.randn(1, 8, 64, device=DEV)
    xb = xa.clone()
    xb[:, -1] = torch.randn(64, device=DEV)
    with torch.no_grad():
        ya, yb = blk(xa, is_causal=True), blk(xb, is_causal=True)
    assert torch.allclose(ya[:, :-1], yb[:, :-1], atol=1e-4)         # DVT-30


def test_llama_block_matches_oracle_composition():
    """RACLlamaBlock (CORDIC mode, n=16) vs the same block composed on the CPU
    from the checker's ops (CORDIC matmul, RoPE table/apply, RMSNorm with
    CORDIC rsqrt, CORDIC softmax and SiLU); QK^T and AV, which the reference
    leaves to torch.matmul, are float64 on the CPU side."""
    from rac_amd import rac_torch as rt
    d, nh, ff, T = 128, 4, 352, 48
    hd = d // nh
    torch.manual_seed(3)
    blk = rt.RACLlamaBlock(d, nh, ff_dim=ff, max_seq_len=64).to(DEV)
    with torch.no_grad():
        for prm in blk.parameters():
            if prm.dim() == 2:
                prm.normal_(0.0, 0.05)
        blk.norm1.weight.normal_(1.0, 0.02)
        blk.norm2.weight.normal_(1.0, 0.02)
    x = torch.randn(1, T, d, device=DEV)
    rt.rac_set_mode('cordic')
    rt.rac_set_precision(16)
    try:
        with torch.no_grad():
            y = H(blk(x, is_causal=True))
    finally:
        rt.rac_set_mode('fast')
        rt.rac_set_precision(24)
    P = {k: H(v) for k, v in blk.state_dict().items()}
    xn = H(x)[0]

    def lin(a, w):
        return rl.orc_matmul(np.ascontiguousarray(a, np.float32), np.ascontiguousarray(w), a.shape[0],
                             w.shape[0], a.shape[1], 16, 1, tb=1)

    h = rl.orc_rmsnorm(xn, P["norm1.weight"], 1e-6)
    qkv = lin(h, P["attn.qkv.weight"])
    q, k, v = qkv[:, :d], qkv[:, d:2 * d], qkv[:, 2 * d:]
    c, s = rl.orc_rope_cache(64, hd)
    q = rl.orc_rope_apply(q.reshape(1, T, nh, hd).transpose(0, 2, 1, 3), c, s)
    k = rl.orc_rope_apply(k.reshape(1, T, nh, hd).transpose(0, 2, 1, 3), c, s)
    v = v.reshape(1, T, nh, hd).transpose(0, 2, 1, 3)
    sc = (q.astype(np.float64) @ k.astype(np.float64).transpose(0, 1, 3, 2)) * hd ** -0.5
    sc = sc + np.triu(np.full((T, T), -np.inf), 1)
    att = rl.orc_softmax(sc.astype(np.float32).reshape(-1, T), 16).reshape(1, nh, T, T)
    o = (att.astype(np.float64) @ v.astype(np.float64)).transpose(0, 2, 1, 3).reshape(T, d)
    x1 = xn + lin(o.astype(np.float32), P["attn.out_proj.weight"])
    h2 = rl.orc_rmsnorm(x1, P["norm2.weight"], 1e-6)
    f1 = rl.orc_unary("orc_silu", lin(h2, P["ffn.fc1.weight"]), 16)
    ref = x1 + lin(f1, P["ffn.fc2.weight"])
    err = np.abs(y[0] - ref) / np.maximum(np.abs(ref), 1.0)
    assert err.max() < 1e-4, err.max()



@pytest.mark.parametrize("cols,rows", [(1024, 16384), (2048, 8192), (4096, 6000)])
def test_softmax_prefetch_path(cols, rows):
    """Short exps (n = 8) over enough rows for the persistent kernel that
    prefetches each workgroup's next row into LDS (every workgroup takes at
    least two rows; the row count is no multiple of the grid): bit-exact with
    the lane-order checker.  Special rows (NaN, +-inf, only -inf, huge
    offsets) sit where workgroups take their first, second and later rows;
    each gives the same bits, NaN payloads included, as the same row alone
    (one row: the one-row-per-workgroup kernel)."""
    x = rl.gen_normal((rows, cols), 31, std=2.0)
    where = [0, 1, 255, 1279, 1280, 1536, 2047, 2048, 2559, 3071, 4095, rows - 2, rows - 1]
    for q, r in enumerate(where):
        kind = q % 6
        if kind == 0:
            x[r, 17] = np.nan
        elif kind == 1:
            x[r, 3] = np.inf
        elif kind == 2:
            x[r, :] = -np.inf
        elif kind == 3:
            x[r] -= 200.0
        elif kind == 4:
            x[r] = -np.abs(x[r]) * 40.0
        else:
            x[r, ::2] = -2e9
    xt = T(x)
    got = H(ext().softmax(xt, iters=8))
    ref = rl.orc_softmax_lanes(x, 8)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    fin = ~np.isnan(ref)
    assert np.array_equal(got[fin], ref[fin])
    for r in where:
        one = H(ext().softmax(xt[r:r + 1], iters=8))
        assert np.array_equal(one.view(np.int32), got[r:r + 1].view(np.int32)), r
    # in place (y == x): each row is read whole before it is written, and the
    # prefetched row is one no workgroup has written yet
    rc = lib().rac_softmax_dev(xt.data_ptr(), xt.data_ptr(), rows, cols, 8, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib().rac_last_error()
    assert np.array_equal(H(xt).view(np.int32), got.view(np.int32))


def test_sincos_large_angles_wrap():
    """The device takes the reference's sequential wrap (rac_cpu.c:92-94) a
    binade at a time; the checker runs the loop itself.  Angles on both sides
    of every binade boundary from 2^4 to 2^26 (the last step that stays in a
    binade and the one that leaves it), spread through each binade, and up
    to the largest float below 2^27: bit-exact, both signs."""
    th = []
    for e in range(4, 27):
        base = np.float32(2.0 ** e)
        for k in (0, 1, 2, 3, 7, 1000, 65535):
            th.append(np.nextafter(base, np.float32(np.inf), dtype=np.float32) if k == 1 else base + np.float32(k) * np.spacing(base))
            th.append(np.float32(2.0 ** (e + 1)) - np.float32(k + 1) * np.spacing(base))
        th.extend((base * np.float32(1.0 + f)).astype(np.float32) for f in (0.1234567, 0.5, 0.7777777, 0.9999))
    th = np.float32(th)
    th = np.concatenate([th, -th, np.float32([np.nextafter(np.float32(2.0 ** 27), np.float32(0))] * 2) * np.float32([1, -1])])
    s, c = ext().sincos(T(th))
    so, co = np.empty_like(th), np.empty_like(th)
    rl.oracle().orc_sincos_batch(rl.p(th), rl.p(so), rl.p(co), th.size)
    assert np.array_equal(H(s), so) and np.array_equal(H(c), co)


def test_rope_cache_long_context_vs_checker():
    """A 65536-position table (angles up to 65535 rad: the reference's wrap
    loop runs up to ~10^4 times per entry) equals the checker bit for bit."""
    c, s = ext().rope_cache(65536, 64, 10000.0, device=DEV)
    oc, os_ = rl.orc_rope_cache(65536, 64)
    assert np.array_equal(H(c), oc) and np.array_equal(H(s), os_)
