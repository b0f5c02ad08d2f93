"""GPU parity of the RAC GEMM for few rows (M <= 16) or few columns
(N <= 16), A not transposed.

Such launches run gemm_skinny_kernel / gemm_skinny_pipe_kernel: the per-MAC
terms of a K-tile (the CORDIC rotation with its gain correction, the
shift-add product) are computed by the lanes, then one lane per output
folds them in k order.
Each output must equal the reference's rac_fma_iters chain
(rac_kernels.hip:204-219) bit for bit, as the block-tiled kernel does, in
all three MAC modes: one row or column and several, NN and NT, ragged
dimensions, the iteration counts with compile-time chains (8, 16, 24) and
a run-time one (5), special operands (the literal rotation chain), alpha /
beta, batches, and the fused bias + activation epilogue of a decode-time
linear and of a classifier head.
"""
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


def lib():
    import rac_amd
    return rac_amd.load()


def ext():
    from rac_amd import ext as e
    return e


def gemm(A, B, M, N, K, tb, iters, mode, alpha=1.0, beta=0.0, C0=None):
    Ad, Bd = T(A), T(B)
    Cd = T(C0) if C0 is not None else torch.zeros((M, N), device=DEV)
    rc = lib().rac_gemm_dev(Ad.data_ptr(), Bd.data_ptr(), Cd.data_ptr(), M, N, K, 0, tb, alpha, beta, iters,
                            mode, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib().rac_last_error()
    return H(Cd)


MODES = [(0, 24), (1, 16), (1, 8), (1, 24), (1, 5), (2, 16), (2, 24)]
# (1, 4096, 1030): one row (1 x 16 blocks, K ragged); (3, 2100, 777): 4 x 16
# (FAST: 512-k tiles on grids of at most one workgroup per CU, both);
# (2, 5000, 300): 4 x 16 on a wider grid (FAST: 256-k tiles); (7, 1500,
# 333): 8 x 8 (FAST 8 x 16); (6, 5000, 300): 8 x 16; (16, 1000, 300) and
# (9, 35, 67): 16 x 8; (16, 5000, 200): 16 x 16 (CORDIC: each lane computes
# its own terms; SHIFTADD 16 x 8); (1, 5, 3): tiny.
SHAPES = [(1, 4096, 1030), (3, 2100, 777), (2, 5000, 300), (7, 1500, 333), (6, 5000, 300), (16, 1000, 300),
          (9, 35, 67), (16, 5000, 200), (1, 5, 3)]


@pytest.mark.parametrize("tb", [0, 1])
@pytest.mark.parametrize("mode,iters", MODES)
def test_skinny_bit_exact(mode, iters, tb):
    for (M, N, K) in SHAPES:
        print(f"skinny mode={mode} iters={iters} tb={tb} shape={(M, N, K)}", flush=True)
        A = rl.gen_normal((M, K), seed=M + K)
        B = rl.gen_normal((N, K) if tb else (K, N), seed=N + 2 * K)
        got = gemm(A, B, M, N, K, tb, iters, mode)
        ref = rl.orc_matmul(A, B, M, N, K, iters, mode, tb=tb)
        assert np.array_equal(got, ref), (M, N, K, float(np.max(np.abs(got - ref))))


SPECIALS = np.array([0.0, -0.0, 1e-45, -3e-39, 2.0 ** -126, -(2.0 ** -110), 1.5 * 2.0 ** -106, 2.0 ** -105,
                     1.9 * 2.0 ** 126, -(2.0 ** 127), 3e38, np.inf, -np.inf, np.nan, 1.0, -0.75], np.float32)


@pytest.mark.parametrize("mode,iters", [(1, 16), (1, 5), (0, 24), (2, 8)])
def test_skinny_special_values(mode, iters):
    """Subnormal, tiny (< 2^-105), top-binade, infinite and NaN operands:
    the CORDIC terms of those A elements take the literal rotation chain;
    bit-exact, NaN exactly where the checker has NaN."""
    rng = np.random.default_rng(mode * 31 + iters)
    for (M, N, K, tb) in [(4, 700, 300, 1), (1, 1500, 513, 0)]:
        print(f"skinny specials mode={mode} iters={iters} shape={(M, N, K)} tb={tb}", flush=True)
        A = rl.gen_uniform((M, K), seed=M + K)
        B = rl.gen_uniform((N, K) if tb else (K, N), seed=N)
        # tiny and subnormal specials in every row; huge, inf and NaN ones in
        # all rows but the last (their rows overflow or turn NaN)
        for r in range(M):
            pool = SPECIALS if r < M - 1 else SPECIALS[:8]
            A[r, rng.integers(0, K, 4)] = rng.choice(pool, 4)
        if M > 1:
            A[0, 7] = np.nan
        B.reshape(-1)[rng.integers(0, B.size, 8)] = rng.choice(SPECIALS[:11], 8)
        got = gemm(A, B, M, N, K, tb, iters, mode)
        ref = rl.orc_matmul(A, B, M, N, K, iters, mode, tb=tb, literal=1)
        assert np.array_equal(got, ref, equal_nan=True), (M, N, K)
        # (SHIFTADD flushes products with a NaN or infinite operand to 0)
        assert np.isfinite(ref).any() and (M == 1 or mode == 2 or np.isnan(ref).any())


@pytest.mark.parametrize("mode,iters", [(1, 16), (0, 24), (2, 16)])
def test_skinny_alpha_beta_and_batch(mode, iters):
    M, N, K = 5, 1300, 400
    A = rl.gen_normal((M, K), 3)
    B = rl.gen_normal((K, N), 4)
    C0 = rl.gen_normal((M, N), 5)
    got = gemm(A, B, M, N, K, 0, iters, mode, alpha=0.5, beta=-2.0, C0=C0)
    assert np.array_equal(got, rl.orc_matmul(A, B, M, N, K, iters, mode, alpha=0.5, beta=-2.0, C0=C0))
    e = ext()
    Z = 3
    Ab = rl.gen_uniform((Z, 2, 600), seed=7)
    Bb = rl.gen_uniform((Z, 900, 600), seed=8)
    out = H(e.bmm(T(Ab), T(Bb), trans_b=True, alpha=0.75, iters=iters, mode=mode))
    for z in range(Z):
        ref = rl.orc_matmul(np.ascontiguousarray(Ab[z]), np.ascontiguousarray(Bb[z]), 2, 900, 600, iters, mode,
                            tb=1, alpha=0.75)
        assert np.array_equal(out[z], ref), z


@pytest.mark.parametrize("N", [11008, 4096])
@pytest.mark.parametrize("mode,iters", [(1, 16), (0, 24)])
def test_skinny_decode_linear(mode, iters, N):
    """A decode step's linear layer: x [1, 4096] @ W[N, 4096]^T + b with
    SiLU, fused and unfused; pre-activations bit-exact vs the checker.
    N = 4096 is a grid of one workgroup per CU: the 512-lane CORDIC
    pipeline and FAST's 8-wide blocks, with the fused epilogue."""
    e = ext()
    M, K = 1, 4096
    print(f"decode linear mode={mode} iters={iters} N={N}", flush=True)
    x = rl.gen_normal((M, K), seed=41)
    w = rl.gen_normal((N, K), seed=42, std=0.02)
    b = rl.gen_normal(N, seed=43)
    out, pre = e.fused_linear_forward(T(x), T(w), T(b), 3, iters=iters, mode=mode, return_pre=True)
    lin = e.linear_forward(T(x), T(w), T(b), iters=iters, mode=mode)
    assert torch.equal(pre, lin)
    assert torch.equal(out, e.silu(lin, iters))
    ref = rl.orc_matmul(x, w, M, N, K, iters, mode, tb=1) + b[None, :]
    assert np.array_equal(H(pre), ref.astype(np.float32))


# Few columns (the same blocks transposed): (4096, 1, 1030) a matrix-vector
# product, 16 x 1 blocks; (2100, 3, 777) 16 x 4; (1500, 7, 333) 8 x 8
# (FAST 16 x 8); (5000, 6, 300) 16 x 8; (1000, 16, 300), (35, 9, 67) and
# (2048, 10, 4096), a classifier head, 8 x 16; (5000, 16, 200) 16 x 16.
COL_SHAPES = [(4096, 1, 1030), (2100, 3, 777), (1500, 7, 333), (5000, 6, 300), (1000, 16, 300), (35, 9, 67),
              (2048, 10, 4096), (5000, 16, 200)]


@pytest.mark.parametrize("tb", [0, 1])
@pytest.mark.parametrize("mode,iters", MODES)
def test_fewcol_bit_exact(mode, iters, tb):
    for (M, N, K) in COL_SHAPES:
        if mode == 2 and M * N * K > 2 ** 26:
            continue                                    # the checker's SHIFTADD loop: keep it short
        print(f"fewcol mode={mode} iters={iters} tb={tb} shape={(M, N, K)}", flush=True)
        A = rl.gen_normal((M, K), seed=M + K + 1)
        B = rl.gen_normal((N, K) if tb else (K, N), seed=N + 2 * K + 1)
        got = gemm(A, B, M, N, K, tb, iters, mode)
        ref = rl.orc_matmul(A, B, M, N, K, iters, mode, tb=tb)
        assert np.array_equal(got, ref), (M, N, K, float(np.max(np.abs(got - ref))))


@pytest.mark.parametrize("mode,iters", [(1, 16), (1, 5), (0, 24), (2, 8)])
def test_fewcol_special_values(mode, iters):
    rng = np.random.default_rng(mode * 37 + iters)
    for (M, N, K, tb) in [(700, 4, 300, 1), (1500, 1, 513, 0)]:
        print(f"fewcol specials mode={mode} iters={iters} shape={(M, N, K)} tb={tb}", flush=True)
        A = rl.gen_uniform((M, K), seed=M + K)
        B = rl.gen_uniform((N, K) if tb else (K, N), seed=N)
        for r in rng.integers(0, M, 40):
            A[r, rng.integers(0, K, 4)] = rng.choice(SPECIALS, 4)
        for r in rng.integers(0, M, 40):
            A[r, rng.integers(0, K, 4)] = rng.choice(SPECIALS[:8], 4)
        got = gemm(A, B, M, N, K, tb, iters, mode)
        ref = rl.orc_matmul(A, B, M, N, K, iters, mode, tb=tb, literal=1)
        assert np.array_equal(got, ref, equal_nan=True), (M, N, K)
        assert np.isfinite(ref).any() and (mode == 2 or np.isnan(ref).any())


@pytest.mark.parametrize("mode,iters", [(1, 16), (0, 24), (2, 16)])
def test_fewcol_alpha_beta_and_batch(mode, iters):
    M, N, K = 1300, 5, 400
    A = rl.gen_normal((M, K), 3)
    B = rl.gen_normal((K, N), 4)
    C0 = rl.gen_normal((M, N), 5)
    got = gemm(A, B, M, N, K, 0, iters, mode, alpha=0.5, beta=-2.0, C0=C0)
    assert np.array_equal(got, rl.orc_matmul(A, B, M, N, K, iters, mode, alpha=0.5, beta=-2.0, C0=C0))
    e = ext()
    Z = 3
    Ab = rl.gen_uniform((Z, 900, 600), seed=7)
    Bb = rl.gen_uniform((Z, 2, 600), seed=8)
    out = H(e.bmm(T(Ab), T(Bb), trans_b=True, alpha=0.75, iters=iters, mode=mode))
    for z in range(Z):
        ref = rl.orc_matmul(np.ascontiguousarray(Ab[z]), np.ascontiguousarray(Bb[z]), 900, 2, 600, iters, mode,
                            tb=1, alpha=0.75)
        assert np.array_equal(out[z], ref), z


@pytest.mark.parametrize("mode,iters", [(1, 16), (0, 24)])
def test_fewcol_classifier_head(mode, iters):
    """x [512, 4096] @ W[10, 4096]^T + b with GELU and without, fused and
    unfused: pre-activations bit-exact vs the checker."""
    e = ext()
    M, N, K = 512, 10, 4096
    x = rl.gen_normal((M, K), seed=51)
    w = rl.gen_normal((N, K), seed=52, std=0.02)
    b = rl.gen_normal(N, seed=53)
    out, pre = e.fused_linear_forward(T(x), T(w), T(b), 2, iters=iters, mode=mode, return_pre=True)
    lin = e.linear_forward(T(x), T(w), T(b), iters=iters, mode=mode)
    assert torch.equal(pre, lin)
    assert torch.equal(out, e.gelu(lin))
    ref = rl.orc_matmul(x, w, M, N, K, iters, mode, tb=1) + b[None, :]
    assert np.array_equal(H(pre), ref.astype(np.float32))
