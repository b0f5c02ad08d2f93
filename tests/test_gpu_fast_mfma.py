"""GPU parity of the FAST-mode GEMM on the matrix cores.

FAST launches with at least a quarter as many 128x128 blocks as CUs, at
least half of their outputs real, and K >= 128 run on
v_mfma_f32_32x32x1_2b_f32, one instruction per k in k order; each
output must equal the reference's fmaf chain (rac_kernels.hip:204-219, mode
FAST) bit for bit, like the VALU tiles do.  Shapes below are chosen to take
that path: ragged on every edge, K not a multiple of 4 (element loads), all
dimensions multiples of 4 (16-byte loads), exact tiles, a base address off
the 16-byte grid, batched launches with alpha / beta, the fused bias +
activation epilogue, special operands (subnormal, infinite, NaN), launches
of fewer blocks than CUs, and the config-5 attention core's P V chunks.
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


def gemm(A, B, M, N, K, ta, tb, alpha=1.0, beta=0.0, C0=None, offset=0):
    """rac_gemm_dev in FAST mode; `offset` floats of padding in front of A
    and B move their base addresses off the 16-byte grid."""
    Ad = torch.zeros(A.size + offset, device=DEV)
    Bd = torch.zeros(B.size + offset, device=DEV)
    Ad[offset:] = T(A.ravel())
    Bd[offset:] = T(B.ravel())
    Cd = T(C0) if C0 is not None else torch.zeros((M, N), device=DEV)
    rc = lib().rac_gemm_dev(Ad.data_ptr() + 4 * offset, Bd.data_ptr() + 4 * offset, Cd.data_ptr(), M, N, K,
                            ta, tb, alpha, beta, 24, 0, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib().rac_last_error()
    return H(Cd)


def operands(M, N, K, ta, tb, seed):
    A = rl.gen_normal((M, K), seed=seed)
    B = rl.gen_normal((K, N), seed=seed + 1)
    As = np.ascontiguousarray(A.T) if ta else A
    Bs = np.ascontiguousarray(B.T) if tb else B
    return As, Bs


# (2100, 2100, 129): ragged tiles, K % 4 != 0 and N % 4 != 0 (element
# loads); (2052, 2100, 260): every dimension a multiple of 4 (16-byte loads),
# ragged tiles; (2048, 2176, 512): exact tiles.  These take wave tiles of
# 64 x 64 (128 x 128 blocks); the 4000 x 4000 shapes fill one round of
# 256 x 128 blocks and take 128 x 64 wave tiles (ragged on both edges).
MF_SHAPES = [(2100, 2100, 129), (2052, 2100, 260), (2048, 2176, 512), (4000, 4000, 129), (4000, 4000, 260)]


@pytest.mark.parametrize("layout", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("shape", MF_SHAPES)
def test_fast_mfma_bit_exact(shape, layout):
    M, N, K = shape
    ta, tb = layout
    print(f"fast mfma shape={shape} layout={layout}", flush=True)
    As, Bs = operands(M, N, K, ta, tb, seed=M + K + 2 * ta + tb)
    got = gemm(As, Bs, M, N, K, ta, tb)
    ref = rl.orc_matmul(As, Bs, M, N, K, 24, 0, ta=ta, tb=tb)
    assert np.array_equal(got, ref), float(np.max(np.abs(got - ref)))


@pytest.mark.parametrize("shape", [(2052, 2100, 260), (4000, 4000, 260)])
@pytest.mark.parametrize("layout", [(0, 0), (0, 1), (1, 0)])
def test_fast_mfma_unaligned_base(layout, shape):
    """Dimensions that allow 16-byte loads, base addresses that do not."""
    M, N, K = shape
    ta, tb = layout
    print(f"fast mfma unaligned layout={layout}", flush=True)
    As, Bs = operands(M, N, K, ta, tb, seed=11)
    got = gemm(As, Bs, M, N, K, ta, tb, offset=1)
    assert np.array_equal(got, rl.orc_matmul(As, Bs, M, N, K, 24, 0, ta=ta, tb=tb))
    assert np.array_equal(got, gemm(As, Bs, M, N, K, ta, tb))


SPECIALS = np.array([0.0, -0.0, 1e-45, -3e-39, 2.0 ** -126, -(2.0 ** -110), 3e38, -(2.0 ** 127),
                     np.inf, -np.inf, np.nan, 1.0, -0.75], np.float32)


@pytest.mark.parametrize("shape", [(2100, 2100, 130), (4000, 4000, 130)])
@pytest.mark.parametrize("layout", [(0, 0), (1, 1)])
def test_fast_mfma_special_values(layout, shape):
    """Subnormal, huge, infinite and NaN operands through the matrix cores:
    every finite output bit-exact, NaN exactly where the checker has NaN."""
    M, N, K = shape
    ta, tb = layout
    rng = np.random.default_rng(5)
    A = rl.gen_uniform((M, K), seed=3)
    B = rl.gen_uniform((K, N), seed=4)
    for r in rng.integers(16, M, 8):
        A[r, rng.integers(0, K, 5)] = rng.choice(SPECIALS, 5)
    B[rng.integers(0, K, 6), rng.integers(16, N, 6)] = rng.choice(SPECIALS, 6)
    # subnormal products and a subnormal sum: row 7 of A and column 9 of B
    # scaled by 2^-70 (no special operand lands in either)
    A[7, :] *= np.float32(2.0 ** -70)
    B[:, 9] *= np.float32(2.0 ** -70)
    As = np.ascontiguousarray(A.T) if ta else A
    Bs = np.ascontiguousarray(B.T) if tb else B
    got = gemm(As, Bs, M, N, K, ta, tb)
    ref = rl.orc_matmul(As, Bs, M, N, K, 24, 0, ta=ta, tb=tb, literal=1)
    assert np.array_equal(got, ref, equal_nan=True)
    assert np.isnan(ref).any() and np.isinf(ref).any()
    assert 0 < abs(ref[7, 9]) < 2.0 ** -126


def test_fast_mfma_alpha_beta():
    M, N, K = 2100, 2052, 300
    A = rl.gen_normal((M, K), 3)
    B = rl.gen_normal((K, N), 4)
    C0 = rl.gen_normal((M, N), 5)
    got = gemm(A, B, M, N, K, 0, 0, alpha=0.5, beta=-2.0, C0=C0)
    assert np.array_equal(got, rl.orc_matmul(A, B, M, N, K, 24, 0, alpha=0.5, beta=-2.0, C0=C0))


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0)])
def test_fast_mfma_batched(ta, tb):
    """4 batch items of 1100 x 1100 (324 tiles): bmm with alpha, then
    accumulating into the result with beta."""
    e = ext()
    Z, M, N, K = 4, 1100, 1100, 200
    A = rl.gen_uniform((Z, K, M) if ta else (Z, M, K), seed=5 + ta)
    B = rl.gen_uniform((Z, N, K) if tb else (Z, K, N), seed=9 + tb)
    C = e.bmm(T(A), T(B), trans_a=bool(ta), trans_b=bool(tb), alpha=0.75, iters=24, mode=0)
    first = H(C).copy()
    e.bmm(T(A), T(B), trans_a=bool(ta), trans_b=bool(tb), alpha=1.0, iters=24, mode=0, out=C, beta=0.5)
    second = H(C)
    for z in range(Z):
        Az, Bz = np.ascontiguousarray(A[z]), np.ascontiguousarray(B[z])
        ref = rl.orc_matmul(Az, Bz, M, N, K, 24, 0, ta=ta, tb=tb, alpha=0.75)
        assert np.array_equal(first[z], ref), z
        ref2 = rl.orc_matmul(Az, Bz, M, N, K, 24, 0, ta=ta, tb=tb, alpha=1.0, beta=0.5, C0=ref)
        assert np.array_equal(second[z], ref2), z


@pytest.mark.parametrize("act", [0, 1, 3])
def test_fast_mfma_fused_linear(act):
    """linear_forward and fused_linear_forward (bias + activation in the
    epilogue) at an MFMA shape: pre-activations equal the unfused product
    plus bias, bit-exact vs the checker; outputs equal the activation kernel
    applied to them."""
    e = ext()
    M, N, K = 2050, 2049, 300
    x = rl.gen_normal((M, K), seed=3)
    w = rl.gen_normal((N, K), seed=4, std=0.2)
    b = rl.gen_normal(N, seed=5)
    out, pre = e.fused_linear_forward(T(x), T(w), T(b), act, iters=24, mode=0, return_pre=True)
    lin = e.linear_forward(T(x), T(w), T(b), iters=24, mode=0)
    assert torch.equal(pre, lin)
    if act == 3:
        assert torch.equal(out, e.silu(lin, 24))
    elif act == 1:
        assert torch.equal(out, e.relu(lin))
    else:
        assert torch.equal(out, lin)
    ref = rl.orc_matmul(x, w, M, N, K, 24, 0, tb=1) + b[None, :]
    assert np.array_equal(H(pre), ref.astype(np.float32))


@pytest.mark.parametrize("causal", [True, False])
def test_fast_attention_config5_mfma_products(causal):
    """The config-5 attention core in FAST mode: each 512-row chunk's P V
    (32 heads of 512 x 128, 128 blocks, the causal K limit per row tile)
    runs on the matrix cores; the output equals the one-chunk form (P V on
    the VALU tiles) and the checker's composition on sampled heads, bit for
    bit."""
    e = ext()
    shape = (1, 32, 2048, 128)
    q = rl.gen_normal(shape, seed=700)
    k = rl.gen_normal(shape, seed=701)
    v = rl.gen_normal(shape, seed=702)
    got = H(e.attention(T(q), T(k), T(v), None, causal, iters=24, mode=0))
    one, _ = e.attention(T(q), T(k), T(v), None, causal, iters=24, mode=0, return_probs=True)
    assert np.array_equal(got, H(one))
    for h in (0, 17):
        sl = (slice(0, 1), slice(h, h + 1))
        assert np.array_equal(got[sl], rl.orc_attention_lanes(q[sl], k[sl], v[sl], None, causal, 24, 0)), h


@pytest.mark.parametrize("Z,M,N,K", [(32, 512, 128, 600), (1, 1024, 1024, 1030), (8, 512, 512, 512)])
def test_fast_mfma_few_blocks(Z, M, N, K):
    """Launches of 64-128 blocks of 128 x 128 (fewer than the CUs) on the
    matrix cores: bit-exact vs the checker."""
    e = ext()
    A = rl.gen_uniform((Z, M, K), seed=Z + M)
    B = rl.gen_uniform((Z, K, N), seed=N + K)
    got = H(e.bmm(T(A), T(B), iters=24, mode=0))
    for z in range(Z):
        ref = rl.orc_matmul(np.ascontiguousarray(A[z]), np.ascontiguousarray(B[z]), M, N, K, 24, 0)
        assert np.array_equal(got[z], ref), z


def _attention_ws(q, k, v, mask, causal, chunk_rows):
    """rac_attention_ws_dev in FAST mode (iters 24) with a NaN-filled
    workspace of `chunk_rows` query rows per chunk: a chunk that read scores
    it had not written would show."""
    L = lib()
    B, Hh, Tn, D = q.shape
    qt, kt, vt = T(q), T(k), T(v)
    mt = T(mask) if mask is not None else None
    out = torch.empty_like(qt)
    nbytes = 4 * B * Hh * chunk_rows * Tn + 256
    ws = torch.full((nbytes // 4,), float("nan"), device=DEV)
    rc = L.rac_attention_ws_dev(qt.data_ptr(), kt.data_ptr(), vt.data_ptr(), mt.data_ptr() if mt is not None else None,
                                int(causal), out.data_ptr(), B, Hh, Tn, D, ws.data_ptr(), nbytes, 24, 0,
                                torch.cuda.current_stream().cuda_stream)
    assert rc == 0, L.rac_last_error()
    return H(out)


def test_fast_attention_chunks_mfma():
    """[1, 16, 512, 128] in FAST mode: the causal scores of each chunk of
    query rows (the trapezoid of 128 x 128 tiles on or below the diagonal)
    and P V run on the matrix cores for chunks of 64 rows and more; every
    chunk size gives the one-chunk bits, which equal the checker's."""
    e = ext()
    shape = (1, 16, 512, 128)
    q = rl.gen_normal(shape, seed=720)
    k = rl.gen_normal(shape, seed=721)
    v = rl.gen_normal(shape, seed=722)
    mask = (rl.gen_normal((512, 512), seed=723) * np.float32(0.5)).astype(np.float32)
    for mk, causal in ((None, True), (mask, True), (mask, False)):
        print(f"fast attention chunks mask={mk is not None} causal={causal}", flush=True)
        ref, _ = e.attention(T(q), T(k), T(v), T(mk) if mk is not None else None, causal, iters=24, mode=0,
                             return_probs=True)
        ref = H(ref)
        for rows in (7, 64, 130, 256, 512):
            got = _attention_ws(q, k, v, mk, causal, rows)
            assert np.array_equal(got, ref, equal_nan=True), (rows, mk is not None, causal)
        for h in (0, 15):
            sl = (slice(0, 1), slice(h, h + 1))
            assert np.array_equal(ref[sl], rl.orc_attention_lanes(q[sl], k[sl], v[sl], mk, causal, 24, 0)), h


@pytest.mark.parametrize("act", [0, 3])
def test_fast_mfma_linear_backward(act):
    """The FAST training products at MFMA sizes: fused_linear_backward's
    grad_input (d W, NN) and grad_weight (d^T x, TN) bit-exact vs the
    checker, d = the activation gradient of the saved pre-activations."""
    e = ext()
    M, N, K = 1024, 2304, 1030         # 144 / 72 / 162 blocks of 128 x 128
    x = rl.gen_normal((M, K), seed=31)
    w = rl.gen_normal((N, K), seed=32, std=0.05)
    b = rl.gen_normal(N, seed=33)
    g = rl.gen_normal((M, N), seed=34)
    _, pre = e.fused_linear_forward(T(x), T(w), T(b), act, iters=24, mode=0, return_pre=True)
    d = H(e.act_grad(T(g), pre, act, iters=24)) if act else g
    gi, gw, gb = e.fused_linear_backward(T(g), T(x), T(w), T(b), pre, act, True, iters=24, mode=0)
    assert np.array_equal(H(gi), rl.orc_matmul(d, w, M, K, N, 24, 0))
    assert np.array_equal(H(gw), rl.orc_matmul(d, x, N, K, M, 24, 0, ta=1))
    assert np.allclose(H(gb), d.astype(np.float64).sum(0), rtol=1e-5, atol=1e-5)
