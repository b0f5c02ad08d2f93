"""Randomized parity sweep: the HIP library against the CPU checker on random
shapes, layouts, MAC modes, step counts and special values (NaN, +-inf,
signed zeros, subnormals, tiny and huge operands), with fixed seeds and a
fixed number of cases per operation.

Each case is bit-exact with the checker (NaN matched by position), except the
Q8_0 GEMV's GELU and SiLU epilogues, which use the device's erff / expf
(within 1e-6 relative, as in test_gpu_q8.py).  The case generators draw:
- matmul: M, N, K in [1, 300), all four layouts, FAST / CORDIC / SHIFTADD,
  step counts 1..24, alpha and beta (with C accumulated), skinny shapes, and
  in CORDIC mode A operands outside the strength-reduced chain's range;
- batched matmul: 1..5 items with transposes and beta;
- softmax: 1..40 rows of 1..20000 columns (multiples of 4 and not), scales up
  to 60, special values, zero-maximum rows with signed zeros;
- softmax over enough rows for the persistent kernel (n <= 8);
- the masked attention softmax (causal, additive masks with -inf);
- RMSNorm and LayerNorm with and without gamma / beta;
- exp, SiLU, sigmoid and tanh on odd lengths and unaligned offsets;
- RoPE on random [B, H, T, D];
- the Q8_0 GEMV with 1..8 input rows, every activation, with and without
  bias;
- the attention core (three MAC modes, masks, causal, scaled inputs);
- the fused linear (bias, the four activations, every MAC mode), whose
  GELU is bounded as in test_gpu_fused_linear.py;
- matmul_backward (each need_grad combination) and linear_backward, the
  bias gradient (torch's column sum, as the reference takes it) within
  1e-5 of the float64 sum;
- the synchronous rac.h entry points on host buffers (matmul, batched
  softmax, RMSNorm, LayerNorm, SiLU, RoPE) in a random sequence of sizes,
  which grows and reuses the cached staging buffers;
- RoPE on [B, T, H, D] storage (strided views, in place and out of place),
  the RoPE table with random bases, sin/cos and rsqrt, the exact vector
  primitives, attention returning its probabilities;
- matmuls up to 2048^3 (sampled entries, tile and matrix edges included),
  rows of 16385..120000 columns (the loop kernels) and Q8_0 GEMVs of up to
  60 M weights;
- the RAC-DSP engine (every op, wide operand ranges) and its systolic
  product, bit-exact (integer).
"""
import numpy as np
import pytest

import raclib as rl

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda"
SPECIAL = np.array([0.0, -0.0, np.nan, np.inf, -np.inf, 1e-40, -1e-40, 1e-33, 3e38, -3e38, 1e-38,
                    2.0 ** -110], np.float32)


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


def sprinkle(rng, a, frac):
    n = max(1, int(a.size * frac))
    a.reshape(-1)[rng.integers(0, a.size, n)] = rng.choice(SPECIAL, n)
    return a


def same(got, ref):
    return np.array_equal(got, ref, equal_nan=True)


def case_gemm(rng, seed):
    skinny = rng.random() < 0.3
    M = int(rng.integers(1, 17)) if skinny and rng.random() < 0.5 else int(rng.integers(1, 300))
    N = int(rng.integers(1, 17)) if skinny and M > 16 else int(rng.integers(1, 300))
    K = int(rng.integers(1, 300))
    ta, tb = int(rng.integers(0, 2)), int(rng.integers(0, 2))
    mode = int(rng.integers(0, 3))
    iters = int(rng.choice([1, 5, 8, 16, 24, int(rng.integers(1, 25))]))
    alpha = float(np.float32(rng.choice([1.0, rng.normal()])))
    beta = float(np.float32(rng.choice([0.0, 0.0, rng.normal()])))
    A = rng.uniform(-2, 2, (K, M) if ta else (M, K)).astype(np.float32)
    B = rng.uniform(-2, 2, (N, K) if tb else (K, N)).astype(np.float32)
    if mode == 1 and rng.random() < 0.2:
        sprinkle(rng, A, 0.01)
    C0 = rng.normal(size=(M, N)).astype(np.float32)
    print(f"matmul seed={seed} M={M} N={N} K={K} ta={ta} tb={tb} mode={mode} n={iters}", flush=True)
    Ad, Bd, Cd = T(A), T(B), T(C0)
    rc = lib().rac_gemm_dev(Ad.data_ptr(), Bd.data_ptr(), Cd.data_ptr(), M, N, K, ta, tb, alpha, beta, iters,
                            mode, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib().rac_last_error()
    assert same(H(Cd), rl.orc_matmul(A, B, M, N, K, iters, mode, ta, tb, alpha, beta, C0)), seed


def case_gemm_fewrow_wide(rng, seed):
    """Few rows (or columns) on grids of up to one workgroup per CU and
    wider: the 512-lane CORDIC pipeline (16, 64 and 128 outputs per
    workgroup), FAST's 8-wide blocks, full and ragged K-tiles, and the
    literal chain on sprinkled special values."""
    cols = rng.random() < 0.3
    small = int(rng.choice([1, 1, 2, 4, int(rng.integers(5, 9)), int(rng.integers(9, 17))]))
    big = int(rng.integers(256, 4200))
    M, N = (big, small) if cols else (small, big)
    K = int(rng.choice([int(rng.integers(1, 1100)), 256 * int(rng.integers(1, 5))]))
    K = max(1, min(K, int(1.5e7) // (small * big)))
    mode = int(rng.choice([0, 1, 1, 2])) if small * big * K <= 3_000_000 else int(rng.choice([0, 1, 1]))
    iters = int(rng.choice([8, 16, 24, int(rng.integers(1, 25))]))
    tb = int(rng.integers(0, 2))
    alpha = float(np.float32(rng.choice([1.0, rng.normal()])))
    beta = float(np.float32(rng.choice([0.0, 0.0, rng.normal()])))
    A = rng.uniform(-2, 2, (M, K)).astype(np.float32)
    B = rng.uniform(-2, 2, (N, K) if tb else (K, N)).astype(np.float32)
    if mode == 1 and rng.random() < 0.3:
        sprinkle(rng, A, 0.01)
    C0 = rng.normal(size=(M, N)).astype(np.float32)
    print(f"matmul few-row wide seed={seed} M={M} N={N} K={K} tb={tb} mode={mode} n={iters}", flush=True)
    Ad, Bd, Cd = T(A), T(B), T(C0)
    rc = lib().rac_gemm_dev(Ad.data_ptr(), Bd.data_ptr(), Cd.data_ptr(), M, N, K, 0, tb, alpha, beta, iters,
                            mode, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib().rac_last_error()
    assert same(H(Cd), rl.orc_matmul(A, B, M, N, K, iters, mode, 0, tb, alpha, beta, C0)), seed


def case_bmm(rng, seed):
    Z = int(rng.integers(1, 6))
    M, N, K = (int(rng.integers(1, 150)) for _ in range(3))
    ta, tb = bool(rng.integers(0, 2)), bool(rng.integers(0, 2))
    mode = int(rng.integers(0, 3))
    iters = int(rng.choice([8, 16, 24, int(rng.integers(1, 25))]))
    alpha = float(np.float32(rng.normal()))
    beta = float(np.float32(rng.choice([0.0, rng.normal()])))
    A = rng.normal(size=(Z, K, M) if ta else (Z, M, K)).astype(np.float32)
    B = rng.normal(size=(Z, N, K) if tb else (Z, K, N)).astype(np.float32)
    C0 = rng.normal(size=(Z, M, N)).astype(np.float32)
    print(f"bmm seed={seed} Z={Z} M={M} N={N} K={K} ta={ta} tb={tb} mode={mode} n={iters}", flush=True)
    out = T(C0)
    ext().bmm(T(A), T(B), ta, tb, alpha, iters, mode, out=out, beta=beta)
    got = H(out)
    for z in range(Z):
        assert same(got[z], rl.orc_matmul(A[z], B[z], M, N, K, iters, mode, int(ta), int(tb), alpha, beta,
                                          C0[z])), (seed, z)


def case_softmax(rng, seed):
    rows = int(rng.integers(1, 40))
    cols = int(rng.choice([4096, 1024, 2048, 8192, 16384, int(rng.integers(1, 20000)),
                           int(rng.integers(1, 300)) * 4]))
    iters = int(rng.choice([8, 16, 24, int(rng.integers(1, 25))]))
    x = (rng.normal(size=(rows, cols)) * float(rng.choice([0.5, 2.0, 10.0, 60.0]))).astype(np.float32)
    if rng.random() < 0.3:
        sprinkle(rng, x, 0.001)
    if rng.random() < 0.2:
        x[0] = -np.abs(x[0])
        x[0, int(rng.integers(0, cols))] = rng.choice([0.0, -0.0])
    print(f"softmax seed={seed} rows={rows} cols={cols} n={iters}", flush=True)
    assert same(H(ext().softmax(T(x), iters=iters)), rl.orc_softmax_lanes(x, iters)), seed


def case_softmax_persistent(rng, seed):
    rows = int(rng.choice([3072, 4000, 5000]))
    cols = int(rng.choice([1024, 2048, 4096]))
    iters = int(rng.choice([8, 5, 1]))
    x = (rng.normal(size=(rows, cols)) * 2).astype(np.float32)
    if rng.random() < 0.5:
        sprinkle(rng, x, 0.0001)
    print(f"softmax persistent seed={seed} rows={rows} cols={cols} n={iters}", flush=True)
    assert same(H(ext().softmax(T(x), iters=iters)), rl.orc_softmax_lanes(x, iters)), seed


def case_masked(rng, seed):
    Tn, Zb = int(rng.integers(1, 300)), int(rng.integers(1, 4))
    iters = int(rng.choice([8, 16, 24, int(rng.integers(1, 25))]))
    causal, use_mask = bool(rng.integers(0, 2)), bool(rng.integers(0, 2))
    x = (rng.normal(size=(Zb, Tn, Tn)) * 3).astype(np.float32)
    mask = None
    if use_mask:
        mask = rng.normal(size=(Tn, Tn)).astype(np.float32)
        if rng.random() < 0.5:
            mask[rng.random((Tn, Tn)) < 0.3] = -np.inf
    print(f"masked softmax seed={seed} T={Tn} Z={Zb} causal={causal} mask={use_mask} n={iters}", flush=True)
    xd = T(x)
    ext().softmax_masked_(xd, T(mask) if mask is not None else None, causal, iters)
    ref = rl.orc_softmax_lanes(x.reshape(-1, Tn), iters, causal=causal, mask=mask, zero_guard=True)
    assert same(H(xd), ref.reshape(x.shape)), seed


def case_norms(rng, seed):
    rows = int(rng.integers(1, 30))
    d = int(rng.choice([4096, 1024, 11008, int(rng.integers(1, 20000)), int(rng.integers(1, 500)) * 4]))
    x = (rng.normal(size=(rows, d)) * float(rng.choice([1.0, 1e-3, 1e3]))).astype(np.float32)
    if rng.random() < 0.2:
        sprinkle(rng, x, 0.001)
    g = rng.normal(1, 0.02, d).astype(np.float32) if rng.random() < 0.8 else None
    b = rng.normal(0, 0.1, d).astype(np.float32) if rng.random() < 0.8 else None
    eps = float(np.float32(rng.choice([1e-6, 1e-5])))
    print(f"norms seed={seed} rows={rows} d={d} gamma={g is not None} beta={b is not None}", flush=True)
    e = ext()
    assert same(H(e.rmsnorm(T(x), T(g) if g is not None else None, eps)), rl.orc_rmsnorm_lanes(x, g, eps)), seed
    got = H(e.layernorm(T(x), T(g) if g is not None else None, T(b) if b is not None else None, eps))
    assert same(got, rl.orc_layernorm_lanes(x, g, b, eps)), seed


def case_activations(rng, seed):
    n = int(rng.choice([int(rng.integers(1, 5000)), int(rng.integers(1, 300000))]))
    off = int(rng.integers(0, 4))
    iters = int(rng.choice([8, 16, 24, int(rng.integers(1, 25))]))
    x = (rng.normal(size=n + off) * float(rng.choice([1.0, 4.0, 30.0]))).astype(np.float32)
    if rng.random() < 0.5:
        sprinkle(rng, x, 0.01)
    print(f"activations seed={seed} n={n} offset={off} n_iters={iters}", flush=True)
    xd = T(x)[off:]
    for name, oname in (("exp", "orc_exp_batch"), ("silu", "orc_silu"), ("sigmoid", "orc_sigmoid"),
                        ("tanh", "orc_tanh")):
        assert same(H(getattr(ext(), name)(xd, iters=iters)), rl.orc_unary(oname, x[off:], iters)), (seed, name)


def case_rope(rng, seed):
    B, Hh, Tt = int(rng.integers(1, 4)), int(rng.integers(1, 6)), int(rng.integers(1, 300))
    D = 2 * int(rng.integers(1, 96))
    x = rng.normal(size=(B, Hh, Tt, D)).astype(np.float32)
    print(f"rope seed={seed} B={B} H={Hh} T={Tt} D={D}", flush=True)
    c, s = rl.orc_rope_cache(Tt, D)
    xd = T(x)
    ext().rope_apply_(xd, T(c), T(s))
    assert same(H(xd), rl.orc_rope_apply(x, c, s)), seed


def case_q8(rng, seed):
    M, N = int(rng.integers(1, 17)), int(rng.integers(1, 3000))
    K = 32 * int(rng.choice([int(rng.integers(1, 300)), 8 * int(rng.integers(1, 40))]))
    act = int(rng.integers(0, 4))
    wq = rl.orc_q8_quantize(rng.normal(size=(N, K)).astype(np.float32))
    x = rng.normal(size=(M, K)).astype(np.float32)
    bias = rng.normal(size=N).astype(np.float32) if rng.random() < 0.5 else None
    print(f"q8 gemv seed={seed} M={M} N={N} K={K} act={act} bias={bias is not None}", flush=True)
    got = H(ext().q8_gemv(T(x), T(wq), T(bias) if bias is not None else None, act))
    ref = rl.orc_q8_gemv(x, wq, bias, act)
    if act in (0, 1):
        assert same(got, ref), seed
    else:
        assert np.all(np.abs(got - ref) <= 1e-6 * (np.abs(ref) + 1.0)), seed


def case_attention(rng, seed):
    B, Hh, Tn = int(rng.integers(1, 3)), int(rng.integers(1, 4)), int(rng.integers(1, 200))
    D = int(rng.choice([16, 32, 64, 128, int(rng.integers(1, 129))]))
    causal = bool(rng.integers(0, 2))
    iters, mode = int(rng.choice([8, 16, 24])), int(rng.integers(0, 3))
    scale = float(rng.choice([1.0, 4.0]))
    q, k, v = ((rng.normal(size=(B, Hh, Tn, D)) * scale).astype(np.float32) for _ in range(3))
    mask = rng.normal(size=(Tn, Tn)).astype(np.float32) if rng.random() < 0.3 else None
    print(f"attention seed={seed} B={B} H={Hh} T={Tn} D={D} causal={causal} mask={mask is not None} n={iters} "
          f"mode={mode} scale={scale}", flush=True)
    got = H(ext().attention(T(q), T(k), T(v), T(mask) if mask is not None else None, causal, iters, mode))
    assert same(got, rl.orc_attention_lanes(q, k, v, mask, causal, iters, mode)), seed


def _act_ref(x, act, iters):
    if act == 0:
        return x
    if act == 1:
        return np.where(x > 0, x, np.float32(0)).astype(np.float32)
    if act == 2:
        return rl.orc_unary("orc_gelu", x)
    return rl.orc_unary("orc_silu", x, iters)


def case_fused_linear(rng, seed):
    M, N, K = int(rng.integers(1, 200)), int(rng.integers(1, 200)), int(rng.integers(1, 200))
    act, mode = int(rng.integers(0, 4)), int(rng.integers(0, 3))
    iters = int(rng.choice([8, 16, 24, int(rng.integers(1, 25))]))
    x = rng.normal(size=(M, K)).astype(np.float32)
    w = (rng.normal(size=(N, K)) * 0.2).astype(np.float32)
    b = rng.normal(size=N).astype(np.float32) if rng.random() < 0.6 else np.zeros(0, np.float32)
    print(f"fused linear seed={seed} M={M} N={N} K={K} act={act} mode={mode} n={iters} bias={b.size > 0}",
          flush=True)
    out, pre = ext().fused_linear_forward(T(x), T(w), T(b), act, iters=iters, mode=mode, return_pre=True)
    out, pre = H(out), H(pre)
    ref_pre = rl.orc_matmul(x, w, M, N, K, iters, mode, tb=1)
    if b.size:
        ref_pre = (ref_pre + b[None, :]).astype(np.float32)
    assert same(pre, ref_pre), seed
    ref = _act_ref(ref_pre, act, iters)
    if act == 2:
        # device erff against glibc's (as test_gpu_fused_linear.py bounds it)
        assert np.all(np.abs(out - ref) <= 2e-6 * np.abs(ref) + 2.4e-7 * np.abs(ref_pre) + 1e-7), seed
    else:
        assert same(out, ref), seed


def case_rac_h(rng, seed):
    """The synchronous rac.h entry points on host buffers, in a random
    sequence of sizes (the staging buffers are cached, grown and reused)."""
    L = lib()
    op = str(rng.choice(["matmul", "softmax", "rmsnorm", "layernorm", "silu", "rope"]))
    iters = int(rng.choice([8, 16, 24, int(rng.integers(1, 25))]))
    L.rac_set_cordic_iters(iters)
    L.rac_clear_error()
    if op == "matmul":
        M, N, K = (int(rng.integers(1, 256)) for _ in range(3))
        mode = int(rng.integers(0, 3))
        L.rac_set_cordic_mode(mode)
        A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
        B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
        C = np.zeros((M, N), np.float32)
        print(f"rac.h matmul seed={seed} M={M} N={N} K={K} mode={mode} n={iters}", flush=True)
        L.rac_matmul(rl.p(A), rl.p(B), rl.p(C), M, N, K)
        ref = rl.orc_matmul(A, B, M, N, K, iters, mode)
    elif op == "softmax":
        rows, n = int(rng.integers(1, 64)), int(rng.integers(1, 5000))
        x = (rng.normal(size=(rows, n)) * 2).astype(np.float32)
        C = np.zeros_like(x)
        print(f"rac.h softmax_batch seed={seed} rows={rows} n={n} iters={iters}", flush=True)
        L.rac_softmax_batch(rl.p(x), rl.p(C), rows, n)
        ref = rl.orc_softmax_lanes(x, iters)
    elif op in ("rmsnorm", "layernorm"):
        rows, d = int(rng.integers(1, 32)), int(rng.integers(1, 6000))
        x = rng.normal(size=(rows, d)).astype(np.float32)
        g = rng.normal(1, 0.02, d).astype(np.float32) if rng.random() < 0.7 else None
        bt = rng.normal(0, 0.1, d).astype(np.float32) if rng.random() < 0.7 else None
        C = np.zeros_like(x)
        print(f"rac.h {op} seed={seed} rows={rows} d={d}", flush=True)
        gp = rl.p(g) if g is not None else None
        if op == "rmsnorm":
            L.rac_rmsnorm(rl.p(x), rl.p(C), gp, 1e-6, rows, d)
            ref = rl.orc_rmsnorm_lanes(x, g, np.float32(1e-6))
        else:
            L.rac_layernorm(rl.p(x), rl.p(C), gp, rl.p(bt) if bt is not None else None, 1e-5, rows, d)
            ref = rl.orc_layernorm_lanes(x, g, bt, np.float32(1e-5))
    elif op == "silu":
        n = int(rng.integers(1, 200000))
        x = (rng.normal(size=n) * 4).astype(np.float32)
        C = np.zeros_like(x)
        print(f"rac.h silu seed={seed} n={n} iters={iters}", flush=True)
        L.rac_silu(rl.p(x), rl.p(C), n)
        ref = rl.orc_unary("orc_silu", x, iters)
    else:
        B, Hh, Tt, D = int(rng.integers(1, 3)), int(rng.integers(1, 5)), int(rng.integers(1, 130)), \
            2 * int(rng.integers(1, 64))
        C = rng.normal(size=(B, Hh, Tt, D)).astype(np.float32)
        c, s = rl.orc_rope_cache(Tt, D)
        ref = rl.orc_rope_apply(C, c, s)
        print(f"rac.h rope_apply seed={seed} B={B} H={Hh} T={Tt} D={D}", flush=True)
        L.rac_rope_apply(rl.p(C), rl.p(c), rl.p(s), B, Hh, Tt, D)
    assert L.rac_last_error() == b"", (seed, L.rac_last_error())
    assert same(C, ref), (seed, op)


def case_backward(rng, seed):
    M, N, K = int(rng.integers(1, 200)), int(rng.integers(1, 200)), int(rng.integers(1, 200))
    mode = int(rng.integers(0, 3))
    iters = int(rng.choice([8, 16, 24, int(rng.integers(1, 25))]))
    need_a, need_b = bool(rng.integers(0, 2)), bool(rng.integers(0, 2))
    A = rng.normal(size=(M, K)).astype(np.float32)
    B = rng.normal(size=(K, N)).astype(np.float32)
    G = rng.normal(size=(M, N)).astype(np.float32)
    print(f"backward seed={seed} M={M} N={N} K={K} mode={mode} n={iters} need=({need_a},{need_b})", flush=True)
    e = ext()
    gA, gB = e.matmul_backward(T(G), T(A), T(B), need_a, need_b, iters=iters, mode=mode)
    assert (gA is None) != need_a and (gB is None) != need_b, seed
    if need_a:
        assert same(H(gA), rl.orc_matmul(G, B, M, K, N, iters, mode, tb=1)), seed
    if need_b:
        assert same(H(gB), rl.orc_matmul(A, G, K, N, M, iters, mode, ta=1)), seed
    # linear: input [M, K], weight [N, K], grad_output [M, N]
    W = rng.normal(size=(N, K)).astype(np.float32)
    gi, gw, gb = e.linear_backward(T(G), T(A), T(W), True, iters=iters, mode=mode)
    assert same(H(gi), rl.orc_matmul(G, W, M, K, N, iters, mode)), seed
    assert same(H(gw), rl.orc_matmul(G, A, N, K, M, iters, mode, ta=1)), seed
    # the bias gradient is torch's column sum, as in the reference
    ref_b = G.astype(np.float64).sum(0)
    assert np.all(np.abs(H(gb) - ref_b) <= 1e-5 * np.abs(G).sum(0) + 1e-7), seed


def case_rope_strided(rng, seed):
    B, Hh, Tt = int(rng.integers(1, 4)), int(rng.integers(1, 9)), int(rng.integers(1, 400))
    D = 2 * int(rng.integers(1, 80))
    x = rng.normal(size=(B, Hh, Tt, D)).astype(np.float32)
    print(f"rope strided seed={seed} B={B} H={Hh} T={Tt} D={D}", flush=True)
    c, s = rl.orc_rope_cache(Tt, D)
    ref = rl.orc_rope_apply(x, c, s)
    view = T(np.ascontiguousarray(x.transpose(0, 2, 1, 3))).transpose(1, 2)     # [B, T, H, D] storage
    assert same(H(ext().rope_apply(view, T(c), T(s))), ref), seed
    ext().rope_apply_(view, T(c), T(s))
    assert same(H(view), ref), seed


def case_rope_cache(rng, seed):
    ms, hd = int(rng.integers(1, 5000)), 2 * int(rng.integers(1, 100))
    base = float(rng.choice([10000.0, 500000.0, 1e4 * rng.random() + 1.5]))
    print(f"rope cache seed={seed} max_seq={ms} head_dim={hd} base={base}", flush=True)
    c, s = ext().rope_cache(ms, hd, base, device=DEV)
    rc, rs = rl.orc_rope_cache(ms, hd, base)
    assert same(H(c), rc) and same(H(s), rs), seed


def case_sincos_rsqrt(rng, seed):
    n = int(rng.integers(1, 200000))
    th = (rng.uniform(-1, 1, n) * float(rng.choice([3.2, 100.0, 16000.0]))).astype(np.float32)
    print(f"sincos / rsqrt seed={seed} n={n}", flush=True)
    s, c = ext().sincos(T(th))
    so, co = np.zeros_like(th), np.zeros_like(th)
    rl.oracle().orc_sincos_batch(rl.p(th), rl.p(so), rl.p(co), th.size)
    assert same(H(s), so) and same(H(c), co), seed
    x = (np.abs(rng.normal(size=n)) * float(rng.choice([1e-30, 1.0, 1e30]))).astype(np.float32)
    ro = np.zeros_like(x)
    rl.oracle().orc_rsqrt_batch(rl.p(x), rl.p(ro), x.size)
    assert same(H(ext().rsqrt(T(x))), ro), seed


def case_prims(rng, seed):
    n = int(rng.integers(1, 50000))
    name = str(rng.choice(["rotate", "rotate_raw", "polar", "complex_mul", "rotate_n"]))
    a = rng.uniform(-50, 50, (n, 2)).astype(np.float32)
    b = rng.uniform(-50, 50, (n, 2)).astype(np.float32)
    th = rng.uniform(-3000, 3000, n).astype(np.float32)
    _, _, nb, nt = rl.PRIM_OPS[name]
    iarg = int(rng.integers(1, 31)) if name == "rotate_n" else 0
    print(f"vector primitive {name} seed={seed} n={n} iters={iarg}", flush=True)
    op = {"rotate_n": "rotate_precision"}.get(name, name)
    got = H(ext().vec2(op, T(a), T(b) if nb else None, T(th) if nt else None, iarg))
    assert same(got, rl.orc_prim(name, a, b if nb else None, th if nt else None, iarg)), seed


def case_attention_probs(rng, seed):
    B, Hh, Tn = int(rng.integers(1, 3)), int(rng.integers(1, 4)), int(rng.integers(1, 160))
    D = int(rng.choice([8, 32, 64, int(rng.integers(1, 100))]))
    causal, iters, mode = bool(rng.integers(0, 2)), int(rng.choice([8, 16, 24])), int(rng.integers(0, 3))
    q, k, v = (rng.normal(size=(B, Hh, Tn, D)).astype(np.float32) for _ in range(3))
    mask = rng.normal(size=(Tn, Tn)).astype(np.float32) if rng.random() < 0.3 else None
    print(f"attention with probabilities seed={seed} B={B} H={Hh} T={Tn} D={D} causal={causal} n={iters} "
          f"mode={mode}", flush=True)
    out, P = ext().attention(T(q), T(k), T(v), T(mask) if mask is not None else None, causal, iters, mode,
                             return_probs=True)
    assert same(H(out), rl.orc_attention_lanes(q, k, v, mask, causal, iters, mode)), seed
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    b, h = int(rng.integers(0, B)), int(rng.integers(0, Hh))
    sc = rl.orc_matmul(q[b, h], k[b, h], Tn, Tn, D, iters, mode, tb=1, alpha=scale)
    assert same(H(P)[b, h], rl.orc_softmax_lanes(sc, iters, causal=causal, mask=mask, zero_guard=True)), seed


def case_big_matmul(rng, seed):
    M, N, K = (int(rng.integers(256, 2049)) for _ in range(3))
    ta, tb = int(rng.integers(0, 2)), int(rng.integers(0, 2))
    mode, iters = int(rng.integers(0, 3)), int(rng.choice([8, 16, 24, 13]))
    A = rng.uniform(-1, 1, (K, M) if ta else (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (N, K) if tb else (K, N)).astype(np.float32)
    print(f"large matmul seed={seed} M={M} N={N} K={K} ta={ta} tb={tb} mode={mode} n={iters}", flush=True)
    Ad, Bd, Cd = T(A), T(B), torch.zeros((M, N), device=DEV)
    rc = lib().rac_gemm_dev(Ad.data_ptr(), Bd.data_ptr(), Cd.data_ptr(), M, N, K, ta, tb, 1.0, 0.0, iters, mode,
                            torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib().rac_last_error()
    rows = rng.integers(0, M, 400).astype(np.int32)
    cols = rng.integers(0, N, 400).astype(np.int32)
    rows[:8] = [0, M - 1, 63, 64, 127, 128, M // 2, M - 2]            # tile and matrix edges
    cols[:8] = [0, N - 1, 63, 64, 127, 128, N // 2, N - 2]
    assert same(H(Cd)[rows, cols], rl.orc_matmul_entries(A, B, M, N, K, iters, mode, rows, cols, ta, tb)), seed


def case_long_rows(rng, seed):
    rows, cols = int(rng.integers(1, 6)), int(rng.integers(16385, 120000))
    iters = int(rng.choice([8, 16, 24, int(rng.integers(1, 25))]))
    x = (rng.normal(size=(rows, cols)) * 3).astype(np.float32)
    g = rng.normal(1, 0.02, cols).astype(np.float32)
    b = rng.normal(0, 0.1, cols).astype(np.float32)
    print(f"long rows seed={seed} rows={rows} cols={cols} n={iters}", flush=True)
    e = ext()
    assert same(H(e.softmax(T(x), iters=iters)), rl.orc_softmax_lanes(x, iters)), seed
    assert same(H(e.rmsnorm(T(x), T(g), 1e-6)), rl.orc_rmsnorm_lanes(x, g, np.float32(1e-6))), seed
    assert same(H(e.layernorm(T(x), T(g), T(b), 1e-5)), rl.orc_layernorm_lanes(x, g, b, np.float32(1e-5))), seed


def case_big_q8(rng, seed):
    K = int(rng.choice([2048, 4096, 5632, 8192, 11008]))
    N = min(int(rng.integers(3000, 40000)), 60_000_000 // K)
    act = int(rng.integers(0, 2))
    wq = rl.orc_q8_quantize(rng.standard_normal((N, K), dtype=np.float32))
    x = rng.normal(size=(1, K)).astype(np.float32)
    print(f"large q8 gemv seed={seed} N={N} K={K} act={act}", flush=True)
    assert same(H(ext().q8_gemv(T(x), T(wq), None, act)), rl.orc_q8_gemv(x, wq, None, act)), seed


def case_dsp(rng, seed):
    n = int(rng.integers(1, 100000))
    op = int(rng.choice([0, 1, 2, 3, 6]))
    span = int(rng.choice([20, 40, 62]))
    x = rng.integers(-2 ** span, 2 ** span, n, dtype=np.int64)
    y = rng.integers(-2 ** span, 2 ** span, n, dtype=np.int64)
    z = rng.integers(-2 ** 63, 2 ** 63 - 1, n, dtype=np.int64)
    print(f"rac-dsp eval seed={seed} op={op} n={n} span=2^{span}", flush=True)
    got = ext().dsp_eval(op, T(x), T(z), T(y))
    for a, b in zip(got, rl.orc_dsp_batch(op, x, y, z)):
        assert np.array_equal(H(a), b), seed
    N, K = int(rng.integers(1, 200)), int(rng.integers(1, 300))
    W = rng.integers(-2 ** 63, 2 ** 63 - 1, (N, N), dtype=np.int64)
    X = rng.integers(-2 ** 40, 2 ** 40, (K, N), dtype=np.int64)
    ref = np.zeros((K, N), np.int64)
    rl.oracle().orc_dsp_systolic(N, K, rl.p(W), rl.p(X), rl.p(ref))
    print(f"rac-dsp systolic seed={seed} N={N} K={K}", flush=True)
    assert np.array_equal(H(ext().dsp_systolic(T(W), T(X))), ref), seed


CASES = {
    "matmul": (case_gemm, 300), "bmm": (case_bmm, 200), "softmax": (case_softmax, 200),
    "softmax_persistent": (case_softmax_persistent, 16), "masked_softmax": (case_masked, 300),
    "norms": (case_norms, 300), "activations": (case_activations, 120), "rope": (case_rope, 300),
    "q8_gemv": (case_q8, 40), "attention": (case_attention, 200),
    "fused_linear": (case_fused_linear, 150), "rac_h_host_buffers": (case_rac_h, 200),
    "backward": (case_backward, 150), "rope_strided": (case_rope_strided, 100),
    "rope_cache": (case_rope_cache, 100), "sincos_rsqrt": (case_sincos_rsqrt, 60), "prims": (case_prims, 100),
    "attention_probs": (case_attention_probs, 100), "large_matmul": (case_big_matmul, 12),
    "long_rows": (case_long_rows, 12), "large_q8_gemv": (case_big_q8, 3), "rac_dsp": (case_dsp, 60),
    "fewrow_wide_matmul": (case_gemm_fewrow_wide, 60),
}


@pytest.mark.parametrize("op", list(CASES))
def test_random_parity(op):
    fn, n = CASES[op]
    base = 7919 * (list(CASES).index(op) + 1)
    L = lib()
    iters, mode = L.rac_get_cordic_iters(), L.rac_get_cordic_mode()
    try:
        for i in range(n):
            seed = base + i
            fn(np.random.default_rng(seed), seed)
    finally:
        # the rac.h cases set the process-wide knobs
        L.rac_set_cordic_iters(iters)
        L.rac_set_cordic_mode(mode)
