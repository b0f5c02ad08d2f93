"""Benchmark config 5 at its real size: RACLlamaBlock(d=4096, H=32,
ff=11008), batch 1, T=2048, causal, CORDIC mode at n = 8, 16, 24.

Each stage's GPU input and output are captured during one forward pass and
the stage is checked on its own GPU input against the CPU checker:
  * the four NT projections (QKV 2048x12288x4096, output 2048x4096x4096,
    fc1 + SiLU 2048x11008x4096, fc2 2048x4096x11008): 256 sampled rows, 32
    sampled columns each, bit-exact with orc_matmul_entries (fc1 through the
    checker's CORDIC SiLU);
  * RoPE on the full Q and K: bit-exact with orc_rope_apply on the CORDIC-16
    table;
  * RMSNorm on 256 sampled rows of each norm: bit-exact with
    orc_rmsnorm_lanes (the kernel's row-sum order) and <= 1e-5 relative to
    the left-to-right orc_rmsnorm;
  * the causal attention core on 256 sampled (head, query) rows: scores
    from orc_matmul_entries, probabilities from orc_softmax_lanes, output
    row from orc_matmul_entries on those probabilities, bit-exact (and
    within the row-sum order bound T * 2^-24 * max|v| of the left-to-right
    softmax);
  * both residual adds, exact.
Then rows 0..3 of the block output are recomputed end to end from x by the
checker's composition (causality makes them depend on rows 0..3 only):
bit-exact with the lane-order sums, and within max|y - ref| / max(|ref|, 1)
< 1e-4 at n = 16, 24 with the left-to-right sums (at n = 8 a one-ulp change
of an exp argument can flip a CORDIC direction and move e^x by ~2^-6, so
only the bit-exact comparison is meaningful there).
Templates: reference lib/c/test_rac_lib_e2e.c:313-378 (block composition
from library ops) and rac_torch/rac_torch.py:1348-1383 (the block).
"""
import numpy as np
import pytest

import raclib as rl

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda"
D_MODEL, N_HEADS, FF, SEQ = 4096, 32, 11008, 2048
HD = D_MODEL // N_HEADS


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    import rac_amd
    rac_amd.load()
    yield
    torch.cuda.synchronize()


def H(t):
    return t.detach().float().cpu().numpy()


@pytest.fixture(scope="module")
def block():
    from rac_amd import rac_torch as rt
    g = torch.Generator(device=DEV)
    g.manual_seed(55)
    blk = rt.RACLlamaBlock(D_MODEL, N_HEADS, ff_dim=FF, max_seq_len=SEQ).to(DEV)
    with torch.no_grad():
        for prm in blk.parameters():
            if prm.dim() == 2:
                prm.normal_(0.0, 0.02, generator=g)
        blk.norm1.weight.normal_(1.0, 0.02, generator=g)
        blk.norm2.weight.normal_(1.0, 0.02, generator=g)
    x = torch.randn((1, SEQ, D_MODEL), device=DEV, generator=g)
    params = {k: H(v) for k, v in blk.state_dict().items()}
    return blk, x, params


def _run_captured(rt, blk, x, n):
    """One forward pass at n iterations; returns the block output and every
    stage's GPU input/output as host arrays."""
    cap = {}
    hooks = []

    def on(name, mod):
        def hook(_m, args, out):
            cap[name] = ([H(a) for a in args if isinstance(a, torch.Tensor)],
                         [H(o) for o in (out if isinstance(out, tuple) else (out,))])
        hooks.append(mod.register_forward_hook(hook))

    on("norm1", blk.norm1)
    on("qkv", blk.attn.qkv)
    on("rope", blk.attn.rope)
    on("out_proj", blk.attn.out_proj)
    on("norm2", blk.norm2)
    on("fc1", blk.ffn.fc1)
    on("fc2", blk.ffn.fc2)
    core = rt.rac_attention

    def core_spy(q, k, v, mask=None, is_causal=False):
        o = core(q, k, v, mask, is_causal)
        cap["attn"] = ([H(q), H(k), H(v)], [H(o)])
        return o

    prev = (rt.rac_get_mode(), rt.rac_get_precision())
    rt.rac_attention = core_spy
    rt.rac_set_mode("cordic")
    rt.rac_set_precision(n)
    try:
        with torch.no_grad():
            y = H(blk(x, is_causal=True))
    finally:
        rt.rac_attention = core
        rt.rac_set_mode(prev[0])
        rt.rac_set_precision(prev[1])
        for h in hooks:
            h.remove()
    return y[0], cap


def _sample_pairs(rng, M, N, rows=256, cols=32):
    r = np.sort(rng.choice(M, rows, replace=False))
    rr = np.repeat(r, cols).astype(np.int32)
    cc = rng.integers(0, N, rows * cols).astype(np.int32)
    return rr, cc


def _check_nt(name, a, w, got, n, rng, post=None):
    """got[r, c] == (a @ w^T)[r, c] (then `post`) on sampled entries, bit-exact."""
    a = np.ascontiguousarray(a.reshape(-1, a.shape[-1]), np.float32)
    w = np.ascontiguousarray(w, np.float32)
    got = got.reshape(-1, w.shape[0])
    M, K = a.shape
    N = w.shape[0]
    rr, cc = _sample_pairs(rng, M, N)
    ref = rl.orc_matmul_entries(a, w, M, N, K, n, 1, rr, cc, tb=1)
    if post is not None:
        ref = post(ref)
    g = got[rr, cc]
    bad = np.flatnonzero(g.view(np.uint32) != ref.view(np.uint32))
    assert bad.size == 0, f"{name} n={n}: {bad.size} of {g.size} sampled entries differ, first " \
                          f"({rr[bad[0]]}, {cc[bad[0]]}): {g[bad[0]]!r} vs {ref[bad[0]]!r}"


def _check_rms(name, x, gamma, got, rng):
    x = x.reshape(-1, D_MODEL)
    got = got.reshape(-1, D_MODEL)
    r = np.sort(rng.choice(x.shape[0], 256, replace=False))
    assert np.array_equal(got[r], rl.orc_rmsnorm_lanes(x[r], gamma, 1e-6)), name
    err = rl.max_rel(got[r], rl.orc_rmsnorm(x[r], gamma, 1e-6), 1e-6)
    assert err < 1e-5, f"{name}: max relative error {err:.3e}"


@pytest.mark.parametrize("n", [8, 16, 24])
def test_llama_block_config5_sampled(block, n):
    from rac_amd import rac_torch as rt
    blk, x, P = block
    print(f"config5 block forward n={n}", flush=True)
    y, cap = _run_captured(rt, blk, x, n)
    assert np.isfinite(y).all()
    rng = np.random.default_rng(1000 + n)
    xn = H(x)[0]

    print(f"config5 n={n}: norms", flush=True)
    _check_rms("norm1", cap["norm1"][0][0], P["norm1.weight"], cap["norm1"][1][0], rng)
    _check_rms("norm2", cap["norm2"][0][0], P["norm2.weight"], cap["norm2"][1][0], rng)
    assert np.array_equal(cap["norm1"][0][0][0], xn)

    print(f"config5 n={n}: projections", flush=True)
    _check_nt("qkv", cap["qkv"][0][0], P["attn.qkv.weight"], cap["qkv"][1][0], n, rng)
    _check_nt("out_proj", cap["out_proj"][0][0], P["attn.out_proj.weight"], cap["out_proj"][1][0], n, rng)
    _check_nt("fc1+silu", cap["fc1"][0][0], P["ffn.fc1.weight"], cap["fc1"][1][0], n, rng,
              post=lambda v: rl.orc_unary("orc_silu", v, n))
    _check_nt("fc2", cap["fc2"][0][0], P["ffn.fc2.weight"], cap["fc2"][1][0], n, rng)

    print(f"config5 n={n}: rope", flush=True)
    c, s = rl.orc_rope_cache(SEQ, HD)
    (q_in, k_in), (q_out, k_out) = cap["rope"]
    assert q_in.shape == (1, N_HEADS, SEQ, HD)
    assert np.array_equal(q_out, rl.orc_rope_apply(q_in, c, s)), f"rope q n={n}"
    assert np.array_equal(k_out, rl.orc_rope_apply(k_in, c, s)), f"rope k n={n}"

    print(f"config5 n={n}: attention core", flush=True)
    (q, k, v), (o,) = cap["attn"]
    assert np.array_equal(q, q_out) and np.array_equal(k, k_out)
    scale = np.float32(1.0) / np.sqrt(np.float32(HD))
    vmax = float(np.abs(v).max())
    heads = rng.integers(0, N_HEADS, 256)
    rows = rng.integers(0, SEQ, 256)
    rows[:4] = (0, 1, SEQ - 2, SEQ - 1)
    for hh, t in zip(heads, rows):
        qh, kh, vh = np.ascontiguousarray(q[0, hh]), np.ascontiguousarray(k[0, hh]), v[0, hh]
        ks = np.arange(t + 1, dtype=np.int32)
        acc = rl.orc_matmul_entries(qh, kh, SEQ, SEQ, HD, n, 1, np.full(t + 1, t, np.int32), ks, tb=1)
        row = np.full((1, SEQ), -np.inf, np.float32)
        row[0, :t + 1] = acc * scale
        prob = rl.orc_softmax_lanes(row, n, zero_guard=True)
        assert not prob[0, t + 1:].any()
        vt = np.ascontiguousarray(vh[:t + 1])
        cols = np.arange(HD, dtype=np.int32)
        ref = rl.orc_matmul_entries(np.ascontiguousarray(prob[:, :t + 1]), vt, 1, HD, t + 1, n, 1,
                                    np.zeros(HD, np.int32), cols)
        assert np.array_equal(o[0, hh, t], ref), (n, int(hh), int(t))
        prob_seq = rl.orc_softmax(row[:, :t + 1], n)
        ref_seq = rl.orc_matmul_entries(prob_seq, vt, 1, HD, t + 1, n, 1, np.zeros(HD, np.int32), cols)
        err = float(np.max(np.abs(o[0, hh, t] - ref_seq)))
        assert err <= (t + 1) * 2.0 ** -24 * vmax + 1e-6 * vmax, (n, int(hh), int(t), err)

    print(f"config5 n={n}: residuals", flush=True)
    a_out = cap["out_proj"][1][0][0]
    x1 = (xn + a_out).astype(np.float32)
    assert np.array_equal(cap["norm2"][0][0][0], x1)
    assert np.array_equal(y, (x1 + cap["fc2"][1][0][0]).astype(np.float32))

    print(f"config5 n={n}: rows 0..3 end to end", flush=True)
    R = 4

    def lin(a, w):
        return rl.orc_matmul(np.ascontiguousarray(a, np.float32), np.ascontiguousarray(w), a.shape[0],
                             w.shape[0], a.shape[1], n, 1, tb=1)

    def composed(rms, softmax_rows):
        h = rms(xn[:R], P["norm1.weight"], 1e-6)
        qkv = lin(h, P["attn.qkv.weight"])
        qe, ke, ve = (qkv[:, i * D_MODEL:(i + 1) * D_MODEL].reshape(1, R, N_HEADS, HD).transpose(0, 2, 1, 3)
                      for i in range(3))
        qe = rl.orc_rope_apply(qe, c[:R], s[:R])
        ke = rl.orc_rope_apply(ke, c[:R], s[:R])
        ve = np.ascontiguousarray(ve)
        oe = np.zeros((1, N_HEADS, R, HD), np.float32)
        for hh in range(N_HEADS):
            sc = rl.orc_matmul(np.ascontiguousarray(qe[0, hh]), np.ascontiguousarray(ke[0, hh]), R, R, HD, n, 1,
                               tb=1, alpha=float(scale))
            oe[0, hh] = rl.orc_matmul(softmax_rows(sc), ve[0, hh], R, HD, R, n, 1)
        x1e = xn[:R] + lin(oe.transpose(0, 2, 1, 3).reshape(R, D_MODEL), P["attn.out_proj.weight"])
        h2 = rms(x1e, P["norm2.weight"], 1e-6)
        f1 = rl.orc_unary("orc_silu", lin(h2, P["ffn.fc1.weight"]), n)
        return x1e + lin(f1, P["ffn.fc2.weight"])

    def causal_lanes(sc):
        return rl.orc_softmax_lanes(sc, n, causal=True, zero_guard=True)

    def causal_seq(sc):
        pr = np.zeros((R, R), np.float32)
        for t in range(R):
            pr[t, :t + 1] = rl.orc_softmax(sc[t:t + 1, :t + 1], n)[0]
        return pr

    ref = composed(rl.orc_rmsnorm_lanes, causal_lanes)
    assert np.array_equal(y[:R], ref), (n, float(np.max(np.abs(y[:R] - ref))))
    if n >= 16:
        ref = composed(rl.orc_rmsnorm, causal_seq)
        err = np.abs(y[:R] - ref) / np.maximum(np.abs(ref), 1.0)
        assert err.max() < 1e-4, (n, float(err.max()))
