"""GPU parity of the decoder stack with a KV cache (rac_amd.decoder, the
full-model path of bench/bench_rac_transformer.c decoder_forward_kv
:557-616 / full_model_forward :618-625): prefill, then token-by-token decode.

Bars:
  * bit-exact against the composition of the CPU checker's stages
    (orc_rmsnorm_lanes, orc_q8_gemv / orc_matmul FAST, orc_softmax_lanes,
    orc_silu), each pinned in its own tests; the key/value cache too.
  * within 1e-5 (iters 24) or 2e-4 (iters 16) of max|ref| against a
    float64 restatement of
    decoder_forward_kv written from the reference loop by loop (per query
    head h its key/value head h // rep, -1e30 causal scores, libm softmax,
    SiLU and 1 / sqrt RMSNorm on dequantized Q8_0 weights for decode and
    fp32 weights for prefill).  This pins the structure (head grouping,
    causal offset, cache positions, residuals) independently of the
    checker composition, which follows the same layout as the product.
"""
import numpy as np
import pytest

import raclib as rl

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda"
F32 = np.float32


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


def _weights(cfg, seed):
    d, dh, nkv, dff = cfg.d_model, cfg.d_head, cfg.n_kv_heads, cfg.d_ff
    shapes = {"W_q": (d, d), "W_k": (nkv * dh, d), "W_v": (nkv * dh, d), "W_o": (d, d),
              "W_g": (dff, d), "W_u": (dff, d), "W_d": (d, dff)}
    out = []
    for L in range(cfg.n_layers):
        w = {}
        for i, (name, (n, k)) in enumerate(shapes.items()):
            w[name] = (rl.gen_normal((n, k), seed=seed + 100 * L + i) / F32(np.sqrt(k))).astype(F32)
        w["rms_att"] = (F32(1) + F32(0.1) * rl.gen_normal((d,), seed=seed + 100 * L + 50)).astype(F32)
        w["rms_ffn"] = (F32(1) + F32(0.1) * rl.gen_normal((d,), seed=seed + 100 * L + 51)).astype(F32)
        out.append(w)
    return out


# ── the checker composition (bit-exact bar) ──────────────────────────────────

def orc_decode_attention(q, K, V, n, n_heads, scale, iters):
    """One token's attention over cache positions 0 .. n-1 as the checker's
    stages: FAST scores (alpha = scale), the lane-order softmax of the row
    padded with -inf to a multiple of 4, FAST P V."""
    nkv, _, dh = K.shape
    rep = n_heads // nkv
    n4 = 4 * ((n + 3) // 4)
    out = np.empty(n_heads * dh, F32)
    for g in range(nkv):
        qg = np.ascontiguousarray(q.reshape(nkv, rep, dh)[g])
        s = rl.orc_matmul(qg, np.ascontiguousarray(K[g, :n]), rep, n, dh, iters, 0, tb=1, alpha=float(scale))
        sp = np.full((rep, n4), -np.inf, F32)
        sp[:, :n] = s
        p = np.ascontiguousarray(rl.orc_softmax_lanes(sp, iters)[:, :n])
        out[g * rep * dh:(g + 1) * rep * dh] = rl.orc_matmul(p, np.ascontiguousarray(V[g, :n]), rep, dh, n,
                                                             iters, 0).reshape(-1)
    return out


class OrcDecoder:
    def __init__(self, cfg, W, t_max, iters):
        self.cfg, self.W, self.iters = cfg, W, iters
        shape = (cfg.n_kv_heads, t_max, cfg.d_head)
        self.K = [np.zeros(shape, F32) for _ in W]
        self.V = [np.zeros(shape, F32) for _ in W]
        self.q8 = [{"qkv": rl.orc_q8_quantize(np.concatenate([w["W_q"], w["W_k"], w["W_v"]])),
                    "o": rl.orc_q8_quantize(w["W_o"]),
                    "gu": rl.orc_q8_quantize(np.concatenate([w["W_g"], w["W_u"]])),
                    "d": rl.orc_q8_quantize(w["W_d"])} for w in W]
        self.length = 0
        self.scale = F32(1) / np.sqrt(F32(cfg.d_head))

    def _lin(self, x, q8, w):
        if x.shape[0] == 1:
            return rl.orc_q8_gemv(x, q8, None, 0)
        return rl.orc_matmul(np.ascontiguousarray(x), np.ascontiguousarray(w), x.shape[0], w.shape[0],
                             w.shape[1], self.iters, 0, tb=1)

    def forward(self, x):
        cfg, n = self.cfg, self.iters
        d, dh, nkv, dff = cfg.d_model, cfg.d_head, cfg.n_kv_heads, cfg.d_ff
        rep = cfg.n_heads // nkv
        Tn, start = x.shape[0], self.length
        total = start + Tn
        for L, w in enumerate(self.W):
            q8 = self.q8[L]
            h = rl.orc_rmsnorm_lanes(x, w["rms_att"], cfg.eps)
            qkv = self._lin(h, q8["qkv"], np.concatenate([w["W_q"], w["W_k"], w["W_v"]]))
            q = qkv[:, :d]
            self.K[L][:, start:total] = qkv[:, d:d + nkv * dh].reshape(Tn, nkv, dh).transpose(1, 0, 2)
            self.V[L][:, start:total] = qkv[:, d + nkv * dh:].reshape(Tn, nkv, dh).transpose(1, 0, 2)
            att = np.empty((Tn, d), F32)
            tq = np.tile(np.arange(Tn), rep)[:, None]
            if Tn == 1:
                att[0] = orc_decode_attention(q[0], self.K[L], self.V[L], total, cfg.n_heads, self.scale, n)
            for g in range(nkv if Tn > 1 else 0):
                qg = q.reshape(Tn, nkv, rep, dh)[:, g].transpose(1, 0, 2).reshape(rep * Tn, dh)
                s = rl.orc_matmul(np.ascontiguousarray(qg), np.ascontiguousarray(self.K[L][g, :total]),
                                  rep * Tn, total, dh, n, 0, tb=1, alpha=float(self.scale))
                s[np.arange(total)[None, :] > start + tq] = -np.inf
                p = rl.orc_softmax_lanes(s, n)
                o = rl.orc_matmul(p, np.ascontiguousarray(self.V[L][g, :total]), rep * Tn, dh, total, n, 0)
                att[:, g * rep * dh:(g + 1) * rep * dh] = o.reshape(rep, Tn, dh).transpose(1, 0, 2).reshape(Tn, -1)
            x = (x + self._lin(att, q8["o"], w["W_o"])).astype(F32)
            h = rl.orc_rmsnorm_lanes(x, w["rms_ffn"], cfg.eps)
            if Tn == 1:
                gu = rl.orc_q8_gemv(h, q8["gu"], None, 0)
                f = rl.orc_unary("orc_silu", gu[:, :dff], n) * gu[:, dff:]
            else:
                f = (rl.orc_unary("orc_silu", self._lin(h, None, w["W_g"]), n) * self._lin(h, None, w["W_u"]))
            x = (x + self._lin(f.astype(F32), q8["d"], w["W_d"])).astype(F32)
        self.length = total
        return x


# ── float64 restatement of decoder_forward_kv (tolerance bar) ────────────────

def _deq(wq, rows, K):
    out = np.empty((rows, K), F32)
    rl.oracle().orc_q8_0_dequantize(rl.p(np.ascontiguousarray(wq)), rl.p(out), rows, K)
    return out.astype(np.float64)


class Ref64Decoder:
    """bench_rac_transformer.c:557-625, with the reference's cache layout
    [T_max, n_kv_heads * d_head] per layer."""

    def __init__(self, cfg, W, t_max):
        self.cfg, self.W = cfg, W
        kv = cfg.n_kv_heads * cfg.d_head
        self.K = [np.zeros((t_max, kv)) for _ in W]
        self.V = [np.zeros((t_max, kv)) for _ in W]
        self.deq = [{k: _deq(rl.orc_q8_quantize(w[k]), *w[k].shape) for k in
                     ("W_q", "W_k", "W_v", "W_o", "W_g", "W_u", "W_d")} for w in W]
        self.length = 0

    @staticmethod
    def _rmsnorm(x, scale):                                   # :316-332
        inv = 1.0 / np.sqrt((x * x).sum(1, keepdims=True) / x.shape[1] + 1e-5)
        return x * scale[None, :] * inv

    def forward(self, x):
        cfg = self.cfg
        d, dh, nh, nkv = cfg.d_model, cfg.d_head, cfg.n_heads, cfg.n_kv_heads
        rep = nh // nkv
        Tn, start = x.shape[0], self.length
        total = start + Tn
        scale = 1.0 / np.sqrt(dh)
        x = x.astype(np.float64)
        for L, w in enumerate(self.W):
            Wt = self.deq[L] if Tn == 1 else {k: w[k].astype(np.float64) for k in self.deq[L]}
            norm = self._rmsnorm(x, w["rms_att"].astype(np.float64))
            Q = norm @ Wt["W_q"].T
            self.K[L][start:total] = norm @ Wt["W_k"].T
            self.V[L][start:total] = norm @ Wt["W_v"].T
            att = np.zeros((Tn, d))
            for h in range(nh):
                kv_h = h // rep
                kcols = slice(kv_h * dh, (kv_h + 1) * dh)
                for i in range(Tn):
                    abs_i = start + i
                    row = self.K[L][:total, kcols] @ Q[i, h * dh:(h + 1) * dh] * scale
                    row[np.arange(total) > abs_i] = -1e30
                    e = np.exp(row - row.max())
                    att[i, h * dh:(h + 1) * dh] = (e / e.sum()) @ self.V[L][:total, kcols]
            x = x + att @ Wt["W_o"].T
            norm = self._rmsnorm(x, w["rms_ffn"].astype(np.float64))
            g = norm @ Wt["W_g"].T
            g = g / (1.0 + np.exp(-g))
            x = x + (g * (norm @ Wt["W_u"].T)) @ Wt["W_d"].T
        self.length = total
        return x


def _decoder(cfg, W, t_max, iters):
    from rac_amd.decoder import RACDecoder
    return RACDecoder(cfg, [{k: T(v) for k, v in w.items()} for w in W], t_max, iters=iters)


CFGS = {
    "gqa": dict(d_model=128, n_heads=8, n_kv_heads=2, d_ff=224, n_layers=2),
    "mha": dict(d_model=96, n_heads=3, n_kv_heads=3, d_ff=160, n_layers=2),
    "mqa": dict(d_model=64, n_heads=4, n_kv_heads=1, d_ff=96, n_layers=3),
    # d_model % 256 == 0: decode runs the fused-norm GEMVs
    "fused": dict(d_model=256, n_heads=4, n_kv_heads=2, d_ff=352, n_layers=2),
}


@pytest.mark.parametrize("iters", [24, 16])
@pytest.mark.parametrize("name", list(CFGS))
def test_decoder_prefill_then_decode(name, iters):
    from rac_amd.decoder import DecoderConfig
    cfg = DecoderConfig(**CFGS[name])
    W = _weights(cfg, seed=11 + iters)
    t_max = 16
    dec, orc, ref = _decoder(cfg, W, t_max, iters), OrcDecoder(cfg, W, t_max, iters), Ref64Decoder(cfg, W, t_max)
    assert dec._fused == (name == "fused")
    schedule = [5, 1, 1, 3, 1, 1]           # prefill, decode, a second prefill chunk, decode
    for step, Tn in enumerate(schedule):
        print(f"decoder {name} iters={iters} step={step} T_new={Tn}", flush=True)
        x = rl.gen_normal((Tn, cfg.d_model), seed=1000 + step)
        got = H(dec.forward(T(x)))
        want = orc.forward(x)
        assert np.array_equal(got, want), (name, step)
        r64 = ref.forward(x)
        err = np.abs(got.astype(np.float64) - r64).max()
        assert err <= (1e-5 if iters >= 24 else 2e-4) * np.abs(r64).max(), (name, step, err)
        assert dec.length == orc.length == ref.length
    for L in range(cfg.n_layers):
        assert np.array_equal(H(dec.k_cache[L][:, :dec.length]), orc.K[L][:, :orc.length])
        assert np.array_equal(H(dec.v_cache[L][:, :dec.length]), orc.V[L][:, :orc.length])


def test_decoder_decode_from_empty_and_reset():
    from rac_amd.decoder import DecoderConfig
    cfg = DecoderConfig(**CFGS["gqa"])
    W = _weights(cfg, seed=3)
    dec, orc = _decoder(cfg, W, 8, 24), OrcDecoder(cfg, W, 8, 24)
    xs = [rl.gen_normal((1, cfg.d_model), seed=50 + i) for i in range(4)]
    first = None
    for i, x in enumerate(xs):
        got = H(dec.step(T(x)))
        assert np.array_equal(got, orc.forward(x)), i
        if i == 0:
            first = got
    dec.reset()
    assert dec.length == 0
    assert np.array_equal(H(dec.step(T(xs[0]))), first)       # an empty cache again


def test_decoder_errors():
    from rac_amd.decoder import DecoderConfig, RACDecoder
    cfg = DecoderConfig(**CFGS["mqa"])
    W = [{k: T(v) for k, v in w.items()} for w in _weights(cfg, seed=5)]
    dec = RACDecoder(cfg, W, t_max=4)
    dec.forward(T(rl.gen_normal((3, cfg.d_model), seed=1)))
    with pytest.raises(RuntimeError, match="cache full"):
        dec.forward(T(rl.gen_normal((2, cfg.d_model), seed=2)))
    dec.step(T(rl.gen_normal((1, cfg.d_model), seed=3)))
    with pytest.raises(RuntimeError, match="cache full"):
        dec.step(T(rl.gen_normal((1, cfg.d_model), seed=4)))
    with pytest.raises(RuntimeError):
        dec.forward(T(rl.gen_normal((1, cfg.d_model + 1), seed=4)))
    dq = RACDecoder(cfg, W, t_max=4, keep_f32=False)
    with pytest.raises(RuntimeError, match="fp32"):
        dq.forward(T(rl.gen_normal((2, cfg.d_model), seed=6)))
    dq.step(T(rl.gen_normal((1, cfg.d_model), seed=7)))      # decode needs only the Q8_0 weights
    with pytest.raises(ValueError):
        RACDecoder(DecoderConfig(96, 5, 5, 96, 1), [W[0]], t_max=4)


@pytest.mark.parametrize("tb", [0, 1])
def test_bmm_on_cache_slices(tb):
    """bmm reads batch items that sit T_max rows apart (a slice of a longer
    cache) in place; bit-exact with the checker on each item."""
    from rac_amd import ext as e
    Z, t_max, dh = 3, 40, 24
    cache = rl.gen_normal((Z, t_max, dh), seed=8)
    Ct = T(cache)
    for total in (1, 7, 33, 40):
        sl = Ct[:, :total, :]
        if tb:
            q = rl.gen_normal((Z, 5, dh), seed=total)
            got = H(e.bmm(T(q), sl, trans_b=True, alpha=0.5, mode=0))
            for z in range(Z):
                ref = rl.orc_matmul(np.ascontiguousarray(q[z]), np.ascontiguousarray(cache[z, :total]), 5, total,
                                    dh, 24, 0, tb=1, alpha=0.5)
                assert np.array_equal(got[z], ref), (total, z)
        else:
            p = rl.gen_uniform((Z, 6, total), seed=total)
            for mode, iters in ((0, 24), (1, 16)):
                got = H(e.bmm(T(p), sl, iters=iters, mode=mode))
                for z in range(Z):
                    ref = rl.orc_matmul(np.ascontiguousarray(p[z]), np.ascontiguousarray(cache[z, :total]), 6, dh,
                                        total, iters, mode)
                    assert np.array_equal(got[z], ref), (total, z, mode)


# ── the decode-step kernels (rac_decode.h) ───────────────────────────────────

@pytest.mark.parametrize("iters", [24, 16, 8, 12])
@pytest.mark.parametrize("heads,kv,dh,t_cap", [(8, 2, 16, 40), (4, 4, 64, 300), (6, 1, 7, 33), (32, 4, 64, 1030),
                                               (2, 2, 256, 9)])
def test_decode_attention_vs_checker(heads, kv, dh, t_cap, iters):
    from rac_amd import ext as e
    K = rl.gen_normal((kv, t_cap, dh), seed=heads + dh)
    V = rl.gen_normal((kv, t_cap, dh), seed=heads + dh + 1)
    q = rl.gen_normal((heads * dh,), seed=t_cap)
    scale = F32(1) / np.sqrt(F32(dh))
    Kt, Vt, qt = T(K), T(V), T(q)
    for n in sorted({1, 2, 3, 4, 5, 17, t_cap // 2 + 1, t_cap - 1, t_cap}):
        if n < 1 or n > t_cap:
            continue
        print(f"decode attention heads={heads} kv={kv} dh={dh} t_cap={t_cap} n={n} iters={iters}", flush=True)
        pos = torch.tensor([n - 1], dtype=torch.int32, device=DEV)
        got = H(e.decode_attention(qt, Kt, Vt, pos, heads, float(scale), iters))
        assert np.array_equal(got, orc_decode_attention(q, K, V, n, heads, scale, iters)), n


def test_decode_attention_scores_spread():
    """Large score spread (exps flushing to 0 beside 1) and equal scores."""
    from rac_amd import ext as e
    heads, kv, dh, t_cap = 4, 2, 32, 64
    K = rl.gen_normal((kv, t_cap, dh), seed=1) * F32(30)
    K[1, :20] = 0.0
    V = rl.gen_normal((kv, t_cap, dh), seed=2)
    q = rl.gen_normal((heads * dh,), seed=3) * F32(3)
    for n in (1, 19, 21, 64):
        pos = torch.tensor([n - 1], dtype=torch.int32, device=DEV)
        got = H(e.decode_attention(T(q), T(K.astype(F32)), T(V), pos, heads, 0.125, 16))
        assert np.array_equal(got, orc_decode_attention(q, K.astype(F32), V, n, heads, F32(0.125), 16)), n


def test_decode_attention_position_outside_cache_gives_nan():
    from rac_amd import ext as e
    K = T(np.ones((1, 8, 4), F32))
    for p in (-1, 8, 100):
        got = H(e.decode_attention(T(np.ones(8, F32)), K, K, torch.tensor([p], dtype=torch.int32, device=DEV), 2, 1.0))
        assert np.isnan(got).all(), p


def test_kv_append_and_advance():
    from rac_amd import ext as e
    kv, dh, t_cap = 3, 5, 7
    Kc = torch.full((kv, t_cap, dh), 7.0, device=DEV)
    Vc = torch.full((kv, t_cap, dh), 9.0, device=DEV)
    pos = torch.zeros(1, dtype=torch.int32, device=DEV)
    want_k, want_v = np.full((kv, t_cap, dh), 7.0, F32), np.full((kv, t_cap, dh), 9.0, F32)
    for step in range(t_cap + 2):
        src = rl.gen_normal((2 * kv * dh,), seed=step)
        e.kv_append_(T(src), Kc, Vc, pos)
        e.position_advance_(pos, 1)
        if step < t_cap:        # beyond the cache: nothing written
            want_k[:, step] = src[:kv * dh].reshape(kv, dh)
            want_v[:, step] = src[kv * dh:].reshape(kv, dh)
    assert int(H(pos)[0]) == t_cap + 2
    assert np.array_equal(H(Kc), want_k) and np.array_equal(H(Vc), want_v)
    e.position_advance_(pos, -3)
    assert int(H(pos)[0]) == t_cap - 1


@pytest.mark.parametrize("iters", [24, 16, 8, 5])
def test_swiglu_vs_checker(iters):
    from rac_amd import ext as e
    for n in (1, 7, 5632, 70001):
        gu = rl.gen_normal((1, 2 * n), seed=n) * F32(4)
        if n >= 4:
            gu[0, :4] = [0.0, -0.0, 60.0, -60.0]
        got = H(e.swiglu(T(gu), iters))
        want = rl.orc_unary("orc_silu", gu[:, :n], iters) * gu[:, n:]
        assert np.array_equal(got, want), n
        assert np.array_equal(got, H(e.silu(T(gu[:, :n]), iters) * T(gu[:, n:])))


@pytest.mark.parametrize("name", ["gqa", "fused"])
def test_decoder_graph_replays_equal_eager(name):
    """The captured decode step replayed per token, with other work and
    synchronisations between the replays, equals the eager step bit for
    bit, and the caches agree afterwards."""
    from rac_amd.decoder import DecoderConfig
    cfg = DecoderConfig(**CFGS[name])
    W = _weights(cfg, seed=21)
    eager, graphed = _decoder(cfg, W, 24, 24), _decoder(cfg, W, 24, 24)
    x0 = rl.gen_normal((4, cfg.d_model), seed=5)
    assert np.array_equal(H(eager.forward(T(x0))), H(graphed.forward(T(x0))))
    graphed.capture()
    other = torch.ones(1000, device=DEV)
    for i in range(9):
        x = rl.gen_normal((1, cfg.d_model), seed=40 + i)
        want = H(eager.step(T(x)))
        got = H(graphed.step(T(x)))
        assert np.array_equal(got, want), i
        other = (other * 1.5).sum().expand(1000).contiguous()      # unrelated eager work between replays
        torch.cuda.synchronize()
    assert eager.length == graphed.length == 13
    assert int(H(graphed.pos)[0]) == 13
    for L in range(cfg.n_layers):
        assert np.array_equal(H(eager.k_cache[L][:, :13]), H(graphed.k_cache[L][:, :13]))
        assert np.array_equal(H(eager.v_cache[L][:, :13]), H(graphed.v_cache[L][:, :13]))
    # a prefill chunk after graph replays, then replays again
    x2 = rl.gen_normal((3, cfg.d_model), seed=77)
    assert np.array_equal(H(eager.forward(T(x2))), H(graphed.forward(T(x2))))
    x = rl.gen_normal((1, cfg.d_model), seed=78)
    assert np.array_equal(H(graphed.step(T(x))), H(eager.step(T(x))))
    graphed.reset()
    eager.reset()
    assert np.array_equal(H(graphed.step(T(x))), H(eager.step(T(x))))


# ── the fused-norm decode GEMVs against their unfused forms ──────────────────

@pytest.mark.parametrize("N,K", [(2560, 2048), (2048, 2048), (4, 256), (700, 768), (11264, 2048), (2048, 5632),
                                 (100, 16384)])
def test_q8_gemv_rmsnorm_equals_unfused(N, K):
    from rac_amd import ext as e
    x = T(rl.gen_normal((1, K), seed=N) * F32(3))
    g = T((F32(1) + F32(0.2) * rl.gen_normal((K,), seed=K)).astype(F32))
    wq = e.q8_quantize(T(rl.gen_normal((N, K), seed=N + K) / F32(np.sqrt(K))))
    b = T(rl.gen_normal((N,), seed=1))
    for act in (0, 1):
        for bias in (None, b):
            got = H(e.q8_gemv_rmsnorm(x, g, 1e-5, wq, bias=bias, act=act))
            want = H(e.q8_gemv(e.rmsnorm(x, g, 1e-5), wq, bias=bias, act=act))
            assert np.array_equal(got, want), (N, K, act, bias is None)
    # against the checker too
    h = rl.orc_rmsnorm_lanes(H(x), H(g), 1e-5)
    assert np.array_equal(H(e.q8_gemv_rmsnorm(x, g, 1e-5, wq)), rl.orc_q8_gemv(h, H(wq), None, 0))


@pytest.mark.parametrize("heads,kv,dh,K", [(32, 4, 64, 2048), (4, 2, 64, 256), (8, 8, 32, 512), (16, 1, 128, 2048)])
def test_decode_qkv_equals_unfused(heads, kv, dh, K):
    from rac_amd import ext as e
    t_cap = 10
    x = T(rl.gen_normal((1, K), seed=heads))
    g = T((F32(1) + F32(0.1) * rl.gen_normal((K,), seed=dh)).astype(F32))
    wq = e.q8_quantize(T(rl.gen_normal(((heads + 2 * kv) * dh, K), seed=K) / F32(np.sqrt(K))))
    K1, V1 = torch.zeros((kv, t_cap, dh), device=DEV), torch.zeros((kv, t_cap, dh), device=DEV)
    K2, V2 = torch.zeros_like(K1), torch.zeros_like(V1)
    for p in (0, 3, t_cap - 1, t_cap, -1):        # the last two lie outside the cache: no write
        pos = torch.tensor([p], dtype=torch.int32, device=DEV)
        q = e.decode_qkv(x, g, 1e-5, wq, K1, V1, heads, pos)
        qkv = e.q8_gemv(e.rmsnorm(x, g, 1e-5), wq)
        e.kv_append_(qkv[0, heads * dh:], K2, V2, pos)
        assert np.array_equal(H(q), H(qkv[0, :heads * dh])), p
        assert np.array_equal(H(K1), H(K2)) and np.array_equal(H(V1), H(V2)), p


@pytest.mark.parametrize("iters", [24, 16, 8])
@pytest.mark.parametrize("n_ff,K", [(5632, 2048), (8, 256), (1000, 512), (96, 4096)])
def test_decode_swiglu_gemv_equals_unfused(n_ff, K, iters):
    from rac_amd import ext as e
    x = T(rl.gen_normal((1, K), seed=n_ff) * F32(2))
    g = T((F32(1) + F32(0.1) * rl.gen_normal((K,), seed=K)).astype(F32))
    Wg = T(rl.gen_normal((n_ff, K), seed=1) * F32(3) / F32(np.sqrt(K)))
    Wu = T(rl.gen_normal((n_ff, K), seed=2) / F32(np.sqrt(K)))
    got = H(e.decode_swiglu_gemv(x, g, 1e-5, e.q8_quantize(e.q8_interleave_rows(Wg, Wu)), iters))
    h = e.rmsnorm(x, g, 1e-5)
    gu = e.q8_gemv(h, e.q8_quantize(torch.cat([Wg, Wu])))
    assert np.array_equal(got, H(e.swiglu(gu, iters)))


def test_fused_gemv_rejects_unsupported_shapes():
    from rac_amd import ext as e
    x = T(rl.gen_normal((1, 96), seed=1))
    g = T(np.ones(96, F32))
    wq = e.q8_quantize(T(rl.gen_normal((8, 96), seed=2)))
    assert not e.fused_gemv_ok(x, g, wq)
    with pytest.raises(RuntimeError, match="multiple of 256"):
        e.q8_gemv_rmsnorm(x, g, 1e-5, wq)
