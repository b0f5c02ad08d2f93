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
            for g in range(nkv):
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
}


@pytest.mark.parametrize("iters", [24, 16])
@pytest.mark.parametrize("name", list(CFGS))
def test_decoder_prefill_then_decode(name, iters):
    from rac_amd.decoder import DecoderConfig
    cfg = DecoderConfig(**CFGS[name])
    W = _weights(cfg, seed=11 + iters)
    t_max = 16
    dec, orc, ref = _decoder(cfg, W, t_max, iters), OrcDecoder(cfg, W, t_max, iters), Ref64Decoder(cfg, W, t_max)
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
