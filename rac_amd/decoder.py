"""A Llama-style decoder stack with a KV cache on the RAC kernels: the
full-model path of the reference's bench/bench_rac_transformer.c
(decoder_forward_kv :557-616, full_model_forward :618-625, the cache of
kv_alloc :476-490), prefill and token-by-token decode.

Per layer, for T_new new tokens at cache position `start`, as the
reference: RMSNorm; the Q, K and V projections; K and V written into the
cache at positions start .. start + T_new - 1; grouped-query causal
attention over the cache (query head h reads key/value head
h // (n_heads / n_kv_heads); token t sees cache positions <= start + t);
the output projection and a residual add; RMSNorm; the SwiGLU feed-forward
(SiLU(gate) * up, then the down projection) and a residual add.  No RoPE,
as in the reference's decoder.  The cache length advances once all layers
have run (full_model_forward).

Weights, as the reference's bench_fused_linear_q8 (:301-312): one new token
(decode) streams Q8_0 weights through the Q8_0 GEMV (rac_q8_0.c:178-211);
several (prefill) run the fp32 weights through the fused RAC linear (FAST
MAC, the reference's rac_hal_fused_linear).  The Q, K and V weight matrices
are stacked into one, as are gate and up for decode: every output row is
computed on its own, so one launch gives the same bits as three (two).

MI355X form: weights resident in HBM; the cache is [n_kv_heads, T_max,
d_head] per layer, so each key/value head's keys and values are one
row-major matrix.  Prefill attention of a head group is two RAC products
(scores = Q_group K^T / sqrt(d_head), out = P V; FAST MAC, the reference's
fp32 dot products) around the RAC softmax, reading the cache in place.  Masked scores are -inf (the reference writes -1e30); either gives
probability 0.  SiLU is the RAC CORDIC SiLU (rac_cpu.c:453-457) at
`iters` and RMSNorm is rac_rmsnorm (rac_cpu.c:548-574, eps 1e-5); the
reference's bench computes those two with libm (expf, 1 / sqrtf), which
differs by float rounding.

Decode (one new token) runs on kernels that read the cache position from
device memory (rac_decode.h): RMSNorm, the Q|K|V GEMV, the cache append,
the fused attention of each query head over the cache, the output GEMV with
the residual as its bias (x + W_o a: the GEMV adds its bias last, and float
addition commutes), RMSNorm, the gate|up GEMV, SiLU(gate) * up, and the down
GEMV with the residual as bias; then the position advances on the device.
Every launch of a decode step then has fixed arguments, so `capture()`
records the whole step, all layers, as one HIP graph that `step()` replays
per token, bit-identical to the eager step.  The attention's softmax sums
the row as the row kernel does on the scores padded with -inf to a
multiple of 4 (a summation order; the padded probabilities are 0).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List

import torch

from . import ext

__all__ = ["DecoderConfig", "RACDecoder", "PRESETS"]


@dataclass(frozen=True)
class DecoderConfig:
    """bench_rac_transformer.c tx_cfg (:52-68): model shape."""
    d_model: int
    n_heads: int
    n_kv_heads: int
    d_ff: int
    n_layers: int
    eps: float = 1e-5

    @property
    def d_head(self) -> int:
        return self.d_model // self.n_heads


# bench_rac_transformer.c cfg_apply_preset (:70-82)
PRESETS = {
    "tiny": DecoderConfig(512, 8, 8, 1536, 4),
    "tinyllama": DecoderConfig(2048, 32, 4, 5632, 22),
}


class _Layer:
    """One layer's weights: fp32 for prefill (kept only when asked) and Q8_0
    blocks for decode."""

    def __init__(self, w: dict, keep_f32: bool):
        wqkv = torch.cat([w["W_q"], w["W_k"], w["W_v"]], 0).contiguous()
        self.q8_qkv = ext.q8_quantize(wqkv)
        self.q8_o = ext.q8_quantize(w["W_o"])
        # gate and up rows interleaved: one GEMV, its epilogue pairs them
        self.q8_gu = ext.q8_quantize(ext.q8_interleave_rows(w["W_g"], w["W_u"]))
        self.q8_d = ext.q8_quantize(w["W_d"])
        self.f32 = None
        if keep_f32:
            self.f32 = {"qkv": wqkv, "o": w["W_o"].contiguous(), "g": w["W_g"].contiguous(),
                        "u": w["W_u"].contiguous(), "d": w["W_d"].contiguous()}
        self.rms_att = w["rms_att"].contiguous()
        self.rms_ffn = w["rms_ffn"].contiguous()


class RACDecoder:
    """Decoder stack with a KV cache.

    layers: one dict per layer of fp32 device tensors W_q [d, d], W_k and
    W_v [n_kv_heads * d_head, d], W_o [d, d], W_g and W_u [d_ff, d], W_d
    [d, d_ff], rms_att and rms_ffn [d] (the reference's tx_weights,
    :86-98).  t_max: cache length.  keep_f32: keep the fp32 weights for
    prefill (several tokens per call); without them only decode runs."""

    def __init__(self, cfg: DecoderConfig, layers: List[dict], t_max: int, iters: int = 24,
                 keep_f32: bool = True):
        if cfg.d_model % cfg.n_heads or cfg.n_heads % cfg.n_kv_heads:
            raise ValueError("RAC: d_model must divide into n_heads, n_heads into n_kv_heads")
        if cfg.d_model % 32 or cfg.d_ff % 32:
            raise ValueError("RAC: Q8_0 weights need d_model and d_ff multiples of 32")
        if len(layers) != cfg.n_layers:
            raise ValueError("RAC: one weight dict per layer")
        if t_max <= 0:
            raise ValueError("RAC: t_max must be positive")
        self.cfg = cfg
        self.iters = iters
        self.t_max = t_max
        self.layers = [_Layer(w, keep_f32) for w in layers]
        if t_max > ext.DECODE_MAX_LEN or cfg.d_head > ext.DECODE_MAX_HEAD:
            raise ValueError(f"RAC: decode supports t_max <= {ext.DECODE_MAX_LEN} and "
                             f"d_head <= {ext.DECODE_MAX_HEAD}")
        dev = layers[0]["W_q"].device
        shape = (cfg.n_kv_heads, t_max, cfg.d_head)
        # positions at or beyond the current length are never read: every
        # product stops at start + T_new
        self.k_cache = [torch.zeros(shape, device=dev) for _ in range(cfg.n_layers)]
        self.v_cache = [torch.zeros(shape, device=dev) for _ in range(cfg.n_layers)]
        self.length = 0
        self.pos = torch.zeros(1, device=dev, dtype=torch.int32)     # the length, on the device
        self._graph = None
        # the fused decode GEMVs (norm inside, cache / SwiGLU epilogues) need
        # d_model % 256 == 0 and 16-byte aligned buffers; other shapes run
        # the same arithmetic unfused
        probe = torch.empty((1, cfg.d_model), device=dev)
        self._fused = all(ext.fused_gemv_ok(probe, g, q) for lw in self.layers
                          for g, q in ((lw.rms_att, lw.q8_qkv), (lw.rms_ffn, lw.q8_gu)))
        # 1.0f / sqrtf((float)d_head), as attention_head_causal (:515)
        self.scale = float(torch.tensor(1.0) / torch.sqrt(torch.tensor(float(cfg.d_head))))

    def reset(self):
        """kv_reset (:492): the cache is empty again."""
        self.length = 0
        self.pos.zero_()

    def _linear(self, x: torch.Tensor, w: torch.Tensor, act: int = 0) -> torch.Tensor:
        return ext.fused_linear_forward(x, w, None, act, iters=self.iters, mode=ext.MODE_FAST)

    def _prefill_attention(self, L: int, q: torch.Tensor, start: int, T: int) -> torch.Tensor:
        cfg = self.cfg
        nkv, dh = cfg.n_kv_heads, cfg.d_head
        rep = cfg.n_heads // nkv
        total = start + T
        # query rows of head group g: row r * T + t is head g * rep + r, token t
        qg = q.view(T, nkv, rep, dh).permute(1, 2, 0, 3).reshape(nkv, rep * T, dh)
        kc = self.k_cache[L][:, :total, :]
        vc = self.v_cache[L][:, :total, :]
        s = ext.bmm(qg, kc, trans_b=True, alpha=self.scale, iters=self.iters, mode=ext.MODE_FAST)
        t = torch.arange(T, device=q.device).repeat(rep).view(rep * T, 1)
        j = torch.arange(total, device=q.device).view(1, total)
        s.masked_fill_(j > start + t, float("-inf"))
        p = ext.softmax(s.view(nkv * rep * T, total), self.iters).view(nkv, rep * T, total)
        o = ext.bmm(p, vc, iters=self.iters, mode=ext.MODE_FAST)          # [nkv, rep * T, dh]
        return o.view(nkv, rep, T, dh).permute(2, 0, 1, 3).reshape(T, cfg.d_model)

    def _prefill_layer(self, L: int, x: torch.Tensor, start: int) -> torch.Tensor:
        cfg, lw = self.cfg, self.layers[L]
        d, dh, nkv = cfg.d_model, cfg.d_head, cfg.n_kv_heads
        T = x.size(0)
        w = lw.f32
        h = ext.rmsnorm(x, lw.rms_att, cfg.eps)
        qkv = self._linear(h, w["qkv"])                                    # [T, d + 2 nkv dh]
        self.k_cache[L][:, start:start + T, :] = qkv[:, d:d + nkv * dh].reshape(T, nkv, dh).transpose(0, 1)
        self.v_cache[L][:, start:start + T, :] = qkv[:, d + nkv * dh:].reshape(T, nkv, dh).transpose(0, 1)
        att = self._prefill_attention(L, qkv[:, :d].contiguous(), start, T)
        x = x + self._linear(att, w["o"])
        h = ext.rmsnorm(x, lw.rms_ffn, cfg.eps)
        f = self._linear(h, w["g"], 3) * self._linear(h, w["u"])             # silu(gate) * up
        return x + self._linear(f, w["d"])

    def _decode_layer(self, L: int, x: torch.Tensor) -> torch.Tensor:
        cfg, lw = self.cfg, self.layers[L]
        d = cfg.d_model
        kc, vc = self.k_cache[L], self.v_cache[L]
        if self._fused:
            # RMSNorm inside the GEMVs; keys / values straight into the cache;
            # SiLU(gate) * up in the gate / up GEMV's epilogue
            q = ext.decode_qkv(x, lw.rms_att, cfg.eps, lw.q8_qkv, kc, vc, cfg.n_heads, self.pos)
        else:
            qkv = ext.q8_gemv(ext.rmsnorm(x, lw.rms_att, cfg.eps), lw.q8_qkv)     # [1, d + 2 nkv dh]
            ext.kv_append_(qkv[0, d:], kc, vc, self.pos)
            q = qkv[0, :d]
        att = ext.decode_attention(q, kc, vc, self.pos, cfg.n_heads, self.scale, self.iters)
        x = ext.q8_gemv(att.view(1, d), lw.q8_o, bias=x.view(d))                  # x + W_o att
        if self._fused:
            f = ext.decode_swiglu_gemv(x, lw.rms_ffn, cfg.eps, lw.q8_gu, self.iters)
        else:
            gu = ext.q8_gemv(ext.rmsnorm(x, lw.rms_ffn, cfg.eps), lw.q8_gu)       # gate / up pairs
            f = ext.swiglu(gu.view(-1, 2).t().reshape(1, -1), self.iters)           # silu(gate) * up
        return ext.q8_gemv(f, lw.q8_d, bias=x.view(d))                            # x + W_d f

    def _decode_step(self, x: torch.Tensor) -> torch.Tensor:
        for L in range(self.cfg.n_layers):
            x = self._decode_layer(L, x)
        ext.position_advance_(self.pos, 1)
        return x

    @torch.no_grad()
    def capture(self) -> None:
        """Records one decode step (every layer and the position's advance)
        as a HIP graph; step() then replays it.  Runs one eager step first
        (launcher set-up happens outside the recording) and restores the
        position, so the cache's visible contents are unchanged."""
        if self.length >= self.t_max:
            raise RuntimeError("RAC: KV cache full")
        dev = self.pos.device
        x0 = torch.zeros((1, self.cfg.d_model), device=dev)
        self._decode_step(x0)
        self.pos.fill_(self.length)
        torch.cuda.synchronize(dev)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = self._decode_step(x0)
        torch.cuda.synchronize(dev)
        self._graph, self._gx, self._gout = graph, x0, out

    def release_graph(self) -> None:
        self._graph = self._gx = self._gout = None

    @torch.no_grad()
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """full_model_forward (:618-625): T_new tokens x [T_new, d_model]
        (fp32, device) through every layer; their keys and values join the
        cache and the length advances by T_new.  Returns the stack's
        output [T_new, d_model]."""
        if x.dim() != 2 or x.size(1) != self.cfg.d_model or x.dtype != torch.float32:
            raise RuntimeError("RAC: forward expects fp32 x of shape [T_new, d_model]")
        T = x.size(0)
        if T == 0:
            return x.clone()
        if self.length + T > self.t_max:
            raise RuntimeError("RAC: KV cache full")
        if T > 1 and self.layers[0].f32 is None:
            raise RuntimeError("RAC: prefill needs the fp32 weights (keep_f32=True)")
        start = self.length
        x = x.contiguous()
        if T == 1:
            if x.data_ptr() % 16:
                x = x.clone()                  # the fused GEMVs read x with 16-byte loads
            if self._graph is not None:
                self._gx.copy_(x)
                self._graph.replay()
                x = self._gout.clone()
            else:
                x = self._decode_step(x)
        else:
            for L in range(self.cfg.n_layers):
                x = self._prefill_layer(L, x, start)
            self.pos.fill_(start + T)
        self.length = start + T
        return x

    def step(self, x: torch.Tensor) -> torch.Tensor:
        """One decode token x [1, d_model]."""
        if x.dim() != 2 or x.size(0) != 1:
            raise RuntimeError("RAC: step expects x of shape [1, d_model]")
        return self.forward(x)

    @staticmethod
    def synthetic_weights(cfg: DecoderConfig, device, seed: int = 0) -> List[dict]:
        """Random weights of the reference's scale (xavier: variance about
        1/fan_in) and unit RMSNorm gains."""
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        dh, nkv = cfg.d_head, cfg.n_kv_heads

        def w(n, k):
            return torch.randn((n, k), device=device, generator=g) / math.sqrt(k)

        out = []
        for _ in range(cfg.n_layers):
            out.append({"W_q": w(cfg.d_model, cfg.d_model), "W_k": w(nkv * dh, cfg.d_model),
                        "W_v": w(nkv * dh, cfg.d_model), "W_o": w(cfg.d_model, cfg.d_model),
                        "W_g": w(cfg.d_ff, cfg.d_model), "W_u": w(cfg.d_ff, cfg.d_model),
                        "W_d": w(cfg.d_model, cfg.d_ff),
                        "rms_att": torch.ones(cfg.d_model, device=device),
                        "rms_ffn": torch.ones(cfg.d_model, device=device)})
        return out
