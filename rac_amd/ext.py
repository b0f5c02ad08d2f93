"""Tensor-level operator surface of the gfx950 kernels.

Mirrors the reference extension module ``rac_cuda_ext``
(rac_torch/rac_torch_bind.cpp:223-258): ``matmul_forward``,
``matmul_backward``, ``linear_forward``, ``linear_backward``,
``set/get_cordic_iters``, ``set/get_cordic_mode`` and ``MODE_*`` keep their
names, keyword arguments, defaults (iters=24, mode=FAST,
rac_torch_bind.cpp:54-55) and argument checks.  Added ops (new names, so the
reference's ``hasattr`` probing keeps working): ``rope_cache``,
``rope_apply_``, ``softmax``, ``rmsnorm``, ``layernorm``, ``silu``, ``gelu``,
``sigmoid``, ``tanh``, ``exp``, ``relu``, ``rsqrt``, ``sincos``, ``bmm``,
``softmax_masked_``, ``attention``, and the rac.h vector primitives
``vec2``, ``inner``, ``outer``, ``dct``.

Every op launches on torch's current HIP stream of the tensor's device and
returns without synchronising.  Only ROCm device tensors are accepted: there
is no CPU path.
"""
from __future__ import annotations

import ctypes
import os
from typing import List, Optional, Tuple

import numpy as np
import torch

from . import _lib
from ._lib import RACError, check

MODE_FAST = 0
MODE_CORDIC = 1
MODE_SHIFTADD = 2

_g_cordic_iters = 24          # rac_torch_bind.cpp:54
_g_cordic_mode = MODE_FAST    # rac_torch_bind.cpp:55


def set_cordic_iters(iters: int) -> None:
    """Process-wide iteration count; <= 0 restores 24, clamp to [1, 24]
    (rac_torch_bind.cpp:205-210)."""
    global _g_cordic_iters
    iters = int(iters)
    if iters <= 0:
        _g_cordic_iters = 24
        return
    _g_cordic_iters = max(1, min(24, iters))


def get_cordic_iters() -> int:
    return _g_cordic_iters


def set_cordic_mode(mode: int) -> None:
    """0=FAST, 1=CORDIC, 2=SHIFTADD; anything else selects FAST
    (rac_torch_bind.cpp:216-219)."""
    global _g_cordic_mode
    mode = int(mode)
    _g_cordic_mode = mode if 0 <= mode <= 2 else MODE_FAST


def get_cordic_mode() -> int:
    return _g_cordic_mode


def _resolve(iters: int, mode: int) -> Tuple[int, int]:
    if iters <= 0:
        iters = _g_cordic_iters
    if mode < 0:
        mode = _g_cordic_mode
    return max(1, min(24, int(iters))), int(mode)


def _resolve_iters(iters: int) -> int:
    return _resolve(iters, 0)[0]


def _stream(t: torch.Tensor) -> int:
    return _lib.stream_handle(t.device)


def _require_gpu(t: torch.Tensor, what: str = "input") -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"RAC: {what} must be a tensor")
    if not t.is_cuda:
        raise RuntimeError(f"RAC: {what} must be a GPU tensor (the gfx950 kernels have no CPU path)")


def _require_f32(t: torch.Tensor, what: str = "input") -> None:
    _require_gpu(t, what)
    if t.dtype != torch.float32:
        raise RuntimeError("RAC: float32 only")


def _gemm(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor, M: int, N: int, K: int,
          ta: int, tb: int, iters: int, mode: int, alpha: float = 1.0, beta: float = 0.0) -> None:
    lib = _lib.load()
    rc = lib.rac_gemm_dev(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, ta, tb,
                          alpha, beta, iters, mode, _stream(C))
    check(rc, "rac_gemm_dev")


def _bias_f32(bias: torch.Tensor, n: int) -> torch.Tensor:
    _require_f32(bias, "bias")
    if bias.numel() != n:
        raise RuntimeError("RAC: bias must have out_features elements")
    return bias.contiguous()


def _fused(x2: torch.Tensor, w: torch.Tensor, bias: Optional[torch.Tensor], out: torch.Tensor,
           pre: Optional[torch.Tensor], M: int, N: int, K: int, act: int, iters: int, mode: int) -> None:
    check(_lib.load().rac_fused_linear_dev(x2.data_ptr(), w.data_ptr(),
                                           bias.data_ptr() if bias is not None else None, out.data_ptr(),
                                           pre.data_ptr() if pre is not None else None, M, N, K, act,
                                           iters, mode, _stream(out)),
          "rac_fused_linear_dev")


# ── reference surface (rac_torch_bind.cpp:68-199) ─────────────────────────

def matmul_forward(A: torch.Tensor, B: torch.Tensor, iters: int = 0, mode: int = -1) -> torch.Tensor:
    """C = A @ B (rac_torch_bind.cpp:68-88): GPU fp32 2-D tensors."""
    _require_gpu(A, "A")
    _require_gpu(B, "B")
    if A.dtype != torch.float32:
        raise RuntimeError("RAC: float32 only")
    if A.dim() != 2 or B.dim() != 2:
        raise RuntimeError("RAC: 2D tensors required")
    if A.size(1) != B.size(0):
        raise RuntimeError("RAC: dimension mismatch")
    A = A.contiguous()
    B = B.contiguous().to(torch.float32)
    M, K = A.shape
    N = B.size(1)
    C = torch.empty((M, N), device=A.device, dtype=torch.float32)
    iters, mode = _resolve(iters, mode)
    _gemm(A, B, C, M, N, K, 0, 0, iters, mode)
    return C


def matmul_backward(grad_C: torch.Tensor, A: torch.Tensor, B: torch.Tensor,
                    need_grad_A: bool = True, need_grad_B: bool = True,
                    iters: int = 0, mode: int = -1) -> List[Optional[torch.Tensor]]:
    """grad_A = grad_C @ B^T (NT), grad_B = A^T @ grad_C (TN)
    (rac_torch_bind.cpp:130-163)."""
    grad_C = grad_C.contiguous()
    A = A.contiguous()
    B = B.contiguous()
    for t, n in ((grad_C, "grad_C"), (A, "A"), (B, "B")):
        _require_f32(t, n)
    M, K = A.shape
    N = B.size(1)
    iters, mode = _resolve(iters, mode)
    grad_A = grad_B = None
    if need_grad_A:
        grad_A = torch.empty((M, K), device=A.device, dtype=A.dtype)
        _gemm(grad_C, B, grad_A, M, K, N, 0, 1, iters, mode)
    if need_grad_B:
        grad_B = torch.empty((K, N), device=B.device, dtype=B.dtype)
        _gemm(A, grad_C, grad_B, K, N, M, 1, 0, iters, mode)
    return [grad_A, grad_B]


def linear_forward(input: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor,
                   iters: int = 0, mode: int = -1) -> torch.Tensor:
    """output = input @ weight^T + bias with the NT kernel
    (rac_torch_bind.cpp:90-128): fp16/bf16 promoted to fp32 and cast back;
    an empty bias tensor means no bias."""
    _require_gpu(input, "input")
    orig_dtype = input.dtype
    if orig_dtype != torch.float32:
        input = input.to(torch.float32)
        weight = weight.to(torch.float32)
        if bias is not None and bias.numel() > 0:
            bias = bias.to(torch.float32)
    in_shape = list(input.shape)
    out_features, in_features = weight.shape
    if in_shape[-1] != in_features:
        raise RuntimeError("RAC: dimension mismatch")
    x2 = input.reshape(-1, in_features).contiguous()
    w = weight.contiguous()
    _require_f32(w, "weight")
    M = x2.size(0)
    out = torch.empty((M, out_features), device=x2.device, dtype=torch.float32)
    iters, mode = _resolve(iters, mode)
    has_bias = bias is not None and bias.numel() > 0
    if M > 0 and in_features == 0:
        out.zero_()
        if has_bias:
            out.add_(bias)
    elif M > 0 and has_bias:
        # bias added in the GEMM epilogue (same rounding as a separate add)
        _fused(x2, w, _bias_f32(bias, out_features), out, None, M, out_features, in_features, 0, iters, mode)
    elif M > 0:
        _gemm(x2, w, out, M, out_features, in_features, 0, 1, iters, mode)
    in_shape[-1] = out_features
    res = out.reshape(in_shape)
    if orig_dtype != torch.float32:
        res = res.to(orig_dtype)
    return res


def linear_backward(grad_output: torch.Tensor, input: torch.Tensor, weight: torch.Tensor,
                    need_bias_grad: bool, iters: int = 0, mode: int = -1) -> List[Optional[torch.Tensor]]:
    """grad_input = go @ W (NN), grad_weight = go^T @ inp (TN), grad_bias =
    go.sum(0) (rac_torch_bind.cpp:165-199)."""
    out_features, in_features = weight.shape
    iters, mode = _resolve(iters, mode)
    go = grad_output.reshape(-1, out_features).contiguous().to(torch.float32)
    inp = input.reshape(-1, in_features).contiguous().to(torch.float32)
    w = weight.contiguous().to(torch.float32)
    for t, n in ((go, "grad_output"), (inp, "input"), (w, "weight")):
        _require_f32(t, n)
    M = inp.size(0)
    grad_input = torch.empty((M, in_features), device=inp.device, dtype=torch.float32)
    grad_weight = torch.empty((out_features, in_features), device=w.device, dtype=torch.float32)
    if M > 0:
        _gemm(go, w, grad_input, M, in_features, out_features, 0, 0, iters, mode)
        _gemm(go, inp, grad_weight, out_features, in_features, M, 1, 0, iters, mode)
    else:
        grad_weight.zero_()
    grad_bias = go.sum(0) if need_bias_grad else None
    shape = list(input.shape)
    shape[-1] = in_features
    return [grad_input.reshape(shape), grad_weight, grad_bias]


def fused_linear_forward(input: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, act: int = 0,
                         iters: int = 0, mode: int = -1, return_pre: bool = False):
    """output = act(input @ weight^T + bias) in one kernel (rac_torch.cu:1037-1083):
    act 0 none, 1 ReLU, 2 GELU, 3 SiLU (CORDIC exp).  fp16/bf16 promoted to
    fp32 and cast back; an empty bias tensor means no bias.  With
    return_pre, also returns the fp32 pre-activation written by the same
    kernel (the reference recomputes it with a second matmul)."""
    _require_gpu(input, "input")
    if not 0 <= int(act) <= 3:
        raise RuntimeError("RAC: act must be 0(none), 1(relu), 2(gelu), 3(silu)")
    orig_dtype = input.dtype
    if orig_dtype != torch.float32:
        input = input.to(torch.float32)
        weight = weight.to(torch.float32)
        if bias is not None and bias.numel() > 0:
            bias = bias.to(torch.float32)
    in_shape = list(input.shape)
    out_features, in_features = weight.shape
    if in_shape[-1] != in_features:
        raise RuntimeError("RAC: dimension mismatch")
    x2 = input.reshape(-1, in_features).contiguous()
    w = weight.contiguous()
    _require_f32(w, "weight")
    M = x2.size(0)
    b = _bias_f32(bias, out_features) if bias is not None and bias.numel() > 0 else None
    out = torch.empty((M, out_features), device=x2.device, dtype=torch.float32)
    pre = torch.empty_like(out) if return_pre else None
    iters, mode = _resolve(iters, mode)
    if M > 0:
        if in_features == 0:
            # no products: pre = bias (or 0), out = act(pre)
            p0 = torch.zeros_like(out) if b is None else b.expand(M, out_features).contiguous()
            if pre is not None:
                pre.copy_(p0)
            act = int(act)
            out.copy_(relu(p0) if act == 1 else gelu(p0) if act == 2 else silu(p0, iters) if act == 3 else p0)
        else:
            _fused(x2, w, b, out, pre, M, out_features, in_features, int(act), iters, mode)
    in_shape[-1] = out_features
    res = out.reshape(in_shape)
    if orig_dtype != torch.float32:
        res = res.to(orig_dtype)
    if return_pre:
        return res, pre.reshape(in_shape)
    return res


def fused_linear_backward(grad_output: torch.Tensor, input: torch.Tensor, weight: torch.Tensor,
                          bias: torch.Tensor, pre_act: torch.Tensor, act: int, need_bias_grad: bool,
                          iters: int = 0, mode: int = -1) -> List[Optional[torch.Tensor]]:
    """(rac_torch.cu:1085-1185) d = grad * act'(pre_act) in one elementwise
    kernel, then grad_input = d @ W (NN), grad_weight = d^T @ input (TN),
    grad_bias = d.sum(0)."""
    _require_gpu(grad_output, "grad_output")
    if not 0 <= int(act) <= 3:
        raise RuntimeError("RAC: act must be 0(none), 1(relu), 2(gelu), 3(silu)")
    orig_dtype = grad_output.dtype
    go = grad_output.to(torch.float32).reshape(-1, weight.size(0)).contiguous()
    pre = pre_act.to(torch.float32).reshape(-1, weight.size(0)).contiguous()
    iters, mode = _resolve(iters, mode)
    if int(act) > 0:
        d = torch.empty_like(go)
        if go.numel():
            check(_lib.load().rac_act_grad_dev(go.data_ptr(), pre.data_ptr(), d.data_ptr(), go.numel(),
                                               int(act), iters, _stream(d)), "rac_act_grad_dev")
    else:
        d = go
    gi, gw, gb = linear_backward(d.reshape(*grad_output.shape[:-1], weight.size(0)), input.to(torch.float32),
                                 weight.to(torch.float32), need_bias_grad, iters, mode)
    if orig_dtype != torch.float32:
        gi = gi.to(orig_dtype)
        gw = gw.to(orig_dtype)
        if gb is not None:
            gb = gb.to(orig_dtype)
    return [gi, gw, gb]


def act_grad(grad: torch.Tensor, pre: torch.Tensor, act: int, iters: int = 0) -> torch.Tensor:
    """grad * act'(pre) elementwise (rac_torch.cu:680-694)."""
    _require_f32(grad, "grad")
    _require_f32(pre, "pre")
    g = grad.contiguous()
    p = pre.contiguous()
    if g.shape != p.shape:
        raise RuntimeError("RAC: grad and pre must have the same shape")
    d = torch.empty_like(g)
    if g.numel():
        check(_lib.load().rac_act_grad_dev(g.data_ptr(), p.data_ptr(), d.data_ptr(), g.numel(), int(act),
                                           _resolve_iters(iters), _stream(d)), "rac_act_grad_dev")
    return d


# ── transformer primitives on the gfx950 kernels ──────────────────────────

def _rows(x: torch.Tensor, what: str) -> Tuple[torch.Tensor, int, int]:
    _require_f32(x, what)
    x = x.contiguous()
    n = x.size(-1) if x.dim() > 0 else 1
    rows = x.numel() // n if n > 0 else 0
    return x, rows, n


def softmax(x: torch.Tensor, iters: int = 0) -> torch.Tensor:
    """Row softmax over the last dim with the n-step hyperbolic-CORDIC exp
    (rac_cpu.c:258-271 structure)."""
    x, rows, n = _rows(x, "x")
    y = torch.empty_like(x)
    if rows > 0 and n > 0:
        check(_lib.load().rac_softmax_dev(x.data_ptr(), y.data_ptr(), rows, n,
                                          _resolve_iters(iters), _stream(x)), "rac_softmax_dev")
    return y


def rmsnorm(x: torch.Tensor, weight: Optional[torch.Tensor], eps: float) -> torch.Tensor:
    """y = (x * rsqrt(mean(x^2) + eps)) * weight over the last dim
    (rac_cpu.c:548-574), rsqrt by hyperbolic vectoring."""
    x, rows, d = _rows(x, "x")
    if weight is not None:
        _require_f32(weight, "weight")
        weight = weight.contiguous()
        if weight.numel() != d:
            raise RuntimeError("RAC: weight must have the size of the last dim")
    y = torch.empty_like(x)
    if rows > 0:
        check(_lib.load().rac_rmsnorm_dev(x.data_ptr(), y.data_ptr(),
                                          weight.data_ptr() if weight is not None else None,
                                          float(eps), rows, d, _stream(x)), "rac_rmsnorm_dev")
    return y


def layernorm(x: torch.Tensor, weight: Optional[torch.Tensor], bias: Optional[torch.Tensor],
              eps: float) -> torch.Tensor:
    """y = weight * (x - mean) * rsqrt(var + eps) + bias (rac_cpu.c:507-546)."""
    x, rows, d = _rows(x, "x")
    ptrs = []
    for t, n in ((weight, "weight"), (bias, "bias")):
        if t is not None:
            _require_f32(t, n)
            if t.numel() != d:
                raise RuntimeError(f"RAC: {n} must have the size of the last dim")
            t = t.contiguous()
        ptrs.append(t)
    y = torch.empty_like(x)
    if rows > 0:
        check(_lib.load().rac_layernorm_dev(
            x.data_ptr(), y.data_ptr(),
            ptrs[0].data_ptr() if ptrs[0] is not None else None,
            ptrs[1].data_ptr() if ptrs[1] is not None else None,
            float(eps), rows, d, _stream(x)), "rac_layernorm_dev")
    return y


def _elementwise(name: str, x: torch.Tensor, iters: Optional[int]) -> torch.Tensor:
    _require_f32(x, "x")
    x = x.contiguous()
    y = torch.empty_like(x)
    n = x.numel()
    if n:
        fn = getattr(_lib.load(), name)
        if iters is None:
            rc = fn(x.data_ptr(), y.data_ptr(), n, _stream(x))
        else:
            rc = fn(x.data_ptr(), y.data_ptr(), n, _resolve_iters(iters), _stream(x))
        check(rc, name)
    return y


def exp(x: torch.Tensor, iters: int = 0) -> torch.Tensor:
    return _elementwise("rac_exp_dev", x, iters)


def silu(x: torch.Tensor, iters: int = 0) -> torch.Tensor:
    """x / (1 + e^-x), e^-x by the n-step CORDIC (rac_cpu.c:453-457)."""
    return _elementwise("rac_silu_dev", x, iters)


def sigmoid(x: torch.Tensor, iters: int = 0) -> torch.Tensor:
    return _elementwise("rac_sigmoid_dev", x, iters)


def tanh(x: torch.Tensor, iters: int = 0) -> torch.Tensor:
    return _elementwise("rac_tanh_dev", x, iters)


def gelu(x: torch.Tensor) -> torch.Tensor:
    """x * 0.5 * (1 + erf(x / sqrt 2)) (rac_cpu.c:447-451)."""
    return _elementwise("rac_gelu_dev", x, None)


def relu(x: torch.Tensor) -> torch.Tensor:
    return _elementwise("rac_relu_dev", x, None)


def rsqrt(x: torch.Tensor) -> torch.Tensor:
    return _elementwise("rac_rsqrt_dev", x, None)


def sincos(theta: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(sin, cos) by one 16-step circular CORDIC rotation of (K_INV, 0)
    (rac_cpu.c:322-328)."""
    _require_f32(theta, "theta")
    theta = theta.contiguous()
    s = torch.empty_like(theta)
    c = torch.empty_like(theta)
    if theta.numel():
        check(_lib.load().rac_sincos_dev(theta.data_ptr(), s.data_ptr(), c.data_ptr(),
                                         theta.numel(), _stream(theta)), "rac_sincos_dev")
    return s, c


def rope_inv_freq(head_dim: int, base: float = 10000.0) -> torch.Tensor:
    """inv_freq[i] = 1/powf(base, 2i/head_dim), computed on the host by the
    library exactly as rac_cpu.c:588-589 (a CPU tensor of head_dim/2)."""
    if head_dim <= 0 or head_dim % 2:
        raise RuntimeError("RAC: head_dim must be even and > 0")
    out = torch.empty(head_dim // 2, dtype=torch.float32)
    check(_lib.load().rac_rope_inv_freq(out.data_ptr(), head_dim, float(base)), "rac_rope_inv_freq")
    return out


def rope_cache(max_seq: int, head_dim: int, base: float = 10000.0,
               device: Optional[torch.device] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """cos/sin tables [max_seq, head_dim/2] by circular CORDIC
    (rac_cpu.c:576-598), bit-exact with the reference table."""
    device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    if device.type != "cuda":
        raise RuntimeError("RAC: rope_cache builds its tables on a GPU device")
    if max_seq <= 0 or head_dim <= 0 or head_dim % 2:
        raise RuntimeError("RAC: max_seq > 0 and even head_dim > 0 required")
    half = head_dim // 2
    inv = rope_inv_freq(head_dim, base).to(device)
    cos = torch.empty((max_seq, half), device=device, dtype=torch.float32)
    sin = torch.empty((max_seq, half), device=device, dtype=torch.float32)
    check(_lib.load().rac_rope_cache_dev(cos.data_ptr(), sin.data_ptr(), max_seq, head_dim,
                                         float(base), inv.data_ptr(), _stream(cos)),
          "rac_rope_cache_dev")
    return cos, sin


def rope_apply_(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """In-place Givens rotation of x[b, h, t, 2i:2i+2] by (cos[t,i], sin[t,i])
    (rac_cpu.c:600-635).  x is a [B, H, T, D] tensor whose last dim is
    contiguous; the other dims may be strided (e.g. the transposed
    [B, T, H, D] projection view).  cos/sin: [>= T, D/2] contiguous."""
    _require_f32(x, "x")
    if x.dim() != 4:
        raise RuntimeError("RAC: rope_apply_ expects [batch, heads, seq, head_dim]")
    if x.stride(-1) != 1:
        raise RuntimeError("RAC: rope_apply_ needs a contiguous last dim")
    B, H, T, D = x.shape
    if D % 2:
        raise RuntimeError("RAC: head_dim must be even")
    for t, n in ((cos, "cos"), (sin, "sin")):
        _require_f32(t, n)
        if not t.is_contiguous() or t.dim() != 2 or t.size(1) != D // 2 or t.size(0) < T:
            raise RuntimeError(f"RAC: {n} must be a contiguous [>= seq, head_dim/2] table")
    if x.numel() == 0:
        return x
    check(_lib.load().rac_rope_apply_dev(x.data_ptr(), cos.data_ptr(), sin.data_ptr(), B, H, T, D,
                                         x.stride(0), x.stride(1), x.stride(2), _stream(x)),
          "rac_rope_apply_dev")
    return x


def rope_apply(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Out-of-place rope_apply_: returns a new contiguous [B, H, T, D] tensor
    holding x rotated (x itself, whose last dim must be contiguous and whose
    other dims may be strided, is only read): one read and one write per
    element."""
    _require_f32(x, "x")
    if x.dim() != 4:
        raise RuntimeError("RAC: rope_apply expects [batch, heads, seq, head_dim]")
    if x.stride(-1) != 1:
        raise RuntimeError("RAC: rope_apply needs a contiguous last dim")
    B, H, T, D = x.shape
    if D % 2:
        raise RuntimeError("RAC: head_dim must be even")
    for t, n in ((cos, "cos"), (sin, "sin")):
        _require_f32(t, n)
        if not t.is_contiguous() or t.dim() != 2 or t.size(1) != D // 2 or t.size(0) < T:
            raise RuntimeError(f"RAC: {n} must be a contiguous [>= seq, head_dim/2] table")
    y = torch.empty((B, H, T, D), device=x.device, dtype=torch.float32)
    if x.numel() == 0:
        return y
    check(_lib.load().rac_rope_apply_out_dev(x.data_ptr(), y.data_ptr(), cos.data_ptr(), sin.data_ptr(), B, H, T,
                                             D, x.stride(0), x.stride(1), x.stride(2), y.stride(0), y.stride(1),
                                             y.stride(2), _stream(y)),
          "rac_rope_apply_out_dev")
    return y


# ── batched products and attention ───────────────────────────────────────

def _rows_contiguous(t: torch.Tensor) -> torch.Tensor:
    """t [Z, R, C] unchanged when every t[z] is a row-major R x C matrix
    (stride(2) == 1, stride(1) == C) and the batch stride is non-negative;
    a contiguous copy otherwise."""
    if ((t.size(2) <= 1 or t.stride(2) == 1) and (t.size(1) <= 1 or t.stride(1) == t.size(2))
            and t.stride(0) >= 0):
        return t
    return t.contiguous()


def bmm(A: torch.Tensor, B: torch.Tensor, trans_a: bool = False, trans_b: bool = False,
        alpha: float = 1.0, iters: int = 0, mode: int = -1, out: Optional[torch.Tensor] = None,
        beta: float = 0.0) -> torch.Tensor:
    """C[z] = alpha * op(A[z]) @ op(B[z]) (+ beta * C[z]) for 3-D fp32
    tensors whose items are row-major matrices (items may be strided apart,
    e.g. a slice of a cache), one launch over the batch (grid z).  op(A[z]) = A[z]
    [M, K], or A[z]^T with A stored [Z, K, M] when trans_a; op(B[z]) = B[z]
    [K, N], or B[z]^T with B stored [Z, N, K] when trans_b.  With `out`
    (a contiguous fp32 [Z, M, N] tensor) the result is written there, and
    beta != 0 accumulates into its contents: fma(alpha, acc, beta * C)."""
    _require_f32(A, "A")
    _require_f32(B, "B")
    if A.dim() != 3 or B.dim() != 3 or A.size(0) != B.size(0):
        raise RuntimeError("RAC: bmm expects [Z, ., .] tensors with the same Z")
    # each batch item must be a row-major matrix; items may sit any
    # (non-negative) distance apart, e.g. a slice of a longer cache
    A = _rows_contiguous(A)
    B = _rows_contiguous(B)
    Z = A.size(0)
    M, K = (A.size(2), A.size(1)) if trans_a else (A.size(1), A.size(2))
    Kb, N = (B.size(2), B.size(1)) if trans_b else (B.size(1), B.size(2))
    if K != Kb:
        raise RuntimeError("RAC: dimension mismatch")
    if out is not None:
        _require_f32(out, "out")
        if tuple(out.shape) != (Z, M, N) or not out.is_contiguous():
            raise RuntimeError("RAC: bmm out must be a contiguous [Z, M, N] tensor")
        C = out
    else:
        if beta != 0.0:
            raise RuntimeError("RAC: bmm beta needs an out tensor to accumulate into")
        C = torch.empty((Z, M, N), device=A.device, dtype=torch.float32)
    if C.numel() == 0:
        return C
    if K == 0:
        return C.mul_(beta) if beta != 0.0 else C.zero_()
    iters, mode = _resolve(iters, mode)
    lib = _lib.load()
    for z0 in range(0, Z, 65535):
        zb = min(65535, Z - z0)
        check(lib.rac_gemm_batched_dev(A[z0].data_ptr(), B[z0].data_ptr(), C[z0].data_ptr(), M, N, K,
                                       int(trans_a), int(trans_b), float(alpha), float(beta), iters, mode, zb,
                                       A.stride(0), B.stride(0), C.stride(0), _stream(C)),
              "rac_gemm_batched_dev")
    return C


def softmax_masked_(scores: torch.Tensor, mask: Optional[torch.Tensor] = None, is_causal: bool = False,
                    iters: int = 0) -> torch.Tensor:
    """In-place attention softmax of contiguous scores [..., T, T]:
    causal -inf above the diagonal, then + mask[T, T], then the CORDIC
    softmax of each row (rac_cpu.c:664-687)."""
    _require_f32(scores, "scores")
    if not scores.is_contiguous() or scores.dim() < 2 or scores.size(-1) != scores.size(-2):
        raise RuntimeError("RAC: scores must be a contiguous [..., T, T] tensor")
    T = scores.size(-1)
    mptr = None
    if mask is not None:
        _require_f32(mask, "mask")
        if mask.shape != (T, T) or not mask.is_contiguous():
            raise RuntimeError("RAC: mask must be a contiguous [T, T] float32 tensor")
        mptr = mask.data_ptr()
    if scores.numel():
        check(_lib.load().rac_softmax_masked_dev(scores.data_ptr(), scores.data_ptr(), scores.numel() // T, T,
                                                 mptr, int(bool(is_causal)), _resolve_iters(iters),
                                                 _stream(scores)),
              "rac_softmax_masked_dev")
    return scores


def attention_scale(head_dim: int) -> float:
    """1.0f / sqrtf((float)head_dim) in float32 arithmetic (rac_cpu.c:652)."""
    return float(np.float32(1.0) / np.sqrt(np.float32(head_dim)))


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask: Optional[torch.Tensor] = None,
              is_causal: bool = False, iters: int = 0, mode: int = -1,
              return_probs: bool = False):
    """rac_attention (rac.h:323-335) on [B, H, T, D] tensors through
    rac_attention_dev: scores = Q K^T / sqrt(D) by the RAC matmul,
    causal/additive [T, T] mask, CORDIC softmax, out = P V by the RAC
    matmul.  With return_probs, also returns P [B, H, T, T] (what the
    backward pass needs)."""
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _require_f32(t, n)
        if t.dim() != 4:
            raise RuntimeError("RAC: attention expects [batch, heads, seq, head_dim]")
    if q.shape != k.shape or q.shape != v.shape:
        raise RuntimeError("RAC: q, k, v must have the same shape")
    B, H, T, D = q.shape
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    iters, mode = _resolve(iters, mode)
    mptr = None
    if mask is not None:
        _require_f32(mask, "mask")
        if tuple(mask.shape) != (T, T):
            raise RuntimeError("RAC: attention mask must be [T, T]")
        mask = mask.contiguous()
        mptr = mask.data_ptr()
    out = torch.empty_like(q)
    lib = _lib.load()
    if return_probs:
        # one chunk: the workspace keeps every probability for the backward pass
        ws = torch.empty(lib.rac_attention_probs_workspace_bytes(B, H, T) // 4, device=q.device,
                         dtype=torch.float32)
        check(lib.rac_attention_probs_dev(q.data_ptr(), k.data_ptr(), v.data_ptr(), mptr, int(bool(is_causal)),
                                          out.data_ptr(), B, H, T, D, ws.data_ptr(), iters, mode, _stream(out)),
              "rac_attention_probs_dev")
        return out, ws[:B * H * T * T].view(B, H, T, T)
    # chunks of query rows: the workspace holds one chunk's scores
    ws = torch.empty(lib.rac_attention_workspace_bytes(B, H, T) // 4, device=q.device, dtype=torch.float32)
    check(lib.rac_attention_dev(q.data_ptr(), k.data_ptr(), v.data_ptr(), mptr, int(bool(is_causal)),
                                out.data_ptr(), B, H, T, D, ws.data_ptr(), iters, mode, _stream(out)),
          "rac_attention_dev")
    return out


def attention_probs_rows(q: torch.Tensor, k: torch.Tensor, mask: Optional[torch.Tensor], is_causal: bool,
                         row0: int, rows: int, iters: int = 0, mode: int = -1) -> torch.Tensor:
    """The attention probabilities of query rows row0 .. row0+rows-1 of every
    head, [B, H, rows, T], through rac_attention_probs_rows_dev: bit for bit
    those rows of the P that attention(..., return_probs=True) returns."""
    for t, n in ((q, "q"), (k, "k")):
        _require_f32(t, n)
        if t.dim() != 4:
            raise RuntimeError("RAC: attention expects [batch, heads, seq, head_dim]")
    if q.shape != k.shape:
        raise RuntimeError("RAC: q and k must have the same shape")
    B, H, T, D = q.shape
    q, k = q.contiguous(), k.contiguous()
    iters, mode = _resolve(iters, mode)
    mptr = None
    if mask is not None:
        _require_f32(mask, "mask")
        if tuple(mask.shape) != (T, T):
            raise RuntimeError("RAC: attention mask must be [T, T]")
        mask = mask.contiguous()
        mptr = mask.data_ptr()
    P = torch.empty((B, H, rows, T), device=q.device, dtype=torch.float32)
    check(_lib.load().rac_attention_probs_rows_dev(q.data_ptr(), k.data_ptr(), mptr, int(bool(is_causal)),
                                                   P.data_ptr(), B, H, T, D, int(row0), int(rows), iters, mode,
                                                   _stream(P)),
          "rac_attention_probs_rows_dev")
    return P


# ── vector primitives (rac.h:101-250) ───────────────────────────────────────

VEC2_OPS = {
    "rotate": 0, "rotate_raw": 1, "compensate": 2, "project": 3, "polar": 4, "normalize": 5,
    "dot": 6, "coherence": 7, "complex_mul": 8, "rotate_precision": 9, "project_precision": 10,
    "inner_term": 11,
}
_PAIR_OUT = {"rotate", "rotate_raw", "compensate", "polar", "normalize", "complex_mul", "rotate_precision"}


def vec2(op: str, a: torch.Tensor, b: Optional[torch.Tensor] = None, theta: Optional[torch.Tensor] = None,
         iarg: int = 0) -> torch.Tensor:
    """Elementwise rac.h primitive over pairs a [n, 2] (b [n, 2], theta [n]);
    returns [n, 2] for pair-valued ops, [n] otherwise."""
    code = VEC2_OPS[op]
    _require_f32(a, "a")
    a = a.contiguous()
    if a.dim() != 2 or a.size(1) != 2:
        raise RuntimeError("RAC: pairs must be [n, 2]")
    n = a.size(0)
    ptrs = []
    for t, name in ((b, "b"), (theta, "theta")):
        if t is None:
            ptrs.append(None)
            continue
        _require_f32(t, name)
        t = t.contiguous()
        if t.numel() != (2 * n if name == "b" else n):
            raise RuntimeError(f"RAC: {name} has the wrong length")
        ptrs.append(t)
    out = torch.empty((n, 2) if op in _PAIR_OUT else (n,), device=a.device, dtype=torch.float32)
    o2 = out.data_ptr() if op in _PAIR_OUT else None
    o1 = None if op in _PAIR_OUT else out.data_ptr()
    check(_lib.load().rac_vec2_dev(code, n, a.data_ptr(), ptrs[0].data_ptr() if ptrs[0] is not None else None,
                                   ptrs[1].data_ptr() if ptrs[1] is not None else None, int(iarg), o2, o1,
                                   _stream(out)), "rac_vec2_dev")
    return out


def inner(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """rac_inner (rac.h:233): sum_i project(a[i], angle b[i]) |b[i]|, a 0-d tensor."""
    _require_f32(a, "a")
    _require_f32(b, "b")
    a = a.contiguous()
    b = b.contiguous()
    if a.shape != b.shape or a.dim() != 2 or a.size(1) != 2:
        raise RuntimeError("RAC: inner expects two [n, 2] tensors")
    out = torch.empty((), device=a.device, dtype=torch.float32)
    check(_lib.load().rac_inner_dev(a.data_ptr(), b.data_ptr(), a.size(0), out.data_ptr(), _stream(out)),
          "rac_inner_dev")
    return out


def outer(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """rac_outer (rac.h:240): C[i, j] = project(a[i], angle b[j]) |b[j]|."""
    _require_f32(a, "a")
    _require_f32(b, "b")
    a = a.contiguous()
    b = b.contiguous()
    if a.dim() != 2 or b.dim() != 2 or a.size(1) != 2 or b.size(1) != 2:
        raise RuntimeError("RAC: outer expects [m, 2] and [n, 2] tensors")
    C = torch.empty((a.size(0), b.size(0)), device=a.device, dtype=torch.float32)
    check(_lib.load().rac_outer_dev(a.data_ptr(), b.data_ptr(), C.data_ptr(), a.size(0), b.size(0),
                                    _stream(C)), "rac_outer_dev")
    return C


def dct(x: torch.Tensor) -> torch.Tensor:
    """rac_dct (rac.h:189): DCT-II of a 1-D tensor."""
    _require_f32(x, "x")
    x = x.contiguous()
    if x.dim() != 1:
        raise RuntimeError("RAC: dct expects a 1-D tensor")
    X = torch.empty_like(x)
    check(_lib.load().rac_dct_dev(x.data_ptr(), X.data_ptr(), x.numel(), _stream(X)), "rac_dct_dev")
    return X


# ── Q8_0 weights and decode GEMV (lib/c/rac_q8_0.h) ─────────────────────────

Q8_BLOCK_BYTES = 34


def q8_quantize(w: torch.Tensor) -> torch.Tensor:
    """fp32 [rows, K] -> Q8_0 blocks as a uint8 tensor [rows, K/32, 34]
    (rac_q8_0.c:68-100: per-block amax/127 scale in fp16, int8 lrintf)."""
    _require_f32(w, "w")
    if w.dim() != 2 or w.size(1) % 32:
        raise RuntimeError("RAC: q8_quantize expects [rows, K] with K % 32 == 0")
    w = w.contiguous()
    rows, K = w.shape
    out = torch.empty((rows, K // 32, Q8_BLOCK_BYTES), device=w.device, dtype=torch.uint8)
    if rows:
        check(_lib.load().rac_q8_0_quantize_dev(w.data_ptr(), out.data_ptr(), rows, K, _stream(out)),
              "rac_q8_0_quantize_dev")
    return out


def q8_dequantize(wq: torch.Tensor) -> torch.Tensor:
    """Q8_0 blocks [rows, K/32, 34] -> fp32 [rows, K]."""
    _require_gpu(wq, "wq")
    if wq.dtype != torch.uint8 or wq.dim() != 3 or wq.size(2) != Q8_BLOCK_BYTES:
        raise RuntimeError("RAC: Q8_0 weights must be a uint8 [rows, K/32, 34] tensor")
    wq = wq.contiguous()
    rows, nb = wq.shape[0], wq.shape[1]
    out = torch.empty((rows, nb * 32), device=wq.device, dtype=torch.float32)
    if rows and nb:
        check(_lib.load().rac_q8_0_dequantize_dev(wq.data_ptr(), out.data_ptr(), rows, nb * 32, _stream(out)),
              "rac_q8_0_dequantize_dev")
    return out


def q8_gemv(x: torch.Tensor, wq: torch.Tensor, bias: Optional[torch.Tensor] = None, act: int = 0) -> torch.Tensor:
    """out[..., N] = act(x[..., K] @ W^T + bias) with W as Q8_0 blocks
    [N, K/32, 34] (rac_q8_0.c:178-211, bit-identical to its AVX2 build for
    act 0/1).  Leading dims of x are decode rows (the weights stream once
    per 8 rows)."""
    _require_f32(x, "x")
    _require_gpu(wq, "wq")
    if wq.dtype != torch.uint8 or wq.dim() != 3 or wq.size(2) != Q8_BLOCK_BYTES:
        raise RuntimeError("RAC: Q8_0 weights must be a uint8 [N, K/32, 34] tensor")
    N, K = wq.size(0), wq.size(1) * 32
    if x.size(-1) != K:
        raise RuntimeError("RAC: dimension mismatch")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, K).contiguous()
    wq = wq.contiguous()
    b = None
    if bias is not None:
        b = _bias_f32(bias, N)
    out = torch.empty((x2.size(0), N), device=x.device, dtype=torch.float32)
    lib = _lib.load()
    for m0 in range(0, x2.size(0), 4096):
        mm = min(4096, x2.size(0) - m0)
        check(lib.rac_q8_0_gemv_dev(x2[m0].data_ptr(), wq.data_ptr(), b.data_ptr() if b is not None else None,
                                    out[m0].data_ptr(), mm, N, K, int(act), _stream(out)),
              "rac_q8_0_gemv_dev")
    return out.reshape(*lead, N)


# ── decode step (bench_rac_transformer.c decoder_forward_kv, T_new = 1) ──

DECODE_MAX_HEAD = 256
DECODE_MAX_LEN = 8192


def _require_pos(pos: torch.Tensor) -> None:
    _require_gpu(pos, "pos")
    if pos.dtype != torch.int32 or pos.numel() != 1:
        raise RuntimeError("RAC: pos must be a one-element int32 device tensor")


def _require_cache(k_cache: torch.Tensor, v_cache: torch.Tensor) -> Tuple[int, int, int]:
    for t, n in ((k_cache, "k_cache"), (v_cache, "v_cache")):
        _require_f32(t, n)
        if t.dim() != 3 or not t.is_contiguous():
            raise RuntimeError(f"RAC: {n} must be a contiguous [n_kv_heads, t_cap, d_head] tensor")
    if k_cache.shape != v_cache.shape:
        raise RuntimeError("RAC: k_cache and v_cache must have the same shape")
    return tuple(k_cache.shape)


def decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, pos: torch.Tensor,
                     n_heads: int, scale: float, iters: int = 0, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Attention of one token's queries q [n_heads * d_head] over cache
    positions 0 .. pos (pos read on the device when the kernel runs); query
    head h reads key/value head h // (n_heads / n_kv_heads)
    (bench_rac_transformer.c:508-548).  Returns [n_heads * d_head]."""
    _require_f32(q, "q")
    _require_pos(pos)
    nkv, t_cap, dh = _require_cache(k_cache, v_cache)
    if q.numel() != n_heads * dh or not q.is_contiguous():
        raise RuntimeError("RAC: q must be a contiguous n_heads * d_head vector")
    if out is None:
        out = torch.empty(n_heads * dh, device=q.device, dtype=torch.float32)
    elif out.dtype != torch.float32 or out.numel() != n_heads * dh or not out.is_contiguous():
        raise RuntimeError("RAC: out must be a contiguous fp32 n_heads * d_head vector")
    check(_lib.load().rac_decode_attention_dev(q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), out.data_ptr(),
                                               int(n_heads), nkv, dh, t_cap, pos.data_ptr(), float(scale),
                                               _resolve_iters(iters), _stream(q)), "rac_decode_attention_dev")
    return out


def kv_append_(kv: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, pos: torch.Tensor) -> None:
    """Writes kv = [k | v] (2 * n_kv_heads * d_head values, contiguous) at
    cache position pos (read on the device)."""
    _require_f32(kv, "kv")
    _require_pos(pos)
    nkv, t_cap, dh = _require_cache(k_cache, v_cache)
    if kv.numel() != 2 * nkv * dh or not kv.is_contiguous():
        raise RuntimeError("RAC: kv must hold 2 * n_kv_heads * d_head contiguous values")
    check(_lib.load().rac_kv_append_dev(kv.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), nkv, dh, t_cap,
                                        pos.data_ptr(), _stream(kv)), "rac_kv_append_dev")


def position_advance_(pos: torch.Tensor, by: int = 1) -> None:
    """pos += by on the stream."""
    _require_pos(pos)
    check(_lib.load().rac_position_advance_dev(pos.data_ptr(), int(by), _stream(pos)), "rac_position_advance_dev")


def _fused_gemv_ok(x: torch.Tensor, norm_weight: torch.Tensor, wq: torch.Tensor) -> bool:
    K = x.size(-1)
    return (K % 256 == 0 and K <= 16384 and x.is_contiguous() and norm_weight.is_contiguous()
            and wq.is_contiguous() and all(t.data_ptr() % 16 == 0 for t in (x, norm_weight, wq)))


def _require_q8(wq: torch.Tensor, K: int) -> int:
    _require_gpu(wq, "wq")
    if wq.dtype != torch.uint8 or wq.dim() != 3 or wq.size(2) != Q8_BLOCK_BYTES or wq.size(1) * 32 != K:
        raise RuntimeError("RAC: Q8_0 weights must be a uint8 [N, K/32, 34] tensor matching x")
    return wq.size(0)


def q8_gemv_rmsnorm(x: torch.Tensor, norm_weight: torch.Tensor, eps: float, wq: torch.Tensor,
                    bias: Optional[torch.Tensor] = None, act: int = 0) -> torch.Tensor:
    """q8_gemv(rmsnorm(x, norm_weight, eps), wq, bias, act) for one row x
    [1, K] in one launch, with the same bits.  Needs K % 256 == 0, K <=
    16384 and 16-byte aligned contiguous buffers (fused_gemv_ok)."""
    _require_f32(x, "x")
    _require_f32(norm_weight, "norm_weight")
    N = _require_q8(wq, x.size(-1))
    if x.numel() != x.size(-1) or norm_weight.numel() != x.size(-1):
        raise RuntimeError("RAC: q8_gemv_rmsnorm takes one row x and a matching norm_weight")
    b = _bias_f32(bias, N) if bias is not None else None
    out = torch.empty((1, N), device=x.device, dtype=torch.float32)
    check(_lib.load().rac_q8_0_gemv_rmsnorm_dev(x.data_ptr(), norm_weight.data_ptr(), float(eps), wq.data_ptr(),
                                                b.data_ptr() if b is not None else None, out.data_ptr(), N,
                                                x.size(-1), int(act), _stream(x)), "rac_q8_0_gemv_rmsnorm_dev")
    return out


def fused_gemv_ok(x: torch.Tensor, norm_weight: torch.Tensor, wq: torch.Tensor) -> bool:
    """Whether the fused-norm decode GEMVs take these buffers."""
    return _fused_gemv_ok(x, norm_weight, wq)


def decode_qkv(x: torch.Tensor, norm_weight: torch.Tensor, eps: float, wq: torch.Tensor, k_cache: torch.Tensor,
               v_cache: torch.Tensor, n_heads: int, pos: torch.Tensor) -> torch.Tensor:
    """h = rmsnorm(x); the rows of wq (W_q, W_k, W_v stacked) over h: the
    queries are returned [n_heads * d_head], keys and values go into the
    caches at position pos (read on the device)."""
    _require_f32(x, "x")
    _require_f32(norm_weight, "norm_weight")
    _require_pos(pos)
    nkv, t_cap, dh = _require_cache(k_cache, v_cache)
    N = _require_q8(wq, x.size(-1))
    if N != (n_heads + 2 * nkv) * dh:
        raise RuntimeError("RAC: wq must hold (n_heads + 2 n_kv_heads) * d_head rows")
    q = torch.empty(n_heads * dh, device=x.device, dtype=torch.float32)
    check(_lib.load().rac_decode_qkv_dev(x.data_ptr(), norm_weight.data_ptr(), float(eps), wq.data_ptr(),
                                         q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), int(n_heads), nkv,
                                         dh, x.size(-1), t_cap, pos.data_ptr(), _stream(x)), "rac_decode_qkv_dev")
    return q


def q8_interleave_rows(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Rows a_0, b_0, a_1, b_1, ... (the gate / up layout of
    decode_swiglu_gemv); works on fp32 rows or Q8_0 block rows alike."""
    if a.shape != b.shape:
        raise RuntimeError("RAC: interleaved row sets must have the same shape")
    return torch.stack([a, b], 1).reshape(2 * a.size(0), *a.shape[1:]).contiguous()


def decode_swiglu_gemv(x: torch.Tensor, norm_weight: torch.Tensor, eps: float, wq_pairs: torch.Tensor,
                       iters: int = 0) -> torch.Tensor:
    """out[i] = silu(gate_i . h) * (up_i . h), h = rmsnorm(x), for Q8_0
    weights whose rows interleave gate and up (q8_interleave_rows)."""
    _require_f32(x, "x")
    _require_f32(norm_weight, "norm_weight")
    N = _require_q8(wq_pairs, x.size(-1))
    if N % 2:
        raise RuntimeError("RAC: gate / up weights need an even row count")
    out = torch.empty((1, N // 2), device=x.device, dtype=torch.float32)
    check(_lib.load().rac_decode_swiglu_gemv_dev(x.data_ptr(), norm_weight.data_ptr(), float(eps),
                                                 wq_pairs.data_ptr(), out.data_ptr(), N // 2, x.size(-1),
                                                 _resolve_iters(iters), _stream(x)), "rac_decode_swiglu_gemv_dev")
    return out


def swiglu(gu: torch.Tensor, iters: int = 0) -> torch.Tensor:
    """silu(gate) * up for gu = [..., 2 n] holding gate then up in its last
    dim; returns [..., n] (CORDIC SiLU, the bits of silu())."""
    _require_f32(gu, "gu")
    if gu.size(-1) % 2:
        raise RuntimeError("RAC: swiglu expects an even last dim (gate then up)")
    n = gu.size(-1) // 2
    gu = gu.contiguous()
    lead = gu.shape[:-1]
    rows = gu.numel() // (2 * n) if n else 0
    out = torch.empty((*lead, n), device=gu.device, dtype=torch.float32)
    lib = _lib.load()
    g2, o2 = gu.view(rows, 2 * n), out.view(rows, n)
    for r in range(rows):
        check(lib.rac_swiglu_dev(g2[r].data_ptr(), o2[r].data_ptr(), n, _resolve_iters(iters), _stream(gu)),
              "rac_swiglu_dev")
    return out


# ── RAC-DSP fixed-point engine (sim/rac_dsp_core.h) ──────────────────────

DSP_OPS = {"rotate": 0, "project": 1, "vectoring": 2, "hyperbolic": 3}


def _require_i64(t: torch.Tensor, what: str) -> None:
    _require_gpu(t, what)
    if t.dtype != torch.int64:
        raise RuntimeError(f"RAC: {what} must be int64 (Q32.32 / Q0.63 fixed point)")


def dsp_eval(op, x: torch.Tensor, z: torch.Tensor, y: Optional[torch.Tensor] = None
             ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(x, y, z) outputs of the RAC-DSP engine (rac_dsp_core.c:95-149) for
    every element: x, y in Q32.32, z in Q0.63 fractions of pi (int64); y
    defaults to 0.  op: 0..3 or a DSP_OPS name."""
    op = DSP_OPS[op] if isinstance(op, str) else int(op)
    _require_i64(x, "x")
    _require_i64(z, "z")
    if y is not None:
        _require_i64(y, "y")
        if y.shape != x.shape:
            raise RuntimeError("RAC: x, y, z shapes differ")
        y = y.contiguous()
    if z.shape != x.shape:
        raise RuntimeError("RAC: x, y, z shapes differ")
    x, z = x.contiguous(), z.contiguous()
    xo, yo, zo = (torch.empty_like(x) for _ in range(3))
    check(_lib.load().rac_dsp_eval_dev(op, x.numel(), x.data_ptr(), y.data_ptr() if y is not None else None,
                                       z.data_ptr(), xo.data_ptr(), yo.data_ptr(), zo.data_ptr(), _stream(x)),
          "rac_dsp_eval_dev")
    return xo, yo, zo


def dsp_systolic(W: torch.Tensor, X: torch.Tensor) -> torch.Tensor:
    """Weight-stationary systolic product of rac_systolic_ref.c:40-55 for a
    batch of activations: Y[k, c] = sum_r project(X[k, r], 0, W[r, c]).x
    (W [N, N] angles in Q0.63, X [K, N] in Q32.32, wrapping int64 sums)."""
    _require_i64(W, "W")
    _require_i64(X, "X")
    if W.dim() != 2 or W.size(0) != W.size(1) or X.dim() != 2 or X.size(1) != W.size(0):
        raise RuntimeError("RAC: systolic shapes must be W [N, N], X [K, N]")
    W, X = W.contiguous(), X.contiguous()
    Y = torch.empty_like(X)
    check(_lib.load().rac_dsp_systolic_dev(W.size(0), X.size(0), W.data_ptr(), X.data_ptr(), Y.data_ptr(),
                                           _stream(X)), "rac_dsp_systolic_dev")
    return Y


# ── safetensors weights into HBM (bench/safetensors_reader.h) ──────────────

class SafeTensors:
    """A mapped safetensors file whose tensors load straight into device
    memory: `tensor(name)` as fp32 (F32 / F16 / BF16 / F64 widened on the
    GPU, bit-exact with the reference reader's st_to_f32), `q8_0(name)` as
    Q8_0 blocks [rows, K/32, 34] quantized on the GPU in the same pass."""

    def __init__(self, path: str):
        self._lib = _lib.load()
        err = ctypes.create_string_buffer(256)
        self._f = self._lib.st_open(os.fsencode(path), err)
        if not self._f:
            raise RACError(f"st_open({path}): {err.value.decode(errors='replace')}")
        self.path = path

    def close(self) -> None:
        if self._f:
            self._lib.st_close(self._f)
            self._f = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001
            pass

    def _t(self, name: str):
        if not self._f:
            raise RACError("safetensors file is closed")
        t = self._lib.st_find(self._f, name.encode())
        if not t:
            raise KeyError(name)
        return t

    def names(self) -> List[str]:
        f = self._f.contents
        return [f.tensors[i].name.decode() for i in range(f.n_tensors)]

    def shape(self, name: str) -> Tuple[int, ...]:
        t = self._t(name).contents
        return tuple(int(t.shape[k]) for k in range(t.ndim))

    def dtype(self, name: str) -> str:
        return self._lib.st_dtype_name(self._t(name).contents.dtype).decode()

    def tensor(self, name: str, device=None) -> torch.Tensor:
        t = self._t(name)
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        out = torch.empty(self.shape(name), dtype=torch.float32, device=dev)
        if out.numel():
            check(self._lib.rac_st_to_f32_dev(self._f, t, out.data_ptr(), _stream(out)), "rac_st_to_f32_dev")
        return out

    def q8_0(self, name: str, device=None) -> torch.Tensor:
        t = self._t(name)
        shape = self.shape(name)
        if not shape or shape[-1] % 32:
            raise RACError(f"{name}: Q8_0 needs a last dimension that is a multiple of 32 (shape {shape})")
        K = shape[-1]
        rows = 1
        for d in shape[:-1]:
            rows *= d
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        out = torch.empty((rows, K // 32, Q8_BLOCK_BYTES), dtype=torch.uint8, device=dev)
        if out.numel():
            check(self._lib.rac_st_to_q8_0_dev(self._f, t, out.data_ptr(), _stream(out)), "rac_st_to_q8_0_dev")
        return out


__all__ = [
    "MODE_FAST", "MODE_CORDIC", "MODE_SHIFTADD", "RACError",
    "set_cordic_iters", "get_cordic_iters", "set_cordic_mode", "get_cordic_mode",
    "matmul_forward", "matmul_backward", "linear_forward", "linear_backward",
    "softmax", "rmsnorm", "layernorm", "exp", "silu", "sigmoid", "tanh", "gelu", "relu",
    "rsqrt", "sincos", "rope_inv_freq", "rope_cache", "rope_apply_", "rope_apply",
    "bmm", "softmax_masked_", "attention", "attention_probs_rows", "vec2", "inner", "outer", "dct", "VEC2_OPS",
    "fused_linear_forward", "fused_linear_backward", "act_grad", "attention_scale",
    "q8_quantize", "q8_dequantize", "q8_gemv", "Q8_BLOCK_BYTES",
    "dsp_eval", "dsp_systolic", "DSP_OPS", "SafeTensors",
]
