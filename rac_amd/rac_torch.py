"""rac_torch operator surface on the gfx950 kernels.

Same public names, constructor signatures, defaults and knobs as the
reference ``rac_torch`` (rac_torch/rac_torch.py:163-1409): ``RACLinear``,
``FusedRACLinear``, ``RACFusedQKV``, ``RACFusedFFN``, ``RACAttention``,
``RACTransformerBlock``, ``RACRoPE``, ``RACRMSNorm``, ``RACLayerNorm``,
``RACRoPEAttention``, ``RACLlamaBlock``, ``rac_matmul``, ``rac_linear``,
``rac_matmul_adaptive``, ``patch_model``, ``unpatch_model``,
``benchmark_model``, ``rac_info``, ``rac_set_precision``,
``rac_get_precision``, ``rac_set_mode``, ``rac_get_mode``, ``ACT_*``,
``MODE_*``; environment ``RAC_CORDIC_ITERS`` (default 24),
``RAC_CORDIC_MODE`` (default fast), ``RAC_MIN_ELEMENTS``.

Differences by design:
  * every op runs on the gfx950 kernels of librac_amd.so, including RoPE,
    RMSNorm, LayerNorm, softmax and SiLU, which the reference leaves to
    plain torch (rac_torch.py:1132-1343);
  * there is no pure-torch fallback: CPU tensors or a missing library raise;
  * RACRoPE's table is the CORDIC-16 table of rac_rope_cache
    (rac_cpu.c:576-598), not torch cos/sin;
  * backward passes of RoPE, the norms, softmax and the activations are
    written with torch tensor ops on the device (the forward kernels are the
    product; the reference's own backward for these modules is torch
    autograd).
"""
from __future__ import annotations

import os
import warnings
from typing import Optional

import torch
import torch.nn as nn
from torch.autograd import Function

from . import _probe
from . import ext as _rac
from .ext import MODE_CORDIC, MODE_FAST, MODE_SHIFTADD

_FLOAT_TYPES = (torch.float32, torch.float16, torch.bfloat16)

# Start-up probe (rac_torch.py:55-108): library present and loadable, a
# gfx950 device, one 4x4 CORDIC product correct on it.  Each failure warns
# with its own diagnosis; without a device nothing is launched and nothing
# is said (CPU-only imports are legitimate: tests, tooling).
_PROBE = _probe.probe(run_kernel=os.environ.get('RAC_PROBE', '1') != '0')
if not _PROBE.ok and _PROBE.stage != 'no-device':
    warnings.warn(f"RAC start-up probe: {_PROBE.message}", RuntimeWarning, stacklevel=2)


def _rac_available() -> bool:
    """True when the start-up probe passed: the library loads, a gfx950
    device is present and a RAC product ran correctly on it."""
    return _PROBE.ok


def _rac_has(op: str) -> bool:
    return _rac_available() and hasattr(_rac, op)


def _need_gpu(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"RAC: {what} must be on the ROCm device; the gfx950 kernels have no CPU path")
    if not _PROBE.ok and _PROBE.stage != 'no-device':
        raise RuntimeError(f"RAC: {_PROBE.message}")


# ── knobs (rac_torch.py:1017-1118) ─────────────────────────────────────────

_MODE_NAMES = {'fast': MODE_FAST, 'cordic': MODE_CORDIC, 'shiftadd': MODE_SHIFTADD,
               0: MODE_FAST, 1: MODE_CORDIC, 2: MODE_SHIFTADD}


def _resolve_mode(m) -> int:
    if isinstance(m, int):
        return m if m in (0, 1, 2) else MODE_FAST
    if isinstance(m, str) and m.lower() in _MODE_NAMES:
        return _MODE_NAMES[m.lower()]
    raise ValueError(f"Unknown RAC mode: {m}. Use 'fast', 'cordic', or 'shiftadd'.")


_RAC_CORDIC_ITERS = int(os.environ.get('RAC_CORDIC_ITERS', '24'))
_RAC_CORDIC_MODE = _resolve_mode(os.environ.get('RAC_CORDIC_MODE', 'fast'))
_RAC_MIN_ELEMENTS = int(os.environ.get('RAC_MIN_ELEMENTS', '4096'))


def rac_set_precision(iters: int) -> None:
    """Global CORDIC iteration count, clamped to [4, 24]
    (rac_torch.py:1075-1114).  Used by matmul/linear in CORDIC and SHIFTADD
    modes and by the hyperbolic-CORDIC exp inside softmax, SiLU, sigmoid."""
    global _RAC_CORDIC_ITERS
    iters = max(4, min(24, int(iters)))
    _RAC_CORDIC_ITERS = iters
    _rac.set_cordic_iters(iters)


def rac_get_precision() -> int:
    return _RAC_CORDIC_ITERS


def rac_set_mode(mode) -> None:
    """'fast' (sign-XOR FMA), 'cordic' (n micro-rotations per MAC) or
    'shiftadd' (integer shift-add product) for matmul/linear."""
    global _RAC_CORDIC_MODE
    _RAC_CORDIC_MODE = _resolve_mode(mode)
    _rac.set_cordic_mode(_RAC_CORDIC_MODE)


def rac_get_mode() -> int:
    return _RAC_CORDIC_MODE


def _kw():
    return dict(iters=_RAC_CORDIC_ITERS, mode=_RAC_CORDIC_MODE)


# ── torch.library ops: the kernels as torch.compile sees them ──────────────
#
# The autograd Functions call the GEMM kernels through these ops.  Run
# eagerly they launch the kernel on the current stream; under torch.compile,
# tracing with fake tensors uses the shape functions registered beside them
# (a kernel cannot run on a fake tensor), and the compiled program calls the
# kernel.  Optional outputs come back as empty tensors.

Tensor = torch.Tensor


@torch.library.custom_op("rac_amd::matmul", mutates_args=())
def _op_matmul(A: Tensor, B: Tensor, iters: int, mode: int) -> Tensor:
    return _rac.matmul_forward(A, B, iters=iters, mode=mode)


@_op_matmul.register_fake
def _(A, B, iters, mode):
    return A.new_empty((A.shape[0], B.shape[1]), dtype=torch.float32)


@torch.library.custom_op("rac_amd::matmul_backward", mutates_args=())
def _op_matmul_backward(grad_C: Tensor, A: Tensor, B: Tensor, need_a: bool, need_b: bool,
                        iters: int, mode: int) -> tuple[Tensor, Tensor]:
    gA, gB = _rac.matmul_backward(grad_C, A, B, need_a, need_b, iters=iters, mode=mode)
    return (gA if gA is not None else A.new_empty(0)), (gB if gB is not None else B.new_empty(0))


@_op_matmul_backward.register_fake
def _(grad_C, A, B, need_a, need_b, iters, mode):
    return (A.new_empty(A.shape) if need_a else A.new_empty(0)), (B.new_empty(B.shape) if need_b else B.new_empty(0))


def _no_bias(x: Tensor) -> Tensor:
    return x.new_empty(0, dtype=torch.float32)


@torch.library.custom_op("rac_amd::linear", mutates_args=())
def _op_linear(input: Tensor, weight: Tensor, bias: Optional[Tensor], iters: int, mode: int) -> Tensor:
    return _rac.linear_forward(input, weight, bias if bias is not None else _no_bias(input), iters=iters, mode=mode)


@_op_linear.register_fake
def _(input, weight, bias, iters, mode):
    return input.new_empty((*input.shape[:-1], weight.shape[0]))


@torch.library.custom_op("rac_amd::linear_backward", mutates_args=())
def _op_linear_backward(grad_output: Tensor, input: Tensor, weight: Tensor, need_bias_grad: bool,
                        iters: int, mode: int) -> tuple[Tensor, Tensor, Tensor]:
    gi, gw, gb = _rac.linear_backward(grad_output, input, weight, need_bias_grad, iters=iters, mode=mode)
    return gi, gw, (gb if gb is not None else _no_bias(grad_output))


@_op_linear_backward.register_fake
def _(grad_output, input, weight, need_bias_grad, iters, mode):
    out_f, in_f = weight.shape
    f32 = torch.float32
    gb = grad_output.new_empty((out_f,), dtype=f32) if need_bias_grad else grad_output.new_empty(0, dtype=f32)
    return (input.new_empty((*input.shape[:-1], in_f), dtype=f32), weight.new_empty((out_f, in_f), dtype=f32), gb)


@torch.library.custom_op("rac_amd::fused_linear", mutates_args=())
def _op_fused_linear(input: Tensor, weight: Tensor, bias: Optional[Tensor], act: int, need_pre: bool,
                     iters: int, mode: int) -> tuple[Tensor, Tensor]:
    b = bias if bias is not None else _no_bias(input)
    if need_pre:
        out, pre = _rac.fused_linear_forward(input, weight, b, act, return_pre=True, iters=iters, mode=mode)
        return out, pre
    return _rac.fused_linear_forward(input, weight, b, act, iters=iters, mode=mode), _no_bias(input)


@_op_fused_linear.register_fake
def _(input, weight, bias, act, need_pre, iters, mode):
    shape = (*input.shape[:-1], weight.shape[0])
    pre = input.new_empty(shape, dtype=torch.float32) if need_pre else input.new_empty(0, dtype=torch.float32)
    return input.new_empty(shape), pre


@torch.library.custom_op("rac_amd::fused_linear_backward", mutates_args=())
def _op_fused_linear_backward(grad_output: Tensor, input: Tensor, weight: Tensor, bias: Optional[Tensor],
                              pre: Tensor, act: int, need_bias_grad: bool, iters: int,
                              mode: int) -> tuple[Tensor, Tensor, Tensor]:
    b = bias if bias is not None else _no_bias(input)
    gi, gw, gb = _rac.fused_linear_backward(grad_output, input, weight, b, pre, act, need_bias_grad,
                                            iters=iters, mode=mode)
    return gi, gw, (gb if gb is not None else _no_bias(grad_output))


@_op_fused_linear_backward.register_fake
def _(grad_output, input, weight, bias, pre, act, need_bias_grad, iters, mode):
    out_f, in_f = weight.shape
    dt = grad_output.dtype
    gb = grad_output.new_empty((out_f,)) if need_bias_grad else grad_output.new_empty(0, dtype=torch.float32)
    return (grad_output.new_empty((*grad_output.shape[:-1], in_f), dtype=dt),
            grad_output.new_empty((out_f, in_f), dtype=dt), gb)


# ── autograd: matmul / linear (rac_torch.py:163-258) ──────────────────────

class RACMatmulFunction(Function):
    """C = A @ B forward; dA = dC @ B^T (NT), dB = A^T @ dC (TN)."""

    @staticmethod
    def forward(ctx, A, B):
        _need_gpu(A, "A")
        ctx.save_for_backward(A, B)
        dtype = A.dtype
        C = _op_matmul(A.float(), B.float(), _RAC_CORDIC_ITERS, _RAC_CORDIC_MODE)
        return C if dtype == torch.float32 else C.to(dtype)

    @staticmethod
    def backward(ctx, grad_C):
        A, B = ctx.saved_tensors
        need_a, need_b = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        gA, gB = _op_matmul_backward(grad_C.float().contiguous(), A.float(), B.float(), need_a, need_b,
                                     _RAC_CORDIC_ITERS, _RAC_CORDIC_MODE)
        return (gA.to(A.dtype) if need_a else None), (gB.to(B.dtype) if need_b else None)


class RACLinearFunction(Function):
    """output = input @ weight^T + bias; backward through the NN/TN kernels."""

    @staticmethod
    def forward(ctx, input, weight, bias):
        _need_gpu(input, "input")
        ctx.save_for_backward(input, weight, bias)
        ctx.has_bias = bias is not None
        return _op_linear(input, weight, bias, _RAC_CORDIC_ITERS, _RAC_CORDIC_MODE)

    @staticmethod
    def backward(ctx, grad_output):
        input, weight, bias = ctx.saved_tensors
        gi, gw, gb = _op_linear_backward(grad_output.contiguous(), input, weight, ctx.has_bias,
                                         _RAC_CORDIC_ITERS, _RAC_CORDIC_MODE)
        grad_input = gi.to(input.dtype) if ctx.needs_input_grad[0] else None
        grad_weight = gw.to(weight.dtype) if ctx.needs_input_grad[1] else None
        grad_bias = gb.to(bias.dtype) if ctx.has_bias else None
        return grad_input, grad_weight, grad_bias


def rac_matmul(A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
    """Drop-in for torch.matmul / torch.mm on 2-D tensors."""
    return RACMatmulFunction.apply(A, B)


def rac_linear(input: torch.Tensor, weight: torch.Tensor,
               bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Drop-in for F.linear."""
    return RACLinearFunction.apply(input, weight, bias)


class RACLinear(nn.Module):
    """Drop-in nn.Linear (rac_torch.py:288-376): same parameters and init."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True,
                 device=None, dtype=None):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        factory_kwargs = {'device': device, 'dtype': dtype}
        self.weight = nn.Parameter(torch.empty((out_features, in_features), **factory_kwargs))
        if bias:
            self.bias = nn.Parameter(torch.empty(out_features, **factory_kwargs))
        else:
            self.register_parameter('bias', None)
        self.reset_parameters()

    def reset_parameters(self):
        nn.init.kaiming_uniform_(self.weight, a=5 ** 0.5)
        if self.bias is not None:
            fan_in, _ = nn.init._calculate_fan_in_and_fan_out(self.weight)
            bound = 1.0 / (fan_in ** 0.5) if fan_in > 0 else 0
            nn.init.uniform_(self.bias, -bound, bound)

    def forward(self, input: torch.Tensor) -> torch.Tensor:
        return RACLinearFunction.apply(input, self.weight, self.bias)

    @classmethod
    def from_linear(cls, linear: nn.Linear) -> 'RACLinear':
        rac = cls(linear.in_features, linear.out_features, bias=linear.bias is not None,
                  device=linear.weight.device, dtype=linear.weight.dtype)
        with torch.no_grad():
            rac.weight.copy_(linear.weight)
            if linear.bias is not None:
                rac.bias.copy_(linear.bias)
        return rac

    def extra_repr(self) -> str:
        return (f'in_features={self.in_features}, out_features={self.out_features}, '
                f'bias={self.bias is not None}, backend=RAC')


# ── activations (rac_torch.py:381-401) ─────────────────────────────────────

ACT_NONE = 0
ACT_RELU = 1
ACT_GELU = 2
ACT_SILU = 3

_ACT_MAP = {'none': ACT_NONE, None: ACT_NONE, 'relu': ACT_RELU, 'gelu': ACT_GELU,
            'silu': ACT_SILU, 'swish': ACT_SILU}


def _resolve_act(act) -> int:
    if isinstance(act, int):
        return act
    if isinstance(act, str):
        act = act.lower()
    if act in _ACT_MAP:
        return _ACT_MAP[act]
    raise ValueError(f"Unknown activation: {act}. Use 'relu', 'gelu', 'silu', or None.")


def _act_forward(x32: torch.Tensor, act_id: int) -> torch.Tensor:
    if act_id == ACT_RELU:
        return _rac.relu(x32)
    if act_id == ACT_GELU:
        return _rac.gelu(x32)
    if act_id == ACT_SILU:
        return _rac.silu(x32, iters=_RAC_CORDIC_ITERS)
    return x32


def _act_backward(go: torch.Tensor, pa: torch.Tensor, act_id: int) -> torch.Tensor:
    # derivative formulas of rac_torch.py:466-477
    if act_id == ACT_RELU:
        return go * (pa > 0).float()
    if act_id == ACT_GELU:
        cdf = 0.5 * (1.0 + torch.erf(pa * 0.7071067811865))
        pdf = 0.3989422804 * torch.exp(-0.5 * pa * pa)
        return go * (cdf + pa * pdf)
    if act_id == ACT_SILU:
        sig = _rac.sigmoid(pa.contiguous(), iters=_RAC_CORDIC_ITERS)
        return go * (sig * (1.0 + pa * (1.0 - sig)))
    return go


class RACActivationFunction(Function):
    """Elementwise activation on the gfx950 kernels (SiLU by CORDIC exp)."""

    @staticmethod
    def forward(ctx, x, act_id):
        _need_gpu(x, "input")
        ctx.act_id = act_id
        ctx.save_for_backward(x)
        return _act_forward(x.float().contiguous(), act_id).to(x.dtype)

    @staticmethod
    def backward(ctx, go):
        (x,) = ctx.saved_tensors
        return _act_backward(go.float(), x.float(), ctx.act_id).to(x.dtype), None


class RACFusedLinearFunction(Function):
    """output = act(input @ weight^T + bias) (rac_torch.py:405-496) in one
    kernel: bias and activation in the RAC GEMM's epilogue, which also
    writes the pre-activation for backward when gradients are needed.
    Backward: act' in one elementwise kernel, then the NN/TN RAC GEMMs."""

    @staticmethod
    def forward(ctx, input, weight, bias, act_id):
        _need_gpu(input, "input")
        ctx.act_id = act_id
        ctx.has_bias = bias is not None
        need_pre = act_id != ACT_NONE and any(ctx.needs_input_grad[:3])
        out, pre = _op_fused_linear(input, weight, bias, act_id, need_pre, _RAC_CORDIC_ITERS, _RAC_CORDIC_MODE)
        ctx.save_for_backward(input, weight, bias, pre if need_pre else out)
        return out

    @staticmethod
    def backward(ctx, grad_output):
        input, weight, bias, pre = ctx.saved_tensors
        gi, gw, gb = _op_fused_linear_backward(grad_output.contiguous(), input, weight, bias, pre, ctx.act_id,
                                               ctx.has_bias, _RAC_CORDIC_ITERS, _RAC_CORDIC_MODE)
        grad_input = gi.to(input.dtype) if ctx.needs_input_grad[0] else None
        grad_weight = gw.to(weight.dtype) if ctx.needs_input_grad[1] else None
        grad_bias = gb.to(bias.dtype) if ctx.has_bias else None
        return grad_input, grad_weight, grad_bias, None


class FusedRACLinear(nn.Module):
    """Linear + activation (rac_torch.py:506-563)."""

    def __init__(self, in_features, out_features, bias=True, activation='relu',
                 device=None, dtype=None):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.act_id = _resolve_act(activation)
        self.activation = activation
        factory_kwargs = {'device': device, 'dtype': dtype}
        self.weight = nn.Parameter(torch.empty((out_features, in_features), **factory_kwargs))
        if bias:
            self.bias = nn.Parameter(torch.empty(out_features, **factory_kwargs))
        else:
            self.register_parameter('bias', None)
        self.reset_parameters()

    def reset_parameters(self):
        nn.init.kaiming_uniform_(self.weight, a=5 ** 0.5)
        if self.bias is not None:
            fan_in, _ = nn.init._calculate_fan_in_and_fan_out(self.weight)
            bound = 1.0 / (fan_in ** 0.5) if fan_in > 0 else 0
            nn.init.uniform_(self.bias, -bound, bound)

    def forward(self, input):
        return RACFusedLinearFunction.apply(input, self.weight, self.bias, self.act_id)

    @classmethod
    def from_linear_and_act(cls, linear, activation='relu'):
        fused = cls(linear.in_features, linear.out_features, bias=linear.bias is not None,
                    activation=activation, device=linear.weight.device, dtype=linear.weight.dtype)
        with torch.no_grad():
            fused.weight.copy_(linear.weight)
            if linear.bias is not None:
                fused.bias.copy_(linear.bias)
        return fused

    def extra_repr(self):
        return (f'in_features={self.in_features}, out_features={self.out_features}, '
                f'bias={self.bias is not None}, activation={self.activation}, backend=RAC-fused')


def rac_matmul_adaptive(A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
    """RAC for M*N >= RAC_MIN_ELEMENTS, torch.matmul below (rac_torch.py:570-583)."""
    M, K = A.shape
    N = B.shape[1]
    if M * N >= _RAC_MIN_ELEMENTS and A.is_cuda:
        return RACMatmulFunction.apply(A, B)
    return torch.matmul(A, B)


class RACFusedQKV(nn.Module):
    """One [3*d_model, d_model] projection, split into Q, K, V (rac_torch.py:588-626)."""

    def __init__(self, d_model, bias=True, device=None, dtype=None):
        super().__init__()
        self.d_model = d_model
        self.qkv = RACLinear(d_model, 3 * d_model, bias=bias, device=device, dtype=dtype)

    def forward(self, x):
        return self.qkv(x).chunk(3, dim=-1)

    @classmethod
    def from_qkv_linears(cls, q_linear, k_linear, v_linear):
        """One fused module from three d_model -> d_model projections: rows
        [0, d), [d, 2d), [2d, 3d) of the fused weight (and bias) are Q's, K's
        and V's, so chunk(3) in forward hands each projection back."""
        parts = (q_linear, k_linear, v_linear)
        d_model, with_bias = _square_projections("from_qkv_linears", parts)
        ref = q_linear.weight
        fused = cls(d_model, bias=with_bias, device=ref.device, dtype=ref.dtype)
        _load_row_blocks(fused.qkv, parts)
        return fused

    def extra_repr(self):
        return f'd_model={self.d_model}, backend=RAC-fused-QKV'


def _square_projections(who: str, parts) -> tuple:
    """(d_model, has_bias) of projections that all map d_model -> d_model and
    agree on having a bias; ValueError otherwise."""
    d_model = parts[0].in_features
    if any(p.in_features != d_model or p.out_features != d_model for p in parts):
        raise ValueError(f"{who}: every projection must map d_model -> d_model")
    with_bias = parts[0].bias is not None
    if any((p.bias is not None) != with_bias for p in parts):
        raise ValueError(f"{who}: the projections must all have a bias or none")
    return d_model, with_bias


def _load_row_blocks(dst: nn.Module, parts) -> None:
    """dst.weight (and bias) := the parts' weights (biases) stacked by rows in
    order, bit for bit: part i fills rows [i*d, (i+1)*d)."""
    with torch.no_grad():
        row = 0
        for p in parts:
            rows = slice(row, row + p.out_features)
            dst.weight[rows].copy_(p.weight)
            if dst.bias is not None:
                dst.bias[rows].copy_(p.bias)
            row += p.out_features


class RACFusedFFN(nn.Module):
    """fc2(act(fc1(x))) (rac_torch.py:631-655); not a gated SwiGLU."""

    def __init__(self, d_model, ff_dim, activation='gelu', bias=True, device=None, dtype=None):
        super().__init__()
        self.fc1 = FusedRACLinear(d_model, ff_dim, bias=bias, activation=activation,
                                  device=device, dtype=dtype)
        self.fc2 = RACLinear(ff_dim, d_model, bias=bias, device=device, dtype=dtype)

    def forward(self, x):
        return self.fc2(self.fc1(x))

    def extra_repr(self):
        return f'd_model={self.fc2.out_features}, ff_dim={self.fc1.out_features}'


# ── softmax / norms / RoPE on the kernels ──────────────────────────────────

class RACSoftmaxFunction(Function):
    """Last-dim softmax with the hyperbolic-CORDIC exp."""

    @staticmethod
    def forward(ctx, x, iters):
        _need_gpu(x, "scores")
        y = _rac.softmax(x.float().contiguous(), iters=iters)
        ctx.save_for_backward(y)
        return y.to(x.dtype)

    @staticmethod
    def backward(ctx, g):
        (y,) = ctx.saved_tensors
        g = g.float()
        return (y * (g - (g * y).sum(-1, keepdim=True))), None


def rac_softmax(x: torch.Tensor, iters: Optional[int] = None) -> torch.Tensor:
    return RACSoftmaxFunction.apply(x, _RAC_CORDIC_ITERS if iters is None else iters)


def rac_silu(x: torch.Tensor) -> torch.Tensor:
    return RACActivationFunction.apply(x, ACT_SILU)


class RACRMSNormFunction(Function):
    @staticmethod
    def forward(ctx, x, weight, eps):
        _need_gpu(x, "input")
        x32 = x.float().contiguous()
        w32 = weight.float().contiguous() if weight is not None else None
        y = _rac.rmsnorm(x32, w32, eps)
        ctx.save_for_backward(x32, w32)
        ctx.eps = eps
        ctx.has_w = weight is not None
        ctx.wdtype = weight.dtype if weight is not None else None
        return y.to(x.dtype)

    @staticmethod
    def backward(ctx, g):
        x, w = ctx.saved_tensors
        g = g.float()
        d = x.size(-1)
        inv = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + ctx.eps)
        xhat = x * inv
        gw = g * w if w is not None else g
        gx = inv * (gw - xhat * (gw * xhat).sum(-1, keepdim=True) / d)
        gwt = (g * xhat).reshape(-1, d).sum(0).to(ctx.wdtype) if ctx.has_w else None
        return gx, gwt, None


class RACRoPE(nn.Module):
    """Rotary embeddings by circular CORDIC (rac_torch.py:1132-1196).

    The cos/sin cache is rac_rope_cache's CORDIC-16 table (bit-exact with
    rac_cpu.c:576-598), built on the device; ``forward`` applies the Givens
    rotation with the rope kernel.  Shapes: Q, K [batch, n_heads, seq,
    head_dim] (any strides with a contiguous last dim), head_dim even."""

    def __init__(self, head_dim: int, max_seq_len: int = 2048, base: float = 10000.0,
                 device=None, dtype=torch.float32):
        super().__init__()
        assert head_dim % 2 == 0, f"head_dim must be even, got {head_dim}"
        self.head_dim = head_dim
        self.max_seq_len = max_seq_len
        self.base = base
        self._dtype = dtype
        self._tables = {}
        if device is not None and torch.device(device).type == 'cuda':
            self._get_tables(torch.device(device))

    def _get_tables(self, device: torch.device):
        key = (device.type, device.index)
        if key not in self._tables:
            cos, sin = _rac.rope_cache(self.max_seq_len, self.head_dim, self.base, device=device)
            self._tables[key] = (cos, sin, -sin)
        return self._tables[key]

    @property
    def cos_cache(self):
        return self._get_tables(torch.device('cuda', torch.cuda.current_device()))[0]

    @property
    def sin_cache(self):
        return self._get_tables(torch.device('cuda', torch.cuda.current_device()))[1]

    def _apply(self, fn, *args, **kwargs):
        self._tables = {}
        return super()._apply(fn, *args, **kwargs)

    def forward(self, q: torch.Tensor, k: torch.Tensor, positions: Optional[torch.Tensor] = None):
        _need_gpu(q, "q")
        seq = q.shape[-2]
        if seq > self.max_seq_len:
            raise RuntimeError(f"RAC: seq {seq} exceeds max_seq_len {self.max_seq_len}")
        cos, sin, nsin = self._get_tables(q.device)
        if positions is not None:
            positions = positions.to(q.device)
            cos, sin, nsin = cos[positions].contiguous(), sin[positions].contiguous(), nsin[positions].contiguous()
        return _RoPEFunction.apply(q, cos, sin, nsin), _RoPEFunction.apply(k, cos, sin, nsin)

    def extra_repr(self):
        return (f'head_dim={self.head_dim}, max_seq_len={self.max_seq_len}, '
                f'base={self.base}, backend=RAC-CORDIC')


class _RoPEFunction(Function):
    """Rotation of [B, H, T, D] (strided views allowed) into a new tensor:
    one read and one write per element (rac_rope_apply_out_dev)."""

    @staticmethod
    def forward(ctx, x, cos, sin, nsin):
        ctx.save_for_backward(cos, nsin)
        x32 = x if x.dtype == torch.float32 else x.float()
        if x32.stride(-1) != 1:
            x32 = x32.contiguous()
        out = _rac.rope_apply(x32, cos, sin)
        return out if x.dtype == torch.float32 else out.to(x.dtype)

    @staticmethod
    def backward(ctx, g):
        cos, nsin = ctx.saved_tensors
        g32 = g if g.dtype == torch.float32 else g.float()
        if g32.stride(-1) != 1:
            g32 = g32.contiguous()
        gx = _rac.rope_apply(g32, cos, nsin)      # transpose of a rotation: angle -> -angle
        return gx if g.dtype == torch.float32 else gx.to(g.dtype), None, None, None


class RACRMSNorm(nn.Module):
    """y = weight * x / sqrt(mean(x^2) + eps) with CORDIC-vectoring rsqrt
    (rac_torch.py:1205-1234)."""

    def __init__(self, d_model: int, eps: float = 1e-6, device=None, dtype=None):
        super().__init__()
        self.d_model = d_model
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(d_model, device=device, dtype=dtype))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return RACRMSNormFunction.apply(x, self.weight, self.eps)

    def extra_repr(self):
        return f'd_model={self.d_model}, eps={self.eps}, backend=RAC-rsqrt'


class RACLayerNormFunction(Function):
    @staticmethod
    def forward(ctx, x, weight, bias, eps):
        _need_gpu(x, "input")
        x32 = x.float().contiguous()
        w32 = weight.float().contiguous() if weight is not None else None
        b32 = bias.float().contiguous() if bias is not None else None
        y = _rac.layernorm(x32, w32, b32, eps)
        ctx.save_for_backward(x32, w32)
        ctx.eps = eps
        ctx.has_b = bias is not None
        ctx.wdtype = weight.dtype if weight is not None else None
        ctx.bdtype = bias.dtype if bias is not None else None
        return y.to(x.dtype)

    @staticmethod
    def backward(ctx, g):
        x, w = ctx.saved_tensors
        g = g.float()
        d = x.size(-1)
        mean = x.mean(-1, keepdim=True)
        inv = torch.rsqrt((x - mean).pow(2).mean(-1, keepdim=True) + ctx.eps)
        xhat = (x - mean) * inv
        gxh = g * w if w is not None else g
        gx = inv * (gxh - gxh.mean(-1, keepdim=True) - xhat * (gxh * xhat).mean(-1, keepdim=True))
        gw = (g * xhat).reshape(-1, d).sum(0).to(ctx.wdtype) if w is not None else None
        gb = g.reshape(-1, d).sum(0).to(ctx.bdtype) if ctx.has_b else None
        return gx, gw, gb, None


class RACLayerNorm(nn.Module):
    """y = weight * (x - mean) / sqrt(var + eps) + bias (rac_torch.py:1239-1274)."""

    def __init__(self, d_model: int, eps: float = 1e-5, bias: bool = True, device=None, dtype=None):
        super().__init__()
        self.d_model = d_model
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(d_model, device=device, dtype=dtype))
        if bias:
            self.bias = nn.Parameter(torch.zeros(d_model, device=device, dtype=dtype))
        else:
            self.register_parameter('bias', None)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return RACLayerNormFunction.apply(x, self.weight, self.bias, self.eps)

    def extra_repr(self):
        return f'd_model={self.d_model}, eps={self.eps}, backend=RAC-rsqrt'


# ── attention and blocks ───────────────────────────────────────────────────

def _causal_scores(scores: torch.Tensor, T: int) -> torch.Tensor:
    causal = torch.triu(torch.full((T, T), float('-inf'), device=scores.device,
                                   dtype=scores.dtype), diagonal=1)
    return scores + causal


class RACBmmFunction(Function):
    """Batched C[z] = A[z] @ B[z] in one RAC-matmul launch; backward
    dA = dC B^T (NT) and dB = A^T dC (TN), batched the same way."""

    @staticmethod
    def forward(ctx, A, B):
        _need_gpu(A, "A")
        A32 = A.float().contiguous()
        B32 = B.float().contiguous()
        ctx.save_for_backward(A32, B32)
        return _rac.bmm(A32, B32, **_kw()).to(A.dtype)

    @staticmethod
    def backward(ctx, g):
        A, B = ctx.saved_tensors
        g = g.float().contiguous()
        dA = _rac.bmm(g, B, trans_b=True, **_kw()) if ctx.needs_input_grad[0] else None
        dB = _rac.bmm(A, g, trans_a=True, **_kw()) if ctx.needs_input_grad[1] else None
        return dA, dB


def rac_bmm(A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
    """A [..., M, K] @ B [..., K, N] with leading dims flattened into one
    batched RAC-matmul launch."""
    lead = A.shape[:-2]
    out = RACBmmFunction.apply(A.reshape(-1, A.shape[-2], A.shape[-1]),
                               B.reshape(-1, B.shape[-2], B.shape[-1]))
    return out.view(*lead, A.shape[-2], B.shape[-1])


# Above this many bytes of probabilities ([B, H, T, T] fp32) the attention
# backward recomputes P one chunk of query rows at a time instead of keeping
# it from the forward pass (RAC_ATTN_KEEP_PROBS_BYTES overrides).
_ATTN_KEEP_PROBS_BYTES = int(os.environ.get('RAC_ATTN_KEEP_PROBS_BYTES', str(1 << 30)))
# Bytes of one [B*H, chunk, T] buffer in that recomputing backward.
_ATTN_BWD_CHUNK_BYTES = 128 << 20


class RACAttentionFunction(Function):
    """Scaled dot-product attention through RAC (rac.h:323-335): Q K^T and
    P V on the CORDIC matmul, causal / [T, T] additive mask and softmax on
    the CORDIC-exp kernel.  Backward (standard softmax-attention gradients,
    every product on the RAC matmul): dV = P^T dO, dP = dO V^T,
    dS = P (dP - rowsum(dP P)), dQ = s dS K, dK = s dS^T Q.  Up to
    _ATTN_KEEP_PROBS_BYTES of P are kept from the forward pass; beyond that
    the forward keeps none and the backward recomputes P a chunk of query
    rows at a time (the same probabilities, bit for bit), accumulating dV
    and dK over the chunks: memory O(B H chunk T) instead of O(B H T^2)."""

    @staticmethod
    def forward(ctx, q, k, v, mask, is_causal):
        _need_gpu(q, "q")
        q32, k32, v32 = (t.float().contiguous() for t in (q, k, v))
        m32 = mask.float().contiguous() if mask is not None else None
        if not any(ctx.needs_input_grad[:3]):
            # no backward: the core runs over query-row chunks and keeps no
            # [B, H, T, T] probabilities (same output bits)
            return _rac.attention(q32, k32, v32, m32, bool(is_causal), **_kw()).to(q.dtype)
        B, H, T, _ = q32.shape
        ctx.is_causal = bool(is_causal)
        if 4 * B * H * T * T <= _ATTN_KEEP_PROBS_BYTES:
            out, P = _rac.attention(q32, k32, v32, m32, bool(is_causal), return_probs=True, **_kw())
            ctx.save_for_backward(q32, k32, v32, m32, P)
        else:
            out = _rac.attention(q32, k32, v32, m32, bool(is_causal), **_kw())
            ctx.save_for_backward(q32, k32, v32, m32, None)
        return out.to(q.dtype)

    @staticmethod
    def backward(ctx, g):
        q, k, v, m, P = ctx.saved_tensors
        B, H, T, D = q.shape
        Z = B * H
        scale = _rac.attention_scale(D)
        need_q, need_k = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        g3 = g.float().contiguous().view(Z, T, D)
        q3, k3, v3 = q.view(Z, T, D), k.view(Z, T, D), v.view(Z, T, D)
        if P is not None:
            P3 = P.view(Z, T, T)
            dV = _rac.bmm(P3, g3, trans_a=True, **_kw())
            dP = _rac.bmm(g3, v3, trans_b=True, **_kw())
            dS = P3 * (dP - (dP * P3).sum(-1, keepdim=True))
            dQ = _rac.bmm(dS, k3, alpha=scale, **_kw()) if need_q else None
            dK = _rac.bmm(dS, q3, trans_a=True, alpha=scale, **_kw()) if need_k else None
        else:
            rows = _ATTN_BWD_CHUNK_BYTES // (4 * Z * T)
            rows = T if rows >= T else max(64, rows // 64 * 64)
            dV = torch.zeros((Z, T, D), device=q.device, dtype=torch.float32)
            dQ = torch.empty((Z, T, D), device=q.device, dtype=torch.float32) if need_q else None
            dK = torch.zeros((Z, T, D), device=q.device, dtype=torch.float32) if need_k else None
            for t0 in range(0, T, rows):
                r = min(rows, T - t0)
                Pc = _rac.attention_probs_rows(q, k, m, ctx.is_causal, t0, r, **_kw()).view(Z, r, T)
                gc = g3[:, t0:t0 + r].contiguous()
                _rac.bmm(Pc, gc, trans_a=True, out=dV, beta=1.0, **_kw())
                dP = _rac.bmm(gc, v3, trans_b=True, **_kw())
                dS = Pc * (dP - (dP * Pc).sum(-1, keepdim=True))
                del dP, Pc
                if need_q:
                    dQ[:, t0:t0 + r] = _rac.bmm(dS, k3, alpha=scale, **_kw())
                if need_k:
                    _rac.bmm(dS, q3[:, t0:t0 + r].contiguous(), trans_a=True, alpha=scale, out=dK, beta=1.0,
                             **_kw())
        shape = (B, H, T, D)
        return (dQ.view(shape) if dQ is not None else None, dK.view(shape) if dK is not None else None,
                dV.view(shape), None, None)


def rac_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask: Optional[torch.Tensor] = None,
                  is_causal: bool = False) -> torch.Tensor:
    """Attention core of [B, H, T, D] tensors through RAC; mask: optional
    additive [T, T]."""
    return RACAttentionFunction.apply(q, k, v, mask, is_causal)


def _dropout_inactive(dropout: nn.Module) -> bool:
    """True when the module between softmax and P V is the identity: an
    nn.Identity, or an nn.Dropout in eval mode or with p = 0.  Anything else
    (active dropout, a user module in its place) must be applied."""
    if type(dropout) is nn.Identity:
        return True
    if type(dropout) is nn.Dropout:
        return not dropout.training or dropout.p == 0
    return False


def _rac_core_ok(mask: Optional[torch.Tensor], T: int, dropout: nn.Module) -> bool:
    """The fused RAC attention core takes a [T, T] additive mask and no
    dropout between softmax and P V; other cases compose the stages."""
    if not _dropout_inactive(dropout):
        return False
    return mask is None or (mask.dim() == 2 and tuple(mask.shape) == (T, T) and mask.is_floating_point())


def _attention_composed(Q, K, V, scale: float, mask: Optional[torch.Tensor], is_causal: bool,
                        dropout: nn.Module) -> torch.Tensor:
    """The stages of rac_torch.py:1327-1337 one by one, every product on the
    batched RAC matmul: S = (Q K^T) * scale, + causal -inf above the diagonal,
    + mask (broadcast; a bool mask adds 1.0 where True, as torch's + does),
    P = dropout(CORDIC softmax(S)), out = P V.  Used where the fused core does
    not apply (a mask other than [T, T] float, or an active dropout)."""
    T = Q.shape[-2]
    scores = rac_bmm(Q, K.transpose(-2, -1)) * scale
    if is_causal:
        scores = _causal_scores(scores, T)
    if mask is not None:
        scores = scores + mask
    return rac_bmm(dropout(rac_softmax(scores)), V)


class RACAttention(nn.Module):
    """Multi-head attention with RAC projections and per-head RAC matmuls
    (rac_torch.py:660-818); softmax on the CORDIC-exp kernel."""

    def __init__(self, d_model, n_heads, bias=True, dropout=0.0, device=None, dtype=None):
        super().__init__()
        assert d_model % n_heads == 0, f"d_model ({d_model}) must be divisible by n_heads ({n_heads})"
        self.d_model = d_model
        self.n_heads = n_heads
        self.d_head = d_model // n_heads
        self.scale = self.d_head ** -0.5
        self.qkv = RACLinear(d_model, 3 * d_model, bias=bias, device=device, dtype=dtype)
        self.out_proj = RACLinear(d_model, d_model, bias=bias, device=device, dtype=dtype)
        self.dropout = nn.Dropout(dropout) if dropout > 0 else nn.Identity()

    def forward(self, x, mask=None, is_causal=False):
        B, T, D = x.shape
        Q, K, V = self.qkv(x).chunk(3, dim=-1)
        Q = Q.reshape(B, T, self.n_heads, self.d_head).transpose(1, 2)
        K = K.reshape(B, T, self.n_heads, self.d_head).transpose(1, 2)
        V = V.reshape(B, T, self.n_heads, self.d_head).transpose(1, 2)
        if _rac_core_ok(mask, T, self.dropout):
            out = rac_attention(Q, K, V, mask, is_causal)
        else:
            # the reference loops RACMatmulFunction over heads
            # (rac_torch.py:781-795); one batched launch does the same products
            out = _attention_composed(Q, K, V, self.scale, mask, is_causal, self.dropout)
        out = out.transpose(1, 2).contiguous().view(B, T, D)
        return self.out_proj(out)

    @classmethod
    def from_attention_layers(cls, q_linear, k_linear, v_linear, out_linear, n_heads, dropout=0.0):
        """Multi-head attention built from four existing d_model -> d_model
        projections (rac_torch.py:781-816): Q, K and V become the row blocks
        of the fused qkv weight in that order, out_linear the output
        projection; parameters are copied bit for bit.  All four must be
        square, agree on having a bias, and n_heads must divide d_model."""
        parts = (q_linear, k_linear, v_linear, out_linear)
        d_model, with_bias = _square_projections("from_attention_layers", parts)
        if n_heads <= 0 or d_model % n_heads:
            raise ValueError(f"from_attention_layers: n_heads ({n_heads}) must divide d_model ({d_model})")
        ref = q_linear.weight
        attn = cls(d_model, n_heads, bias=with_bias, dropout=dropout, device=ref.device, dtype=ref.dtype)
        _load_row_blocks(attn.qkv, parts[:3])
        _load_row_blocks(attn.out_proj, parts[3:])
        return attn

    def extra_repr(self):
        return (f'd_model={self.d_model}, n_heads={self.n_heads}, '
                f'd_head={self.d_head}, backend=RAC')


class RACTransformerBlock(nn.Module):
    """Post-norm block: norm1(x + attn(x)), norm2(x + ffn(x)) (rac_torch.py:823-860)."""

    def __init__(self, d_model, n_heads, ff_dim=None, activation='gelu', dropout=0.0,
                 bias=True, device=None, dtype=None):
        super().__init__()
        if ff_dim is None:
            ff_dim = 4 * d_model
        self.attn = RACAttention(d_model, n_heads, bias=bias, dropout=dropout, device=device, dtype=dtype)
        self.ffn = RACFusedFFN(d_model, ff_dim, activation=activation, bias=bias, device=device, dtype=dtype)
        self.norm1 = RACLayerNorm(d_model, device=device, dtype=dtype)
        self.norm2 = RACLayerNorm(d_model, device=device, dtype=dtype)

    def forward(self, x, mask=None, is_causal=False):
        x = self.norm1(x + self.attn(x, mask=mask, is_causal=is_causal))
        x = self.norm2(x + self.ffn(x))
        return x

    def extra_repr(self):
        return (f'd_model={self.attn.d_model}, n_heads={self.attn.n_heads}, '
                f'ff_dim={self.ffn.fc1.out_features}')


class RACRoPEAttention(nn.Module):
    """Llama-style attention (rac_torch.py:1279-1343): RAC QKV and output
    projections, RoPE kernel on the strided Q/K views, and the attention core
    through RAC (Q K^T and P V on the CORDIC matmul, causal / [T, T] mask and
    CORDIC softmax).  With dropout active or another mask shape, the
    reference's stages run one by one, still with every product on the
    batched RAC matmul and the CORDIC-exp softmax."""

    def __init__(self, d_model: int, n_heads: int, max_seq_len: int = 4096, bias: bool = False,
                 dropout: float = 0.0, rope_base: float = 10000.0, device=None, dtype=None):
        super().__init__()
        assert d_model % n_heads == 0
        self.d_model = d_model
        self.n_heads = n_heads
        self.d_head = d_model // n_heads
        self.scale = self.d_head ** -0.5
        self.qkv = RACLinear(d_model, 3 * d_model, bias=bias, device=device, dtype=dtype)
        self.out_proj = RACLinear(d_model, d_model, bias=bias, device=device, dtype=dtype)
        self.rope = RACRoPE(self.d_head, max_seq_len=max_seq_len, base=rope_base,
                            device=device, dtype=dtype or torch.float32)
        self.dropout = nn.Dropout(dropout) if dropout > 0 else nn.Identity()

    def forward(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None, is_causal: bool = False,
                positions: Optional[torch.Tensor] = None) -> torch.Tensor:
        B, T, D = x.shape
        qkv = self.qkv(x)
        Q, K, V = qkv.chunk(3, dim=-1)
        Q = Q.view(B, T, self.n_heads, self.d_head).transpose(1, 2)
        K = K.view(B, T, self.n_heads, self.d_head).transpose(1, 2)
        V = V.view(B, T, self.n_heads, self.d_head).transpose(1, 2)
        Q, K = self.rope(Q, K, positions=positions)
        if _rac_core_ok(mask, T, self.dropout):
            out = rac_attention(Q, K, V, mask, is_causal).to(x.dtype)
        else:
            out = _attention_composed(Q, K, V, self.scale, mask, is_causal, self.dropout).to(x.dtype)
        out = out.transpose(1, 2).contiguous().view(B, T, D)
        return self.out_proj(out)

    def extra_repr(self):
        return (f'd_model={self.d_model}, n_heads={self.n_heads}, '
                f'd_head={self.d_head}, backend=RAC-RoPE')


class RACLlamaBlock(nn.Module):
    """x = x + attn(RMSNorm(x)); x = x + ffn(RMSNorm(x)) (rac_torch.py:1348-1383)."""

    def __init__(self, d_model: int, n_heads: int, ff_dim: int = None, max_seq_len: int = 4096,
                 activation: str = 'silu', dropout: float = 0.0, bias: bool = False,
                 rms_eps: float = 1e-6, rope_base: float = 10000.0, device=None, dtype=None):
        super().__init__()
        if ff_dim is None:
            ff_dim = 4 * d_model
        self.norm1 = RACRMSNorm(d_model, eps=rms_eps, device=device, dtype=dtype)
        self.attn = RACRoPEAttention(d_model, n_heads, max_seq_len=max_seq_len, bias=bias,
                                     dropout=dropout, rope_base=rope_base, device=device, dtype=dtype)
        self.norm2 = RACRMSNorm(d_model, eps=rms_eps, device=device, dtype=dtype)
        self.ffn = RACFusedFFN(d_model, ff_dim, activation=activation, bias=bias,
                               device=device, dtype=dtype)

    def forward(self, x, mask=None, is_causal=False, positions=None):
        x = x + self.attn(self.norm1(x), mask=mask, is_causal=is_causal, positions=positions)
        x = x + self.ffn(self.norm2(x))
        return x

    def extra_repr(self):
        return (f'd_model={self.norm1.d_model}, n_heads={self.attn.n_heads}, '
                f'ff_dim={self.ffn.fc1.out_features}')


# ── model patching (rac_torch.py:865-985) ──────────────────────────────────
#
# The interface fixes the names, the arguments, the min_features rule (both
# dimensions at least min_features), exact weight preservation and the keys
# of benchmark_model's result.  The traversal works on a snapshot of
# (owner, attribute) slots taken before anything is replaced, so swapping a
# child never disturbs the walk.

def _child_slots(model: nn.Module):
    """Every (dotted name, owner module, attribute, child) of the tree."""
    slots = []
    for owner_name, owner in model.named_modules():
        for attr, child in owner.named_children():
            slots.append((f'{owner_name}.{attr}' if owner_name else attr, owner, attr, child))
    return slots


def _copy_params(dst: nn.Module, src: nn.Module) -> nn.Module:
    """dst.weight/bias := src.weight/bias, bit for bit."""
    with torch.no_grad():
        dst.weight.copy_(src.weight)
        if src.bias is not None:
            dst.bias.copy_(src.bias)
    return dst


def patch_model(model: nn.Module, verbose: bool = True, min_features: int = 64) -> nn.Module:
    """Swap every plain nn.Linear whose in and out features are both at least
    min_features for a RACLinear holding the same parameters; smaller layers
    stay as they are.  Returns the model (modified in place)."""
    swapped, kept = [], []
    for name, owner, attr, child in _child_slots(model):
        if not isinstance(child, nn.Linear):    # RACLinear is not an nn.Linear subclass
            continue
        shape = (child.in_features, child.out_features)
        if min(shape) < min_features:
            kept.append((name, shape))
            continue
        setattr(owner, attr, RACLinear.from_linear(child))
        swapped.append((name, shape))
    if verbose:
        for name, (fi, fo) in kept:
            print(f'patch_model: {name} stays nn.Linear ({fi} x {fo} is below min_features={min_features})')
        print(f'patch_model: {len(swapped)} of {len(swapped) + len(kept)} nn.Linear layers now run through RAC')
        for name, (fi, fo) in swapped:
            print(f'    {name:<40s} {fi:>6d} -> {fo:<6d}')
    return model


def unpatch_model(model: nn.Module, verbose: bool = True) -> nn.Module:
    """Undo patch_model: every RACLinear (not the fused variants) becomes an
    nn.Linear with the same parameters, device and dtype."""
    count = 0
    for name, owner, attr, child in _child_slots(model):
        if type(child) is not RACLinear:
            continue
        plain = nn.Linear(child.in_features, child.out_features, bias=child.bias is not None,
                          device=child.weight.device, dtype=child.weight.dtype)
        setattr(owner, attr, _copy_params(plain, child))
        count += 1
    if verbose:
        print(f'unpatch_model: {count} RACLinear layer(s) turned back into nn.Linear')
    return model


def benchmark_model(model: nn.Module, input_shape: tuple, n_warmup: int = 10, n_iters: int = 100,
                    device: str = 'cuda') -> dict:
    """Mean forward time of `model` on one random input as given, then with
    its linear layers on RAC (patch_model), then restored (unpatch_model).
    Times come from device events on the current stream."""
    model = model.to(device).eval()
    sample = torch.randn(*input_shape, device=device)

    def mean_ms(m):
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.inference_mode():
            for _ in range(n_warmup):
                m(sample)
            start.record()
            for _ in range(n_iters):
                m(sample)
            stop.record()
        stop.synchronize()
        return start.elapsed_time(stop) / max(n_iters, 1)

    torch_ms = mean_ms(model)
    rac_ms = mean_ms(patch_model(model, verbose=False))
    unpatch_model(model, verbose=False)
    return {'baseline_ms': torch_ms, 'rac_ms': rac_ms,
            'speedup': (torch_ms / rac_ms) if rac_ms > 0 else float('inf'), 'n_iters': n_iters}


def rac_info():
    """Print the extension status (rac_torch.py:1388-1409)."""
    print("RAC on MI355X (gfx950) — rotation-accumulate kernels")
    print(f"  ROCm device available: {torch.cuda.is_available()}")
    try:
        lib = _rac._lib.load()
        print(f"  kernel library:        {_rac._lib.LIB_PATH} (v{lib.rac_version()})")
    except Exception as e:  # noqa: BLE001
        print(f"  kernel library:        NOT LOADED ({e})")
    if torch.cuda.is_available():
        print(f"  device:                {torch.cuda.get_device_properties(0).name}")
    print(f"  start-up probe:        {_PROBE.stage}: {_PROBE.message}")
    mode_name = {0: 'fast', 1: 'cordic', 2: 'shiftadd'}.get(_RAC_CORDIC_MODE, '?')
    print(f"  CORDIC iters:          {_RAC_CORDIC_ITERS} (rac_set_precision)")
    print(f"  compute mode:          {mode_name} (rac_set_mode)")
    print("  kernels:               matmul/linear (FAST/CORDIC/SHIFTADD), softmax + SiLU + sigmoid "
          "(hyperbolic CORDIC exp), RMSNorm/LayerNorm (CORDIC rsqrt), RoPE (circular CORDIC)")
    print(f"  adaptive threshold:    {_RAC_MIN_ELEMENTS} elements (RAC_MIN_ELEMENTS)")
