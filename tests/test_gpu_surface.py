"""The reference extension surface beyond the forward products:

  * ``import rac_cuda_ext`` (the reference's module name,
    rac_torch/rac_torch_bind.cpp:223-258) and its linear_forward vs the
    checker;
  * ``matmul_backward`` (rac_torch_bind.cpp:130-163): NT grad_A and TN grad_B
    bit-exact with orc_matmul, each need_grad flag on and off, and a
    backward() through rac_matmul;
  * dtypes and autocast (reference test_rac_dvt.py:373-455, DVT-13/14/15/17):
    fp16/bf16 parameters and inputs, torch.autocast fp16/bf16 with a
    GradScaler training step;
  * torch.compile (DVT-16): RACLinear and FusedRACLinear compiled through
    dynamo + AOTAutograd (backend "aot_eager") and with CUDA graphs (backend
    "cudagraphs", replayed several times with eager work between), equal to
    eager bit for bit, gradients included;
  * gradcheck (DVT-4/5, tolerances eps 1e-4, atol 1e-3, rtol 1e-3 in the
    reference): rac_matmul, rac_linear and the fused linear with float64
    inputs, which the kernels evaluate in float32.
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


def rt():
    from rac_amd import rac_torch
    return rac_torch


class _knobs:
    """Set the rac_torch mode and precision for a block, restore after."""

    def __init__(self, mode, iters):
        self.mode, self.iters = mode, iters

    def __enter__(self):
        r = rt()
        self.prev = (r.rac_get_mode(), r.rac_get_precision())
        r.rac_set_mode(self.mode)
        r.rac_set_precision(self.iters)

    def __exit__(self, *exc):
        r = rt()
        r.rac_set_mode(self.prev[0])
        r.rac_set_precision(self.prev[1])


def test_rac_cuda_ext_module_name():
    import rac_cuda_ext
    from rac_amd import ext
    assert rac_cuda_ext.MODE_FAST == 0 and rac_cuda_ext.MODE_CORDIC == 1 and rac_cuda_ext.MODE_SHIFTADD == 2
    for name in ("matmul_forward", "matmul_backward", "linear_forward", "linear_backward",
                 "set_cordic_iters", "get_cordic_iters", "set_cordic_mode", "get_cordic_mode",
                 "fused_linear_forward", "fused_linear_backward"):
        assert getattr(rac_cuda_ext, name) is getattr(ext, name), name
    x = rl.gen_uniform((37, 96), seed=70)
    w = rl.gen_uniform((80, 96), seed=71)
    b = rl.gen_uniform((80,), seed=72)
    got = H(rac_cuda_ext.linear_forward(T(x), T(w), torch.empty(0), iters=16, mode=1))
    ref = rl.orc_matmul(x, w, 37, 80, 96, 16, 1, tb=1)
    assert np.array_equal(got, ref)
    got_b = H(rac_cuda_ext.linear_forward(T(x), T(w), T(b), iters=16, mode=1))
    assert np.array_equal(got_b, (ref + b).astype(np.float32))
    # the knob is shared with rac_amd.ext
    old = ext.get_cordic_iters()
    try:
        rac_cuda_ext.set_cordic_iters(8)
        assert ext.get_cordic_iters() == 8
    finally:
        ext.set_cordic_iters(old)


@pytest.mark.parametrize("mode,iters", [(1, 16), (1, 8), (0, 24), (2, 16)])
def test_matmul_backward_bitexact(mode, iters):
    from rac_amd import ext
    M, K, N = 37, 53, 29
    A = rl.gen_uniform((M, K), seed=80)
    B = rl.gen_uniform((K, N), seed=81)
    G = rl.gen_normal((M, N), seed=82)
    ref_a = rl.orc_matmul(G, B, M, K, N, iters, mode, tb=1)      # grad_C @ B^T
    ref_b = rl.orc_matmul(A, G, K, N, M, iters, mode, ta=1)      # A^T @ grad_C
    for need_a, need_b in ((True, True), (True, False), (False, True), (False, False)):
        gA, gB = ext.matmul_backward(T(G), T(A), T(B), need_a, need_b, iters=iters, mode=mode)
        assert (gA is None) == (not need_a) and (gB is None) == (not need_b)
        if need_a:
            assert np.array_equal(H(gA), ref_a), (need_a, need_b)
        if need_b:
            assert np.array_equal(H(gB), ref_b), (need_a, need_b)


def test_rac_matmul_backward_through_autograd():
    M, K, N = 41, 67, 23
    A = rl.gen_uniform((M, K), seed=90)
    B = rl.gen_uniform((K, N), seed=91)
    G = rl.gen_normal((M, N), seed=92)
    with _knobs("cordic", 16):
        for ga, gb in ((True, True), (True, False), (False, True)):
            a, b = T(A).requires_grad_(ga), T(B).requires_grad_(gb)
            c = rt().rac_matmul(a, b)
            assert np.array_equal(H(c), rl.orc_matmul(A, B, M, N, K, 16, 1))
            c.backward(T(G))
            if ga:
                assert np.array_equal(H(a.grad), rl.orc_matmul(G, B, M, K, N, 16, 1, tb=1))
            else:
                assert a.grad is None
            if gb:
                assert np.array_equal(H(b.grad), rl.orc_matmul(A, G, K, N, M, 16, 1, ta=1))
            else:
                assert b.grad is None


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_half_precision_parameters_and_inputs(dtype):
    """DVT-13/14/17: fp16/bf16 tensors are widened to fp32 (exact), the RAC
    product runs in fp32 and the result is rounded once to the input dtype."""
    r = rt()
    torch.manual_seed(3)
    with _knobs("cordic", 16):
        layer = r.RACLinear(128, 64, bias=True).to(DEV).to(dtype)
        x = torch.randn(8, 128, device=DEV).to(dtype)
        y = layer(x)
        assert y.dtype == dtype
        x32, w32, b32 = (H(t.float()) for t in (x, layer.weight, layer.bias))
        ref = (rl.orc_matmul(x32, w32, 8, 64, 128, 16, 1, tb=1) + b32).astype(np.float32)
        assert torch.equal(y, torch.from_numpy(ref).to(DEV).to(dtype))
        C = r.rac_matmul(x, layer.weight.t().contiguous())
        assert C.dtype == dtype
        ref_c = rl.orc_matmul(x32, np.ascontiguousarray(w32.T), 8, 64, 128, 16, 1)
        assert torch.equal(C, torch.from_numpy(ref_c).to(DEV).to(dtype))
        model = torch.nn.Sequential(r.RACLinear(128, 64), torch.nn.ReLU(), r.RACLinear(64, 32)).to(DEV)
        xm = torch.randn(4, 128, device=DEV)
        assert torch.isfinite(model(xm)).all()
        yh = model.to(dtype)(xm.to(dtype))
        assert yh.dtype == dtype and torch.isfinite(yh).all()
        assert torch.isfinite(model.float()(xm)).all()          # back to fp32 (rounded weights)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_autocast_forward_and_gradscaler_step(dtype):
    """DVT-15: under torch.autocast the RAC layers keep computing in fp32
    (their kernels take fp32): the output equals the fp32 output bit for bit,
    and a GradScaler training step runs and updates the weights."""
    r = rt()
    torch.manual_seed(4)
    with _knobs("cordic", 16):
        layer = r.RACLinear(256, 128, bias=True).to(DEV)
        fused = r.FusedRACLinear(256, 128, bias=True, activation="silu").to(DEV)
        x = torch.randn(16, 256, device=DEV)
        ref, ref_f = layer(x), fused(x)
        with torch.autocast("cuda", dtype=dtype):
            y, yf = layer(x), fused(x)
        assert torch.equal(y.float(), ref) and torch.equal(yf.float(), ref_f)
        scaler = torch.amp.GradScaler("cuda")
        opt = torch.optim.SGD(list(layer.parameters()) + list(fused.parameters()), lr=0.01)
        w0 = layer.weight.detach().clone()
        opt.zero_grad()
        with torch.autocast("cuda", dtype=dtype):
            loss = layer(x).sum() + fused(x).sum()
        scaler.scale(loss).backward()
        assert layer.weight.grad is not None and torch.isfinite(layer.weight.grad).all()
        assert fused.weight.grad is not None and torch.isfinite(fused.weight.grad).all()
        scaler.step(opt)
        scaler.update()
        assert not torch.equal(layer.weight.detach(), w0)


@pytest.mark.parametrize("backend", ["aot_eager", "cudagraphs"])
def test_torch_compile_matches_eager(backend):
    """DVT-16: the RAC layers under torch.compile.  The kernels are
    torch.library ops with registered shape functions, so dynamo and
    AOTAutograd trace them without running them; the compiled module must
    give the eager bits, forward and backward."""
    import torch._dynamo
    r = rt()
    torch._dynamo.reset()
    torch.manual_seed(5)
    with _knobs("cordic", 16):
        model = torch.nn.Sequential(r.RACLinear(128, 96), r.FusedRACLinear(96, 64, activation="silu"),
                                    r.RACLinear(64, 32, bias=False)).to(DEV)
        compiled = torch.compile(model, backend=backend, fullgraph=(backend == "aot_eager"))
        for step in range(3):
            x = torch.randn(8, 128, device=DEV)
            ref = model(x)
            got = compiled(x).clone()
            assert got.shape == (8, 32)
            assert torch.equal(got, ref), (backend, step)
            torch.cuda.synchronize()
        if backend == "aot_eager":
            x = torch.randn(8, 128, device=DEV, requires_grad=True)
            g = torch.randn(8, 32, device=DEV)
            model(x).backward(g)
            ref_grads = [x.grad.clone()] + [p.grad.clone() for p in model.parameters()]
            x.grad = None
            for p in model.parameters():
                p.grad = None
            compiled(x).backward(g)
            got_grads = [x.grad] + [p.grad for p in model.parameters()]
            for a, b in zip(got_grads, ref_grads):
                assert torch.equal(a, b)
    torch._dynamo.reset()


@pytest.mark.parametrize("mode", ["fast", "cordic"])
def test_gradcheck_matmul_linear_fused(mode):
    """DVT-4/5 with float64 inputs.  The kernels evaluate in float32, so the
    finite differences use eps = 1e-2: the products are linear in each
    perturbed input, so a larger step adds no truncation error and keeps
    the float32 rounding of the outputs (~1e-7 relative) well below the
    reference's atol = rtol = 1e-3.  The fused layer's GELU (device erf) is
    smooth; eps = 1e-3 keeps its truncation error near 1e-6."""
    from torch.autograd import gradcheck
    r = rt()
    with _knobs(mode, 24):
        for (M, K, N) in ((8, 8, 8), (16, 32, 16), (4, 64, 8)):
            A = torch.randn(M, K, device=DEV, dtype=torch.float64, requires_grad=True)
            B = torch.randn(K, N, device=DEV, dtype=torch.float64, requires_grad=True)
            assert gradcheck(r.RACMatmulFunction.apply, (A, B), eps=1e-2, atol=1e-3, rtol=1e-3)
        x = torch.randn(3, 5, 16, device=DEV, dtype=torch.float64, requires_grad=True)
        w = torch.randn(12, 16, device=DEV, dtype=torch.float64, requires_grad=True)
        b = torch.randn(12, device=DEV, dtype=torch.float64, requires_grad=True)
        assert gradcheck(r.RACLinearFunction.apply, (x, w, b), eps=1e-2, atol=1e-3, rtol=1e-3)
        assert gradcheck(r.RACLinearFunction.apply, (x, w, None), eps=1e-2, atol=1e-3, rtol=1e-3)
        xs = (x * 0.3).detach().requires_grad_(True)
        ws = (w * 0.3).detach().requires_grad_(True)
        assert gradcheck(lambda a, b_, c: r.RACFusedLinearFunction.apply(a, b_, c, r.ACT_GELU), (xs, ws, b),
                         eps=1e-3, atol=1e-3, rtol=1e-3)
