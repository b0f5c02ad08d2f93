"""GPU parity of the fused linear layer (RAC GEMM with bias + activation in
its epilogue, rac_torch.cu:705-780) and of its backward pass
(rac_torch.cu:1085-1185), against the CPU checker and against the unfused
path of the same library.

Bars: pre-activation bit-exact with the checker's NT product plus bias;
ReLU / SiLU (CORDIC exp) outputs and their gradients bit-exact; GELU within
the device-vs-glibc erff/expf difference; the fused kernel bit-identical to
the separate GEMM + activation kernels.
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


def ext():
    from rac_amd import ext as e
    return e


def _np_act(x, act, iters):
    if act == 0:
        return x
    if act == 1:
        return np.where(x > 0, x, np.float32(0)).astype(np.float32)
    if act == 2:
        return rl.orc_unary("orc_gelu", x)
    return rl.orc_unary("orc_silu", x, iters)


def _np_act_grad(g, x, act, iters):
    f1 = np.float32(1)
    if act == 1:
        return (g * np.where(x > 0, f1, np.float32(0))).astype(np.float32)
    if act == 2:
        x64 = x.astype(np.float64)
        from scipy.special import erf
        cdf = 0.5 * (1 + erf(x64 * 0.7071067811865))
        pdf = 0.3989422804 * np.exp(-0.5 * x64 * x64)
        return (g.astype(np.float64) * (cdf + x64 * pdf)).astype(np.float32)
    if act == 3:
        sig = rl.orc_unary("orc_sigmoid", x, iters)
        return (g * (sig * (f1 + x * (f1 - sig)))).astype(np.float32)
    return g


SHAPES = [(1, 1, 1), (5, 7, 3), (64, 96, 48), (67, 130, 83)]


@pytest.mark.parametrize("mode,iters", [(1, 16), (1, 8), (0, 24), (1, 24), (2, 16), (1, 5)])
@pytest.mark.parametrize("act", [0, 1, 2, 3])
def test_fused_linear_forward(mode, iters, act):
    e = ext()
    for (M, N, K) in SHAPES:
        for with_bias in (False, True):
            print(f"fused linear mode={mode} iters={iters} act={act} shape={(M, N, K)} bias={with_bias}",
                  flush=True)
            x = rl.gen_normal((M, K), seed=M + K)
            w = rl.gen_normal((N, K), seed=N + 2 * K, std=0.2)
            b = rl.gen_normal(N, seed=N) if with_bias else np.zeros(0, np.float32)
            out, pre = e.fused_linear_forward(T(x), T(w), T(b), act, iters=iters, mode=mode, return_pre=True)
            out, pre = H(out), H(pre)
            ref_pre = rl.orc_matmul(x, w, M, N, K, iters, mode, tb=1)
            if with_bias:
                ref_pre = (ref_pre + b[None, :]).astype(np.float32)
            assert np.array_equal(pre, ref_pre)
            ref = _np_act(ref_pre, act, iters)
            if act == 2:
                # device erff vs glibc erff: a few ulp of erf, which 1 + erf
                # turns into an absolute error ~2^-23 |x| / 2 for x << 0
                assert np.all(np.abs(out - ref) <= 2e-6 * np.abs(ref) + 2.4e-7 * np.abs(ref_pre) + 1e-7)
            else:
                assert np.array_equal(out, ref)
            # the unfused path of the same library (GEMM, then the activation kernel)
            lin = e.linear_forward(T(x), T(w), T(b), iters=iters, mode=mode)
            sep = {0: lambda t: t, 1: e.relu, 2: e.gelu, 3: lambda t: e.silu(t, iters)}[act](lin)
            assert np.array_equal(out, H(sep))
            assert np.array_equal(H(e.fused_linear_forward(T(x), T(w), T(b), act, iters=iters, mode=mode)), out)


@pytest.mark.parametrize("act", [0, 1, 2, 3])
def test_fused_linear_backward(act):
    e = ext()
    M, N, K, iters, mode = 45, 70, 33, 16, 1
    print(f"fused linear backward act={act}", flush=True)
    x = rl.gen_normal((M, K), seed=1)
    w = rl.gen_normal((N, K), seed=2, std=0.2)
    b = rl.gen_normal(N, seed=3)
    g = rl.gen_normal((M, N), seed=4)
    _, pre = e.fused_linear_forward(T(x), T(w), T(b), act, iters=iters, mode=mode, return_pre=True)
    pre_h = H(pre)
    d = H(e.act_grad(T(g), pre, act, iters=iters)) if act else g
    ref_d = _np_act_grad(g, pre_h, act, iters)
    if act == 2:
        assert np.all(np.abs(d - ref_d) <= 4e-6 * np.abs(ref_d) + 4e-7 * np.abs(g) * (1 + np.abs(pre_h)))
    else:
        assert np.array_equal(d, ref_d)
    gi, gw, gb = e.fused_linear_backward(T(g), T(x), T(w), T(b), pre, act, True, iters=iters, mode=mode)
    assert np.array_equal(H(gi), rl.orc_matmul(d, w, M, K, N, iters, mode))
    assert np.array_equal(H(gw), rl.orc_matmul(d, x, N, K, M, iters, mode, ta=1))
    assert np.allclose(H(gb), d.astype(np.float64).sum(0), rtol=1e-5, atol=1e-5)


def test_fused_rac_linear_module_autograd():
    from rac_amd import rac_torch as rt
    torch.manual_seed(0)
    old = (rt.rac_get_precision(), rt.rac_get_mode())
    try:
        rt.rac_set_precision(24)
        rt.rac_set_mode("cordic")
        for act in ("relu", "gelu", "silu", None):
            m = rt.FusedRACLinear(48, 40, bias=True, activation=act).to(DEV)
            x = torch.randn(3, 5, 48, device=DEV, requires_grad=True)
            y = m(x)
            y.backward(torch.ones_like(y))
            x64 = x.detach().double().cpu().requires_grad_(True)
            w64 = m.weight.detach().double().cpu().requires_grad_(True)
            b64 = m.bias.detach().double().cpu().requires_grad_(True)
            z = x64 @ w64.t() + b64
            f = {"relu": torch.relu, "gelu": torch.nn.functional.gelu, "silu": torch.nn.functional.silu,
                 None: lambda t: t}[act]
            r = f(z)
            r.backward(torch.ones_like(r))
            # CORDIC-24 products (|rel| ~6e-6 of |x||w|) and CORDIC exp (2^-22)
            assert np.max(np.abs(H(y) - r.detach().numpy())) < 1e-4, act
            for t, r_ in ((x, x64), (m.weight, w64), (m.bias, b64)):
                ref = r_.grad.numpy()
                assert np.max(np.abs(H(t.grad) - ref)) < 2e-4 * max(1.0, float(np.abs(ref).max())), act
    finally:
        rt.rac_set_precision(old[0])
        rt.rac_set_mode(old[1])


def test_fused_linear_fp16_and_empty_bias_and_errors():
    e = ext()
    x = torch.randn(4, 16, device=DEV, dtype=torch.float16)
    w = torch.randn(8, 16, device=DEV, dtype=torch.float16)
    y = e.fused_linear_forward(x, w, torch.empty(0, device=DEV), 1, iters=16, mode=0)
    assert y.dtype == torch.float16 and y.shape == (4, 8)
    ref = torch.relu(x.float() @ w.float().t())
    assert torch.allclose(y.float(), ref, atol=1e-2, rtol=1e-2)
    with pytest.raises(RuntimeError):
        e.fused_linear_forward(x.float(), w.float(), torch.empty(0, device=DEV), 7)
