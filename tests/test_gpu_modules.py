"""GPU checks of the rac_torch module surface not covered elsewhere: the
fused QKV projection (rac_torch.py:588-626), the fused FFN
(rac_torch.py:631-655), multi-head attention on both of its paths
(rac_torch.py:660-818), the post-norm transformer block
(rac_torch.py:823-860), rac_matmul_adaptive (rac_torch.py:570-583),
benchmark_model (rac_torch.py:945-985) and rac_info (rac_torch.py:1388-1409).

Each module runs in FAST mode at n=24 and is compared, forward and backward,
with the same composition in float64 torch on the CPU built from the
module's own parameters.  Bars: products within 1e-4 of |a|.|b| (the matmul
bar), everything downstream of them within 1e-4 of the output's scale
(CORDIC-exp softmax / SiLU at n=24 are within 2^-20 relative, GELU within the
device erff rounding).
"""
import io
import contextlib

import numpy as np
import pytest

torch = pytest.importorskip("torch")
F = torch.nn.functional
pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    import rac_amd
    rac_amd.load()
    from rac_amd import rac_torch as rt
    old = (rt.rac_get_precision(), rt.rac_get_mode())
    rt.rac_set_precision(24)
    rt.rac_set_mode("fast")
    yield
    rt.rac_set_precision(old[0])
    rt.rac_set_mode(old[1])
    torch.cuda.synchronize()


def rt():
    from rac_amd import rac_torch
    return rac_torch


def c64(t):
    """Detached float64 CPU copy that takes gradients."""
    return t.detach().double().cpu().requires_grad_(True)


def params64(module):
    return {k: v.detach().double().cpu() for k, v in module.named_parameters()}


def close(got, ref, scale=None, tol=1e-4, what=""):
    g = got.detach().double().cpu()
    r = ref.detach().double().cpu()
    s = float(r.abs().max()) if scale is None else scale
    err = float((g - r).abs().max())
    assert err <= tol * max(s, 1.0), f"{what}: max err {err:.3e} vs scale {s:.3e}"


def _gelu64(x):
    return 0.5 * x * (1.0 + torch.erf(x / np.sqrt(2.0)))


ACT64 = {"relu": torch.relu, "gelu": _gelu64, "silu": lambda x: x * torch.sigmoid(x)}


def test_fused_qkv_from_linears_matches_float64():
    torch.manual_seed(1)
    d = 96
    lq, lk, lv = (torch.nn.Linear(d, d).to(DEV) for _ in range(3))
    m = rt().RACFusedQKV.from_qkv_linears(lq, lk, lv)
    x = torch.randn(2, 13, d, device=DEV, requires_grad=True)
    q, k, v = m(x)
    assert q.shape == k.shape == v.shape == (2, 13, d)
    g = [torch.randn_like(t) for t in (q, k, v)]
    torch.autograd.backward((q, k, v), g)
    x64 = c64(x)
    W64 = [(c64(l.weight), c64(l.bias)) for l in (lq, lk, lv)]
    outs = [F.linear(x64, w, b) for w, b in W64]
    torch.autograd.backward(outs, [t.double().cpu() for t in g])
    bound = float(x64.detach().abs().sum(-1).max()) * float(lq.weight.detach().abs().max())
    for got, ref in zip((q, k, v), outs):
        close(got, ref, scale=bound, what="qkv forward")
    close(x.grad, x64.grad, what="qkv grad input")
    close(m.qkv.weight.grad, torch.cat([w.grad for w, _ in W64]), what="qkv grad weight")
    close(m.qkv.bias.grad, torch.cat([b.grad for _, b in W64]), what="qkv grad bias")


@pytest.mark.parametrize("act", ["gelu", "silu", "relu"])
def test_fused_ffn_matches_float64(act):
    torch.manual_seed(2)
    d, ff = 64, 176
    m = rt().RACFusedFFN(d, ff, activation=act).to(DEV)
    x = torch.randn(3, 9, d, device=DEV, requires_grad=True)
    y = m(x)
    g = torch.randn_like(y)
    y.backward(g)
    P = params64(m)
    x64 = c64(x)
    h = ACT64[act](F.linear(x64, P["fc1.weight"].requires_grad_(True), P["fc1.bias"].requires_grad_(True)))
    y64 = F.linear(h, P["fc2.weight"].requires_grad_(True), P["fc2.bias"].requires_grad_(True))
    y64.backward(g.double().cpu())
    close(y, y64, what=f"ffn {act} forward")
    close(x.grad, x64.grad, what=f"ffn {act} grad input")
    for name, prm in m.named_parameters():
        close(prm.grad, P[name].grad, what=f"ffn {act} grad {name}")


def _mha64(x64, P, nh, mask=None, is_causal=False):
    B, T, D = x64.shape
    hd = D // nh
    qkv = F.linear(x64, P["qkv.weight"], P["qkv.bias"])
    q, k, v = (t.reshape(B, T, nh, hd).transpose(1, 2) for t in qkv.chunk(3, -1))
    s = q @ k.transpose(-1, -2) * hd ** -0.5
    if is_causal:
        s = s.masked_fill(torch.triu(torch.ones(T, T, dtype=torch.bool), 1), float("-inf"))
    if mask is not None:
        s = s + mask
    o = (torch.softmax(s, -1) @ v).transpose(1, 2).reshape(B, T, D)
    return F.linear(o, P["out_proj.weight"], P["out_proj.bias"])


@pytest.mark.parametrize("case", ["causal_core", "mask2d_core", "mask4d_composed", "bool_causal_composed"])
def test_attention_module_both_paths_match_float64(case):
    """mask None or [T, T] float: the fused RAC attention core; a [B, 1, T, T]
    mask: the composed path (batched RAC products around the CORDIC
    softmax).  Forward and every gradient against float64."""
    torch.manual_seed(3)
    d, nh, B, T = 128, 4, 2, 24
    m = rt().RACAttention(d, nh).to(DEV)
    x = torch.randn(B, T, d, device=DEV, requires_grad=True)
    mask, causal = None, False
    if case == "causal_core":
        causal = True
    elif case == "mask2d_core":
        mask = torch.randn(T, T, device=DEV) * 0.5
    elif case == "mask4d_composed":
        mask = torch.randn(B, 1, T, T, device=DEV) * 0.5
    else:
        mask = torch.zeros(1, 1, T, T, device=DEV)
        causal = True
    assert rt()._rac_core_ok(mask, T, m.dropout) == case.endswith("core")
    y = m(x, mask=mask, is_causal=causal)
    g = torch.randn_like(y)
    y.backward(g)
    P = {k: v.requires_grad_(True) for k, v in params64(m).items()}
    x64 = c64(x)
    y64 = _mha64(x64, P, nh, mask.double().cpu() if mask is not None else None, causal)
    y64.backward(g.double().cpu())
    close(y, y64, what=f"{case} forward")
    close(x.grad, x64.grad, what=f"{case} grad input")
    for name, prm in m.named_parameters():
        close(prm.grad, P[name].grad, what=f"{case} grad {name}")


def test_attention_module_paths_agree_and_eval_dropout_takes_core():
    torch.manual_seed(4)
    m = rt().RACAttention(64, 2, dropout=0.1).to(DEV)
    x = torch.randn(2, 16, 64, device=DEV)
    m.eval()
    assert rt()._rac_core_ok(None, 16, m.dropout)
    m.train()
    assert not rt()._rac_core_ok(None, 16, m.dropout)
    m.eval()
    with torch.no_grad():
        y_core = m(x, is_causal=True)
        old = rt()._rac_core_ok
        rt()._rac_core_ok = lambda *a: False
        try:
            y_comp = m(x, is_causal=True)
        finally:
            rt()._rac_core_ok = old
    close(y_core, y_comp, tol=1e-5, what="core vs composed")
    # training mode with dropout: composed path, finite and differentiable
    m.train()
    xt = x.clone().requires_grad_(True)
    y = m(xt, is_causal=True)
    y.sum().backward()
    assert torch.isfinite(y).all() and torch.isfinite(xt.grad).all()


def test_transformer_block_matches_float64():
    torch.manual_seed(5)
    d, nh, ff, B, T = 64, 4, 160, 2, 12
    blk = rt().RACTransformerBlock(d, nh, ff_dim=ff).to(DEV)
    with torch.no_grad():
        blk.norm1.weight.normal_(1.0, 0.1)
        blk.norm1.bias.normal_(0.0, 0.1)
        blk.norm2.weight.normal_(1.0, 0.1)
        blk.norm2.bias.normal_(0.0, 0.1)
    x = torch.randn(B, T, d, device=DEV, requires_grad=True)
    y = blk(x, is_causal=True)
    g = torch.randn_like(y)
    y.backward(g)
    P = {k: v.requires_grad_(True) for k, v in params64(blk).items()}
    x64 = c64(x)
    att = {k[5:]: v for k, v in P.items() if k.startswith("attn.")}
    h = F.layer_norm(x64 + _mha64(x64, att, nh, None, True), (d,), P["norm1.weight"], P["norm1.bias"], 1e-5)
    f = F.linear(_gelu64(F.linear(h, P["ffn.fc1.weight"], P["ffn.fc1.bias"])), P["ffn.fc2.weight"],
                 P["ffn.fc2.bias"])
    y64 = F.layer_norm(h + f, (d,), P["norm2.weight"], P["norm2.bias"], 1e-5)
    y64.backward(g.double().cpu())
    close(y, y64, what="block forward")
    close(x.grad, x64.grad, what="block grad input")
    for name, prm in blk.named_parameters():
        close(prm.grad, P[name].grad, what=f"block grad {name}")


def test_matmul_adaptive_threshold():
    r = rt()
    torch.manual_seed(6)
    small_a, small_b = torch.randn(8, 40, device=DEV), torch.randn(40, 16, device=DEV)
    assert 8 * 16 < r._RAC_MIN_ELEMENTS
    assert torch.equal(r.rac_matmul_adaptive(small_a, small_b), torch.matmul(small_a, small_b))
    big_a, big_b = torch.randn(96, 40, device=DEV), torch.randn(40, 64, device=DEV)
    assert 96 * 64 >= r._RAC_MIN_ELEMENTS
    got = r.rac_matmul_adaptive(big_a, big_b)
    assert torch.equal(got, r.rac_matmul(big_a, big_b))
    close(got, big_a.double().cpu() @ big_b.double().cpu(), scale=float(big_a.abs().sum(1).max()) * 4.0,
          what="adaptive large")
    cpu = r.rac_matmul_adaptive(big_a.cpu(), big_b.cpu())   # CPU tensors go to torch.matmul
    assert torch.equal(cpu, torch.matmul(big_a.cpu(), big_b.cpu()))


def test_benchmark_model_patches_and_restores():
    r = rt()
    model = torch.nn.Sequential(torch.nn.Linear(128, 256), torch.nn.ReLU(), torch.nn.Linear(256, 128))
    res = r.benchmark_model(model, (4, 128), n_warmup=2, n_iters=5)
    assert set(res) >= {"baseline_ms", "rac_ms", "speedup", "n_iters"}
    assert res["baseline_ms"] > 0 and res["rac_ms"] > 0 and res["n_iters"] == 5
    assert all(type(mod) is not r.RACLinear for mod in model.modules())


def test_rac_info_reports_loaded_library():
    buf = io.StringIO()
    with contextlib.redirect_stdout(buf):
        rt().rac_info()
    text = buf.getvalue()
    assert "NOT LOADED" not in text and "librac_amd" in text
    assert "ROCm device available: True" in text
