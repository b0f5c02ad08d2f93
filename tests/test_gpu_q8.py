"""GPU parity of the Q8_0 weight format and decode GEMV (lib/c/rac_q8_0.h)
against the CPU checker (itself bit-exact with the compiled reference, see
test_oracle.py).

Bars: quantize / dequantize bit-exact; GEMV bit-exact for activation NONE and
RELU (same block-dot tree and block-order fma accumulation); GELU / SiLU
within the device-vs-glibc erff / expf rounding.
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


def _weights(N, K, seed):
    rng = np.random.default_rng(seed)
    W = rng.normal(0, 0.05, (N, K)).astype(np.float32)
    W[0, :32] = 0.0
    if N > 3:
        W[3, 5] = 30.0
        W[min(N - 1, 4), K - 32:] = 1e-30
    return W


def test_quantize_dequantize_bit_exact():
    e = ext()
    for (N, K) in ((1, 32), (40, 512), (300, 4096), (7, 11008)):
        print(f"q8 quantize {N}x{K}", flush=True)
        W = _weights(N, K, N + K)
        wq = H(e.q8_quantize(T(W)))
        ref = rl.orc_q8_quantize(W)
        assert np.array_equal(wq, ref)
        deq = H(e.q8_dequantize(T(ref)))
        dref = np.zeros((N, K), np.float32)
        rl.oracle().orc_q8_0_dequantize(rl.p(ref), rl.p(dref), N, K)
        assert np.array_equal(deq.view(np.uint32), dref.view(np.uint32))
    # special values: inf / nan in a block, and a block whose 1/d overflows
    W = np.ones((1, 96), np.float32)
    W[0, 3] = np.inf
    W[0, 40] = np.nan
    W[0, 64:96] = np.float32(1e-38) * np.linspace(-1, 1, 32, dtype=np.float32)
    assert np.array_equal(H(e.q8_quantize(T(W))), rl.orc_q8_quantize(W))


# K = 256 / 768: rows shorter than one 32-block chunk (8-block chunks);
# 1280: one full chunk plus a last chunk that overlaps it by 24 blocks;
# 96 / 800: K % 256 != 0 (generic kernel)
@pytest.mark.parametrize("K", [256, 768, 1280, 4096, 96, 800])
@pytest.mark.parametrize("M", [1, 3, 4, 7, 16])
def test_gemv_vs_oracle(K, M):
    e = ext()
    N = 200
    W = _weights(N, K, K)
    wq = rl.orc_q8_quantize(W)
    rng = np.random.default_rng(M)
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    bias = rng.normal(0, 1, N).astype(np.float32)
    for act in range(4):
        for b in (None, bias):
            print(f"q8 gemv M={M} K={K} act={act} bias={b is not None}", flush=True)
            got = H(e.q8_gemv(T(x), T(wq), T(b) if b is not None else None, act))
            ref = rl.orc_q8_gemv(x, wq, b, act)
            if act in (0, 1):
                assert np.array_equal(got, ref)
            else:
                assert np.all(np.abs(got - ref) <= 1e-6 * (np.abs(ref) + 1.0)), float(np.max(np.abs(got - ref)))


def test_gemv_every_fp16_scale():
    """Row r's first block carries the fp16 scale with bit pattern r (all
    65536: zeros, subnormal halves, infinities, NaN payloads), the other
    blocks scale 0: the device fp16 decode and the block-order fold
    bit-exact with the checker, fast and generic kernels."""
    N, K = 65536, 256
    rng = np.random.default_rng(5)
    wq = np.zeros((N, K // 32, 34), np.uint8)
    wq[:, :, 2:] = rng.integers(0, 256, (N, K // 32, 32), dtype=np.uint8)
    r = np.arange(N, dtype=np.uint32)
    wq[:, 0, 0] = (r & 0xFF).astype(np.uint8)
    wq[:, 0, 1] = (r >> 8).astype(np.uint8)
    x = rng.normal(0, 1, K).astype(np.float32)
    e = ext()
    ref = rl.orc_q8_gemv(x, wq, None, 0)[0]
    got = H(e.q8_gemv(T(x), T(wq), None, 0))
    assert np.array_equal(got, ref, equal_nan=True)
    # the fast kernel decodes the scale by the hardware conversion, the
    # generic kernel (weights not 16-byte aligned) by the bit operations of
    # rac_fp16_to_fp32: their outputs agree bit for bit, NaN payloads included
    buf = torch.empty(wq.size + 2, dtype=torch.uint8, device=DEV)
    buf[2:] = T(wq.reshape(-1))
    wmis = buf[2:].view(wq.shape)
    assert wmis.data_ptr() % 16 == 2
    for act in range(4):
        fast = e.q8_gemv(T(x), T(wq), None, act).view(torch.int32)
        gen = e.q8_gemv(T(x), wmis, None, act).view(torch.int32)
        assert torch.equal(fast, gen), act
    K2 = 224                                      # K % 256 != 0: generic kernel
    ref2 = rl.orc_q8_gemv(x[:K2], np.ascontiguousarray(wq[:, :K2 // 32]), None, 0)[0]
    got2 = H(e.q8_gemv(T(x[:K2]), T(np.ascontiguousarray(wq[:, :K2 // 32])), None, 0))
    assert np.array_equal(got2, ref2, equal_nan=True)


def test_gemv_unaligned_input_takes_generic_path():
    e = ext()
    N, K = 70, 512
    W = _weights(N, K, 3)
    wq = rl.orc_q8_quantize(W)
    x = np.random.default_rng(9).normal(0, 1, K + 1).astype(np.float32)
    xt = T(x)[1:]              # 4-byte offset: not 16-byte aligned
    got = H(e.q8_gemv(xt, T(wq), None, 0))
    assert np.array_equal(got, rl.orc_q8_gemv(x[1:], wq, None, 0)[0])


def test_gemv_llama_shapes_bit_exact():
    e = ext()
    for (N, K) in ((11008, 4096), (4096, 11008), (4096, 4096)):
        print(f"q8 gemv llama shape {N}x{K}", flush=True)
        W = _weights(N, K, N)
        wq = rl.orc_q8_quantize(W)
        x = np.random.default_rng(K).normal(0, 1, K).astype(np.float32)
        got = H(e.q8_gemv(T(x), T(wq), None, 0))
        assert np.array_equal(got, rl.orc_q8_gemv(x, wq, None, 0)[0])


@pytest.mark.parametrize("N,K", [(12301, 256), (14336, 4096), (12288, 2048)])
def test_gemv_wide_launch_bit_exact(N, K):
    """N >= 12288 takes 32 rows per workgroup: full and ragged last
    workgroups, one and several chunks along K, bias and activations."""
    e = ext()
    W = _weights(N, K, N + K)
    wq = rl.orc_q8_quantize(W)
    rng = np.random.default_rng(N)
    x = rng.normal(0, 1, K).astype(np.float32)
    bias = rng.normal(0, 1, N).astype(np.float32)
    for act, b in ((0, None), (1, bias), (3, bias)):
        print(f"q8 gemv wide N={N} K={K} act={act}", flush=True)
        got = H(e.q8_gemv(T(x), T(wq), T(b) if b is not None else None, act))
        ref = rl.orc_q8_gemv(x, wq, b, act)[0]
        if act in (0, 1):
            assert np.array_equal(got, ref)
        else:
            assert np.all(np.abs(got - ref) <= 1e-6 * (np.abs(ref) + 1.0)), float(np.max(np.abs(got - ref)))


def test_reference_api_golden_host_pointers():
    import os
    import rac_amd
    L = rac_amd.load()
    d = dict(np.load(os.path.join(rl.GOLDEN, "q8.npz")))   # arrays held: their pointers go to C
    W, wq_ref, x, bias = d["W"], d["wq"], d["x"], d["bias"]
    N, K = W.shape
    wq = np.zeros_like(wq_ref)
    L.rac_q8_0_quantize_matrix(rl.p(W), rl.p(wq), N, K)
    assert np.array_equal(wq, wq_ref)
    for act in range(4):
        for with_bias in (0, 1):
            out = np.zeros(N, np.float32)
            rc = L.rac_q8_0_gemv(rl.p(x), rl.p(wq_ref), rl.p(bias) if with_bias else None, rl.p(out), N, K, act)
            assert rc == 0, L.rac_last_error()
            ref = d[f"out_a{act}_b{with_bias}"]
            if act in (0, 1):
                assert np.array_equal(out, ref), (act, with_bias)
            else:
                assert np.all(np.abs(out - ref) <= 1e-6 * (np.abs(ref) + 1.0)), (act, with_bias)
    row = np.zeros(K, np.float32)
    w1 = np.ascontiguousarray(wq_ref[1])
    L.rac_q8_0_dequantize_row(rl.p(w1), rl.p(row), K)
    ref = np.zeros(K, np.float32)
    rl.oracle().orc_q8_0_dequantize(rl.p(w1), rl.p(ref), 1, K)
    assert np.array_equal(row, ref)
