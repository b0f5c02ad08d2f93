"""GPU parity of the RAC-DSP fixed-point CORDIC engine (sim/rac_dsp_core.c)
against the CPU checker, itself bit-exact with the compiled reference model
and pinned by closed forms in test_oracle.py.

Bar: bit-exact (integer datapath) for every op, the systolic product, the
rac_dsp.h host entry points and replaced ROMs; at the benchmark size through
a seeded sample of indices.
"""
import ctypes

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


def golden():
    return np.load(rl.GOLDEN + "/dsp.npz")


def _inputs(n, seed):
    rng = np.random.default_rng(seed)
    x = rng.integers(-2 ** 62, 2 ** 62, n, dtype=np.int64)
    y = rng.integers(-2 ** 62, 2 ** 62, n, dtype=np.int64)
    z = rng.integers(-2 ** 63, 2 ** 63 - 1, n, dtype=np.int64)
    x[: n // 4] >>= 22                                       # in-range magnitudes as well as wrapping ones
    y[: n // 4] >>= 22
    return x, y, z


@pytest.mark.parametrize("op", [0, 1, 2, 3])
def test_eval_bit_exact_vs_reference_golden(op):
    print(f"dsp golden op {op}", flush=True)
    d = golden()
    xo, yo, zo = ext().dsp_eval(op, T(d["x"]), T(d["z"]), T(d["y"]))
    assert np.array_equal(np.stack([H(xo), H(yo), H(zo)], 1), d[f"op{op}"])


@pytest.mark.parametrize("op", [0, 1, 2, 3, 6])
@pytest.mark.parametrize("n", [1, 255, 4099, 1 << 20])
def test_eval_bit_exact_vs_oracle(op, n):
    print(f"dsp eval op {op} n {n}", flush=True)
    x, y, z = _inputs(n, 1000 + n + op)
    ref = rl.orc_dsp_batch(op, x, y, z)
    got = ext().dsp_eval(op, T(x), T(z), T(y))
    for a, b in zip(got, ref):
        assert np.array_equal(H(a), b)


def test_eval_without_y_and_optional_outputs():
    from rac_amd import _lib
    e = ext()
    lib = _lib.load()
    x, y, z = _inputs(5000, 9)
    ref = rl.orc_dsp_batch(1, x, np.zeros_like(x), z)
    xo, yo, zo = e.dsp_eval("project", T(x), T(z))
    assert np.array_equal(H(xo), ref[0]) and np.array_equal(H(yo), ref[1]) and np.array_equal(H(zo), ref[2])
    tx, tz = T(x), T(z)
    out = torch.zeros_like(tx)
    assert lib.rac_dsp_eval_dev(1, x.size, tx.data_ptr(), None, tz.data_ptr(), out.data_ptr(), None, None,
                                torch.cuda.current_stream().cuda_stream) == 0
    assert np.array_equal(H(out), ref[0])


def test_eval_sampled_at_benchmark_size():
    n = 1 << 24
    print(f"dsp eval sampled n {n}", flush=True)
    x, y, z = _inputs(n, 24)
    idx = np.random.default_rng(3).choice(n, 8192, replace=False)
    for op in (1, 3):
        got = ext().dsp_eval(op, T(x), T(z), T(y))
        ref = rl.orc_dsp_batch(op, x[idx], y[idx], z[idx])
        for a, b in zip(got, ref):
            assert np.array_equal(H(a)[idx], b)


def test_systolic_vs_reference_golden_and_oracle():
    d = golden()
    Y = ext().dsp_systolic(T(d["W"]), T(d["X"]))
    assert np.array_equal(H(Y), d["Y"])
    o = rl.oracle()
    rng = np.random.default_rng(11)
    for N, K in ((1, 1), (64, 37), (200, 5), (33, 300)):
        print(f"dsp systolic N {N} K {K}", flush=True)
        W = rng.integers(-2 ** 63, 2 ** 63 - 1, (N, N), dtype=np.int64)
        X = rng.integers(-2 ** 40, 2 ** 40, (K, N), dtype=np.int64)
        ref = np.zeros((K, N), np.int64)
        o.orc_dsp_systolic(N, K, rl.p(W), rl.p(X), rl.p(ref))
        assert np.array_equal(H(ext().dsp_systolic(T(W), T(X))), ref), (N, K)


def test_rac_dsp_h_host_entry_points():
    from rac_amd import _lib
    lib = _lib.load()
    d = golden()
    a, b, c = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    for i in range(0, 1500, 97):
        for op in range(4):
            lib.rac_dsp_eval(int(d["x"][i]), int(d["y"][i]), int(d["z"][i]), op, ctypes.byref(a), ctypes.byref(b),
                             ctypes.byref(c))
            assert (a.value, b.value, c.value) == tuple(int(v) for v in d[f"op{op}"][i]), (i, op)
    # project_batch on host pointers, then on device pointers
    xs, zs = d["x"], d["z"]
    ref = rl.orc_dsp_batch(1, xs, np.zeros_like(xs), zs)[0]
    out = np.zeros_like(xs)
    lib.rac_dsp_project_batch(xs.size, rl.p(xs), rl.p(zs), rl.p(out))
    assert np.array_equal(out, ref)
    tx, tz, to = T(xs), T(zs), torch.zeros(xs.size, dtype=torch.int64, device=DEV)
    lib.rac_dsp_project_batch(xs.size, tx.data_ptr(), tz.data_ptr(), to.data_ptr())
    assert np.array_equal(H(to), ref)
    # one systolic column = rac_dsp_project_sum (golden written through it)
    W, X, Y = d["W"], d["X"], d["Y"]
    for k in range(X.shape[0]):
        for col in range(W.shape[1]):
            wc, xk = np.ascontiguousarray(W[:, col]), np.ascontiguousarray(X[k])
            assert lib.rac_dsp_project_sum(W.shape[0], rl.p(xk), rl.p(wc)) == Y[k, col]


def test_replaced_roms_reach_the_device():
    from rac_amd import _lib
    lib = _lib.load()
    o = rl.oracle()
    d = golden()
    g_lut, g_at, g_ath = d["lut"], d["atan"], d["atanh"]
    lut2 = np.ascontiguousarray(g_lut[::-1])
    at2 = np.ascontiguousarray(g_at + 12345)
    ath2 = np.ascontiguousarray(g_ath - 777)
    x, y, z = _inputs(20000, 5)
    try:
        lib.rac_dsp_set_roms(rl.p(lut2), rl.p(at2), rl.p(ath2))
        o.orc_dsp_set_roms(rl.p(lut2), rl.p(at2), rl.p(ath2))
        for op in range(4):
            got = ext().dsp_eval(op, T(x), T(z), T(y))
            ref = rl.orc_dsp_batch(op, x, y, z)
            for a, b in zip(got, ref):
                assert np.array_equal(H(a), b), op
    finally:
        lib.rac_dsp_set_roms(rl.p(g_lut), rl.p(g_at), rl.p(g_ath))
        o.orc_dsp_set_roms(rl.p(g_lut), rl.p(g_at), rl.p(g_ath))
    xo = ext().dsp_eval(0, T(d["x"]), T(d["z"]), T(d["y"]))[0]
    assert np.array_equal(H(xo), d["op0"][:, 0])
