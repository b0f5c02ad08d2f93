"""GPU parity of the safetensors loader (bench/safetensors_reader.h) and its
device forms: widening to fp32 and quantizing to Q8_0 on the GPU against the
compiled reference reader's golden outputs and the CPU checker.

Bar: bit-exact (NaN payloads and signed zeros included) for every float
dtype, single and multi-chunk tensors, host and device destinations.
"""
import os

import numpy as np
import pytest

import raclib as rl

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda"
GOLD_FLOAT = ["f32", "f16", "bf16", "f64", "model.layers.0.mlp.up_proj.weight", "scalar", "empty"]


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    import rac_amd
    rac_amd.load()
    yield
    torch.cuda.synchronize()


def H(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


@pytest.fixture(scope="module")
def sample(tmp_path_factory):
    d = np.load(os.path.join(rl.GOLDEN, "st.npz"))
    path = tmp_path_factory.mktemp("st") / "sample.safetensors"
    path.write_bytes(d["sample"].tobytes())
    return str(path), d


def test_golden_fp32_and_q8(sample):
    from rac_amd import ext
    path, d = sample
    with ext.SafeTensors(path) as sf:
        for name in GOLD_FLOAT:
            print(f"st golden {name}", flush=True)
            got = H(sf.tensor(name)).reshape(-1)
            assert np.array_equal(got.view(np.uint32), d[f"f32_{name}"].view(np.uint32)), name
            if f"q8_{name}" in d:
                assert np.array_equal(H(sf.q8_0(name)), d[f"q8_{name}"]), name
        with pytest.raises(Exception):
            sf.tensor("i8")


def test_st_to_f32_host_and_device_destinations(sample):
    from rac_amd import _lib
    lib = _lib.load()
    path, d = sample
    import ctypes
    err = ctypes.create_string_buffer(256)
    f = lib.st_open(path.encode(), err)
    assert f, err.value
    try:
        for name in ("f16", "bf16", "f64", "f32"):
            t = lib.st_find(f, name.encode())
            n = lib.st_numel(t)
            host = np.full(n, 7.0, np.float32)
            assert lib.st_to_f32(f, t, rl.p(host)) == 0
            assert np.array_equal(host.view(np.uint32), d[f"f32_{name}"].view(np.uint32)), name
            dev = torch.full((n,), 7.0, device=DEV)
            torch.cuda.synchronize()
            assert lib.st_to_f32(f, t, dev.data_ptr()) == 0
            assert np.array_equal(H(dev).view(np.uint32), d[f"f32_{name}"].view(np.uint32)), name
    finally:
        lib.st_close(f)


def _write(path, tensors):
    """tensors: name -> (dtype string, shape, raw bytes)."""
    header, data = {}, b""
    for name, (dt, shape, raw) in tensors.items():
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [len(data), len(data) + len(raw)]}
        data += raw
    with open(path, "wb") as fh:
        fh.write(rl.st_bytes(header, data))


def test_multi_chunk_tensors_vs_oracle(tmp_path):
    from rac_amd import ext
    rng = np.random.default_rng(17)
    bf = rng.integers(0, 1 << 16, 4096 * 11008, dtype=np.uint32).astype(np.uint16)   # 3 chunks, all bit patterns
    h = (rng.normal(0, 1, 3000 * 4096).astype(np.float16)).view(np.uint16)
    h[::997] = 0x7E01                                                              # NaN payloads here and there
    f64 = rng.normal(0, 1, 1000 * 8192 + 0) * np.exp(rng.uniform(-100, 100, 1000 * 8192))
    f32 = rng.normal(0, 1, (5000, 3000)).astype(np.float32)
    spec = {"bf": ("BF16", (4096, 11008), bf.tobytes()), "h": ("F16", (3000, 4096), h.tobytes()),
            "d": ("F64", (1000, 8192), f64.tobytes()), "f": ("F32", (5000, 3000), f32.tobytes())}
    path = tmp_path / "big.safetensors"
    _write(path, spec)
    with ext.SafeTensors(str(path)) as sf:
        for name, (dt, shape, raw) in spec.items():
            print(f"st multi-chunk {name} {dt} {shape}", flush=True)
            n = int(np.prod(shape))
            ref = rl.orc_st_to_f32(rl.ST_DTYPES[dt], raw, n)
            got = H(sf.tensor(name)).reshape(-1)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), name
            if shape[-1] % 32 == 0:
                q = H(sf.q8_0(name))
                idx = np.random.default_rng(1).choice(q.shape[0], min(64, q.shape[0]), replace=False)
                refq = rl.orc_q8_quantize(ref.reshape(shape[0], -1)[idx].reshape(-1, shape[-1]))
                assert np.array_equal(q[idx], refq.reshape(q[idx].shape)), name
            del raw


def test_device_raw_conversions_unaligned_and_tails():
    from rac_amd import _lib
    lib = _lib.load()
    rng = np.random.default_rng(23)
    st = torch.cuda.current_stream().cuda_stream
    for dt, es in ((2, 2), (3, 2), (4, 8), (1, 4)):
        for n, shift in ((1, 0), (13, 0), (1000, 2 * es if es < 8 else 8), (4099, 0)):
            print(f"st convert dtype {dt} n {n} shift {shift}", flush=True)
            raw = rng.integers(0, 256, n * es, dtype=np.uint8)
            if dt == 4:   # finite doubles (the NaN rule is covered by the golden file)
                raw = (rng.normal(0, 1, n) * 1e3).tobytes()
                raw = np.frombuffer(raw, np.uint8).copy()
            buf = torch.zeros(n * es + 64, dtype=torch.uint8, device=DEV)
            buf[shift:shift + n * es] = torch.from_numpy(raw).to(DEV)
            out = torch.zeros(n + 8, device=DEV)
            dst = out[1:] if shift else out
            assert lib.rac_st_convert_dev(dt, buf.data_ptr() + shift, n, dst.data_ptr(), st) == 0
            ref = rl.orc_st_to_f32(dt, raw.tobytes(), n)
            assert np.array_equal(H(dst)[:n].view(np.uint32), ref.view(np.uint32)), (dt, n, shift)
        # quantize from raw device bytes, aligned and not
        nb = 37
        raw = (rng.normal(0, 1, nb * 32) * 3).astype({2: np.float16, 3: np.float32, 4: np.float64, 1: np.float32}[dt])
        if dt == 3:
            raw = (raw.view(np.uint32) >> 16).astype(np.uint16)
        rb = np.frombuffer(raw.tobytes(), np.uint8).copy()
        ref = rl.orc_q8_quantize(rl.orc_st_to_f32(dt, rb.tobytes(), nb * 32).reshape(1, -1))
        for shift in (0, 2):
            buf = torch.zeros(rb.size + 64, dtype=torch.uint8, device=DEV)
            buf[shift:shift + rb.size] = torch.from_numpy(rb).to(DEV)
            q = torch.zeros(nb * 34, dtype=torch.uint8, device=DEV)
            assert lib.rac_st_quantize_dev(dt, buf.data_ptr() + shift, nb, q.data_ptr(), st) == 0
            assert np.array_equal(H(q), ref.reshape(-1)), (dt, shift)


def test_device_half_widening_every_pattern():
    """F16 and BF16 -> F32 on the device for all 65536 bit patterns (zeros,
    subnormal halves, infinities, NaN payloads): bit-exact with the
    checker's restatement of the reference reader."""
    from rac_amd import _lib
    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    raw = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    rb = np.frombuffer(raw.tobytes(), np.uint8).copy()
    for dt in (2, 3):
        buf = torch.from_numpy(rb).to(DEV)
        out = torch.zeros(65536, device=DEV)
        assert lib.rac_st_convert_dev(dt, buf.data_ptr(), 65536, out.data_ptr(), st) == 0
        ref = rl.orc_st_to_f32(dt, rb.tobytes(), 65536)
        assert np.array_equal(H(out).view(np.uint32), ref.view(np.uint32)), dt


def test_loader_feeds_the_q8_gemv(sample):
    """End to end: weights from the file, quantized on the GPU, drive the
    decode GEMV exactly as the reference's load-then-quantize path does."""
    from rac_amd import ext
    path, d = sample
    name = "model.layers.0.mlp.up_proj.weight"
    x = np.random.default_rng(3).normal(0, 1, (1, 64)).astype(np.float32)
    with ext.SafeTensors(path) as sf:
        wq = sf.q8_0(name)
        y = H(ext.q8_gemv(torch.from_numpy(x).to(DEV), wq))
    ref = rl.orc_q8_gemv(x, d[f"q8_{name}"], None, 0)
    assert np.array_equal(y, ref)
