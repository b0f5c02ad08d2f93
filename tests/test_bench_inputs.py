"""bench.py's device-side input generator against the NumPy twin that the
parity tests use (tests/raclib.py): uniforms bit for bit, normals within one
float32 ulp (float64 log / cos of torch's CPU or device library vs NumPy's);
on the CPU here, and on the GPU under -m gpu."""
import os
import sys

import numpy as np
import pytest

import raclib as rl

torch = pytest.importorskip("torch")
sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import bench  # noqa: E402


def _check(dev):
    for seed in (0, 1, 7, 123456789):
        u = bench.dev_u01(4099, seed, dev).cpu().numpy()
        assert np.array_equal(u, rl.gen_u01(4099, seed)), seed
        a = bench.dev_uniform((33, 65), seed, dev).cpu().numpy()
        assert np.array_equal(a, rl.gen_uniform((33, 65), seed)), seed
        n = bench.dev_normal((129, 31), seed, dev, mean=1.0, std=0.02).cpu().numpy()
        ref = rl.gen_normal((129, 31), seed, mean=1.0, std=0.02)
        ulp = np.abs(n.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
        assert ulp.max() <= 1, (seed, int(ulp.max()))


def test_generator_matches_numpy_twin_cpu():
    _check("cpu")


@pytest.mark.gpu
def test_generator_matches_numpy_twin_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    _check("cuda")
