"""rac_attention_noalloc_dev, the allocation-free attention entry point,
against rac_attention_dev (workspace argument): bit-identical outputs on two
calls in a row, the second with a smaller input, through the C ABI; and
shapes past its limit refused before any device work."""
import ctypes

import numpy as np
import pytest

import raclib as rl

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    import rac_amd
    return rac_amd.load()


def _run(lib, q, k, v, mask, causal, iters, mode, noalloc):
    B, Hh, Tn, D = q.shape
    qt, kt, vt = (torch.from_numpy(np.ascontiguousarray(a)).to(DEV) for a in (q, k, v))
    mt = torch.from_numpy(mask).to(DEV) if mask is not None else None
    mp = mt.data_ptr() if mt is not None else None
    out = torch.full_like(qt, float("nan"))
    stream = torch.cuda.current_stream().cuda_stream
    print(f"no-alloc attention shape={q.shape} causal={causal} iters={iters} mode={mode} noalloc={noalloc}",
          flush=True)
    if noalloc:
        rc = lib.rac_attention_noalloc_dev(qt.data_ptr(), kt.data_ptr(), vt.data_ptr(), mp, int(causal),
                                           out.data_ptr(), B, Hh, Tn, D, iters, mode, stream)
    else:
        ws = torch.empty(lib.rac_attention_workspace_bytes(B, Hh, Tn) // 4, device=DEV)
        rc = lib.rac_attention_dev(qt.data_ptr(), kt.data_ptr(), vt.data_ptr(), mp, int(causal), out.data_ptr(),
                                   B, Hh, Tn, D, ws.data_ptr(), iters, mode, stream)
    assert rc == 0, lib.rac_last_error()
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _qkv(shape, seed):
    return tuple(rl.gen_normal(shape, seed=seed + i) for i in range(3))


def test_noalloc_attention_matches_workspace_entry_twice(lib):
    # call 1: config 5's attention core, [1, 32, 2048, 128] causal, n = 16
    # (256 query rows per chunk in the scratch)
    q, k, v = _qkv((1, 32, 2048, 128), seed=800)
    got = _run(lib, q, k, v, None, True, 16, 1, noalloc=True)
    ref = _run(lib, q, k, v, None, True, 16, 1, noalloc=False)
    assert np.isfinite(got).all() and np.array_equal(got, ref)
    # call 2, smaller: [2, 3, 200, 32], additive mask, not causal, n = 8 (one
    # chunk); the scratch still holds call 1's scores
    q2, k2, v2 = _qkv((2, 3, 200, 32), seed=810)
    mask = (rl.gen_normal((200, 200), seed=813) * np.float32(0.5)).astype(np.float32)
    got2 = _run(lib, q2, k2, v2, mask, False, 8, 1, noalloc=True)
    ref2 = _run(lib, q2, k2, v2, mask, False, 8, 1, noalloc=False)
    assert np.isfinite(got2).all() and np.array_equal(got2, ref2)
    assert np.array_equal(got2, rl.orc_attention_lanes(q2, k2, v2, mask, False, 8, 1))
    # call 3, causal again at a third shape, FAST products
    q3, k3, v3 = _qkv((1, 4, 333, 64), seed=820)
    got3 = _run(lib, q3, k3, v3, None, True, 24, 0, noalloc=True)
    assert np.array_equal(got3, _run(lib, q3, k3, v3, None, True, 24, 0, noalloc=False))


def test_noalloc_attention_refuses_beyond_scratch(lib):
    buf = (ctypes.c_float * 64)()
    a = ctypes.addressof(buf)
    # batch*n_heads*seq = 16777216: one query row of every head is 64 MiB,
    # past the limit; refused before any device work
    lib.rac_clear_error()
    assert lib.rac_attention_noalloc_dev(a, a, a, None, 1, a, 1, 64, 262144, 4, 16, 1, None) == -2
    assert b"16777215" in lib.rac_last_error()
