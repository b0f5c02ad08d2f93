"""rac_attention_noalloc_dev, the allocation-free attention entry point,
against rac_attention_dev (workspace argument): bit-identical outputs on two
calls in a row, the second with a smaller input, through the C ABI; and the
same call recorded in a HIP graph and replayed.  (Shapes past its limit are
refused before any device work: tests/test_capi.py, on the CPU.)"""
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


def test_noalloc_attention_recorded_in_a_graph_replays_bit_identical(lib):
    """The call recorded under stream capture (torch.cuda.graph) and replayed
    three times, with eager work (including another no-alloc call, which
    overwrites the shared scratch) and synchronisation between the replays:
    every replay equals the eager call bit for bit.  The eager call comes
    first, so the scratch address is resolved outside the capture."""
    q, k, v = _qkv((1, 4, 256, 64), seed=830)
    eager = _run(lib, q, k, v, None, True, 16, 1, noalloc=True)
    q2, k2, v2 = _qkv((2, 2, 96, 32), seed=840)
    other = _run(lib, q2, k2, v2, None, False, 8, 1, noalloc=True)
    qt, kt, vt = (torch.from_numpy(np.ascontiguousarray(a)).to(DEV) for a in (q, k, v))
    out = torch.full_like(qt, float("nan"))
    torch.cuda.synchronize()
    print("recording rac_attention_noalloc_dev [1, 4, 256, 64] causal n=16 in a graph", flush=True)
    g = torch.cuda.CUDAGraph()
    rcs = []
    with torch.cuda.graph(g):
        stream = torch.cuda.current_stream().cuda_stream
        rcs.append(lib.rac_attention_noalloc_dev(qt.data_ptr(), kt.data_ptr(), vt.data_ptr(), None, 1,
                                                 out.data_ptr(), 1, 4, 256, 64, 16, 1, stream))
    assert rcs == [0], lib.rac_last_error()
    for rep in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        print(f"replay {rep}", flush=True)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), eager), f"replay {rep}"
        assert np.array_equal(_run(lib, q2, k2, v2, None, False, 8, 1, noalloc=True), other)
    del g
    torch.cuda.synchronize()
