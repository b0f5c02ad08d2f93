#!/usr/bin/env python3
"""bench.py — the RAC rotation-accumulate hot path on one MI355X.

Headline metric: rac_matmul equiv-GFLOP/s at 4096^3 with 16 CORDIC
iterations; RoPE / softmax / RMSNorm HBM GB/s.  A "step" is one 4096^3
CORDIC-16 matmul (rotate-project-accumulate: 16 micro-rotations per MAC)
over synthetic U[-1,1] operands resident in HBM.  value = 2*4096^3 / t.

Also measured in the same run (fields "ops" and "cpu_baseline"):
  * the matmul at n = 8 and 24, and config 1 (1024^3, n = 16) both
    device-resident and through the synchronous rac.h call on host buffers,
    and in FAST mode (the rac_torch default MAC, on the matrix cores);
  * decode-time linears (one token: 1x4096x4096, 1x11008x4096) and a
    matrix-vector product (4096x4096 by a vector), FAST and CORDIC n = 16;
  * the Llama block (config 5) at n = 8/16/24 with a per-op breakdown, and
    in rac_torch's default configuration (FAST): forward, per-op breakdown
    and one training step (forward + backward);
  * the config-5 attention core through RAC ([1,32,2048,128], causal, n=16)
    and the Q8_0 decode GEMV (11008x4096, 32000x4096, 65536x8192; HBM GB/s);
  * the decoder stack over those kernels (tinyllama shape, 22 layers):
    prefill of 128 tokens and decode per token, eager and as a HIP graph;
  * softmax 4096x4096 N(0, std 2) at n = 8/16/24, RoPE on Q and K
    [8,32,4096,128], RMSNorm 16384x4096, SiLU 16384x11008 (n=16): HBM GB/s
    of 1 read + 1 write per element, buffers rotated past the 256 MB MALL;
  * the reference lib/c on the host cores (oracle/_ref, compiled from the
    reference sources): rac_hal_matmul 4096^3 and 1024^3, softmax, RoPE,
    RMSNorm, SiLU (rac_hal_silu), the Q8_0 GEMV and the RAC-DSP batch,
    timed in a child process.

Each "ms"/"us" figure is the average over back-to-back calls (HIP events
on the launch stream); p10 / median / p90 are of separately bracketed calls,
which also carry each launch's ramp-up and drain, so for kernels of tens of
microseconds they sit above the back-to-back average.

Roofline of the dominant kernel (the matmul): VALU-bound; algorithmic work
per MAC is W(n) = 2n+1 FP32 FMA lane-ops (n micro-rotations on the (x, y)
pair plus the projecting FMA), i.e. 2*(2n+1) FLOP; achieved = that over the
kernel's average launch time (HIP events on the launch stream); peak =
MI355X FP32 vector 157.3 TFLOP/s.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--iters 16]
                       [--no-cpu-baseline] [--matmul-only] [--rowops-only]
                       [--q8-only] [--decode-only]
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBPS = 8000.0


class Timing(float):
    """Seconds per call, averaged over back-to-back calls, carrying the
    10th / 50th / 90th percentiles of separately bracketed calls."""
    p10 = p50 = p90 = None


def _percentiles(vals):
    v = sorted(vals)
    pick = lambda q: v[min(len(v) - 1, int(round(q * (len(v) - 1))))]  # noqa: E731
    return pick(0.1), pick(0.5), pick(0.9)


def _events_time(fn, reps, torch, warm_s=0.03, min_timed_s=0.02, dist_calls=20):
    """Average time of fn() per call from HIP events on the current stream.

    The GPU's clocks drop while it idles (host-side phases of this script)
    and take milliseconds to recover, so fn() first runs for ~warm_s of
    wall time; the timed region then repeats it at least `reps` times and
    for at least ~min_timed_s.  Then `dist_calls` more calls, each between
    its own pair of events, give the per-call percentiles."""
    t0 = time.perf_counter()
    k = 0
    while True:
        fn()
        k += 1
        if k % 4 == 0 or k == 1:
            torch.cuda.synchronize()
            if time.perf_counter() - t0 >= warm_s:
                break
    est = (time.perf_counter() - t0) / k
    reps = max(reps, min(2000, int(min_timed_s / max(est, 1e-7)) + 1))
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    e.synchronize()
    out = Timing(s.elapsed_time(e) / reps / 1e3)
    if dist_calls:
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(dist_calls)]
        for a, b in ev:
            a.record()
            fn()
            b.record()
        torch.cuda.synchronize()
        out.p10, out.p50, out.p90 = _percentiles([a.elapsed_time(b) / 1e3 for a, b in ev])
    return out


# The configs' seeded generator, evaluated on the device: u =
# (splitmix64(seed * 0xD1B54A32D192ED03 + i) >> 40) * 2^-24; uniform lo +
# (hi - lo) u; normal by Box-Muller in float64 from the pairs (u_2i, u_2i+1),
# cast to float32.  The NumPy twin is tests/raclib.py (gen_u01 / gen_uniform
# / gen_normal): the same uniforms bit for bit; normals agree but for rare
# last-bit differences of the device's float64 log and cos.  int64 tensor
# arithmetic wraps like uint64; logical right shifts are masked.
_M64 = (1 << 64) - 1


def _s64(v):
    v &= _M64
    return v - (1 << 64) if v >= (1 << 63) else v


def _lsr(x, s):
    return (x >> s) & ((1 << (64 - s)) - 1)


def dev_u01(count, seed, dev):
    import torch
    x = torch.arange(count, dtype=torch.int64, device=dev) + _s64(seed * 0xD1B54A32D192ED03)
    x = x + _s64(0x9E3779B97F4A7C15)
    x = (x ^ _lsr(x, 30)) * _s64(0xBF58476D1CE4E5B9)
    x = (x ^ _lsr(x, 27)) * _s64(0x94D049BB133111EB)
    x = x ^ _lsr(x, 31)
    return _lsr(x, 40).to(torch.float64) * (1.0 / 16777216.0)


def dev_uniform(shape, seed, dev, lo=-1.0, hi=1.0):
    n = 1
    for d in shape:
        n *= d
    return (lo + (hi - lo) * dev_u01(n, seed, dev)).float().reshape(shape)


def dev_normal(shape, seed, dev, mean=0.0, std=1.0):
    import math
    import torch
    n = 1
    for d in shape:
        n *= d
    u = dev_u01(2 * n, seed, dev)
    r = torch.sqrt(-2.0 * torch.log(1.0 - u[0::2]))
    out = (mean + std * r * torch.cos(2.0 * math.pi * u[1::2])).float().reshape(shape)
    del u, r
    return out


def _dist_fields(t, scale, unit):
    """p10 / median / p90 of a Timing in `unit` (empty if it has none)."""
    if getattr(t, "p50", None) is None:
        return {}
    return {f"p10_{unit}": round(t.p10 * scale, 3), f"median_{unit}": round(t.p50 * scale, 3),
            f"p90_{unit}": round(t.p90 * scale, 3)}


def bench_gpu(args):
    import torch

    sys.path.insert(0, ROOT)
    from rac_amd import ext

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    M = N = K = 4096
    A = dev_uniform((M, K), 0, dev)
    B = dev_uniform((K, N), 1, dev)
    C = torch.empty((M, N), device=dev)
    lib = ext._lib.load()
    stream = torch.cuda.current_stream(dev).cuda_stream

    def mm(n):
        rc = lib.rac_gemm_dev(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, 0, 0, 1.0, 0.0,
                              n, ext.MODE_CORDIC, stream)
        if rc:
            raise RuntimeError(lib.rac_last_error())

    n = args.iters
    for _ in range(args.warmup):
        mm(n)
    torch.cuda.synchronize()
    # timed region: exactly `steps` steps, synchronised on both sides
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(args.steps)]
    t0 = time.perf_counter()
    for a, b in ev:
        a.record()
        mm(n)
        b.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    launch_s = Timing(sum(a.elapsed_time(b) for a, b in ev) / len(ev) / 1e3)
    launch_s.p10, launch_s.p50, launch_s.p90 = _percentiles([a.elapsed_time(b) / 1e3 for a, b in ev])
    ms_per_step = wall / args.steps * 1e3
    print(f"# matmul 4096^3 CORDIC n={n}: {launch_s * 1e3:.2f} ms/launch, wall {ms_per_step:.2f} ms/step",
          file=sys.stderr, flush=True)

    ops = {"matmul_4096_cordic": {}}
    for nn in (8, 16, 24):
        if nn == n:
            t = launch_s
        else:
            mm(nn)
            torch.cuda.synchronize()
            t = _events_time(lambda: mm(nn), max(3, args.steps // 4), torch)
        w = 2 * nn + 1
        ops["matmul_4096_cordic"][f"n{nn}"] = {
            "ms": round(t * 1e3, 3),
            "equiv_GFLOPs": round(2 * M * N * K / t / 1e9, 1),
            "valu_TFLOPs": round(M * N * K * 2 * w / t / 1e12, 2),
            "frac_of_fp32_peak": round(M * N * K * 2 * w / t / 1e12 / PEAK_FP32_TFLOPS, 4),
            **_dist_fields(t, 1e3, "ms"),
        }
        print(f"# matmul n={nn}: {t * 1e3:.2f} ms", file=sys.stderr, flush=True)

    # FAST mode (the rac_torch default, rac_kernels.hip:55-62): the plain
    # fmaf(a, b, acc) MAC, 2 FLOP per MAC; at this size it runs on the FP32
    # matrix cores (one fused MAC per k), whose dense peak equals the VALU's
    def mmf():
        rc = lib.rac_gemm_dev(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, 0, 0, 1.0, 0.0,
                              24, ext.MODE_FAST, stream)
        if rc:
            raise RuntimeError(lib.rac_last_error())

    t = _events_time(mmf, 10, torch)
    ops["matmul_4096_fast"] = {"ms": round(t * 1e3, 3), "GFLOPs": round(2 * M * N * K / t / 1e9, 1),
                               "frac_of_fp32_peak": round(2 * M * N * K / t / 1e12 / PEAK_FP32_TFLOPS, 4),
                               **_dist_fields(t, 1e3, "ms")}
    print(f"# matmul FAST: {t * 1e3:.2f} ms", file=sys.stderr, flush=True)
    del A, B, C

    # Benchmark config 1: rac_matmul 1024^3, U[-1,1], CORDIC n = 16.  Device-
    # resident launch time, and the synchronous rac.h call on host buffers
    # (rac_matmul(A, B, C, M, N, K) with the knobs at 16 / cordic: staging
    # over PCIe included, reported only)
    import numpy as np
    M1 = 1024
    A1 = dev_uniform((M1, M1), 0, dev)
    B1 = dev_uniform((M1, M1), 1, dev)
    C1 = torch.empty((M1, M1), device=dev)

    def mm1():
        rc = lib.rac_gemm_dev(A1.data_ptr(), B1.data_ptr(), C1.data_ptr(), M1, M1, M1, 0, 0, 1.0, 0.0,
                              16, ext.MODE_CORDIC, stream)
        if rc:
            raise RuntimeError(lib.rac_last_error())

    mm1()
    torch.cuda.synchronize()
    t1 = _events_time(mm1, 10, torch)
    Ah, Bh = A1.cpu().numpy(), B1.cpu().numpy()
    Ch = np.empty_like(Ah)
    prev = (lib.rac_get_cordic_iters(), lib.rac_get_cordic_mode())
    lib.rac_set_cordic_iters(16)
    lib.rac_set_cordic_mode(ext.MODE_CORDIC)
    try:
        lib.rac_matmul(Ah.ctypes.data, Bh.ctypes.data, Ch.ctypes.data, M1, M1, M1)
        t0 = time.perf_counter()
        for _ in range(5):
            lib.rac_matmul(Ah.ctypes.data, Bh.ctypes.data, Ch.ctypes.data, M1, M1, M1)
        th = (time.perf_counter() - t0) / 5
    finally:
        lib.rac_set_cordic_iters(prev[0])
        lib.rac_set_cordic_mode(prev[1])
    ops["matmul_1024_cordic_n16"] = {
        "ms": round(t1 * 1e3, 3),
        "equiv_GFLOPs": round(2 * M1 ** 3 / t1 / 1e9, 1),
        "frac_of_fp32_peak": round(M1 ** 3 * 2 * 33 / t1 / 1e12 / PEAK_FP32_TFLOPS, 4),
        "rac_h_host_buffers_ms": round(th * 1e3, 3),
        **_dist_fields(t1, 1e3, "ms")}
    print(f"# matmul 1024^3 n=16: {t1 * 1e3:.3f} ms device, {th * 1e3:.2f} ms rac.h on host buffers",
          file=sys.stderr, flush=True)
    del A1, B1, C1

    # Decode-time linears (one token): x[1, K] @ W[N, K]^T, the few-row GEMM
    # path, FAST and CORDIC n = 16; the weights are read once (N*K*4 bytes)
    for (Nd, Kd) in ((4096, 4096), (11008, 4096)):
        xd = dev_uniform((1, Kd), 2, dev)
        wd = dev_uniform((Nd, Kd), 3, dev)
        yd = torch.empty((1, Nd), device=dev)
        for mode_name, mode, nit in (("fast", ext.MODE_FAST, 24), ("cordic_n16", ext.MODE_CORDIC, 16)):
            def dec():
                rc = lib.rac_gemm_dev(xd.data_ptr(), wd.data_ptr(), yd.data_ptr(), 1, Nd, Kd, 0, 1, 1.0, 0.0,
                                      nit, mode, stream)
                if rc:
                    raise RuntimeError(lib.rac_last_error())
            dec()
            torch.cuda.synchronize()
            t = _events_time(dec, 10, torch)
            ops[f"decode_linear_1x{Nd}x{Kd}_{mode_name}"] = {
                "us": round(t * 1e6, 2), "weights_GBps": round(Nd * Kd * 4 / t / 1e9, 1), **_dist_fields(t, 1e6, "us")}
            print(f"# decode linear 1x{Nd}x{Kd} {mode_name}: {t * 1e6:.1f} us", file=sys.stderr, flush=True)
        del xd, wd, yd
    # a matrix-vector product through rac_matmul: A[4096, 4096] @ x[4096, 1]
    # (the few-column path)
    Am = dev_uniform((4096, 4096), 4, dev)
    xm = dev_uniform((4096, 1), 5, dev)
    ym = torch.empty((4096, 1), device=dev)
    for mode_name, mode, nit in (("fast", ext.MODE_FAST, 24), ("cordic_n16", ext.MODE_CORDIC, 16)):
        def mv():
            rc = lib.rac_gemm_dev(Am.data_ptr(), xm.data_ptr(), ym.data_ptr(), 4096, 1, 4096, 0, 0, 1.0, 0.0, nit,
                                  mode, stream)
            if rc:
                raise RuntimeError(lib.rac_last_error())
        mv()
        torch.cuda.synchronize()
        t = _events_time(mv, 10, torch)
        ops[f"matvec_4096x4096_{mode_name}"] = {"us": round(t * 1e6, 2), "A_GBps": round(4096 * 4096 * 4 / t / 1e9, 1),
                                                **_dist_fields(t, 1e6, "us")}
        print(f"# matvec 4096x4096 {mode_name}: {t * 1e6:.1f} us", file=sys.stderr, flush=True)
    del Am, xm, ym

    if not args.matmul_only:
        ops.update(bench_row_ops(torch, ext, dev, g))
        ops.update(bench_block_ops(torch, ext, dev, g))

    w = 2 * n + 1
    achieved = M * N * K * 2 * w / launch_s / 1e12
    traffic = None
    try:   # HBM bytes per launch from the committed rocprofv3 --pmc runs
        with open(os.path.join(ROOT, "profiles", "pmc_traffic.json")) as f:
            pm = json.load(f)
        k = pm["kernels"][f"gemm_cordic_4096_n{n}"]
        traffic = int(k["fetch_kib"] * 1024 * pm["fetch_scale"] + k["write_kib"] * 1024 * pm["write_scale"])
    except (OSError, KeyError, ValueError):
        pass
    return {
        "value": round(2 * M * N * K / (ms_per_step / 1e3) / 1e9, 1),
        "ms_per_step": round(ms_per_step, 3),
        "roofline": {"bound": "valu", "achieved": round(achieved, 3), "peak": PEAK_FP32_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_TFLOPS, 4),
                     "traffic": traffic,
                     "traffic_note": "HBM bytes/launch (FETCH_SIZE x2 + WRITE_SIZE, copy-calibrated; "
                                     "profiles/gemm_cordic16_4096_pmc.md); algorithmic A+B+C = 2.01e8",
                     "kernel": f"gemm_kernel<CORDIC,{n},NN> 64x64 tile, 4x4 per lane",
                     "avg_launch_ms": round(launch_s * 1e3, 3),
                     **{f"launch_{k}": v for k, v in _dist_fields(launch_s, 1e3, "ms").items()},
                     "work_per_mac": f"{w} FMA lane-ops (2n+1)",
                     # the kernel executes 2n-1 VALU lane-ops per MAC (x0 sign flip,
                     # x0 * 1.5, 2(n-3)+1 chain FMAs, the gain multiply and the
                     # accumulate FMA), two fewer than the 2n+1 the roofline counts
                     "executed_lane_ops_per_mac": 2 * n - 1,
                     "executed_frac": round(achieved * (2 * n - 1) / w / PEAK_FP32_TFLOPS, 4)},
        "ops": ops,
    }


def _llama_breakdown(torch, blk, xb):
    """Per-op milliseconds of one RACLlamaBlock forward: HIP events recorded by
    forward hooks around each submodule on the current stream.  attention_core
    is the attention module minus its QKV / RoPE / output-projection children
    (Q K^T, causal CORDIC softmax, P V and the head transposes); residual_adds
    is the block minus its four children."""
    ev = {}

    def mark(name):
        def pre(_m, _a):
            e = torch.cuda.Event(enable_timing=True)
            e.record()
            ev[name] = [e]

        def post(_m, _a, _o):
            e = torch.cuda.Event(enable_timing=True)
            e.record()
            ev[name].append(e)
        return pre, post

    mods = {"block": blk, "rmsnorm1": blk.norm1, "attention": blk.attn, "qkv_proj": blk.attn.qkv,
            "rope": blk.attn.rope, "out_proj": blk.attn.out_proj, "rmsnorm2": blk.norm2, "ffn": blk.ffn,
            "fc1_silu": blk.ffn.fc1, "fc2": blk.ffn.fc2}
    handles = []
    for name, m in mods.items():
        pre, post = mark(name)
        handles += [m.register_forward_pre_hook(pre), m.register_forward_hook(post)]
    try:
        blk(xb, is_causal=True)
        torch.cuda.synchronize()
    finally:
        for h in handles:
            h.remove()
    ms = {k: v[0].elapsed_time(v[1]) for k, v in ev.items()}
    res = {k: round(ms[k], 3) for k in ("rmsnorm1", "qkv_proj", "rope", "out_proj", "rmsnorm2", "fc1_silu", "fc2")}
    res["attention_core"] = round(ms["attention"] - ms["qkv_proj"] - ms["rope"] - ms["out_proj"], 3)
    res["residual_adds"] = round(ms["block"] - ms["rmsnorm1"] - ms["attention"] - ms["rmsnorm2"] - ms["ffn"], 3)
    res["total"] = round(ms["block"], 3)
    return res


def bench_row_ops(torch, ext, dev, g):
    """Softmax, RoPE, RMSNorm and SiLU at the benchmark shapes (HBM-bound row and
    elementwise kernels), with torch copies of the same bytes for scale."""
    lib = ext._lib.load()
    stream = torch.cuda.current_stream(dev).cuda_stream
    out = {}

    def chk(rc):
        if rc:
            raise RuntimeError(lib.rac_last_error())

    def record(name, nbytes, t):
        out[name] = {"us": round(t * 1e6, 2), "GBps": round(nbytes / t / 1e9, 1),
                     "frac_of_hbm_peak": round(nbytes / t / 1e9 / PEAK_HBM_GBPS, 4),
                     **_dist_fields(t, 1e6, "us")}
        print(f"# {name}: {t * 1e6:.1f} us, {nbytes / t / 1e9:.0f} GB/s", file=sys.stderr, flush=True)

    reps = 20
    # softmax 4096 x 4096, N(0, std 2); 4 buffer sets (512 MiB) rotate past MALL
    R, Cn = 4096, 4096
    xs = [dev_normal((R, Cn), i, dev, std=2.0) for i in range(4)]
    ys = [torch.empty_like(xs[0]) for _ in range(4)]
    for n in (8, 16, 24):
        state = {"i": 0}

        def sm():
            i = state["i"] = (state["i"] + 1) % 4
            chk(lib.rac_softmax_dev(xs[i].data_ptr(), ys[i].data_ptr(), R, Cn, n, stream))

        sm()
        torch.cuda.synchronize()
        record(f"softmax_4096x4096_n{n}", 2 * 4 * R * Cn, _events_time(sm, reps, torch))
    # torch's own device copy of the same bytes with the same rotation, for
    # scale: what a generic streaming kernel achieves at this transfer size
    st_c = {"i": 0}

    def cp():
        i = st_c["i"] = (st_c["i"] + 1) % 4
        ys[i].copy_(xs[i])

    cp()
    torch.cuda.synchronize()
    record("torch_copy_4096x4096", 2 * 4 * R * Cn, _events_time(cp, reps, torch))
    del xs, ys

    # RoPE: Q and K [8,32,4096,128] in place (2 GiB moved per step)
    shape = (8, 32, 4096, 128)
    q = dev_normal(shape, 0, dev)
    k = dev_normal(shape, 1, dev)
    cos, sin = ext.rope_cache(4096, 128, 10000.0, device=dev)
    Bq, Hq, Tq, Dq = shape

    def rope():
        for t in (q, k):
            chk(lib.rac_rope_apply_dev(t.data_ptr(), cos.data_ptr(), sin.data_ptr(), Bq, Hq, Tq, Dq,
                                       Hq * Tq * Dq, Tq * Dq, Dq, stream))

    rope()
    torch.cuda.synchronize()
    record("rope_qk_8x32x4096x128", 2 * 2 * 4 * q.numel(), _events_time(rope, reps, torch))

    # the same tensors read as [B, T, H, D] (the layout a fused QKV projection
    # produces): position stride H*D, head stride D
    def rope_bthd():
        for t in (q, k):
            chk(lib.rac_rope_apply_dev(t.data_ptr(), cos.data_ptr(), sin.data_ptr(), Bq, Hq, Tq, Dq,
                                       Tq * Hq * Dq, Dq, Hq * Dq, stream))

    rope_bthd()
    torch.cuda.synchronize()
    record("rope_qk_bthd_8x4096x32x128", 2 * 2 * 4 * q.numel(), _events_time(rope_bthd, reps, torch))

    # the operator surface: RACRoPE forward on the same Q and K (out of place:
    # each output is a new tensor, one read and one write per element)
    from rac_amd import rac_torch as rt
    rope_mod = rt.RACRoPE(Dq, max_seq_len=Tq).to(dev)

    def rope_module():
        with torch.no_grad():
            rope_mod(q, k)

    rope_module()
    torch.cuda.synchronize()
    record("rope_module_qk_8x32x4096x128", 2 * 2 * 4 * q.numel(), _events_time(rope_module, reps, torch))
    del rope_mod

    # the table itself: rac_rope_cache(4096, 128, 10000) on the device, 16
    # circular CORDIC steps per entry after the reference's sequential wrap
    # of theta (inv_freq from the host's powf, already in device memory)
    inv = ext.rope_inv_freq(Dq, 10000.0).to(dev)
    ct, stb = torch.empty_like(cos), torch.empty_like(sin)

    def rope_tab():
        chk(lib.rac_rope_cache_dev(ct.data_ptr(), stb.data_ptr(), Tq, Dq, 10000.0, inv.data_ptr(), stream))

    rope_tab()
    torch.cuda.synchronize()
    t = _events_time(rope_tab, reps, torch)
    out["rope_cache_4096x128"] = {"us": round(t * 1e6, 2), "entries": Tq * Dq // 2,
                                  "Gentries_per_s": round(Tq * Dq // 2 / t / 1e9, 2), **_dist_fields(t, 1e6, "us")}
    print(f"# rope_cache_4096x128: {t * 1e6:.1f} us", file=sys.stderr, flush=True)
    del q, k

    # RMSNorm 16384 x 4096, gamma ~ N(1, 0.02), eps 1e-6; 2 sets (1 GiB)
    R, D = 16384, 4096
    xr = [dev_normal((R, D), i, dev) for i in range(2)]
    yr = [torch.empty_like(xr[0]) for _ in range(2)]
    gam = dev_normal((D,), 2, dev, mean=1.0, std=0.02)
    st = {"i": 0}

    def rms():
        i = st["i"] = (st["i"] + 1) % 2
        chk(lib.rac_rmsnorm_dev(xr[i].data_ptr(), yr[i].data_ptr(), gam.data_ptr(), 1e-6, R, D, stream))

    rms()
    torch.cuda.synchronize()
    record("rmsnorm_16384x4096", 2 * 4 * R * D + 4 * D, _events_time(rms, reps, torch))
    st_c = {"i": 0}

    def cp():
        i = st_c["i"] = (st_c["i"] + 1) % 2
        yr[i].copy_(xr[i])

    cp()
    torch.cuda.synchronize()
    record("torch_copy_16384x4096", 2 * 4 * R * D, _events_time(cp, reps, torch))
    del xr, yr

    # SiLU 16384 x 11008 (n = 16)
    xsilu = dev_normal((16384, 11008), 0, dev)
    ysilu = torch.empty_like(xsilu)

    def silu():
        chk(lib.rac_silu_dev(xsilu.data_ptr(), ysilu.data_ptr(), xsilu.numel(), 16, stream))

    silu()
    torch.cuda.synchronize()
    record("silu_16384x11008_n16", 2 * 4 * xsilu.numel(), _events_time(silu, 10, torch))
    del xsilu, ysilu
    return out


def bench_q8_ops(torch, ext, dev, g):
    """Q8_0 decode GEMV (M = 1) at 11008x4096, 32000x4096 and 65536x8192."""
    lib = ext._lib.load()
    stream = torch.cuda.current_stream(dev).cuda_stream
    out = {}
    reps = 20

    def chk(rc):
        if rc:
            raise RuntimeError(lib.rac_last_error())

    def record(name, nbytes, t):
        out[name] = {"us": round(t * 1e6, 2), "GBps": round(nbytes / t / 1e9, 1),
                     "frac_of_hbm_peak": round(nbytes / t / 1e9 / PEAK_HBM_GBPS, 4),
                     **_dist_fields(t, 1e6, "us")}
        print(f"# {name}: {t * 1e6:.1f} us, {nbytes / t / 1e9:.0f} GB/s", file=sys.stderr, flush=True)

    # Q8_0 decode GEMV (M = 1): weight bytes N*K/32*34 streamed once; buffer
    # sets rotate past the MALL
    for (Nq, Kq) in ((11008, 4096), (32000, 4096), (65536, 8192)):
        wbytes = Nq * (Kq // 32) * 34
        nsets = max(2, -(-600_000_000 // wbytes))
        wsets = []
        for _ in range(nsets):
            wq = torch.randint(0, 256, (Nq, Kq // 32, 34), device=dev, dtype=torch.uint8, generator=g)
            wq[:, :, 0] = 0x00
            wq[:, :, 1] = 0x20          # block scale 2^-7 (fp16 0x2000)
            wsets.append(wq)
        xq = torch.randn((1, Kq), device=dev, generator=g)
        yq = torch.empty((1, Nq), device=dev)
        stq = {"i": 0}

        def q8():
            i = stq["i"] = (stq["i"] + 1) % nsets
            chk(lib.rac_q8_0_gemv_dev(xq.data_ptr(), wsets[i].data_ptr(), None, yq.data_ptr(), 1, Nq, Kq, 0,
                                      stream))

        q8()
        torch.cuda.synchronize()
        record(f"q8_0_gemv_{Nq}x{Kq}", wbytes + 4 * (Kq + Nq), _events_time(q8, reps, torch))
        del wsets

    return out


def bench_decode_ops(torch, dev):
    """The decoder stack (rac_amd.decoder, the reference's full-model path of
    bench_rac_transformer.c) at the tinyllama shape: 22 layers, d_model 2048,
    32 query / 4 key-value heads, d_ff 5632, synthetic weights; CORDIC SiLU
    at n = 16.  Prefill of 128 tokens (fp32 weights, fused RAC linears,
    FAST MAC) and decode of one token (Q8_0 weights) at cache length
    128..., eager and replayed as one HIP graph per token; ms/token and
    tok/s as the reference prints them (bench_rac_transformer.c:844-851),
    and for decode the Q8_0 weight bytes streamed per token over the time."""
    from rac_amd.decoder import PRESETS, RACDecoder
    out = {}
    cfg = PRESETS["tinyllama"]
    dec = RACDecoder(cfg, RACDecoder.synthetic_weights(cfg, dev, seed=7), t_max=2048, iters=16)
    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    tp = 128
    xp = torch.randn((tp, cfg.d_model), device=dev, generator=gen)

    def prefill():
        dec.reset()
        dec.forward(xp)

    prefill()
    torch.cuda.synchronize()
    t = _events_time(prefill, 2, torch, dist_calls=5)
    out[f"decoder_tinyllama_prefill_T{tp}"] = {"ms_per_token": round(t * 1e3 / tp, 4),
                                               "tok_per_s": round(tp / t, 1), **_dist_fields(t, 1e3, "ms")}
    print(f"# decoder tinyllama prefill T={tp}: {t * 1e3 / tp:.3f} ms/token", file=sys.stderr, flush=True)
    wbytes = sum(q.numel() * q.element_size() for lw in dec.layers for q in (lw.q8_qkv, lw.q8_o, lw.q8_gu, lw.q8_d))
    xt = torch.randn((1, cfg.d_model), device=dev, generator=gen)
    for name, graph in (("eager", False), ("graph", True)):
        prefill()
        if graph:
            dec.capture()
        t = _events_time(lambda: dec.step(xt), 5, torch, dist_calls=10)
        at = dec.length
        dec.release_graph()
        out[f"decoder_tinyllama_decode_{name}"] = {
            "ms_per_token": round(t * 1e3, 4), "tok_per_s": round(1.0 / t, 1),
            "q8_weight_bytes_per_token": wbytes, "weight_GBps": round(wbytes / t / 1e9, 1),
            "frac_of_hbm_peak": round(wbytes / t / 1e9 / PEAK_HBM_GBPS, 4),
            "cache_length_at_end": at, **_dist_fields(t, 1e3, "ms")}
        print(f"# decoder tinyllama decode ({name}): {t * 1e3:.3f} ms/token", file=sys.stderr, flush=True)
    del dec
    return out


def bench_block_ops(torch, ext, dev, g):
    """Llama block, attention core, Q8_0 GEMV, RAC-DSP and the safetensors loader."""
    lib = ext._lib.load()
    stream = torch.cuda.current_stream(dev).cuda_stream
    out = {}

    def chk(rc):
        if rc:
            raise RuntimeError(lib.rac_last_error())

    def record(name, nbytes, t):
        out[name] = {"us": round(t * 1e6, 2), "GBps": round(nbytes / t / 1e9, 1),
                     "frac_of_hbm_peak": round(nbytes / t / 1e9 / PEAK_HBM_GBPS, 4),
                     **_dist_fields(t, 1e6, "us")}
        print(f"# {name}: {t * 1e6:.1f} us, {nbytes / t / 1e9:.0f} GB/s", file=sys.stderr, flush=True)

    reps = 20
    # Benchmark config 5: RACLlamaBlock forward, d=4096, H=32, ff=11008, batch 1,
    # seq 2048, causal, weights ~ N(0, 0.02), x ~ N(0, 1), CORDIC mode
    from rac_amd import rac_torch as rt
    torch.manual_seed(0)
    blk = rt.RACLlamaBlock(4096, 32, ff_dim=11008, max_seq_len=2048).to(dev)
    with torch.no_grad():
        for i, prm in enumerate(p for p in blk.parameters() if p.dim() == 2):
            prm.copy_(dev_normal(tuple(prm.shape), 100 + i, dev, std=0.02))
    xb = dev_normal((1, 2048, 4096), 0, dev)
    prev_mode, prev_iters = rt.rac_get_mode(), rt.rac_get_precision()
    rt.rac_set_mode("cordic")
    try:
        for n in (8, 16, 24):
            rt.rac_set_precision(n)
            with torch.no_grad():
                blk(xb, is_causal=True)
                torch.cuda.synchronize()
                t = _events_time(lambda: blk(xb, is_causal=True), 2, torch, dist_calls=5)
                parts = _llama_breakdown(torch, blk, xb)
            out[f"llama_block_T2048_n{n}"] = {"ms": round(t * 1e3, 2),
                                              "linear_equiv_TFLOPs": round(644.2e9 / t / 1e12, 3),
                                              "per_op_ms": parts, **_dist_fields(t, 1e3, "ms")}
            print(f"# llama block n={n}: {t * 1e3:.1f} ms", file=sys.stderr, flush=True)
        # the same block in rac_torch's default configuration (FAST MAC,
        # precision 24 for the CORDIC activations and softmax exp)
        rt.rac_set_mode("fast")
        rt.rac_set_precision(24)
        with torch.no_grad():
            blk(xb, is_causal=True)
            torch.cuda.synchronize()
            t = _events_time(lambda: blk(xb, is_causal=True), 3, torch, dist_calls=5)
            parts = _llama_breakdown(torch, blk, xb)
        out["llama_block_T2048_fast"] = {"ms": round(t * 1e3, 2),
                                         "linear_TFLOPs": round(644.2e9 / t / 1e12, 3),
                                         "per_op_ms": parts, **_dist_fields(t, 1e3, "ms")}
        print(f"# llama block FAST: {t * 1e3:.1f} ms", file=sys.stderr, flush=True)
        # one training step of it: forward, then backward of a fixed output
        # gradient through every autograd function (weight, input and
        # attention gradients)
        xg = xb.clone().requires_grad_(True)
        gy = dev_normal((1, 2048, 4096), 1, dev)

        def train_step():
            blk(xg, is_causal=True).backward(gy)

        train_step()
        torch.cuda.synchronize()
        t = _events_time(train_step, 3, torch, dist_calls=5)
        blk.zero_grad(set_to_none=True)
        out["llama_block_T2048_fast_train_step"] = {"ms": round(t * 1e3, 2), **_dist_fields(t, 1e3, "ms")}
        print(f"# llama block FAST forward + backward: {t * 1e3:.1f} ms", file=sys.stderr, flush=True)
        del xg, gy
    finally:
        rt.rac_set_mode(prev_mode)
        rt.rac_set_precision(prev_iters)
    del blk, xb

    # attention core of config 5 through RAC (rac_attention_dev): [1, 32, 2048,
    # 128], causal, CORDIC mode n = 16; Q K^T and P V 8.6 G causal MACs each
    Ba, Ha, Ta, Da = 1, 32, 2048, 128
    qa, ka, va = (dev_normal((Ba, Ha, Ta, Da), i, dev) for i in range(3))
    oa = torch.empty_like(qa)
    wsa = torch.empty(lib.rac_attention_workspace_bytes(Ba, Ha, Ta) // 4, device=dev)

    def attn():
        chk(lib.rac_attention_dev(qa.data_ptr(), ka.data_ptr(), va.data_ptr(), None, 1, oa.data_ptr(), Ba, Ha,
                                  Ta, Da, wsa.data_ptr(), 16, ext.MODE_CORDIC, stream))

    attn()
    torch.cuda.synchronize()
    t = _events_time(attn, 3, torch)
    # causal work: query row t needs t+1 scores (Q K^T) and t+1 rows of V
    # (P V), so each product has B*H*D*T(T+1)/2 MACs; the dense count would
    # credit the masked half that is never computed
    macs = 2 * Ba * Ha * Da * Ta * (Ta + 1) // 2
    ws_mib = lib.rac_attention_workspace_bytes(Ba, Ha, Ta) / 2 ** 20
    out["attention_core_1x32x2048x128_n16"] = {
        "ms": round(t * 1e3, 3), "causal_macs": macs,
        "equiv_TFLOPs": round(2 * macs / t / 1e12, 3),
        "valu_frac_of_fp32_peak": round(macs * 2 * 33 / t / 1e12 / PEAK_FP32_TFLOPS, 4),
        "workspace_MiB": round(ws_mib, 1), "path": "rac_attention_dev: query-row chunks",
        **_dist_fields(t, 1e3, "ms")}
    print(f"# attention core n=16 (chunks, {ws_mib:.0f} MiB workspace): {t * 1e3:.2f} ms", file=sys.stderr, flush=True)
    del wsa
    # the same core in one chunk (the [B*H, T, T] score matrix the reference
    # materialises; what the autograd path keeps for backward) and through the
    # allocation-free entry point (64 MiB static scratch): same output bits
    wsp = torch.empty(lib.rac_attention_probs_workspace_bytes(Ba, Ha, Ta) // 4, device=dev)

    def attn_one():
        chk(lib.rac_attention_probs_dev(qa.data_ptr(), ka.data_ptr(), va.data_ptr(), None, 1, oa.data_ptr(), Ba, Ha,
                                        Ta, Da, wsp.data_ptr(), 16, ext.MODE_CORDIC, stream))

    def attn_noalloc():
        chk(lib.rac_attention_noalloc_dev(qa.data_ptr(), ka.data_ptr(), va.data_ptr(), None, 1, oa.data_ptr(), Ba,
                                          Ha, Ta, Da, 16, ext.MODE_CORDIC, stream))

    for name, fn, mib in (("attention_core_one_chunk_1x32x2048x128_n16", attn_one, wsp.numel() * 4 / 2 ** 20),
                          ("attention_core_noalloc_1x32x2048x128_n16", attn_noalloc, 64.0)):
        fn()
        torch.cuda.synchronize()
        t = _events_time(fn, 3, torch)
        out[name] = {"ms": round(t * 1e3, 3), "equiv_TFLOPs": round(2 * macs / t / 1e12, 3),
                     "workspace_MiB": round(mib, 1), **_dist_fields(t, 1e3, "ms")}
        print(f"# {name}: {t * 1e3:.2f} ms", file=sys.stderr, flush=True)
    del qa, ka, va, oa, wsp

    out.update(bench_q8_ops(torch, ext, dev, g))
    out.update(bench_decode_ops(torch, dev))

    # RAC-DSP fixed-point engine (Q32.32 / Q0.63 int64): 2^24 evaluations of
    # rotate (x, y, z in and out: 48 B each) and of project (x, z in, x out:
    # 24 B, the rac_dsp_project_batch form); the 256 x 256 systolic product of
    # 256 activation vectors (2^24 projections, outputs K x N)
    nd = 1 << 24
    xd, yd, zd = (torch.randint(-2 ** 62, 2 ** 62, (nd,), device=dev, dtype=torch.int64, generator=g)
                  for _ in range(3))
    od = [torch.empty_like(xd) for _ in range(3)]
    for opd, name, nbytes in ((0, "rotate", 48), (1, "project", 24)):
        def dsp():
            if opd == 0:
                chk(lib.rac_dsp_eval_dev(0, nd, xd.data_ptr(), yd.data_ptr(), zd.data_ptr(), od[0].data_ptr(),
                                         od[1].data_ptr(), od[2].data_ptr(), stream))
            else:
                chk(lib.rac_dsp_eval_dev(1, nd, xd.data_ptr(), None, zd.data_ptr(), od[0].data_ptr(), None, None,
                                         stream))

        dsp()
        torch.cuda.synchronize()
        t = _events_time(dsp, reps, torch)
        out[f"dsp_{name}_16M"] = {"us": round(t * 1e6, 2), "Geval_per_s": round(nd / t / 1e9, 2),
                                  "GBps": round(nbytes * nd / t / 1e9, 1),
                                  "frac_of_hbm_peak": round(nbytes * nd / t / 1e9 / PEAK_HBM_GBPS, 4),
                                  **_dist_fields(t, 1e6, "us")}
        print(f"# dsp {name}: {t * 1e6:.1f} us, {nd / t / 1e9:.1f} G-evals/s", file=sys.stderr, flush=True)
    del xd, yd, zd, od
    Ns = Ks = 256
    Wd = torch.randint(-2 ** 63, 2 ** 63 - 1, (Ns, Ns), device=dev, dtype=torch.int64, generator=g)
    Xd = torch.randint(-2 ** 40, 2 ** 40, (Ks, Ns), device=dev, dtype=torch.int64, generator=g)
    Yd = torch.empty_like(Xd)

    def sysd():
        chk(lib.rac_dsp_systolic_dev(Ns, Ks, Wd.data_ptr(), Xd.data_ptr(), Yd.data_ptr(), stream))

    sysd()
    torch.cuda.synchronize()
    t = _events_time(sysd, reps, torch)
    out["dsp_systolic_256x256_k256"] = {"us": round(t * 1e6, 2), "Geval_per_s": round(Ns * Ns * Ks / t / 1e9, 2),
                                        **_dist_fields(t, 1e6, "us")}
    print(f"# dsp systolic: {t * 1e6:.1f} us", file=sys.stderr, flush=True)
    del Wd, Xd, Yd

    # safetensors loader: a BF16 [11008, 4096] weight (Llama-7B MLP shape, 90 MB)
    # in a file in the page cache -> HBM as fp32 and as Q8_0 (wall clock per
    # call incl. the host copies and PCIe; "GBps" counts file bytes); and the
    # device-resident conversion kernels alone (bf16 bytes already in HBM:
    # 2 B read + 4 B written per element for fp32, 2 + 34/32 B for Q8_0)
    import tempfile
    Nw, Kw = 11008, 4096
    wbits = (torch.randn(Nw * Kw, generator=torch.Generator().manual_seed(5)) * 0.02).view(torch.int32)
    wbits = (wbits >> 16).to(torch.int16)                         # bf16 = top half of the fp32 word
    raw = wbits.numpy().tobytes()
    hdr = json.dumps({"w": {"dtype": "BF16", "shape": [Nw, Kw], "data_offsets": [0, len(raw)]}}).encode()
    tmpd = tempfile.mkdtemp(prefix="rac_st_")
    pathw = os.path.join(tmpd, "w.safetensors")
    with open(pathw, "wb") as fh:
        fh.write(len(hdr).to_bytes(8, "little") + hdr + raw)
    del raw
    sfw = ext.SafeTensors(pathw)
    wf = torch.empty((Nw, Kw), device=dev)
    wq8 = torch.empty((Nw, Kw // 32, 34), device=dev, dtype=torch.uint8)
    tw = lib.st_find(sfw._f, b"w")
    for name, fn in (("st_load_bf16_to_f32_11008x4096",
                      lambda: chk(lib.rac_st_to_f32_dev(sfw._f, tw, wf.data_ptr(), stream))),
                     ("st_load_bf16_to_q8_0_11008x4096",
                      lambda: chk(lib.rac_st_to_q8_0_dev(sfw._f, tw, wq8.data_ptr(), stream)))):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(5):
            fn()
        torch.cuda.synchronize()
        t = (time.perf_counter() - t0) / 5
        out[name] = {"ms": round(t * 1e3, 3), "GBps_file": round(2 * Nw * Kw / t / 1e9, 2)}
        print(f"# {name}: {t * 1e3:.2f} ms, {2 * Nw * Kw / t / 1e9:.1f} GB/s of file", file=sys.stderr, flush=True)
    sfw.close()
    os.remove(pathw)
    os.rmdir(tmpd)
    draw = wbits.to(dev)
    record("st_convert_bf16_to_f32_11008x4096", 6 * Nw * Kw,
           _events_time(lambda: chk(lib.rac_st_convert_dev(3, draw.data_ptr(), Nw * Kw, wf.data_ptr(), stream)),
                        reps, torch))
    record("st_quantize_bf16_to_q8_0_11008x4096", 2 * Nw * Kw + Nw * Kw // 32 * 34,
           _events_time(lambda: chk(lib.rac_st_quantize_dev(3, draw.data_ptr(), Nw * Kw // 32, wq8.data_ptr(),
                                                            stream)), reps, torch))
    del draw, wf, wq8, wbits

    return out


# ── CPU baseline: the compiled reference lib/c, in a child process ─────────

def cpu_baseline_child():
    """Runs without torch: times oracle/_ref (reference lib/c) on host cores."""
    import ctypes

    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import raclib as rl

    if not rl.have_ref():
        print(json.dumps({"error": "oracle/_ref/librac_ref.so not present"}))
        return
    cpus = os.environ.get("RAC_BENCH_CPUS", "")
    if cpus:
        # before the reference's OpenMP runtime starts: its threads inherit this
        os.sched_setaffinity(0, [int(c) for c in cpus.split(",")])
    r = rl.ref()
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    res = {"threads": threads}
    M = N = K = 4096
    A = rl.gen_uniform((M, K), 0)
    B = rl.gen_uniform((K, N), 1)
    Cm = np.zeros((M, N), np.float32)
    r.rac_hal_matmul(rl.p(A), rl.p(B), rl.p(Cm), M, N, K)   # warm-up (HAL init, page-in)
    t0 = time.perf_counter()
    reps = 0
    while True:
        r.rac_hal_matmul(rl.p(A), rl.p(B), rl.p(Cm), M, N, K)
        reps += 1
        if time.perf_counter() - t0 > 10.0 or reps >= 40:
            break
    t = (time.perf_counter() - t0) / reps
    res["matmul"] = {"seconds": t, "reps": reps, "GFLOPs": 2 * M * N * K / t / 1e9}
    del A, B, Cm
    # benchmark config 1 shape on the same path
    M1 = 1024
    A1 = rl.gen_uniform((M1, M1), 0)
    B1 = rl.gen_uniform((M1, M1), 1)
    C1 = np.zeros((M1, M1), np.float32)
    r.rac_hal_matmul(rl.p(A1), rl.p(B1), rl.p(C1), M1, M1, M1)
    t0 = time.perf_counter()
    for _ in range(10):
        r.rac_hal_matmul(rl.p(A1), rl.p(B1), rl.p(C1), M1, M1, M1)
    t = (time.perf_counter() - t0) / 10
    res["matmul_1024"] = {"seconds": t, "GFLOPs": 2 * M1 ** 3 / t / 1e9}
    del A1, B1, C1

    def timeit(fn, n):
        fn()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        return (time.perf_counter() - t0) / n

    x = rl.gen_normal((4096, 4096), 0, std=2.0)
    y = np.empty_like(x)
    t = timeit(lambda: r.rac_softmax_batch(rl.p(x), rl.p(y), 4096, 4096), 3)
    res["softmax"] = {"seconds": t, "GBps": 2 * x.nbytes / t / 1e9}
    q = np.random.default_rng(0).standard_normal((8, 32, 4096, 128), dtype=np.float32)
    c = np.zeros((4096, 64), np.float32)
    s = np.zeros((4096, 64), np.float32)
    t = timeit(lambda: r.rac_rope_cache(rl.p(c), rl.p(s), 4096, 128, 10000.0), 3)
    res["rope_cache_4096x128"] = {"seconds": t, "Gentries_per_s": 4096 * 64 / t / 1e9}
    t = timeit(lambda: r.rac_rope_apply(rl.p(q), rl.p(c), rl.p(s), 8, 32, 4096, 128, None), 2)
    res["rope_per_tensor"] = {"seconds": t, "GBps": 2 * q.nbytes / t / 1e9}
    del q
    x = np.random.default_rng(1).standard_normal((16384, 4096), dtype=np.float32)
    y = np.empty_like(x)
    gam = np.ones(4096, np.float32)
    t = timeit(lambda: r.rac_rmsnorm(rl.p(x), rl.p(y), rl.p(gam), 1e-6, 16384, 4096, None), 2)
    res["rmsnorm"] = {"seconds": t, "GBps": 2 * x.nbytes / t / 1e9}
    del x, y
    # SiLU 16384 x 11008 (rac_hal_silu: the reference's AVX2 dispatch)
    x = np.random.default_rng(5).standard_normal((16384, 11008), dtype=np.float32)
    y = np.empty_like(x)
    t = timeit(lambda: r.rac_hal_silu(rl.p(x), rl.p(y), x.size), 2)
    res["silu"] = {"seconds": t, "GBps": 2 * x.nbytes / t / 1e9}
    del x, y
    # Q8_0 decode GEMV 11008 x 4096 (reference AVX2 path)
    Wf = np.random.default_rng(2).standard_normal((11008, 4096), dtype=np.float32) * np.float32(0.02)
    wq = np.zeros((11008, 128, 34), np.uint8)
    r.rac_q8_0_quantize_matrix(rl.p(Wf), rl.p(wq), 11008, 4096)
    del Wf
    xv = np.random.default_rng(3).standard_normal(4096, dtype=np.float32)
    yv = np.zeros(11008, np.float32)
    t = timeit(lambda: r.rac_q8_0_gemv(rl.p(xv), rl.p(wq), None, rl.p(yv), 11008, 4096, 0), 20)
    res["q8_0_gemv_11008x4096"] = {"seconds": t, "GBps": wq.nbytes / t / 1e9}
    del wq
    # RAC-DSP project batch, 2^20 evaluations (reference sim/rac_dsp_core.c,
    # ROMs generated by the rtl/gen_coarse_lut.py rule)
    lut, at, ath = np.zeros(1024, np.uint64), np.zeros(17, np.int64), np.zeros(9, np.int64)
    rl.oracle().orc_dsp_gen_roms(rl.p(lut), rl.p(at), rl.p(ath))
    ctypes.memmove(ctypes.addressof(ctypes.c_uint64.in_dll(r, "rac_coarse_lut")), lut.ctypes.data, lut.nbytes)
    ctypes.memmove(ctypes.addressof(ctypes.c_int64.in_dll(r, "rac_atan_rom")), at.ctypes.data, at.nbytes)
    ctypes.memmove(ctypes.addressof(ctypes.c_int64.in_dll(r, "rac_atanh_tab")), ath.ctypes.data, ath.nbytes)
    nd = 1 << 20
    rng = np.random.default_rng(4)
    xs = rng.integers(-2 ** 62, 2 ** 62, nd, dtype=np.int64)
    zs = rng.integers(-2 ** 63, 2 ** 63 - 1, nd, dtype=np.int64)
    xo = np.zeros(nd, np.int64)
    t = timeit(lambda: r.rac_dsp_project_batch(nd, rl.p(xs), rl.p(zs), rl.p(xo)), 3)
    res["dsp_project"] = {"seconds": t, "evals": nd, "Geval_per_s": nd / t / 1e9}
    print(json.dumps(res))


def _cpu_list(text):
    """'0-3,8,10-11' -> [0, 1, 2, 3, 8, 10, 11]."""
    cpus = []
    for part in text.strip().split(","):
        if not part:
            continue
        lo, _, hi = part.partition("-")
        cpus.extend(range(int(lo), int(hi or lo) + 1))
    return cpus


def _read(path):
    try:
        with open(path) as f:
            return f.read().strip()
    except OSError:
        return None


def _gpu0_host_placement():
    """Where the CPU baseline runs: the host CPU model, GPU 0's PCI address
    and NUMA node (sysfs), and one logical CPU per physical core of that node
    among the CPUs this process may use (all allowed cores when the node is
    unknown or none of its cores are allowed)."""
    info = {"cpu_model": None, "gpu_pci_bus": None, "numa_node": None}
    for line in (_read("/proc/cpuinfo") or "").splitlines():
        if line.startswith("model name"):
            info["cpu_model"] = line.split(":", 1)[1].strip()
            break
    try:
        import ctypes
        hip = ctypes.CDLL("libamdhip64.so.7")       # the runtime torch already loaded
        buf = ctypes.create_string_buffer(64)
        if hip.hipDeviceGetPCIBusId(buf, 64, 0) == 0:
            info["gpu_pci_bus"] = buf.value.decode().lower()
    except Exception:  # noqa: BLE001
        pass
    allowed = sorted(os.sched_getaffinity(0))
    local = allowed
    if info["gpu_pci_bus"]:
        dev = f"/sys/bus/pci/devices/{info['gpu_pci_bus']}"
        node = _read(dev + "/numa_node")
        if node is not None and node.lstrip("-").isdigit():
            info["numa_node"] = int(node)
        lst = _read(dev + "/local_cpulist")
        if lst and info["numa_node"] is not None and info["numa_node"] >= 0:
            local = sorted(set(_cpu_list(lst)) & set(allowed)) or allowed
    cores = {}
    for c in local:
        key = (_read(f"/sys/devices/system/cpu/cpu{c}/topology/physical_package_id"),
               _read(f"/sys/devices/system/cpu/cpu{c}/topology/core_id") or str(c))
        cores.setdefault(key, c)
    info["allowed_logical_cpus"] = len(allowed)
    info["node_local_allowed_logical_cpus"] = len(local)
    info["cpus"] = sorted(cores.values())
    info["physical_cores"] = len(info["cpus"])
    return info


def run_cpu_baseline():
    """Times the reference lib/c in a child process pinned to GPU 0's NUMA
    node: one OpenMP thread per physical core of that node (at most the
    environment's OMP_NUM_THREADS, which the GPU boxes cap)."""
    place = _gpu0_host_placement()
    threads = place["physical_cores"]
    cap = os.environ.get("OMP_NUM_THREADS", "")
    if cap.isdigit() and int(cap) > 0:
        threads = min(threads, int(cap))
    cpus = place["cpus"][:threads]
    env = dict(os.environ)
    env["OMP_NUM_THREADS"] = str(threads)
    env["OMP_PROC_BIND"] = "close"
    env["OMP_PLACES"] = ",".join("{%d}" % c for c in cpus)
    env["RAC_BENCH_CPUS"] = ",".join(str(c) for c in cpus)
    try:
        out = subprocess.run([sys.executable, os.path.abspath(__file__), "--cpu-baseline-child"],
                             capture_output=True, text=True, env=env, timeout=240)
        line = [ln for ln in out.stdout.splitlines() if ln.startswith("{")][-1]
        res = json.loads(line)
    except Exception as e:  # noqa: BLE001
        res = {"error": f"cpu baseline failed: {e}"}
    res["placement"] = {k: place[k] for k in ("cpu_model", "gpu_pci_bus", "numa_node", "allowed_logical_cpus",
                                              "node_local_allowed_logical_cpus", "physical_cores")}
    res["placement"]["cpus_used"] = env["RAC_BENCH_CPUS"]
    return res


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--iters", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--matmul-only", action="store_true")
    ap.add_argument("--rowops-only", action="store_true",
                    help="only time softmax, RoPE, RMSNorm and SiLU and print their figures "
                         "(a short run for rocprofv3 --pmc passes; not the benchmark line)")
    ap.add_argument("--decode-only", action="store_true",
                    help="only time the decoder stack (tinyllama shape: prefill and decode per token)")
    ap.add_argument("--q8-only", action="store_true",
                    help="only time the Q8_0 decode GEMV shapes (a short run for rocprofv3 --pmc passes)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 256 MiB device-to-device tensor copy 3 times (scales the "
                         "FETCH_SIZE/WRITE_SIZE counters of rocprofv3 --pmc runs)")
    ap.add_argument("--cpu-baseline-child", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()

    if args.cpu_baseline_child:
        cpu_baseline_child()
        return
    if args.copy_calibration:
        import torch
        x = torch.ones(64 * 1024 * 1024, device="cuda")
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_per_dispatch": x.numel() * 4}))
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}, WORLD_SIZE {world}): this "
              "build's hot path is single-GPU (every op would shard by rows or output columns with at most one all-reduce per block).", file=sys.stderr)
        sys.exit(2)

    if args.decode_only:
        import torch
        sys.path.insert(0, ROOT)
        dev = torch.device("cuda", 0)
        torch.cuda.set_device(dev)
        print(json.dumps({"ops": bench_decode_ops(torch, dev)}), flush=True)
        return
    if args.q8_only:
        import torch
        sys.path.insert(0, ROOT)
        from rac_amd import ext
        dev = torch.device("cuda", 0)
        torch.cuda.set_device(dev)
        g = torch.Generator(device=dev)
        g.manual_seed(0)
        print(json.dumps({"ops": bench_q8_ops(torch, ext, dev, g)}), flush=True)
        return
    if args.rowops_only:
        import torch
        sys.path.insert(0, ROOT)
        from rac_amd import ext
        dev = torch.device("cuda", 0)
        torch.cuda.set_device(dev)
        g = torch.Generator(device=dev)
        g.manual_seed(0)
        print(json.dumps({"ops": bench_row_ops(torch, ext, dev, g)}), flush=True)
        return
    gpu = bench_gpu(args)
    cpu = None if args.no_cpu_baseline else run_cpu_baseline()
    line = {
        "metric": "rac_matmul equiv-GFLOP/s at 4096³ (16 iters); RoPE/softmax/RMSNorm HBM GB/s",
        "value": gpu["value"],
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": gpu["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic, the configs' splitmix64 generator (A U[-1,1] seed 0, B seed 1), resident in HBM",
        "config": {"workload": f"rac_matmul 4096x4096x4096 fp32 CORDIC mode n={args.iters} (NN, row-major)",
                   "M": 4096, "N": 4096, "K": 4096, "cordic_iters": args.iters, "mode": "cordic"},
        "roofline": gpu["roofline"],
        "ops": gpu["ops"],
    }
    if cpu is not None and "matmul" in cpu:
        pl = cpu.get("placement", {})
        line["cpu_baseline"] = {
            "value": round(cpu["matmul"]["GFLOPs"], 1), "unit": "GFLOP/s", "cores": cpu["threads"],
            "kind": "reference",
            "sample": f"reference lib/c rac_hal_matmul (AVX2 GotoBLAS, FMA; ignores n) 4096^3 x "
                      f"{cpu['matmul']['reps']} reps, {cpu['threads']} OpenMP threads, one per physical core "
                      + (f"of GPU 0's NUMA node {pl['numa_node']}" if pl.get("numa_node") is not None and pl["numa_node"] >= 0 else
                         "this process may use (sysfs gives GPU 0 no NUMA node)")
                      + f" ({pl.get('cpu_model')})",
            "cpu_model": pl.get("cpu_model"), "numa_node": pl.get("numa_node"),
            "placement": pl,
            "ops": {k: {kk: round(vv, 4) for kk, vv in v.items()} for k, v in cpu.items()
                    if isinstance(v, dict) and k not in ("matmul", "placement")},
        }
    elif cpu is not None:
        line["cpu_baseline"] = {"value": None, "unit": "GFLOP/s", "cores": 0, "kind": "reference",
                                "sample": cpu.get("error", "unavailable")}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
