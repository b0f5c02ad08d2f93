"""Start-up diagnosis of the kernel library.

The reference probes torch's device and then runs one 4x4 RAC matmul when
rac_torch is imported, with a distinct warning for each failure
(rac_torch/rac_torch.py:55-108).  Here the stages are: the library file
exists, it loads, torch sees a ROCm device, that device is a gfx950 (the
only code the library carries), and one 4x4 CORDIC-mode product run on it
through rac_gemm_dev agrees with a float64 product within the matmul bar
1e-4 |a_i| |b_j|.  Each failure has its own stage name and message, so
"rebuild the library" is never confused with "this GPU has no gfx950
code".  There is no CPU fallback: ops raise with this message when the
probe failed.
"""
from __future__ import annotations

import os
from typing import NamedTuple

import torch

from . import _lib

ARCH = "gfx950"


class ProbeResult(NamedTuple):
    ok: bool
    stage: str      # "ok", "no-library", "library-load", "no-device", "arch", "kernel"
    message: str


def probe(run_kernel: bool = True) -> ProbeResult:
    """Diagnose the library and the current device (one tiny kernel launch
    when a gfx950 device is present and run_kernel)."""
    path = _lib.LIB_PATH
    if not os.path.exists(path):
        return ProbeResult(False, "no-library",
                           f"RAC kernel library not built: {path} is missing; build it with "
                           "`make -C rac_amd/csrc` (hipcc --offload-arch=gfx950)")
    try:
        lib = _lib.load()
    except Exception as e:   # a broken or foreign .so
        return ProbeResult(False, "library-load",
                           f"RAC kernel library {path} exists but does not load: {type(e).__name__}: {e}")
    if not torch.cuda.is_available():
        return ProbeResult(False, "no-device",
                           "no ROCm device is visible to torch; the RAC kernels have no CPU path")
    dev = torch.cuda.current_device()
    arch = getattr(torch.cuda.get_device_properties(dev), "gcnArchName", "") or "unknown"
    if arch.split(":")[0] != ARCH:
        return ProbeResult(False, "arch",
                           f"no {ARCH} code for this device: device {dev} is {arch}, and "
                           f"{os.path.basename(path)} is built for {ARCH} (MI355X) only")
    if not run_kernel:
        return ProbeResult(True, "ok", f"RAC library loaded on {arch} (kernel probe skipped)")
    try:
        g = torch.Generator().manual_seed(0)
        a = torch.rand(4, 4, generator=g, dtype=torch.float64) * 2 - 1
        b = torch.rand(4, 4, generator=g, dtype=torch.float64) * 2 - 1
        A = a.float().to(f"cuda:{dev}")
        B = b.float().to(f"cuda:{dev}")
        C = torch.empty(4, 4, device=A.device)
        stream = torch.cuda.current_stream(dev).cuda_stream
        rc = lib.rac_gemm_dev(A.data_ptr(), B.data_ptr(), C.data_ptr(), 4, 4, 4, 0, 0, 1.0, 0.0, 16, 1,
                              stream)
        if rc != 0:
            err = lib.rac_last_error()
            raise _lib.RACError(err.decode() if err else f"status {rc}")
        torch.cuda.synchronize(dev)
        got = C.double().cpu()
    except Exception as e:
        return ProbeResult(False, "kernel",
                           f"the {ARCH} kernels failed on device {dev} ({arch}): {type(e).__name__}: "
                           f"{str(e).splitlines()[0][:160] if str(e) else ''}")
    ref = a.float().double() @ b.float().double()
    bound = 1e-4 * a.abs().sum(1, keepdim=True) * b.abs().sum(0, keepdim=True)
    if not bool(((got - ref).abs() <= bound).all()):
        return ProbeResult(False, "kernel",
                           f"the {ARCH} kernels ran on device {dev} ({arch}) but a 4x4 CORDIC product "
                           f"is off by {float((got - ref).abs().max()):.3e}")
    return ProbeResult(True, "ok", f"RAC kernels OK on device {dev} ({arch})")
