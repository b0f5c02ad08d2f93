"""CPU check of the binade-at-a-time angle wrap behind the device sin/cos
and RoPE table (rac_amd/csrc/rac_math.hpp wrap_binades): tests/wrap_check.c
restates it in C with the same float operations and compares it with the
reference's step-by-step loop (rac_cpu.c:92-94) on every float in
(pi, 2^11), both signs, and on strided samples up to 2^27; it also checks
the condition the method rests on (2 pi never falls exactly half-way on a
binade's grid for binades 4 .. 26).  The device code itself is checked
against the checker's loop by tests/test_gpu_parity.py
(test_sincos_large_angles_wrap, test_rope_cache_long_context_vs_checker)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def wrap_check(tmp_path_factory):
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    exe = str(tmp_path_factory.mktemp("wrap") / "wrap_check")
    subprocess.run([cc, "-O2", "-ffp-contract=off", "-o", exe, os.path.join(HERE, "wrap_check.c"), "-lm"],
                   check=True)
    return exe


@pytest.mark.parametrize("lim,stride", [(11, 1), (16, 61), (20, 8191), (27, 2097143)])
def test_fast_wrap_equals_sequential_loop(wrap_check, lim, stride):
    r = subprocess.run([wrap_check, str(lim), str(stride)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 mismatches" in r.stdout
