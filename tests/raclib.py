"""Test helpers: ctypes bindings of the CPU checker (oracle/liboracle.so), of
the compiled reference (oracle/_ref/librac_ref.so, when built), and a
deterministic input generator.

Only tests, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module; the product never imports it.
"""
from __future__ import annotations

import ctypes as C
import hashlib
import json
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "librac_ref.so")
GOLDEN = os.path.join(ROOT, "tests", "golden")

_vp, _i, _l, _f = C.c_void_p, C.c_int, C.c_long, C.c_float
_fp = C.POINTER(C.c_float)



class Vec2(C.Structure):
    """struct { float x, y; }: rac_vec2 (rac_cpu.h:35) / float2 (rac.h:31)."""

    _fields_ = [("x", C.c_float), ("y", C.c_float)]


class StTensor(C.Structure):
    """st_tensor (bench/safetensors_reader.h:51-58)."""

    _fields_ = [("name", C.c_char * 256), ("dtype", C.c_int), ("ndim", C.c_int), ("shape", C.c_int64 * 8),
                ("offset", C.c_size_t), ("nbytes", C.c_size_t)]


class StFile(C.Structure):
    """st_file (bench/safetensors_reader.h:60-69)."""

    _fields_ = [("fd", C.c_int), ("mmap_base", C.c_void_p), ("mmap_len", C.c_size_t), ("data_offset", C.c_size_t),
                ("tensors", C.POINTER(StTensor)), ("n_tensors", C.c_int), ("header_copy", C.c_char_p),
                ("err", C.c_char * 256)]


_stf, _stt = C.POINTER(StFile), C.POINTER(StTensor)
ST_DTYPES = {"F32": 1, "F16": 2, "BF16": 3, "F64": 4, "I8": 5, "U8": 6, "I16": 7, "I32": 8, "I64": 9, "BOOL": 10}

_ORACLE_SIGS = {
    "orc_tables": (None, [_vp, _vp, _vp]),
    "orc_cordic_rotate": (None, [_f, _f, _f, _i, _fp, _fp]),
    "orc_cordic_dirs": (None, [_i, _vp]),
    "orc_cordic_kinv": (_f, [_i]),
    "orc_fma_cordic": (_f, [_f, _f, _f, _i]),
    "orc_cordic_project": (_f, [_f, _i]),
    "orc_cordic_chain_fast": (_f, [_f, _i]),
    "orc_shiftadd_mul": (_f, [_f, _f, _i]),
    "orc_fma_iters": (_f, [_f, _f, _f, _i, _i]),
    "orc_matmul": (_i, [_i, _i, _vp, _vp, _vp, _i, _i, _i, _f, _f, _i, _i, _i]),
    "orc_matmul_entries": (_i, [_i, _i, _vp, _vp, _i, _i, _i, _i, _i, _vp, _vp, _i, _vp]),
    "orc_rope_inv_freq": (None, [_vp, _i, _f]),
    "orc_sincos": (None, [_f, _fp, _fp]),
    "orc_sincos_batch": (None, [_vp, _vp, _vp, _l]),
    "orc_rope_cache": (_i, [_vp, _vp, _i, _i, _f]),
    "orc_rope_apply": (_i, [_vp, _vp, _vp, _i, _i, _i, _i]),
    "orc_rope_apply_strided": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _l, _l, _l]),
    "orc_hyp_schedule": (_i, [_i, _vp]),
    "orc_hyp_kinv": (_f, [_i]),
    "orc_exp_xy": (_f, [_f, _i, _f]),
    "orc_exp_n": (_f, [_f, _i]),
    "orc_exp_batch": (None, [_vp, _vp, _l, _i]),
    "orc_softmax_rows": (None, [_vp, _vp, _i, _i, _i]),
    "orc_rsqrt": (_f, [_f]),
    "orc_rsqrt_batch": (None, [_vp, _vp, _l]),
    "orc_rmsnorm": (_i, [_vp, _vp, _vp, _f, _i, _i, _i]),
    "orc_layernorm": (_i, [_vp, _vp, _vp, _vp, _f, _i, _i, _i]),
    "orc_silu": (None, [_vp, _vp, _l, _i]),
    "orc_rmsnorm_lanes": (_i, [_vp, _vp, _vp, _f, _i, _i]),
    "orc_layernorm_lanes": (_i, [_vp, _vp, _vp, _vp, _f, _i, _i]),
    "orc_softmax_lanes": (_i, [_vp, _vp, _i, _i, _i, _i, _vp, _i]),
    "orc_sigmoid": (None, [_vp, _vp, _l, _i]),
    "orc_gelu": (None, [_vp, _vp, _l]),
    "orc_tanh": (None, [_vp, _vp, _l, _i]),
    "orc_polar": (None, [_f, _f, _fp, _fp]),
    "orc_project": (_f, [_f, _f, _f]),
    "orc_prim": (None, [_i, _l, _vp, _vp, _vp, _i, _vp, _vp]),
    "orc_outer": (None, [_vp, _vp, _vp, _i, _i]),
    "orc_dct": (None, [_vp, _vp, _i]),
    "orc_attention": (_i, [_vp, _vp, _vp, _vp, _i, _vp, _i, _i, _i, _i, _i, _i]),
    "orc_fp16_to_fp32": (_f, [C.c_uint16]),
    "orc_fp32_to_fp16": (C.c_uint16, [_f]),
    "orc_q8_0_quantize": (None, [_vp, _vp, _l, _i]),
    "orc_q8_0_dequantize": (None, [_vp, _vp, _l, _i]),
    "orc_q8_0_block_dot": (_f, [_vp, _vp]),
    "orc_q8_0_gemv": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i]),
    "orc_dsp_gen_roms": (None, [_vp, _vp, _vp]),
    "orc_dsp_set_roms": (None, [_vp, _vp, _vp]),
    "orc_dsp_eval": (None, [C.c_int64, C.c_int64, C.c_int64, _i, _vp, _vp, _vp]),
    "orc_dsp_eval_batch": (None, [_i, _l, _vp, _vp, _vp, _vp, _vp, _vp]),
    "orc_dsp_systolic": (None, [_i, _i, _vp, _vp, _vp]),
    "orc_check_chain_all_mantissas": (_l, [_i, _i]),
    "orc_st_to_f32": (_i, [_i, _vp, _l, _vp]),
    "orc_check_projection_identity": (_l, [_i, _l, C.c_uint64]),
}

_REF_SIGS = {
    "ref_tables": (None, [_vp, _vp, _vp, _vp]),
    "ref_cordic_rotate": (None, [_f, _f, _f, _i, _fp, _fp]),
    "rac_matmul": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "rac_sgemm": (_i, [_vp, _vp, _vp, _i, _i, _i, _f, _f, _vp]),
    "rac_hal_matmul": (_i, [_vp, _vp, _vp, _i, _i, _i]),
    "rac_softmax_batch": (None, [_vp, _vp, _i, _i]),
    "rac_rope_cache": (_i, [_vp, _vp, _i, _i, _f]),
    "rac_rope_apply": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "rac_rmsnorm": (_i, [_vp, _vp, _vp, _f, _i, _i, _vp]),
    "rac_layernorm": (_i, [_vp, _vp, _vp, _vp, _f, _i, _i, _vp]),
    "rac_silu": (None, [_vp, _vp, _i]),
    "rac_gelu": (None, [_vp, _vp, _i]),
    "rac_hal_silu": (None, [_vp, _vp, _i]),
    "rac_rsqrt": (_f, [_f]),
    "rac_sigmoid": (_f, [_f]),
    "rac_sincos": (None, [_f, _fp, _fp]),
    "rac_alu_exp": (_f, [_f]),
    "rac_rotate": (Vec2, [Vec2, _f]),
    "rac_rotate_raw": (Vec2, [Vec2, _f]),
    "rac_compensate": (Vec2, [Vec2, _i]),
    "rac_project": (_f, [Vec2, _f]),
    "rac_polar": (None, [Vec2, _fp, _fp]),
    "rac_norm": (_f, [Vec2]),
    "rac_normalize": (Vec2, [Vec2]),
    "rac_dot": (_f, [Vec2, Vec2]),
    "rac_coherence": (_f, [Vec2, Vec2]),
    "rac_complex_mul": (Vec2, [Vec2, Vec2]),
    "rac_rotate_n": (Vec2, [Vec2, _f, _i]),
    "rac_project_n": (_f, [Vec2, _f, _i]),
    "rac_dct": (None, [_vp, _vp, _i]),
    "rac_rotate_batch": (None, [_vp, _vp, _vp, _i]),
    "rac_inner": (_f, [_vp, _vp, _i]),
    "rac_outer": (None, [_vp, _vp, _vp, _i, _i]),
    "rac_scaled_dot_attention": (_i, [_vp, _vp, _vp, _vp, _i, _vp, _i, _i, _i, _i, _vp]),
    "rac_load_all_roms": (_i, [C.c_char_p, C.c_char_p, C.c_char_p]),
    "rac_dsp_eval": (None, [C.c_int64, C.c_int64, C.c_int64, _i, _vp, _vp, _vp]),
    "rac_dsp_project_sum": (C.c_int64, [_i, _vp, _vp]),
    "rac_dsp_project_batch": (None, [_i, _vp, _vp, _vp]),
    "st_open": (_stf, [C.c_char_p, C.c_char_p]),
    "st_close": (None, [_stf]),
    "st_find": (_stt, [_stf, C.c_char_p]),
    "st_to_f32": (_i, [_stf, _stt, _vp]),
    "st_numel": (C.c_size_t, [_stt]),
    "rac_fp16_to_fp32": (_f, [C.c_uint16]),
    "rac_fp32_to_fp16": (C.c_uint16, [_f]),
    "rac_q8_0_quantize_matrix": (None, [_vp, _vp, _i, _i]),
    "rac_q8_0_dequantize_row": (None, [_vp, _vp, _i]),
    "rac_q8_0_gemv": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i]),
}

# Vector-primitive op codes shared by orc_prim and rac_vec2_dev:
# name -> (code, writes a pair, reads b, reads theta)
PRIM_OPS = {
    "rotate": (0, True, False, True),
    "rotate_raw": (1, True, False, True),
    "compensate": (2, True, False, False),
    "project": (3, False, False, True),
    "polar": (4, True, False, False),
    "normalize": (5, True, False, False),
    "dot": (6, False, True, False),
    "coherence": (7, False, True, False),
    "complex_mul": (8, True, True, False),
    "rotate_n": (9, True, False, True),
    "project_n": (10, False, False, True),
    "inner_term": (11, False, True, False),
}

_cache = {}


def _load(path, sigs):
    if path in _cache:
        return _cache[path]
    lib = C.CDLL(path, mode=C.RTLD_LOCAL)
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _cache[path] = lib
    return lib


def oracle():
    return _load(ORACLE_SO, _ORACLE_SIGS)


def have_ref() -> bool:
    return os.path.exists(REF_SO)


def ref():
    return _load(REF_SO, _REF_SIGS)


def p(a: np.ndarray) -> int:
    """Data pointer of a C-contiguous numpy array."""
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ── deterministic inputs ────────────────────────────────────────────────────

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def _splitmix(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        x = x + np.uint64(0x9E3779B97F4A7C15)
        x = (x ^ (x >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        x = (x ^ (x >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return x ^ (x >> np.uint64(31))


def gen_u01(count: int, seed: int) -> np.ndarray:
    """u = (splitmix64(seed*C + i) >> 40) * 2^-24, exactly representable."""
    with np.errstate(over="ignore"):
        base = np.uint64(seed) * np.uint64(0xD1B54A32D192ED03)
        idx = np.arange(count, dtype=np.uint64) + base
    z = _splitmix(idx)
    return (z >> np.uint64(40)).astype(np.float64) * (1.0 / 16777216.0)


def gen_uniform(shape, seed: int, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape))
    return (lo + (hi - lo) * gen_u01(n, seed)).astype(np.float32).reshape(shape)


def gen_normal(shape, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """Box-Muller in float64 from two uniform streams, cast to float32."""
    n = int(np.prod(shape))
    u = gen_u01(2 * n, seed)
    u1, u2 = u[0::2], u[1::2]
    r = np.sqrt(-2.0 * np.log(1.0 - u1))
    return (mean + std * r * np.cos(2.0 * np.pi * u2)).astype(np.float32).reshape(shape)


def sha256(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


# ── oracle wrappers on numpy arrays ─────────────────────────────────────────

def orc_matmul(A, B, M, N, K, iters, mode, ta=0, tb=0, alpha=1.0, beta=0.0, C0=None, literal=0):
    Cm = np.zeros((M, N), np.float32) if C0 is None else np.array(C0, np.float32, copy=True)
    rc = oracle().orc_matmul(ta, tb, p(A), p(B), p(Cm), M, N, K, alpha, beta, iters, mode, literal)
    assert rc == 0
    return Cm


def orc_matmul_entries(A, B, M, N, K, iters, mode, rows, cols, ta=0, tb=0):
    rows = np.ascontiguousarray(rows, np.int32)
    cols = np.ascontiguousarray(cols, np.int32)
    out = np.empty(len(rows), np.float32)
    oracle().orc_matmul_entries(ta, tb, p(A), p(B), M, N, K, iters, mode, p(rows), p(cols),
                                len(rows), p(out))
    return out


def orc_unary(name, x, iters=None):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    fn = getattr(oracle(), name)
    if iters is None:
        fn(p(x), p(y), x.size)
    else:
        fn(p(x), p(y), x.size, iters)
    return y


def orc_softmax(x, iters):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    oracle().orc_softmax_rows(p(x), p(y), x.shape[0], x.shape[1], iters)
    return y


def orc_rmsnorm(x, g, eps, use_cordic=1):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    assert oracle().orc_rmsnorm(p(x), p(y), p(g) if g is not None else None, eps,
                                x.shape[0], x.shape[1], use_cordic) == 0
    return y


def orc_layernorm(x, g, b, eps, use_cordic=1):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    assert oracle().orc_layernorm(p(x), p(y), p(g) if g is not None else None,
                                  p(b) if b is not None else None, eps,
                                  x.shape[0], x.shape[1], use_cordic) == 0
    return y


def orc_rmsnorm_lanes(x, g, eps):
    """RMSNorm with the row kernels' lane-order sum (bit-exact checker)."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    assert oracle().orc_rmsnorm_lanes(p(x), p(y), p(g) if g is not None else None, eps,
                                      x.shape[0], x.shape[1]) == 0
    return y


def orc_layernorm_lanes(x, g, b, eps):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    assert oracle().orc_layernorm_lanes(p(x), p(y), p(g) if g is not None else None,
                                        p(b) if b is not None else None, eps, x.shape[0], x.shape[1]) == 0
    return y


def orc_softmax_lanes(x, iters, causal=False, mask=None, zero_guard=False):
    """Row softmax with the row kernels' lane-order sum; with masking, row r
    is query position r % n (the attention layout)."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    m = None if mask is None else np.ascontiguousarray(mask, np.float32)
    assert oracle().orc_softmax_lanes(p(x), p(y), x.shape[0], x.shape[1], iters, int(causal),
                                      p(m) if m is not None else None, int(zero_guard)) == 0
    return y


def orc_rope_cache(max_seq, head_dim, base=10000.0):
    half = head_dim // 2
    c = np.empty((max_seq, half), np.float32)
    s = np.empty((max_seq, half), np.float32)
    assert oracle().orc_rope_cache(p(c), p(s), max_seq, head_dim, base) == 0
    return c, s


def orc_rope_apply(x, c, s):
    x = np.array(x, np.float32, copy=True, order="C")
    B, H, T, D = x.shape
    assert oracle().orc_rope_apply(p(x), p(c), p(s), B, H, T, D) == 0
    return x


def max_rel(a, b, floor=1e-30):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b) / np.maximum(np.abs(b), floor))) if a.size else 0.0


def orc_prim(name, a, b=None, th=None, iarg=0):
    """Oracle primitive `name` over pairs a [n, 2] (and b [n, 2], th [n])."""
    code, pair, _, _ = PRIM_OPS[name]
    a = np.ascontiguousarray(a, np.float32).reshape(-1, 2)
    n = a.shape[0]
    b = None if b is None else np.ascontiguousarray(b, np.float32).reshape(-1, 2)
    th = None if th is None else np.ascontiguousarray(th, np.float32)
    out = np.zeros((n, 2) if pair else (n,), np.float32)
    oracle().orc_prim(code, n, p(a), p(b) if b is not None else None,
                      p(th) if th is not None else None, iarg,
                      p(out) if pair else None, None if pair else p(out))
    return out


def orc_attention(q, k, v, mask, causal, iters, mode):
    q, k, v = (np.ascontiguousarray(t, np.float32) for t in (q, k, v))
    B, H, T, D = q.shape
    out = np.empty_like(q)
    m = None if mask is None else np.ascontiguousarray(mask, np.float32)
    assert oracle().orc_attention(p(q), p(k), p(v), p(m) if m is not None else None, int(causal),
                                  p(out), B, H, T, D, iters, mode) == 0
    return out


def orc_attention_lanes(q, k, v, mask, causal, iters, mode):
    """rac_attention composed from the checker's products and the lane-order
    masked softmax (zero-sum guard on), head by head: the GPU's bits."""
    q, k, v = (np.ascontiguousarray(t, np.float32) for t in (q, k, v))
    B, Hh, Tn, D = q.shape
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    out = np.empty_like(q)
    for b in range(B):
        for h in range(Hh):
            sc = orc_matmul(q[b, h], k[b, h], Tn, Tn, D, iters, mode, tb=1, alpha=scale)
            pr = orc_softmax_lanes(sc, iters, causal=causal, mask=mask, zero_guard=True)
            out[b, h] = orc_matmul(pr, v[b, h], Tn, D, Tn, iters, mode)
    return out


Q8_BYTES = 34


def orc_q8_quantize(w):
    """[rows, K] float32 -> [rows, K/32, 34] uint8 Q8_0 blocks (oracle)."""
    w = np.ascontiguousarray(w, np.float32)
    rows, K = w.shape
    out = np.zeros((rows, K // 32, Q8_BYTES), np.uint8)
    oracle().orc_q8_0_quantize(p(w), p(out), rows, K)
    return out


def orc_q8_gemv(x, wq, bias, act, contract=1):
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    M, K = x.shape
    N = wq.shape[0]
    out = np.zeros((M, N), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    assert oracle().orc_q8_0_gemv(p(x), p(np.ascontiguousarray(wq)), p(b) if b is not None else None, p(out),
                                  M, N, K, act, contract) == 0
    return out


def orc_dsp_batch(op, x, y, z):
    x, y, z = (np.ascontiguousarray(t, np.int64) for t in (x, y, z))
    n = x.size
    xo, yo, zo = (np.zeros(n, np.int64) for _ in range(3))
    oracle().orc_dsp_eval_batch(op, n, p(x), p(y), p(z), p(xo), p(yo), p(zo))
    return xo, yo, zo


# ── safetensors files ───────────────────────────────────────────────────────

def st_bytes(header, data: bytes) -> bytes:
    """A safetensors file: u64 little-endian header length, header JSON, data."""
    h = header if isinstance(header, (bytes, str)) else json.dumps(header, separators=(",", ":"))
    h = h.encode() if isinstance(h, str) else h
    return len(h).to_bytes(8, "little") + h + data


def orc_st_to_f32(dtype: int, raw: bytes, n: int) -> np.ndarray:
    """The CPU checker's widening of n raw elements (safetensors_reader.c:406-425)."""
    src = np.frombuffer(raw, np.uint8).copy()
    out = np.zeros(max(n, 1), np.float32)
    assert oracle().orc_st_to_f32(dtype, p(src), n, p(out)) == 0
    return out[:n]
