"""ctypes binding of librac_amd.so, the gfx950 kernel library.

The library is loaded after torch so that it shares torch's HIP runtime
(same soname, libamdhip64.so.7): device pointers and streams are then
interchangeable between the two.  There is no fallback: if the library is
missing or the device is not usable, every op raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "librac_amd.so")

_lock = threading.Lock()
_lib = None

c_float_p = ctypes.POINTER(ctypes.c_float)
_vp = ctypes.c_void_p
_i = ctypes.c_int
_l = ctypes.c_long
_f = ctypes.c_float



class Vec2(ctypes.Structure):
    """The rac.h pair type: struct { float x, y; } (rac.h:31), by value."""

    _fields_ = [("x", ctypes.c_float), ("y", ctypes.c_float)]


_v2 = Vec2

ST_MAX_TENSORS, ST_MAX_NAME, ST_MAX_NDIM = 8192, 256, 8


class StTensor(ctypes.Structure):
    """st_tensor (safetensors_reader.h:51-58)."""

    _fields_ = [("name", ctypes.c_char * ST_MAX_NAME), ("dtype", ctypes.c_int), ("ndim", ctypes.c_int),
                ("shape", ctypes.c_int64 * ST_MAX_NDIM), ("offset", ctypes.c_size_t),
                ("nbytes", ctypes.c_size_t)]


class StFile(ctypes.Structure):
    """st_file (safetensors_reader.h:60-69)."""

    _fields_ = [("fd", ctypes.c_int), ("mmap_base", ctypes.c_void_p), ("mmap_len", ctypes.c_size_t),
                ("data_offset", ctypes.c_size_t), ("tensors", ctypes.POINTER(StTensor)),
                ("n_tensors", ctypes.c_int), ("header_copy", ctypes.c_char_p), ("err", ctypes.c_char * 256)]


_stf = ctypes.POINTER(StFile)
_stt = ctypes.POINTER(StTensor)

# name -> (restype, argtypes)
_SIGNATURES = {
    # rac_ext.h — device pointers, explicit stream
    "rac_gemm_dev": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _f, _i, _i, _vp]),
    "rac_gemm_batched_dev": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _f, _i, _i, _i, _l, _l, _l, _vp]),
    "rac_softmax_masked_dev": (_i, [_vp, _vp, _l, _l, _vp, _i, _i, _vp]),
    "rac_fused_linear_dev": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp]),
    "rac_act_grad_dev": (_i, [_vp, _vp, _vp, _l, _i, _i, _vp]),
    "rac_softmax_dev": (_i, [_vp, _vp, _l, _l, _i, _vp]),
    "rac_exp_dev": (_i, [_vp, _vp, _l, _i, _vp]),
    "rac_silu_dev": (_i, [_vp, _vp, _l, _i, _vp]),
    "rac_sigmoid_dev": (_i, [_vp, _vp, _l, _i, _vp]),
    "rac_tanh_dev": (_i, [_vp, _vp, _l, _i, _vp]),
    "rac_gelu_dev": (_i, [_vp, _vp, _l, _vp]),
    "rac_relu_dev": (_i, [_vp, _vp, _l, _vp]),
    "rac_rsqrt_dev": (_i, [_vp, _vp, _l, _vp]),
    "rac_sincos_dev": (_i, [_vp, _vp, _vp, _l, _vp]),
    "rac_rmsnorm_dev": (_i, [_vp, _vp, _vp, _f, _l, _l, _vp]),
    "rac_layernorm_dev": (_i, [_vp, _vp, _vp, _vp, _f, _l, _l, _vp]),
    "rac_rope_cache_dev": (_i, [_vp, _vp, _i, _i, _f, _vp, _vp]),
    "rac_rope_inv_freq": (_i, [_vp, _i, _f]),
    "rac_rope_apply_out_dev": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _l, _l, _l, _l, _l, _l, _vp]),
    "rac_rope_apply_dev": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _l, _l, _l, _vp]),
    "rac_vec2_dev": (_i, [_i, _l, _vp, _vp, _vp, _i, _vp, _vp, _vp]),
    "rac_inner_dev": (_i, [_vp, _vp, _l, _vp, _vp]),
    "rac_outer_dev": (_i, [_vp, _vp, _vp, _i, _i, _vp]),
    "rac_dct_dev": (_i, [_vp, _vp, _i, _vp]),
    "rac_attention_workspace_bytes": (_l, [_i, _i, _i]),
    "rac_attention_dev": (_i, [_vp, _vp, _vp, _vp, _i, _vp, _i, _i, _i, _i, _vp, _i, _i, _vp]),
    "rac_attention_probs_workspace_bytes": (_l, [_i, _i, _i]),
    "rac_attention_noalloc_dev": (_i, [_vp, _vp, _vp, _vp, _i, _vp, _i, _i, _i, _i, _i, _i, _vp]),
    "rac_attention_ws_dev": (_i, [_vp, _vp, _vp, _vp, _i, _vp, _i, _i, _i, _i, _vp, _l, _i, _i, _vp]),
    "rac_attention_probs_dev": (_i, [_vp, _vp, _vp, _vp, _i, _vp, _i, _i, _i, _i, _vp, _i, _i, _vp]),
    "rac_attention_probs_rows_dev": (_i, [_vp, _vp, _vp, _i, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _vp]),
    # rac_decode.h — decode step pieces, cache position in device memory
    "rac_decode_attention_dev": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _l, _vp, _f, _i, _vp]),
    "rac_kv_append_dev": (_i, [_vp, _vp, _vp, _i, _i, _l, _vp, _vp]),
    "rac_position_advance_dev": (_i, [_vp, _i, _vp]),
    "rac_swiglu_dev": (_i, [_vp, _vp, _l, _i, _vp]),
    "rac_q8_0_gemv_rmsnorm_dev": (_i, [_vp, _vp, _f, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "rac_decode_qkv_dev": (_i, [_vp, _vp, _f, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _l, _vp, _vp]),
    "rac_decode_swiglu_gemv_dev": (_i, [_vp, _vp, _f, _vp, _vp, _i, _i, _i, _vp]),
    "rac_q8_0_gemv_dev": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "rac_q8_0_quantize_dev": (_i, [_vp, _vp, _l, _i, _vp]),
    "rac_q8_0_dequantize_dev": (_i, [_vp, _vp, _l, _i, _vp]),
    "rac_q8_0_gemv": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i]),
    "rac_q8_0_quantize_row": (None, [_vp, _vp, _i]),
    "rac_q8_0_quantize_matrix": (None, [_vp, _vp, _i, _i]),
    "rac_q8_0_dequantize_row": (None, [_vp, _vp, _i]),
    # rac_dsp.h — the fixed-point RAC-DSP engine (int64 operands)
    "rac_load_hex_lut": (_i, [ctypes.c_char_p, _vp, _i]),
    "rac_load_all_roms": (_i, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p]),
    "rac_dsp_set_roms": (None, [_vp, _vp, _vp]),
    "rac_dsp_get_roms": (None, [_vp, _vp, _vp]),
    "rac_dsp_eval": (None, [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _i, _vp, _vp, _vp]),
    "rac_dsp_project_batch": (None, [_i, _vp, _vp, _vp]),
    "rac_dsp_project_sum": (ctypes.c_int64, [_i, _vp, _vp]),
    "rac_dsp_eval_dev": (_i, [_i, _l, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "rac_dsp_systolic_dev": (_i, [_i, _i, _vp, _vp, _vp, _vp]),
    # rac_safetensors.h — the reader (safetensors_reader.h:73-96) + device forms
    "st_open": (_stf, [ctypes.c_char_p, ctypes.c_char_p]),
    "st_close": (None, [_stf]),
    "st_find": (_stt, [_stf, ctypes.c_char_p]),
    "st_data": (_vp, [_stf, _stt]),
    "st_to_f32": (_i, [_stf, _stt, _vp]),
    "st_numel": (ctypes.c_size_t, [_stt]),
    "st_dtype_name": (ctypes.c_char_p, [_i]),
    "st_dump": (None, [_stf]),
    "rac_st_to_f32_dev": (_i, [_stf, _stt, _vp, _vp]),
    "rac_st_to_q8_0_dev": (_i, [_stf, _stt, _vp, _vp]),
    "rac_st_convert_dev": (_i, [_i, _vp, _l, _vp, _vp]),
    "rac_st_quantize_dev": (_i, [_i, _vp, _l, _vp, _vp]),
    "rac_fp16_to_fp32": (_f, [ctypes.c_uint16]),
    "rac_fp32_to_fp16": (ctypes.c_uint16, [_f]),
    "rac_last_error": (ctypes.c_char_p, []),
    "rac_clear_error": (None, []),
    "rac_release_cached_memory": (_l, []),
    "rac_set_cordic_iters": (None, [_i]),
    "rac_get_cordic_iters": (_i, []),
    "rac_set_cordic_mode": (None, [_i]),
    "rac_get_cordic_mode": (_i, []),
    "rac_set_stream": (None, [_vp]),
    "rac_get_stream": (_vp, []),
    "rac_version": (_i, []),
    "rac_cordic_direction_bits": (_i, [_i, _vp]),
    "rac_exp_gain_inverse": (_f, [_i]),
    "rac_rsqrt_gain_inverse": (_f, []),
    # rac.h — synchronous, pointer-agnostic
    "rac_matmul": (None, [_vp, _vp, _vp, _i, _i, _i]),
    "rac_softmax": (None, [_vp, _vp, _i]),
    "rac_softmax_batch": (None, [_vp, _vp, _i, _i]),
    "rac_exp": (_f, [_f]),
    "rac_tanh": (_f, [_f]),
    "rac_sigmoid": (_f, [_f]),
    "rac_rsqrt": (_f, [_f]),
    "rac_sincos": (None, [_f, c_float_p, c_float_p]),
    "rac_rmsnorm": (None, [_vp, _vp, _vp, _f, _i, _i]),
    "rac_layernorm": (None, [_vp, _vp, _vp, _vp, _f, _i, _i]),
    "rac_rope_cache": (None, [_vp, _vp, _i, _i, _f]),
    "rac_rope_apply": (None, [_vp, _vp, _vp, _i, _i, _i, _i]),
    "rac_relu": (None, [_vp, _vp, _i]),
    "rac_gelu": (None, [_vp, _vp, _i]),
    "rac_silu": (None, [_vp, _vp, _i]),
    "rac_rotate": (_v2, [_v2, _f]),
    "rac_rotate_raw": (_v2, [_v2, _f]),
    "rac_compensate": (_v2, [_v2, _i]),
    "rac_project": (_f, [_v2, _f]),
    "rac_polar": (None, [_v2, c_float_p, c_float_p]),
    "rac_norm": (_f, [_v2]),
    "rac_normalize": (_v2, [_v2]),
    "rac_dot": (_f, [_v2, _v2]),
    "rac_coherence": (_f, [_v2, _v2]),
    "rac_complex_mul": (_v2, [_v2, _v2]),
    "rac_dct": (None, [_vp, _vp, _i]),
    "rac_rotate_batch": (None, [_vp, _vp, _vp, _i]),
    "rac_inner": (_f, [_vp, _vp, _i]),
    "rac_outer": (None, [_vp, _vp, _vp, _i, _i]),
    "rac_attention": (None, [_vp, _vp, _vp, _vp, _i, _vp, _i, _i, _i, _i]),
    "rac_rotate_precision": (_v2, [_v2, _f, _i]),
    "rac_project_precision": (_f, [_v2, _f, _i]),
    "rac_create_context": (_vp, [_i]),
    "rac_destroy_context": (None, [_vp]),
    "rac_query_capability": (_i, [_vp, _i]),
    "rac_execute": (_i, [_vp, _i, _vp]),
    # reference launcher ABI (rac_kernels.hip:822-909)
    "rac_launch_nn_iters": (None, [_vp, _vp, _vp, _i, _i, _i, _f, _f, _i, _i, _vp]),
    "rac_launch_nt_iters": (None, [_vp, _vp, _vp, _i, _i, _i, _f, _f, _i, _i, _vp]),
    "rac_launch_tn_iters": (None, [_vp, _vp, _vp, _i, _i, _i, _f, _f, _i, _i, _vp]),
    "rac_launch_nn": (None, [_vp, _vp, _vp, _i, _i, _i, _f, _f, _vp]),
    "rac_launch_nt": (None, [_vp, _vp, _vp, _i, _i, _i, _f, _f, _vp]),
    "rac_launch_tn": (None, [_vp, _vp, _vp, _i, _i, _i, _f, _f, _vp]),
}


class RACError(RuntimeError):
    """A librac_amd call failed (bad arguments, or a HIP error)."""


def load(path: str | None = None) -> ctypes.CDLL:
    """Load librac_amd.so (once) and declare every exported signature."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = path or LIB_PATH
        if not os.path.exists(p):
            raise RACError(
                f"{p} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
                "or `make -C rac_amd/csrc` (hipcc, gfx950)")
        lib = ctypes.CDLL(p, mode=ctypes.RTLD_LOCAL)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if path is None:
            _lib = lib
        return lib


def release_cached_memory() -> int:
    """Free the device staging buffers the synchronous rac.h calls keep
    cached (at most RAC_STAGE_CACHE_MB per GPU); returns the bytes freed.
    Call it when another allocator in the process (torch's) runs short."""
    return int(load().rac_release_cached_memory())


def symbols() -> list[str]:
    return list(_SIGNATURES)


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().rac_last_error()
        raise RACError(f"{what} failed ({rc}): {msg.decode() if msg else ''}")


def stream_handle(device: torch.device | None = None) -> int:
    """Raw hipStream_t of torch's current stream on `device`."""
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor) -> int:
    return t.data_ptr()
