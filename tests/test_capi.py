"""C ABI of librac_amd.so and the Python surface — CPU only (no kernel launch).

Checks that the library loads, exports every function include/*.h declares,
that the headers compile as plain C against it, that the host-side constants
equal the CPU checker's, and that argument errors are reported before any
device call.
"""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

import raclib as rl

ROOT = rl.ROOT
HEADERS = [os.path.join(ROOT, "include", h) for h in ("rac.h", "rac_ext.h", "rac_q8_0.h", "rac_dsp.h",
                                                               "rac_safetensors.h", "rac_decode.h")]


def declared_functions():
    names = set()
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b([a-z_][a-z0-9_]*)\s*\(", text):
            name = m.group(1)
            if (name.startswith("rac_") or name.startswith("st_")) and not name.startswith("rac_context"):
                names.add(name)
    return sorted(names)


@pytest.fixture(scope="module")
def lib():
    import torch  # noqa: F401  (share torch's HIP runtime, as the product does)
    import rac_amd
    return rac_amd.load()


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", os.path.join(ROOT, "rac_amd", "librac_amd.so")],
                         capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, missing
    assert len(declared_functions()) > 40


def test_python_binding_covers_headers():
    from rac_amd import _lib
    assert set(declared_functions()) <= set(_lib.symbols())


def test_headers_compile_and_link_as_c(tmp_path):
    src = tmp_path / "t.c"
    src.write_text('#include "rac.h"\n#include "rac_ext.h"\n#include "rac_q8_0.h"\n#include "rac_dsp.h"\n'
                   '#include "rac_safetensors.h"\n#include "rac_decode.h"\n'
                   "int main(void){ rac_set_cordic_iters(8); return rac_get_cordic_iters() == 8 ? 0 : 1; }\n")
    exe = tmp_path / "t"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
                    str(src), "-o", str(exe), "-L", os.path.join(ROOT, "rac_amd"), "-lrac_amd",
                    "-Wl,-rpath," + os.path.join(ROOT, "rac_amd")], check=True)


def test_constants_match_checker(lib):
    o = rl.oracle()
    d = (ctypes.c_int * 24)()
    dd = np.zeros(24, np.int32)
    for n in (1, 8, 16, 24):
        assert lib.rac_cordic_direction_bits(n, d) == n
        o.orc_cordic_dirs(n, rl.p(dd))
        assert list(d)[:n] == list(dd[:n])
    for n in range(1, 25):
        assert np.float32(lib.rac_exp_gain_inverse(n)) == np.float32(o.orc_hyp_kinv(n))
    assert np.float32(lib.rac_rsqrt_gain_inverse()) == np.float32(o.orc_hyp_kinv(16))
    inv = np.zeros(64, np.float32)
    ref = np.zeros(64, np.float32)
    assert lib.rac_rope_inv_freq(rl.p(inv), 128, 10000.0) == 0
    o.orc_rope_inv_freq(rl.p(ref), 128, 10000.0)
    assert np.array_equal(inv, ref)


def test_knob_semantics(lib):
    lib.rac_set_cordic_iters(99)
    assert lib.rac_get_cordic_iters() == 24
    lib.rac_set_cordic_iters(0)
    assert lib.rac_get_cordic_iters() == 16
    lib.rac_set_cordic_iters(8)
    assert lib.rac_get_cordic_iters() == 8
    lib.rac_set_cordic_mode(7)
    assert lib.rac_get_cordic_mode() == 0
    lib.rac_set_cordic_mode(1)
    assert lib.rac_get_cordic_mode() == 1
    lib.rac_set_cordic_iters(16)


def test_argument_errors_before_device(lib):
    assert lib.rac_gemm_dev(None, None, None, 4, 4, 4, 0, 0, 1.0, 0.0, 16, 1, None) == -1
    assert b"null" in lib.rac_last_error()
    buf = (ctypes.c_float * 16)()
    a = ctypes.addressof(buf)
    assert lib.rac_gemm_dev(a, a, a, 0, 4, 4, 0, 0, 1.0, 0.0, 16, 1, None) == -2
    assert lib.rac_gemm_dev(a, a, a, 4, 4, 4, 0, 0, 1.0, 0.0, 16, 5, None) == -2
    assert lib.rac_softmax_dev(a, a, 0, 4, 16, None) == -2
    assert lib.rac_rmsnorm_dev(None, a, None, 1e-6, 1, 4, None) == -1
    assert lib.rac_rope_apply_dev(a, a, a, 1, 1, 4, 3, 12, 12, 3, None) == -2   # odd head_dim
    assert lib.rac_rope_cache_dev(a, a, 4, 6, 1e4, None, None) == -1
    assert lib.rac_rope_inv_freq(a, 5, 1e4) == -2
    # reference-style void entry points report through rac_last_error
    lib.rac_clear_error()
    lib.rac_matmul(None, a, a, 2, 2, 2)
    assert b"null" in lib.rac_last_error()
    lib.rac_rmsnorm(a, a, None, 1e-6, 0, 4)
    assert b"must be > 0" in lib.rac_last_error()
    # context stub semantics of rac_hip.cpp:416-435
    ctx = lib.rac_create_context(1)
    assert ctx
    assert lib.rac_query_capability(ctx, 0xFF) == 0 and lib.rac_query_capability(ctx, 16) == 1
    assert lib.rac_execute(ctx, 16, None) == 0
    lib.rac_destroy_context(ctx)


def test_python_knobs_and_cpu_tensors_raise():
    import torch
    from rac_amd import ext, rac_torch as rt

    ext.set_cordic_iters(0)
    assert ext.get_cordic_iters() == 24
    ext.set_cordic_iters(30)
    assert ext.get_cordic_iters() == 24
    ext.set_cordic_iters(5)
    assert ext.get_cordic_iters() == 5
    ext.set_cordic_mode(9)
    assert ext.get_cordic_mode() == ext.MODE_FAST
    rt.rac_set_precision(2)
    assert rt.rac_get_precision() == 4          # rac_torch.py:1100 clamp
    rt.rac_set_precision(99)
    assert rt.rac_get_precision() == 24
    rt.rac_set_mode('cordic')
    assert rt.rac_get_mode() == rt.MODE_CORDIC
    with pytest.raises(ValueError):
        rt.rac_set_mode('bogus')
    rt.rac_set_mode('fast')
    with pytest.raises(RuntimeError, match="GPU"):
        ext.matmul_forward(torch.ones(2, 2), torch.ones(2, 2))
    with pytest.raises(RuntimeError):
        rt.RACLinear(4, 4)(torch.ones(2, 4))
    with pytest.raises(RuntimeError):
        ext.softmax(torch.ones(2, 4))


def test_module_shapes_and_parameters():
    import torch.nn as nn
    from rac_amd import rac_torch as rt

    lin = rt.RACLinear(16, 8)
    assert lin.weight.shape == (8, 16) and lin.bias.shape == (8,)
    ref = nn.Linear(16, 8)
    r2 = rt.RACLinear.from_linear(ref)
    assert (r2.weight == ref.weight).all()
    blk = rt.RACLlamaBlock(64, 4, ff_dim=176, max_seq_len=32)
    names = {n for n, _ in blk.named_parameters()}
    assert {"norm1.weight", "attn.qkv.weight", "attn.out_proj.weight", "norm2.weight",
            "ffn.fc1.weight", "ffn.fc2.weight"} <= names
    assert blk.attn.qkv.bias is None                        # bias=False default
    model = nn.Sequential(nn.Linear(128, 128), nn.ReLU(), nn.Linear(128, 32))
    rt.patch_model(model, verbose=False, min_features=64)
    assert isinstance(model[0], rt.RACLinear) and not isinstance(model[2], rt.RACLinear)
    rt.unpatch_model(model, verbose=False)
    assert type(model[0]) is nn.Linear
    assert rt._resolve_act('swish') == rt.ACT_SILU
    with pytest.raises(ValueError):
        rt._resolve_act('tanhh')


def test_fp16_helpers_match_reference_golden(lib):
    d = np.load(os.path.join(rl.GOLDEN, "q8.npz"))
    h2f = np.array([lib.rac_fp16_to_fp32(int(h)) for h in d["halves"]], np.float32)
    assert np.array_equal(h2f.view(np.uint32), d["h2f"].view(np.uint32))
    f2h = np.array([lib.rac_fp32_to_fp16(float(v)) for v in d["floats"]], np.uint16)
    assert np.array_equal(f2h, d["f2h"])


def test_q8_argument_errors_before_device(lib):
    buf = (ctypes.c_float * 64)()
    a = ctypes.addressof(buf)
    assert lib.rac_q8_0_gemv(a, a, None, a, 4, 48, 0) == -2       # K not a multiple of 32
    assert lib.rac_q8_0_gemv(None, a, None, a, 4, 64, 0) == -1
    assert lib.rac_q8_0_gemv_dev(a, a, None, a, 1, 4, 64, 9, None) == -2   # act
    assert lib.rac_q8_0_quantize_dev(a, a, 0, 64, None) == -2


def _dsp_roms(lib):
    lut, at, ath = np.zeros(1024, np.uint64), np.zeros(17, np.int64), np.zeros(9, np.int64)
    lib.rac_dsp_get_roms(rl.p(lut), rl.p(at), rl.p(ath))
    return lut, at, ath


def _write_mem(path, values, comment=True):
    with open(path, "w") as f:
        if comment:
            f.write("// generated for the test\n\n")
        for v in values:
            f.write("%016x\n" % (int(v) & (2 ** 64 - 1)))


def test_dsp_generated_roms_equal_rtl_mem_golden(lib):
    d = np.load(os.path.join(rl.GOLDEN, "dsp.npz"))
    lut, at, ath = _dsp_roms(lib)
    assert np.array_equal(lut, d["lut"]) and np.array_equal(at, d["atan"]) and np.array_equal(ath, d["atanh"])


def test_dsp_rom_loaders(lib, tmp_path):
    d = np.load(os.path.join(rl.GOLDEN, "dsp.npz"))
    paths = [str(tmp_path / n) for n in ("lut.mem", "atan.mem", "atanh.mem")]
    lut2 = d["lut"][::-1].copy()
    at2 = d["atan"] + 3
    _write_mem(paths[0], lut2)
    _write_mem(paths[1], at2)
    _write_mem(paths[2], d["atanh"], comment=False)
    buf = np.zeros(1024, np.uint64)
    assert lib.rac_load_hex_lut(paths[0].encode(), rl.p(buf), 1024) == 1024
    assert np.array_equal(buf, lut2)
    assert lib.rac_load_hex_lut(paths[1].encode(), rl.p(buf), 5) == 5           # capped at `expected`
    assert lib.rac_load_hex_lut(str(tmp_path / "absent").encode(), rl.p(buf), 4) == -1
    g_lut, g_at, g_ath = d["lut"], d["atan"], d["atanh"]       # held: rl.p does not own the memory

    def restore():
        lib.rac_dsp_set_roms(rl.p(g_lut), rl.p(g_at), rl.p(g_ath))

    try:
        missing = str(tmp_path / "absent").encode()
        # the files are applied in order and a failure stops there, with the
        # earlier ROMs already replaced (sim/rac_dsp_core.c:74-89)
        assert lib.rac_load_all_roms(missing, paths[1].encode(), paths[2].encode()) == 1
        lut, at, ath = _dsp_roms(lib)
        assert np.array_equal(lut, g_lut) and np.array_equal(at, g_at)
        assert lib.rac_load_all_roms(paths[0].encode(), missing, paths[2].encode()) == 2
        lut, at, ath = _dsp_roms(lib)
        assert np.array_equal(lut, lut2) and np.array_equal(at, g_at)
        restore()
        assert lib.rac_load_all_roms(paths[0].encode(), paths[1].encode(), missing) == 3
        lut, at, ath = _dsp_roms(lib)
        assert np.array_equal(lut, lut2) and np.array_equal(at, at2) and np.array_equal(ath, g_ath)
        restore()
        assert lib.rac_load_all_roms(*(p.encode() for p in paths)) == 0
        lut, at, ath = _dsp_roms(lib)
        assert np.array_equal(lut, lut2) and np.array_equal(at, at2) and np.array_equal(ath, g_ath)
        lib.rac_dsp_set_roms(None, rl.p(g_at), None)
        lut, at, _ = _dsp_roms(lib)
        assert np.array_equal(lut, lut2) and np.array_equal(at, g_at)
        # a short file replaces only the entries it holds; the rest keep
        # their previous values (for the LUT exactly as the reference does)
        restore()
        short = [str(tmp_path / n) for n in ("lut_short.mem", "atan_short.mem", "atanh_short.mem")]
        _write_mem(short[0], lut2[:10])
        _write_mem(short[1], at2[:5])
        _write_mem(short[2], g_ath[:2] + 7)
        assert lib.rac_load_all_roms(*(p.encode() for p in short)) == 0
        lut, at, ath = _dsp_roms(lib)
        assert np.array_equal(lut[:10], lut2[:10]) and np.array_equal(lut[10:], g_lut[10:])
        assert np.array_equal(at[:5], at2[:5]) and np.array_equal(at[5:], g_at[5:])
        assert np.array_equal(ath[:2], g_ath[:2] + 7) and np.array_equal(ath[2:], g_ath[2:])
    finally:
        restore()
    lut, at, ath = _dsp_roms(lib)
    assert np.array_equal(lut, d["lut"]) and np.array_equal(at, d["atan"]) and np.array_equal(ath, d["atanh"])


def test_dsp_argument_errors_before_device(lib):
    buf = (ctypes.c_int64 * 16)()
    a = ctypes.addressof(buf)
    assert lib.rac_dsp_eval_dev(0, 4, None, None, a, a, None, None, None) == -1
    assert lib.rac_dsp_eval_dev(0, -1, a, None, a, a, None, None, None) == -2
    assert lib.rac_dsp_eval_dev(0, 0, a, None, a, a, None, None, None) == 0
    assert lib.rac_dsp_systolic_dev(0, 1, a, a, a, None) == -2
    assert lib.rac_dsp_systolic_dev(4, 1, None, a, a, None) == -1
    assert lib.rac_dsp_systolic_dev(65536, 1, a, a, a, None) == -2              # N*N >= 2^31
    lib.rac_clear_error()
    assert lib.rac_dsp_project_sum(0, a, a) == 0
    lib.rac_dsp_project_batch(4, None, a, a)
    assert b"null" in lib.rac_last_error()


# ── safetensors reader (host side: parsing, lookup, argument checks) ─────

def _st_open(lib, path):
    err = ctypes.create_string_buffer(256)
    f = lib.st_open(str(path).encode(), err)
    return f, err.value.decode()


def _st_records(f):
    out = []
    for i in range(f.contents.n_tensors):
        t = f.contents.tensors[i]
        out.append({"name": t.name.decode(), "dtype": t.dtype, "ndim": t.ndim,
                    "shape": [t.shape[k] for k in range(t.ndim)], "offset": t.offset, "nbytes": t.nbytes})
    return out


def test_st_parse_matches_reference_reader(lib, tmp_path):
    import json
    d = np.load(os.path.join(rl.GOLDEN, "st.npz"))
    path = tmp_path / "sample.safetensors"
    blob = d["sample"].tobytes()
    path.write_bytes(blob)
    f, err = _st_open(lib, path)
    assert f, err
    try:
        assert _st_records(f) == json.loads(str(d["parse"]))
        hl = int.from_bytes(blob[:8], "little")
        assert f.contents.data_offset == 8 + hl and f.contents.mmap_len == len(blob)
        t = lib.st_find(f, b"model.layers.0.mlp.up_proj.weight")
        assert t and lib.st_numel(t) == 512
        assert not lib.st_find(f, b"not_there")
        raw = ctypes.string_at(lib.st_data(f, t), t.contents.nbytes)
        assert raw == blob[8 + hl + t.contents.offset: 8 + hl + t.contents.offset + t.contents.nbytes]
        assert lib.st_dtype_name(3) == b"BF16" and lib.st_dtype_name(0) == b"UNKNOWN"
        assert lib.st_dtype_name(99) == b"UNKNOWN"
        scalar = lib.st_find(f, b"scalar")
        assert scalar.contents.ndim == 0 and lib.st_numel(scalar) == 1
    finally:
        lib.st_close(f)
    lib.st_close(None)


def test_st_dump_lists_tensors(lib, tmp_path, capfd):
    d = np.load(os.path.join(rl.GOLDEN, "st.npz"))
    path = tmp_path / "sample.safetensors"
    path.write_bytes(d["sample"].tobytes())
    f, err = _st_open(lib, path)
    lib.st_dump(f)
    lib.st_close(f)
    text = capfd.readouterr().out
    assert "8 tensors" in text and "model.layers.0.mlp.up_proj.weight" in text and "[8, 64]" in text


def test_st_refuses_what_the_reference_refuses(lib, tmp_path):
    import json
    d = np.load(os.path.join(rl.GOLDEN, "st.npz"))
    names = json.loads(str(d["bad_names"]))
    assert not d["bad_opened"].any()
    for i, name in enumerate(names):
        path = tmp_path / f"bad{i}.safetensors"
        path.write_bytes(d[f"bad_{i}"].tobytes())
        f, err = _st_open(lib, path)
        assert not f and err, name
        assert b"st_open" in lib.rac_last_error()
    f, err = _st_open(lib, tmp_path / "absent.safetensors")
    assert not f and "absent" in err


def test_st_validates_ranges_and_sizes(lib, tmp_path):
    """Stricter than the reference reader, which accepts these and later
    reads past the tensor or the mapping."""
    cases = {
        "past_the_end": ({"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}, b"\0" * 4),
        "size_mismatch": ({"a": {"dtype": "F16", "shape": [3], "data_offsets": [0, 8]}}, b"\0" * 8),
        "reversed": ({"a": {"dtype": "F32", "shape": [1], "data_offsets": [4, 0]}}, b"\0" * 8),
        "nine_dims": ({"a": {"dtype": "U8", "shape": [1] * 9, "data_offsets": [0, 1]}}, b"\0"),
        "negative_dim": ({"a": {"dtype": "U8", "shape": [-1], "data_offsets": [0, 1]}}, b"\0"),
    }
    for name, (hdr, data) in cases.items():
        path = tmp_path / f"{name}.safetensors"
        path.write_bytes(rl.st_bytes(hdr, data))
        f, err = _st_open(lib, path)
        assert not f, name
    # unknown dtypes are kept (their size is not checked), escaped names raw
    path = tmp_path / "odd.safetensors"
    path.write_bytes(rl.st_bytes('{"q\\"x":{"dtype":"F8_E4M3","shape":[3],"data_offsets":[0,3]},"__metadata__":{}}',
                                 b"abc"))
    f, err = _st_open(lib, path)
    assert f, err
    assert _st_records(f) == [{"name": 'q\\"x', "dtype": 0, "ndim": 1, "shape": [3], "offset": 0, "nbytes": 3}]
    lib.st_close(f)
    path.write_bytes(rl.st_bytes("{}", b""))
    f, err = _st_open(lib, path)
    assert f and f.contents.n_tensors == 0
    lib.st_close(f)


def test_st_reads_files_written_by_safetensors(lib, tmp_path):
    torch = pytest.importorskip("torch")
    st_torch = pytest.importorskip("safetensors.torch")
    from safetensors import safe_open
    g = torch.Generator().manual_seed(0)
    tensors = {
        "w_bf16": torch.randn(33, 64, generator=g).to(torch.bfloat16),
        "w_f16": torch.randn(7, 96, generator=g).to(torch.float16),
        "w_f32": torch.randn(5, 3, 2, generator=g),
        "w_f64": torch.randn(4, 32, generator=g, dtype=torch.float64),
        "ids": torch.arange(10, dtype=torch.int32),
        "mask": torch.ones(6, dtype=torch.bool),
        "b": torch.zeros(0),
    }
    path = tmp_path / "model.safetensors"
    st_torch.save_file(tensors, str(path), metadata={"format": "pt"})
    f, err = _st_open(lib, path)
    assert f, err
    try:
        recs = {r["name"]: r for r in _st_records(f)}
        assert set(recs) == set(tensors)
        with safe_open(str(path), framework="pt") as sf:
            for name in tensors:
                sl = sf.get_slice(name)
                assert recs[name]["shape"] == list(sl.get_shape()), name
                assert recs[name]["dtype"] == rl.ST_DTYPES[sl.get_dtype()], name
        blob = path.read_bytes()
        base = f.contents.data_offset
        for name, t in tensors.items():
            r = recs[name]
            raw = blob[base + r["offset"]: base + r["offset"] + r["nbytes"]]
            assert raw == t.contiguous().view(torch.uint8).numpy().tobytes(), name
    finally:
        lib.st_close(f)


def test_st_argument_errors_before_device(lib, tmp_path):
    d = np.load(os.path.join(rl.GOLDEN, "st.npz"))
    path = tmp_path / "sample.safetensors"
    path.write_bytes(d["sample"].tobytes())
    f, err = _st_open(lib, path)
    f2, _ = _st_open(lib, path)
    buf = (ctypes.c_float * 1024)()
    a = ctypes.addressof(buf)
    try:
        i8 = lib.st_find(f, b"i8")
        assert lib.st_to_f32(f, i8, a) == -1                             # integer dtype, as the reference
        assert lib.rac_st_to_f32_dev(f, i8, a, None) == -5
        assert lib.rac_st_to_q8_0_dev(f, i8, a, None) == -5
        assert lib.rac_st_to_f32_dev(f, None, a, None) == -1
        assert lib.rac_st_to_f32_dev(f, lib.st_find(f2, b"f16"), a, None) == -1   # tensor of another file
        assert b"another file" in lib.rac_last_error() or b"belong" in lib.rac_last_error()
        assert lib.rac_st_to_q8_0_dev(f, lib.st_find(f, b"f32"), a, None) == -2   # last dim 6
        assert lib.rac_st_convert_dev(5, a, 4, a, None) == -5
        assert lib.rac_st_convert_dev(3, None, 4, a, None) == -1
        assert lib.rac_st_quantize_dev(3, a, -1, a, None) == -2
    finally:
        lib.st_close(f)
        lib.st_close(f2)


def test_dimension_guards_match_reference(lib):
    """Non-positive dimensions are refused with RAC_ERR_INVALID_DIM before any
    device work, as the reference's guards do (rac_cpu.c:393, 482, 515, 556,
    581, 608, 646); an odd head_dim is refused by the RoPE entry points; an
    empty elementwise batch is a no-op and a negative one an error."""
    buf = (ctypes.c_float * 64)()
    a = ctypes.addressof(buf)
    bad = (0, -3)
    for v in bad:
        for M, N, K in ((v, 4, 4), (4, v, 4), (4, 4, v)):
            assert lib.rac_gemm_dev(a, a, a, M, N, K, 0, 0, 1.0, 0.0, 16, 1, None) == -2, (M, N, K)
            assert lib.rac_gemm_batched_dev(a, a, a, M, N, K, 0, 0, 1.0, 0.0, 16, 1, 1, 16, 16, 16,
                                            None) == -2, (M, N, K)
        assert lib.rac_gemm_batched_dev(a, a, a, 4, 4, 4, 0, 0, 1.0, 0.0, 16, 1, v, 16, 16, 16, None) == -2
        for rows, n in ((v, 4), (4, v)):
            assert lib.rac_softmax_dev(a, a, rows, n, 16, None) == -2, (rows, n)
            assert lib.rac_rmsnorm_dev(a, a, a, 1e-6, rows, n, None) == -2, (rows, n)
            assert lib.rac_layernorm_dev(a, a, a, a, 1e-5, rows, n, None) == -2, (rows, n)
        assert lib.rac_softmax_masked_dev(a, a, v, 4, None, 1, 16, None) == -2
        assert lib.rac_softmax_masked_dev(a, a, 4, v, None, 1, 16, None) == -2
        for ms, hd in ((v, 4), (4, v), (4, 5)):
            assert lib.rac_rope_cache_dev(a, a, ms, hd, 1e4, a, None) == -2, (ms, hd)
        for dims in ((v, 1, 4, 4), (1, v, 4, 4), (1, 1, v, 4), (1, 1, 4, v), (1, 1, 4, 5)):
            assert lib.rac_rope_apply_dev(a, a, a, *dims, 16, 16, 4, None) == -2, dims
        for dims in ((v, 1, 4, 4), (1, v, 4, 4), (1, 1, v, 4), (1, 1, 4, v)):
            assert lib.rac_attention_dev(a, a, a, None, 0, a, *dims, a, 16, 1, None) == -2, dims
        for name in ("rac_exp_dev", "rac_silu_dev", "rac_sigmoid_dev", "rac_tanh_dev"):
            rc = getattr(lib, name)(a, a, v, 16, None)
            assert rc == (0 if v == 0 else -2), (name, v)
        for name in ("rac_gelu_dev", "rac_relu_dev", "rac_rsqrt_dev"):
            assert getattr(lib, name)(a, a, v, None) == (0 if v == 0 else -2), (name, v)
    # one softmax workgroup per score row: more than 16777215 rows is refused
    # before the scores product runs
    assert lib.rac_attention_dev(a, a, a, None, 1, a, 1, 4096, 4097, 4, a, 16, 1, None) == -2
    assert b"16777215" in lib.rac_last_error()
    # the reference-style void entry points record the same refusal
    lib.rac_clear_error()
    lib.rac_layernorm(a, a, None, None, 1e-5, 4, 0)
    assert b"must be > 0" in lib.rac_last_error()
    lib.rac_clear_error()
    lib.rac_rope_cache(a, a, 4, 0, 1e4)
    assert lib.rac_last_error() != b""
    lib.rac_clear_error()
    lib.rac_rope_apply(a, a, a, 1, 1, 0, 4)
    assert lib.rac_last_error() != b""
    lib.rac_clear_error()
    lib.rac_attention(a, a, a, None, 0, a, 1, 1, 0, 4)
    assert lib.rac_last_error() != b""


def test_rac_cuda_ext_exports_the_reference_surface():
    """The reference's extension module name (rac_torch_bind.cpp:223-258)
    resolves to rac_amd.ext's objects (no compute calls here)."""
    import rac_cuda_ext
    from rac_amd import ext
    for name in ("matmul_forward", "matmul_backward", "linear_forward", "linear_backward", "set_cordic_iters",
                 "get_cordic_iters", "set_cordic_mode", "get_cordic_mode", "MODE_FAST", "MODE_CORDIC",
                 "MODE_SHIFTADD", "fused_linear_forward", "fused_linear_backward", "softmax", "rmsnorm",
                 "rope_apply_", "attention"):
        assert getattr(rac_cuda_ext, name) is getattr(ext, name), name
    assert set(rac_cuda_ext.__all__) == set(ext.__all__)


def test_patch_helpers_and_qkv_fusion_on_cpu(capsys):
    """patch_model / unpatch_model keep parameters bit for bit and follow the
    min_features rule through nested modules; from_qkv_linears stacks Q, K, V
    rows in that order and refuses mismatched projections."""
    import torch
    import torch.nn as nn
    from rac_amd import rac_torch as rt

    torch.manual_seed(0)
    model = nn.Sequential(nn.Linear(96, 128), nn.Sequential(nn.ReLU(), nn.Linear(128, 80)), nn.Linear(80, 8))
    before = {k: v.clone() for k, v in model.state_dict().items()}
    rt.patch_model(model, verbose=True, min_features=64)
    out = capsys.readouterr().out
    assert isinstance(model[0], rt.RACLinear) and isinstance(model[1][1], rt.RACLinear)
    assert type(model[2]) is nn.Linear                                   # 80 -> 8 is below 64
    assert "2 of 3" in out and "1.1" in out and "min_features=64" in out
    assert all(torch.equal(before[k], v) for k, v in model.state_dict().items())
    rt.unpatch_model(model, verbose=True)
    assert "2 RACLinear" in capsys.readouterr().out
    assert type(model[0]) is nn.Linear and type(model[1][1]) is nn.Linear
    assert all(torch.equal(before[k], v) for k, v in model.state_dict().items())

    lq, lk, lv = (nn.Linear(16, 16) for _ in range(3))
    fused = rt.RACFusedQKV.from_qkv_linears(lq, lk, lv)
    w = fused.qkv.weight.detach()
    assert torch.equal(w[:16], lq.weight) and torch.equal(w[16:32], lk.weight) and torch.equal(w[32:], lv.weight)
    b = fused.qkv.bias.detach()
    assert torch.equal(b[:16], lq.bias) and torch.equal(b[32:], lv.bias)
    with pytest.raises(ValueError):
        rt.RACFusedQKV.from_qkv_linears(lq, nn.Linear(16, 8), lv)
    with pytest.raises(ValueError):
        rt.RACFusedQKV.from_qkv_linears(lq, nn.Linear(16, 16, bias=False), lv)



def test_attention_from_layers_and_path_choice_on_cpu():
    """RACAttention.from_attention_layers stacks Q, K, V into the fused
    projection's row blocks and copies the output projection bit for bit,
    refusing non-square or bias-mismatched layers and heads that do not
    divide d_model; the fused attention core is taken only when nothing sits
    between softmax and P V (identity, or nn.Dropout in eval mode / p = 0)
    and the mask is None or a float [T, T]."""
    import torch
    import torch.nn as nn
    from rac_amd import rac_torch as rt

    torch.manual_seed(1)
    lq, lk, lv, lo = (nn.Linear(32, 32) for _ in range(4))
    attn = rt.RACAttention.from_attention_layers(lq, lk, lv, lo, n_heads=4)
    w = attn.qkv.weight.detach()
    assert torch.equal(w[:32], lq.weight) and torch.equal(w[32:64], lk.weight) and torch.equal(w[64:], lv.weight)
    b = attn.qkv.bias.detach()
    assert torch.equal(b[:32], lq.bias) and torch.equal(b[32:64], lk.bias) and torch.equal(b[64:], lv.bias)
    assert torch.equal(attn.out_proj.weight, lo.weight) and torch.equal(attn.out_proj.bias, lo.bias)
    assert attn.n_heads == 4 and attn.d_head == 8
    nb = rt.RACAttention.from_attention_layers(*(nn.Linear(32, 32, bias=False) for _ in range(4)), n_heads=2)
    assert nb.qkv.bias is None and nb.out_proj.bias is None
    with pytest.raises(ValueError):
        rt.RACAttention.from_attention_layers(lq, lk, lv, nn.Linear(32, 32, bias=False), n_heads=4)
    with pytest.raises(ValueError):
        rt.RACAttention.from_attention_layers(lq, nn.Linear(32, 16), lv, lo, n_heads=4)
    with pytest.raises(ValueError):
        rt.RACAttention.from_attention_layers(lq, lk, lv, lo, n_heads=5)

    T = 8
    drop = nn.Dropout(0.1)
    assert not rt._rac_core_ok(None, T, drop)
    drop.eval()
    assert rt._rac_core_ok(None, T, drop)
    assert rt._rac_core_ok(None, T, nn.Identity()) and rt._rac_core_ok(None, T, nn.Dropout(0.0))

    class Other(nn.Module):
        def forward(self, x):
            return x

    class SubDropout(nn.Dropout):
        pass

    assert not rt._rac_core_ok(None, T, Other()) and not rt._rac_core_ok(None, T, SubDropout(0.1).eval())
    assert rt._rac_core_ok(torch.zeros(T, T), T, nn.Identity())
    assert not rt._rac_core_ok(torch.zeros(1, 1, T, T), T, nn.Identity())
    assert not rt._rac_core_ok(torch.ones(T, T, dtype=torch.bool), T, nn.Identity())


def test_startup_probe_diagnoses_each_stage():
    """The import-time probe (rac_torch.py:55-108) names its failure: a
    missing library is "not built" (and rac_torch still imports, with that
    warning), a non-gfx950 device is "no gfx950 code", no device is
    reported without a warning; ops then raise with the diagnosis."""
    import sys
    import types
    code = ("import warnings, rac_amd._lib as L\n"
            "L.LIB_PATH = '/nonexistent/librac_amd.so'\n"
            "warnings.simplefilter('always')\n"
            "with warnings.catch_warnings(record=True) as w:\n"
            "    import rac_amd.rac_torch as rt\n"
            "print('STAGE', rt._PROBE.stage)\n"
            "print('WARN', ' | '.join(str(x.message) for x in w))\n")
    env = dict(os.environ, PYTHONPATH=ROOT)
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, cwd=ROOT,
                         timeout=300)
    assert out.returncode == 0, out.stderr[-2000:]
    assert "STAGE no-library" in out.stdout
    assert "not built" in out.stdout and "/nonexistent/librac_amd.so" in out.stdout

    import torch
    from rac_amd import _probe
    real_avail, real_props, real_cur = torch.cuda.is_available, torch.cuda.get_device_properties, \
        torch.cuda.current_device
    try:
        torch.cuda.is_available = lambda: True
        torch.cuda.current_device = lambda: 0
        torch.cuda.get_device_properties = lambda d: types.SimpleNamespace(gcnArchName="gfx942:sramecc+:xnack-")
        r = _probe.probe()
        assert (r.ok, r.stage) == (False, "arch")
        assert "no gfx950 code for this device" in r.message and "gfx942" in r.message
    finally:
        torch.cuda.is_available, torch.cuda.get_device_properties, torch.cuda.current_device = \
            real_avail, real_props, real_cur
    if not torch.cuda.is_available():
        r = _probe.probe()
        assert (r.ok, r.stage) == (False, "no-device")

def test_attention_workspace_sizes(lib):
    """The attention workspace holds one chunk of query rows (at most 128 MiB
    of scores, or 64 rows of every head), plus 256 bytes for a flag; the
    probability-keeping form holds the whole [B*H, T, T] matrix.  A
    workspace below one row of every head is refused before device work."""
    MiB = 2 ** 20
    assert lib.rac_attention_workspace_bytes(1, 32, 2048) == 128 * MiB + 256      # 512 rows per chunk
    assert lib.rac_attention_workspace_bytes(2, 3, 200) == 4 * 6 * 200 * 200 + 256  # one chunk
    assert lib.rac_attention_workspace_bytes(1, 64, 65536) == 4 * 64 * 64 * 65536 + 256   # floor of 64 rows
    assert lib.rac_attention_probs_workspace_bytes(1, 32, 2048) == 512 * MiB + 256
    assert lib.rac_attention_workspace_bytes(0, 1, 1) == 0
    buf = (ctypes.c_float * 64)()
    a = ctypes.addressof(buf)
    assert lib.rac_attention_ws_dev(a, a, a, None, 1, a, 1, 2, 16, 4, a, 4 * 2 * 16 + 255, 16, 1, None) == -2
    assert b"below" in lib.rac_last_error()
    # the allocation-free form: batch*n_heads*seq = 16777216 (one query row
    # of every head is 64 MiB, past its 64 MiB scratch) is refused before
    # any device work
    lib.rac_clear_error()
    assert lib.rac_attention_noalloc_dev(a, a, a, None, 1, a, 1, 64, 262144, 4, 16, 1, None) == -2
    assert b"16777215" in lib.rac_last_error()


def test_every_device_entry_point_refuses_null_buffers(lib):
    """Every *_dev entry point, called with null buffers and otherwise valid
    sizes, returns an error code and sets the error text, without touching
    the device or crashing (no GPU in this container)."""
    from rac_amd import _lib as L
    args_for = {L._vp: None, L._i: 4, L._l: 4, L._f: 1.0}
    checked = 0
    for name, (res, argtypes) in L._SIGNATURES.items():
        if not name.endswith("_dev") or res is not L._i:
            continue
        lib.rac_clear_error()
        args = []
        for t in argtypes:
            args.append(args_for.get(t, None))
        rc = getattr(lib, name)(*args)
        assert rc < 0, name
        assert lib.rac_last_error() != b"", name
        checked += 1
    assert checked >= 30
