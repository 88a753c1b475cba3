"""The C ABI on the CPU: the library is built, loads, and exports exactly what include/rda.h declares; the ctypes
table of the Python side covers every declaration. No compute call is made (there is no GPU here)."""
import ctypes
import os
import re
import subprocess

import pytest

from conftest import ROOT
from comfyui_rdna2_attention_amd import _lib

HEADER = os.path.join(ROOT, "include", "rda.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(rda_\w+)\s*\(", text))


def exported():
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.split()[-1].startswith("rda_")}


@pytest.fixture(scope="module")
def built():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} is missing: run __graft_entry__.build() first")
    return _lib.LIB_PATH


def test_header_matches_exports(built):
    assert declared() == exported()


def test_ctypes_table_covers_header(built):
    assert set(_lib.SIGNATURES) == declared()


def _params(text):
    """Parameter types of a C parameter list, names dropped: "const float* x, int n" -> ["const float*", "int"]."""
    text = " ".join(text.split())
    if text in ("", "void"):
        return []
    types = []
    for p in text.split(","):
        p = re.sub(r"\s*\*\s*", "* ", p.strip()).strip()
        types.append(re.sub(r"\s+\w+$", "", p).replace("* ", "*").strip())
    return types


def _signatures(text, pattern):
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return {m.group(2): (m.group(1), _params(m.group(3))) for m in re.finditer(pattern, text, flags=re.S)}


def test_definitions_match_header_and_ctypes():
    """Every entry point's definition in csrc/ has the parameter types include/rda.h declares, and the ctypes table
    passes exactly those (a pointer as c_void_p, int, long, float), so a changed signature cannot go unnoticed."""
    decl = _signatures(open(HEADER).read(), r"\b(int|size_t)\s+(rda_\w+)\s*\(([^)]*)\)\s*;")
    csrc = os.path.join(ROOT, "comfyui-rdna2-attention_amd", "csrc")
    defs = {}
    for name in sorted(os.listdir(csrc)):
        if name.endswith(".hip"):
            defs.update(_signatures(open(os.path.join(csrc, name)).read(), r"\b(int|size_t)\s+(rda_\w+)\s*\(([^)]*)\)\s*\{"))
    assert set(decl) == declared() and set(defs) == set(decl)
    ctype = {"int": ctypes.c_int, "long": ctypes.c_long, "float": ctypes.c_float, "size_t": ctypes.c_size_t}
    for name, (ret, params) in decl.items():
        assert defs[name] == (ret, params), f"{name}: header {ret} ({', '.join(params)}) vs definition {defs[name]}"
        res, args = _lib.SIGNATURES[name]
        assert res is ctype[ret], name
        want = [ctypes.c_void_p if t.endswith("*") else ctype[t.replace("const ", "")] for t in params]
        assert list(args) == want, f"{name}: ctypes {args} vs {want}"


def test_library_loads_and_binds(built):
    lib = _lib.declare(ctypes.CDLL(built))
    assert lib.rda_version() == 1
    assert lib.rda_decode_splits() == 32
    assert lib.rda_attn_i8_workspace(1, 24, 4096) == 24 * 4096 * 132


def test_argument_checks_reject_before_any_launch(built):
    """Checks that return RDA_ERR_INVALID before the device is touched (the pointers are never dereferenced): the
    fused rotation's output overlapping its input, rows or outputs not on 16-byte boundaries, the multi-matrix
    GEMV's table limits, and attention layouts that do not exist or do not fit the rows."""
    lib = _lib.declare(ctypes.CDLL(built))
    a = 1 << 20  # a 16-byte aligned address, never read
    K = 4096
    for rotated in (a, a + 4 * K - 16, a - 4 * K + 16):  # the same buffer, overlapping from above and from below
        assert lib.rda_rotate_gemv_i8(a, 256, a, a, None, a, rotated, 64, K, None) == 1
    assert lib.rda_rot_quant_pack_a(a + 2, K, a, a, 4, K, 256, None) == 1  # row 0 misaligned
    assert lib.rda_rot_quant_pack_a(a, K + 4, a, a, 4, K, 256, None) == 1  # pitch not a multiple of 8 values
    assert lib.rda_rot_quant_pack_a(a, K - 8, a, a, 4, K, 256, None) == 1  # rows overlapping
    assert lib.rda_situ_rot_quant_pack_a(a, K, a, a, 4, K, 256, None) == 1  # [hidden | gate] rows of 2K values
    assert lib.rda_swiglu_rot_quant_pack_a(a, a + 8, a, a, 4, K, 256, None) == 1
    assert lib.rda_gemm(a, a, a, a, None, a + 2, 256, 256, 256, None, None, 1, None) == 1  # output misaligned
    assert lib.rda_gemm(a, a, a, a, None, a, 256, 256, 256, a + 8, a, 1, None) == 1  # residual misaligned
    ptrs = (ctypes.c_void_p * 2)(a, a)
    n = (ctypes.c_int * 2)(64, 64)
    assert lib.rda_gemv_i8_multi(a, 0, 256, 0, ptrs, ptrs, None, ptrs, n, K, None, None) == 1  # no matrices
    assert lib.rda_gemv_i8_multi(a, 0, 256, 5, ptrs, ptrs, None, ptrs, n, K, None, None) == 1  # more than 4
    assert lib.rda_gemv_i8_multi(a, 0, 256, 2, ptrs, ptrs, None, ptrs, n, 12288, None, None) == 1  # K past 8192
    assert lib.rda_gemv_i8_multi(a, 1, 256, 2, ptrs, ptrs, None, ptrs, n, K, None, None) == 1  # fp16 x with a rotation
    assert lib.rda_gemv_i8_multi(a, 0, 256, 2, ptrs, ptrs, None, ptrs, n, K, a + 16, None) == 1  # rotation onto x
    strides = _lib.long_array([384 * 128, 384 * 128, 128] * 4)
    for waves, lq in ((5, 384), (8, 384), (12, 383), (12, 32)):  # no such layout; twelve waves need 384 rows per head
        assert lib.rda_attn_waves(a, a, a, a, 1, 1, 1, lq, 64, strides, 0.1, waves, None) == 1
        assert lib.rda_attn_i8_waves(a, a, a, a, 1, 1, 1, lq, 64, strides, 0.1, waves, None) == 1


def test_no_cpu_fallback_without_gpu(monkeypatch):
    """The product path raises when the GPU is missing; it never computes on the CPU."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        _lib.load()


def test_m0_is_only_set_by_the_copies(tmp_path):
    """The global->LDS copy helpers (csrc/common.h) set m0 from asm with the compiler's warning about clobbering a
    reserved register silenced: that is sound only while no other code in the kernels uses m0. Every m0 reference in
    the generated gfx950 code must be the copies' own `s_mov_b32 m0, s<n>`."""
    import shutil
    import importlib.util
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc is not installed")
    spec = importlib.util.spec_from_file_location("rda_build", os.path.join(ROOT, "comfyui-rdna2-attention_amd", "build.py"))
    build = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(build)
    setter = re.compile(r"^s_mov_b32 m0, (s\d+|vcc_lo|vcc_hi)$")
    for src in build.sources():
        asm = tmp_path / (os.path.basename(src) + ".s")
        flags = [f for f in build.HIPFLAGS if f != "-fPIC"] + build.FILE_FLAGS.get(os.path.basename(src), [])
        subprocess.run([hipcc, *flags, "--cuda-device-only", "-S", src, "-o", str(asm)], capture_output=True, check=True)
        code = [line.split(";")[0].strip() for line in asm.read_text().splitlines()]
        code = [line for line in code if line and not line.startswith(".") and not line.endswith(":")]
        for i, line in enumerate(code):
            if re.search(r"\bm0\b", line):
                # an m0 write of a copy helper, directly followed by its copy
                assert setter.match(line) and code[i + 1].startswith("global_load_lds_dword"), \
                    f"{os.path.basename(src)}: m0 used outside the copies: {line!r}, then {code[i + 1]!r}"
