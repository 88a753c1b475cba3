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


def test_library_loads_and_binds(built):
    lib = _lib.declare(ctypes.CDLL(built))
    assert lib.rda_version() == 1
    assert lib.rda_decode_splits() == 32
    assert lib.rda_attn_i8_workspace(1, 24, 4096) == 24 * 4096 * 132


def test_no_cpu_fallback_without_gpu(monkeypatch):
    """The product path raises when the GPU is missing; it never computes on the CPU."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        _lib.load()
