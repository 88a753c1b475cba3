"""Loads librda_gfx950.so (the C ABI declared in include/rda.h) through ctypes.

This replaces the reference's runtime layer (hip_attention.py:11-42): there the kernels are
compiled with hipcc on first use and launched with hipModuleLaunchKernel; here they are built
ahead of time for gfx950 and each operation is one typed C call on torch's current stream.
Nothing falls back: without the library or without a ROCm GPU the first call raises.
"""
import ctypes
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_NAME = "librda_gfx950.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)

_p, _i, _l, _f, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_long, ctypes.c_float, ctypes.c_size_t

# name -> (restype, argtypes); the stream is always the last argument.
SIGNATURES = {
    "rda_version": (_i, []),
    "rda_quant_pack_a": (_i, [_p, _l, _p, _p, _i, _i, _p]),
    "rda_rot_quant_pack_a": (_i, [_p, _l, _p, _p, _i, _i, _i, _p]),
    "rda_situ_rot_quant_pack_a": (_i, [_p, _l, _p, _p, _i, _i, _i, _p]),
    "rda_swiglu_rot_quant_pack_a": (_i, [_p, _p, _p, _p, _i, _i, _i, _p]),
    "rda_gate_rot_quant_pack_a": (_i, [_p, _p, _p, _p, _i, _i, _i, _p]),
    "rda_mod_rot_quant_pack_a": (_i, [_p, _p, _p, _i, _i, _p, _p, _p, _i, _f, _p]),
    "rda_rot_quant_pack_a_i4": (_i, [_p, _l, _p, _p, _i, _i, _i, _p]),
    "rda_gemm": (_i, [_p, _p, _p, _p, _p, _p, _i, _i, _i, _p, _p, _i, _p]),
    "rda_gemm_i4": (_i, [_p, _p, _p, _p, _p, _p, _i, _i, _i, _p]),
    "rda_gemm_w4a8": (_i, [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _p]),
    "rda_rot_quant_pack_a_il": (_i, [_p, _l, _p, _p, _i, _i, _i, _p]),
    "rda_gemm_w4a8_il": (_i, [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _p]),
    "rda_gemm_acc": (_i, [_p, _p, _i, _p, _i, _i, _i, _p]),
    "rda_attn": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _i, _p, _f, _p]),
    "rda_attn_i8_workspace": (_sz, [_i, _i, _i]),
    "rda_pack_k_i8": (_i, [_p, _p, _i, _i, _i, _l, _l, _l, _p]),
    "rda_attn_i8": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _i, _p, _f, _p]),
    "rda_attn_waves": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _i, _p, _f, _i, _p]),
    "rda_attn_i8_waves": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _i, _p, _f, _i, _p]),
    "rda_rotate": (_i, [_p, _p, _i, _i, _p]),
    "rda_gemv_i8": (_i, [_p, _i, _p, _p, _p, _p, _i, _i, _p]),
    "rda_rotate_gemv_i8": (_i, [_p, _i, _p, _p, _p, _p, _p, _i, _i, _p]),
    "rda_gemv_i8_multi": (_i, [_p, _i, _i, _i, _p, _p, _p, _p, _p, _i, _p, _p]),
    "rda_gemv_bf16": (_i, [_p, _p, _p, _i, _i, _p]),
    "rda_attn_decode": (_i, [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _f, _p]),
    "rda_attn_merge": (_i, [_p, _p, _p, _i, _p]),
    "rda_decode_splits": (_i, []),
    "rda_attention_decode_noalloc": (_i, [_p, _p, _p, _p, _p, _i, _i, _i, _i, _f, _p]),
    "rda_calib_mfma_peak": (_i, [_i, _i, _i, _p, _p, _p]),
    "rda_calib_mfma_peak_data": (_i, [_i, _i, _i, _p, _p, _p, _p]),
    "rda_rms_norm_head": (_i, [_p, _p, _p, _i, _i, _i, _i, _l, _l, _l, _f, _p]),
    "rda_rms_norm_row": (_i, [_p, _p, _p, _i, _i, _i, _i, _l, _l, _l, _f, _p]),
    "rda_rms_norm_rope": (_i, [_p, _p, _p, _i, _i, _i, _i, _l, _l, _l, _f, _p, _l, _p]),
}

_lib = None


def check(error):
    """Raises like the reference's check() (hip_attention.py:14-16)."""
    if error != 0:
        raise RuntimeError(f"HIP error {error}")


def declare(lib):
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def _hip_runtimes():
    """Distinct libamdhip64 files mapped into this process."""
    paths = set()
    with open("/proc/self/maps") as f:
        for line in f:
            if "libamdhip64" in line:
                paths.add(os.path.realpath(line.split()[-1]))
    return paths


def load():
    """The library, loaded once. Raises if it is missing or no ROCm GPU is present."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_NAME} is not built: run build.py in {HERE} (or __graft_entry__.build())")
        if not torch.cuda.is_available():
            raise RuntimeError("the gfx950 kernels need a ROCm GPU; none is visible")
        torch.cuda.init()
        lib = declare(ctypes.CDLL(LIB_PATH))
        runtimes = _hip_runtimes()
        if len(runtimes) > 1:
            raise RuntimeError(f"two HIP runtimes in one process: {sorted(runtimes)}")
        _lib = lib
    return _lib


def stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def ptr(t):
    return ctypes.c_void_p(None if t is None else t.data_ptr())


def call(name, *args):
    """Calls an entry point with the current stream appended and checks its status."""
    check(getattr(load(), name)(*args, stream()))


def long_array(values):
    return (ctypes.c_long * len(values))(*values)
