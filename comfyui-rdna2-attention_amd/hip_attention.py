"""Fused attention for head dim 128 (fp16, and int8 QK^T) on MI355X, plus the launch helpers the
other modules share. Mirrors hip_attention.py of the reference: same names and signatures.

The reference compiles its kernels with hipcc on first use and launches them through
hipModuleLaunchKernel (hip_attention.py:11-42). Here the kernels are built ahead of time into
librda_gfx950.so; ``Kernels`` binds its entry points by the reference's kernel names and
``launch`` calls one on torch's current stream (the library picks the gfx950 grid itself).
"""
import math

import torch

from . import _lib

BLOCK_ROWS = 128  # query rows per workgroup of the attention kernel (QB in csrc/attention.hip)
HEAD_DIM = 128

check = _lib.check


def compile_kernels(name):
    """Builds the whole library ahead of time (every module's kernels live in one .so) and returns its path."""
    from . import build
    return build.build()


class Kernels:
    """The library's entry points for the reference module ``name``, one attribute per kernel name."""

    def __init__(self, name, functions):
        lib = _lib.load()
        self.name = name
        for function in functions:
            setattr(self, function, getattr(lib, "rda_" + function))


def launch(func, grid_x, grid_y, block, args, shared=0):
    """Calls entry point ``func`` with ``args`` on the current stream. The grid, block and LDS size
    of the reference's call are accepted for compatibility; the library sizes its own launch."""
    check(func(*args, _lib.stream()))


kernels = None


def _dma_ready(t):
    """K and V rows reach LDS by 16-byte copies: a 16-byte aligned start and (batch, head, row) strides of 8 values."""
    return t.data_ptr() % 16 == 0 and all(s % 8 == 0 for s in t.stride()[:3])


def attention(q, k, v, out, scale, int8_qk=False):
    """q, k, v, out are (batch, heads, length, 128) fp16 tensors with a contiguous last dimension. k and v may have
    fewer heads than q, which then share them. out is written in place."""
    global kernels
    if kernels is None:
        kernels = Kernels("hip_attention", ("attn", "pack_k_i8", "attn_i8", "attn_i8_workspace"))
    for t in (q, k, v, out):
        if t.dim() != 4 or t.dtype != torch.float16 or t.shape[-1] != HEAD_DIM or t.stride(-1) != 1 or not t.is_cuda:
            raise ValueError("attention expects (B, H, L, 128) fp16 GPU tensors with a contiguous last dimension")
    if out.shape != q.shape or v.shape != k.shape or k.shape[0] != q.shape[0] or k.shape[1] == 0 or q.shape[1] % k.shape[1]:
        raise ValueError("attention expects out shaped as q, v as k, one batch size, and q's heads a multiple of k's")
    b, heads, q_len, _ = q.shape
    _, kv_heads, k_len, _ = k.shape
    if out.numel() == 0:  # nothing to compute (the kernels reject empty shapes)
        return
    k, v = (t if _dma_ready(t) else t.clone(memory_format=torch.contiguous_format) for t in (k, v))
    strides = _lib.long_array([*q.stride()[:3], *k.stride()[:3], *v.stride()[:3], *out.stride()[:3]])
    p = _lib.ptr
    if int8_qk:
        workspace = torch.empty(kernels.attn_i8_workspace(b, kv_heads, k_len), dtype=torch.uint8, device=q.device)
        launch(kernels.pack_k_i8, 0, 0, 0, [p(k), p(workspace), b, kv_heads, k_len, *k.stride()[:3]])
        launch(kernels.attn_i8, 0, 0, 0, [p(q), p(workspace), p(v), p(out), b, heads, kv_heads, q_len, k_len, strides, scale])
    else:
        launch(kernels.attn, 0, 0, 0, [p(q), p(k), p(v), p(out), b, heads, kv_heads, q_len, k_len, strides, scale])


def scale_log2(scale):
    """The exp2-domain factor the kernels use, scale * log2(e)."""
    return scale * math.log2(math.e)
