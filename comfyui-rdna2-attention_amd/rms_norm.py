"""fp16 RMSNorm (and the QK-norm + RoPE of a Krea 2 block) on MI355X. Mirrors rms_norm.py of the reference:
same names, signatures, eligibility and fallback (rms_norm.py:1-64)."""
import functools

import torch

from . import _lib
from .hip_attention import Kernels, launch

try:  # The kernel wrappers work without ComfyUI; forward() and patch() need it.
    import comfy.model_management
    from comfy.ldm.krea2.model import RMSNorm
except ImportError:
    comfy = None
    RMSNorm = None

THREADS = 256  # NT in csrc/norm.hip
HEAD_DIM = 128  # rows up to this width use 16 threads each (rms_norm_head)
MAX_DIM = 8192  # 256 threads x 4 chunks x 8 values (rms_norm_row)

kernels = None


def get_kernels():
    global kernels
    if kernels is None:
        kernels = Kernels("rms_norm", ("rms_norm_head", "rms_norm_row", "rms_norm_rope"))
    return kernels


def _weight_fp32(scale, device):
    if comfy is not None:
        return comfy.model_management.cast_to(scale, dtype=torch.float32, device=device)
    return scale.to(device=device, dtype=torch.float32)


def rms_norm(x, weight, eps):
    """x is (B, L, D) or (B, H, L, D) fp16 with a contiguous last dimension, weight (D,) fp32 and zero-centered. Returns contiguous fp16."""
    if not eligible(x) or weight.dtype != torch.float32 or weight.numel() != x.shape[-1] or not weight.is_contiguous():
        raise ValueError("rms_norm takes (B, L, D) or (B, H, L, D) fp16 with a contiguous last dimension (D a multiple of 8, "
                         f"at most {MAX_DIM}) and D contiguous fp32 weights")
    k = get_kernels()
    rows = x if x.ndim == 4 else x.unsqueeze(1)
    B, H, L, D = rows.shape
    sb, sh, sl = rows.stride()[:3]
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    if out.numel() == 0:  # nothing to compute (the kernels reject empty shapes)
        return out
    entry = k.rms_norm_head if D <= HEAD_DIM else k.rms_norm_row
    p = _lib.ptr
    launch(entry, 0, 0, THREADS, [p(x), p(weight), p(out), B, H, L, D, sb, sh, sl, float(eps)])
    return out


def rms_norm_rope(x, heads, module, freqs):
    """x is (B, L, heads * 128) fp16 and freqs (B or 1, 1, L, 64, 2, 2) fp32. Returns (B, heads, L, 128) with QK-norm and rope applied."""
    if x.dim() != 3 or x.dtype != torch.float16 or x.shape[2] != heads * HEAD_DIM or x.stride(2) != 1:
        raise ValueError(f"rms_norm_rope takes x as (B, L, {heads} x {HEAD_DIM}) fp16 with a contiguous last dimension")
    B, L, _ = x.shape
    if (freqs.dtype != torch.float32 or not freqs.is_contiguous() or freqs.shape[0] not in (1, B)
            or freqs.numel() != freqs.shape[0] * L * HEAD_DIM * 2):
        raise ValueError(f"rms_norm_rope takes contiguous fp32 freqs of shape (1 or {B}, 1, {L}, 64, 2, 2)")
    out = torch.empty((B, heads, L, HEAD_DIM), dtype=x.dtype, device=x.device)
    if out.numel() == 0:
        return out
    weight = _weight_fp32(module.scale, x.device)
    if weight.numel() != HEAD_DIM or not weight.is_contiguous():
        raise ValueError(f"rms_norm_rope takes {HEAD_DIM} norm weights")
    batch_stride = L * HEAD_DIM // 2 if freqs.shape[0] > 1 else 0
    p = _lib.ptr
    launch(get_kernels().rms_norm_rope, 0, 0, THREADS, [p(x), p(weight), p(out), B, heads, L, HEAD_DIM, x.stride(0), HEAD_DIM, x.stride(1),
                                                        float(module.eps), p(freqs), batch_stride])
    return out


def eligible(x):
    return x.dtype == torch.float16 and x.ndim in (3, 4) and x.stride(-1) == 1 and x.shape[-1] % 8 == 0 and x.shape[-1] <= MAX_DIM


def forward(module, x):
    if not eligible(x):
        return RMSNorm.forward(module, x)
    return rms_norm(x, _weight_fp32(module.scale, x.device), module.eps)


def patch(model):
    for name, module in model.get_model_object("diffusion_model").named_modules():
        if isinstance(module, RMSNorm):
            model.add_object_patch(f"diffusion_model.{name}.forward", functools.partial(forward, module))
