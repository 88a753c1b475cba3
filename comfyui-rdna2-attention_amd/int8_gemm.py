"""W8A8 / W4 linears on MI355X int8 matrix cores, and the hooks that route ComfyUI-INT8-Fast-ROCM's linears
through them. Mirrors int8_gemm.py of the reference: same names, signatures, module globals, eligibility
checks and fallbacks (int8_gemm.py:1-271).

A linear is two launches: the activation -> ConvRot rotation -> per-token int8 pass
(``*_rot_quant_pack_a``), then the GEMM with the dequantizing epilogue. The GEMM reads the (N, K) weight
in place, so the reference's per-call weight re-layout (pack_b, int8_gemm.hip:270) is gone.
"""
import functools
import logging
import sys

import torch
import torch.nn.functional as F

from . import _lib, hip_attention, rms_norm
from .hip_attention import Kernels, launch

try:  # The kernel wrappers work without ComfyUI; the hooks below need it.
    import comfy.model_management
    import comfy.ops
    from comfy.ldm.krea2.model import SingleStreamBlock, SwiGLU
except ImportError:
    comfy = None
    SingleStreamBlock = SwiGLU = None

BLOCK_ROWS = 256  # rows of the GEMM's tallest tile (BM in csrc/gemm.hip); activation buffers are padded to it
ROT_THREADS = 256  # threads per row of the rotate-quant pass (QT in csrc/quant.hip)
MIN_ROWS = 512  # Below this a GEMV-shaped call is better served by the original path.
MAX_ROT_K = 16384  # Keeps the rotated row within the LDS of a workgroup.
ROT_GROUP = 256

KERNELS = ("quant_pack_a", "rot_quant_pack_a", "situ_rot_quant_pack_a", "swiglu_rot_quant_pack_a", "gate_rot_quant_pack_a", "mod_rot_quant_pack_a",
           "rot_quant_pack_a_i4", "gemm", "gemm_i4", "gemm_w4a8", "gemm_acc", "rot_quant_pack_a_il", "gemm_w4a8_il")

kernels = None
# The functions and classes the hooks replace, saved the first time enable() runs.
originals = {}
# Side channel between the hooks (the hooked code calls them one after another on one thread):
fusable = False         # the Int8 Linear now running has no dynamic LoRA, so its ConvRot may move into the kernel
pending = None          # the activation whose ConvRot was deferred; the next int8 linear rotates it itself
situ_next = False       # the next int8 linear receives [hidden | gate] of a situ activation
swiglu_up = None        # the next int8 linear receives a SwiGLU gate; this is its up projection
sigmoid_gate = None     # the next int8 linear receives an attention output; this is its raw sigmoid gate
shared = None           # (packed activations, scales) every input linear of a fused block reads
residual = None         # (x, gate): the next int8 linear returns x + gate * y
swiglu_fusable = False  # INT8-Fast-ROCM's Triton path is live, the only route by which Int8 layers reach wrap()


def get_kernels():
    global kernels
    if kernels is None:
        kernels = Kernels("int8_gemm", KERNELS)
    return kernels


def quantized(M, row_bytes, device):
    """(int8 activations [M, row_bytes] as int32 words, padded to BLOCK_ROWS rows; fp32 scales [M])."""
    blocks = (M + BLOCK_ROWS - 1) // BLOCK_ROWS
    return (torch.empty(blocks * BLOCK_ROWS * row_bytes // 4, dtype=torch.int32, device=device),
            torch.empty(M, dtype=torch.float32, device=device))


def _rows(x):
    """x as rows the quantization kernels can address by a row pitch: contiguous last dimension, rows not overlapping,
    and every row starting on a 16-byte boundary (the kernels read rows in 16-byte vectors)."""
    if x.stride(-1) != 1 or (x.shape[0] > 1 and (x.stride(0) < x.shape[1] or x.stride(0) % 8)) or x.data_ptr() % 16:
        return x.clone(memory_format=torch.contiguous_format)
    return x


def _dense(x):
    """x contiguous and 16-byte aligned (a contiguous view at an odd offset is copied)."""
    if not x.is_contiguous() or x.data_ptr() % 16:
        return x.clone(memory_format=torch.contiguous_format)
    return x


def quantize(quant, x, K, up=None, group=ROT_GROUP):
    """Runs one activation -> rotate -> quantize entry point. x is (M, K) fp16, or (M, 2K) for situ; any strides
    (layouts the kernels cannot address are copied first). Returns (packed, scales)."""
    k = get_kernels()
    M = x.shape[0]
    packed_a, a_scale = quantized(M, K, x.device)
    p = _lib.ptr
    if quant is k.swiglu_rot_quant_pack_a or quant is k.gate_rot_quant_pack_a:  # both operands at a pitch of K
        x, up = _dense(x), _dense(up)
    else:
        x = _rows(x)
    if quant is k.quant_pack_a:
        launch(quant, M, 1, ROT_THREADS, [p(x), x.stride(0), p(packed_a), p(a_scale), M, K])
    elif quant is k.swiglu_rot_quant_pack_a or quant is k.gate_rot_quant_pack_a:
        launch(quant, M, 1, ROT_THREADS, [p(x), p(up), p(packed_a), p(a_scale), M, K, group])
    else:
        launch(quant, M, 1, ROT_THREADS, [p(x), x.stride(0), p(packed_a), p(a_scale), M, K, group])
    return packed_a, a_scale


def _check_linear(what, x, x_cols, K, weight, weight_dtypes, row_bytes, scales, n_scales, scales_dtype, bias, activations, up=None):
    """Raises ValueError unless the tensors have the shapes, dtypes and layouts the kernels read: x (M, x_cols) fp16 (and
    up, if given, M x K fp16 values); a contiguous weight (N, row_bytes); contiguous scales of n_scales values; bias None or N
    contiguous fp16 values; activations, if given, holding M rows of K codes and M fp32 scales. (The kernels trust
    these sizes.)"""
    if x.dim() != 2 or x.dtype != torch.float16 or x.shape[1] != x_cols:
        raise ValueError(f"{what} takes x as (M, {x_cols}) fp16, not {tuple(x.shape)} {x.dtype}")
    if up is not None and (up.dtype != torch.float16 or up.numel() != x.shape[0] * K):
        raise ValueError(f"{what} takes its second input as {x.shape[0]} x {K} fp16 values, not {tuple(up.shape)} {up.dtype}")
    if weight.dim() != 2 or weight.dtype not in weight_dtypes or weight.shape[1] != row_bytes or not weight.is_contiguous():
        raise ValueError(f"{what} takes a contiguous (N, {row_bytes}) weight of {' or '.join(str(d) for d in weight_dtypes)}")
    N = weight.shape[0]
    if scales.dtype != scales_dtype or scales.numel() != n_scales or not scales.is_contiguous():
        raise ValueError(f"{what}: the weight scales must be {n_scales} contiguous {scales_dtype} values")
    if bias is not None and (bias.dtype != torch.float16 or bias.numel() != N or not bias.is_contiguous()):
        raise ValueError(f"{what}: bias must be {N} contiguous fp16 values")
    if activations is not None:
        packed_a, a_scale = activations
        M = x.shape[0]
        if packed_a.numel() * packed_a.element_size() < M * K or a_scale.dtype != torch.float32 or a_scale.numel() < M:
            raise ValueError(f"{what}: activations must hold {M} rows of {K} codes and {M} fp32 scales")


def run(quant, gemm, x, weight, weight_scale, bias, K, up=None, activations=None, res=None, group=ROT_GROUP):
    """K is the number of values per row. weight is (N, row_bytes) int8 (row_bytes = K, or K / 2 for packed int4)
    and weight_scale (N,) fp32. Returns (M, N) fp16."""
    k = get_kernels()
    int4 = gemm is k.gemm_i4
    _check_linear("run", x, 2 * K if quant is k.situ_rot_quant_pack_a else K, K, weight, (torch.int8, torch.uint8) if int4 else (torch.int8,),
                  K // 2 if int4 else K, weight_scale, weight.shape[0] if weight.dim() == 2 else -1, torch.float32, bias, activations, up)
    return _run(quant, gemm, x, weight, weight_scale, bias, K, up, activations, res, group)


def _run(quant, gemm, x, weight, weight_scale, bias, K, up, activations, res, group):
    """run() on arguments already checked."""
    k = get_kernels()
    M = x.shape[0]
    N = weight.shape[0]
    out = torch.empty((M, N), dtype=torch.float16, device=x.device)
    if out.numel() == 0:  # nothing to compute (the kernels reject empty shapes)
        return out
    packed_a, a_scale = quantize(quant, x, K, up, group) if activations is None else activations
    if res is not None:  # the epilogue reads the residual and its gate in 16-byte vectors
        res = (_dense(res[0]), _dense(res[1]))
    p = _lib.ptr
    if gemm is k.gemm_i4:
        launch(gemm, 0, 0, 0, [p(packed_a), p(weight), p(a_scale), p(weight_scale), p(bias), p(out), M, N, K])
    else:
        launch(gemm, 0, 0, 0, [p(packed_a), p(weight), p(a_scale), p(weight_scale), p(bias), p(out), M, N, K,
                               p(res[0] if res is not None else None), p(res[1] if res is not None else None),
                               res[0].shape[1] if res is not None else 1])
    return out


def linear(x, weight, weight_scale, bias, rotate=False, situ=False, up=None, gate=None, activations=None, res=None, group=ROT_GROUP):
    """x is (M, K) fp16, or (M, 2K) with situ, weight (N, K) int8 and weight_scale (N,) fp32. With up, x is the gate of a SwiGLU.
    With gate, x is multiplied by its sigmoid. Returns (M, N) fp16."""
    K = weight.shape[1] if weight.dim() == 2 else -1
    second = up if gate is None else gate
    _check_linear("linear", x, 2 * K if situ and second is None else K, K, weight, (torch.int8,), K, weight_scale,
                  weight.shape[0] if weight.dim() == 2 else -1, torch.float32, bias, activations, second)
    k = get_kernels()
    quant = (k.gate_rot_quant_pack_a if gate is not None else k.swiglu_rot_quant_pack_a if up is not None else k.situ_rot_quant_pack_a if situ
             else k.rot_quant_pack_a if rotate else k.quant_pack_a)
    return _run(quant, k.gemm, x, weight, weight_scale, bias, K, second, activations, res, group)


def _interleaved(qweight, group_scales, bias, N, K, rotate, scale_group):
    """Whether a W4A8 linear can run on k-interleaved activations (each 8 values of k as their 4 even ones, then their 4
    odd ones: the order in which the GEMM widens packed int4, so it needs no byte interleave). That GEMM is the
    direct-copy kernel only: 128-wide scale groups, K and N multiples of 128, the weight and scales on 16-byte and the
    bias on 8-byte boundaries, and K within the rotated rows a workgroup holds."""
    return (rotate and scale_group == 128 and K % 128 == 0 and N % 128 == 0 and K <= MAX_ROT_K and qweight.data_ptr() % 16 == 0
            and group_scales.data_ptr() % 16 == 0 and (bias is None or bias.data_ptr() % 8 == 0))


def linear_w4a8(x, qweight, group_scales, bias=None, rotate=True, group=ROT_GROUP, scale_group=128, activations=None):
    """W4A8: x (M, K) fp16 is rotated (group-size blocks) and quantized per token to int8; qweight (N, K/2) signed int4,
    two per byte, low nibble first; group_scales (N, K / scale_group) fp16. activations, if given, are x already
    quantized by rot_quant_pack_a (or quant_pack_a) in natural order. Returns (M, N) fp16."""
    if x.dim() != 2 or x.shape[1] % scale_group or x.shape[1] % 2:
        raise ValueError(f"linear_w4a8 takes x as (M, K) with K a multiple of {scale_group} and of 2, not {tuple(x.shape)}")
    M, K = x.shape
    N = qweight.shape[0] if qweight.dim() == 2 else -1
    _check_linear("linear_w4a8", x, K, K, qweight, (torch.int8, torch.uint8), K // 2, group_scales, N * (K // scale_group), torch.float16, bias,
                  activations)
    k = get_kernels()
    if M == 0 or N == 0:
        return torch.empty((M, N), dtype=torch.float16, device=x.device)
    gemm = k.gemm_w4a8
    if activations is None:
        if _interleaved(qweight, group_scales, bias, N, K, rotate, scale_group):
            activations, gemm = quantize(k.rot_quant_pack_a_il, x, K, None, group), k.gemm_w4a8_il
        else:
            activations = quantize(k.rot_quant_pack_a if rotate else k.quant_pack_a, x, K, None, group)
    packed_a, a_scale = activations
    out = torch.empty((M, N), dtype=torch.float16, device=x.device)
    p = _lib.ptr
    launch(gemm, 0, 0, 0, [p(packed_a), p(qweight), p(a_scale), p(group_scales), p(bias), p(out), M, N, K, scale_group])
    return out


def gemm_acc(packed_a, weight, M, K, int4=False):
    """Raw int32 accumulators (M, N) of the quantized activations times weight -- the parity check of the GEMM."""
    N = weight.shape[0]
    acc = torch.empty((M, N), dtype=torch.int32, device=weight.device)
    launch(get_kernels().gemm_acc, 0, 0, 0, [_lib.ptr(packed_a), _lib.ptr(weight), int(int4), _lib.ptr(acc), M, N, K])
    return acc


FUSED_BLOCK_ERROR = "RDNA2 Attention: a fused Krea 2 block reached a layer the int8 kernels can't run."


def _w4a4_eligible(x, qweight, bias, convrot_groupsize, compute_dtype, skip_rotation, x_rot):
    N, row_bytes = qweight.shape
    K = 2 * row_bytes
    if x_rot is not None or skip_rotation:
        return False
    if convrot_groupsize != ROT_GROUP or compute_dtype != torch.float16:
        return False
    if bias is not None and bias.dtype != torch.float16:
        return False
    return x.shape[-1] == K and K <= MAX_ROT_K and K % 128 == 0 and N % 64 == 0 and x.numel() // K >= MIN_ROWS


def wrap_w4a4(original):
    """Replacement for INT8-Fast-ROCM's int4_quant.convrot_w4a4_forward (the reference hook: int8_gemm.py:90-102):
    rotation + int4 activations + int4 x int4 GEMM with per-channel scales in two launches; anything else goes to
    ``original``."""
    def convrot_w4a4_forward(x, qweight, wscales, bias, convrot_groupsize, compute_dtype, skip_rotation=False, qweight_unpacked=None, x_rot=None,
                             orig_shape=None):
        if not _w4a4_eligible(x, qweight, bias, convrot_groupsize, compute_dtype, skip_rotation, x_rot):
            return original(x, qweight, wscales, bias, convrot_groupsize, compute_dtype, skip_rotation, qweight_unpacked, x_rot, orig_shape)
        N, K = qweight.shape[0], 2 * qweight.shape[1]
        k = get_kernels()
        rows = x.reshape(-1, K).to(torch.float16).contiguous()
        y = run(k.rot_quant_pack_a_i4, k.gemm_i4, rows, qweight.contiguous(), wscales.reshape(N).float().contiguous(), bias, K)
        return y.reshape(*x.shape[:-1], N)
    return convrot_w4a4_forward


def _int8_eligible(x, weight, bias, compute_dtype, x_q):
    N, K = weight.shape
    if x_q is not None or x.dtype != torch.float16 or compute_dtype != torch.float16:
        return False
    if bias is not None and bias.dtype != torch.float16:
        return False
    return N % 64 == 0 and K % 64 == 0 and x.numel() // x.shape[-1] >= MIN_ROWS


def _take_side_channel(x):
    """Reads and clears what the preceding hooks left for this linear: (rotate, situ, up, gate, res)."""
    global pending, situ_next, swiglu_up, sigmoid_gate, residual
    state = (x is pending, situ_next, swiglu_up, sigmoid_gate, residual)
    pending, situ_next, swiglu_up, sigmoid_gate, residual = None, False, None, None, None
    return state


def _replay_in_torch(x, rotate, situ, up):
    """The deferred input transforms, applied with the original functions before an ineligible linear."""
    if situ:
        x = originals["eager_input_act"](x, "situ")
    if up is not None:
        x = F.silu(x).mul_(up.reshape(x.shape))
    if rotate:
        H = originals["build_hadamard"](ROT_GROUP, device=x.device, dtype=x.dtype)
        x = originals["rotate_activation"](x, H, ROT_GROUP)
    return x


def wrap(original):
    """Replacement for INT8-Fast-ROCM's triton_int8_linear[_per_row] (the reference hook: int8_gemm.py:105-129)."""
    def int8_linear(x, weight, weight_scale, bias=None, compute_dtype=torch.float16, x_q=None):
        rotate, situ, up, gate, res = _take_side_channel(x)
        if not _int8_eligible(x, weight, bias, compute_dtype, x_q):
            if shared is not None or gate is not None or res is not None:
                raise RuntimeError(FUSED_BLOCK_ERROR)
            return original(_replay_in_torch(x, rotate, situ, up), weight, weight_scale, bias, compute_dtype, x_q)
        N, K = weight.shape
        if isinstance(weight_scale, torch.Tensor) and weight_scale.numel() == N:
            scale = weight_scale.reshape(N).float().contiguous()
        else:
            scale = torch.full((N,), float(weight_scale), dtype=torch.float32, device=x.device)
        rows = x.reshape(-1, x.shape[-1]).contiguous()
        ups = None if up is None else up.reshape(-1, K).contiguous()
        y = linear(rows, weight.contiguous(), scale, bias, rotate, situ, ups, gate, shared, res)
        return y.reshape(*x.shape[:-1], N)
    return int8_linear


def _defer_rotation(x, group_size):
    """Whether this ConvRot can be done by the next int8 linear's quantization pass instead."""
    return (fusable and group_size == ROT_GROUP and x.dtype == torch.float16 and x.dim() == 2 and x.shape[1] % ROT_GROUP == 0
            and x.shape[1] <= MAX_ROT_K)


def rotate_activation(x, H, group_size):
    """Replacement for INT8-Fast-ROCM's convrot.rotate_activation (the reference hook: int8_gemm.py:132-142)."""
    global pending
    if shared is not None:  # a fused block's linears read already rotated, quantized activations
        return x
    if situ_next or swiglu_up is not None or sigmoid_gate is not None or _defer_rotation(x, group_size):
        pending = x
        return x
    return originals["rotate_activation"](x, H, group_size)


def fuse_act(layer, x, K):
    """Whether `layer` is an Int8 ConvRot layer (group 256, no LoRA) whose input activation of width K can be fused into its
    quantization pass (the reference predicate: int8_gemm.py:145-149)."""
    if not (getattr(layer, "_is_quantized", False) and getattr(layer, "_use_convrot", False)) or getattr(layer, "_is_w4a8", False):
        return False
    if getattr(layer, "_convrot_groupsize", 0) != ROT_GROUP or layer.lora_patches or x.dtype != torch.float16:
        return False
    width = layer.in_features
    return K == width and width % ROT_GROUP == 0 and width <= MAX_ROT_K


def linear_input_act(linear, x, input_act, act_weight=None, act_eps=0.0, residual=None, residual_scale=None):
    """Replacement for comfy.ops.linear_input_act: a situ input goes to the kernel raw (int8_gemm.py:152-157)."""
    global situ_next
    if input_act == "situ" and residual is None and fuse_act(linear, x, x.shape[-1] // 2):
        situ_next = True
        return linear(x)
    return originals["linear_input_act"](linear, x, input_act, act_weight, act_eps, residual, residual_scale)


def swiglu_forward(module, x):
    """Krea 2 SwiGLU.forward with silu(gate) * up done inside the down projection's quantization pass
    (int8_gemm.py:160-167). Int4 down layers carry the same flags but are not Int8 layers, so they keep the torch path."""
    global swiglu_up
    gate, up = module.gate(x), module.up(x)
    if swiglu_fusable and isinstance(module.down, originals["layer"]) and fuse_act(module.down, gate, gate.shape[-1]):
        swiglu_up = up
        return module.down(gate)
    return module.down(F.silu(gate).mul_(up))


def patch_swiglu(model):
    for name, module in model.get_model_object("diffusion_model").named_modules():
        if isinstance(module, SwiGLU):
            model.add_object_patch(f"diffusion_model.{name}.forward", functools.partial(swiglu_forward, module))


def quantize_block_input(x, norm, scale, shift):
    """Quantizes (1 + scale) * norm(x) + shift once and publishes it in `shared` for all of a block's input linears
    (int8_gemm.py:176-186)."""
    global shared
    B, L, K = x.shape
    packed_a, a_scale = quantized(B * L, K, x.device)
    x = _dense(x)  # read at a row pitch of K, in 16-byte vectors
    weight = _dense(comfy.model_management.cast_to(norm.scale, dtype=torch.float32, device=x.device))
    s, t = _dense(1 + scale), _dense(shift)
    p = _lib.ptr
    launch(get_kernels().mod_rot_quant_pack_a, B * L, 1, ROT_THREADS,
           [p(x), p(packed_a), p(a_scale), B * L, K, p(weight), p(s), p(t), L, float(norm.eps)])
    shared = packed_a, a_scale


def _block_fusable(module, x, freqs, mask, timestep_zero_index, transformer_options):
    attn, mlp = module.attn, module.mlp
    patches = transformer_options.get("patches", {})
    if not swiglu_fusable or mask is not None or timestep_zero_index is not None or freqs is None:
        return False
    if "attn1_patch" in patches or "attn1_output_patch" in patches:
        return False
    if x.dtype != torch.float16 or x.shape[0] * x.shape[1] < MIN_ROWS or attn.headdim != rms_norm.HEAD_DIM:
        return False
    layers = (attn.wq, attn.wk, attn.wv, attn.gate, attn.wo, mlp.gate, mlp.up, mlp.down)
    return all(isinstance(layer, originals["layer"]) and layer.bias is None and fuse_act(layer, x, layer.in_features) for layer in layers)


def block_forward(module, int8_qk, x, vec, freqs, mask=None, timestep_zero_index=None, transformer_options={}):
    """Krea 2 SingleStreamBlock.forward with everything between the matmuls fused (int8_gemm.py:189-226). Rounds at the same
    points as the unfused fused_norm + fused_swiglu path."""
    global shared, swiglu_up, sigmoid_gate, residual
    if not _block_fusable(module, x, freqs, mask, timestep_zero_index, transformer_options):
        return SingleStreamBlock.forward(module, x, vec, freqs, mask, timestep_zero_index, transformer_options)
    attn, mlp = module.attn, module.mlp
    B, L, D = x.shape
    prescale, preshift, pregate, postscale, postshift, postgate = module.mod(vec)
    try:
        # Attention half: one quantization of the modulated norm feeds q, k, v and the output gate.
        quantize_block_input(x, module.prenorm, prescale, preshift)
        q, k, v, gate = attn.wq(x), attn.wk(x), attn.wv(x), attn.gate(x)
        shared = None
        q = rms_norm.rms_norm_rope(q, attn.heads, attn.qknorm.qnorm, freqs)
        k = rms_norm.rms_norm_rope(k, attn.kvheads, attn.qknorm.knorm, freqs)
        v = v.view(B, L, attn.kvheads, attn.headdim).transpose(1, 2)
        heads_out = torch.empty((B, L, attn.heads, attn.headdim), dtype=x.dtype, device=x.device)
        hip_attention.attention(q, k, v, heads_out.transpose(1, 2), attn.headdim ** -0.5, int8_qk)
        # wo quantizes sigmoid(gate) * attention and adds x + pregate * y in its epilogue.
        sigmoid_gate, residual = gate.view(-1, D), (x, pregate.contiguous())
        x = attn.wo(heads_out.view(B, L, D))
        # MLP half: the same pattern, with SwiGLU folded into down's quantization.
        quantize_block_input(x, module.postnorm, postscale, postshift)
        gate, up = mlp.gate(x), mlp.up(x)
        shared = None
        swiglu_up, residual = up, (x, postgate.contiguous())
        return mlp.down(gate)
    finally:
        # An exception (or an interrupted prompt) must not leak state into the next layer.
        shared = swiglu_up = sigmoid_gate = residual = None


def patch_block(model, int8_qk):
    for name, module in model.get_model_object("diffusion_model").named_modules():
        if isinstance(module, SingleStreamBlock):
            model.add_object_patch(f"diffusion_model.{name}.forward", functools.partial(block_forward, module, int8_qk))


def wrap_forward(forward):
    """Int8 Linear.forward that marks, for its duration, whether the layer's ConvRot may move into the kernel: dynamic LoRA
    reads the rotated activation after the linear, so layers with LoRA patches keep the separate rotation."""
    def int8_forward(self, x):
        global fusable
        fusable = not self.lora_patches
        try:
            return forward(self, x)
        finally:
            fusable = False
    return int8_forward


def _find_module(suffix, attribute):
    return next((m for name, m in list(sys.modules.items()) if name.endswith(suffix) and hasattr(m, attribute)), None)


def enable(on):
    """Installs (on) or removes the hooks into ComfyUI-INT8-Fast-ROCM's modules wherever they are loaded (int8_gemm.py:247-271).
    The originals are saved once, so repeated calls toggle cleanly."""
    global swiglu_fusable
    int4 = _find_module(".int4_quant", "convrot_w4a4_forward")
    if int4 is not None:
        originals.setdefault("convrot_w4a4_forward", int4.convrot_w4a4_forward)
        int4.convrot_w4a4_forward = wrap_w4a4(originals["convrot_w4a4_forward"]) if on else originals["convrot_w4a4_forward"]
    pack = _find_module(".int8_quant", "triton_int8_linear_per_row")
    if pack is None:
        if on:
            logging.warning("RDNA2 Attention: int8_gemm skipped, ComfyUI-INT8-Fast-ROCM is not loaded.")
        return
    convrot = _find_module(".convrot", "rotate_activation")
    layer = pack.Int8TensorwiseOps.Linear
    if "forward" not in originals:
        originals.update(layer=layer, forward=layer.forward, triton_int8_linear=pack.triton_int8_linear,
                         triton_int8_linear_per_row=pack.triton_int8_linear_per_row, rotate_activation=convrot.rotate_activation,
                         build_hadamard=convrot.build_hadamard, linear_input_act=comfy.ops.linear_input_act,
                         eager_input_act=comfy.ops._eager_input_act)
    pick = (lambda hook, name: hook(originals[name])) if on else (lambda hook, name: originals[name])
    pack.triton_int8_linear = pick(wrap, "triton_int8_linear")
    pack.triton_int8_linear_per_row = pick(wrap, "triton_int8_linear_per_row")
    layer.forward = pick(wrap_forward, "forward")
    convrot.rotate_activation = rotate_activation if on else originals["rotate_activation"]
    comfy.ops.linear_input_act = linear_input_act if on else originals["linear_input_act"]
    swiglu_fusable = on and pack._TRITON_AVAILABLE
