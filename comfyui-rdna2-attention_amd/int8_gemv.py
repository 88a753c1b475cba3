"""Single-token (decode) linears and attention on MI355X for text generation. Mirrors int8_gemv.py of the
reference: same names, signatures, eligibility and fallbacks (int8_gemv.py:1-148).

The int8 GEMV reads the stored int8 weight once per token (HBM-bound), the bf16 GEMV the embedding table for the
logits, and decode attention splits the cached positions of each KV head into SPLITS chunks whose partial
softmaxes are merged by a second launch. The decode launches have a fixed grid and read the cache length on the
device, so a captured HIP graph stays valid as the cache grows.
"""
import functools

import torch
import torch.nn.functional as F

from . import _lib
from .hip_attention import Kernels, launch

try:  # The kernel wrappers work without ComfyUI; the patches below need it.
    import comfy_kitchen
    import comfy.ops
    from comfy.ops import MixedPrecisionOp
    from comfy.text_encoders.llama import MLP, BaseQwen3, FixedKV
except ImportError:
    comfy_kitchen = comfy = None
    MixedPrecisionOp = MLP = BaseQwen3 = FixedKV = None

BLOCK_ROWS = 16  # patch() eligibility: N a multiple, as in the reference (int8_gemv.py:14, 135); gemv_i8 itself takes any N
STEP = 512  # K must be a multiple: a half step of gemv_i8 (64 lanes x 8 int8)
BF16_STEP = 256  # K granularity of gemv_bf16 (64 lanes x 4 bf16)
SPLITS = 32  # position chunks per KV head in attn_decode (SPLITS in csrc/decode.hip)
GROUPS = 4  # query heads per KV head that patch() requires
HEAD = 128
FAST_DEQUANT_GROUP = 256  # Larger ConvRot groups make kitchen's dequantize fall back to a dense matmul.
FUSED_ROTATION_GROUPS = (4, 16, 64, 256)  # ConvRot groups that rotate_gemv rotates inside the GEMV's launch


def fuse_rotation(K):
    """Whether linear_forward rotates inside the GEMV launch for rows of K values: up to 8192, and past it when K is a
    multiple of 1024 (16-wave workgroups). Rows past 8192 with a half step of 512 keep 8-wave workgroups whose registers
    leave one per CU, slower than rotate then GEMV."""
    return K <= 8192 or K % 1024 == 0

kernels = None
# True inside generate(): prompt encoding keeps core's exact rounding, since it decides the image.
generating = False


def get_kernels():
    global kernels
    if kernels is None:
        kernels = Kernels("int8_gemv", ("rotate", "gemv_i8", "rotate_gemv_i8", "gemv_bf16", "attn_decode", "attn_merge"))
    return kernels


def patched(module):
    return module.weight_function or module.bias_function or getattr(module, "weight_lowvram_function", None) is not None


def quantized_weight(module, weight_dtype, x):
    return comfy.ops.CastBiasWeightContext(module, input=None, dtype=weight_dtype, device=x.device, bias_dtype=x.dtype, offloadable=True,
                                          compute_dtype=x.dtype, want_requant=True)


def rotate(x, group):
    """ConvRot of every `group` values of fp32 x (group a power of 4), scaled by 1 / sqrt(group)."""
    rotated = torch.empty_like(x)
    launch(get_kernels().rotate, x.numel() // group, 1, 256, [_lib.ptr(x), _lib.ptr(rotated), x.numel() // group, group])
    return rotated


# The ConvRot of the last single-token input. Consecutive linears that read the same activation -- q, k and v of an
# attention layer, gate and up of an MLP -- rotate it once. An entry is reused only for the same tensor object (held
# here, so its memory cannot be handed to another tensor meanwhile), at the same version counter (in-place writes
# bump it; inference tensors have none, and are matched by object alone), the same group, and the same graph-capture
# state (a rotation launched outside a capture is never read inside one, nor the reverse).
_last_rotation = None


def _version(x):
    try:
        return x._version
    except RuntimeError:  # inference tensors do not track versions
        return None


def _capturing(x):
    return x.is_cuda and torch.cuda.is_current_stream_capturing()


def cached_rotation(x, group):
    """The rotation remembered for this same input x and group, or None."""
    hit = _last_rotation
    if hit is not None and hit[0] is x and hit[1] == _version(x) and hit[2] == group and hit[3] == _capturing(x):
        return hit[4]
    return None


def remember_rotation(x, group, rotated):
    global _last_rotation
    _last_rotation = (x, _version(x), group, _capturing(x), rotated)


def rotate_once(x, group):
    """rotate(x, group), or the rotation of the previous call when it had this same input."""
    rotated = cached_rotation(x, group)
    if rotated is None:
        rotated = rotate(x, group)
        remember_rotation(x, group, rotated)
    return rotated


def forget_rotation():
    global _last_rotation
    _last_rotation = None


def gemv(x, weight, scale, bias=None):
    """out[n] = scale[n] * dot(weight[n], x) (+ bias[n]) for one row x (K values, fp32 or fp16; the output has its dtype),
    weight (N, K) int8, scale (N,) fp32, bias (N,) fp32 or None."""
    if x.data_ptr() % 16:  # the kernels read x in 16-byte vectors
        x = x.clone()
    N, K = weight.shape
    out = torch.empty((*x.shape[:-1], N), dtype=x.dtype, device=x.device)
    p = _lib.ptr
    launch(get_kernels().gemv_i8, N // BLOCK_ROWS, 1, 256, [p(x), int(x.dtype == torch.float16), p(weight), p(scale), p(bias), p(out), N, K])
    return out


def rotate_gemv(x, group, weight, scale, bias=None, rotated=None):
    """gemv(rotate(x, group), weight, scale, bias) as one launch, bit for bit: fp32 x of K values (contiguous), the
    ConvRot of its K / group groups done by each workgroup of the GEMV in LDS; group one of FUSED_ROTATION_GROUPS.
    rotated (fp32, K values, or None) receives rotate(x, group) as well. Returns fp32 (..., N)."""
    if group not in FUSED_ROTATION_GROUPS:
        raise ValueError(f"rotate_gemv rotates groups of {FUSED_ROTATION_GROUPS}, not {group}")
    if x.data_ptr() % 16:  # the kernel reads x in 16-byte vectors
        x = x.clone()
    N, K = weight.shape
    out = torch.empty((*x.shape[:-1], N), dtype=torch.float32, device=x.device)
    p = _lib.ptr
    launch(get_kernels().rotate_gemv_i8, N // BLOCK_ROWS, 1, 256, [p(x), group, p(weight), p(scale), p(bias), p(out), p(rotated), N, K])
    return out


def linear_forward(module, N, K, weight_dtype, group, x, *args, **kwargs):
    """Int8 Linear.forward for text generation (int8_gemv.py:48-64): one token goes to the GEMV; several tokens of a
    generate() prefill with a large ConvRot group use a dequantized matmul; everything else keeps the layer's forward."""
    single = x.numel() == K
    if x.dtype != torch.float32 or patched(module) or not (single or (group > FAST_DEQUANT_GROUP and generating)):
        return type(module).forward(module, x, *args, **kwargs)
    x = x.contiguous()
    with quantized_weight(module, weight_dtype, x) as (weight, bias):
        scale = weight._params.scale.to(device=x.device)
        if group:
            rotated = cached_rotation(x, group)
            if rotated is None and single and group in FUSED_ROTATION_GROUPS and fuse_rotation(K):
                # the first linear of this input rotates it inside its GEMV launch and keeps the rotation for the next
                rotated = torch.empty_like(x)
                out = rotate_gemv(x, group, weight._qdata, scale, bias, rotated)
                remember_rotation(x, group, rotated)
                return out
            x = rotate_once(x, group) if rotated is None else rotated
        if not single:
            return F.linear(x, weight._qdata.to(x.dtype) * scale, bias)
        return gemv(x, weight._qdata, scale, bias)


def mlp_forward(module, weight_dtype, x, norm=None):
    """MLP.forward for a generate() prefill: gate and up dequantized into one matmul (int8_gemv.py:67-75)."""
    if not generating or norm is not None or x.dtype != torch.float32 or x.numel() == x.shape[-1] or patched(module.gate_proj) or patched(module.up_proj):
        return type(module).forward(module, x, norm)
    with quantized_weight(module.gate_proj, weight_dtype, x) as (gate, _), quantized_weight(module.up_proj, weight_dtype, x) as (up, _):
        merged = torch.cat((gate.to(dtype=x.dtype).dequantize(), up.to(dtype=x.dtype).dequantize()))
    gate, up = F.linear(x, merged).chunk(2, dim=-1)
    return module.down_proj(module.activation(gate) * up)


def generate(transformer, *args, **kwargs):
    global generating
    generating = True
    forget_rotation()
    try:
        return type(transformer).generate(transformer, *args, **kwargs)
    finally:
        generating = False
        forget_rotation()


def logits_gemv(x, weight):
    """fp32 logits (1, 1, N) of the last position of x (fp32) against a bf16 (N, K) table."""
    N, K = weight.shape
    out = torch.empty((1, 1, N), dtype=torch.float32, device=x.device)
    launch(get_kernels().gemv_bf16, N // BLOCK_ROWS, 1, 256, [_lib.ptr(x), _lib.ptr(weight), _lib.ptr(out), N, K])
    return out


def logits(transformer, x):
    embed = transformer.model.embed_tokens
    if x.shape[0] != 1 or x.dtype != torch.float32 or embed.weight_function or getattr(embed, "weight_lowvram_function", None) is not None:
        return type(transformer).logits(transformer, x)
    last = x[:, -1:].contiguous()
    with comfy.ops.CastBiasWeightContext(embed, input=None, dtype=torch.bfloat16, device=x.device, offloadable=True) as (weight, _):
        return logits_gemv(last, weight)


def attention_decode(q, k, v, lengths):
    """q is (batch, 1, heads, 128), k and v are (batch, capacity, kv heads, 128) and lengths (batch,) int32, all but lengths fp32."""
    batch, _, heads, _ = q.shape
    _, capacity, kv_heads, _ = k.shape
    k_ = get_kernels()
    q = q.contiguous()
    out = torch.empty_like(q)
    partial = torch.empty((batch * heads, SPLITS, HEAD), dtype=torch.float32, device=q.device)
    stats = torch.empty((batch * heads, SPLITS, 2), dtype=torch.float32, device=q.device)
    p = _lib.ptr
    launch(k_.attn_decode, SPLITS, batch * kv_heads, 256, [p(q), p(k), p(v), p(lengths), p(partial), p(stats), batch, heads, kv_heads, capacity,
                                                          HEAD ** -0.5])
    launch(k_.attn_merge, batch * heads, 1, HEAD, [p(partial), p(stats), p(out), batch * heads])
    return out


def init_kv_cache(model, batch, capacity, device, dtype):
    """A fixed-capacity cache (FixedKV) lets core replay each layer from a graph (int8_gemv.py:117-126)."""
    config = model.config
    position = torch.empty((batch,), device=device, dtype=torch.int64)
    length = torch.zeros((batch,), device=device, dtype=torch.int32)
    caches = []
    for _ in range(config.num_hidden_layers):
        key = torch.empty((batch, capacity, config.num_key_value_heads, HEAD), device=device, dtype=dtype)
        caches.append(FixedKV(key, torch.empty_like(key), 0, position, length))
    return caches


def _int8_gemv_layer(module):
    if not (isinstance(module, MixedPrecisionOp) and type(module).__name__ == "Linear" and module.quant_format == "int8_tensorwise"):
        return False
    N, K = module.weight.shape
    params = module.weight._params
    return N % BLOCK_ROWS == 0 and K % STEP == 0 and params.scale.numel() == N and params.scale.dtype == torch.float32 and not params.transposed


def patch(clip):
    """Single token steps of text generation read int8 and bf16 weights directly instead of dequantizing them on every token
    (int8_gemv.py:129-148)."""
    for name, module in clip.patcher.model.named_modules():
        if _int8_gemv_layer(module):
            N, K = module.weight.shape
            params = module.weight._params
            group = params.convrot_groupsize if params.convrot else 0
            clip.patcher.add_object_patch(f"{name}.forward", functools.partial(linear_forward, module, N, K, module.weight.dtype, group))
        elif (isinstance(module, MLP) and not module.merged_mlp and getattr(module.gate_proj, "quant_format", None) == "int8_tensorwise"
              and module.up_proj.quant_format == "int8_tensorwise"):
            clip.patcher.add_object_patch(f"{name}.forward", functools.partial(mlp_forward, module, module.gate_proj.weight.dtype))
        elif isinstance(module, BaseQwen3) and not module.model.config.lm_head:
            embed = module.model.embed_tokens
            if embed.weight.dtype == torch.bfloat16 and embed.weight.shape[0] % BLOCK_ROWS == 0 and embed.weight.shape[1] % BF16_STEP == 0:
                clip.patcher.add_object_patch(f"{name}.logits", functools.partial(logits, module))
            clip.patcher.add_object_patch(f"{name}.generate", functools.partial(generate, module))
            config = module.model.config
            if module.model.fixed_kv and config.head_dim == HEAD and config.num_attention_heads == config.num_key_value_heads * GROUPS:
                comfy_kitchen.flash_attention_decode = attention_decode
                clip.patcher.add_object_patch(f"{name}.model.init_kv_cache", functools.partial(init_kv_cache, module.model))
