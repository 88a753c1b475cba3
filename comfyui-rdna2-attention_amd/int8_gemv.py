"""Single-token (decode) linears and attention on MI355X for text generation. Mirrors int8_gemv.py of the
reference: same names, signatures, eligibility and fallbacks (int8_gemv.py:1-148).

The int8 GEMV reads the stored int8 weight once per token (HBM-bound), the bf16 GEMV the embedding table for the
logits, and decode attention splits the cached positions of each KV head into SPLITS chunks whose partial
softmaxes are merged by a second launch. The decode launches have a fixed grid and read the cache length on the
device, so a captured HIP graph stays valid as the cache grows.
"""
import contextlib
import ctypes
import functools
import weakref

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
    if x.dtype != torch.float32 or x.numel() % group:
        raise ValueError(f"rotate takes fp32 values in whole groups of {group}, not {x.numel()} of {x.dtype}")
    x = x.contiguous()
    rotated = torch.empty_like(x)
    launch(get_kernels().rotate, x.numel() // group, 1, 256, [_lib.ptr(x), _lib.ptr(rotated), x.numel() // group, group])
    return rotated


def _row(x, K, dtypes, what):
    """x as one contiguous, 16-byte aligned row of K values of one of `dtypes` (the GEMVs read it in 16-byte vectors and
    trust its length), or ValueError."""
    if x.dtype not in dtypes or x.numel() != K:
        raise ValueError(f"{what} takes {K} values of {' or '.join(str(d) for d in dtypes)}, not {x.numel()} of {x.dtype}")
    if not x.is_contiguous() or x.data_ptr() % 16:
        x = x.clone(memory_format=torch.contiguous_format)
    return x


def _weight_args(weight, scale, bias, what):
    """Raises ValueError unless weight is a contiguous int8 (N, K) matrix and scale (and bias, if given) contiguous fp32
    with N values: the kernels read N fp32 scales and biases and whole weight rows."""
    if weight.dim() != 2 or weight.dtype != torch.int8 or not weight.is_contiguous():
        raise ValueError(f"{what} takes a contiguous int8 (N, K) weight")
    N = weight.shape[0]
    for name, t in (("scale", scale), ("bias", bias)):
        if t is not None and (t.dtype != torch.float32 or t.numel() != N or not t.is_contiguous()):
            raise ValueError(f"{what}: {name} must be contiguous fp32 with {N} values")


def gemv(x, weight, scale, bias=None):
    """out[n] = scale[n] * dot(weight[n], x) (+ bias[n]) for one row x (K values, fp32 or fp16; the output has its dtype),
    weight (N, K) int8, scale (N,) fp32, bias (N,) fp32 or None."""
    _weight_args(weight, scale, bias, "gemv")
    N, K = weight.shape
    x = _row(x, K, (torch.float32, torch.float16), "gemv")
    out = torch.empty((*x.shape[:-1], N), dtype=x.dtype, device=x.device)
    p = _lib.ptr
    launch(get_kernels().gemv_i8, N // BLOCK_ROWS, 1, 256, [p(x), int(x.dtype == torch.float16), p(weight), p(scale), p(bias), p(out), N, K])
    return out


def _rotated_buffer(rotated, K):
    if rotated is not None and (rotated.dtype != torch.float32 or rotated.numel() != K or not rotated.is_contiguous()):
        raise ValueError(f"rotated must be a contiguous fp32 tensor of {K} values")
    return rotated


def rotate_gemv(x, group, weight, scale, bias=None, rotated=None):
    """gemv(rotate(x, group), weight, scale, bias) as one launch, bit for bit: fp32 x of K values, the ConvRot of its
    K / group groups done by each workgroup of the GEMV in LDS; group one of FUSED_ROTATION_GROUPS. rotated (fp32,
    K values, not overlapping x, or None) receives rotate(x, group) as well. Returns fp32 (..., N)."""
    if group not in FUSED_ROTATION_GROUPS:
        raise ValueError(f"rotate_gemv rotates groups of {FUSED_ROTATION_GROUPS}, not {group}")
    _weight_args(weight, scale, bias, "rotate_gemv")
    N, K = weight.shape
    x = _row(x, K, (torch.float32,), "rotate_gemv")
    rotated = _rotated_buffer(rotated, K)
    out = torch.empty((*x.shape[:-1], N), dtype=torch.float32, device=x.device)
    p = _lib.ptr
    launch(get_kernels().rotate_gemv_i8, N // BLOCK_ROWS, 1, 256, [p(x), group, p(weight), p(scale), p(bias), p(out), p(rotated), N, K])
    return out


MULTI_MAX = 4  # matrices per gemv_multi launch
MULTI_MAX_K = 8192


def gemv_multi(x, layers, group=0, rotated=None):
    """[gemv(x, w, s, b) for w, s, b in layers] (group 0), or [rotate_gemv(x, group, w, s, b) ...] (group one of
    FUSED_ROTATION_GROUPS, fp32 x), as one launch and bit for bit the same outputs: 1-4 weights (N_i, K) int8 over
    one row x of K <= 8192 values. rotated as in rotate_gemv."""
    if not 1 <= len(layers) <= MULTI_MAX:
        raise ValueError(f"gemv_multi takes 1 to {MULTI_MAX} weights, not {len(layers)}")
    K = layers[0][0].shape[1]
    if group and group not in FUSED_ROTATION_GROUPS:
        raise ValueError(f"gemv_multi rotates groups of {FUSED_ROTATION_GROUPS}, not {group}")
    x = _row(x, K, (torch.float32,) if group else (torch.float32, torch.float16), "gemv_multi")
    rotated = _rotated_buffer(rotated, K)
    outs, n = [], []
    for w, s, b in layers:
        _weight_args(w, s, b, "gemv_multi")
        if w.shape[1] != K:
            raise ValueError("gemv_multi weights share one K")
        outs.append(torch.empty((*x.shape[:-1], w.shape[0]), dtype=x.dtype, device=x.device))
        n.append(w.shape[0])
    c = len(layers)
    ptrs = lambda ts: (ctypes.c_void_p * c)(*[None if t is None else t.data_ptr() for t in ts])  # noqa: E731
    biases = [b for _, _, b in layers]
    bias_table = ptrs(biases) if any(b is not None for b in biases) else None
    _lib.call("rda_gemv_i8_multi", _lib.ptr(x), int(x.dtype == torch.float16), group, c, ptrs([w for w, _, _ in layers]),
              ptrs([s for _, s, _ in layers]), bias_table, ptrs(outs), (ctypes.c_int * c)(*n), K, _lib.ptr(rotated))
    return outs


# Sibling linears: the single-token int8 linears that one parent forward applies to the same input, in a row -- q, k
# and v of an attention layer, gate and up of an MLP (patch() registers them from the module tree). The first of them
# to be called computes all of them with one gemv_multi launch (one ConvRot, one pass over x) and leaves the others'
# outputs here; each is handed out once, to the call of its own module with the same input tensor object at the same
# version (in-place writes bump it) and the same graph-capture state and stream. Any other linear_forward call, a
# mismatch, or a repeated call clears what is left, so that outputs are never stale across calls that do not share
# their input. Inference tensors carry no version counter: for them an in-place write to the input between two
# siblings of one parent forward goes unseen (the parent forwards patched here never write it).
def _ref(obj):
    """A weak reference where the object allows one (modules do), else a strong one."""
    try:
        return weakref.ref(obj)
    except TypeError:
        return lambda: obj


class Siblings:
    def __init__(self, members):
        self.refs = [_ref(m[0]) for m in members]  # modules by reference: a registration does not keep a model alive
        self.shapes = [m[1:] for m in members]  # (N, K, weight_dtype, group)
        self.index = {id(m[0]): i for i, m in enumerate(members)}

    def modules(self):
        return [r() for r in self.refs]


_siblings = {}  # id(module) -> Siblings
_stash = None  # (siblings, x, version, capture key, {member index: output})


def register_siblings(members):
    """Registers linears (module, N, K, weight_dtype, group) that one parent forward calls in a row on one input; they
    must share K, the weight dtype and the ConvRot group, and K must fit one gemv_multi launch."""
    if not 2 <= len(members) <= MULTI_MAX or len({m[2:] for m in members}) != 1 or members[0][2] > MULTI_MAX_K:
        raise ValueError("siblings are 2-4 linears of one K (<= 8192), weight dtype and ConvRot group")
    group = Siblings(list(members))
    for m in members:
        _siblings[id(m[0])] = group


def _siblings_of(module):
    sib = _siblings.get(id(module))
    if sib is not None and sib.modules()[sib.index[id(module)]] is not module:  # a registered module died, its id reused
        del _siblings[id(module)]
        return None
    return sib


def forget_siblings():
    global _stash
    _siblings.clear()
    _stash = None


def _version(x):
    try:
        return x._version
    except RuntimeError:  # inference tensors do not track versions
        return None


def _capture_key(x):
    return (torch.cuda.is_current_stream_capturing(), torch.cuda.current_stream(x.device).cuda_stream) if x.is_cuda else None


def _take_stashed(sib, module, x):
    """The output the first sibling computed for this module and this same input, or None; clears the stash unless
    other siblings still have outputs waiting."""
    global _stash
    st, _stash = _stash, None
    if st is None or sib is None or st[0] is not sib or st[1] is not x or st[2] != _version(x) or st[3] != _capture_key(x):
        return None
    out = st[4].pop(sib.index[id(module)], None)
    if out is not None and st[4]:
        _stash = st
    return out


def _siblings_forward(sib, module, weight_dtype, group, x, x_in):
    """Runs every sibling on x (fp32, one row) in one launch; returns this module's output and stashes the others."""
    global _stash
    with contextlib.ExitStack() as stack:
        layers = []
        for m in sib.modules():
            weight, bias = stack.enter_context(quantized_weight(m, weight_dtype, x))
            layers.append((weight._qdata, weight._params.scale.to(device=x.device), bias))
        outs = gemv_multi(x, layers, group if group in FUSED_ROTATION_GROUPS else 0)
    mine = sib.index[id(module)]
    _stash = (sib, x_in, _version(x_in), _capture_key(x_in), {i: o for i, o in enumerate(outs) if i != mine})
    return outs[mine]


def linear_forward(module, N, K, weight_dtype, group, x, *args, **kwargs):
    """Int8 Linear.forward for text generation (int8_gemv.py:48-64): one token goes to the GEMV (with its registered
    siblings, all in one launch); several tokens of a generate() prefill with a large ConvRot group use a dequantized
    matmul; everything else keeps the layer's forward."""
    single = x.numel() == K
    sib = _siblings_of(module)
    stashed = _take_stashed(sib, module, x)
    if stashed is not None:
        return stashed
    if x.dtype != torch.float32 or patched(module) or not (single or (group > FAST_DEQUANT_GROUP and generating)):
        return type(module).forward(module, x, *args, **kwargs)
    x_in, x = x, x.contiguous()
    fused = single and (not group or (group in FUSED_ROTATION_GROUPS and fuse_rotation(K)))
    if fused and sib is not None and all(m is not None and not patched(m) for m in sib.modules()):
        return _siblings_forward(sib, module, weight_dtype, group, x, x_in)
    with quantized_weight(module, weight_dtype, x) as (weight, bias):
        scale = weight._params.scale.to(device=x.device)
        if single and group in FUSED_ROTATION_GROUPS and fuse_rotation(K):
            return rotate_gemv(x, group, weight._qdata, scale, bias)
        if group:
            x = rotate(x, group)
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
    global generating, _stash
    generating = True
    _stash = None
    try:
        return type(transformer).generate(transformer, *args, **kwargs)
    finally:
        generating = False
        _stash = None


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
    """q is (batch, 1, heads, 128), k and v are (batch, capacity, kv heads, 128) and lengths (batch,) int32, all but lengths fp32.
    Lengths are read on the device (a captured graph stays valid as the cache grows); one past capacity counts as
    capacity."""
    if q.dim() != 4 or k.dim() != 4 or q.shape[1] != 1 or q.shape[3] != HEAD or k.shape[3] != HEAD or v.shape != k.shape:
        raise ValueError("attention_decode takes q (batch, 1, heads, 128) and k, v (batch, capacity, kv heads, 128)")
    batch, _, heads, _ = q.shape
    _, capacity, kv_heads, _ = k.shape
    if (k.shape[0] != batch or kv_heads == 0 or heads % kv_heads or heads // kv_heads not in (1, 2, 4, 8)
            or any(t.dtype != torch.float32 for t in (q, k, v)) or not (k.is_contiguous() and v.is_contiguous())
            or lengths.dtype != torch.int32 or lengths.numel() != batch):
        raise ValueError("attention_decode takes fp32 q and contiguous fp32 k, v of one batch size, 1, 2, 4 or 8 query heads per "
                         "kv head, and int32 lengths, one per batch row")
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


SIBLING_NAMES = (("q_proj", "k_proj", "v_proj"), ("gate_proj", "up_proj"))  # linears a parent forward applies to one input


def _gemv_args(module):
    """(module, N, K, weight dtype, ConvRot group) of an int8 layer, as linear_forward takes them."""
    N, K = module.weight.shape
    params = module.weight._params
    return module, N, K, module.weight.dtype, params.convrot_groupsize if params.convrot else 0


def patch(clip):
    """Single token steps of text generation read int8 and bf16 weights directly instead of dequantizing them on every token
    (int8_gemv.py:129-148). The linears that one parent applies to the same input (SIBLING_NAMES) are registered as
    siblings, so that a token runs them in one GEMV launch."""
    for name, module in clip.patcher.model.named_modules():
        for names in SIBLING_NAMES:
            layers = [getattr(module, n, None) for n in names]
            if all(layer is not None and _int8_gemv_layer(layer) for layer in layers):
                members = [_gemv_args(layer) for layer in layers]
                if len({m[2:] for m in members}) == 1 and members[0][2] <= MULTI_MAX_K:
                    register_siblings(members)
        if _int8_gemv_layer(module):
            module, N, K, dtype, group = _gemv_args(module)
            clip.patcher.add_object_patch(f"{name}.forward", functools.partial(linear_forward, module, N, K, dtype, group))
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
