"""The reference's own torch fallbacks, restated for the host CPU -- TEST AND BENCH INFRASTRUCTURE ONLY.

bench.py's cpu_baseline leg times these on the host cores of the machine that runs each GPU workload; tests/test_cpu_baseline.py
pins each against float64 closed forms. The product (the package comfyui-rdna2-attention_amd) never imports them.

What the reference runs when its kernels do not take a call:

* Linears: the weight dequantized and a float matmul, ``F.linear(x, W.to(dtype) * scale, bias)`` (int8_gemv.py:58-59;
  the int8 GEMM hooks hand ineligible calls to INT8-Fast-ROCM's torch path, int8_gemm.py:96, 121), after the dense
  ConvRot ``x.view(..., K / g, g) @ H / sqrt(g)`` (the plugin's rotate_activation, int8_gemm.py:120). int4 weights are
  unpacked (low nibble = even k, int8_gemm.hip:62, 85) and multiplied by their group scales first.
* Attention: attention_bmm (attention.py:15-43): per chunk of <= 128 MB of scores, baddbmm(beta=0, alpha=scale) ->
  softmax -> bmm.
* RMSNorm: the fp32 cast path of the norm the fused kernel replaces (rms_norm.py:55-58): x.float() * rsqrt(mean(x^2)
  + eps) * (w + 1), back to fp16.
* SwiGLU before the down projection: F.silu(gate).mul_(up) (int8_gemm.py:118, 167), then ConvRot and the per-token
  int8 quantization the plugin's triton path performs (floor(x / s + 1/2), s = absmax / 127).
* Decode attention: fp32 softmax(q K^T scale) V over the cached positions, each KV head shared by H / Hkv query
  heads (the computation flash_attention_decode replaces, int8_gemv.py:101-114).
"""
import math

import torch
import torch.nn.functional as F


def hadamard(group, dtype=torch.float32):
    """The ConvRot matrix of one group, orthonormal: kron(H4, H4, H4, H4) / 16 for 256, kron(H2, H4, H4, H4) / sqrt(128)
    for 128, any power of 4 for the decode rotation."""
    H4 = torch.tensor([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=torch.float64)
    H2 = torch.tensor([[1, 1], [1, -1]], dtype=torch.float64)
    H = torch.ones(1, 1, dtype=torch.float64)
    n = group
    factors = []
    while n % 4 == 0 and n > 1:
        factors.append(H4)
        n //= 4
    if n == 2:
        factors.insert(0, H2)
    elif n != 1:
        raise ValueError(f"no ConvRot matrix of order {group}")
    for f in factors:
        H = torch.kron(H, f)
    return (H / math.sqrt(group)).to(dtype)


def rotate(x, group, H=None):
    """Dense block rotation of the last dimension (the plugin's rotate_activation: a matmul per group)."""
    H = hadamard(group, x.dtype) if H is None else H
    shape = x.shape
    return (x.reshape(-1, shape[-1] // group, group) @ H).reshape(shape)


def quant_rows(x):
    """Per-token int8 quantization: s = max(absmax / 127, 1e-30), q = clamp(floor(x / s + 1/2), -128, 127)."""
    s = (x.abs().amax(-1, keepdim=True) / 127).clamp_min(1e-30)
    return torch.floor(x / s + 0.5).clamp_(-128, 127).to(torch.int8), s.squeeze(-1)


def linear_dequant(x, w, scale, bias=None):
    """int8_gemv.py:58-59: F.linear(x, W.to(x.dtype) * scale, bias) with per-output-channel scales."""
    return F.linear(x, w.to(x.dtype) * scale.to(x.dtype).reshape(-1, 1), bias)


def unpack_int4(packed):
    """(N, K / 2) uint8, low nibble = even k -> int8 (N, K)."""
    lo = (packed & 0xF).to(torch.int16)
    hi = (packed >> 4).to(torch.int16)
    lo = torch.where(lo >= 8, lo - 16, lo)
    hi = torch.where(hi >= 8, hi - 16, hi)
    return torch.stack((lo, hi), -1).reshape(packed.shape[0], -1).to(torch.int8)


def linear_w4_dequant(x, packed, group_scales, scale_group=128, bias=None):
    """int4 weights unpacked and multiplied by their [N, K / scale_group] group scales, then F.linear."""
    w = unpack_int4(packed).to(x.dtype)
    gs = group_scales.to(x.dtype).repeat_interleave(scale_group, dim=1)
    return F.linear(x, w * gs, bias)


def w8a8_linear(x, w, scale, group, H=None):
    """The reference's torch path of a ConvRot int8 linear: rotate, then the dequantized matmul."""
    return linear_dequant(rotate(x, group, H), w, scale)


def w4a8_linear(x, packed, group_scales, group=256, scale_group=128, H=None):
    return linear_w4_dequant(rotate(x, group, H), packed, group_scales, scale_group)


def rms_norm(x, w, eps):
    """rms_norm.py:55-58's fallback: the fp32 cast path, x / sqrt(mean(x^2) + eps) * (w + 1), to x's dtype."""
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * (w.float() + 1)).to(x.dtype)


def swiglu_rot_quant(gate, up, group, H=None):
    """F.silu(gate).mul_(up) (int8_gemm.py:118, 167) in the activations' dtype, ConvRot in fp32, per-token int8."""
    return quant_rows(rotate(F.silu(gate).mul_(up).float(), group, H))


def rot_quant(x, group, H=None):
    return quant_rows(rotate(x.float(), group, H))


def attention_bmm(q, k, v, scale, chunk_bytes=128 * 1024 * 1024):
    """attention_bmm (attention.py:15-43) with torch on the CPU: per chunk of heads, baddbmm(beta=0, alpha=scale) ->
    softmax -> bmm. q/k/v (B, H, L, D); returns (B, H, L, D)."""
    b, heads, q_len, d = q.shape
    k_len = k.shape[2]
    batch = b * heads
    q = q.reshape(batch, q_len, d).contiguous()
    k = k.reshape(batch, k_len, d).contiguous().transpose(1, 2).contiguous()
    v = v.reshape(batch, k_len, -1)
    out = torch.empty((batch, q_len, v.shape[-1]), dtype=q.dtype)
    step = min(batch, max(1, chunk_bytes // (q_len * k_len * q.element_size())))
    scores = torch.empty((step, q_len, k_len), dtype=q.dtype)
    for i in range(0, batch, step):
        s = scores[:min(step, batch - i)]
        torch.baddbmm(s, q[i:i + step], k[i:i + step], beta=0, alpha=scale, out=s)
        torch.softmax(s, -1, out=s)
        torch.bmm(s, v[i:i + step], out=out[i:i + step])
    return out.view(b, heads, q_len, -1)


def attention_decode(q, k, v, length, scale=128 ** -0.5):
    """fp32 GQA decode attention: q (B, 1, H, D), k/v (B, capacity, Hkv, D), the first `length` positions."""
    B, _, H, D = q.shape
    Hkv = k.shape[2]
    kk = k[:, :length].permute(0, 2, 3, 1)  # (B, Hkv, D, L)
    vv = v[:, :length].transpose(1, 2)  # (B, Hkv, L, D)
    qq = q.reshape(B, Hkv, H // Hkv, D)  # query heads h = kv * rep + r share KV head kv
    p = torch.softmax(torch.matmul(qq, kk) * scale, -1)
    return torch.matmul(p, vv).reshape(B, 1, H, D)


def gemv(x, w, scale):
    """int8_gemv.py:58-59 for one token: the whole weight is dequantized on every call."""
    return linear_dequant(x, w, scale)


def decode_layer(x, w, s, kc, vc, length, H, group=256, Hrot=None):
    """One token through a layer's seven ConvRot int8 linears (rotate + dequantized matmul each) and decode
    attention, in the order of bench.py's decode_layer workload. w, s: dicts of int8 weights and fp32 scales."""
    D = x.shape[-1]
    lin = lambda name, t: linear_dequant(rotate(t, group, Hrot), w[name], s[name])  # noqa: E731
    q = lin("q", x)
    lin("k", x)
    lin("v", x)
    o = attention_decode(q.view(1, 1, H, 128), kc, vc, length)
    h = lin("o", o.view(1, 1, D))
    gate = lin("gate", h)
    lin("up", h)
    return lin("down", gate)


def block(x, blk, freqs, group=256, H=None):
    """The Krea 2 block that block_forward fuses (int8_gemm.py:189-226), unfused in fp32 with the reference's torch
    fallbacks for each stage: modulated RMSNorm, four ConvRot int8 linears (dequantized), QK-norm + rope, attention_bmm,
    sigmoid(gate) * attention -> output linear with gated residual, modulated RMSNorm, gate/up linears, SwiGLU, down
    linear with gated residual. blk carries CPU fp32 tensors: weights w_<name> int8, scales s_<name>, norm gains
    (zero-centred) prenorm, postnorm, qnorm, knorm, eps, and mod = six (B, 1, D) modulation rows."""
    B, L, D = x.shape
    heads = D // 128
    pre_s, pre_t, pre_g, post_s, post_t, post_g = blk["mod"]
    lin = lambda name, t: linear_dequant(rotate(t, group, H), blk["w_" + name], blk["s_" + name])  # noqa: E731

    def norm_mod(t, w, s, sh):
        return rms_norm(t, w, blk["eps"]) * (1 + s) + sh

    def qk(t, w):
        t = rms_norm(t.view(B, L, heads, 128).transpose(1, 2), w, blk["eps"])
        pairs = t.reshape(B, heads, L, 64, 1, 2)
        return (freqs * pairs).sum(-1).reshape(B, heads, L, 128)  # [m0 m1; m2 m3] applied to (x0, x1)

    h = norm_mod(x, blk["prenorm"], pre_s, pre_t)
    q, k, v, gate = (lin(n, h) for n in ("q", "k", "v", "gate"))
    o = attention_bmm(qk(q, blk["qnorm"]), qk(k, blk["knorm"]), v.view(B, L, heads, 128).transpose(1, 2), 128 ** -0.5)
    o = o.transpose(1, 2).reshape(B, L, D)
    x = x + pre_g * lin("o", torch.sigmoid(gate) * o)
    h = norm_mod(x, blk["postnorm"], post_s, post_t)
    return x + post_g * lin("down", F.silu(lin("gate_mlp", h)) * lin("up", h))


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), or the platform's processor string."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"
