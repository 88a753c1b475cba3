"""ComfyUI attention backends: the fused MI355X kernel (fp16, and int8 QK^T) with the chunked bmm path as the
fallback. Mirrors attention.py of the reference: same names, signatures, eligibility and fallbacks
(attention.py:1-65)."""
import torch

from . import hip_attention

try:  # attention_bmm needs ComfyUI only for masks and GQA.
    from comfy.ldm.modules.attention import attention_pytorch
except ImportError:
    attention_pytorch = None

# Scores are computed a few heads at a time so each chunk stays inside the 256 MB Infinity Cache of an MI355X.
BMM_CHUNK_BYTES = 256 * 1024 * 1024


def to_heads(t, b, heads, dim_head):
    return t.reshape(b, -1, heads, dim_head).transpose(1, 2)


def attention_bmm(q, k, v, heads, mask=None, attn_precision=None, skip_reshape=False, skip_output_reshape=False, **kwargs):
    """softmax(q k^T * scale) v with baddbmm / softmax / bmm over chunks of heads (the reference fallback, attention.py:15-43)."""
    if mask is not None or kwargs.get("enable_gqa", False):
        return attention_pytorch(q, k, v, heads, mask=mask, attn_precision=attn_precision, skip_reshape=skip_reshape,
                                 skip_output_reshape=skip_output_reshape, **kwargs)
    b = q.shape[0]
    dim_head = q.shape[-1] if skip_reshape else q.shape[-1] // heads
    if not skip_reshape:
        q, k, v = (to_heads(t, b, heads, dim_head) for t in (q, k, v))
    batch, q_len, k_len = b * heads, q.shape[2], k.shape[2]
    q = q.reshape(batch, q_len, dim_head).contiguous()
    kt = k.reshape(batch, k_len, dim_head).contiguous().transpose(1, 2).contiguous()
    v = v.reshape(batch, k_len, -1)
    out = torch.empty((batch, q_len, v.shape[-1]), dtype=q.dtype, device=q.device)
    step = min(batch, max(1, BMM_CHUNK_BYTES // (q_len * k_len * q.element_size())))
    scores = torch.empty((step, q_len, k_len), dtype=q.dtype, device=q.device)
    scale = kwargs.get("scale", dim_head ** -0.5)
    for i in range(0, batch, step):
        n = min(step, batch - i)
        s = scores[:n]
        torch.baddbmm(s, q[i:i + n], kt[i:i + n], beta=0, alpha=scale, out=s)
        torch.softmax(s, -1, out=s)
        torch.bmm(s, v[i:i + n], out=out[i:i + n])
    out = out.view(b, heads, q_len, -1)
    if skip_output_reshape:
        return out
    return out.transpose(1, 2).reshape(b, q_len, -1)


def _fused_eligible(q, v, heads, mask, skip_reshape, kwargs):
    dim_head = q.shape[-1] if skip_reshape else q.shape[-1] // heads
    return mask is None and not kwargs.get("enable_gqa", False) and dim_head == hip_attention.HEAD_DIM and v.shape[-1] == q.shape[-1] and \
        q.dtype == torch.float16


def attention_hip(q, k, v, heads, mask=None, attn_precision=None, skip_reshape=False, skip_output_reshape=False, int8_qk=False, **kwargs):
    """ComfyUI optimized_attention backend: the fused kernel when eligible (no mask, no GQA flag, head dim 128, fp16),
    attention_bmm otherwise (attention.py:46-61)."""
    if not _fused_eligible(q, v, heads, mask, skip_reshape, kwargs):
        return attention_bmm(q, k, v, heads, mask=mask, attn_precision=attn_precision, skip_reshape=skip_reshape,
                             skip_output_reshape=skip_output_reshape, **kwargs)
    b = q.shape[0]
    dim_head = hip_attention.HEAD_DIM
    if not skip_reshape:
        q, k, v = (to_heads(t, b, heads, dim_head) for t in (q, k, v))
    q_len = q.shape[2]
    q, k, v = (t if t.stride(-1) == 1 else t.contiguous() for t in (q, k, v))
    # (B, L, H, D) storage seen as (B, H, L, D): the kernel writes the layout the caller reshapes to.
    out = torch.empty((b, q_len, heads, dim_head), dtype=q.dtype, device=q.device).transpose(1, 2)
    hip_attention.attention(q, k, v, out, kwargs.get("scale", dim_head ** -0.5), int8_qk)
    if skip_output_reshape:
        return out
    return out.transpose(1, 2).reshape(b, q_len, heads * dim_head)


def attention_hip_int8(*args, **kwargs):
    return attention_hip(*args, int8_qk=True, **kwargs)
