"""The fused Krea 2 block (int8_gemm.block_forward, the reference's int8_gemm.py:189-226) end to end on the GPU.

The block runs through the hooks exactly as ComfyUI would drive it: a stand-in INT8-Fast-ROCM layer whose forward
does ConvRot then triton_int8_linear, with int8_gemm's hooks installed over both. The expected output is the chain
of the oracle's stages -- modulated RMSNorm + rotation + quantization, the GEMM epilogue (with the gated residual),
QK-norm + rope, sigmoid-gate and SwiGLU quantization -- in the order and with the roundings of the reference's fused
path. Attention is the one stage whose kernel is tolerance-tested rather than bit-exact, so the chain runs the
attention kernel on the oracle's own q, k, v: from there on every stage is exact, and the block must agree bit for
bit. (The attention kernel itself is checked against float64 softmax in tests/test_gpu_attention.py.)"""
import numpy as np
import pytest
import torch

import fakes
import oracle
from comfyui_rdna2_attention_amd import hip_attention, int8_gemm
from helpers import assert_same, bits, gen

pytestmark = pytest.mark.gpu


def freqs_for(L, seed):
    ang = torch.randn(1, 1, L, 64, generator=gen(seed))
    return torch.stack([torch.cos(ang), -torch.sin(ang), torch.sin(ang), torch.cos(ang)], -1).reshape(1, 1, L, 64, 2, 2).float()


def oracle_block(blk, x, freqs, attend):
    """The fused block's stages on the oracle; attend(q, k, v) -> (B, H, L, 128) fp16 is the attention stage."""
    B, L, D = x.shape
    M, H = B * L, blk.attn.heads
    pre_s, pre_t, pre_g, post_s, post_t, post_g = blk.mod(None)
    host = lambda t: t.reshape(B, D).cpu().numpy()  # noqa: E731  (one modulation row per batch)

    def lin(a, s, layer, R=None, G=None):
        acc = oracle.gemm_acc(a, layer.weight.cpu().numpy())
        return oracle.gemm_epilogue(acc, s, layer.weight_scale.cpu().numpy(), R=R, G=G, L=L)

    def mod_quant(rows, norm, scale, shift):
        a, s, _ = oracle.rot_quant_rows(rows, act=oracle.ACT_MOD, group=256,
                                        mod=(norm.scale.cpu().numpy(), host(1 + scale), host(shift), L, norm.eps))
        return a, s

    def heads(t):
        return t.reshape(B, L, H, 128).transpose(0, 2, 1, 3)

    xs = x.reshape(M, D).cpu().numpy()
    a, s = mod_quant(xs, blk.prenorm, pre_s, pre_t)
    q, k, v, gate = (lin(a, s, layer) for layer in (blk.attn.wq, blk.attn.wk, blk.attn.wv, blk.attn.gate))
    f = freqs.numpy()
    q = oracle.rms_norm(heads(q), blk.attn.qknorm.qnorm.scale.cpu().numpy(), blk.attn.qknorm.qnorm.eps, freqs=f)
    k = oracle.rms_norm(heads(k), blk.attn.qknorm.knorm.scale.cpu().numpy(), blk.attn.qknorm.knorm.eps, freqs=f)
    o = attend(q, k, np.ascontiguousarray(heads(v)))
    heads_out = np.ascontiguousarray(np.asarray(o, np.float16).transpose(0, 2, 1, 3)).reshape(M, D)
    a, s, _ = oracle.rot_quant_rows(heads_out, act=oracle.ACT_GATE, group=256, u=gate)
    x1 = lin(a, s, blk.attn.wo, R=xs, G=host(pre_g))
    a, s = mod_quant(x1, blk.postnorm, post_s, post_t)
    g, u = lin(a, s, blk.mlp.gate), lin(a, s, blk.mlp.up)
    a, s, _ = oracle.rot_quant_rows(g, act=oracle.ACT_SWIGLU, group=256, u=u)
    return lin(a, s, blk.mlp.down, R=x1, G=host(post_g)).reshape(B, L, D)


@pytest.fixture
def hooked(monkeypatch):
    _, mods = fakes.install(monkeypatch, real=True)
    int8_gemm.enable(True)
    yield mods["fakepack.int8_quant"].Int8TensorwiseOps.Linear
    int8_gemm.enable(False)


@pytest.mark.parametrize("int8_qk", [False, True])
@pytest.mark.parametrize("B,L,D,heads,hidden", [(1, 512, 256, 2, 512), (2, 384, 512, 4, 768)])
def test_block_forward_matches_oracle_chain(dev, hooked, B, L, D, heads, hidden, int8_qk):
    print(f"block_forward B={B} L={L} D={D} heads={heads} hidden={hidden} int8_qk={int8_qk}", flush=True)
    blk = fakes.make_krea2_block(hooked, D, heads, hidden, B, dev, seed=7)
    x = torch.randn(B, L, D, generator=gen(8)).half()
    freqs = freqs_for(L, 9)
    out = int8_gemm.block_forward(blk, int8_qk, x.to(dev), None, freqs.to(dev))
    assert out.shape == (B, L, D) and out.dtype == torch.float16
    assert int8_gemm.shared is None and int8_gemm.residual is None and int8_gemm.swiglu_up is None

    def gpu_attention(q, k, v):
        qt, kt, vt = (torch.from_numpy(np.ascontiguousarray(t)).to(dev) for t in (q, k, v))
        o = torch.empty_like(qt)
        hip_attention.attention(qt, kt, vt, o, 128 ** -0.5, int8_qk)
        return o.cpu().numpy()

    ref = oracle_block(blk, x, freqs, gpu_attention)
    assert_same(bits(out), bits(ref))


@pytest.mark.parametrize("seed", range(6))
def test_block_forward_random_shapes(dev, hooked, seed):
    """Seeded random block shapes, bit for bit against the oracle's chain: B 1 or 2, L with B L >= 512 (the fused path's
    minimum) up to 900 tokens, 2, 4 or 6 heads, an MLP width a multiple of 256 up to 2048; int8 QK^T on odd seeds."""
    rng = np.random.default_rng(8000 + seed)
    B = 2 if seed % 3 == 2 else 1
    L = int(rng.integers(-(-512 // B), 901))
    heads = int(rng.choice([2, 4, 6]))
    D, hidden = heads * 128, 256 * int(rng.integers(1, 9))
    int8_qk = bool(seed % 2)
    print(f"block_forward random seed={seed} B={B} L={L} D={D} heads={heads} hidden={hidden} int8_qk={int8_qk}", flush=True)
    blk = fakes.make_krea2_block(hooked, D, heads, hidden, B, dev, seed=8100 + seed)
    x = torch.randn(B, L, D, generator=gen(8200 + seed)).half()
    freqs = freqs_for(L, 8300 + seed)
    xd, fd = x.to(dev), freqs.to(dev)
    assert int8_gemm._block_fusable(blk, xd, fd, None, None, {}), "the shape must take the fused path"
    out = int8_gemm.block_forward(blk, int8_qk, xd, None, fd)

    def gpu_attention(q, k, v):
        qt, kt, vt = (torch.from_numpy(np.ascontiguousarray(t)).to(dev) for t in (q, k, v))
        o = torch.empty_like(qt)
        hip_attention.attention(qt, kt, vt, o, 128 ** -0.5, int8_qk)
        return o.cpu().numpy()

    assert_same(bits(out), bits(oracle_block(blk, x, freqs, gpu_attention)))
