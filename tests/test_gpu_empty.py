"""Empty inputs: the wrappers return empty outputs of the right shape without launching (the kernels reject empty
shapes with an invalid-argument error)."""
import pytest
import torch

from comfyui_rdna2_attention_amd import hip_attention, int8_gemm, rms_norm
from helpers import int8_weights

pytestmark = pytest.mark.gpu


def test_empty_linears(dev):
    w = int8_weights(64, 256, seed=1).to(dev)
    ws = torch.ones(64, device=dev)
    out = int8_gemm.linear(torch.empty(0, 256, dtype=torch.float16, device=dev), w, ws, None, rotate=True)
    assert out.shape == (0, 64) and out.dtype == torch.float16
    qw = torch.zeros(128, 128, dtype=torch.uint8, device=dev)
    gs = torch.ones(128, 2, dtype=torch.float16, device=dev)
    out = int8_gemm.linear_w4a8(torch.empty(0, 256, dtype=torch.float16, device=dev), qw, gs)
    assert out.shape == (0, 128)


@pytest.mark.parametrize("shape", [(1, 0, 3072), (0, 4, 5, 128), (2, 3, 0, 64)])
def test_empty_rms_norm(dev, shape):
    x = torch.empty(shape, dtype=torch.float16, device=dev)
    out = rms_norm.rms_norm(x, torch.zeros(shape[-1], device=dev), 1e-6)
    assert out.shape == x.shape


def test_empty_rms_norm_rope(dev):
    class Norm:
        scale, eps = torch.zeros(128, device=dev), 1e-6

    x = torch.empty(2, 0, 3 * 128, dtype=torch.float16, device=dev)
    freqs = torch.empty(1, 1, 0, 64, 2, 2, device=dev)
    assert rms_norm.rms_norm_rope(x, 3, Norm(), freqs).shape == (2, 3, 0, 128)


@pytest.mark.parametrize("int8_qk", [False, True])
@pytest.mark.parametrize("B,H,Lq,Lk", [(1, 2, 0, 64), (0, 2, 16, 64)])
def test_empty_attention(dev, B, H, Lq, Lk, int8_qk):
    q = torch.empty(B, H, Lq, 128, dtype=torch.float16, device=dev)
    k = torch.randn(B, H, Lk, 128, device=dev).half()
    out = torch.empty_like(q)
    hip_attention.attention(q, k, k, out, 128 ** -0.5, int8_qk)
    assert out.shape == (B, H, Lq, 128)
