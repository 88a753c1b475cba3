"""The CPU baselines bench.py times (oracle/cpu_baseline.py, the reference's own torch fallbacks) against float64
closed forms and the oracle, at small sizes: what is timed beside each GPU workload computes what it claims to."""
import numpy as np
import torch

import oracle
from oracle import cpu_baseline as cb

g = torch.Generator().manual_seed(99)


def f64(t):
    return t.double().numpy() if isinstance(t, torch.Tensor) else np.asarray(t, np.float64)


def test_hadamard_is_the_closed_form():
    for group in (256, 128):
        assert np.array_equal(f64(cb.hadamard(group, torch.float64)) * np.sqrt(group), oracle.hadamard_matrix(group).astype(np.float64))
    H = f64(cb.hadamard(4096, torch.float64))
    assert np.allclose(H @ H.T, np.eye(4096), atol=1e-12)


def test_rotate_and_quant_rows():
    x = torch.randn(6, 512, generator=g).half()
    rot = cb.rotate(x.float(), 256)
    ref = (f64(x).reshape(6, 2, 256) @ oracle.hadamard_matrix(256).T / 16).reshape(6, 512)
    assert np.abs(f64(rot) - ref).max() < 1e-5
    # Per-token quantization: identical to the oracle's quantizer on fp16 rows.
    q, s = cb.quant_rows(x.float())
    q_ref, s_ref = oracle.quant_rows(x.numpy())
    assert np.array_equal(q.numpy(), q_ref) and np.array_equal(s.numpy(), s_ref)


def test_linear_dequant_and_int4():
    x = torch.randn(5, 256, generator=g)
    w = torch.randint(-127, 128, (64, 256), generator=g, dtype=torch.int8)
    s = torch.rand(64, generator=g) * 2e-3 + 1e-3
    ref = f64(x) @ (f64(w) * f64(s)[:, None]).T
    assert np.abs(f64(cb.linear_dequant(x, w, s)) - ref).max() < 1e-4
    w4 = torch.randint(-8, 8, (64, 256), generator=g, dtype=torch.int8)
    packed = torch.from_numpy(oracle.pack_int4(w4.numpy()))
    assert torch.equal(cb.unpack_int4(packed), w4)
    gs = (torch.rand(64, 2, generator=g) * 1.5e-2 + 5e-3).half()
    ref = f64(x) @ (f64(w4) * np.repeat(f64(gs), 128, axis=1)).T
    assert np.abs(f64(cb.linear_w4_dequant(x, packed, gs)) - ref).max() < 1e-5


def test_rms_norm_fp32_path():
    x = torch.randn(2, 7, 3072, generator=g).half()
    w = torch.randn(3072, generator=g) * 0.1
    out = cb.rms_norm(x, w, 1e-6)
    ref = oracle.rms_norm_f64(x.numpy(), w.numpy(), 1e-6)
    assert out.dtype == torch.float16
    assert np.all(np.abs(f64(out) - ref) <= np.abs(ref) * 2 ** -10 + 2 ** -24)


def test_swiglu_rot_quant_codes_track_the_oracle():
    gate = (torch.randn(4, 512, generator=g) * 3).half()
    up = torch.randn(4, 512, generator=g).half()
    q, s = cb.swiglu_rot_quant(gate, up, 256)
    q_ref, s_ref, _ = oracle.rot_quant_rows(gate.numpy(), act=oracle.ACT_SWIGLU, u=up.numpy())
    # torch's fp16 silu and fp32 matmul rotation differ from the kernels' roundings only in the last bits.
    assert np.abs(q.numpy().astype(int) - q_ref.astype(int)).max() <= 1
    assert np.allclose(s.numpy(), s_ref, rtol=2e-3)


def test_attention_bmm_and_decode():
    q, k, v = (torch.randn(1, 3, 40, 128, generator=g) for _ in range(3))
    out = cb.attention_bmm(q, k, v, 128 ** -0.5, chunk_bytes=40 * 40 * 4)  # one head per chunk
    assert np.abs(f64(out) - oracle.attention_f64(q.numpy(), k.numpy(), v.numpy(), 128 ** -0.5)).max() < 1e-5
    q = torch.randn(1, 1, 8, 128, generator=g)
    k, v = (torch.randn(1, 50, 2, 128, generator=g) for _ in range(2))
    out = cb.attention_decode(q, k, v, 37)
    assert np.abs(f64(out) - oracle.attention_decode_f64(q.numpy(), k.numpy(), v.numpy(), [37])).max() < 1e-5


def test_block_chain_invariants():
    """With zero residual gates, or zero weights, the block returns its input unchanged; otherwise a finite output."""
    B, L, D, hidden = 1, 64, 256, 512
    blk = {"eps": 1e-6, "prenorm": torch.randn(D, generator=g) * 0.1, "postnorm": torch.randn(D, generator=g) * 0.1,
           "qnorm": torch.randn(128, generator=g) * 0.1, "knorm": torch.randn(128, generator=g) * 0.1}
    for name, (n, k) in {"q": (D, D), "k": (D, D), "v": (D, D), "gate": (D, D), "o": (D, D), "gate_mlp": (hidden, D), "up": (hidden, D),
                         "down": (D, hidden)}.items():
        blk["w_" + name] = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
        blk["s_" + name] = torch.rand(n, generator=g) * 2e-3 + 1e-3
    mods = [torch.randn(B, 1, D, generator=g) * 0.2 for _ in range(6)]
    ang = torch.randn(1, 1, L, 64, generator=g)
    freqs = torch.stack([torch.cos(ang), -torch.sin(ang), torch.sin(ang), torch.cos(ang)], -1).reshape(1, 1, L, 64, 2, 2)
    x = torch.randn(B, L, D, generator=g)
    blk["mod"] = mods
    out = cb.block(x, blk, freqs)
    assert out.shape == x.shape and bool(torch.isfinite(out).all()) and not torch.equal(out, x)
    blk["mod"] = mods[:2] + [torch.zeros(B, 1, D)] + mods[3:5] + [torch.zeros(B, 1, D)]
    assert torch.equal(cb.block(x, blk, freqs), x)


def test_cpu_model_string():
    assert isinstance(cb.cpu_model(), str) and cb.cpu_model()


def test_fp16_legs_compute_the_same_functions():
    """bench.py also times the linears and attention_bmm with fp16 inputs: the same functions, within fp16 rounding."""
    x = torch.randn(5, 256, generator=g)
    w = torch.randint(-127, 128, (64, 256), generator=g, dtype=torch.int8)
    s = torch.rand(64, generator=g) * 2e-3 + 1e-3
    ref = f64(x.half()) @ (f64(w) * f64(s)[:, None]).T
    out = cb.linear_dequant(x.half(), w, s)
    assert out.dtype == torch.float16
    assert np.abs(f64(out) - ref).max() <= 2e-3 * np.abs(ref).max()
    q, k, v = (torch.randn(1, 2, 64, 128, generator=g).half() for _ in range(3))
    out = cb.attention_bmm(q, k, v, 128 ** -0.5)
    assert out.dtype == torch.float16
    ref = oracle.attention_f64(q.numpy(), k.numpy(), v.numpy(), 128 ** -0.5)
    assert np.abs(f64(out) - ref).max() < 5e-3
