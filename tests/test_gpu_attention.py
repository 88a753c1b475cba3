"""Parity of the fused attention (fp16 and int8-QK) on the GPU against the oracle.

fp16 attention has no bit-exact pin (the matrix cores' summation order and the hardware exp2 are not reproducible
on the CPU), so it is held to a stated tolerance against the float64 closed form: |out - ref| <= ATOL + RTOL |ref|
with ATOL = RTOL = 2e-3 (P is rounded to fp16 before PV, 2^-11 relative; the output to fp16). The int8-QK variant is
checked against the closed form of its own quantized scores (the Q/K codes and int32 scores are exact) to the
same tolerance, and its quantized K against the oracle bit for bit."""
import math

import numpy as np
import pytest
import torch

import oracle
from comfyui_rdna2_attention_amd import _lib, attention, hip_attention
from helpers import assert_same, gen

pytestmark = pytest.mark.gpu

ATOL = RTOL = 2e-3


def qkv(B, H, Hkv, Lq, Lk, seed, D=128):
    g = gen(seed)
    q = torch.randn(B, H, Lq, D, generator=g).half()
    k = torch.randn(B, Hkv, Lk, D, generator=g).half()
    v = torch.randn(B, Hkv, Lk, D, generator=g).half()
    return q, k, v


def close(out, ref):
    out = out.detach().cpu().float().numpy().astype(np.float64)
    err = np.abs(out - ref)
    bound = ATOL + RTOL * np.abs(ref)
    assert np.all(err <= bound), f"max abs err {err.max():.3e}, worst excess {(err - bound).max():.3e}"


@pytest.mark.parametrize("int8_qk", [False, True])
# Key tiles of 32: 2, 10, 32, 1, 128, 33, 3, 5, 6 and 7 -- every count of steps the pipelined tile loop takes one at a
# time before its six-step passes (0-5), whole and partial last tiles. Heads of 384 query rows or more also run the
# twelve-wave workgroups (384 rows per workgroup over the (batch, head, row) range, each head's rows padded to a
# multiple of 32), checked bit for bit against the automatic layout: one head with padding rows (513); two whole heads;
# rows spanning heads with GQA 3:1 over two batches and a partial last workgroup; spanning heads with GQA 2:1 and a
# partial last key tile; padded heads spanning workgroups (400, 1000); and 1, 2, 3, 4, 5, 7, 10, 33 and 128 key tiles.
@pytest.mark.parametrize("B,H,Hkv,Lq,Lk", [(1, 2, 2, 128, 64), (1, 2, 2, 300, 300), (2, 4, 1, 77, 1000), (1, 3, 3, 1, 5), (1, 1, 1, 513, 4096),
                                          (1, 2, 1, 200, 1049), (1, 1, 1, 64, 96), (1, 2, 2, 130, 150), (1, 1, 1, 129, 192), (2, 2, 1, 70, 210),
                                          (1, 2, 2, 384, 100), (2, 3, 1, 416, 300), (1, 4, 2, 640, 1049), (1, 3, 3, 400, 300), (2, 2, 1, 1000, 77),
                                          (1, 2, 2, 384, 20), (1, 1, 1, 400, 40), (1, 2, 1, 384, 224), (1, 1, 1, 500, 160)])
def test_attention(dev, B, H, Hkv, Lq, Lk, int8_qk):
    print(f"attention B={B} H={H} Hkv={Hkv} Lq={Lq} Lk={Lk} int8_qk={int8_qk}", flush=True)
    q, k, v = qkv(B, H, Hkv, Lq, Lk, seed=Lq + Lk)
    out = torch.empty(B, H, Lq, 128, dtype=torch.float16, device=dev)
    scale = 128 ** -0.5
    hip_attention.attention(q.to(dev), k.to(dev), v.to(dev), out, scale, int8_qk)
    ref = (oracle.attention_i8qk_f64 if int8_qk else oracle.attention_f64)(q.numpy(), k.numpy(), v.numpy(), scale)
    close(out, ref)
    # Each workgroup layout that fits the shape (the automatic choice is one of them) gives the same bits.
    for waves in (4, 12) if Lq >= 384 else (4,):
        assert torch.equal(attention_layout(q.to(dev), k.to(dev), v.to(dev), scale, int8_qk, waves).view(torch.int16), out.view(torch.int16)), waves


@pytest.mark.parametrize("seed", range(12))
def test_attention_random_shapes_every_layout(dev, seed):
    """Seeded random shapes (batch 1-3, GQA 1:1-4:1, query rows 1-900, keys 1-700, fp16 and int8-QK): the automatic
    layout within the tolerance of the float64 closed form, and every layout that fits the shape bit for bit equal to it."""
    r = np.random.default_rng(1000 + seed)
    B, Hkv, rep = int(r.integers(1, 4)), int(r.integers(1, 4)), int(r.choice([1, 2, 4]))
    H, Lq, Lk, int8_qk = Hkv * rep, int(r.integers(1, 901)), int(r.integers(1, 701)), bool(seed % 2)
    print(f"random attention B={B} H={H} Hkv={Hkv} Lq={Lq} Lk={Lk} int8_qk={int8_qk}", flush=True)
    q, k, v = qkv(B, H, Hkv, Lq, Lk, seed=seed)
    out = torch.empty(B, H, Lq, 128, dtype=torch.float16, device=dev)
    scale = 128 ** -0.5
    hip_attention.attention(q.to(dev), k.to(dev), v.to(dev), out, scale, int8_qk)
    ref = (oracle.attention_i8qk_f64 if int8_qk else oracle.attention_f64)(q.numpy(), k.numpy(), v.numpy(), scale)
    close(out, ref)
    for waves in (4, 12) if Lq >= 384 else (4,):
        assert torch.equal(attention_layout(q.to(dev), k.to(dev), v.to(dev), scale, int8_qk, waves).view(torch.int16), out.view(torch.int16)), waves


def attention_layout(q, k, v, scale, int8_qk, waves):
    """rda_attn_waves / rda_attn_i8_waves: the attention with its workgroup layout fixed (4 or 12 waves)."""
    lib, p = _lib.load(), _lib.ptr
    B, H, Lq, _ = q.shape
    _, Hkv, Lk, _ = k.shape
    out = torch.empty_like(q)
    strides = _lib.long_array([*q.stride()[:3], *k.stride()[:3], *v.stride()[:3], *out.stride()[:3]])
    if int8_qk:
        ws = torch.empty(lib.rda_attn_i8_workspace(B, Hkv, Lk), dtype=torch.uint8, device=q.device)
        _lib.check(lib.rda_pack_k_i8(p(k), p(ws), B, Hkv, Lk, *k.stride()[:3], _lib.stream()))
        _lib.check(lib.rda_attn_i8_waves(p(q), p(ws), p(v), p(out), B, H, Hkv, Lq, Lk, strides, scale, waves, _lib.stream()))
    else:
        _lib.check(lib.rda_attn_waves(p(q), p(k), p(v), p(out), B, H, Hkv, Lq, Lk, strides, scale, waves, _lib.stream()))
    return out


@pytest.mark.parametrize("int8_qk", [False, True])
def test_attention_zero_query_rows(dev, int8_qk):
    """All-zero query rows (the int8 row scale then sits at its 1e-30 floor) with a partial last key tile: the keys past
    Lk must get no weight, so each such row is the mean of the valid V rows."""
    print(f"attention zero query rows int8_qk={int8_qk}", flush=True)
    q, k, v = qkv(1, 2, 2, 70, 150, seed=8)
    q[:, :, ::3] = 0
    out = torch.empty(1, 2, 70, 128, dtype=torch.float16, device=dev)
    hip_attention.attention(q.to(dev), k.to(dev), v.to(dev), out, 128 ** -0.5, int8_qk)
    ref = (oracle.attention_i8qk_f64 if int8_qk else oracle.attention_f64)(q.numpy(), k.numpy(), v.numpy(), 128 ** -0.5)
    close(out, ref)
    mean = v.double().numpy().mean(axis=2)  # (B, H, 128)
    assert np.abs(out[:, :, ::3].cpu().double().numpy() - mean[:, :, None]).max() <= 2e-3


def test_attention_matches_reference_loop(dev):
    """Tighter: the reference's own loop restated in fp32 (wave-voted lazy rescale, fp16 P) agrees with the kernel."""
    q, k, v = qkv(1, 2, 2, 256, 700, seed=3)
    out = torch.empty(1, 2, 256, 128, dtype=torch.float16, device=dev)
    hip_attention.attention(q.to(dev), k.to(dev), v.to(dev), out, 128 ** -0.5)
    ref = oracle.attention_faithful(q.numpy(), k.numpy(), v.numpy(), 128 ** -0.5).astype(np.float64)
    err = np.abs(out.cpu().float().numpy() - ref)
    assert err.max() <= 1e-3


def test_attention_large_scores(dev):
    """Scores far above the lazy-rescale threshold (8 in log2 units): the running maximum must move."""
    q, k, v = qkv(1, 2, 2, 200, 1200, seed=5)
    q = (q.float() * 4).half()
    out = torch.empty(1, 2, 200, 128, dtype=torch.float16, device=dev)
    hip_attention.attention(q.to(dev), k.to(dev), v.to(dev), out, 128 ** -0.5)
    close(out, oracle.attention_f64(q.numpy(), k.numpy(), v.numpy(), 128 ** -0.5))


@pytest.mark.parametrize("int8_qk", [False, True])
def test_attention_rising_scores(dev, int8_qk):
    """Scores that climb along the keys by ~4 (log2 units) per 32-key tile, to ~98 over the row: the running maximum
    moves every two or three tiles, and most tiles' P sums outgrow the fast path's bound, so they take the path that
    recomputes the scores and applies the lazy-rescale rule."""
    B, H, Lq, Lk = 1, 2, 96, 800
    g = gen(21)
    q = (torch.rand(B, H, Lq, 128, generator=g) * 0.5 + 0.5).half()
    ramp = torch.linspace(0.0, 1.0, Lk).view(1, 1, Lk, 1)
    k = (ramp * 8.0 + torch.randn(B, H, Lk, 128, generator=g) * 0.05).half()
    v = torch.randn(B, H, Lk, 128, generator=g).half()
    out = torch.empty(B, H, Lq, 128, dtype=torch.float16, device=dev)
    hip_attention.attention(q.to(dev), k.to(dev), v.to(dev), out, 128 ** -0.5, int8_qk)
    ref = (oracle.attention_i8qk_f64 if int8_qk else oracle.attention_f64)(q.numpy(), k.numpy(), v.numpy(), 128 ** -0.5)
    close(out, ref)


def test_comfy_backend_strided_layout(dev):
    """attention_hip on (B, L, H*D) inputs: the kernel reads the strided (B, H, L, D) views and writes (B, L, H, D)."""
    B, L, H = 1, 640, 3
    g = gen(8)
    q, k, v = (torch.randn(B, L, H * 128, generator=g).half() for _ in range(3))
    out = attention.attention_hip(q.to(dev), k.to(dev), v.to(dev), H)
    th = lambda t: t.reshape(B, L, H, 128).transpose(1, 2).numpy()  # noqa: E731
    ref = oracle.attention_f64(th(q), th(k), th(v), 128 ** -0.5)
    close(out.reshape(B, L, H, 128).transpose(1, 2), ref)
    out8 = attention.attention_hip_int8(q.to(dev), k.to(dev), v.to(dev), H)
    close(out8.reshape(B, L, H, 128).transpose(1, 2), oracle.attention_i8qk_f64(th(q), th(k), th(v), 128 ** -0.5))


@pytest.mark.parametrize("B,Hkv,Lk", [(1, 2, 100), (2, 3, 33), (1, 1, 64), (1, 2, 70), (1, 1, 4101)])
def test_pack_k_i8_bit_exact(dev, B, Hkv, Lk):
    """Every key's codes and scale against the oracle; rows past Lk, up to the padded length (a multiple of the 32-key
    tile), are zero. Lk values end the 64-key workgroups at each kind of boundary."""
    print(f"pack_k_i8 B={B} Hkv={Hkv} Lk={Lk}", flush=True)
    _, k, _ = qkv(B, Hkv, Hkv, 1, Lk, seed=4)
    lib = _lib.load()
    ws = torch.empty(lib.rda_attn_i8_workspace(B, Hkv, Lk), dtype=torch.uint8, device=dev)
    kd = k.to(dev)
    _lib.check(lib.rda_pack_k_i8(_lib.ptr(kd), _lib.ptr(ws), B, Hkv, Lk, *kd.stride()[:3], _lib.stream()))
    pad = (Lk + 31) // 32 * 32
    assert ws.numel() == B * Hkv * pad * (128 + 4)
    k8 = ws[:B * Hkv * pad * 128].view(torch.int8).view(B * Hkv, pad, 128).cpu().numpy()
    ks = ws[B * Hkv * pad * 128:].view(torch.float32).view(B * Hkv, pad).cpu().numpy()
    for bh in range(B * Hkv):
        q_ref, s_ref = oracle.quant_rows_rint(k[bh // Hkv, bh % Hkv].numpy())
        assert_same(k8[bh, :Lk], q_ref)
        assert_same(ks[bh, :Lk], s_ref)
        assert not k8[bh, Lk:].any()


def test_attention_full_size_every_row(dev):
    """The fused-attention configuration at full size (B=1, H=24, S=4096, D=128): every one of the 98,304 query rows
    against a float64 reference computed on the GPU head by head (torch float64 matmuls and softmax), fp16 and
    int8-QK (the latter against the softmax of its own exact quantized scores: codes from the oracle's quantizer, the
    int32 scores exact in float64, scaled in fp32 in the kernel's order). Tolerance as everywhere in this file."""
    B, H, L = 1, 24, 4096
    q, k, v = qkv(B, H, H, L, L, seed=4)
    scale = 128 ** -0.5
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    scale_log2 = np.float32(scale * math.log2(math.e))
    for int8_qk in (False, True):
        print(f"attention full size, every row, int8_qk={int8_qk}", flush=True)
        out = torch.empty(B, H, L, 128, dtype=torch.float16, device=dev)
        hip_attention.attention(qd, kd, vd, out, scale, int8_qk)
        worst = 0.0
        for h in range(H):
            vh = vd[0, h].double()
            if int8_qk:
                q8, qs = oracle.quant_rows_rint(q[0, h].numpy())
                k8, ks = oracle.quant_rows_rint(k[0, h].numpy())
                si = torch.from_numpy(q8).to(dev).double() @ torch.from_numpy(k8).to(dev).double().T  # exact integers
                sc = torch.from_numpy((qs * scale_log2).astype(np.float32)).to(dev)
                s2 = ((si.float() * sc[:, None]) * torch.from_numpy(ks).to(dev)[None, :]).double()
                p = torch.exp2(s2 - s2.max(dim=1, keepdim=True).values)
            else:
                sc = (qd[0, h].double() @ kd[0, h].double().T) * scale
                p = torch.exp(sc - sc.max(dim=1, keepdim=True).values)
            ref = (p @ vh) / p.sum(dim=1, keepdim=True)
            err = (out[0, h].double() - ref).abs()
            excess = (err - (ATOL + RTOL * ref.abs())).max().item()
            worst = max(worst, err.max().item())
            assert excess <= 0, f"head {h}: max abs err {err.max().item():.3e}, worst excess {excess:.3e}"
        print(f"  max abs err over all rows {worst:.3e}", flush=True)


def test_attention_full_size_sampled(dev):
    """The fused-attention configuration at full size (B=1, H=24, S=4096, D=128): 64 sampled query rows in each of
    3 sampled heads against the float64 closed form, for fp16 and int8-QK."""
    B, H, L = 1, 24, 4096
    q, k, v = qkv(B, H, H, L, L, seed=4)
    scale = 128 ** -0.5
    rows = torch.randperm(L, generator=gen(1))[:64].numpy()
    heads = [0, 11, 23]
    for int8_qk in (False, True):
        out = torch.empty(B, H, L, 128, dtype=torch.float16, device=dev)
        hip_attention.attention(q.to(dev), k.to(dev), v.to(dev), out, scale, int8_qk)
        o = out.cpu()
        for h in heads:
            qs = q[:, h:h + 1, rows]
            fn = oracle.attention_i8qk_f64 if int8_qk else oracle.attention_f64
            ref = fn(qs.numpy(), k[:, h:h + 1].numpy(), v[:, h:h + 1].numpy(), scale)
            close(o[:, h:h + 1, rows], ref)


@pytest.mark.parametrize("int8_qk", [False, True])
def test_attention_unaligned_kv_views(dev, int8_qk):
    """K and V views that start 4 bytes into their storage (not 16-byte aligned, as the kernel's global->LDS copies
    need): the wrapper copies them, and the result equals the one from aligned tensors."""
    q, k, v = qkv(1, 2, 2, 100, 300, seed=21)
    kb = torch.empty(k.numel() + 2, dtype=torch.float16, device=dev)
    vb = torch.empty(v.numel() + 2, dtype=torch.float16, device=dev)
    ku, vu = kb[2:].view(k.shape), vb[2:].view(v.shape)
    ku.copy_(k.to(dev))
    vu.copy_(v.to(dev))
    assert ku.data_ptr() % 16 != 0 and vu.data_ptr() % 16 != 0
    out_u = torch.empty(1, 2, 100, 128, dtype=torch.float16, device=dev)
    out_a = torch.empty_like(out_u)
    hip_attention.attention(q.to(dev), ku, vu, out_u, 128 ** -0.5, int8_qk)
    hip_attention.attention(q.to(dev), k.to(dev), v.to(dev), out_a, 128 ** -0.5, int8_qk)
    assert torch.equal(out_u.view(torch.int16), out_a.view(torch.int16))


def test_attention_abi_rejects_unaligned_kv(dev):
    """The C entry point itself refuses K / V rows that are not 16-byte aligned (invalid-argument error)."""
    q, k, v = (t.to(dev) for t in qkv(1, 1, 1, 32, 64, seed=22))
    kb = torch.empty(k.numel() + 2, dtype=torch.float16, device=dev)
    ku = kb[2:].view(k.shape)
    out = torch.empty_like(q)
    lib = _lib.load()
    strides = _lib.long_array([*q.stride()[:3], *ku.stride()[:3], *v.stride()[:3], *out.stride()[:3]])
    p = _lib.ptr
    assert lib.rda_attn(p(q), p(ku), p(v), p(out), 1, 1, 1, 32, 64, strides, 128 ** -0.5, _lib.stream()) == 1
