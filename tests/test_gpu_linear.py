"""Parity of the linear path on the GPU (through the C ABI) against the oracle: quantized activations and scales
bit-exact, int32 accumulators bit-exact, fp16 outputs bit-exact (the epilogue is IEEE fp32 in a fixed order)."""
import numpy as np
import pytest
import torch

import oracle
from comfyui_rdna2_attention_amd import _lib, int8_gemm
from helpers import assert_same, activations, bits, channel_scales, gen, int4_weights, int8_weights, q_of

pytestmark = pytest.mark.gpu


def kern():
    return int8_gemm.get_kernels()


@pytest.mark.parametrize("M,K,group", [(7, 256, 256), (300, 3072, 256), (257, 3072, 128), (64, 16384, 256), (33, 8192, 128), (5, 128, 128)])
def test_rot_quant_bit_exact(dev, M, K, group):
    print(f"rot_quant M={M} K={K} group={group}", flush=True)
    x = activations(M, K, seed=M + K)
    x[M // 2] = 0  # an all-zero row: scale 1e-30, codes 0
    packed, scale = int8_gemm.quantize(kern().rot_quant_pack_a, x.to(dev), K, group=group)
    q_ref, s_ref, _ = oracle.rot_quant_rows(x.numpy(), group=group)
    assert_same(scale.cpu().numpy(), s_ref)
    assert_same(q_of(packed, M, K), q_ref)


@pytest.mark.parametrize("M,K", [(3, 64), (100, 3072), (9, 16384), (5, 18432), (4, 24576)])  # rows past 16384 are re-read, not staged
def test_quant_pack_a_bit_exact(dev, M, K):
    print(f"quant_pack_a M={M} K={K}", flush=True)
    x = activations(M, K, seed=3)
    packed, scale = int8_gemm.quantize(kern().quant_pack_a, x.to(dev), K)
    q_ref, s_ref = oracle.quant_rows(x.numpy())
    assert_same(scale.cpu().numpy(), s_ref)
    assert_same(q_of(packed, M, K), q_ref)


@pytest.mark.parametrize("act", ["swiglu", "gate", "situ"])
@pytest.mark.parametrize("M,K,group", [(37, 1024, 256), (16, 8192, 256), (21, 512, 128)])
def test_activation_rot_quant_bit_exact(dev, act, M, K, group):
    print(f"{act}_rot_quant M={M} K={K} group={group}", flush=True)
    g = gen(11)
    k = kern()
    if act == "situ":
        x = (torch.randn(M, 2 * K, generator=g) * 3).half()
        packed, scale = int8_gemm.quantize(k.situ_rot_quant_pack_a, x.to(dev), K, group=group)
        q_ref, s_ref, _ = oracle.rot_quant_rows(x.numpy(), act=oracle.ACT_SITU, group=group)
    else:
        a = (torch.randn(M, K, generator=g) * 4).half()
        b = (torch.randn(M, K, generator=g) * 4).half()
        entry = k.swiglu_rot_quant_pack_a if act == "swiglu" else k.gate_rot_quant_pack_a
        packed, scale = int8_gemm.quantize(entry, a.to(dev), K, up=b.to(dev), group=group)
        q_ref, s_ref, _ = oracle.rot_quant_rows(a.numpy(), act=oracle.ACT_SWIGLU if act == "swiglu" else oracle.ACT_GATE, group=group, u=b.numpy())
    assert_same(scale.cpu().numpy(), s_ref)
    assert_same(q_of(packed, M, K), q_ref)


def test_swiglu_every_fp16_gate(dev):
    """Every finite fp16 gate value through the SwiGLU kernel (whose silu takes a fast path away from fp16 rounding
    midpoints): row r has gate g_r at element 0 and 0 elsewhere, up = 16 there (1 where |g| > 2048, so the product
    stays finite) and 1 elsewhere. The rotated row is then +-r16(silu(g_r)) up / 16 in every element, exactly, so
    the row scale fixes |r16(silu(g_r))| and the codes its sign."""
    g = np.arange(65536, dtype=np.uint16).view(np.float16)
    g = g[np.isfinite(g)]
    M, K = len(g), 256
    gate = np.zeros((M, K), np.float16)
    gate[:, 0] = g
    up = np.ones((M, K), np.float16)
    up[:, 0] = np.where(np.abs(g) <= 2048, 16, 1)
    packed, scale = int8_gemm.quantize(kern().swiglu_rot_quant_pack_a, torch.from_numpy(gate).to(dev), K, up=torch.from_numpy(up).to(dev), group=256)
    q_ref, s_ref, _ = oracle.rot_quant_rows(gate, act=oracle.ACT_SWIGLU, group=256, u=up)
    assert_same(scale.cpu().numpy(), s_ref)
    assert_same(q_of(packed, M, K), q_ref)


def test_gate_every_fp16_gate(dev):
    """Every finite fp16 gate value through the sigmoid-gate kernel (whose sigmoid takes a fast path away from fp16
    rounding midpoints): row r has x = 16 and gate g_r at element 0, x = 0 elsewhere. The rotated row is then
    +-r16(16 r16(sigmoid(g_r))) / 16 in every element, exactly, so the row scale fixes r16(sigmoid(g_r))."""
    g = np.arange(65536, dtype=np.uint16).view(np.float16)
    g = g[np.isfinite(g)]
    M, K = len(g), 256
    x = np.zeros((M, K), np.float16)
    x[:, 0] = 16
    gate = np.zeros((M, K), np.float16)
    gate[:, 0] = g
    packed, scale = int8_gemm.quantize(kern().gate_rot_quant_pack_a, torch.from_numpy(x).to(dev), K, up=torch.from_numpy(gate).to(dev), group=256)
    q_ref, s_ref, _ = oracle.rot_quant_rows(x, act=oracle.ACT_GATE, group=256, u=gate)
    assert_same(scale.cpu().numpy(), s_ref)
    assert_same(q_of(packed, M, K), q_ref)


@pytest.mark.parametrize("B,L,K", [(1, 77, 3072), (2, 40, 1024)])
def test_mod_rot_quant_bit_exact(dev, B, L, K):
    print(f"mod_rot_quant B={B} L={L} K={K}", flush=True)
    g = gen(5)
    x = torch.randn(B * L, K, generator=g).half()
    w = (torch.randn(K, generator=g) * 0.1).float()
    s = (1 + torch.randn(B, K, generator=g) * 0.2).half()
    t = (torch.randn(B, K, generator=g) * 0.2).half()
    eps = 1e-6
    packed, scale = int8_gemm.quantized(B * L, K, dev)
    p = int8_gemm._lib.ptr
    # Device copies stay referenced until the launch: a temporary freed earlier would be reused by the next copy.
    xd, wd, sd, td = x.to(dev), w.to(dev), s.to(dev), t.to(dev)
    int8_gemm.launch(kern().mod_rot_quant_pack_a, 0, 0, 0, [p(xd), p(packed), p(scale), B * L, K, p(wd), p(sd), p(td), L, eps])
    q_ref, s_ref, _ = oracle.rot_quant_rows(x.numpy(), act=oracle.ACT_MOD, mod=(w.numpy(), s.numpy(), t.numpy(), L, eps))
    assert_same(scale.cpu().numpy(), s_ref)
    assert_same(q_of(packed, B * L, K), q_ref)


@pytest.mark.parametrize("M,K", [(40, 1024), (9, 3072)])
def test_rot_quant_i4_bit_exact(dev, M, K):
    x = activations(M, K, seed=17)
    packed, scale = int8_gemm.quantize(kern().rot_quant_pack_a_i4, x.to(dev), K)
    q_ref, s_ref, _ = oracle.rot_quant_rows(x.numpy(), i4=True)
    assert_same(scale.cpu().numpy(), s_ref)
    q = q_of(packed, M, K)
    assert np.abs(q).max() <= 7
    assert_same(q, q_ref)


@pytest.mark.parametrize("seed", range(8))
def test_w4a4_and_residual_random_shapes(dev, seed):
    """Seeded random shapes, bit for bit against the oracle: the W4A4 hook pair (rot_quant_pack_a_i4 + gemm_i4; M 1-1200,
    N a multiple of 64 up to 1280, K a multiple of 256 up to 4096) and the W8A8 linear with the block's gated residual
    in its epilogue (B 1-3 rows of L 1-600 tokens, N a multiple of 64 up to 1280, K a multiple of 256 up to 4096)."""
    rng = np.random.default_rng(9000 + seed)
    M, N, K = int(rng.integers(1, 1201)), 64 * int(rng.integers(1, 21)), 256 * int(rng.integers(1, 17))
    print(f"random w4a4 seed={seed} M={M} N={N} K={K}", flush=True)
    x = activations(M, K, seed=9100 + seed)
    w, wp = int4_weights(N, K, seed=9200 + seed)
    ws = channel_scales(N, seed=9300 + seed)
    k = kern()
    out = int8_gemm.run(k.rot_quant_pack_a_i4, k.gemm_i4, x.to(dev), wp.to(dev), ws.to(dev), None, K)
    q_ref, s_ref, _ = oracle.rot_quant_rows(x.numpy(), i4=True)
    assert_same(bits(out), bits(oracle.gemm_epilogue(oracle.gemm_acc(q_ref, w.numpy()), s_ref, ws.numpy())))

    B, L = int(rng.integers(1, 4)), int(rng.integers(1, 601))
    N, K = 64 * int(rng.integers(1, 21)), 256 * int(rng.integers(1, 17))
    M = B * L
    print(f"  residual epilogue B={B} L={L} K={K} N={N}", flush=True)
    g = gen(9400 + seed)
    x = activations(M, K, seed=9500 + seed)
    w8 = int8_weights(N, K, seed=9600 + seed)
    ws = channel_scales(N, seed=9700 + seed)
    R = torch.randn(B, L, N, generator=g).half()
    G = torch.randn(B, N, generator=g).half()
    out = int8_gemm.linear(x.to(dev), w8.to(dev), ws.to(dev), None, rotate=True, res=(R.to(dev), G.to(dev)))
    q_ref, s_ref, _ = oracle.rot_quant_rows(x.numpy())
    ref = oracle.gemm_epilogue(oracle.gemm_acc(q_ref, w8.numpy()), s_ref, ws.numpy(), R=R.numpy().reshape(M, N), G=G.numpy(), L=L)
    assert_same(bits(out), bits(ref))


QUANT_KINDS = ["plain", "rot", "i4", "swiglu", "gate", "situ", "mod"]


@pytest.mark.parametrize("seed", range(14))
def test_quantizers_random_shapes(dev, seed):
    """Seeded random shapes through every activation quantizer, codes and scales bit for bit against the oracle: M
    from 1 to 600 rows; K a multiple of the rotation group (128 or 256) up to the 16384 values a row keeps in LDS
    (MOD: up to 8192, group 256); plain quantization K a multiple of 16 up to 25600 (past 16384 the row is read
    again, not staged); an all-zero row where there are two rows or more."""
    kind = QUANT_KINDS[seed % len(QUANT_KINDS)]
    rng = np.random.default_rng(5000 + seed)
    M = int(rng.integers(1, 601))
    group = 256 if kind == "mod" else int(rng.choice([128, 256]))
    K = (16 * int(rng.integers(1, 1601)) if kind == "plain" else 256 * int(rng.integers(1, 33)) if kind == "mod"
         else group * int(rng.integers(1, 16384 // group + 1)))
    print(f"random quantizer seed={seed} {kind} M={M} K={K} group={group}", flush=True)
    g = gen(5100 + seed)
    k = kern()
    if kind in ("plain", "rot", "i4"):
        x = activations(M, K, seed=5200 + seed, outliers=int(rng.integers(0, 9)))
        if M >= 2:
            x[int(rng.integers(0, M))] = 0
        if kind == "plain":
            packed, scale = int8_gemm.quantize(k.quant_pack_a, x.to(dev), K)
            q_ref, s_ref = oracle.quant_rows(x.numpy())
        else:
            entry = k.rot_quant_pack_a if kind == "rot" else k.rot_quant_pack_a_i4
            packed, scale = int8_gemm.quantize(entry, x.to(dev), K, group=group)
            q_ref, s_ref, _ = oracle.rot_quant_rows(x.numpy(), group=group, i4=kind == "i4")
    elif kind == "situ":
        x = (torch.randn(M, 2 * K, generator=g) * 3).half()
        packed, scale = int8_gemm.quantize(k.situ_rot_quant_pack_a, x.to(dev), K, group=group)
        q_ref, s_ref, _ = oracle.rot_quant_rows(x.numpy(), act=oracle.ACT_SITU, group=group)
    elif kind in ("swiglu", "gate"):
        a = (torch.randn(M, K, generator=g) * 4).half()
        b = (torch.randn(M, K, generator=g) * 4).half()
        entry = k.swiglu_rot_quant_pack_a if kind == "swiglu" else k.gate_rot_quant_pack_a
        packed, scale = int8_gemm.quantize(entry, a.to(dev), K, up=b.to(dev), group=group)
        q_ref, s_ref, _ = oracle.rot_quant_rows(a.numpy(), act=oracle.ACT_SWIGLU if kind == "swiglu" else oracle.ACT_GATE, group=group,
                                                u=b.numpy())
    else:
        L = int(rng.integers(1, M + 1))
        while M % L:
            L -= 1
        B = M // L
        x = torch.randn(M, K, generator=g).half()
        w = (torch.randn(K, generator=g) * 0.1).float()
        sm = (1 + torch.randn(B, K, generator=g) * 0.2).half()
        t = (torch.randn(B, K, generator=g) * 0.2).half()
        packed, scale = int8_gemm.quantized(M, K, dev)
        p = int8_gemm._lib.ptr
        xd, wd, sd, td = x.to(dev), w.to(dev), sm.to(dev), t.to(dev)
        int8_gemm.launch(k.mod_rot_quant_pack_a, 0, 0, 0, [p(xd), p(packed), p(scale), M, K, p(wd), p(sd), p(td), L, 1e-6])
        q_ref, s_ref, _ = oracle.rot_quant_rows(x.numpy(), act=oracle.ACT_MOD, mod=(w.numpy(), sm.numpy(), t.numpy(), L, 1e-6))
    assert_same(scale.cpu().numpy(), s_ref)
    assert_same(q_of(packed, M, K), q_ref)


def packed_from(a_int8):
    return torch.from_numpy(np.ascontiguousarray(a_int8)).view(torch.int32).reshape(-1)


@pytest.mark.parametrize("M,N,K", [(4096, 3072, 3072), (1000, 192, 512), (513, 64, 64), (256, 256, 8192), (77, 128, 1024), (300, 320, 192),
                                   (512, 3072, 6144),  # the shape of the reference's gemm_k6144 (int8_gemm.hip:414)
                                   # the reference's own GEMM check shapes (prototypes/bg.py:26, given there as M, K, N)
                                   (4056, 8192, 2048), (4056, 2048, 8192), (4056, 2048, 2048), (3014, 16384, 3072),
                                   (4096, 3072, 8192)])  # the Krea 2 MLP's down projection: 256 x 192 tiles, 64 k-slices
def test_gemm_int32_accumulators_exact(dev, M, N, K):
    print(f"gemm_acc M={M} N={N} K={K}", flush=True)
    g = gen(M + N + K)
    a = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8).numpy()
    w = torch.randint(-128, 128, (N, K), generator=g, dtype=torch.int8)
    acc = int8_gemm.gemm_acc(packed_from(a).to(dev), w.to(dev), M, K)
    assert_same(acc.cpu().numpy(), oracle.gemm_acc(a, w.numpy()))


@pytest.mark.parametrize("M,N,K", [(600, 256, 1024), (128, 64, 256), (1000, 384, 512), (300, 192, 1408)])
def test_gemm_int4_weight_accumulators_exact(dev, M, N, K):
    print(f"gemm_acc int4 M={M} N={N} K={K}", flush=True)
    a = torch.randint(-128, 128, (M, K), generator=gen(1), dtype=torch.int8).numpy()
    w, wp = int4_weights(N, K, seed=2)
    acc = int8_gemm.gemm_acc(packed_from(a).to(dev), wp.to(dev), M, K, int4=True)
    assert_same(oracle.unpack_int4(wp.numpy(), K), w.numpy())
    assert_same(acc.cpu().numpy(), oracle.gemm_acc(a, w.numpy()))


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("M,N,K,group", [(4096, 3072, 3072, 128), (520, 256, 1024, 256), (700, 192, 768, 256), (515, 64, 512, 128)])
def test_w8a8_linear_bit_exact(dev, M, N, K, group, bias):
    print(f"w8a8 linear M={M} N={N} K={K} group={group} bias={bias}", flush=True)
    x = activations(M, K, seed=1)
    w = int8_weights(N, K, seed=2)
    ws = channel_scales(N, seed=3)
    b = (torch.randn(N, generator=gen(4)) * 0.5).half() if bias else None
    out = int8_gemm.linear(x.to(dev), w.to(dev), ws.to(dev), None if b is None else b.to(dev), rotate=True, group=group)
    q_ref, s_ref, _ = oracle.rot_quant_rows(x.numpy(), group=group)
    ref = oracle.gemm_epilogue(oracle.gemm_acc(q_ref, w.numpy()), s_ref, ws.numpy(), None if b is None else b.numpy())
    assert_same(bits(out), bits(ref))


# 128-, 192- and 256-wide tiles of the direct-copy GEMM; N = 320 (no such width divides it) takes the register-load GEMM
@pytest.mark.parametrize("B,L,K,N", [(2, 300, 512, 256), (1, 600, 256, 576), (2, 2048, 256, 8192), (1, 520, 256, 320)])
def test_gemm_residual_epilogue_bit_exact(dev, B, L, K, N):
    print(f"residual epilogue B={B} L={L} K={K} N={N}", flush=True)
    M = B * L
    g = gen(9)
    x = activations(M, K, seed=7)
    w = int8_weights(N, K, seed=8)
    ws = channel_scales(N, seed=9)
    R = torch.randn(B, L, N, generator=g).half()  # the block's x: (B, L, D), so L = R.shape[1]
    G = torch.randn(B, N, generator=g).half()
    out = int8_gemm.linear(x.to(dev), w.to(dev), ws.to(dev), None, rotate=True, res=(R.to(dev), G.to(dev)))
    q_ref, s_ref, _ = oracle.rot_quant_rows(x.numpy())
    ref = oracle.gemm_epilogue(oracle.gemm_acc(q_ref, w.numpy()), s_ref, ws.numpy(), R=R.numpy().reshape(M, N), G=G.numpy(), L=L)
    assert_same(bits(out), bits(ref))


@pytest.mark.parametrize("M,K,N", [(512, 2048, 256), (4096, 8192, 3072)])  # the second is the Krea 2 MLP's down projection
def test_swiglu_down_linear_bit_exact(dev, M, K, N):
    print(f"swiglu down linear M={M} K={K} N={N}", flush=True)
    g = gen(12)
    gate = torch.randn(M, K, generator=g).half()
    up = torch.randn(M, K, generator=g).half()
    w = int8_weights(N, K, seed=13)
    ws = channel_scales(N, seed=14)
    out = int8_gemm.linear(gate.to(dev), w.to(dev), ws.to(dev), None, up=up.to(dev))
    q_ref, s_ref, _ = oracle.rot_quant_rows(gate.numpy(), act=oracle.ACT_SWIGLU, u=up.numpy())
    ref = oracle.gemm_epilogue(oracle.gemm_acc(q_ref, w.numpy()), s_ref, ws.numpy())
    assert_same(bits(out), bits(ref))


# K / 128 = 8, 4, 24 and 26 slices: whole and partial passes of the slice loop over the three stages; 2, 6 and 10 slices
# (tail slices only; one pass and its tail); K = 12288 and 8192 (past K = 3456 the block's group scales no longer fit
# two blocks per CU: one block per CU)
@pytest.mark.parametrize("M,N,K", [(520, 512, 1024), (300, 192, 512), (4096, 1024, 3072), (200, 256, 3328), (520, 256, 12288), (300, 384, 8192),
                                   (64, 128, 256), (200, 256, 768), (129, 128, 1280)])
def test_w4a8_bit_exact(dev, M, N, K):
    print(f"w4a8 M={M} N={N} K={K}", flush=True)
    x = activations(M, K, seed=7, outliers=0)
    w, wp = int4_weights(N, K, seed=8)
    gs = (torch.rand(N, K // 128, generator=gen(9)) * 1.5e-2 + 5e-3).half()
    out = int8_gemm.linear_w4a8(x.to(dev), wp.to(dev), gs.to(dev))
    q_ref, s_ref, _ = oracle.rot_quant_rows(x.numpy())
    ref = oracle.w4a8_epilogue(oracle.w4a8_partials(q_ref, w.numpy()), s_ref, gs.numpy())
    assert_same(bits(out), bits(ref))


def test_w4a8_full_size_sampled_rows(dev):
    """The W4A8 configuration at full size (4096 x 12288 x 3072): every output row of a seeded sample of 48 rows
    against the oracle, bit for bit."""
    M, N, K = 4096, 12288, 3072
    x = activations(M, K, seed=7, outliers=0)
    w, wp = int4_weights(N, K, seed=8)
    gs = (torch.rand(N, K // 128, generator=gen(9)) * 1.5e-2 + 5e-3).half()
    out = int8_gemm.linear_w4a8(x.to(dev), wp.to(dev), gs.to(dev)).cpu().numpy()
    rows = torch.randperm(M, generator=gen(10))[:48].numpy()
    q_ref, s_ref, _ = oracle.rot_quant_rows(x.numpy()[rows])
    ref = oracle.w4a8_epilogue(oracle.w4a8_partials(q_ref, w.numpy()), s_ref, gs.numpy())
    assert_same(bits(out[rows]), bits(ref))


def test_w4a8_full_size_every_output(dev):
    """The W4A8 configuration at full size (4096 x 12288 x 3072): all 50 M outputs bit for bit. The reference is built
    on the GPU from pinned pieces: the int32 partial of every 128-wide group from rda_gemm_acc on that K slice (the
    accumulator entry point, bit-exact above), then the W4A8 epilogue evaluated in float64, where each step is exact
    before its single rounding to fp32 -- p_g gs_g + y (p_g < 2^18, gs fp16, y fp32: the exact sum fits 53 bits, which
    the test asserts) rounded once is the fp32 fma; y as rounded once is the fp32 product -- then fp16."""
    M, N, K = 4096, 12288, 3072
    x = activations(M, K, seed=7, outliers=0)
    w, wp = int4_weights(N, K, seed=8)
    gs = (torch.rand(N, K // 128, generator=gen(9)) * 1.5e-2 + 5e-3).half()
    xd, wpd, gsd = x.to(dev), wp.to(dev), gs.to(dev)
    out = int8_gemm.linear_w4a8(xd, wpd, gsd)
    packed, a_scale = int8_gemm.quantize(kern().rot_quant_pack_a, xd, K)
    a8 = packed.view(torch.int8)[:M * K].view(M, K)
    y = torch.zeros(M, N, dtype=torch.float64, device=dev)
    for g in range(K // 128):
        print(f"w4a8 full size: group {g}", flush=True)
        part = int8_gemm.gemm_acc(a8[:, g * 128:(g + 1) * 128].contiguous(), wpd[:, g * 64:(g + 1) * 64].contiguous(), M, 128, int4=True)
        prod = part.double() * gsd[:, g].double()[None, :]
        total = prod + y
        assert torch.equal(total - y, prod), "a float64 step was inexact"
        y = total.float().double()
    ref = (y * a_scale.double()[:, None]).float().half()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"{(out != ref).sum().item()} outputs differ"


# Shapes of each block the k-interleaved pair runs (two 128 x 128 blocks per CU; past K = 3456 one 128 x 256 block, or
# one 128 x 128 block when N % 256 != 0), rotation groups 256 and 128, a partial last row block, with and without bias.
@pytest.mark.parametrize("M,N,K,group,with_bias", [(520, 512, 1024, 256, False), (200, 256, 12288, 256, True), (300, 384, 8192, 128, False),
                                                   (129, 128, 1280, 256, True), (64, 128, 128, 128, False)])
def test_w4a8_interleaved_pair_matches_natural(dev, M, N, K, group, with_bias):
    """rot_quant_pack_a_il writes rot_quant_pack_a's scales, and its codes with each 8 values of k as the 4 even ones,
    then the 4 odd ones; gemm_w4a8_il on them (linear_w4a8's default route) gives gemm_w4a8's outputs on the natural
    codes bit for bit."""
    print(f"w4a8 interleaved M={M} N={N} K={K} group={group} bias={with_bias}", flush=True)
    x = activations(M, K, seed=71, outliers=0).to(dev)
    _, wp = int4_weights(N, K, seed=72)
    gs = (torch.rand(N, K // 128, generator=gen(73)) * 1.5e-2 + 5e-3).half().to(dev)
    bias = (torch.rand(N, generator=gen(74)) - 0.5).half().to(dev) if with_bias else None
    wp = wp.to(dev)
    k = kern()
    assert int8_gemm._interleaved(wp, gs, bias, N, K, True, 128)
    nat = int8_gemm.quantize(k.rot_quant_pack_a, x, K, group=group)
    il = int8_gemm.quantize(k.rot_quant_pack_a_il, x, K, group=group)
    assert torch.equal(il[1], nat[1])
    qn = nat[0].view(torch.int8)[:M * K].view(M, K // 8, 8)
    qi = il[0].view(torch.int8)[:M * K].view(M, K // 8, 8)
    assert torch.equal(qi, torch.cat([qn[..., 0::2], qn[..., 1::2]], dim=-1))
    out_nat = int8_gemm.linear_w4a8(x, wp, gs, bias, group=group, activations=nat)
    out_il = int8_gemm.linear_w4a8(x, wp, gs, bias, group=group)
    assert torch.equal(out_il.view(torch.int16), out_nat.view(torch.int16)), f"{(out_il != out_nat).sum().item()} outputs differ"


def test_w4a8_interleaved_gemm_refuses_other_shapes(dev):
    """gemm_w4a8_il serves only its direct-copy kernel: N % 128 != 0 and a 64-wide scale group are refused before any
    launch, where linear_w4a8 keeps the natural-order pair."""
    M, N, K = 64, 192, 256
    a = torch.zeros(256 * K // 4, dtype=torch.int32, device=dev)
    s = torch.ones(M, dtype=torch.float32, device=dev)
    w = torch.zeros(N, K // 2, dtype=torch.int8, device=dev)
    out = torch.empty(M, N, dtype=torch.float16, device=dev)
    p = _lib.ptr
    for n, group, gs in ((N, 128, torch.ones(N, K // 128, dtype=torch.float16, device=dev)),
                         (128, 64, torch.ones(128, K // 64, dtype=torch.float16, device=dev))):
        with pytest.raises(RuntimeError, match="HIP error 1"):
            _lib.call("rda_gemm_w4a8_il", p(a), p(w), p(s), p(gs), None, p(out), M, n, K, group)
    assert not int8_gemm._interleaved(w, torch.ones(N, K // 128, dtype=torch.float16, device=dev), None, N, K, True, 128)


def test_w4a4_hook_path_bit_exact(dev):
    """rot_quant_pack_a_i4 + gemm_i4 (the convrot_w4a4_forward replacement) against the oracle."""
    M, N, K = 600, 256, 1024
    x = activations(M, K, seed=21)
    w, wp = int4_weights(N, K, seed=22)
    ws = channel_scales(N, seed=23)
    k = kern()
    out = int8_gemm.run(k.rot_quant_pack_a_i4, k.gemm_i4, x.to(dev), wp.to(dev), ws.to(dev), None, K)
    q_ref, s_ref, _ = oracle.rot_quant_rows(x.numpy(), i4=True)
    ref = oracle.gemm_epilogue(oracle.gemm_acc(q_ref, w.numpy()), s_ref, ws.numpy())
    assert_same(bits(out), bits(ref))


def test_rejects_unsupported_shapes(dev):
    x = activations(8, 100, seed=1)
    with pytest.raises(RuntimeError, match="HIP error 1"):
        int8_gemm.quantize(kern().rot_quant_pack_a, x.to(dev), 100)


def test_w8a8_linear_unaligned_weight_view(dev):
    """A weight view that starts 4 bytes into its storage (not 16-byte aligned, as the direct-copy kernel needs) is
    served by the register-load GEMM, bit-exact all the same."""
    M, N, K = 600, 256, 1024
    x = activations(M, K, seed=31)
    w = int8_weights(N, K, seed=32)
    ws = channel_scales(N, seed=33)
    buf = torch.empty(N * K + 4, dtype=torch.int8, device=dev)
    wu = buf[4:].view(N, K)
    wu.copy_(w.to(dev))
    assert wu.data_ptr() % 16 != 0
    out = int8_gemm.linear(x.to(dev), wu, ws.to(dev), None, rotate=True)
    q_ref, s_ref, _ = oracle.rot_quant_rows(x.numpy())
    assert_same(bits(out), bits(oracle.gemm_epilogue(oracle.gemm_acc(q_ref, w.numpy()), s_ref, ws.numpy())))


def test_plain_int8_linear_long_rows(dev):
    """A non-rotated int8 linear (quant_pack_a + GEMM, the path of any eligible int8 layer without ConvRot) with
    K = 18432, past the rows the quantization pass holds in LDS: bit-exact, as the reference takes any K here."""
    M, N, K = 520, 128, 18432
    x = activations(M, K, seed=41)
    w = int8_weights(N, K, seed=42)
    ws = channel_scales(N, seed=43)
    out = int8_gemm.linear(x.to(dev), w.to(dev), ws.to(dev), None)
    q_ref, s_ref = oracle.quant_rows(x.numpy())
    assert_same(bits(out), bits(oracle.gemm_epilogue(oracle.gemm_acc(q_ref, w.numpy()), s_ref, ws.numpy())))


# Scale groups of 64 and 256 are served by the register-load GEMM's per-group fold; 128 by the direct-copy kernel.
@pytest.mark.parametrize("scale_group", [64, 256])
def test_w4a8_other_scale_groups_bit_exact(dev, scale_group):
    M, N, K = 520, 256, 1024
    print(f"w4a8 scale_group={scale_group} M={M} N={N} K={K}", flush=True)
    x = activations(M, K, seed=51, outliers=0)
    w, wp = int4_weights(N, K, seed=52)
    gs = (torch.rand(N, K // scale_group, generator=gen(53)) * 1.5e-2 + 5e-3).half()
    out = int8_gemm.linear_w4a8(x.to(dev), wp.to(dev), gs.to(dev), scale_group=scale_group)
    q_ref, s_ref, _ = oracle.rot_quant_rows(x.numpy())
    ref = oracle.w4a8_epilogue(oracle.w4a8_partials(q_ref, w.numpy(), group=scale_group), s_ref, gs.numpy())
    assert_same(bits(out), bits(ref))


@pytest.mark.parametrize("layout", ["every_other_column", "transposed", "offset_columns", "odd_pitch"])
def test_linears_take_strided_activations(dev, layout):
    """Activations the quantization pass cannot read as 16-byte aligned rows -- a last dimension that is not
    contiguous, rows starting one value into their storage (big[:, 1:K + 1]), a row pitch that is not a multiple of 8
    values -- are copied into rows first: the W4A8 and W8A8 linears give the results of the contiguous input."""
    M, N, K = 512, 256, 1024
    print(f"strided activations {layout}", flush=True)
    x = activations(M, K, seed=61, outliers=0)
    if layout == "every_other_column":
        big = torch.zeros(M, 2 * K, dtype=torch.float16, device=dev)
        big[:, ::2] = x.to(dev)
        xv = big[:, ::2]
    elif layout == "transposed":
        xv = x.t().contiguous().to(dev).t()
    elif layout == "offset_columns":
        big = torch.zeros(M, K + 8, dtype=torch.float16, device=dev)
        big[:, 1:K + 1] = x.to(dev)
        xv = big[:, 1:K + 1]
        assert xv.data_ptr() % 16
    else:
        big = torch.zeros(M, K + 4, dtype=torch.float16, device=dev)
        big[:, :K] = x.to(dev)
        xv = big[:, :K]
        assert xv.stride(0) % 8
    w, wp = int4_weights(N, K, seed=62)
    gs = (torch.rand(N, K // 128, generator=gen(63)) * 1.5e-2 + 5e-3).half()
    q_ref, s_ref, _ = oracle.rot_quant_rows(x.numpy())
    out = int8_gemm.linear_w4a8(xv, wp.to(dev), gs.to(dev))
    assert_same(bits(out), bits(oracle.w4a8_epilogue(oracle.w4a8_partials(q_ref, w.numpy()), s_ref, gs.numpy())))
    w8 = int8_weights(N, K, seed=64)
    ws = channel_scales(N, seed=65)
    out = int8_gemm.linear(xv, w8.to(dev), ws.to(dev), None, rotate=True)
    assert_same(bits(out), bits(oracle.gemm_epilogue(oracle.gemm_acc(q_ref, w8.numpy()), s_ref, ws.numpy())))


@pytest.mark.parametrize("seed", range(10))
def test_linears_random_shapes(dev, seed):
    """Seeded random shapes through both linears, each against the oracle bit for bit: M from 1 to 1200 rows (partial
    row tiles, and fewer rows than one tile), N a multiple of 64 up to 1280 (tile widths of 64 to 256, or none of them,
    which takes the register-load GEMM), K a multiple of the rotation group up to 4096, bias on half the cases."""
    rng = np.random.default_rng(2000 + seed)
    M = int(rng.integers(1, 1201))
    N = 64 * int(rng.integers(1, 21))
    group = int(rng.choice([128, 256]))
    K = group * int(rng.integers(1, 4096 // group + 1))
    with_bias = bool(rng.integers(0, 2))
    print(f"random linears seed={seed} M={M} N={N} K={K} group={group} bias={with_bias}", flush=True)
    x = activations(M, K, seed=3000 + seed, outliers=int(rng.integers(0, 9)))
    b = (torch.randn(N, generator=gen(3100 + seed)) * 0.5).half() if with_bias else None
    bd = None if b is None else b.to(dev)
    bn = None if b is None else b.numpy()
    q_ref, s_ref, _ = oracle.rot_quant_rows(x.numpy(), group=group)
    w8 = int8_weights(N, K, seed=3200 + seed)
    ws = channel_scales(N, seed=3300 + seed)
    out = int8_gemm.linear(x.to(dev), w8.to(dev), ws.to(dev), bd, rotate=True, group=group)
    assert_same(bits(out), bits(oracle.gemm_epilogue(oracle.gemm_acc(q_ref, w8.numpy()), s_ref, ws.numpy(), bn)))
    w, wp = int4_weights(N, K, seed=3400 + seed)
    gs = (torch.rand(N, K // 128, generator=gen(3500 + seed)) * 1.5e-2 + 5e-3).half()
    out = int8_gemm.linear_w4a8(x.to(dev), wp.to(dev), gs.to(dev), bd, group=group)
    assert_same(bits(out), bits(oracle.w4a8_epilogue(oracle.w4a8_partials(q_ref, w.numpy()), s_ref, gs.numpy(), bn)))
