"""Parity of the decode kernels and RMSNorm on the GPU against the oracle.

Bit-exact: the decode rotation (fp32 butterflies, exact power-of-two scale) and RMSNorm (the reference's summation
order, FMAs, correctly rounded 1/sqrt). Tolerance-based: the GEMVs and decode attention, whose fp32 sums run in a
different order than any CPU restatement. GEMV bound: |out - ref| <= 1e-5 * scale * sum_k |w x| (+ 2^-10 relative for
fp16 outputs); decode attention: |out - ref| <= 1e-5 + 1e-4 |ref|."""
import numpy as np
import pytest
import torch

import oracle
from comfyui_rdna2_attention_amd import int8_gemv, rms_norm
from helpers import assert_same, bits, channel_scales, gen, int8_weights

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,group", [(1, 256), (3, 1024), (2, 64), (1, 16384), (5, 16), (7, 4), (16, 256), (48, 256), (3, 64), (13, 16)])
def test_rotate_bit_exact(dev, rows, group):
    x = torch.randn(rows, group, generator=gen(group)).float()
    out = int8_gemv.rotate(x.to(dev), group)
    assert_same(out.cpu().numpy(), oracle.rotate_f32(x.numpy(), group))


def test_rotate_unaligned_view(dev):
    """A contiguous view that starts 4 bytes into its storage: same values as the oracle's rotation."""
    base = torch.randn(1 + 4096, generator=gen(41)).float().to(dev)
    x = base[1:].view(1, 4096)
    assert x.is_contiguous() and x.data_ptr() % 16 != 0
    out = int8_gemv.rotate(x, 256)
    assert_same(out.cpu().numpy(), oracle.rotate_f32(x.cpu().numpy().reshape(16, 256), 256).reshape(1, 4096))


def gemv_bound(w, x, scale, half):
    mag = np.abs(w.astype(np.float64)) @ np.abs(x.astype(np.float64)) * np.abs(scale)
    return 1e-5 * mag + 1e-12


@pytest.mark.parametrize("x_half", [False, True])
# one row per wave: (4096, 4096), (12288, 4096), (64, 512), (4100, 9728), (16, 1536), (1000, 1536), and with fp16 x read straight
# into registers (2049-4096 rows, K a multiple of 1024 up to 4096): (4096, 4096), (3000, 2048), (2500, 1024); K split over 4
# waves per row: (1024, 4096), (1002, 16384), (8, 4096); over 2: (2048, 8192), (1500, 2048)
@pytest.mark.parametrize("N,K", [(4096, 4096), (1024, 4096), (12288, 4096), (64, 512), (4100, 9728), (16, 1536), (1000, 1536), (1002, 16384),
                                 (8, 1024), (2048, 8192), (1500, 2048), (3000, 2048), (2500, 1024)])
def test_gemv_i8(dev, N, K, x_half):
    print(f"gemv_i8 N={N} K={K} half={x_half}", flush=True)
    x = torch.randn(1, K, generator=gen(16))
    x = x.half() if x_half else x.float()
    w = int8_weights(N, K, seed=17)
    s = channel_scales(N, seed=18)
    bias = torch.randn(N, generator=gen(19)).float() if N == 64 else None
    out = int8_gemv.gemv(x.to(dev), w.to(dev), s.to(dev), None if bias is None else bias.to(dev))
    assert out.dtype == x.dtype and out.shape == (1, N)
    xf = x.float().numpy().reshape(-1)
    ref = oracle.gemv_f64(xf, w.numpy(), s.numpy(), None if bias is None else bias.numpy())
    bound = gemv_bound(w.numpy(), xf, s.numpy(), x_half) + (np.abs(ref) * 2.0 ** -10 if x_half else 0)
    err = np.abs(out.cpu().double().numpy().reshape(-1) - ref)
    assert np.all(err <= bound), f"max err {err.max():.3e}"


# split K (N <= 2048): (1024, 4096), (8, 1024), (2048, 8192), (1500, 2048), (1002, 16384); one row per wave: (4096, 4096),
# (12288, 4096), (3000, 2048), and in 16-wave workgroups past K = 8192: (4096, 12288), (4096, 16384), (100, 9216); with a
# half step (K % 1024 == 512): (64, 512), (16, 1536), (4100, 9728), (40, 15872)
@pytest.mark.parametrize("N,K,group", [(1024, 4096, 256), (8, 1024, 4), (2048, 8192, 256), (1500, 2048, 16), (1002, 16384, 256), (4096, 4096, 256),
                                       (12288, 4096, 64), (4096, 12288, 256), (3000, 2048, 64), (64, 512, 64), (16, 1536, 256), (4100, 9728, 256),
                                       (4096, 16384, 16), (100, 4096, 4), (40, 15872, 256), (100, 9216, 64)])
def test_rotate_gemv_i8_bit_exact(dev, N, K, group):
    """rda_rotate_gemv_i8 (the ConvRot inside the GEMV launch) == rda_rotate then rda_gemv_i8, bit for bit; and the
    rotation itself is the oracle's (rotate is bit-exact), the GEMV within its bound."""
    print(f"rotate_gemv_i8 N={N} K={K} group={group}", flush=True)
    x = torch.randn(1, K, generator=gen(K + group)).float()
    w = int8_weights(N, K, seed=27)
    s = channel_scales(N, seed=28)
    bias = torch.randn(N, generator=gen(29)).float() if N in (64, 3000) else None
    wd, sd, bd = w.to(dev), s.to(dev), None if bias is None else bias.to(dev)
    xd = x.to(dev)
    kept = torch.full_like(xd, float("nan"))
    out = int8_gemv.rotate_gemv(xd, group, wd, sd, bd, kept)
    rotated = int8_gemv.rotate(xd, group)
    ref = int8_gemv.gemv(rotated, wd, sd, bd)
    assert out.shape == (1, N) and out.dtype == torch.float32
    assert torch.equal(xd.cpu(), x), "x was modified"
    assert_same(out.cpu().numpy(), ref.cpu().numpy())
    assert_same(kept.cpu().numpy(), rotated.cpu().numpy(), "stored rotation")
    assert torch.equal(int8_gemv.rotate_gemv(xd, group, wd, sd, bd), out)  # without a rotation to store
    xr = oracle.rotate_f32(x.numpy().reshape(-1, group), group).reshape(-1)
    f64 = oracle.gemv_f64(xr, w.numpy(), s.numpy(), None if bias is None else bias.numpy())
    assert np.all(np.abs(out.cpu().double().numpy().reshape(-1) - f64) <= gemv_bound(w.numpy(), xr, s.numpy(), False))


@pytest.mark.parametrize("seed", range(12))
def test_gemvs_random_shapes(dev, seed):
    """Seeded random shapes through the decode GEMVs: N from 1 to 6000 rows (split K, one row per wave, and the 16-wave
    workgroups past K = 8192), K a multiple of 512 up to 16384, fp32 or fp16 x, bias on half the cases. gemv within
    its bound of float64; rotate_gemv (a random rotation group) == rotate then gemv bit for bit, its stored rotation the
    oracle's; for K <= 8192, gemv_multi over 1-4 matrices of random heights == one launch per matrix bit for bit."""
    rng = np.random.default_rng(6000 + seed)
    N = int(rng.integers(1, 6001))
    K = 512 * int(rng.integers(1, 33))
    x_half = bool(rng.integers(0, 2))
    group = int(rng.choice(int8_gemv.FUSED_ROTATION_GROUPS))
    with_bias = bool(rng.integers(0, 2))
    print(f"random gemvs seed={seed} N={N} K={K} half={x_half} group={group} bias={with_bias}", flush=True)
    x = torch.randn(1, K, generator=gen(6100 + seed))
    w = int8_weights(N, K, seed=6200 + seed)
    sc = channel_scales(N, seed=6300 + seed)
    b = torch.randn(N, generator=gen(6400 + seed)).float() if with_bias else None
    wd, sd, bd = w.to(dev), sc.to(dev), None if b is None else b.to(dev)
    bn = None if b is None else b.numpy()
    xv = x.half() if x_half else x.float()
    out = int8_gemv.gemv(xv.to(dev), wd, sd, bd)
    xf = xv.float().numpy().reshape(-1)
    ref = oracle.gemv_f64(xf, w.numpy(), sc.numpy(), bn)
    bound = gemv_bound(w.numpy(), xf, sc.numpy(), x_half) + (np.abs(ref) * 2.0 ** -10 if x_half else 0)
    err = np.abs(out.cpu().double().numpy().reshape(-1) - ref)
    assert np.all(err <= bound), f"gemv: max err {err.max():.3e}"

    xd = x.float().to(dev)
    kept = torch.full_like(xd, float("nan"))
    fused = int8_gemv.rotate_gemv(xd, group, wd, sd, bd, kept)
    rotated = int8_gemv.rotate(xd, group)
    assert_same(fused.cpu().numpy(), int8_gemv.gemv(rotated, wd, sd, bd).cpu().numpy())
    assert_same(kept.cpu().numpy(), oracle.rotate_f32(x.float().numpy().reshape(-1, group), group).reshape(1, K), "stored rotation")

    if K <= 8192:
        layers = [(wd, sd, bd)]
        for i in range(int(rng.integers(0, 4))):
            n = int(rng.integers(1, 6001))
            layers.append((int8_weights(n, K, seed=6500 + 10 * seed + i).to(dev), channel_scales(n, seed=6600 + 10 * seed + i).to(dev),
                           torch.randn(n, generator=gen(6700 + 10 * seed + i)).float().to(dev) if rng.integers(0, 2) else None))
        mgroup = int(rng.choice([0, group]))
        xm = xd if mgroup else xv.to(dev)
        print(f"  gemv_multi heights={[l[0].shape[0] for l in layers]} group={mgroup}", flush=True)
        outs = int8_gemv.gemv_multi(xm, layers, group=mgroup)
        for o, (lw, ls, lb) in zip(outs, layers):
            one = int8_gemv.rotate_gemv(xm, mgroup, lw, ls, lb) if mgroup else int8_gemv.gemv(xm, lw, ls, lb)
            assert_same(o.cpu().numpy(), one.cpu().numpy())


@pytest.mark.parametrize("half", [False, True])
def test_gemv_unaligned_view(dev, half):
    """An input view one element into its storage (taken through an aligned copy): within the bound of the others."""
    base = torch.randn(1 + 4096, generator=gen(46))
    base = (base.half() if half else base.float()).to(dev)
    x = base[1:].view(1, 4096)
    assert x.data_ptr() % 16 != 0
    w, s = int8_weights(4096, 4096, seed=47), channel_scales(4096, seed=48)
    out = int8_gemv.gemv(x, w.to(dev), s.to(dev))
    xf = x.float().cpu().numpy().reshape(-1)
    ref = oracle.gemv_f64(xf, w.numpy(), s.numpy())
    bound = gemv_bound(w.numpy(), xf, s.numpy(), half) + (np.abs(ref) * 2.0 ** -10 if half else 0)
    assert np.all(np.abs(out.cpu().double().numpy().reshape(-1) - ref) <= bound)


def test_rotate_gemv_unaligned_view(dev):
    """An input view 4 bytes into its storage (taken through a 16-byte aligned copy): the same outputs and stored
    rotation as rotate then gemv of the view."""
    base = torch.randn(1 + 4096, generator=gen(43)).float().to(dev)
    x = base[1:].view(1, 4096)
    assert x.data_ptr() % 16 != 0
    w, s = int8_weights(1024, 4096, seed=44).to(dev), channel_scales(1024, seed=45).to(dev)
    kept = torch.empty(1, 4096, device=dev)
    out = int8_gemv.rotate_gemv(x, 256, w, s, None, kept)
    rotated = int8_gemv.rotate(x, 256)
    assert torch.equal(out, int8_gemv.gemv(rotated, w, s)) and torch.equal(kept, rotated)


@pytest.mark.parametrize("N,K", [(512, 1024), (64, 2560), (8, 256)])
def test_gemv_bf16(dev, N, K):
    x = torch.randn(1, 1, K, generator=gen(20)).float()
    w = torch.randn(N, K, generator=gen(21)).bfloat16()
    out = int8_gemv.logits_gemv(x.to(dev), w.to(dev))
    ref = w.double().numpy() @ x.double().numpy().reshape(-1)
    bound = 1e-5 * (np.abs(w.double().numpy()) @ np.abs(x.double().numpy().reshape(-1)))
    assert np.all(np.abs(out.cpu().double().numpy().reshape(-1) - ref) <= bound)


@pytest.mark.parametrize("B,H,Hkv,cap,lengths", [(1, 32, 8, 2048, [2048]), (2, 8, 2, 300, [1, 257]), (1, 4, 4, 64, [33]), (1, 16, 2, 100, [100])])
def test_attention_decode(dev, B, H, Hkv, cap, lengths):
    print(f"attention_decode B={B} H={H} Hkv={Hkv} cap={cap} lengths={lengths}", flush=True)
    g = gen(19)
    q = torch.randn(B, 1, H, 128, generator=g).float()
    k = torch.randn(B, cap, Hkv, 128, generator=g).float()
    v = torch.randn(B, cap, Hkv, 128, generator=g).float()
    ln = torch.tensor(lengths, dtype=torch.int32)
    out = int8_gemv.attention_decode(q.to(dev), k.to(dev), v.to(dev), ln.to(dev))
    ref = oracle.attention_decode_f64(q.numpy(), k.numpy(), v.numpy(), lengths)
    err = np.abs(out.cpu().double().numpy() - ref)
    assert np.all(err <= 1e-5 + 1e-4 * np.abs(ref)), f"max err {err.max():.3e}"


@pytest.mark.parametrize("seed", range(10))
def test_attention_decode_random_shapes(dev, seed):
    """Seeded random caches: batch 1-4, 1-8 KV heads with 1, 2, 4 or 8 query heads each, capacity 1-2600 and a ragged
    length per batch row in [1, capacity] (the last row's at capacity on even seeds), against float64."""
    rng = np.random.default_rng(4000 + seed)
    B = int(rng.integers(1, 5))
    Hkv = int(rng.choice([1, 2, 4, 8]))
    H = Hkv * int(rng.choice([1, 2, 4, 8]))
    cap = int(rng.integers(1, 2601))
    lengths = [int(n) for n in rng.integers(1, cap + 1, size=B)]
    if seed % 2 == 0:
        lengths[-1] = cap
    print(f"attention_decode random seed={seed} B={B} H={H} Hkv={Hkv} cap={cap} lengths={lengths}", flush=True)
    g = gen(4100 + seed)
    q = torch.randn(B, 1, H, 128, generator=g).float()
    k = torch.randn(B, cap, Hkv, 128, generator=g).float()
    v = torch.randn(B, cap, Hkv, 128, generator=g).float()
    out = int8_gemv.attention_decode(q.to(dev), k.to(dev), v.to(dev), torch.tensor(lengths, dtype=torch.int32).to(dev))
    ref = oracle.attention_decode_f64(q.numpy(), k.numpy(), v.numpy(), lengths)
    err = np.abs(out.cpu().double().numpy() - ref)
    assert np.all(err <= 1e-5 + 1e-4 * np.abs(ref)), f"max err {err.max():.3e}"


def test_attention_decode_length_past_capacity(dev):
    """A length past the cache's capacity reads no row beyond it: the kernel takes it as the capacity, bit for bit."""
    g = gen(23)
    q = torch.randn(2, 1, 8, 128, generator=g).to(dev)
    k = torch.randn(2, 96, 2, 128, generator=g).to(dev)
    v = torch.randn(2, 96, 2, 128, generator=g).to(dev)
    past = int8_gemv.attention_decode(q, k, v, torch.tensor([97, 5000], dtype=torch.int32, device=dev))
    full = int8_gemv.attention_decode(q, k, v, torch.tensor([96, 96], dtype=torch.int32, device=dev))
    assert torch.equal(past.view(torch.int32), full.view(torch.int32))


# D > 128: one wave per row, 1-4 steps per slot (D = 136 .. 8192, chunk counts that leave slots and steps partly or
# wholly empty), row counts that leave a workgroup's last waves without a row; D <= 128: 16 lanes per row.
@pytest.mark.parametrize("shape", [(1, 4096, 3072), (2, 3, 50, 128), (1, 7, 64), (1, 5, 8192), (2, 9, 136), (1, 3, 5120), (3, 2, 2048),
                                   (1, 6, 4104), (1, 1, 1032)])
def test_rms_norm_bit_exact(dev, shape):
    print(f"rms_norm {shape}", flush=True)
    g = gen(10)
    x = torch.randn(*shape, generator=g).half()
    w = (torch.randn(shape[-1], generator=g) * 0.1).float()  # gain ~ N(1, 0.1), stored zero-centred
    out = rms_norm.rms_norm(x.to(dev), w.to(dev), 1e-6)
    assert out.shape == x.shape and out.is_contiguous()
    assert_same(bits(out), bits(oracle.rms_norm(x.numpy(), w.numpy(), 1e-6)))


@pytest.mark.parametrize("D", [128, 256])
def test_rms_norm_strided_heads(dev, D):
    """(B, H, L, D) views of a (B, L, H*D) buffer: the kernel reads with strides, writes contiguous (B, H, L, D)."""
    B, L, H = 2, 33, 4
    g = gen(11)
    base = torch.randn(B, L, H * D, generator=g).half()
    w = (torch.randn(D, generator=g) * 0.1).float()
    view = base.to(dev).view(B, L, H, D).transpose(1, 2)
    out = rms_norm.rms_norm(view, w.to(dev), 1e-6)
    ref = oracle.rms_norm(base.view(B, L, H, D).transpose(1, 2).contiguous().numpy(), w.numpy(), 1e-6)
    assert_same(bits(out), bits(ref))


class _Norm:
    def __init__(self, scale, eps):
        self.scale, self.eps = scale, eps


@pytest.mark.parametrize("fb", [1, 2])
def test_rms_norm_rope_bit_exact(dev, fb):
    B, L, H = 2, 40, 3
    g = gen(12)
    x = torch.randn(B, L, H * 128, generator=g).half()
    w = (torch.randn(128, generator=g) * 0.1).float()
    ang = torch.randn(fb, 1, L, 64, generator=g)
    freqs = torch.stack([torch.cos(ang), -torch.sin(ang), torch.sin(ang), torch.cos(ang)], -1).reshape(fb, 1, L, 64, 2, 2).float()
    out = rms_norm.rms_norm_rope(x.to(dev), H, _Norm(w.to(dev), 1e-6), freqs.to(dev))
    xh = x.view(B, L, H, 128).transpose(1, 2).contiguous().numpy()
    f = freqs.numpy() if fb > 1 else np.broadcast_to(freqs.numpy(), (B,) + freqs.shape[1:])
    ref = oracle.rms_norm(xh, w.numpy(), 1e-6, freqs=np.ascontiguousarray(f))
    assert_same(bits(out), bits(ref))


@pytest.mark.parametrize("seed", range(10))
def test_norms_random_shapes(dev, seed):
    """Seeded random shapes, bit for bit against the oracle: RMSNorm of (B, L, D) or (B, H, L, D) (up to 1 x 600, 4 x 300,
    3 x 5 x 200 rows) and D a multiple of 8 up to 8192, eps 1e-6 or 1e-5; QK-norm + RoPE of B = 1-3, L = 1-700 and 1-24 heads, read
    from the q, k or v third of a fused (B, L, 3 H 128) buffer, with one set of rotations or one per batch row."""
    rng = np.random.default_rng(7000 + seed)
    g = gen(7100 + seed)
    caps = {1: [1, 600], 2: [4, 300], 3: [3, 5, 200]}[int(rng.integers(1, 4))]  # (B, L, D) or (B, H, L, D)
    lead = [int(rng.integers(1, c + 1)) for c in caps]
    D = 8 * int(rng.integers(1, 1025))
    eps = float(rng.choice([1e-6, 1e-5]))
    print(f"random norms seed={seed} rms_norm {(*lead, D)} eps={eps}", flush=True)
    x = torch.randn(*lead, D, generator=g).half()
    w = (torch.randn(D, generator=g) * 0.1).float()
    out = rms_norm.rms_norm(x.to(dev), w.to(dev), eps)
    assert_same(bits(out), bits(oracle.rms_norm(x.numpy(), w.numpy(), eps)))

    B, L, H = int(rng.integers(1, 4)), int(rng.integers(1, 701)), int(rng.integers(1, 25))
    fb = int(rng.choice([1, B]))
    third = int(rng.integers(0, 3))
    print(f"  rms_norm_rope B={B} L={L} H={H} freq batches={fb} third={third}", flush=True)
    fused = torch.randn(B, L, 3 * H * 128, generator=g).half()
    w = (torch.randn(128, generator=g) * 0.1).float()
    ang = torch.randn(fb, 1, L, 64, generator=g) * 3
    freqs = torch.stack([torch.cos(ang), -torch.sin(ang), torch.sin(ang), torch.cos(ang)], -1).reshape(fb, 1, L, 64, 2, 2).float()
    view = fused.to(dev)[:, :, third * H * 128:(third + 1) * H * 128]
    out = rms_norm.rms_norm_rope(view, H, _Norm(w.to(dev), eps), freqs.to(dev))
    xh = fused[:, :, third * H * 128:(third + 1) * H * 128].reshape(B, L, H, 128).transpose(1, 2).contiguous().numpy()
    f = freqs.numpy() if fb > 1 else np.broadcast_to(freqs.numpy(), (B,) + freqs.shape[1:])
    assert_same(bits(out), bits(oracle.rms_norm(xh, w.numpy(), eps, freqs=np.ascontiguousarray(f))))
