"""Seeded synthetic inputs shared by the tests. Everything is generated on the CPU with a torch.Generator, so the
GPU run and the oracle see identical values."""
import numpy as np
import torch


def gen(seed):
    return torch.Generator().manual_seed(seed)


def activations(M, K, seed, outliers=8, factor=30.0):
    """fp16 [M, K] ~ N(0, 1) with `outliers` channels scaled by `factor` (the W8A8 configuration's input)."""
    g = gen(seed)
    x = torch.randn(M, K, generator=g)
    if outliers:
        cols = torch.randperm(K, generator=g)[:outliers]
        x[:, cols] *= factor
    return x.half()


def int8_weights(N, K, seed):
    return torch.randint(-127, 128, (N, K), generator=gen(seed), dtype=torch.int8)


def channel_scales(N, seed, lo=1e-3, hi=3e-3):
    return (torch.rand(N, generator=gen(seed)) * (hi - lo) + lo).float()


def int4_weights(N, K, seed):
    """int8 values in [-8, 7] and their packed (N, K/2) uint8 form, low nibble = even k."""
    w = torch.randint(-8, 8, (N, K), generator=gen(seed), dtype=torch.int8)
    lo = (w[:, 0::2].to(torch.int16) & 0xF).to(torch.uint8)
    hi = (w[:, 1::2].to(torch.int16) & 0xF).to(torch.uint8)
    return w, (lo | (hi << 4)).to(torch.uint8)


def q_of(packed, M, K):
    """The int8 [M, K] view of a packed activation buffer (row-major, possibly padded)."""
    return packed.view(torch.int8)[:M * K].view(M, K).cpu().numpy()


def bits(t):
    a = t.detach().cpu().numpy() if isinstance(t, torch.Tensor) else np.asarray(t)
    return np.ascontiguousarray(a, dtype=np.float16).view(np.uint16)


def assert_same(got, ref, what=""):
    """Bit-exact comparison that reports how many elements differ and where."""
    got, ref = np.asarray(got), np.asarray(ref)
    assert got.shape == ref.shape, f"{what} shape {got.shape} != {ref.shape}"
    if got.dtype.kind == "f":
        got, ref = got.view(np.uint8 if got.itemsize == 1 else f"u{got.itemsize}"), ref.astype(got.dtype).view(f"u{got.itemsize}")
    bad = np.argwhere(got != ref)
    if len(bad):
        where = ", ".join(f"{tuple(int(v) for v in i)}: {got[tuple(i)]} vs {ref[tuple(i)]}" for i in bad[:5])
        raise AssertionError(f"{what} {len(bad)} of {got.size} elements differ; first: {where}")
