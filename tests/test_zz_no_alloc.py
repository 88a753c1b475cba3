"""rda_attention_decode_noalloc (decode attention with its split partials in the library's own device array) against
the allocating path it shares its kernels with -- int8_gemv.attention_decode, i.e. rda_attn_decode + rda_attn_merge
on torch-allocated partials -- bit for bit, through the C ABI: several calls in a row on one GPU, each smaller than
the one before (the array keeps the previous call's contents), up to the 256-head limit, and the rejection of a call
past it."""
import pytest
import torch

from comfyui_rdna2_attention_amd import _lib, int8_gemv
from helpers import gen

pytestmark = pytest.mark.gpu


def noalloc(q, k, v, lengths, scale=128 ** -0.5):
    B, _, H, _ = q.shape
    _, capacity, Hkv, _ = k.shape
    out = torch.empty_like(q)
    p = _lib.ptr
    _lib.check(_lib.load().rda_attention_decode_noalloc(p(q), p(k), p(v), p(lengths), p(out), B, H, Hkv, capacity, scale, _lib.stream()))
    return out


def inputs(dev, B, H, Hkv, capacity, lengths, seed):
    g = gen(seed)
    q = torch.randn(B, 1, H, 128, generator=g).to(dev)
    k = torch.randn(B, capacity, Hkv, 128, generator=g).to(dev)
    v = torch.randn(B, capacity, Hkv, 128, generator=g).to(dev)
    return q, k, v, torch.tensor(lengths, dtype=torch.int32, device=dev)


# (B, H, Hkv, capacity, lengths): the largest call the array holds (8 x 32 = 256 query heads), then smaller ones.
CALLS = [(8, 32, 8, 512, [512, 1, 300, 511, 64, 200, 3, 128]), (2, 32, 8, 2048, [2048, 1500]), (1, 8, 2, 300, [77])]


def test_noalloc_matches_allocating_path(dev):
    for i, (B, H, Hkv, capacity, lengths) in enumerate(CALLS):
        print(f"decode attention no-alloc call {i}: B={B} H={H} Hkv={Hkv} capacity={capacity} lengths={lengths}", flush=True)
        q, k, v, ln = inputs(dev, B, H, Hkv, capacity, lengths, seed=70 + i)
        got = noalloc(q, k, v, ln)
        ref = int8_gemv.attention_decode(q, k, v, ln)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int32), ref.view(torch.int32)), f"call {i} differs from rda_attn_decode + rda_attn_merge"


def test_noalloc_rejects_more_heads_than_its_array(dev):
    q, k, v, ln = inputs(dev, 1, 512, 128, 16, [16], seed=79)  # 512 query heads > 256: rejected before any launch
    with pytest.raises(RuntimeError, match="HIP error 1"):
        noalloc(q, k, v, ln)


def test_noalloc_replays_from_a_captured_graph(dev):
    """The stated use: rda_attention_decode_noalloc captured into a HIP graph (no allocation inside the capture) and
    replayed as the cache grows -- the lengths are read on the device, so the same graph serves every step. Each
    replay, with eager work and synchronizations between replays, equals the allocating path on that step's lengths
    bit for bit."""
    B, H, Hkv, capacity = 2, 32, 8, 1024
    q, k, v, ln = inputs(dev, B, H, Hkv, capacity, [100, 37], seed=81)
    out = torch.empty_like(q)
    p = _lib.ptr
    lib = _lib.load()
    args = (p(q), p(k), p(v), p(ln), p(out), B, H, Hkv, capacity, 128 ** -0.5)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        _lib.check(lib.rda_attention_decode_noalloc(*args, _lib.stream()))  # warm-up on the capturing stream
        side.synchronize()
        with torch.cuda.graph(graph, stream=side):
            _lib.check(lib.rda_attention_decode_noalloc(*args, _lib.stream()))
    torch.cuda.current_stream().wait_stream(side)
    for step, lengths in enumerate(([100, 37], [101, 38], [512, 700], [1024, 1], [3, 1023])):
        print(f"decode attention no-alloc graph replay {step}: lengths={lengths}", flush=True)
        ln.copy_(torch.tensor(lengths, dtype=torch.int32))
        noise = torch.randn(B, 1, H, 128, generator=gen(90 + step)).to(dev)
        q.copy_(noise)
        out.fill_(float("nan"))
        graph.replay()
        ref = int8_gemv.attention_decode(q, k, v, ln)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), ref.view(torch.int32)), f"replay {step} differs from the allocating path"
