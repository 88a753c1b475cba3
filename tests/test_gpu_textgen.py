"""The text-generation path around the decode kernels (int8_gemv.py:48-126) on the GPU: linear_forward's single-token
GEMV with and without the ConvRot of its input, the bf16 logits of the last position, and a decode attention step
captured once in a HIP graph and replayed as the cache grows. ComfyUI's quantized-weight context
(comfy.ops.CastBiasWeightContext) is stood in for: it hands the layer's int8 weight (`_qdata`, `_params.scale`) and
bias to the code under test, which is all the patched forwards read from it.

Bounds: the GEMVs as in test_gpu_decode_norm (|out - ref| <= 1e-5 * scale * sum_k |w x| against float64; the rotation
is bit-exact, so the GEMV sees the oracle's rotated input); decode attention |out - ref| <= 1e-5 + 1e-4 |ref|, and
every graph replay equal bit for bit to an eager call at the same length."""
import types

import numpy as np
import pytest
import torch

import oracle
from comfyui_rdna2_attention_amd import int8_gemv
from helpers import channel_scales, gen, int8_weights

pytestmark = pytest.mark.gpu


def stand_in_comfy(monkeypatch, pairs):
    """comfy.ops.CastBiasWeightContext yielding pairs[id(module)] = (weight, bias) for the module it is given."""
    class CastBiasWeightContext:
        def __init__(self, module, **kwargs):
            self.pair = pairs[id(module)]

        def __enter__(self):
            return self.pair

        def __exit__(self, *exc):
            return False

    monkeypatch.setattr(int8_gemv, "comfy", types.SimpleNamespace(ops=types.SimpleNamespace(CastBiasWeightContext=CastBiasWeightContext)))


def int8_layer():
    layer = types.SimpleNamespace(weight_function=[], bias_function=[])
    layer.forward = None  # never reached on the single-token path
    return layer


@pytest.mark.parametrize("group", [0, 64, 256, 1024])
@pytest.mark.parametrize("N,K,bias", [(1024, 4096, False), (4096, 4096, True), (512, 12288, False)])
def test_linear_forward_single_token(dev, monkeypatch, N, K, bias, group):
    print(f"linear_forward N={N} K={K} bias={bias} group={group}", flush=True)
    w = int8_weights(N, K, seed=30)
    s = channel_scales(N, seed=31)
    b = torch.randn(N, generator=gen(32)).float() if bias else None
    layer = int8_layer()
    weight = types.SimpleNamespace(_qdata=w.to(dev), _params=types.SimpleNamespace(scale=s.to(dev)))
    stand_in_comfy(monkeypatch, {id(layer): (weight, None if b is None else b.to(dev))})
    x = torch.randn(1, 1, K, generator=gen(33)).float()
    out = int8_gemv.linear_forward(layer, N, K, torch.int8, group, x.to(dev))
    assert out.shape == (1, 1, N) and out.dtype == torch.float32
    xr = oracle.rotate_f32(x.numpy().reshape(1, K), group).reshape(-1) if group else x.numpy().reshape(-1)
    ref = oracle.gemv_f64(xr, w.numpy(), s.numpy(), None if b is None else b.numpy())
    bound = 1e-5 * (np.abs(w.numpy().astype(np.float64)) @ np.abs(xr.astype(np.float64))) * np.abs(s.numpy()) + 1e-12
    err = np.abs(out.cpu().double().numpy().reshape(-1) - ref)
    assert np.all(err <= bound), f"max err {err.max():.3e}"


def _weights(shapes, K, seed, bias=False, dev="cuda"):
    out = []
    for i, N in enumerate(shapes):
        w, s = int8_weights(N, K, seed=seed + i), channel_scales(N, seed=seed + 10 + i)
        b = torch.randn(N, generator=gen(seed + 20 + i)).float().to(dev) if bias and i % 2 == 0 else None
        out.append((w.to(dev), s.to(dev), b))
    return out


@pytest.mark.parametrize("shapes,K,group,half", [
    ((4096, 1024, 1024), 4096, 256, False),   # q|k|v of a Qwen3-8B layer: one row per wave + split-by-4 rows
    ((12288, 12288), 4096, 256, False),        # gate|up
    ((2048, 512, 64, 16), 4096, 64, False),    # split by 2 and 4, a partial last block
    ((1024, 4096), 8192, 16, False),           # 8 steps per row: split 4 with 2 steps per wave
    ((2560, 512, 512), 2560, 256, False),      # K with a half step (one row per wave throughout)
    ((4096, 1024, 1024), 4096, 0, False),      # already rotated input
    ((4096, 1024, 1024), 4096, 0, True),       # fp16 input and outputs
    ((3072, 1000), 3584, 4, False),            # odd N, half step, group 4
    ((12288, 1024, 2048), 4096, 256, False),   # two rows per wave beside split rows
    ((12288, 12296), 2560, 256, False),        # four rows per wave, half step, a partial last block
    ((16384, 8192), 4096, 0, True),            # four rows per wave, fp16
])
def test_gemv_multi_equals_one_launch_per_matrix(dev, shapes, K, group, half):
    """rda_gemv_i8_multi gives each matrix, bit for bit, what its own rda_gemv_i8 / rda_rotate_gemv_i8 launch gives,
    and the same stored rotation."""
    print(f"gemv_multi shapes={shapes} K={K} group={group} half={half}", flush=True)
    layers = _weights(shapes, K, seed=70, bias=True, dev=dev)
    x = torch.randn(1, K, generator=gen(71)).to(dev)
    x = x.half() if half else x
    kept = torch.empty(K, device=dev) if group else None
    outs = int8_gemv.gemv_multi(x, layers, group, kept)
    for (w, s, b), out in zip(layers, outs):
        ref = int8_gemv.rotate_gemv(x, group, w, s, b) if group else int8_gemv.gemv(x, w, s, b)
        assert out.dtype == ref.dtype and out.shape == ref.shape
        assert torch.equal(out, ref), f"N={w.shape[0]}: {(out != ref).sum().item()} outputs differ"
    if group:
        assert torch.equal(kept.view(1, K), int8_gemv.rotate(x, group))
        assert torch.equal(int8_gemv.gemv_multi(x, layers, group)[0], outs[0])  # without a rotation to store


def _layers_for_linear_forward(monkeypatch, shapes, K, seed, dev):
    mods, pairs = [], {}
    for N, (w, s, b) in zip(shapes, _weights(shapes, K, seed, dev=dev)):
        layer = int8_layer()
        pairs[id(layer)] = (types.SimpleNamespace(_qdata=w, _params=types.SimpleNamespace(scale=s)), b)
        mods.append((layer, N, w, s))
    stand_in_comfy(monkeypatch, pairs)
    return mods


def test_sibling_linears_run_as_one_launch(dev, monkeypatch):
    """q, k and v registered as siblings: one gemv_multi launch for the three single-token linear_forward calls, each
    output equal bit for bit to its own rotate then GEMV; after an in-place write to the input the next sibling call
    computes from the new values."""
    K = 4096
    mods = _layers_for_linear_forward(monkeypatch, (4096, 1024, 1024), K, 40, dev)
    int8_gemv.forget_siblings()
    int8_gemv.register_siblings([(m, N, K, torch.int8, 256) for m, N, _, _ in mods])
    calls = []
    multi = int8_gemv.gemv_multi
    monkeypatch.setattr(int8_gemv, "gemv_multi", lambda *a, **k: calls.append(1) or multi(*a, **k))
    try:
        x = torch.randn(1, 1, K, generator=gen(60)).float().to(dev)
        for _ in range(2):
            rotated = int8_gemv.rotate(x, 256)
            for layer, N, w, s in mods:
                out = int8_gemv.linear_forward(layer, N, K, torch.int8, 256, x)
                assert out.shape == (1, 1, N) and torch.equal(out, int8_gemv.gemv(rotated, w, s))
            x.mul_(-0.5)
        assert len(calls) == 2
    finally:
        int8_gemv.forget_siblings()


def test_sibling_outputs_stay_inside_their_graph(dev, monkeypatch):
    """Two graphs captured over the same input tensor, each running q, k and v as siblings: replaying only the second,
    after new values are written into the input, gives every sibling the second graph's own result for those values
    (no output of the first capture is handed to the second)."""
    K = 4096
    mods = _layers_for_linear_forward(monkeypatch, (4096, 1024, 1024), K, 40, dev)
    int8_gemv.forget_siblings()
    int8_gemv.register_siblings([(m, N, K, torch.int8, 256) for m, N, _, _ in mods])
    try:
        x = torch.randn(1, 1, K, generator=gen(61)).float().to(dev)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        graphs, outs = [], []
        with torch.cuda.stream(side):
            for layer, N, _, _ in mods:  # warm-up on the capture stream
                int8_gemv.linear_forward(layer, N, K, torch.int8, 256, x)
            for _ in range(2):
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, stream=side):
                    outs.append([int8_gemv.linear_forward(layer, N, K, torch.int8, 256, x) for layer, N, _, _ in mods])
                graphs.append(graph)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        for trial in range(3):
            print(f"sibling graph replay {trial}", flush=True)
            x.copy_(torch.randn(1, 1, K, generator=gen(62 + trial)).to(dev))
            graphs[1].replay()
            torch.cuda.synchronize()
            rotated = int8_gemv.rotate(x, 256)
            for (layer, N, w, s), out in zip(mods, outs[1]):
                assert torch.equal(out, int8_gemv.gemv(rotated, w, s))
    finally:
        int8_gemv.forget_siblings()


def test_linear_forward_prefill_rotates_each_call(dev, monkeypatch):
    """A generate() prefill (3 tokens, ConvRot group 1024): q, k and v each rotate their input and run the dequantized
    matmul; each output matches the oracle, also after an in-place write to the input. Bound: 1e-4 of
    scale * sum_k |w x| (fp32 matmul of 4096 terms)."""
    K, T, group = 4096, 3, 1024
    layers, pairs = [], {}
    for i, N in enumerate((4096, 1024, 1024)):
        w, s = int8_weights(N, K, seed=40 + i), channel_scales(N, seed=50 + i)
        layer = int8_layer()
        # per-channel scales as a column, as the dequantized matmul broadcasts them over the (N, K) weight
        pairs[id(layer)] = (types.SimpleNamespace(_qdata=w.to(dev), _params=types.SimpleNamespace(scale=s.view(N, 1).to(dev))), None)
        layers.append((layer, N, w, s))
    stand_in_comfy(monkeypatch, pairs)
    monkeypatch.setattr(int8_gemv, "generating", True)
    x = torch.randn(1, T, K, generator=gen(60)).float().to(dev)

    def check(layer, N, w, s, out):
        xr = oracle.rotate_f32(x.cpu().numpy().reshape(T, K), group).astype(np.float64)
        wd = w.numpy().astype(np.float64)
        ref = (xr @ wd.T) * s.numpy()
        bound = 1e-4 * (np.abs(xr) @ np.abs(wd).T) * np.abs(s.numpy()) + 1e-12
        assert np.all(np.abs(out.cpu().double().numpy().reshape(T, N) - ref) <= bound)

    for layer, N, w, s in layers:
        check(layer, N, w, s, int8_gemv.linear_forward(layer, N, K, torch.int8, group, x))
    x.mul_(-0.5)
    layer, N, w, s = layers[1]
    check(layer, N, w, s, int8_gemv.linear_forward(layer, N, K, torch.int8, group, x))


def test_logits_of_the_last_position(dev, monkeypatch):
    N, K, L = 4096, 2560, 7
    table = torch.randn(N, K, generator=gen(34)).bfloat16()
    embed = types.SimpleNamespace(weight_function=[])
    transformer = types.SimpleNamespace(model=types.SimpleNamespace(embed_tokens=embed))
    stand_in_comfy(monkeypatch, {id(embed): (table.to(dev), None)})
    x = torch.randn(1, L, K, generator=gen(35)).float()
    out = int8_gemv.logits(transformer, x.to(dev))
    assert out.shape == (1, 1, N) and out.dtype == torch.float32
    wd, xd = table.double().numpy(), x[0, -1].double().numpy()
    ref = wd @ xd
    bound = 1e-5 * (np.abs(wd) @ np.abs(xd))
    assert np.all(np.abs(out.cpu().double().numpy().reshape(-1) - ref) <= bound)


def test_decode_step_graph_replays_as_the_cache_grows(dev):
    """One capture, replays at growing lengths (the length is read on the device, int8_gemv.py:117-126); eager work
    between the replays, each replay checked against an eager call and the float64 restatement."""
    B, H, Hkv, cap = 1, 32, 8, 2048
    g = gen(36)
    q = torch.randn(B, 1, H, 128, generator=g).float().to(dev)
    k = torch.randn(B, cap, Hkv, 128, generator=g).float().to(dev)
    v = torch.randn(B, cap, Hkv, 128, generator=g).float().to(dev)
    lengths = torch.ones(B, dtype=torch.int32, device=dev)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        int8_gemv.attention_decode(q, k, v, lengths)  # warm-up on the capture stream
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            out = int8_gemv.attention_decode(q, k, v, lengths)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for L in (1, 33, 700, 2047, 2048, 5):
        print(f"graph replay at length {L}", flush=True)
        lengths.fill_(L)
        graph.replay()
        torch.cuda.synchronize()
        eager = int8_gemv.attention_decode(q, k, v, lengths)
        assert torch.equal(out, eager)
        ref = oracle.attention_decode_f64(q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy(), [L])
        err = np.abs(out.cpu().double().numpy() - ref)
        assert np.all(err <= 1e-5 + 1e-4 * np.abs(ref)), f"length {L}: max err {err.max():.3e}"

