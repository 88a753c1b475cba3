"""The Python API mirror on the CPU: hook installation and removal, the deferred-ConvRot side channel, eligibility
predicates and fallbacks to the original functions, state reset, and that an eligible call never computes on the
CPU (it raises without a GPU). ComfyUI and ComfyUI-INT8-Fast-ROCM are replaced by the stand-ins of tests/fakes.py."""
import logging
import types

import numpy as np
import pytest
import torch

import fakes
import oracle
from comfyui_rdna2_attention_amd import attention, hip_attention, int8_gemm, int8_gemv, rms_norm


def test_enable_without_pack_warns(monkeypatch, caplog):
    fakes.install(monkeypatch, pack=False)
    with caplog.at_level(logging.WARNING):
        int8_gemm.enable(True)
    assert "ComfyUI-INT8-Fast-ROCM is not loaded" in caplog.text


def test_enable_installs_and_removes_hooks(monkeypatch):
    comfy, mods = fakes.install(monkeypatch)
    pack, int4, convrot = mods["fakepack.int8_quant"], mods["fakepack.int4_quant"], mods["fakepack.convrot"]
    orig = (pack.triton_int8_linear, pack.triton_int8_linear_per_row, int4.convrot_w4a4_forward, convrot.rotate_activation,
            pack.Int8TensorwiseOps.Linear.forward, comfy.ops.linear_input_act)
    int8_gemm.enable(True)
    assert pack.triton_int8_linear.__name__ == "int8_linear" and pack.triton_int8_linear_per_row.__name__ == "int8_linear"
    assert int4.convrot_w4a4_forward.__name__ == "convrot_w4a4_forward" and int4.convrot_w4a4_forward is not orig[2]
    assert convrot.rotate_activation is int8_gemm.rotate_activation
    assert comfy.ops.linear_input_act is int8_gemm.linear_input_act
    assert int8_gemm.swiglu_fusable
    int8_gemm.enable(True)  # idempotent: the originals are saved once
    assert int8_gemm.originals["triton_int8_linear"] is orig[0]
    int8_gemm.enable(False)
    now = (pack.triton_int8_linear, pack.triton_int8_linear_per_row, int4.convrot_w4a4_forward, convrot.rotate_activation,
           pack.Int8TensorwiseOps.Linear.forward, comfy.ops.linear_input_act)
    assert all(a is b for a, b in zip(now, orig))
    assert not int8_gemm.swiglu_fusable


def test_swiglu_fusable_follows_triton(monkeypatch):
    fakes.install(monkeypatch, triton=False)
    int8_gemm.enable(True)
    assert not int8_gemm.swiglu_fusable


def test_wrap_forward_scopes_fusable(monkeypatch):
    fakes.install(monkeypatch)
    seen = []

    def forward(self, x):
        seen.append(int8_gemm.fusable)
        if x is None:
            raise ValueError("boom")
        return x

    wrapped = int8_gemm.wrap_forward(forward)
    layer = type("L", (), {"lora_patches": []})()
    wrapped(layer, 1)
    layer.lora_patches = ["lora"]
    wrapped(layer, 1)
    with pytest.raises(ValueError):
        layer.lora_patches = []
        wrapped(layer, None)
    assert seen == [True, False, True] and int8_gemm.fusable is False


def test_rotate_activation_defers_only_when_fusable(monkeypatch):
    _, mods = fakes.install(monkeypatch)
    int8_gemm.enable(True)
    x = torch.zeros(4, 512, dtype=torch.float16)
    assert torch.equal(int8_gemm.rotate_activation(x, None, 256), x * 2)  # not fusable: the original rotation
    assert int8_gemm.pending is None
    monkeypatch.setattr(int8_gemm, "fusable", True)
    assert int8_gemm.rotate_activation(x, None, 256) is x and int8_gemm.pending is x
    monkeypatch.setattr(int8_gemm, "pending", None)
    for bad in (torch.zeros(4, 512), torch.zeros(2, 4, 512, dtype=torch.float16), torch.zeros(4, 384, dtype=torch.float16),
                torch.zeros(4, 32768, dtype=torch.float16)):
        int8_gemm.rotate_activation(bad, None, 256)
        assert int8_gemm.pending is None
    int8_gemm.rotate_activation(x, None, 128)
    assert int8_gemm.pending is None
    monkeypatch.setattr(int8_gemm, "shared", ("packed", "scales"))
    assert int8_gemm.rotate_activation(x, None, 256) is x and int8_gemm.pending is None


def test_int8_linear_falls_back_with_replayed_transforms(monkeypatch):
    _, mods = fakes.install(monkeypatch)
    pack, convrot = mods["fakepack.int8_quant"], mods["fakepack.convrot"]
    orig = pack.triton_int8_linear
    int8_gemm.enable(True)
    w = torch.randint(-5, 6, (64, 256), dtype=torch.int8)
    # fp32 input: ineligible; the deferred rotation is replayed with the original before the original linear.
    x = torch.randn(600, 256)
    monkeypatch.setattr(int8_gemm, "pending", x)
    y = pack.triton_int8_linear(x, w, 0.5)
    (args, _), = orig.calls[-1:]
    assert torch.equal(args[0], x * 2) and len(convrot.build_hadamard.calls) == 1
    assert int8_gemm.pending is None and y.shape == (600, 64)
    # too few rows: ineligible; a pending SwiGLU up projection is applied as silu(gate) * up.
    g = torch.randn(8, 256, dtype=torch.float16)
    up = torch.randn(8, 256, dtype=torch.float16)
    monkeypatch.setattr(int8_gemm, "swiglu_up", up)
    pack.triton_int8_linear(g, w, 0.5)
    (args, _), = orig.calls[-1:]
    assert torch.equal(args[0], torch.nn.functional.silu(g) * up)
    assert int8_gemm.swiglu_up is None


def test_int8_linear_fused_block_error(monkeypatch):
    _, mods = fakes.install(monkeypatch)
    int8_gemm.enable(True)
    monkeypatch.setattr(int8_gemm, "residual", (torch.zeros(1), torch.zeros(1)))
    with pytest.raises(RuntimeError, match="a fused Krea 2 block reached a layer the int8 kernels can't run"):
        mods["fakepack.int8_quant"].triton_int8_linear(torch.randn(4, 256), torch.zeros(64, 256, dtype=torch.int8), 1.0)
    assert int8_gemm.residual is None


def test_eligible_int8_linear_never_runs_on_cpu(monkeypatch):
    """An eligible call goes to the GPU kernels; without a GPU it raises instead of computing on the CPU."""
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    _, mods = fakes.install(monkeypatch)
    int8_gemm.enable(True)
    monkeypatch.setattr(int8_gemm, "kernels", None)
    monkeypatch.setattr(int8_gemm._lib, "_lib", None)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        mods["fakepack.int8_quant"].triton_int8_linear(torch.randn(600, 256, dtype=torch.float16), torch.zeros(64, 256, dtype=torch.int8), 1.0)


def test_w4a4_hook_eligibility(monkeypatch):
    _, mods = fakes.install(monkeypatch)
    int4 = mods["fakepack.int4_quant"]
    orig = int4.convrot_w4a4_forward
    int8_gemm.enable(True)
    q = torch.zeros(64, 128, dtype=torch.uint8)
    x = torch.zeros(600, 256, dtype=torch.float16)
    for kwargs in ({"skip_rotation": True}, {"x_rot": x}):
        assert int4.convrot_w4a4_forward(x, q, torch.ones(64), None, 256, torch.float16, **kwargs) == "original-w4a4"
    assert int4.convrot_w4a4_forward(x, q, torch.ones(64), None, 128, torch.float16) == "original-w4a4"
    assert int4.convrot_w4a4_forward(x, q, torch.ones(64), None, 256, torch.bfloat16) == "original-w4a4"
    assert int4.convrot_w4a4_forward(x[:100], q, torch.ones(64), None, 256, torch.float16) == "original-w4a4"
    assert len(orig.calls) == 5


class _Layer:
    def __init__(self, **kw):
        self._is_quantized, self._use_convrot, self._convrot_groupsize, self.lora_patches, self.in_features = True, True, 256, [], 512
        self.__dict__.update(kw)


def test_fuse_act_predicate():
    x = torch.zeros(2, 512, dtype=torch.float16)
    assert int8_gemm.fuse_act(_Layer(), x, 512)
    assert not int8_gemm.fuse_act(_Layer(_is_w4a8=True), x, 512)
    assert not int8_gemm.fuse_act(_Layer(_use_convrot=False), x, 512)
    assert not int8_gemm.fuse_act(_Layer(_convrot_groupsize=128), x, 512)
    assert not int8_gemm.fuse_act(_Layer(lora_patches=["l"]), x, 512)
    assert not int8_gemm.fuse_act(_Layer(), x.float(), 512)
    assert not int8_gemm.fuse_act(_Layer(), x, 256)
    assert not int8_gemm.fuse_act(_Layer(in_features=384), x, 384)
    assert not int8_gemm.fuse_act(_Layer(in_features=32768), x, 32768)


def test_linear_input_act_situ_routing(monkeypatch):
    comfy, _ = fakes.install(monkeypatch)
    int8_gemm.enable(True)
    layer = _Layer(in_features=256)
    calls = []
    linear = lambda x: calls.append(int8_gemm.situ_next) or "fused"  # noqa: E731
    linear.__dict__.update(layer.__dict__)
    x = torch.zeros(2, 512, dtype=torch.float16)
    assert int8_gemm.linear_input_act(linear, x, "situ") == "fused" and calls == [True]
    assert int8_gemm.linear_input_act(linear, x, "gelu") == "original-input-act"
    assert int8_gemm.linear_input_act(linear, x, "situ", residual=x) == "original-input-act"


def test_block_forward_resets_state_on_error(monkeypatch):
    """block_forward's finally clears the side channel even when a step raises."""
    fakes.install(monkeypatch)
    int8_gemm.enable(True)

    class Block:
        pass

    class Attn:
        headdim, heads, kvheads = 128, 2, 2

    mod = Block()
    mod.attn, mod.mlp = Attn(), Block()
    Linear = int8_gemm.originals["layer"]
    layers = [Linear(256, 256) for _ in range(8)]
    mod.attn.wq, mod.attn.wk, mod.attn.wv, mod.attn.gate, mod.attn.wo = layers[:5]
    mod.mlp.gate, mod.mlp.up, mod.mlp.down = layers[5:]
    monkeypatch.setattr(int8_gemm, "swiglu_fusable", True)
    mod.mod = lambda vec: (torch.zeros(1, 256, dtype=torch.float16),) * 6
    mod.prenorm = mod.postnorm = None

    def boom(*a):
        int8_gemm.shared = ("x", "y")
        int8_gemm.residual = ("r", "g")
        raise RuntimeError("kernel failed")

    monkeypatch.setattr(int8_gemm, "quantize_block_input", boom)
    x = torch.zeros(1, 600, 256, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="kernel failed"):
        int8_gemm.block_forward(mod, False, x, None, torch.zeros(1))
    assert int8_gemm.shared is None and int8_gemm.residual is None and int8_gemm.swiglu_up is None and int8_gemm.sigmoid_gate is None


def test_block_forward_falls_back_when_not_fusable(monkeypatch):
    fakes.install(monkeypatch)
    called = []

    class SSB:
        @staticmethod
        def forward(module, *args):
            called.append(args)
            return "unfused"

    monkeypatch.setattr(int8_gemm, "SingleStreamBlock", SSB)
    mod = type("M", (), {})()
    mod.attn, mod.mlp = type("A", (), {"headdim": 128})(), type("P", (), {})()
    assert int8_gemm.block_forward(mod, False, torch.zeros(1, 600, 8, dtype=torch.float16), "vec", None) == "unfused"


def test_attention_hip_falls_back_to_bmm(monkeypatch):
    """Ineligible inputs (fp32, head dim 64) take attention_bmm, which matches the float64 softmax on the CPU."""
    g = torch.Generator().manual_seed(0)
    for dtype, heads, d in ((torch.float32, 2, 128), (torch.float16, 4, 64)):
        q, k, v = (torch.randn(1, 50, heads * d, generator=g).to(dtype) for _ in range(3))
        if dtype == torch.float16:
            q, k, v = q.float(), k.float(), v.float()
        out = attention.attention_hip(q, k, v, heads)
        th = lambda t: t.reshape(1, 50, heads, d).transpose(1, 2).double().numpy()  # noqa: E731
        ref = oracle.attention_f64(th(q), th(k), th(v), d ** -0.5)
        got = out.reshape(1, 50, heads, d).transpose(1, 2).double().numpy()
        assert np.abs(got - ref).max() < 1e-5


def test_attention_bmm_chunks(monkeypatch):
    monkeypatch.setattr(attention, "BMM_CHUNK_BYTES", 50 * 60 * 4 * 2)  # two heads per chunk
    g = torch.Generator().manual_seed(1)
    q = torch.randn(2, 3, 50, 16, generator=g)
    k = torch.randn(2, 3, 60, 16, generator=g)
    v = torch.randn(2, 3, 60, 16, generator=g)
    out = attention.attention_bmm(q, k, v, 3, skip_reshape=True, skip_output_reshape=True, scale=0.3)
    ref = oracle.attention_f64(q.numpy(), k.numpy(), v.numpy(), 0.3)
    assert np.abs(out.double().numpy() - ref).max() < 1e-5


def test_rms_norm_forward_eligibility(monkeypatch):
    calls = []

    class RMS:
        @staticmethod
        def forward(module, x):
            calls.append(x)
            return "original"

    monkeypatch.setattr(rms_norm, "RMSNorm", RMS)
    for x in (torch.zeros(2, 4, 64), torch.zeros(2, 64, dtype=torch.float16), torch.zeros(2, 4, 12, dtype=torch.float16),
              torch.zeros(2, 4, 16384, dtype=torch.float16), torch.zeros(2, 64, 4, dtype=torch.float16).transpose(1, 2)):
        assert rms_norm.forward(None, x) == "original"
    assert len(calls) == 5
    assert rms_norm.eligible(torch.zeros(1, 4, 3072, dtype=torch.float16))


def test_gemv_linear_forward_eligibility(monkeypatch):
    class Lin:
        weight_function = bias_function = None

        @staticmethod
        def forward(module, x, *a, **k):
            return "original"

    m = Lin()
    m.__class__ = type("Linear", (Lin,), {})
    assert int8_gemv.linear_forward(m, 64, 512, None, 0, torch.zeros(1, 512, dtype=torch.float16)) == "original"  # not fp32
    assert int8_gemv.linear_forward(m, 64, 512, None, 0, torch.zeros(3, 512)) == "original"  # prefill outside generate()
    m.weight_function = ["patch"]
    assert int8_gemv.linear_forward(m, 64, 512, None, 0, torch.zeros(1, 512)) == "original"  # patched (LoRA)


def test_launch_shim_ignores_reference_grid():
    """launch() keeps the reference's signature: grid, block and LDS size are accepted and left to the library."""
    import inspect
    assert list(inspect.signature(hip_attention.launch).parameters) == ["func", "grid_x", "grid_y", "block", "args", "shared"]
    with pytest.raises(RuntimeError, match="HIP error 7"):
        hip_attention.check(7)


def test_init_kv_cache_layout(monkeypatch):
    """init_kv_cache (int8_gemv.py:117-126): one fixed-capacity (batch, capacity, kv heads, 128) K and V per layer,
    all layers sharing the position and the int32 length tensors that the decode kernels read on the device."""
    import collections
    FixedKV = collections.namedtuple("FixedKV", "key value index position length")
    monkeypatch.setattr(int8_gemv, "FixedKV", FixedKV)
    model = types.SimpleNamespace(config=types.SimpleNamespace(num_hidden_layers=3, num_key_value_heads=8))
    caches = int8_gemv.init_kv_cache(model, 2, 64, torch.device("cpu"), torch.float32)
    assert len(caches) == 3
    for c in caches:
        assert c.key.shape == c.value.shape == (2, 64, 8, 128) and c.key.dtype == torch.float32 and c.index == 0
        assert c.key.data_ptr() != c.value.data_ptr()
        assert c.position is caches[0].position and c.length is caches[0].length
    assert caches[0].length.dtype == torch.int32 and int(caches[0].length.abs().sum()) == 0
