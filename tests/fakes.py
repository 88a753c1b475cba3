"""Stand-ins for the ComfyUI and ComfyUI-INT8-Fast-ROCM objects the hooks touch, so that the hook logic (discovery,
eligibility, fallbacks, side-channel state) is testable on the CPU. Each fake records its calls."""
import sys
import types

import torch
import torch.nn.functional as F


class Recorder:
    def __init__(self, name, result=None):
        self.name, self.calls, self.result = name, [], result

    def __call__(self, *args, **kwargs):
        self.calls.append((args, kwargs))
        if callable(self.result):
            return self.result(*args, **kwargs)
        return self.result


def make_pack(triton=True, real=False):
    """A fake INT8-Fast-ROCM: int8_quant, int4_quant and convrot modules under a package prefix. With real, its Linear
    holds an int8 weight and a per-channel scale and its forward does what the plugin's does -- ConvRot, then
    triton_int8_linear -- looking both up in their modules at call time, so installed hooks take effect."""
    int8_quant = types.ModuleType("fakepack.int8_quant")

    def triton_int8_linear(x, weight, weight_scale, bias=None, compute_dtype=torch.float16, x_q=None):
        return F.linear(x.float(), weight.float() * torch.as_tensor(weight_scale).float().reshape(-1, 1)).to(compute_dtype)

    int8_quant.triton_int8_linear = Recorder("triton_int8_linear", triton_int8_linear)
    int8_quant.triton_int8_linear_per_row = Recorder("triton_int8_linear_per_row", triton_int8_linear)
    int8_quant._TRITON_AVAILABLE = triton

    class Linear(torch.nn.Module):
        def __init__(self, in_features=256, out_features=64):
            super().__init__()
            self.in_features, self.out_features = in_features, out_features
            self.lora_patches = []
            self._is_quantized = True
            self._use_convrot = True
            self._convrot_groupsize = 256
            self.bias = None

        def forward(self, x):
            if not real:
                return x
            convrot = sys.modules["fakepack.convrot"]
            H = convrot.build_hadamard(self._convrot_groupsize, device=x.device, dtype=x.dtype)
            x = convrot.rotate_activation(x, H, self._convrot_groupsize)
            return sys.modules["fakepack.int8_quant"].triton_int8_linear(x, self.weight, self.weight_scale, self.bias, torch.float16)

    int8_quant.Int8TensorwiseOps = types.SimpleNamespace(Linear=Linear)
    int4_quant = types.ModuleType("fakepack.int4_quant")
    int4_quant.convrot_w4a4_forward = Recorder("convrot_w4a4_forward", lambda x, *a, **k: "original-w4a4")
    convrot = types.ModuleType("fakepack.convrot")
    convrot.rotate_activation = Recorder("rotate_activation", lambda x, H, g: x * 2)
    convrot.build_hadamard = Recorder("build_hadamard", lambda n, device=None, dtype=None: torch.eye(n, dtype=dtype))
    if real:  # built once, not recorded: a block calls it for every linear, and the recorder would keep every copy
        eye = {}

        def build_hadamard(n, device=None, dtype=None):
            if (n, device, dtype) not in eye:
                eye[n, device, dtype] = torch.eye(n, dtype=dtype, device=device)
            return eye[n, device, dtype]

        convrot.build_hadamard = build_hadamard
    return {"fakepack.int8_quant": int8_quant, "fakepack.int4_quant": int4_quant, "fakepack.convrot": convrot}


def make_comfy():
    comfy = types.ModuleType("comfy")
    ops = types.ModuleType("comfy.ops")
    ops.linear_input_act = Recorder("linear_input_act", lambda linear, x, *a, **k: "original-input-act")
    ops._eager_input_act = Recorder("_eager_input_act", lambda x, act: x[..., : x.shape[-1] // 2] * 3)
    mm = types.ModuleType("comfy.model_management")
    mm.cast_to = lambda t, dtype=None, device=None: t.to(dtype=dtype, device=device)
    comfy.ops, comfy.model_management = ops, mm
    return comfy


def install(monkeypatch, pack=True, triton=True, real=False):
    """Puts the fake modules into sys.modules and the product modules' globals. Returns (comfy, pack modules)."""
    from comfyui_rdna2_attention_amd import int8_gemm, rms_norm
    comfy = make_comfy()
    mods = make_pack(triton, real) if pack else {}
    for name, mod in mods.items():
        monkeypatch.setitem(sys.modules, name, mod)
    monkeypatch.setattr(int8_gemm, "comfy", comfy)
    monkeypatch.setattr(rms_norm, "comfy", comfy)
    monkeypatch.setattr(int8_gemm, "originals", {})
    for name in ("fusable", "situ_next", "swiglu_fusable"):
        monkeypatch.setattr(int8_gemm, name, False)
    for name in ("pending", "swiglu_up", "sigmoid_gate", "shared", "residual"):
        monkeypatch.setattr(int8_gemm, name, None)
    return comfy, mods


class _Norm:
    def __init__(self, scale, eps):
        self.scale, self.eps = scale, eps


def make_krea2_block(layer_cls, D, heads, hidden, B, device, seed=0):
    """A Krea 2 SingleStreamBlock stand-in with the attributes block_forward reads: attn (wq, wk, wv, gate, wo of
    int8 layers, heads = kvheads, headdim 128, qknorm), mlp (gate, up, down), prenorm / postnorm and mod(vec) -> six
    (B, 1, D) fp16 modulation tensors. Weights are int8 uniform in [-127, 127] with per-channel scales ~U(1e-3, 3e-3)
    (the W8A8 linear configuration); norm gains ~N(1, 0.1) stored zero-centred."""
    g = torch.Generator().manual_seed(seed)

    def layer(k, n):
        m = layer_cls(k, n)
        m.weight = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).to(device)
        m.weight_scale = (torch.rand(n, generator=g) * 2e-3 + 1e-3).float().to(device)
        return m

    def norm(d):
        return _Norm((torch.randn(d, generator=g) * 0.1).float().to(device), 1e-6)

    blk = types.SimpleNamespace()
    blk.attn = types.SimpleNamespace(heads=heads, kvheads=heads, headdim=128, wq=layer(D, D), wk=layer(D, D), wv=layer(D, D), gate=layer(D, D),
                                     wo=layer(D, D), qknorm=types.SimpleNamespace(qnorm=norm(128), knorm=norm(128)))
    blk.mlp = types.SimpleNamespace(gate=layer(D, hidden), up=layer(D, hidden), down=layer(hidden, D))
    blk.prenorm, blk.postnorm = norm(D), norm(D)
    mods = [(torch.randn(B, 1, D, generator=g) * 0.2).half().to(device) for _ in range(6)]
    blk.mod = lambda vec: tuple(mods)
    return blk
