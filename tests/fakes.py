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


def make_pack(triton=True):
    """A fake INT8-Fast-ROCM: int8_quant, int4_quant and convrot modules under a package prefix."""
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
            return x

    int8_quant.Int8TensorwiseOps = types.SimpleNamespace(Linear=Linear)
    int4_quant = types.ModuleType("fakepack.int4_quant")
    int4_quant.convrot_w4a4_forward = Recorder("convrot_w4a4_forward", lambda x, *a, **k: "original-w4a4")
    convrot = types.ModuleType("fakepack.convrot")
    convrot.rotate_activation = Recorder("rotate_activation", lambda x, H, g: x * 2)
    convrot.build_hadamard = Recorder("build_hadamard", lambda n, device=None, dtype=None: torch.eye(n, dtype=dtype))
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


def install(monkeypatch, pack=True, triton=True):
    """Puts the fake modules into sys.modules and the product modules' globals. Returns (comfy, pack modules)."""
    from comfyui_rdna2_attention_amd import int8_gemm, rms_norm
    comfy = make_comfy()
    mods = make_pack(triton) if pack else {}
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
