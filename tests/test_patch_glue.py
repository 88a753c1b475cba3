"""The model-patch glue and the node shim on the CPU, with stand-ins for the ComfyUI objects they touch: which object
patches each patch() installs (and on which modules it does not), the fallbacks each patched forward takes, the
generate() scope, the merged gate/up prefill of mlp_forward, and RDNA2Attention.execute / RDNA2TextGenerate.execute
with relayout_weights (reference: int8_gemv.py:67-148, rms_norm.py:61-64, int8_gemm.py:160-173, 229-232,
__init__.py:22-93)."""
import importlib.util
import logging
import sys
import types

import pytest
import torch
import torch.nn.functional as F

import __graft_entry__
from comfyui_rdna2_attention_amd import int8_gemm, int8_gemv, rms_norm


class Patcher:
    """Records add_object_patch calls; model holds the module tree."""

    def __init__(self, model):
        self.model, self.patches, self.callbacks = model, {}, []

    def add_object_patch(self, name, obj):
        self.patches[name] = obj

    def get_model_object(self, name):
        return getattr(self.model, name)


def named(root, tree):
    """A module tree whose named_modules() yields `tree` (name -> module) under `root`."""
    root.named_modules = lambda: [("", root), *tree.items()]
    return root


# ----------------------------------------------------------------------------------------------- int8_gemv.patch

class MixedPrecisionOp:
    pass


class Linear(MixedPrecisionOp):
    def __init__(self, N, K, fmt="int8_tensorwise", scale_n=None, scale_dtype=torch.float32, transposed=False, convrot=False, group=256):
        self.quant_format = fmt
        self.weight = types.SimpleNamespace(shape=(N, K), dtype=torch.int8, _params=types.SimpleNamespace(
            scale=torch.ones(scale_n or N, dtype=scale_dtype), transposed=transposed, convrot=convrot, convrot_groupsize=group))
        self.weight_function = self.bias_function = None


class MLP:
    def __init__(self, merged=False):
        self.merged_mlp = merged
        self.gate_proj, self.up_proj = Linear(64, 512), Linear(64, 512)


class BaseQwen3:
    def __init__(self, lm_head=False, fixed_kv=True, heads=32, kv_heads=8, head_dim=128, embed_dtype=torch.bfloat16, vocab=1024, hidden=512):
        cfg = types.SimpleNamespace(lm_head=lm_head, head_dim=head_dim, num_attention_heads=heads, num_key_value_heads=kv_heads)
        embed = types.SimpleNamespace(weight=torch.zeros(vocab, hidden, dtype=embed_dtype))
        self.model = types.SimpleNamespace(config=cfg, fixed_kv=fixed_kv, embed_tokens=embed)


@pytest.fixture
def gemv_fakes(monkeypatch):
    kitchen = types.SimpleNamespace(flash_attention_decode="kitchen-original")
    monkeypatch.setattr(int8_gemv, "comfy_kitchen", kitchen)
    monkeypatch.setattr(int8_gemv, "MixedPrecisionOp", MixedPrecisionOp)
    monkeypatch.setattr(int8_gemv, "MLP", MLP)
    monkeypatch.setattr(int8_gemv, "BaseQwen3", BaseQwen3)
    return kitchen


def test_int8_gemv_patch_installs_eligible_objects(gemv_fakes):
    tree = {
        "ok": Linear(4096, 4096, convrot=True, group=256),
        "ok_plain": Linear(1024, 512),
        "bad_rows": Linear(4100, 512),  # N % 16
        "bad_k": Linear(64, 500),  # K % 512
        "bad_scale_count": Linear(64, 512, scale_n=1),
        "bad_scale_dtype": Linear(64, 512, scale_dtype=torch.float16),
        "bad_transposed": Linear(64, 512, transposed=True),
        "bad_format": Linear(64, 512, fmt="float8"),
        "mlp": MLP(),
        "mlp_merged": MLP(merged=True),
        "attn": types.SimpleNamespace(q_proj=Linear(512, 512), k_proj=Linear(128, 512), v_proj=Linear(128, 512)),
        "attn_mixed": types.SimpleNamespace(q_proj=Linear(512, 512), k_proj=Linear(128, 512, convrot=True), v_proj=Linear(128, 512)),
        "qwen": BaseQwen3(),
        "qwen_lm_head": BaseQwen3(lm_head=True),
    }
    clip = types.SimpleNamespace(patcher=Patcher(named(types.SimpleNamespace(), tree)))
    int8_gemv.forget_siblings()
    int8_gemv.patch(clip)
    p = clip.patcher.patches
    assert set(p) == {"ok.forward", "ok_plain.forward", "mlp.forward", "qwen.logits", "qwen.generate", "qwen.model.init_kv_cache"}
    # siblings: q/k/v and gate/up of one parent with one K, weight dtype and ConvRot group (not the mixed-group set)
    attn, mixed = tree["attn"], tree["attn_mixed"]
    assert int8_gemv._siblings_of(attn.k_proj).modules() == [attn.q_proj, attn.k_proj, attn.v_proj]
    assert int8_gemv._siblings_of(tree["mlp"].up_proj).modules() == [tree["mlp"].gate_proj, tree["mlp"].up_proj]
    assert all(int8_gemv._siblings_of(m) is None for m in (mixed.q_proj, mixed.k_proj, tree["ok"]))
    int8_gemv.forget_siblings()
    assert p["ok.forward"].func is int8_gemv.linear_forward and p["ok.forward"].args == (tree["ok"], 4096, 4096, torch.int8, 256)
    assert p["ok_plain.forward"].args[-1] == 0  # no ConvRot: group 0
    assert p["mlp.forward"].func is int8_gemv.mlp_forward and p["mlp.forward"].args == (tree["mlp"], torch.int8)
    assert p["qwen.logits"].func is int8_gemv.logits and p["qwen.generate"].func is int8_gemv.generate
    assert p["qwen.model.init_kv_cache"].func is int8_gemv.init_kv_cache
    assert gemv_fakes.flash_attention_decode is int8_gemv.attention_decode


@pytest.mark.parametrize("kw", [{"fixed_kv": False}, {"head_dim": 64}, {"heads": 16}])
def test_int8_gemv_patch_keeps_kitchen_decode_when_ineligible(gemv_fakes, kw):
    clip = types.SimpleNamespace(patcher=Patcher(named(types.SimpleNamespace(), {"qwen": BaseQwen3(**kw)})))
    int8_gemv.patch(clip)
    assert set(clip.patcher.patches) == {"qwen.logits", "qwen.generate"}
    assert gemv_fakes.flash_attention_decode == "kitchen-original"


def test_int8_gemv_patch_logits_needs_bf16_table(gemv_fakes):
    clip = types.SimpleNamespace(patcher=Patcher(named(types.SimpleNamespace(), {"qwen": BaseQwen3(embed_dtype=torch.float16, fixed_kv=False)})))
    int8_gemv.patch(clip)
    assert set(clip.patcher.patches) == {"qwen.generate"}


def test_generate_scopes_the_flag():
    seen = []

    class T:
        def generate(self, *a, **k):
            seen.append((int8_gemv.generating, a, k))
            if k.get("fail"):
                raise ValueError("stop")
            return "tokens"

    assert int8_gemv.generate(T(), 1, max_new=2) == "tokens"
    with pytest.raises(ValueError):
        int8_gemv.generate(T(), fail=True)
    assert seen[0] == (True, (1,), {"max_new": 2}) and seen[1][0] is True and int8_gemv.generating is False


class QTensor:
    """A quantized weight whose dequantize() gives W * scale, as comfy's int8 QuantizedTensor does."""

    def __init__(self, w, scale):
        self.w, self.scale = w, scale

    def to(self, dtype=None):
        return QTensor(self.w, self.scale) if dtype is None else types.SimpleNamespace(dequantize=lambda: self.w.to(dtype) * self.scale.to(dtype)[:, None])


def cast_context(monkeypatch):
    calls = []

    class CastBiasWeightContext:
        def __init__(self, module, **kw):
            self.module, self.kw = module, kw
            calls.append(kw)

        def __enter__(self):
            return self.module.qweight, getattr(self.module, "bias", None)

        def __exit__(self, *a):
            return False

    monkeypatch.setattr(int8_gemv, "comfy", types.SimpleNamespace(ops=types.SimpleNamespace(CastBiasWeightContext=CastBiasWeightContext)))
    return calls


def test_mlp_forward_merges_gate_and_up(monkeypatch):
    calls = cast_context(monkeypatch)
    g = torch.Generator().manual_seed(5)
    K, N = 64, 96
    wg, wu = (torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8) for _ in range(2))
    sg, su = (torch.rand(N, generator=g) * 1e-2 for _ in range(2))

    class Module:
        def __init__(self):
            self.gate_proj = types.SimpleNamespace(qweight=QTensor(wg, sg), weight_function=None, bias_function=None)
            self.up_proj = types.SimpleNamespace(qweight=QTensor(wu, su), weight_function=None, bias_function=None)
            self.activation = F.silu
            self.down_proj = lambda h: h * 2

        def forward(self, x, norm=None):
            return "original"

    m = Module()
    x = torch.randn(3, K, generator=g)
    monkeypatch.setattr(int8_gemv, "generating", True)
    out = int8_gemv.mlp_forward(m, torch.int8, x)
    ref = 2 * F.silu(x @ (wg.float() * sg[:, None]).T) * (x @ (wu.float() * su[:, None]).T)
    assert torch.allclose(out, ref, rtol=1e-5, atol=1e-5)
    assert len(calls) == 2 and all(c["want_requant"] and c["dtype"] is torch.int8 for c in calls)
    # Fallbacks: outside generate(), a norm argument, fp16 x, one token, patched layers.
    monkeypatch.setattr(int8_gemv, "generating", False)
    assert int8_gemv.mlp_forward(m, torch.int8, x) == "original"
    monkeypatch.setattr(int8_gemv, "generating", True)
    assert int8_gemv.mlp_forward(m, torch.int8, x, norm="n") == "original"
    assert int8_gemv.mlp_forward(m, torch.int8, x.half()) == "original"
    assert int8_gemv.mlp_forward(m, torch.int8, x[:1]) == "original"
    m.up_proj.weight_function = ["lora"]
    assert int8_gemv.mlp_forward(m, torch.int8, x) == "original"


def test_logits_fallbacks(monkeypatch):
    class T:
        def __init__(self, dtype=torch.bfloat16):
            self.model = types.SimpleNamespace(embed_tokens=types.SimpleNamespace(weight_function=None))

        def logits(self, x):
            return "original"

    t = T()
    assert int8_gemv.logits(t, torch.zeros(2, 3, 8)) == "original"  # batch of 2
    assert int8_gemv.logits(t, torch.zeros(1, 3, 8, dtype=torch.float16)) == "original"
    t.model.embed_tokens.weight_function = ["patch"]
    assert int8_gemv.logits(t, torch.zeros(1, 3, 8)) == "original"


def test_linear_forward_prefill_uses_dequantized_matmul_only_inside_generate(monkeypatch):
    """Several tokens with a ConvRot group above 256: the dequantized matmul inside generate(), the layer's own forward
    outside it (int8_gemv.py:48-64); the rotation is a GPU kernel, so without a GPU the eligible call raises."""
    class Lin:
        weight_function = bias_function = None

        @staticmethod
        def forward(module, x, *a, **k):
            return "original"

    m = Lin()
    m.__class__ = type("Linear", (Lin,), {})
    x = torch.zeros(3, 1024)
    assert int8_gemv.linear_forward(m, 64, 1024, torch.int8, 1024, x) == "original"  # outside generate()
    monkeypatch.setattr(int8_gemv, "generating", True)
    assert int8_gemv.linear_forward(m, 64, 1024, torch.int8, 256, x) == "original"  # group <= 256: kitchen's fast dequantize
    if torch.cuda.is_available():
        return
    cast_context(monkeypatch)
    m.qweight = types.SimpleNamespace(_qdata=torch.zeros(64, 1024, dtype=torch.int8), _params=types.SimpleNamespace(scale=torch.ones(64)))
    monkeypatch.setattr(int8_gemv, "kernels", None)
    monkeypatch.setattr(int8_gemv._lib, "_lib", None)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        int8_gemv.linear_forward(m, 64, 1024, torch.int8, 1024, x)


# ------------------------------------------------------------------------------------ rms_norm / int8_gemm patches

def diffusion_model(tree):
    dm = named(types.SimpleNamespace(), tree)
    return Patcher(types.SimpleNamespace(diffusion_model=dm))


def test_rms_norm_patch(monkeypatch):
    class RMSNorm:
        pass

    monkeypatch.setattr(rms_norm, "RMSNorm", RMSNorm)
    a, b = RMSNorm(), RMSNorm()
    m = diffusion_model({"blocks.0.norm": a, "blocks.0.other": object(), "blocks.1.norm": b})
    rms_norm.patch(m)
    assert set(m.patches) == {"diffusion_model.blocks.0.norm.forward", "diffusion_model.blocks.1.norm.forward"}
    p = m.patches["diffusion_model.blocks.1.norm.forward"]
    assert p.func is rms_norm.forward and p.args == (b,)


def test_patch_swiglu_and_patch_block(monkeypatch):
    class SwiGLU:
        pass

    class SingleStreamBlock:
        pass

    monkeypatch.setattr(int8_gemm, "SwiGLU", SwiGLU)
    monkeypatch.setattr(int8_gemm, "SingleStreamBlock", SingleStreamBlock)
    s, blk = SwiGLU(), SingleStreamBlock()
    m = diffusion_model({"b.0.mlp": s, "b.0": blk, "b.0.attn": object()})
    int8_gemm.patch_swiglu(m)
    assert set(m.patches) == {"diffusion_model.b.0.mlp.forward"}
    assert m.patches["diffusion_model.b.0.mlp.forward"].func is int8_gemm.swiglu_forward
    int8_gemm.patch_block(m, True)
    p = m.patches["diffusion_model.b.0.forward"]
    assert p.func is int8_gemm.block_forward and p.args == (blk, True)


def test_swiglu_forward_routes(monkeypatch):
    import fakes
    fakes.install(monkeypatch)
    int8_gemm.enable(True)
    Layer = int8_gemm.originals["layer"]
    seen = []

    class Down(Layer):
        def __call__(self, x):
            seen.append((x, int8_gemm.swiglu_up))
            return x

    g = torch.Generator().manual_seed(3)
    gate_x = torch.randn(4, 256, generator=g).half()
    up_x = torch.randn(4, 256, generator=g).half()
    module = types.SimpleNamespace(gate=lambda x: gate_x, up=lambda x: up_x, down=Down(256, 64))
    # Fusable: down receives the raw gate, the up projection waits in the side channel.
    int8_gemm.swiglu_forward(module, None)
    assert seen[-1][0] is gate_x and seen[-1][1] is up_x
    monkeypatch.setattr(int8_gemm, "swiglu_up", None)
    # Not fusable (no Triton path, a LoRA'd down, or not an Int8 layer): silu(gate) * up in torch.
    monkeypatch.setattr(int8_gemm, "swiglu_fusable", False)
    int8_gemm.swiglu_forward(module, None)
    assert torch.equal(seen[-1][0], F.silu(gate_x) * up_x) and seen[-1][1] is None
    monkeypatch.setattr(int8_gemm, "swiglu_fusable", True)
    module.down.lora_patches = ["lora"]
    int8_gemm.swiglu_forward(module, None)
    assert torch.equal(seen[-1][0], F.silu(gate_x) * up_x)
    module.down = lambda x: ("plain", x)
    assert int8_gemm.swiglu_forward(module, None)[0] == "plain"


# ---------------------------------------------------------------------------------------------------- node shim

def comfy_stubs():
    """Stand-ins for the ComfyUI modules the node shim imports (comfy.patcher_extension, comfy.quant_ops,
    comfy_api.latest)."""
    comfy = types.ModuleType("comfy")
    pe = types.ModuleType("comfy.patcher_extension")
    pe.CallbacksMP = types.SimpleNamespace(ON_PRE_RUN="on_pre_run")
    qo = types.ModuleType("comfy.quant_ops")

    class QuantizedTensor(torch.Tensor):
        pass

    qo.QuantizedTensor = QuantizedTensor
    api = types.ModuleType("comfy_api")
    latest = types.ModuleType("comfy_api.latest")

    def field(kind):
        return types.SimpleNamespace(Input=lambda *a, **k: (kind, a, k), Output=lambda *a, **k: (kind, a, k))

    latest.io = types.SimpleNamespace(ComfyNode=object, Schema=lambda **k: k, NodeOutput=lambda *a: a, Model=field("model"),
                                      Combo=field("combo"), Boolean=field("bool"), Clip=field("clip"))
    latest.ComfyExtension = object
    comfy.patcher_extension, comfy.quant_ops = pe, qo
    return {"comfy": comfy, "comfy.patcher_extension": pe, "comfy.quant_ops": qo, "comfy_api": api, "comfy_api.latest": latest}


@pytest.fixture
def shim(monkeypatch):
    """The package loaded afresh, under its own name, with the ComfyUI stand-ins importable: the node classes exist."""
    for name, mod in comfy_stubs().items():
        monkeypatch.setitem(sys.modules, name, mod)
    name = "rda_node_shim"
    spec = importlib.util.spec_from_file_location(name, __graft_entry__.PKG_DIR + "/__init__.py", submodule_search_locations=[__graft_entry__.PKG_DIR])
    pkg = importlib.util.module_from_spec(spec)
    monkeypatch.setitem(sys.modules, name, pkg)
    spec.loader.exec_module(pkg)
    yield pkg
    for key in [k for k in sys.modules if k.startswith(name + ".")]:
        del sys.modules[key]


class Model:
    def __init__(self, dynamic=False, tree=None):
        self.dynamic, self.calls, self.patches, self.callbacks = dynamic, [], {}, []
        self.model = types.SimpleNamespace(diffusion_model=named(types.SimpleNamespace(), tree or {}))

    def clone(self):
        self.calls.append("clone")
        return self

    def set_model_optimized_attention(self, fn):
        self.calls.append(("attention", fn))

    def add_object_patch(self, name, obj):
        self.patches[name] = obj

    def get_model_object(self, name):
        return getattr(self.model, name)

    def is_dynamic(self):
        return self.dynamic

    def add_callback(self, kind, fn):
        self.callbacks.append((kind, fn))


def test_node_schemas(shim):
    s = shim.RDNA2Attention.define_schema()
    assert s["node_id"] == "RDNA2Attention"
    names = [i[1][0] for i in s["inputs"]]
    assert names == ["model", "backend", "transpose_weights", "int8_gemm", "fused_norm", "fused_swiglu"]
    assert s["inputs"][1][2]["options"] == ["hip", "hip_int8", "bmm"] and s["inputs"][1][2]["default"] == "hip"
    assert shim.RDNA2TextGenerate.define_schema()["node_id"] == "RDNA2TextGenerate"
    import asyncio
    ext = asyncio.run(shim.comfy_entrypoint())
    assert asyncio.run(ext.get_node_list()) == [shim.RDNA2Attention, shim.RDNA2TextGenerate]


def test_execute_call_sequence(shim, monkeypatch, caplog):
    events = []
    monkeypatch.setattr(shim.int8_kernels, "enable", lambda on: events.append(("enable", on)))
    monkeypatch.setattr(shim.rms_norm, "patch", lambda m: events.append("rms_norm.patch"))
    monkeypatch.setattr(shim.int8_kernels, "patch_swiglu", lambda m: events.append("patch_swiglu"))
    monkeypatch.setattr(shim.int8_kernels, "patch_block", lambda m, q: events.append(("patch_block", q)))
    m = Model()
    out = shim.RDNA2Attention.execute(m, "hip")
    assert out == (m,) and m.calls == ["clone", ("attention", shim.attention_hip)] and events == [("enable", False)]
    events.clear()
    shim.RDNA2Attention.execute(Model(), "hip_int8", int8_gemm=True, fused_norm=True, fused_swiglu=True)
    assert events == [("enable", True), "rms_norm.patch", "patch_swiglu", ("patch_block", True)]
    events.clear()
    m = Model()
    shim.RDNA2Attention.execute(m, "bmm", fused_norm=True, fused_swiglu=True)  # no fused block without a hip backend
    assert events == [("enable", False), "rms_norm.patch", "patch_swiglu"] and m.calls[1] == ("attention", shim.attention_bmm)
    m = Model()
    shim.RDNA2Attention.execute(m, "hip", transpose_weights=True)
    assert m.callbacks == [("on_pre_run", shim.relayout_weights)]
    m = Model(dynamic=True)
    with caplog.at_level(logging.WARNING):
        shim.RDNA2Attention.execute(m, "hip", transpose_weights=True)
    assert m.callbacks == [] and "transpose_weights skipped" in caplog.text


def test_text_generate_execute(shim, monkeypatch):
    seen = []
    monkeypatch.setattr(shim.int8_gemv, "patch", lambda clip: seen.append(clip))
    clip = Model()
    assert shim.RDNA2TextGenerate.execute(clip) == (clip,) and seen == [clip] and clip.calls == ["clone"]


def test_relayout_weights(shim):
    """fp16 Linear weights of at least 1024 x 1024 off the CPU become K-major (same shape and values); CPU, small,
    quantized, non-fp16 and already K-major weights are left alone. The meta device stands in for the GPU."""
    big = torch.nn.Linear(1024, 2048, bias=False, device="meta", dtype=torch.float16)
    small = torch.nn.Linear(512, 2048, bias=False, device="meta", dtype=torch.float16)
    fp32 = torch.nn.Linear(1024, 1024, bias=False, device="meta")
    cpu = torch.nn.Linear(1024, 1024, bias=False, dtype=torch.float16)
    tree = types.SimpleNamespace(modules=lambda: [big, small, fp32, cpu, torch.nn.ReLU()])
    patcher = types.SimpleNamespace(model=types.SimpleNamespace(diffusion_model=tree))
    strides = [m.weight.stride() for m in (small, fp32, cpu)]
    shim.relayout_weights(patcher)
    assert big.weight.shape == (2048, 1024) and big.weight.stride() == (1, 2048)
    assert [m.weight.stride() for m in (small, fp32, cpu)] == strides
    shim.relayout_weights(patcher)  # already K-major: unchanged
    assert big.weight.stride() == (1, 2048)


def test_package_without_comfyui_defines_no_nodes():
    pkg = sys.modules[__graft_entry__.PKG_NAME]
    assert pkg.io is None and not hasattr(pkg, "RDNA2Attention")


def _gemv_layer(N, K):
    m = types.SimpleNamespace(weight_function=None, bias_function=None)
    m.qweight = types.SimpleNamespace(_qdata=torch.zeros(N, K, dtype=torch.int8), _params=types.SimpleNamespace(scale=torch.ones(N)))
    return m


def _record_gemv_kernels(monkeypatch, calls):
    """Stand-ins for the GEMV launches (no GPU here): each records its call and the sum of the input it saw, and
    returns outputs that name the call (value = number of the call) so that a stale hand-out is visible."""
    def out(n):
        return torch.full((n,), float(len(calls)))

    def multi(x, layers, group=0, rotated=None):
        calls.append(("multi", group, float(x.sum()), tuple(w.shape[0] for w, _, _ in layers)))
        return [out(w.shape[0]) for w, _, _ in layers]

    monkeypatch.setattr(int8_gemv, "gemv_multi", multi)
    monkeypatch.setattr(int8_gemv, "rotate_gemv", lambda x, group, w, s, b=None, rotated=None: calls.append(("fused", group, float(x.sum()))) or out(w.shape[0]))
    monkeypatch.setattr(int8_gemv, "rotate", lambda x, group: calls.append(("rotate", group, x.shape[-1])) or x * 2)
    monkeypatch.setattr(int8_gemv, "gemv", lambda x, w, s, b=None: calls.append(("gemv", float(x.sum()), w.shape[1])) or out(w.shape[0]))


def test_sibling_linears_run_in_one_launch(monkeypatch):
    """q, k and v registered as siblings: the first call runs all three in one gemv_multi launch and k and v receive
    its outputs; a new input object, an in-place write (version counter), an interleaved other linear, a repeated
    call and generate() all make the next sibling compute afresh, never a stale output."""
    cast_context(monkeypatch)
    calls = []
    _record_gemv_kernels(monkeypatch, calls)
    int8_gemv.forget_siblings()
    K = 4096
    q, k, v, o = _gemv_layer(4096, K), _gemv_layer(1024, K), _gemv_layer(1024, K), _gemv_layer(4096, K)
    int8_gemv.register_siblings([(q, 4096, K, torch.int8, 256), (k, 1024, K, torch.int8, 256), (v, 1024, K, torch.int8, 256)])
    lin = lambda m, x: int8_gemv.linear_forward(m, m.qweight._qdata.shape[0], K, torch.int8, 256, x)  # noqa: E731
    x = torch.ones(1, K)
    outs = [lin(m, x) for m in (q, k, v)]
    assert calls == [("multi", 256, 4096.0, (4096, 1024, 1024))] and [float(t[0]) for t in outs] == [1, 1, 1]
    lin(o, outs[0].view(1, K))  # not a sibling: its own fused rotation + GEMV
    assert calls[-1][0] == "fused" and len(calls) == 2
    # k first this time: any sibling may lead; a repeated call computes again
    lin(k, x)
    lin(k, x)
    assert [c[0] for c in calls[2:]] == ["multi", "multi"]
    assert float(lin(q, x)[0]) == 4 and float(lin(v, x)[0]) == 4  # the second of those launches
    # an in-place write between siblings bumps the version counter: k computes on the new values
    assert float(lin(q, x)[0]) == 5
    x.mul_(-0.5)
    assert float(lin(k, x)[0]) == 6 and calls[-1] == ("multi", 256, -2048.0, (4096, 1024, 1024))
    assert float(lin(q, x)[0]) == 6 and len(calls) == 6
    # another object with equal values, and a linear in between, both force a new launch
    assert float(lin(k, x.clone())[0]) == 7
    assert float(lin(q, x)[0]) == 8
    lin(o, x)
    assert float(lin(v, x)[0]) == 10
    assert [c[0] for c in calls[6:]] == ["multi", "multi", "fused", "multi"]

    class T:
        def generate(self):
            return "tokens"

    lin(q, x)
    int8_gemv.generate(T())
    lin(k, x)
    assert [c[0] for c in calls[-2:]] == ["multi", "multi"]
    int8_gemv.forget_siblings()


def test_inference_mode_write_between_linears_is_seen(monkeypatch):
    """Under torch.inference_mode() (no version counters, as ComfyUI runs nodes) an in-place write to an input between
    two linears that are not registered siblings reaches the second: each computes from the values it is given."""
    cast_context(monkeypatch)
    calls = []
    _record_gemv_kernels(monkeypatch, calls)
    int8_gemv.forget_siblings()
    K = 4096
    a, b = _gemv_layer(64, K), _gemv_layer(64, K)
    with torch.inference_mode():
        x = torch.ones(1, K)
        int8_gemv.linear_forward(a, 64, K, torch.int8, 256, x)
        x.mul_(-0.5)
        int8_gemv.linear_forward(b, 64, K, torch.int8, 256, x)
        int8_gemv.linear_forward(a, 64, K, torch.int8, 0, x)
    assert calls == [("fused", 256, 4096.0), ("fused", 256, -2048.0), ("gemv", -2048.0, K)]


def test_single_token_linears_without_siblings(monkeypatch):
    """linear_forward's single-token path (int8_gemv.py:58-63) for a linear with no registered siblings: the ConvRot
    inside the GEMV launch for the fused groups up to K = 8192 and past it when K % 1024 == 0 (K = 12288); K = 9728
    (past 8192 with a half step), a group outside FUSED_ROTATION_GROUPS and no group take rotate then GEMV, or the
    plain GEMV; siblings whose K is past one gemv_multi launch are refused at registration."""
    cast_context(monkeypatch)
    calls = []
    _record_gemv_kernels(monkeypatch, calls)
    int8_gemv.forget_siblings()
    x = torch.ones(1, 4096)
    int8_gemv.linear_forward(_gemv_layer(64, 4096), 64, 4096, torch.int8, 256, x)
    int8_gemv.linear_forward(_gemv_layer(64, 12288), 64, 12288, torch.int8, 256, torch.ones(1, 12288))
    int8_gemv.linear_forward(_gemv_layer(64, 9728), 64, 9728, torch.int8, 256, torch.ones(1, 9728))
    int8_gemv.linear_forward(_gemv_layer(64, 4096), 64, 4096, torch.int8, 1024, x)
    int8_gemv.linear_forward(_gemv_layer(64, 4096), 64, 4096, torch.int8, 0, x)
    assert calls == [("fused", 256, 4096.0), ("fused", 256, 12288.0), ("rotate", 256, 9728), ("gemv", 2 * 9728.0, 9728),
                     ("rotate", 1024, 4096), ("gemv", 2 * 4096.0, 4096), ("gemv", 4096.0, 4096)]
    with pytest.raises(ValueError):
        int8_gemv.register_siblings([(_gemv_layer(64, 12288), 64, 12288, torch.int8, 256), (_gemv_layer(64, 12288), 64, 12288, torch.int8, 256)])
    with pytest.raises(ValueError):
        int8_gemv.register_siblings([(_gemv_layer(64, 4096), 64, 4096, torch.int8, 256), (_gemv_layer(64, 4096), 64, 4096, torch.int8, 64)])


def test_gemv_wrappers_check_their_inputs():
    """The public GEMV wrappers refuse inputs the kernels would read past (wrong dtype or length) before any launch."""
    w, s = torch.zeros(64, 512, dtype=torch.int8), torch.ones(64)
    with pytest.raises(ValueError):
        int8_gemv.rotate_gemv(torch.zeros(512, dtype=torch.float16), 256, w, s)
    with pytest.raises(ValueError):
        int8_gemv.rotate_gemv(torch.zeros(256), 256, w, s)
    with pytest.raises(ValueError):
        int8_gemv.rotate_gemv(torch.zeros(512), 256, w, s, rotated=torch.zeros(512, dtype=torch.float16))
    with pytest.raises(ValueError):
        int8_gemv.rotate_gemv(torch.zeros(512), 256, w, s, rotated=torch.zeros(256))
    with pytest.raises(ValueError):
        int8_gemv.gemv(torch.zeros(500), w, s)
    with pytest.raises(ValueError):
        int8_gemv.gemv(torch.zeros(512, dtype=torch.float64), w, s)
    with pytest.raises(ValueError):
        int8_gemv.gemv_multi(torch.zeros(512, dtype=torch.float16), [(w, s, None)], group=256)
    with pytest.raises(ValueError):
        int8_gemv.gemv_multi(torch.zeros(512), [(w, s, None)] * 5)
    with pytest.raises(ValueError):
        int8_gemv.gemv_multi(torch.zeros(512), [(w, s, None), (torch.zeros(64, 1024, dtype=torch.int8), s, None)])
    with pytest.raises(ValueError):
        int8_gemv.rotate(torch.zeros(500), 256)
    for bad_scale, bad_bias in ((s.half(), None), (torch.ones(32), None), (s, torch.zeros(64, dtype=torch.float16)), (s, torch.zeros(63))):
        with pytest.raises(ValueError):
            int8_gemv.gemv(torch.zeros(512), w, bad_scale, bad_bias)
        with pytest.raises(ValueError):
            int8_gemv.rotate_gemv(torch.zeros(512), 256, w, bad_scale, bad_bias)
        with pytest.raises(ValueError):
            int8_gemv.gemv_multi(torch.zeros(512), [(w, bad_scale, bad_bias)])
    with pytest.raises(ValueError):
        int8_gemv.gemv(torch.zeros(512), w.t().contiguous().t(), s)  # a transposed (non-contiguous) weight


def test_gemm_wrappers_check_their_inputs():
    """linear / run and linear_w4a8 refuse tensors the kernels would read past or misread (a weight of the wrong width,
    dtype or layout, scales or a bias of the wrong length or dtype, an x of the wrong width, too small activations)
    before any allocation on the device or launch."""
    M, N, K = 8, 64, 256
    x, w, ws = torch.zeros(M, K, dtype=torch.float16), torch.zeros(N, K, dtype=torch.int8), torch.ones(N)
    bad_linear = [dict(x=x.float()), dict(x=torch.zeros(M, K + 16, dtype=torch.float16)), dict(weight=torch.zeros(N, K - 16, dtype=torch.int8)),
                  dict(weight=w.to(torch.uint8)), dict(weight=torch.zeros(K, N, dtype=torch.int8).t()), dict(weight_scale=ws.half()),
                  dict(weight_scale=torch.ones(N - 1)), dict(bias=torch.zeros(N)), dict(bias=torch.zeros(N - 1, dtype=torch.float16)),
                  dict(activations=(torch.zeros(M * K // 8, dtype=torch.int32), torch.ones(M)))]
    for bad in bad_linear:
        args = dict(x=x, weight=w, weight_scale=ws, bias=None, activations=None) | bad
        with pytest.raises(ValueError):
            int8_gemm.linear(args["x"], args["weight"], args["weight_scale"], args["bias"], rotate=True, activations=args["activations"])
    with pytest.raises(ValueError):  # SwiGLU: the up projection must match the gate
        int8_gemm.linear(x, w, ws, None, up=torch.zeros(M, K // 2, dtype=torch.float16))
    with pytest.raises(ValueError):  # situ reads rows of 2K values
        int8_gemm.linear(x, w, ws, None, situ=True)
    w4, gs = torch.zeros(N, K // 2, dtype=torch.uint8), torch.ones(N, K // 128, dtype=torch.float16)
    bad_w4a8 = [dict(x=torch.zeros(M, K + 64, dtype=torch.float16)), dict(qweight=torch.zeros(N, K, dtype=torch.uint8)),
                dict(group_scales=gs.float()), dict(group_scales=torch.ones(N, K // 64, dtype=torch.float16)),
                dict(group_scales=torch.ones(K // 128, N, dtype=torch.float16).t()), dict(bias=torch.zeros(N))]
    for bad in bad_w4a8:
        args = dict(x=x, qweight=w4, group_scales=gs, bias=None) | bad
        with pytest.raises(ValueError):
            int8_gemm.linear_w4a8(args["x"], args["qweight"], args["group_scales"], args["bias"])


def test_decode_attention_checks_its_inputs():
    """attention_decode refuses what its kernels would misread or read past -- a cache of another dtype or layout, v
    shaped unlike k, heads not a multiple of the KV heads, lengths not one int32 per batch row -- before any launch."""
    q, k = torch.zeros(2, 1, 8, 128), torch.zeros(2, 64, 2, 128)
    ln = torch.full((2,), 64, dtype=torch.int32)
    bad = [dict(k=k.half(), v=k.half()), dict(v=torch.zeros(2, 32, 2, 128)), dict(q=torch.zeros(2, 1, 7, 128)), dict(q=torch.zeros(2, 1, 6, 128)),
           dict(k=k.transpose(1, 2).contiguous().transpose(1, 2), v=k.transpose(1, 2).contiguous().transpose(1, 2)),
           dict(lengths=ln.long()), dict(lengths=ln[:1]), dict(q=torch.zeros(2, 1, 8, 64)), dict(q=torch.zeros(3, 1, 8, 128))]
    for b in bad:
        args = dict(q=q, k=k, v=k.clone(), lengths=ln) | b
        with pytest.raises(ValueError):
            int8_gemv.attention_decode(args["q"], args["k"], args["v"], args["lengths"])


def test_rms_norm_wrappers_check_their_inputs():
    """rms_norm and rms_norm_rope refuse weights, frequencies and inputs whose sizes the kernels would read past."""
    x = torch.zeros(1, 4, 256, dtype=torch.float16)
    for bad in ((x.float(), torch.zeros(256)), (x, torch.zeros(128)), (x, torch.zeros(256, dtype=torch.float16)), (x[..., :250], torch.zeros(250))):
        with pytest.raises(ValueError):
            rms_norm.rms_norm(*bad, 1e-6)
    norm = types.SimpleNamespace(scale=torch.zeros(128), eps=1e-6)
    q, f = torch.zeros(2, 4, 256, dtype=torch.float16), torch.zeros(1, 1, 4, 64, 2, 2)
    for bad in ((q, 3, f), (q.float(), 2, f), (q, 2, torch.zeros(1, 1, 3, 64, 2, 2)), (q, 2, f.double()), (q, 2, torch.zeros(3, 1, 4, 64, 2, 2))):
        with pytest.raises(ValueError):
            rms_norm.rms_norm_rope(bad[0], bad[1], norm, bad[2])
