"""MI355X (gfx950) quantized-inference hot path for the ComfyUI node of d1c0n/ComfyUI-RDNA2-Attention.

Drop-in for the reference's kernel modules -- ``hip_attention``, ``int8_gemm``, ``int8_gemv``, ``rms_norm`` and
``attention`` keep their names, signatures, eligibility checks and fallbacks -- with hand-written gfx950 kernels
behind a C ABI (librda_gfx950.so, include/rda.h). When ComfyUI is importable the package also registers the two
nodes of the reference (``RDNA2Attention``, ``RDNA2TextGenerate``) as a thin shim over these modules.
"""
import logging

try:
    import torch
    from typing_extensions import override
    from comfy.patcher_extension import CallbacksMP
    from comfy.quant_ops import QuantizedTensor
    from comfy_api.latest import ComfyExtension, io
except ImportError:  # not running inside ComfyUI: the kernel modules are still importable
    io = None

if io is not None:
    from . import int8_gemm as int8_kernels
    from . import int8_gemv, rms_norm
    from .attention import attention_bmm, attention_hip, attention_hip_int8

    BACKENDS = {"hip": attention_hip, "hip_int8": attention_hip_int8, "bmm": attention_bmm}

    def relayout_weights(patcher):
        """Stores fp16 Linear weights K-major (same shape, transposed strides), a layout rocBLAS may prefer."""
        for module in patcher.model.diffusion_model.modules():
            if not isinstance(module, torch.nn.Linear):
                continue
            w = module.weight
            if isinstance(w, QuantizedTensor) or w.dtype != torch.float16 or w.device.type == "cpu" or min(w.shape) < 1024 or w.stride(0) == 1:
                continue
            w.data = w.data.t().contiguous().t()

    class RDNA2Attention(io.ComfyNode):
        @classmethod
        def define_schema(cls):
            return io.Schema(
                node_id="RDNA2Attention",
                display_name="RDNA2 Attention (MI355X)",
                category="model/patch",
                description="Fused attention, int8/int4 linears and fp16 RMSNorm on MI355X (gfx950) kernels.",
                inputs=[
                    io.Model.Input("model"),
                    io.Combo.Input("backend", options=list(BACKENDS), default="hip",
                                   tooltip="hip: fused fp16 attention for head dim 128, anything else uses bmm. hip_int8: int8 QK^T. bmm: matmuls."),
                    io.Boolean.Input("transpose_weights", default=False, tooltip="Store fp16 weights K-major."),
                    io.Boolean.Input("int8_gemm", default=False, tooltip="Run Int8/Int4 loader layers on the int8 matrix-core kernels (global)."),
                    io.Boolean.Input("fused_norm", default=False, tooltip="Krea 2: fp16 RMSNorm kernel."),
                    io.Boolean.Input("fused_swiglu", default=False, tooltip="Krea 2 Int8, needs int8_gemm: SwiGLU inside the down layer's quantization."),
                ],
                outputs=[io.Model.Output()],
            )

        @classmethod
        def execute(cls, model, backend, transpose_weights=False, int8_gemm=False, fused_norm=False, fused_swiglu=False) -> io.NodeOutput:
            m = model.clone()
            int8_kernels.enable(int8_gemm)
            m.set_model_optimized_attention(BACKENDS[backend])
            if fused_norm:
                rms_norm.patch(m)
            if fused_swiglu:
                int8_kernels.patch_swiglu(m)
            if fused_norm and fused_swiglu and backend != "bmm":
                int8_kernels.patch_block(m, backend == "hip_int8")
            if transpose_weights:
                if m.is_dynamic():
                    logging.warning("RDNA2 Attention: transpose_weights skipped, it needs --highvram or --disable-dynamic-vram.")
                else:
                    m.add_callback(CallbacksMP.ON_PRE_RUN, relayout_weights)
            return io.NodeOutput(m)

    class RDNA2TextGenerate(io.ComfyNode):
        @classmethod
        def define_schema(cls):
            return io.Schema(
                node_id="RDNA2TextGenerate",
                display_name="RDNA2 Text Generate (MI355X)",
                category="model/patch",
                description="Generate Text with int8 text encoders on MI355X decode kernels. Prompt encoding is unaffected.",
                inputs=[io.Clip.Input("clip")],
                outputs=[io.Clip.Output()],
            )

        @classmethod
        def execute(cls, clip) -> io.NodeOutput:
            clip = clip.clone()
            int8_gemv.patch(clip)
            return io.NodeOutput(clip)

    class RDNA2AttentionExtension(ComfyExtension):
        @override
        async def get_node_list(self) -> list[type[io.ComfyNode]]:
            return [RDNA2Attention, RDNA2TextGenerate]

    async def comfy_entrypoint() -> RDNA2AttentionExtension:
        return RDNA2AttentionExtension()
