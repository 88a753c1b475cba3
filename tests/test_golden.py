"""The committed golden vectors (tests/golden/golden.npz, written by tests/golden/make_golden.py): the oracle must
reproduce them bit for bit on the CPU, and the GPU kernels must reproduce them bit for bit on the GPU."""
import os

import numpy as np
import pytest
import torch

import oracle
from helpers import assert_same, bits

HERE = os.path.dirname(os.path.abspath(__file__))
G = dict(np.load(os.path.join(HERE, "golden", "golden.npz")))


def test_oracle_reproduces_golden():
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(HERE, "golden", "make_golden.py"))
    mk = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mk)
    fresh = mk.build()
    assert set(fresh) == set(G)
    for name, value in fresh.items():
        assert value.dtype == G[name].dtype, name
        assert_same(value.view(np.uint8), G[name].view(np.uint8), name)


@pytest.mark.gpu
def test_kernels_reproduce_golden(dev):
    from comfyui_rdna2_attention_amd import _lib, int8_gemm, int8_gemv, rms_norm
    k = int8_gemm.get_kernels()
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731

    def quant(entry, x, K, group=256, up=None, q_name=None, s_name=None):
        packed, scale = int8_gemm.quantize(entry, d(x), K, up=None if up is None else d(up), group=group)
        M = x.shape[0]
        assert_same(packed.view(torch.int8)[:M * K].view(M, K).cpu().numpy(), G[q_name], q_name)
        assert_same(scale.cpu().numpy(), G[s_name], s_name)

    quant(k.rot_quant_pack_a, G["rot256_x"], 512, 256, q_name="rot256_q", s_name="rot256_s")
    quant(k.rot_quant_pack_a, G["rot128_x"], 384, 128, q_name="rot128_q", s_name="rot128_s")
    quant(k.quant_pack_a, G["quant_x"], 64, q_name="quant_q", s_name="quant_s")
    quant(k.rot_quant_pack_a_i4, G["i4_x"], 256, q_name="i4_q", s_name="i4_s")
    quant(k.swiglu_rot_quant_pack_a, G["act_a"], 256, up=G["act_b"], q_name="swiglu_q", s_name="swiglu_s")
    quant(k.gate_rot_quant_pack_a, G["act_a"], 256, up=G["act_b"], q_name="gate_q", s_name="gate_s")
    quant(k.situ_rot_quant_pack_a, G["situ_x"], 256, q_name="situ_q", s_name="situ_s")

    packed, scale = int8_gemm.quantized(4, 512, dev)
    p = _lib.ptr
    mx, mw, ms, mt = d(G["mod_x"]), d(G["mod_w"]), d(G["mod_s"]), d(G["mod_t"])  # referenced until the launch
    int8_gemm.launch(k.mod_rot_quant_pack_a, 0, 0, 0, [p(mx), p(packed), p(scale), 4, 512, p(mw), p(ms), p(mt), 2, 1e-6])
    assert_same(packed.view(torch.int8)[:4 * 512].view(4, 512).cpu().numpy(), G["mod_q"])
    assert_same(scale.cpu().numpy(), G["mod_sc"])

    a = d(G["gemm_a"]).view(torch.int32).reshape(-1)
    w = d(G["gemm_w"])
    acc = int8_gemm.gemm_acc(a, w, 8, 128)
    assert_same(acc.cpu().numpy(), G["gemm_acc"])
    for bias, res, name in ((None, None, "gemm_out"), (G["gemm_bias"], None, "gemm_out_bias"), (None, (G["gemm_R"].reshape(2, 4, 64), G["gemm_G"]), "gemm_out_res")):
        out = int8_gemm.linear(torch.empty(8, 128, dtype=torch.float16, device=dev), w, d(G["gemm_ws"]), None if bias is None else d(bias),
                               activations=(a, d(G["gemm_as"])), res=None if res is None else (d(res[0]), d(res[1])))
        assert_same(bits(out), bits(G[name]), name)

    out = int8_gemm.linear_w4a8(torch.empty(8, 256, dtype=torch.float16, device=dev), d(G["w4_packed"]), d(G["w4_gs"]),
                                activations=(d(G["w4_a"]).view(torch.int32).reshape(-1), d(G["w4_as"])))
    assert_same(bits(out), bits(G["w4_out"]))

    assert_same(bits(rms_norm.rms_norm(d(G["rms_x"]), d(G["rms_w"]), 1e-6)), bits(G["rms_out"]), "rms_out")
    assert_same(bits(rms_norm.rms_norm(d(G["rmsh_x"]), d(G["rmsh_w"]), 1e-6)), bits(G["rmsh_out"]), "rmsh_out")

    class Norm:
        scale, eps = d(G["rmsh_w"]), 1e-6
    assert_same(bits(rms_norm.rms_norm_rope(d(G["rope_x"]), 2, Norm, d(G["rope_freqs"]))), bits(G["rope_out"]), "rope_out")
    assert_same(int8_gemv.rotate(d(G["rotate_x"]), 256).cpu().numpy(), G["rotate_out"])
