"""Writes tests/golden/golden.npz: small seeded input/output vectors of the oracle for every bit-exact function of
the hot path. The reference ships no golden vectors, fixtures or tests for this path; these are produced by the
oracle after the checks in tests/test_oracle.py pin it, and freeze it: tests/test_golden.py re-derives them on the
CPU and checks the GPU kernels against them.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import oracle  # noqa: E402


def build():
    rng = np.random.default_rng(20261201)
    g = {}

    def acts(M, K, outliers=True):
        x = rng.standard_normal((M, K)).astype(np.float32)
        if outliers:
            x[:, rng.choice(K, 4, replace=False)] *= 30
        return x.astype(np.float16)

    x = acts(6, 512)
    x[2] = 0
    g["rot256_x"] = x
    g["rot256_q"], g["rot256_s"], _ = oracle.rot_quant_rows(x, group=256)
    g["rot128_x"] = acts(5, 384)
    g["rot128_q"], g["rot128_s"], _ = oracle.rot_quant_rows(g["rot128_x"], group=128)
    g["quant_x"] = acts(3, 64)
    g["quant_q"], g["quant_s"] = oracle.quant_rows(g["quant_x"])
    g["i4_x"] = acts(3, 256)
    g["i4_q"], g["i4_s"], _ = oracle.rot_quant_rows(g["i4_x"], i4=True)
    a, b = (rng.standard_normal((4, 256)) * 4).astype(np.float16), (rng.standard_normal((4, 256)) * 4).astype(np.float16)
    g["act_a"], g["act_b"] = a, b
    g["swiglu_q"], g["swiglu_s"], _ = oracle.rot_quant_rows(a, act=oracle.ACT_SWIGLU, u=b)
    g["gate_q"], g["gate_s"], _ = oracle.rot_quant_rows(a, act=oracle.ACT_GATE, u=b)
    g["situ_x"] = (rng.standard_normal((3, 512)) * 3).astype(np.float16)
    g["situ_q"], g["situ_s"], _ = oracle.rot_quant_rows(g["situ_x"], act=oracle.ACT_SITU)
    g["mod_x"] = rng.standard_normal((4, 512)).astype(np.float16)
    g["mod_w"] = (rng.standard_normal(512) * 0.1).astype(np.float32)
    g["mod_s"] = (1 + rng.standard_normal((2, 512)) * 0.2).astype(np.float16)
    g["mod_t"] = (rng.standard_normal((2, 512)) * 0.2).astype(np.float16)
    g["mod_q"], g["mod_sc"], _ = oracle.rot_quant_rows(g["mod_x"], act=oracle.ACT_MOD, mod=(g["mod_w"], g["mod_s"], g["mod_t"], 2, 1e-6))

    g["gemm_a"] = rng.integers(-128, 128, (8, 128)).astype(np.int8)
    g["gemm_w"] = rng.integers(-128, 128, (64, 128)).astype(np.int8)
    g["gemm_as"] = rng.uniform(1e-3, 1e-1, 8).astype(np.float32)
    g["gemm_ws"] = rng.uniform(1e-3, 3e-3, 64).astype(np.float32)
    g["gemm_bias"] = rng.standard_normal(64).astype(np.float16)
    g["gemm_acc"] = oracle.gemm_acc(g["gemm_a"], g["gemm_w"])
    g["gemm_out"] = oracle.gemm_epilogue(g["gemm_acc"], g["gemm_as"], g["gemm_ws"])
    g["gemm_out_bias"] = oracle.gemm_epilogue(g["gemm_acc"], g["gemm_as"], g["gemm_ws"], g["gemm_bias"])
    g["gemm_R"] = rng.standard_normal((8, 64)).astype(np.float16)
    g["gemm_G"] = rng.standard_normal((2, 64)).astype(np.float16)
    g["gemm_out_res"] = oracle.gemm_epilogue(g["gemm_acc"], g["gemm_as"], g["gemm_ws"], R=g["gemm_R"], G=g["gemm_G"], L=4)

    w4 = rng.integers(-8, 8, (64, 256)).astype(np.int8)
    g["w4_packed"] = oracle.pack_int4(w4)
    g["w4_a"] = rng.integers(-128, 128, (8, 256)).astype(np.int8)
    g["w4_as"] = rng.uniform(1e-3, 1e-1, 8).astype(np.float32)
    g["w4_gs"] = rng.uniform(5e-3, 2e-2, (64, 2)).astype(np.float16)
    g["w4_out"] = oracle.w4a8_epilogue(oracle.w4a8_partials(g["w4_a"], w4), g["w4_as"], g["w4_gs"])

    g["rms_x"] = rng.standard_normal((2, 3, 136)).astype(np.float16)
    g["rms_w"] = (rng.standard_normal(136) * 0.1).astype(np.float32)
    g["rms_out"] = oracle.rms_norm(g["rms_x"], g["rms_w"], 1e-6)
    g["rmsh_x"] = rng.standard_normal((1, 2, 5, 128)).astype(np.float16)
    g["rmsh_w"] = (rng.standard_normal(128) * 0.1).astype(np.float32)
    g["rmsh_out"] = oracle.rms_norm(g["rmsh_x"], g["rmsh_w"], 1e-6)
    ang = rng.standard_normal((1, 1, 5, 64)).astype(np.float32)
    g["rope_freqs"] = np.stack([np.cos(ang), -np.sin(ang), np.sin(ang), np.cos(ang)], -1).reshape(1, 1, 5, 64, 2, 2).astype(np.float32)
    g["rope_x"] = rng.standard_normal((1, 5, 2 * 128)).astype(np.float16)
    xh = g["rope_x"].reshape(1, 5, 2, 128).transpose(0, 2, 1, 3).copy()
    g["rope_out"] = oracle.rms_norm(xh, g["rmsh_w"], 1e-6, freqs=g["rope_freqs"])

    g["rotate_x"] = rng.standard_normal((2, 256)).astype(np.float32)
    g["rotate_out"] = oracle.rotate_f32(g["rotate_x"], 256)
    g["exp_x"] = np.concatenate([np.linspace(-88, 88, 257), rng.uniform(-5, 5, 64)]).astype(np.float32)
    g["exp_y"] = np.array([oracle.expf(v) for v in g["exp_x"]], np.float32)
    g["exp2_y"] = np.array([oracle.exp2f(v) for v in g["exp_x"]], np.float32)
    return g


if __name__ == "__main__":
    path = os.path.join(HERE, "golden.npz")
    np.savez_compressed(path, **build())
    print(path, os.path.getsize(path), "bytes")
