"""The MFMA calibration entry points (measurement only): they run, report a shader clock, reject bad operand buffers,
and the data-driven int8 variant computes exactly the products its documentation states, so the rate it reports
is that of those operands."""
import ctypes

import numpy as np
import pytest
import torch

from comfyui_rdna2_attention_amd import _lib
from helpers import gen

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("int8", [0, 1])
def test_fixed_operand_calibration_runs(dev, int8):
    lib = _lib.load()
    out = torch.empty(4 * 256, dtype=torch.int32, device=dev)
    clocks = torch.zeros(2, dtype=torch.int64, device=dev)
    _lib.check(lib.rda_calib_mfma_peak(int8, 4, 20, _lib.ptr(out), _lib.ptr(clocks), _lib.stream()))
    torch.cuda.synchronize()
    assert int(clocks[0]) > 0 and int(clocks[1]) > 0


def test_data_calibration_rejects_unaligned_operands(dev):
    lib = _lib.load()
    ops = torch.zeros(1 * 256 * 16 * 16 + 16, dtype=torch.int8, device=dev)
    out = torch.empty(256, dtype=torch.int32, device=dev)
    clocks = torch.zeros(2, dtype=torch.int64, device=dev)
    assert lib.rda_calib_mfma_peak_data(1, 1, 4, ctypes.c_void_p(ops.data_ptr() + 4), _lib.ptr(out), _lib.ptr(clocks), _lib.stream()) == 1
    assert lib.rda_calib_mfma_peak_data(1, 1, 4, None, _lib.ptr(out), _lib.ptr(clocks), _lib.stream()) == 1


@pytest.mark.parametrize("iters", [1, 2, 5])
def test_int8_data_calibration_computes_its_products(dev, iters):
    """Lane l of wave w supplies row l % 32 and k half l / 32 (16 bytes) of A chain c (fragment c) and of B (fragment
    8 + c); chain c multiplies A_c by B_(c+3)%8 in even rounds and B_(c+4)%8 in odd ones; each lane outputs the sum of
    its 16 accumulators, rows 8 (r / 4) + 4 (l / 32) + r % 4 of column l % 32."""
    blocks = 2
    lib = _lib.load()
    g = gen(31)
    ops = torch.randint(-128, 128, (blocks * 256 * 16 * 16,), generator=g, dtype=torch.int8)
    out = torch.empty(blocks * 256, dtype=torch.int32, device=dev)
    clocks = torch.zeros(2, dtype=torch.int64, device=dev)
    _lib.check(lib.rda_calib_mfma_peak_data(1, blocks, iters, _lib.ptr(ops.to(dev)), _lib.ptr(out), _lib.ptr(clocks), _lib.stream()))
    got = out.cpu().numpy().astype(np.int64)
    frags = ops.numpy().astype(np.int64).reshape(blocks, 4, 64, 16, 16)  # block, wave, lane, fragment, byte
    want = np.zeros((blocks, 4, 64), np.int64)
    for b in range(blocks):
        for w in range(4):
            def matrix(f):  # 32 x 32: [row i][k], lane l holds row l % 32, k = 16 (l / 32) + byte
                m = np.zeros((32, 32), np.int64)
                for lane in range(64):
                    m[lane % 32, 16 * (lane // 32):16 * (lane // 32) + 16] = frags[b, w, lane, f]
                return m
            A = [matrix(c) for c in range(8)]
            B = [matrix(8 + c) for c in range(8)]
            for c in range(8):
                acc = np.zeros((32, 32), np.int64)
                for i in range(iters):
                    acc += A[c] @ B[(c + 3 + (i & 1)) % 8].T  # C[i][j] = sum_k A[i][k] B[j][k]
                for lane in range(64):
                    rows = [8 * (r // 4) + 4 * (lane // 32) + r % 4 for r in range(16)]
                    want[b, w, lane] += acc[rows, lane % 32].sum()
    assert np.array_equal(got.reshape(blocks, 4, 64), want)
