"""CPU oracle for the quantized-inference hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg import this package, and only as the reference results or the timed CPU baseline. The
product path (the package ``comfyui-rdna2-attention_amd``) never imports it.

Two halves:

* ``librda_oracle.so`` (``rda_oracle.c``, built by ``oracle/Makefile``): the
  bit-exact restatement of the reference's fp32/fp16 arithmetic -- the ConvRot
  block Hadamard, the activations, per-token quantization, the GEMM epilogues
  and RMSNorm -- in the reference's operation order.
* numpy: integer GEMM accumulators (float64 matmul of int8 operands is exact,
  every partial sum is an integer below 2**53), float64 closed forms for the
  floating-point kernels (attention, GEMV, decode attention), and a
  reference-faithful fp32 restatement of the fused attention loop.

Each function names the reference file:line it restates.
"""
import ctypes
import math
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "librda_oracle.so")

ACT_NONE, ACT_SITU, ACT_SWIGLU, ACT_GATE, ACT_MOD = 0, 1, 2, 3, 4

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def load(path):
    """A build of rda_oracle.c at `path`, with its entry points' C signatures declared."""
    L = ctypes.CDLL(path)
    f32, i32, u16, i64 = ctypes.c_float, ctypes.c_int, ctypes.c_uint16, ctypes.c_long
    p = ctypes.c_void_p
    L.orc_expf.restype = f32
    L.orc_expf.argtypes = [f32]
    L.orc_exp2f.restype = f32
    L.orc_exp2f.argtypes = [f32]
    L.orc_h2f.restype = f32
    L.orc_h2f.argtypes = [u16]
    L.orc_f2h.restype = u16
    L.orc_f2h.argtypes = [f32]
    for name in ("orc_swiglu", "orc_sigmoid_gate", "orc_situ"):
        getattr(L, name).restype = f32
        getattr(L, name).argtypes = [f32, f32]
    L.orc_modulate.restype = f32
    L.orc_modulate.argtypes = [f32, f32, f32, f32, f32]
    L.orc_quant_rows.argtypes = [i32, i32, p, i32, p, p]
    L.orc_rot_quant_rows.argtypes = [i32, i32, i32, i32, i32, p, i32, p, p, p, p, i32, f32, p, p, p]
    L.orc_gemm_epilogue.argtypes = [i32, i32, p, p, p, p, p, p, i32, p]
    L.orc_w4a8_epilogue.argtypes = [i32, i32, i32, p, p, p, p, p]
    L.orc_rms_norm.argtypes = [i32, i32, i32, i32, p, i64, i64, i64, p, f32, p, i64, p]
    L.orc_rotate_f32.argtypes = [i32, i32, p, p]
    L.orc_quant_rows_rint.argtypes = [i32, i32, p, i64, p, p]
    return L


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = load(LIB_PATH)
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _f16(a):
    return np.ascontiguousarray(a, dtype=np.float16)


# ------------------------------------------------------------ scalar functions

def expf(x):
    """The kernels' exp (Cody-Waite + degree-7 polynomial), see rda_oracle.c."""
    return np.float32(lib().orc_expf(float(x)))


def exp2f(x):
    return np.float32(lib().orc_exp2f(float(x)))


def vectorize(name, *args):
    f = getattr(lib(), name)
    arrays = np.broadcast_arrays(*[np.asarray(a, dtype=np.float32) for a in args])
    flat = [a.ravel() for a in arrays]
    return np.array([f(*[float(a[i]) for a in flat]) for i in range(flat[0].size)], dtype=np.float32).reshape(arrays[0].shape)


# --------------------------------------------------------- rotate + quantize

def quant_rows(x):
    """quant_pack_a (int8_gemm.hip:93-103): per-row absmax int8, no rotation. x fp16 [M, K]."""
    x = _f16(x)
    M, K = x.shape
    q = np.empty((M, K), np.int8)
    s = np.empty(M, np.float32)
    lib().orc_quant_rows(M, K, _ptr(x), K, _ptr(q), _ptr(s))
    return q, s


def rot_quant_rows(x, act=ACT_NONE, group=256, u=None, i4=False, mod=None):
    """rot_quant<ACT, I4> (int8_gemm.hip:151-243). x fp16 [M, K] ([M, 2K] for situ).

    mod = (w fp32 [K], s fp16 [M/L, K], t fp16 [M/L, K], L, eps) for ACT_MOD.
    Returns (q int8 [M, K], scale fp32 [M], rotated fp16 [M, K])."""
    x = _f16(x)
    M = x.shape[0]
    K = x.shape[1] // 2 if act == ACT_SITU else x.shape[1]
    assert K % group == 0 and group in (128, 256)
    q = np.empty((M, K), np.int8)
    s = np.empty(M, np.float32)
    rot = np.empty((M, K), np.uint16)
    uu = None if u is None else _f16(u)
    w = ms = mt = None
    L, eps = 1, 0.0
    if mod is not None:
        w, ms, mt, L, eps = mod
        w = np.ascontiguousarray(w, np.float32)
        ms, mt = _f16(ms), _f16(mt)
    lib().orc_rot_quant_rows(act, int(i4), group, M, K, _ptr(x), x.shape[1], _ptr(uu), _ptr(w), _ptr(ms), _ptr(mt),
                             L, eps, _ptr(q), _ptr(s), _ptr(rot))
    return q, s, rot.view(np.float16)


def quant_rows_rint(x):
    """Per-row absmax int8 with rint (pack_kv_i8 hip_attention.hip:85-91; attn_i8 183-193). x fp16 [R, D]."""
    x = _f16(x)
    R, D = x.shape
    q = np.empty((R, D), np.int8)
    s = np.empty(R, np.float32)
    lib().orc_quant_rows_rint(R, D, _ptr(x), D, _ptr(q), _ptr(s))
    return q, s


# -------------------------------------------------------------------- GEMMs

def gemm_acc(a, w):
    """int32 C[m, n] = sum_k a[m, k] * w[n, k]; exact through float64 (|partial sums| < 2**53)."""
    assert a.shape[1] == w.shape[1]
    assert a.shape[1] * 128 * 128 < 2 ** 53
    return (a.astype(np.float64) @ w.astype(np.float64).T).astype(np.int64).astype(np.int32)


def gemm_epilogue(acc, a_scale, w_scale, bias=None, R=None, G=None, L=1):
    """gemm_body epilogue (int8_gemm.hip:371-405), bit-exact."""
    acc = np.ascontiguousarray(acc, np.int32)
    M, N = acc.shape
    out = np.empty((M, N), np.uint16)
    a_scale = np.ascontiguousarray(a_scale, np.float32)
    w_scale = np.ascontiguousarray(w_scale, np.float32)
    b = None if bias is None else _f16(bias)
    r = None if R is None else _f16(R)
    g = None if G is None else _f16(G)
    lib().orc_gemm_epilogue(M, N, _ptr(acc), _ptr(a_scale), _ptr(w_scale), _ptr(b), _ptr(r), _ptr(g), L, _ptr(out))
    return out.view(np.float16)


def unpack_int4(packed, K):
    """Signed int4 weights, two per byte, low nibble = even k (int8_gemm.hip:62, 85). Returns int8 [N, K]."""
    p = np.asarray(packed).view(np.uint8)
    lo = (p & 0xF).astype(np.int8)
    hi = (p >> 4).astype(np.int8)
    lo = np.where(lo >= 8, lo - 16, lo).astype(np.int8)
    hi = np.where(hi >= 8, hi - 16, hi).astype(np.int8)
    out = np.empty((p.shape[0], K), np.int8)
    out[:, 0::2] = lo
    out[:, 1::2] = hi
    return out


def pack_int4(w):
    """Inverse of unpack_int4: int8 values in [-8, 7] -> uint8 [N, K/2]."""
    w = np.asarray(w, np.int8)
    lo = (w[:, 0::2].astype(np.int16) & 0xF).astype(np.uint8)
    hi = (w[:, 1::2].astype(np.int16) & 0xF).astype(np.uint8)
    return (lo | (hi << 4)).astype(np.uint8)


def w4a8_partials(a, w, group=128):
    """Per-group int32 partials p[g, m, n] = sum_{k in group g} a[m, k] * w[n, k]."""
    K = a.shape[1]
    G = K // group
    return np.stack([gemm_acc(a[:, g * group:(g + 1) * group], w[:, g * group:(g + 1) * group]) for g in range(G)])


def w4a8_epilogue(partials, a_scale, group_scales, bias=None):
    """W4A8 epilogue: y = fma((float)p_g, gs[n, g], y) over g in order; out = fp16(y * as[m] (+ bias))."""
    partials = np.ascontiguousarray(partials, np.int32)
    G, M, N = partials.shape
    out = np.empty((M, N), np.uint16)
    gs = _f16(group_scales)
    assert gs.shape == (N, G)
    a_scale = np.ascontiguousarray(a_scale, np.float32)
    b = None if bias is None else _f16(bias)
    lib().orc_w4a8_epilogue(M, N, G, _ptr(partials), _ptr(a_scale), _ptr(gs), _ptr(b), _ptr(out))
    return out.view(np.float16)


def hadamard_matrix(group):
    """Closed form of the rotation: kron(H4, H4, H4, H4) for 256, kron(H2, H4, H4, H4) for 128 (the factor
    acting on the slowest index first), as an integer matrix; the kernels scale by 1/16 resp. fp32(2**-3.5)."""
    H4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], np.int64)
    H2 = np.array([[1, 1], [1, -1]], np.int64)
    H = np.array([[1]], np.int64)
    for f in ([H4] * 4 if group == 256 else [H2, H4, H4, H4]):
        H = np.kron(H, f)
    return H


# ------------------------------------------------------------------ RMSNorm

def rms_norm(x, w, eps, freqs=None):
    """norm_row (rms_norm.hip:9-65) on x of shape (B, L, D) or (B, H, L, D) (any strides, last dim contiguous).
    Returns contiguous fp16 (B, H, L, D) -- or (B, L, D) for 3-D input. freqs (B or 1, 1, L, D/2, 2, 2) fp32."""
    x = np.asarray(x, dtype=np.float16)
    v = x if x.ndim == 4 else x[:, None]
    B, H, L, D = v.shape
    # The values are what matter here; the kernels' strided addressing is tested on the GPU side.
    flat = np.ascontiguousarray(v).reshape(-1)
    sb, sh, sl = H * L * D, L * D, D
    out = np.empty((B, H, L, D), np.uint16)
    w = np.ascontiguousarray(w, np.float32)
    f = None
    fb = 0
    if freqs is not None:
        f = np.ascontiguousarray(freqs, np.float32)
        fb = L * D // 2 if f.shape[0] > 1 else 0
    lib().orc_rms_norm(B, H, L, D, _ptr(flat), sb, sh, sl, _ptr(w), eps, _ptr(f), fb, _ptr(out))
    out = out.view(np.float16)
    return out if x.ndim == 4 else out[:, 0]


def rms_norm_f64(x, w, eps):
    """Closed form in float64: x / sqrt(mean(x^2) + eps) * (w + 1)."""
    x = np.asarray(x, np.float64)
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * (np.asarray(w, np.float64) + 1)


# ----------------------------------------------------------------- decode path

def rotate_f32(x, group):
    """rotate (int8_gemv.hip:31-52). x fp32 [..., group multiple]."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().orc_rotate_f32(x.size // group, group, _ptr(x), _ptr(out))
    return out


def gemv_f64(x, w, scale, bias=None):
    """out[n] = scale[n] * sum_k w[n, k] x[k] (+ bias[n]) in float64 (int8_gemv.hip:54-85)."""
    out = (w.astype(np.float64) @ np.asarray(x, np.float64).reshape(-1)) * np.asarray(scale, np.float64)
    if bias is not None:
        out = out + np.asarray(bias, np.float64)
    return out


def attention_decode_f64(q, k, v, lengths, scale=128 ** -0.5):
    """attn_decode + attn_merge (int8_gemv.hip:121-195) in float64: q (B, 1, H, D), k/v (B, cap, Hkv, D)."""
    q, k, v = (np.asarray(t, np.float64) for t in (q, k, v))
    B, _, H, D = q.shape
    Hkv = k.shape[2]
    rep = H // Hkv
    out = np.zeros((B, 1, H, D))
    for b in range(B):
        n = int(lengths[b])
        for h in range(H):
            kk, vv = k[b, :n, h // rep], v[b, :n, h // rep]
            s = kk @ (q[b, 0, h] * scale)
            p = np.exp(s - s.max())
            out[b, 0, h] = (p @ vv) / p.sum()
    return out


# ------------------------------------------------------------------ attention

def attention_f64(q, k, v, scale):
    """softmax(q k^T * scale) v in float64. q (B, H, Lq, D), k/v (B, Hkv, Lk, D)."""
    q, k, v = (np.asarray(t, np.float64) for t in (q, k, v))
    rep = q.shape[1] // k.shape[1]
    k = np.repeat(k, rep, axis=1)
    v = np.repeat(v, rep, axis=1)
    s = q @ np.swapaxes(k, -1, -2) * scale
    s -= s.max(-1, keepdims=True)
    p = np.exp(s)
    return (p @ v) / p.sum(-1, keepdims=True)


def attention_i8qk_scores(q, k, scale):
    """attn_i8's scores (hip_attention.hip:172-227) in the exp2 domain, fp32 like the kernel:
    s = ((float)si * (q_scale * scale_log2)) * k_scale with si exact int32. q (B, H, Lq, D), k (B, Hkv, Lk, D)."""
    q, k = np.asarray(q, np.float16), np.asarray(k, np.float16)
    B, H, Lq, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    rep = H // Hkv
    scale_log2 = np.float32(scale * math.log2(math.e))
    out = np.empty((B, H, Lq, Lk), np.float32)
    for b in range(B):
        kq = [quant_rows_rint(k[b, h]) for h in range(Hkv)]
        for h in range(H):
            q8, qs = quant_rows_rint(q[b, h])
            k8, ks = kq[h // rep]
            si = gemm_acc(q8, k8)
            score_scale = (qs * scale_log2).astype(np.float32)
            out[b, h] = (si.astype(np.float32) * score_scale[:, None]).astype(np.float32) * ks[None, :]
    return out


def attention_i8qk_f64(q, k, v, scale):
    """Closed form of the int8-QK attention: softmax in base 2 of the fp32 scores above, times v, in float64."""
    s2 = attention_i8qk_scores(q, k, scale).astype(np.float64)
    v = np.asarray(v, np.float64)
    rep = q.shape[1] // v.shape[1]
    v = np.repeat(v, rep, axis=1)
    s2 -= s2.max(-1, keepdims=True)
    p = np.exp2(s2)
    return (p @ v) / p.sum(-1, keepdims=True)


def attention_faithful(q, k, v, scale, block=16, threshold=8.0, wave=32, stats=False):
    """The reference's fused loop (hip_attention.hip:280-373) restated per query row in fp32.

    Query rows run in waves of `wave` consecutive rows (hip_attention.hip:284-287; the padding lanes of a last,
    partial wave repeat its last row, so they never change the vote). Per block of 16 keys: scores in fp32,
    mx = fp32(max_j s_j) * scale_log2; when ANY row of the wave has mx > m + threshold, EVERY row of that wave
    moves to m' = max(m, mx) and scales l and o by exp2(m - m') (hip_attention.hip:334-340); then
    p = exp2(fp32(fma(s, scale_log2, -m))), l += p0 + p1 over the pairs in order, P rounded to fp16 for PV, and
    out = fp16(o * (1 / l)). Exponentials in float64 rounded to fp32 (the hardware's exp2 is not reproducible, so
    this restatement is tolerance-level, not bit-level). With stats=True also returns each row's final running
    maximum m and sum l, shape (B, H, Lq)."""
    q, k, v = (np.asarray(t, np.float16) for t in (q, k, v))
    B, H, Lq, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    rep = H // Hkv
    scale_log2 = np.float32(scale * math.log2(math.e))
    waves = np.arange(Lq) // wave
    out = np.empty((B, H, Lq, D), np.float16)
    m_out = np.empty((B, H, Lq), np.float32)
    l_out = np.empty((B, H, Lq), np.float32)
    for b in range(B):
        for h in range(H):
            kk = k[b, h // rep].astype(np.float32)
            vv = v[b, h // rep].astype(np.float32)
            qq = q[b, h].astype(np.float32)
            m = np.full(Lq, -1e30, np.float32)
            l = np.zeros(Lq, np.float32)
            o = np.zeros((Lq, D), np.float32)
            for g in range(0, Lk, block):
                s = (qq.astype(np.float64) @ kk[g:g + block].astype(np.float64).T).astype(np.float32)
                mx = (s.max(1) * scale_log2).astype(np.float32)
                vote = np.bincount(waves, weights=(mx > m + np.float32(threshold)).astype(np.float64)) > 0
                up = vote[waves]
                if up.any():
                    mn = np.maximum(m, mx)
                    alpha = np.where(up, np.exp2((m.astype(np.float64) - mn)).astype(np.float32), np.float32(1))
                    m = np.where(up, mn, m).astype(np.float32)
                    l = (l * alpha).astype(np.float32)
                    o = (o * alpha[:, None]).astype(np.float32)
                arg = (s.astype(np.float64) * float(scale_log2) - m[:, None].astype(np.float64)).astype(np.float32)
                p = np.exp2(arg.astype(np.float64)).astype(np.float32)
                for j in range(0, p.shape[1] - 1, 2):
                    l = (l + (p[:, j] + p[:, j + 1]).astype(np.float32)).astype(np.float32)
                if p.shape[1] % 2:
                    l = (l + p[:, -1]).astype(np.float32)
                o = (o + (p.astype(np.float16).astype(np.float64) @ vv[g:g + block].astype(np.float64))).astype(np.float32)
            out[b, h] = (o * (np.float32(1) / l)[:, None]).astype(np.float16)
            m_out[b, h], l_out[b, h] = m, l
    return (out, m_out, l_out) if stats else out
