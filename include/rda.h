/*
 * librda_gfx950.so -- the C ABI of the MI355X (gfx950) quantized-inference hot path.
 *
 * Every entry point takes raw device pointers, sizes, scalars and a hipStream_t passed as
 * void* (0 = the null stream). Work is enqueued asynchronously on that stream; nothing
 * allocates, frees or synchronises. The return value is a hipError_t: 0 on success,
 * 1 (hipErrorInvalidValue) for a shape or argument the kernels do not support, otherwise
 * the launch error. The callers (the Python modules of the package) allocate every
 * output and workspace.
 *
 * Each declaration names the reference launch it replaces: the reference JIT-compiles its
 * kernels and calls hipModuleLaunchKernel through ctypes (hip_attention.py:28-42); the
 * entry points below are what that FFI would bind instead.
 */
#ifndef RDA_H
#define RDA_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

int rda_version(void);

/* ------------------------------------------------------------------ linear path ---------- */
/* Activations: x fp16 rows of K values at a pitch of ldx elements. Outputs: a_q int8 [M, K]
 * row-major, a_scale fp32 [M]. With a rotation, K must be a multiple of group (256 or 128) and
 * <= 16384 (the rotated row is held in LDS). */

/* quant_pack_a, int8_gemm.py:67 (kernel int8_gemm.hip:93-103): per-row absmax int8, no rotation.
 * Any K that is a multiple of 16. */
int rda_quant_pack_a(const void* x, long ldx, void* a_q, float* a_scale, int M, int K, void* stream);

/* rot_quant_pack_a, int8_gemm.py:67 (int8_gemm.hip:245-247): block Hadamard + per-row int8. */
int rda_rot_quant_pack_a(const void* x, long ldx, void* a_q, float* a_scale, int M, int K, int group, void* stream);

/* situ_rot_quant_pack_a, int8_gemm.py:67 via linear(situ=True) (int8_gemm.hip:249-251):
 * x is [M, 2K] = [hidden | gate] at pitch ldx. */
int rda_situ_rot_quant_pack_a(const void* x, long ldx, void* a_q, float* a_scale, int M, int K, int group, void* stream);

/* swiglu_rot_quant_pack_a, int8_gemm.py:67 via linear(up=...) (int8_gemm.hip:253-255):
 * fp16(fp16(silu(gate)) * up) -> rotate -> quantize; gate and up fp16 [M, K] contiguous. */
int rda_swiglu_rot_quant_pack_a(const void* gate, const void* up, void* a_q, float* a_scale, int M, int K, int group, void* stream);

/* gate_rot_quant_pack_a, int8_gemm.py:67 via linear(gate=...) (int8_gemm.hip:257-259):
 * fp16(x * fp16(sigmoid(gate))) -> rotate -> quantize. */
int rda_gate_rot_quant_pack_a(const void* x, const void* gate, void* a_q, float* a_scale, int M, int K, int group, void* stream);

/* mod_rot_quant_pack_a, int8_gemm.py:184-185 (int8_gemm.hip:261-264): RMSNorm (w zero-centred,
 * fp32 [K]) -> (fp16 s = 1 + scale, t = shift, one row per L rows) -> rotate(256) -> quantize.
 * K <= 8192. */
int rda_mod_rot_quant_pack_a(const void* x, void* a_q, float* a_scale, int M, int K, const float* w, const void* s, const void* t, int L, float eps,
                             void* stream);

/* rot_quant_pack_a_i4, int8_gemm.py:100 (int8_gemm.hip:266-268): W4A4 activations, int4 values in
 * [-7, 7] stored one per byte in a_q, scale = max(absmax, 1e-10) / 7. */
int rda_rot_quant_pack_a_i4(const void* x, long ldx, void* a_q, float* a_scale, int M, int K, int group, void* stream);

/* gemm (+ pack_b), int8_gemm.py:72-79 (int8_gemm.hip:270-276, 315-411). W int8 [N, K] row-major
 * read in place (no per-call re-layout). c = fp16(((float)acc * a_scale[m]) * w_scale[n]
 * (+ bias[n])); with res: c = fp16(res + fp16(res_gate[m / L] * y)). N % 64 == 0, K % 64 == 0.
 * bias, res, res_gate fp16 or NULL. */
int rda_gemm(const void* a_q, const void* w, const float* a_scale, const float* w_scale, const void* bias, void* c, int M, int N, int K, const void* res,
             const void* res_gate, int L, void* stream);

/* gemm_i4, int8_gemm.py:100 (int8_gemm.hip:412): W4A4 with per-channel fp32 w_scale. w_packed
 * [N, K/2] signed int4, low nibble = even k; a_q from rda_rot_quant_pack_a_i4. K % 128 == 0. */
int rda_gemm_i4(const void* a_q, const void* w_packed, const float* a_scale, const float* w_scale, const void* bias, void* c, int M, int N, int K,
                void* stream);

/* W4A8 (no reference kernel; the convrot_w4a4_forward hook at int8_gemm.py:90-102 is its caller
 * shape): int8 activations, int4 weights [N, K/2], fp16 group scales [N, K / group]. After each
 * group the int32 partial p is folded as y = fma((float)p, scale, y); c = fp16(y * a_scale[m]
 * (+ bias[n])). group % 64 == 0, K % 128 == 0. */
int rda_gemm_w4a8(const void* a_q, const void* w_packed, const float* a_scale, const void* group_scales, const void* bias, void* c, int M, int N, int K,
                  int group, void* stream);

/* W4A8 on k-interleaved activations (no reference counterpart; linear_w4a8's own quantize-then-GEMM pair):
 * rda_rot_quant_pack_a_il writes the same int8 codes and scales as rda_rot_quant_pack_a, but each 8 values of k as
 * its 4 even ones, then its 4 odd ones -- the order in which the GEMM widens packed int4 weights (low nibbles, then
 * high ones), so that it needs no byte interleave; rda_gemm_w4a8_il takes those activations and gives rda_gemm_w4a8's
 * outputs bit for bit. It takes only shapes its direct-copy kernel runs: group 128, K % 128 == 0, N % 128 == 0,
 * K up to 40960 (the block's group scales are staged in LDS), a_q, w_packed, c and group_scales on 16-byte and bias
 * on 8-byte boundaries (RDA_ERR_INVALID otherwise). */
int rda_rot_quant_pack_a_il(const void* x, long ldx, void* a_q, float* a_scale, int M, int K, int group, void* stream);
int rda_gemm_w4a8_il(const void* a_q, const void* w_packed, const float* a_scale, const void* group_scales, const void* bias, void* c, int M, int N,
                     int K, int group, void* stream);

/* Parity entry (no reference counterpart): the raw int32 accumulators [M, N] of the int8 x int8
 * (w_int4 = 0) or int8 x int4 (w_int4 = 1) product. */
int rda_gemm_acc(const void* a_q, const void* w, int w_int4, void* acc, int M, int N, int K, void* stream);

/* ------------------------------------------------------------------ attention ------------ */
/* q, out (B, H, Lq, 128) fp16 and k, v (B, Hkv, Lk, 128) fp16 with a contiguous last dimension;
 * strides[12] = element strides (batch, head, row) of q, k, v, out. scale is the softmax scale
 * (the kernels use scale * log2 e). k and v (and the int8-QK workspace) must start 16-byte aligned
 * with strides that are multiples of 8 (their rows are copied to LDS 16 bytes at a time); other
 * layouts are rejected with 1. */

/* attn (+ pack_kv), hip_attention.py:61-66 (hip_attention.hip:30-54, 280-373). No workspace. */
int rda_attn(const void* q, const void* k, const void* v, void* out, int B, int H, int Hkv, int Lq, int Lk, const long* strides, float scale,
             void* stream);

/* Workspace bytes for the int8-QK path (hip_attention.py:58 allocates the reference's). */
size_t rda_attn_i8_workspace(int B, int Hkv, int Lk);

/* pack_kv_i8, hip_attention.py:61-63 (hip_attention.hip:56-103): per-key int8 K + fp32 scales. */
int rda_pack_k_i8(const void* k, void* workspace, int B, int Hkv, int Lk, long skb, long skh, long skl, void* stream);

/* attn_i8, hip_attention.py:64-66 (hip_attention.hip:160-278): int8 QK^T, fp16 PV. */
int rda_attn_i8(const void* q, const void* workspace, const void* v, void* out, int B, int H, int Hkv, int Lq, int Lk, const long* strides, float scale,
                void* stream);

/* rda_attn / rda_attn_i8 with the workgroup layout fixed: waves 4 (four-wave workgroups of 128 rows of one head) or 12
 * (twelve-wave workgroups of 384 rows of the (batch, head, row) range; needs Lq >= 384), or 0 for the choice
 * rda_attn makes (twelve waves when Lq >= 384 and their grid covers at least two thirds of the CUs). Both layouts
 * give the same bits. No reference counterpart: for tests and measurement of each layout. Other values return 1. */
int rda_attn_waves(const void* q, const void* k, const void* v, void* out, int B, int H, int Hkv, int Lq, int Lk, const long* strides, float scale,
                   int waves, void* stream);
int rda_attn_i8_waves(const void* q, const void* workspace, const void* v, void* out, int B, int H, int Hkv, int Lq, int Lk, const long* strides,
                      float scale, int waves, void* stream);

/* ------------------------------------------------------------------ decode path ---------- */

/* rotate, int8_gemv.py:42-45 (int8_gemv.hip:31-52): fp32 rows of `group` (a power of 4). */
int rda_rotate(const float* x, float* out, int rows, int group, void* stream);

/* gemv_i8, int8_gemv.py:60-63 (int8_gemv.hip:54-85): out[n] = scale[n] * dot(w[n], x) (+ bias[n]).
 * x_half = 0: x, out fp32; x_half = 1: x, out fp16. K % 512 == 0, K <= 16384; x 16-byte aligned. */
int rda_gemv_i8(const void* x, int x_half, const void* w, const float* scale, const float* bias, void* out, int N, int K, void* stream);

/* rotate followed by gemv_i8, int8_gemv.py:58-63 (int8_gemv.hip:31-85) -- linear_forward's single-token ConvRot
 * linear -- as one launch: out (fp32) equals, bit for bit, rda_rotate of fp32 x in K / group groups of `group` (4, 16,
 * 64 or 256) followed by rda_gemv_i8 of the rotated row. `rotated` (K floats, or NULL) receives that rotation too, for
 * further linears of the same input. K % 512 == 0, K <= 16384; x and rotated 16-byte aligned and not overlapping
 * (RDA_ERR_INVALID otherwise); x is not modified. */
int rda_rotate_gemv_i8(const float* x, int group, const void* w, const float* scale, const float* bias, float* out, float* rotated, int N, int K,
                       void* stream);

/* `count` (1-4) gemv_i8 launches over one input row as one launch -- the sibling linears one parent forward applies
 * to the same activation, each a linear_forward call in the reference (int8_gemv.py:48-64; q, k, v of an attention
 * layer, gate and up of an MLP). Matrix i: w[i] int8 [n[i], K], scale[i] fp32 [n[i]], bias[i] fp32 [n[i]] (bias
 * itself or any bias[i] may be NULL), out[i] [n[i]] in x's type. group 0: x_half as in rda_gemv_i8, and each out[i]
 * equals rda_gemv_i8's bit for bit; group 4, 16, 64 or 256: fp32 x is rotated first and each out[i] equals
 * rda_rotate_gemv_i8's bit for bit, `rotated` (K floats, or NULL) receiving the rotation. The pointer and size
 * arrays are host memory, read during the call. K % 512 == 0, K <= 8192; x and rotated 16-byte aligned and not
 * overlapping. */
int rda_gemv_i8_multi(const void* x, int x_half, int group, int count, const void* const* w, const float* const* scale, const float* const* bias,
                      void* const* out, const int* n, int K, float* rotated, void* stream);

/* gemv_bf16, int8_gemv.py:97 (int8_gemv.hip:87-119): fp32 logits of a bf16 table. K % 256 == 0, N % 8 == 0. */
int rda_gemv_bf16(const float* x, const void* w, float* out, int N, int K, void* stream);

/* attn_decode, int8_gemv.py:111-112 (int8_gemv.hip:121-180): q (B, 1, H, 128), k/v (B, capacity,
 * Hkv, 128) fp32, lengths (B,) int32 read on the device (one past capacity counts as capacity); partial (B*H, splits, 128) and stats
 * (B*H, splits, 2) fp32 with splits = rda_decode_splits(). H / Hkv in {1, 2, 4, 8}. */
int rda_attn_decode(const float* q, const float* k, const float* v, const int* lengths, float* partial, float* stats, int B, int H, int Hkv,
                    int capacity, float scale, void* stream);

/* attn_merge, int8_gemv.py:113 (int8_gemv.hip:182-195). */
int rda_attn_merge(const float* partial, const float* stats, float* out, int heads, void* stream);

int rda_decode_splits(void);

/* attention_decode without allocation. No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The same result as
 * rda_attn_decode + rda_attn_merge, bit for bit; out (B, 1, H, 128) fp32. The split partials live in a device
 * array inside the library (4.06 MiB per GPU, held until the process ends), so B * H must be <= 256: larger
 * calls return 1 (hipErrorInvalidValue) without launching. Calls that overlap on one GPU share that array and
 * race; serialise them (one stream, or events). Nothing is allocated, freed or cleared. */
int rda_attention_decode_noalloc(const float* q, const float* k, const float* v, const int* lengths, float* out, int B, int H, int Hkv,
                                 int capacity, float scale, void* stream);

/* ------------------------------------------------------------------ RMSNorm -------------- */
/* x (B, H, L, D) fp16 addressed by element strides sb, sh, sl (last dim contiguous); w fp32 [D],
 * zero-centred (the kernels use w + 1); y contiguous (B, H, L, D). */

/* rms_norm_head, rms_norm.py:36-38 (rms_norm.hip:67-69): D <= 128. */
int rda_rms_norm_head(const void* x, const float* w, void* y, int B, int H, int L, int D, long sb, long sh, long sl, float eps, void* stream);

/* rms_norm_row, rms_norm.py:36-38 (rms_norm.hip:71-73): 128 < D <= 8192. */
int rda_rms_norm_row(const void* x, const float* w, void* y, int B, int H, int L, int D, long sb, long sh, long sl, float eps, void* stream);

/* rms_norm_rope, rms_norm.py:49-51 (rms_norm.hip:75-77): D == 128, freqs fp32 [.., L, 64, 2, 2],
 * fb = batch stride in 2x2 matrices (0 broadcasts). */
int rda_rms_norm_rope(const void* x, const float* w, void* y, int B, int H, int L, int D, long sb, long sh, long sl, float eps, const float* freqs,
                      long fb, void* stream);

/* ------------------------------------------------------------------ calibration -------- */
/* Measurement only, no counterpart in the reference: `blocks` workgroups of four waves each issue `iters` rounds of
 * 8 independent MFMAs (int8 = 1: v_mfma_i32_32x32x32_i8, 65536 ops each; int8 = 0: v_mfma_f32_32x32x16_f16, 32768
 * FLOP each), back to back. out: blocks * 256 ints (written to keep the products live); clocks[0] = shader-clock
 * ticks and clocks[1] = 100 MHz real-time ticks over the run of workgroup 0's first wave. */
int rda_calib_mfma_peak(int int8, int blocks, int iters, int* out, long long* clocks, void* stream);

/* Measurement only, no counterpart in the reference: as rda_calib_mfma_peak, with each lane's operands taken from
 * `operands` (16-byte aligned; blocks * 256 * 16 fragments of 16 bytes: lane l of workgroup b uses fragments
 * (b * 256 + l) * 16 + 0..7 as A and + 8..15 as B, fp16 or int8 by `int8`), so the sustained rate on a given
 * distribution of values (the matrix cores' power, and so the clock, depends on them) can be measured. */
int rda_calib_mfma_peak_data(int int8, int blocks, int iters, const void* operands, int* out, long long* clocks, void* stream);

#ifdef __cplusplus
}
#endif

#endif
