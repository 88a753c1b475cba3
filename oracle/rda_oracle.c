/*
 * CPU oracle for the quantized-inference hot path. TEST INFRASTRUCTURE ONLY:
 * the tests, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this
 * library as the source of reference results. The product path never links or calls it.
 *
 * Every function restates, operation by operation, the arithmetic that the
 * reference kernels perform (citations are file:line in the reference repo),
 * with the three documented substitutions the HIP kernels also make so that
 * GPU and oracle agree bit for bit:
 *   - expf / __builtin_amdgcn_exp2f  ->  orc_expf / orc_exp2f below (Cody-Waite
 *     reduction + degree-7 Taylor polynomial; every step is an IEEE fp32 op).
 *   - rsqrtf(v)                      ->  1.0f / sqrtf(v) (both correctly rounded).
 *   - a rotation group of 128 (not in the reference) is H2 (x) H4 (x) H4 (x) H4.
 * Built with -ffp-contract=off so that gcc never fuses a multiply and an add
 * that the kernels keep separate; every fused multiply-add is an explicit fmaf.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* ---------------------------------------------------------------- fp16 --- */

static float h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu, bits;
    if (e == 0) {
        float f = (float)m * (1.0f / 16777216.0f); /* exact: m < 2^10, scale 2^-24 */
        return sign ? -f : f;
    }
    if (e == 31) bits = sign | 0x7f800000u | (m << 13);
    else bits = sign | ((e - 15 + 127) << 23) | (m << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* Round to nearest even, with subnormals and overflow to infinity, as v_cvt_f16_f32. */
static uint16_t f2h(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    if (ax < 0x38800000u) {                                    /* below 2^-14: subnormal */
        float af;
        memcpy(&af, &ax, 4);
        uint32_t m = (uint32_t)rintf(af * 16777216.0f); /* exact scaling, then RNE */
        return (uint16_t)(sign | m);
    }
    uint32_t h = ((((ax >> 23) - 127 + 15) << 10) | ((ax & 0x7fffffu) >> 13));
    uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

static float r16(float f) { return h2f(f2h(f)); }

float orc_h2f(uint16_t h) { return h2f(h); }
uint16_t orc_f2h(float f) { return f2h(f); }

/* ------------------------------------------------------- exp, exp2 ------- */
/* exp(x) = 2^n * e^r with n = rint(x * log2 e) and r = x - n ln2 (Cody-Waite:
 * ln2 split into a 16-bit head and a tail), e^r by a degree-7 Taylor polynomial
 * in Horner form (|r| <= 0.35, truncation < 0.05 ulp), 2^n applied as two exact
 * power-of-two factors. Inputs below -88 return 0 (1 + e^x == 1 there, which is
 * all the activations need); above 88.72 return +inf. */
#define LN2_HI 0.693145751953125f      /* 0x3f317200 */
#define LN2_LO 1.42860682030941723e-6f /* ln 2 - LN2_HI */
#define LOG2E 1.44269504088896341f

static float pow2i(int n) {
    uint32_t bits = (uint32_t)(n + 127) << 23;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static float scale2(float p, int n) {
    int h = n / 2;
    return (p * pow2i(h)) * pow2i(n - h);
}

float orc_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return INFINITY;
    if (x < -88.0f) return 0.0f;
    float n = rintf(x * LOG2E);
    float r = fmaf(-n, LN2_HI, x);
    r = fmaf(-n, LN2_LO, r);
    float p = 1.98412701138295233e-4f; /* 1/5040 */
    p = fmaf(p, r, 1.38888892251998186e-3f); /* 1/720 */
    p = fmaf(p, r, 8.33333376795053482e-3f); /* 1/120 */
    p = fmaf(p, r, 4.16666679084300995e-2f); /* 1/24 */
    p = fmaf(p, r, 1.66666671633720398e-1f); /* 1/6 */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return scale2(p, (int)n);
}

/* 2^y = 2^n * 2^f, n = rint(y), f = y - n exact; 2^f = e^(f ln2) by the same
 * polynomial with its coefficients multiplied through by powers of ln 2. */
float orc_exp2f(float y) {
    if (y != y) return y;
    if (y >= 128.0f) return INFINITY;
    if (y < -127.0f) return 0.0f;
    float n = rintf(y);
    float f = y - n;
    float p = 1.52527336467755958e-5f; /* ln2^7/5040 */
    p = fmaf(p, f, 1.54035296873189509e-4f); /* ln2^6/720 */
    p = fmaf(p, f, 1.33335578721016645e-3f); /* ln2^5/120 */
    p = fmaf(p, f, 9.61812864989042282e-3f); /* ln2^4/24 */
    p = fmaf(p, f, 5.55041097104549408e-2f); /* ln2^3/6 */
    p = fmaf(p, f, 2.40226507186889648e-1f); /* ln2^2/2 */
    p = fmaf(p, f, 6.93147182464599609e-1f); /* ln2 */
    p = fmaf(p, f, 1.0f);
    return scale2(p, (int)n);
}

/* ------------------------------------------------------ activations ------ */

/* int8_gemm.hip:130-132: fp16 rounding at the points F.silu(gate).mul_(up) rounds. */
float orc_swiglu(float gate, float up) {
    return r16(r16(gate / (1.0f + orc_expf(-gate))) * up);
}

/* int8_gemm.hip:135-137: x * F.sigmoid(gate). */
float orc_sigmoid_gate(float x, float gate) {
    return r16(x * r16(1.0f / (1.0f + orc_expf(-gate))));
}

/* int8_gemm.hip:118-122 */
static float soft_tanh(float x) {
    float ax = fabsf(x), t = orc_exp2f(-2.885390082f * ax), y = (1.0f - t) / (1.0f + t);
    if (ax < 0.02f) y = ax * (1.0f - ax * ax * (1.0f / 3.0f - ax * ax * (2.0f / 15.0f)));
    return x < 0.0f ? -y : y;
}

/* int8_gemm.hip:124-127 */
float orc_situ(float hidden, float gate) {
    float sigmoid = 1.0f / (1.0f + orc_exp2f(-1.442695041f * gate));
    return r16(4.0f * soft_tanh(gate * 0.25f) * sigmoid * 25.0f * soft_tanh(hidden * 0.04f));
}

/* int8_gemm.hip:140-143 */
float orc_modulate(float x, float rstd, float w, float s, float t) {
    return r16(r16(r16(x * rstd * (w + 1.0f)) * s) + t);
}

/* ------------------------------------------------ block Hadamard ------- */

/* int8_gemm.hip:106-109: one H4 step, s = ((a + b) + c) + d. */
static void h4(float *a, float *b, float *c, float *d) {
    float s = *a + *b + *c + *d, a0 = *a, b0 = *b;
    *a = s - 2.0f * *d;
    *b = s - 2.0f * *c;
    *c = s - 2.0f * b0;
    *d = s - 2.0f * a0;
}

/* Rotates one group in place, in fp32, digit by digit from the fastest index:
 * strides 1, 4, 16, 64 for 256 (int8_gemm.hip:193-236, whose two h16 calls
 * around the LDS transpose apply exactly this stage order), and strides 1, 4,
 * 16 followed by an H2 step (a + b, a - b) at stride 64 for 128. */
static void hadamard_group(float *v, int group) {
    for (int stride = 1; stride < 64; stride *= 4)
        for (int q = 0; q < group / 4; q++) {
            int i = (q / stride) * stride * 4 + q % stride;
            h4(&v[i], &v[i + stride], &v[i + 2 * stride], &v[i + 3 * stride]);
        }
    if (group == 256) {
        for (int i = 0; i < 64; i++) h4(&v[i], &v[i + 64], &v[i + 128], &v[i + 192]);
    } else {
        for (int i = 0; i < 64; i++) {
            float a = v[i], b = v[i + 64];
            v[i] = a + b;
            v[i + 64] = a - b;
        }
    }
}

/* The normalisation after the butterflies: 1/16 for 256 (int8_gemm.hip:233, exact),
 * the fp32 rounding of 2^-3.5 for 128. */
static float group_norm(int group) { return group == 256 ? 0.0625f : 0.0883883461356163025f; }

/* ------------------------------------------------------ quantization ------ */

/* int8_gemm.hip:38, 53 */
static void quant_row_i8(const float *y, int K, float mx, int8_t *q, float *scale) {
    float s = fmaxf(mx / 127.0f, 1e-30f);
    *scale = s;
    for (int k = 0; k < K; k++) {
        float f = floorf(y[k] / s + 0.5f);
        f = fminf(fmaxf(f, -128.0f), 127.0f);
        q[k] = (int8_t)(int)f;
    }
}

/* int8_gemm.hip:71, 84 (W4A4 activations, stored one value per byte). */
static void quant_row_i4(const float *y, int K, float mx, int8_t *q, float *scale) {
    float s = fmaxf(mx, 1e-10f) / 7.0f;
    *scale = s;
    for (int k = 0; k < K; k++) {
        float f = rintf(y[k] / s);
        f = fminf(fmaxf(f, -7.0f), 7.0f);
        q[k] = (int8_t)(int)f;
    }
}

/* quant_pack_a (int8_gemm.hip:93-103): per-row absmax of the fp16 input, no rotation. */
void orc_quant_rows(int M, int K, const uint16_t *x, int ldx, int8_t *q, float *scale) {
    static float row[65536];
    for (int m = 0; m < M; m++) {
        float mx = 0.0f;
        for (int k = 0; k < K; k++) {
            row[k] = h2f(x[(size_t)m * ldx + k]);
            mx = fmaxf(mx, fabsf(row[k]));
        }
        quant_row_i8(row, K, mx, q + (size_t)m * K, scale + m);
    }
}

enum { ACT_NONE = 0, ACT_SITU = 1, ACT_SWIGLU = 2, ACT_GATE = 3, ACT_MOD = 4 };

/* The sum of squares of one row in the order of the reference's rms_norm_row
 * (rms_norm.hip:19-37, TPR 256, CHUNKS 4): thread t adds x*x with an FMA over
 * its chunks t + 256c, eight values each; each 32-lane group folds its partial
 * sums by xor butterflies 16, 8, 4, 2, 1; the eight group sums are added in
 * order. For TPR 16 (rms_norm_head, D <= 128) one chunk per thread and the
 * butterflies 8, 4, 2, 1. int8_gemm.hip:168-189 reproduces the TPR-256 order. */
static float row_sum_squares(const float *x, int D, int tpr) {
    float part[256];
    int chunks = tpr == 256 ? 4 : 1;
    for (int t = 0; t < tpr; t++) {
        float s = 0.0f;
        for (int c = 0; c < chunks; c++) {
            int i = t + c * tpr;
            if (i < D / 8)
                for (int j = 0; j < 8; j++) s = fmaf(x[i * 8 + j], x[i * 8 + j], s);
        }
        part[t] = s;
    }
    int width = tpr < 32 ? tpr : 32;
    float groups[8];
    int ngroups = tpr / width;
    for (int g = 0; g < ngroups; g++) {
        float v[32], nv[32];
        for (int i = 0; i < width; i++) v[i] = part[g * width + i];
        for (int o = width / 2; o > 0; o >>= 1) {
            for (int i = 0; i < width; i++) nv[i] = v[i] + v[i ^ o];
            memcpy(v, nv, sizeof(float) * width);
        }
        groups[g] = v[0];
    }
    if (ngroups == 1) return groups[0];
    float total = 0.0f;
    for (int g = 0; g < ngroups; g++) total += groups[g];
    return total;
}

static float rstd_of(float sum, int D, float eps) { return 1.0f / sqrtf(sum / (float)D + eps); }

/* rot_quant<ACT, I4> (int8_gemm.hip:151-243) for every row, with group 256 or 128.
 * x: fp16 rows of width K (2K for SITU, [hidden | gate]) at pitch ldx elements;
 * u: fp16 [M, K] up rows (SWIGLU) or gate rows (GATE);
 * mod_w fp32 [K], mod_s / mod_t fp16 [M / L, K] (MOD);
 * writes q (int8 [M, K]; int4 values in [-7, 7] when i4), scale [M], and when
 * rotated is non-null the fp16 rotated row. */
void orc_rot_quant_rows(int act, int i4, int group, int M, int K, const uint16_t *x, int ldx, const uint16_t *u,
                        const float *mod_w, const uint16_t *mod_s, const uint16_t *mod_t, int L, float eps,
                        int8_t *q, float *scale, uint16_t *rotated) {
    static float row[65536], xin[65536];
    float norm = group_norm(group);
    for (int m = 0; m < M; m++) {
        const uint16_t *xr = x + (size_t)m * ldx;
        float rstd = 0.0f;
        if (act == ACT_MOD) {
            for (int k = 0; k < K; k++) xin[k] = h2f(xr[k]);
            rstd = rstd_of(row_sum_squares(xin, K, 256), K, eps);
        }
        for (int k = 0; k < K; k++) {
            float h = h2f(xr[k]), v;
            switch (act) {
            case ACT_SITU: v = orc_situ(h, h2f(xr[K + k])); break;
            case ACT_SWIGLU: v = orc_swiglu(h, h2f(u[(size_t)m * K + k])); break;
            case ACT_GATE: v = orc_sigmoid_gate(h, h2f(u[(size_t)m * K + k])); break;
            case ACT_MOD: {
                const size_t b = (size_t)(m / (L ? L : 1)) * K + k;
                v = orc_modulate(h, rstd, mod_w[k], h2f(mod_s[b]), h2f(mod_t[b]));
                break;
            }
            default: v = h;
            }
            row[k] = v;
        }
        float mx = 0.0f;
        for (int g = 0; g < K / group; g++) {
            float *v = row + g * group;
            hadamard_group(v, group);
            for (int i = 0; i < group; i++) {
                v[i] = r16(v[i] * norm);
                mx = fmaxf(mx, fabsf(v[i]));
            }
        }
        if (rotated)
            for (int k = 0; k < K; k++) rotated[(size_t)m * K + k] = f2h(row[k]);
        if (i4) quant_row_i4(row, K, mx, q + (size_t)m * K, scale + m);
        else quant_row_i8(row, K, mx, q + (size_t)m * K, scale + m);
    }
}

/* --------------------------------------------------------- epilogues ------ */

/* gemm_body epilogue (int8_gemm.hip:382-383, 394-400):
 *   y = fp16(((float)acc * as[m]) * ws[n] (+ bias[n]))
 *   with R: C = fp16(R + fp16(G[m / L] * y)), contraction off. */
void orc_gemm_epilogue(int M, int N, const int32_t *acc, const float *as, const float *ws, const uint16_t *bias,
                       const uint16_t *R, const uint16_t *G, int L, uint16_t *out) {
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            float y = (float)acc[(size_t)m * N + n] * as[m] * ws[n];
            if (bias) y = y + h2f(bias[n]);
            uint16_t h = f2h(y);
            if (R) {
                float res = h2f(R[(size_t)m * N + n]), gate = h2f(G[(size_t)(m / L) * N + n]);
                h = f2h(res + r16(gate * h2f(h)));
            }
            out[(size_t)m * N + n] = h;
        }
}

/* W4A8 epilogue (no reference counterpart; the W4A8 linear with group-128 fp16 scales):
 * per-group int32 partials p[g][m][n], fp16 group scales gs[n][G];
 *   y = 0; for g in order: y = fma((float)p_g, gs[n][g], y)
 *   out = fp16(y * as[m] (+ bias[n])) */
void orc_w4a8_epilogue(int M, int N, int G, const int32_t *partials, const float *as, const uint16_t *gs,
                       const uint16_t *bias, uint16_t *out) {
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            float y = 0.0f;
            for (int g = 0; g < G; g++)
                y = fmaf((float)partials[((size_t)g * M + m) * N + n], h2f(gs[(size_t)n * G + g]), y);
            float t = y * as[m];
            if (bias) t = t + h2f(bias[n]);
            out[(size_t)m * N + n] = f2h(t);
        }
}

/* ------------------------------------------------------------ rms_norm ---- */

/* norm_row<TPR, CHUNKS> (rms_norm.hip:9-65) for rows addressed as (b, h, l) with
 * element strides sb, sh, sl; rows are enumerated n = (b * H + h) * L + l and
 * written contiguous. With freqs (fp32 [.., L, D/2, 2, 2], batch stride fb in
 * 2x2 matrices) the RoPE step of rms_norm_rope follows (rms_norm.hip:48-61):
 *   a = fma(m1, x1, fp32(m0 * x0)), c = fma(m3, x1, fp32(m2 * x0)), each to fp16. */
void orc_rms_norm(int B, int H, int L, int D, const uint16_t *x, long sb, long sh, long sl, const float *w, float eps,
                  const float *freqs, long fb, uint16_t *y) {
    static float row[65536];
    int tpr = D <= 128 ? 16 : 256;
    for (int b = 0; b < B; b++)
        for (int h = 0; h < H; h++)
            for (int l = 0; l < L; l++) {
                const uint16_t *xr = x + b * sb + h * sh + l * sl;
                for (int i = 0; i < D; i++) row[i] = h2f(xr[i]);
                float rstd = rstd_of(row_sum_squares(row, D, tpr), D, eps);
                uint16_t *yr = y + (((size_t)b * H + h) * L + l) * D;
                for (int i = 0; i < D; i++) yr[i] = f2h(row[i] * rstd * (w[i] + 1.0f));
                if (freqs) {
                    const float *f = freqs + ((size_t)b * fb + (size_t)l * (D / 2)) * 4;
                    for (int p = 0; p < D / 2; p++) {
                        float x0 = h2f(yr[2 * p]), x1 = h2f(yr[2 * p + 1]);
                        const float *m = f + p * 4;
                        float a = fmaf(m[1], x1, m[0] * x0), c = fmaf(m[3], x1, m[2] * x0);
                        yr[2 * p] = f2h(a);
                        yr[2 * p + 1] = f2h(c);
                    }
                }
            }
}

/* --------------------------------------------------- decode rotate ------- */

/* rotate (int8_gemv.hip:31-52): fp32 H4 steps at strides 1, 4, 16, ... < group,
 * then times 1/sqrt(group) (exact for a power of 4). */
void orc_rotate_f32(int rows, int group, const float *x, float *out) {
    static float s[65536];
    float norm = 1.0f / sqrtf((float)group);
    for (int r = 0; r < rows; r++) {
        memcpy(s, x + (size_t)r * group, sizeof(float) * group);
        for (int stride = 1; stride < group; stride *= 4)
            for (int q = 0; q < group / 4; q++) {
                int i = (q / stride) * stride * 4 + q % stride;
                float a = s[i], b = s[i + stride], c = s[i + 2 * stride], d = s[i + 3 * stride];
                float sum = a + b + c + d;
                s[i] = sum - 2.0f * d;
                s[i + stride] = sum - 2.0f * c;
                s[i + 2 * stride] = sum - 2.0f * b;
                s[i + 3 * stride] = sum - 2.0f * a;
            }
        for (int i = 0; i < group; i++) out[(size_t)r * group + i] = s[i] * norm;
    }
}

/* ------------------------------------------- attention Q/K quantization --- */

/* pack_kv_i8 / attn_i8 (hip_attention.hip:85, 91, 183, 192): per-row absmax over
 * D values, s = max(mx / 127, 1e-30), k8 = rint(k / s) (no clamp needed: |k/s| <= 127). */
void orc_quant_rows_rint(int rows, int D, const uint16_t *x, long ld, int8_t *q, float *scale) {
    for (int r = 0; r < rows; r++) {
        float mx = 0.0f;
        for (int d = 0; d < D; d++) mx = fmaxf(mx, fabsf(h2f(x[r * ld + d])));
        float s = fmaxf(mx / 127.0f, 1e-30f);
        scale[r] = s;
        for (int d = 0; d < D; d++) q[(size_t)r * D + d] = (int8_t)(int)rintf(h2f(x[r * ld + d]) / s);
    }
}
