// RMSNorm for fp16 rows with fp32 math, reading and writing each value once, plus the QK-norm +
// RoPE variant of a Krea 2 block.
//
// norm_row (rms_norm.hip:9-65): TPR threads share a row, thread t owns the 8-value chunks
// t + c TPR. Its sum of squares is accumulated with FMAs chunk by chunk; the partial sums are
// folded by xor butterflies inside each 32-lane half-wave (16, 8, 4, 2, 1; 8, 4, 2, 1 for TPR 16)
// and, for TPR 256, the eight half-wave sums are added in order. rstd = 1 / sqrt(sum / D + eps)
// (correctly rounded, where the reference has rsqrtf), y = fp16(x * rstd * (w + 1)).
// Rows are addressed with (b, h, l) strides, so Q and K are read straight from a linear output;
// the result is written contiguous (B, H, L, D).
#include "common.h"

#define NT 256

template <int TPR, int CHUNKS, bool ROPE>
__global__ __launch_bounds__(NT) void norm_kernel(const half_t* __restrict__ X, const float* __restrict__ W, half_t* __restrict__ Y, int rows, int D, int L,
                                                  int H, long sb, long sh, long sl, float eps, const f4* __restrict__ F, long fb) {
    __shared__ float red[NT / 32];
    const int t = threadIdx.x % TPR, n = blockIdx.x * (NT / TPR) + threadIdx.x / TPR;
    if (TPR < NT && n >= rows) return;
    // Heads go first, so a block reads neighbouring heads of one token.
    const int h = n % H, l = (n / H) % L, b = n / H / L;
    const h8* x = (const h8*)(X + b * sb + h * sh + l * sl);
    // Every load is issued up front, x then the weight, with no load under a branch (chunks past D / 8
    // re-read chunk 0 and are not used), so the weight arrives during the reduction instead of after it;
    // the host picks CHUNKS as the chunks D needs per thread.
    h8 v[CHUNKS];
    f4 wv[CHUNKS][2];
#pragma unroll
    for (int c = 0; c < CHUNKS; c++) {
        const int i = t + c * TPR;
        v[c] = x[i < D / 8 ? i : 0];
    }
#pragma unroll
    for (int c = 0; c < CHUNKS; c++) {
        const int i = t + c * TPR, iw = i < D / 8 ? i : 0;
        wv[c][0] = ((const f4*)W)[iw * 2];
        wv[c][1] = ((const f4*)W)[iw * 2 + 1];
    }
    float sum = 0.f;
#pragma unroll
    for (int c = 0; c < CHUNKS; c++) {
        const int i = t + c * TPR;
        if (i < D / 8) {
#pragma unroll
            for (int j = 0; j < 8; j++) sum = __builtin_fmaf((float)v[c][j], (float)v[c][j], sum);
        }
    }
    sum = xor_butterfly_sum<(TPR < 32 ? TPR : 32)>(sum);
    if (TPR > 32) {
        if ((threadIdx.x & 31) == 0) red[threadIdx.x >> 5] = sum;
        __syncthreads();
        sum = 0.f;
#pragma unroll
        for (int i = 0; i < NT / 32; i++) sum += red[i];
    }
    const float rstd = 1.f / sqrtf(sum / (float)D + eps);
    h8* y = (h8*)(Y + ((size_t)(b * H + h) * L + l) * D);
#pragma unroll
    for (int c = 0; c < CHUNKS; c++) {
        const int i = t + c * TPR;
        if (i < D / 8) {
            const f4 lo = wv[c][0], hi = wv[c][1];
            h8 o;
#pragma unroll
            for (int j = 0; j < 8; j++) o[j] = to_half((float)v[c][j] * rstd * ((j < 4 ? lo[j & 3] : hi[j & 3]) + 1.f));
            if (ROPE) {
                // rms_norm.hip:48-61: a = fma(m1, x1, fp32(m0 x0)), c = fma(m3, x1, fp32(m2 x0)), each
                // rounded to fp32 and then to fp16 (to_half), like the reference.
                const f4* f = F + b * fb + (long)l * (D / 2) + i * 4;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const f4 m = f[j];
                    const float x0 = (float)o[j * 2], x1 = (float)o[j * 2 + 1];
                    const float a = __builtin_fmaf(m[1], x1, m[0] * x0), cc = __builtin_fmaf(m[3], x1, m[2] * x0);
                    o[j * 2] = to_half(a);
                    o[j * 2 + 1] = to_half(cc);
                }
            }
            y[i] = o;
        }
    }
}

static bool norm_ok(int B, int H, int L, int D) { return B > 0 && H > 0 && L > 0 && D > 0 && D % 8 == 0; }

extern "C" {

// rms_norm_head (rms_norm.hip:67-69): D <= 128, 16 threads per row.
int rda_rms_norm_head(const void* x, const float* w, void* y, int B, int H, int L, int D, long sb, long sh, long sl, float eps, void* stream) {
    if (!norm_ok(B, H, L, D) || D > 128) return RDA_ERR_INVALID;
    const int rows = B * H * L;
    hipLaunchKernelGGL((norm_kernel<16, 1, false>), dim3((rows + 15) / 16), dim3(NT), 0, (hipStream_t)stream, (const half_t*)x, w, (half_t*)y, rows, D, L,
                       H, sb, sh, sl, eps, nullptr, 0L);
    return (int)hipGetLastError();
}

// rms_norm_row (rms_norm.hip:71-73): 128 < D <= 8192, 256 threads per row.
int rda_rms_norm_row(const void* x, const float* w, void* y, int B, int H, int L, int D, long sb, long sh, long sl, float eps, void* stream) {
    if (!norm_ok(B, H, L, D) || D > 8192) return RDA_ERR_INVALID;
    const int rows = B * H * L;
    // Chunks per thread: as many as D needs (the loads of a thread's unused chunks are not free).
    auto launch = [&](auto kern) {
        hipLaunchKernelGGL(kern, dim3(rows), dim3(NT), 0, (hipStream_t)stream, (const half_t*)x, w, (half_t*)y, rows, D, L, H, sb, sh, sl, eps, nullptr,
                           0L);
        return (int)hipGetLastError();
    };
    switch ((D / 8 + NT - 1) / NT) {
    case 1: return launch(norm_kernel<NT, 1, false>);
    case 2: return launch(norm_kernel<NT, 2, false>);
    case 3: return launch(norm_kernel<NT, 3, false>);
    default: return launch(norm_kernel<NT, 4, false>);
    }
}

// rms_norm_rope (rms_norm.hip:75-77): QK-norm over D = 128 then RoPE; freqs [.., L, 64, 2, 2] fp32,
// fb = the batch stride in 2x2 matrices (0 to broadcast one batch).
int rda_rms_norm_rope(const void* x, const float* w, void* y, int B, int H, int L, int D, long sb, long sh, long sl, float eps, const float* freqs,
                      long fb, void* stream) {
    if (!norm_ok(B, H, L, D) || D != 128) return RDA_ERR_INVALID;
    const int rows = B * H * L;
    hipLaunchKernelGGL((norm_kernel<16, 1, true>), dim3((rows + 15) / 16), dim3(NT), 0, (hipStream_t)stream, (const half_t*)x, w, (half_t*)y, rows, D, L,
                       H, sb, sh, sl, eps, (const f4*)freqs, fb);
    return (int)hipGetLastError();
}

int rda_version(void) { return 1; }

}  // extern "C"
