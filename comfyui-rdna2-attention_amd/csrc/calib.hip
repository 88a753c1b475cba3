// Measurement only (no reference counterpart): the matrix-core rate this GPU sustains, the denominator next to the
// nominal peaks. Every wave issues chains of independent MFMAs back to back (8 accumulators, so no product waits for
// the one before it), 4 waves per workgroup and enough workgroups for several waves per SIMD. The first wave of
// workgroup 0 also reads the shader clock (s_memtime) and the 100 MHz real-time counter (s_memrealtime) at its start
// and end, so the caller can report the clock the products ran at.
#include "common.h"

#define CHAINS 8

template <bool I8>
__global__ __launch_bounds__(256) void mfma_peak_kernel(int iters, int* __restrict__ out, long long* __restrict__ clocks) {
    const int t = threadIdx.x;
    long long c0 = 0, r0 = 0;
    if (blockIdx.x == 0 && t == 0) {
        c0 = (long long)__builtin_amdgcn_s_memtime();
        r0 = (long long)__builtin_amdgcn_s_memrealtime();
    }
    int sum = 0;
    if constexpr (I8) {
        const i4v a = {t, t + 1, t + 2, t + 3}, b = {t ^ 5, t ^ 6, t ^ 7, t ^ 8};
        i16v acc[CHAINS];
#pragma unroll
        for (int c = 0; c < CHAINS; c++) acc[c] = (i16v){};
        for (int i = 0; i < iters; i++)
#pragma unroll
            for (int c = 0; c < CHAINS; c++) acc[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc[c], 0, 0, 0);
#pragma unroll
        for (int c = 0; c < CHAINS; c++)
#pragma unroll
            for (int r = 0; r < 16; r++) sum += acc[c][r];
    } else {
        h8 a, b;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            a[e] = (half_t)(float)((t + e) & 7);
            b[e] = (half_t)(float)((t ^ e) & 3);
        }
        f16v acc[CHAINS];
#pragma unroll
        for (int c = 0; c < CHAINS; c++) acc[c] = (f16v){};
        for (int i = 0; i < iters; i++)
#pragma unroll
            for (int c = 0; c < CHAINS; c++) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[c], 0, 0, 0);
#pragma unroll
        for (int c = 0; c < CHAINS; c++)
#pragma unroll
            for (int r = 0; r < 16; r++) sum += (int)acc[c][r];
    }
    out[(size_t)blockIdx.x * 256 + t] = sum;  // keeps the products live
    if (blockIdx.x == 0 && t == 0) {
        const long long c1 = (long long)__builtin_amdgcn_s_memtime(), r1 = (long long)__builtin_amdgcn_s_memrealtime();
        clocks[0] = c1 - c0;
        clocks[1] = r1 - r0;
    }
}

extern "C" {

int rda_calib_mfma_peak(int int8, int blocks, int iters, int* out, long long* clocks, void* stream) {
    if (blocks <= 0 || iters <= 0) return RDA_ERR_INVALID;
    if (int8) hipLaunchKernelGGL(mfma_peak_kernel<true>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, iters, out, clocks);
    else hipLaunchKernelGGL(mfma_peak_kernel<false>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, iters, out, clocks);
    return (int)hipGetLastError();
}

}  // extern "C"
