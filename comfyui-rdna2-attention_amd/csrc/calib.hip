// Measurement only (no reference counterpart): the matrix-core rate this GPU sustains, the denominator next to the
// nominal peaks. Every wave issues chains of independent MFMAs back to back (8 accumulators, so no product waits for
// the one before it), 4 waves per workgroup and enough workgroups for several waves per SIMD. The first wave of
// workgroup 0 also reads the shader clock (s_memtime) and the 100 MHz real-time counter (s_memrealtime) at its start
// and end, so the caller can report the clock the products ran at.
//
// The operands either stay fixed per lane (small integers: few bits toggle in the multipliers) or come from a buffer
// of caller-supplied values (e.g. N(0, 1) fp16, uniform int8), eight A and eight B fragments per lane that the
// products cycle through. The chip's clock under sustained matrix work depends on those values: with random operands
// it settles lower, and that rate -- not the nominal one -- is what a kernel on random data can reach.
#include "common.h"

#define CHAINS 8

template <bool I8, bool DATA>
__global__ __launch_bounds__(256) void mfma_peak_kernel(int iters, const i4v* __restrict__ src, int* __restrict__ out, long long* __restrict__ clocks) {
    const int t = threadIdx.x;
    long long c0 = 0, r0 = 0;
    if (blockIdx.x == 0 && t == 0) {
        c0 = (long long)__builtin_amdgcn_s_memtime();
        r0 = (long long)__builtin_amdgcn_s_memrealtime();
    }
    int sum = 0;
    // DATA: fragments f (A) and 8 + f (B) of this lane are src[(block * 256 + t) * 16 + f]. Rounds alternate between
    // two pairings of the A and B fragments (the loop runs them in pairs, plus one for an odd count).
    const i4v* lsrc = DATA ? src + ((size_t)blockIdx.x * 256 + t) * 16 : nullptr;
    if constexpr (I8 && DATA) {
        i4v a[CHAINS], b[CHAINS];
#pragma unroll
        for (int c = 0; c < CHAINS; c++) {
            a[c] = lsrc[c];
            b[c] = lsrc[CHAINS + c];
        }
        i16v acc[CHAINS];
#pragma unroll
        for (int c = 0; c < CHAINS; c++) acc[c] = (i16v){};
        for (int i = 0; i + 1 < iters; i += 2) {
#pragma unroll
            for (int c = 0; c < CHAINS; c++) acc[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[c], b[(c + 3) % CHAINS], acc[c], 0, 0, 0);
#pragma unroll
            for (int c = 0; c < CHAINS; c++) acc[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[c], b[(c + 4) % CHAINS], acc[c], 0, 0, 0);
        }
        if (iters & 1)
#pragma unroll
            for (int c = 0; c < CHAINS; c++) acc[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[c], b[(c + 3) % CHAINS], acc[c], 0, 0, 0);
#pragma unroll
        for (int c = 0; c < CHAINS; c++)
#pragma unroll
            for (int r = 0; r < 16; r++) sum += acc[c][r];
    } else if constexpr (DATA) {
        h8 a[CHAINS], b[CHAINS];
#pragma unroll
        for (int c = 0; c < CHAINS; c++) {
            a[c] = __builtin_bit_cast(h8, lsrc[c]);
            b[c] = __builtin_bit_cast(h8, lsrc[CHAINS + c]);
        }
        f16v acc[CHAINS];
#pragma unroll
        for (int c = 0; c < CHAINS; c++) acc[c] = (f16v){};
        for (int i = 0; i + 1 < iters; i += 2) {
#pragma unroll
            for (int c = 0; c < CHAINS; c++) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[c], b[(c + 3) % CHAINS], acc[c], 0, 0, 0);
#pragma unroll
            for (int c = 0; c < CHAINS; c++) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[c], b[(c + 4) % CHAINS], acc[c], 0, 0, 0);
        }
        if (iters & 1)
#pragma unroll
            for (int c = 0; c < CHAINS; c++) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[c], b[(c + 3) % CHAINS], acc[c], 0, 0, 0);
#pragma unroll
        for (int c = 0; c < CHAINS; c++)
#pragma unroll
            for (int r = 0; r < 16; r++) sum += (int)acc[c][r];
    } else if constexpr (I8) {
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
    if (int8) hipLaunchKernelGGL((mfma_peak_kernel<true, false>), dim3(blocks), dim3(256), 0, (hipStream_t)stream, iters, nullptr, out, clocks);
    else hipLaunchKernelGGL((mfma_peak_kernel<false, false>), dim3(blocks), dim3(256), 0, (hipStream_t)stream, iters, nullptr, out, clocks);
    return (int)hipGetLastError();
}

int rda_calib_mfma_peak_data(int int8, int blocks, int iters, const void* operands, int* out, long long* clocks, void* stream) {
    if (blocks <= 0 || iters <= 0 || !operands || ((uintptr_t)operands & 15) != 0) return RDA_ERR_INVALID;
    const i4v* src = (const i4v*)operands;
    if (int8) hipLaunchKernelGGL((mfma_peak_kernel<true, true>), dim3(blocks), dim3(256), 0, (hipStream_t)stream, iters, src, out, clocks);
    else hipLaunchKernelGGL((mfma_peak_kernel<false, true>), dim3(blocks), dim3(256), 0, (hipStream_t)stream, iters, src, out, clocks);
    return (int)hipGetLastError();
}

}  // extern "C"
