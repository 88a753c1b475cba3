// int8 GEMM on CDNA4 matrix cores: C[m, n] = sum_k A[m, k] W[n, k], int32 accumulators from
// v_mfma_i32_32x32x32_i8, with a dequantizing epilogue.
//
// A: int8 activations row-major [M, K] (written by the rotate-quant pass).
// W: int8 weights row-major [N, K], or signed int4 packed two per byte [N, K/2] with the low
//    nibble holding the even k (int8_gemm.hip:62, 85); int4 is widened to int8 on its way into
//    LDS, so the matrix cores always see int8 x int8.
// Epilogues:
//   PER_CHANNEL  y = fp16(((float)acc * as[m]) * ws[n] (+ bias[n])), optionally
//                C = fp16(R + fp16(G[m / L] * y))            (int8_gemm.hip:371-405)
//   GROUP_SCALED W4A8 with fp16 group scales gs[n, k / group]: after every group the int32
//                partial is folded into an fp32 sum, y = fma((float)p, gs, y), in group order;
//                C = fp16(y * as[m] (+ bias[n]))
//   RAW_ACC      the int32 accumulators themselves (parity checks).
//
// A workgroup of four wave64s computes a BM x BN tile; operands stream through a double
// buffered LDS stage in 64-byte k slices (row pitch 80 B, so the 16-byte fragment reads of 16
// consecutive rows hit distinct banks). Each wave owns a (BM/WM) x (BN/WN) sub-tile of 32x32
// MFMA blocks. In a 32x32 block, lane l supplies row l % 32 of A (and of W) at k offset
// 16 * (l / 32) within each 32-wide k step, and receives C[8 (r / 4) + 4 (l / 32) + r % 4][l % 32]
// in accumulator register r.
#include "common.h"

enum Epi { PER_CHANNEL = 0, GROUP_SCALED = 1, RAW_ACC = 2 };

#define BK 64
#define PITCH 80
#define GT 256

template <int BM, int BN, int WM, int WN, bool W4, int EPI>
__global__ __launch_bounds__(GT, 1) void gemm_kernel(const int8_t* __restrict__ A, const int8_t* __restrict__ W, const float* __restrict__ as,
                                                     const float* __restrict__ ws, const half_t* __restrict__ gs, const half_t* __restrict__ bias,
                                                     void* __restrict__ Cout, int M, int N, int K, int group, const half_t* __restrict__ R,
                                                     const half_t* __restrict__ G, int L) {
    constexpr int TM = BM / WM, TN = BN / WN, FI = TM / 32, FJ = TN / 32;
    constexpr int ACH = BM * 4 / GT;                 // 16-byte A chunks per thread per k slice
    constexpr int BTOT = W4 ? BN * 2 : BN * 4;       // 16-byte W chunks per k slice (packed bytes for int4)
    constexpr int BCH = (BTOT + GT - 1) / GT;
    static_assert(WM * WN == 4 && TM % 32 == 0 && TN % 32 == 0 && ACH >= 1 && BCH >= 1, "tile");
    extern __shared__ __attribute__((aligned(16))) char smem[];
    // Stage buf: A rows at smem + buf * (BM + BN) * PITCH, W rows right after them.
    auto sA = [&](int buf) { return smem + buf * (BM + BN) * PITCH; };
    auto sB = [&](int buf) { return smem + buf * (BM + BN) * PITCH + BM * PITCH; };

    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int wm = wave / WN, wn = wave % WN;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int row_bytes = W4 ? K / 2 : K;

    i16v acc[FI][FJ];
    f16v yacc[EPI == GROUP_SCALED ? FI : 1][EPI == GROUP_SCALED ? FJ : 1];
#pragma unroll
    for (int i = 0; i < FI; i++)
#pragma unroll
        for (int j = 0; j < FJ; j++) acc[i][j] = (i16v){};
    if (EPI == GROUP_SCALED)
#pragma unroll
        for (int i = 0; i < FI; i++)
#pragma unroll
            for (int j = 0; j < FJ; j++) yacc[i][j] = (f16v){};

    u4v ra[ACH], rb[BCH];
    auto load = [&](int k0) {
#pragma unroll
        for (int p = 0; p < ACH; p++) {
            const int c = t + p * GT, r = c >> 2, kc = c & 3;
            const int m = min(m0 + r, M - 1);  // rows past M re-read the last row; their results are not stored
            ra[p] = __builtin_nontemporal_load((const u4v*)(A + (size_t)m * K + k0 + kc * 16));
        }
#pragma unroll
        for (int p = 0; p < BCH; p++) {
            const int c = t + p * GT;
            if (BTOT % GT != 0 && c >= BTOT) break;
            if (W4) {
                const int r = c >> 1, kc = c & 1;
                rb[p] = *(const u4v*)(W + (size_t)(n0 + r) * row_bytes + k0 / 2 + kc * 16);
            } else {
                const int r = c >> 2, kc = c & 3;
                rb[p] = *(const u4v*)(W + (size_t)(n0 + r) * row_bytes + k0 + kc * 16);
            }
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int p = 0; p < ACH; p++) {
            const int c = t + p * GT, r = c >> 2, kc = c & 3;
            *(u4v*)(sA(buf) + r * PITCH + kc * 16) = ra[p];
        }
#pragma unroll
        for (int p = 0; p < BCH; p++) {
            const int c = t + p * GT;
            if (BTOT % GT != 0 && c >= BTOT) break;
            if (W4) {
                // 32 nibbles -> 32 bytes. lo holds the even k of each byte pair, hi the odd k; a nibble
                // n is sign-extended as n | (n & 8) * 0x1e (0xf0 when the sign bit is set).
                const int r = c >> 1, kc = c & 1;
                u4v o0, o1;
#pragma unroll
                for (int d = 0; d < 4; d++) {
                    const u32 w = rb[p][d];
                    u32 lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
                    lo |= (lo & 0x08080808u) * 0x1eu;
                    hi |= (hi & 0x08080808u) * 0x1eu;
                    const u32 e0 = __builtin_amdgcn_perm(hi, lo, 0x05010400u), e1 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
                    if (d < 2) { o0[d * 2] = e0; o0[d * 2 + 1] = e1; }
                    else { o1[(d - 2) * 2] = e0; o1[(d - 2) * 2 + 1] = e1; }
                }
                *(u4v*)(sB(buf) + r * PITCH + kc * 32) = o0;
                *(u4v*)(sB(buf) + r * PITCH + kc * 32 + 16) = o1;
            } else {
                const int r = c >> 2, kc = c & 3;
                *(u4v*)(sB(buf) + r * PITCH + kc * 16) = rb[p];
            }
        }
    };

    const int KT = K / BK;
    load(0);
    store(0);
    __syncthreads();
    const int frag = (lane & 31) * PITCH + (lane >> 5) * 16;
    for (int kt = 0; kt < KT; kt++) {
        const int buf = kt & 1;
        if (kt + 1 < KT) load((kt + 1) * BK);
#pragma unroll
        for (int kk = 0; kk < 2; kk++) {
            i4v a[FI], b[FJ];
#pragma unroll
            for (int i = 0; i < FI; i++) a[i] = *(const i4v*)(sA(buf) + (wm * TM + i * 32) * PITCH + frag + kk * 32);
#pragma unroll
            for (int j = 0; j < FJ; j++) b[j] = *(const i4v*)(sB(buf) + (wn * TN + j * 32) * PITCH + frag + kk * 32);
#pragma unroll
            for (int i = 0; i < FI; i++)
#pragma unroll
                for (int j = 0; j < FJ; j++) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (EPI == GROUP_SCALED && ((kt + 1) * BK) % group == 0) {
            const int g = (kt + 1) * BK / group - 1, G = K / group;
#pragma unroll
            for (int j = 0; j < FJ; j++) {
                const float s = (float)gs[(size_t)(n0 + wn * TN + j * 32 + (lane & 31)) * G + g];
#pragma unroll
                for (int i = 0; i < FI; i++) {
#pragma unroll
                    for (int r = 0; r < 16; r++) yacc[i][j][r] = __builtin_fmaf((float)acc[i][j][r], s, yacc[i][j][r]);
                    acc[i][j] = (i16v){};
                }
            }
        }
        if (kt + 1 < KT) store(buf ^ 1);
        __syncthreads();
    }

    if (EPI == RAW_ACC) {
        int* C = (int*)Cout;
#pragma unroll
        for (int i = 0; i < FI; i++)
#pragma unroll
            for (int j = 0; j < FJ; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int m = m0 + wm * TM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    const int n = n0 + wn * TN + j * 32 + (lane & 31);
                    if (m < M) C[(size_t)m * N + n] = acc[i][j][r];
                }
        return;
    }

    // fp16 epilogue staged through LDS, 32 rows of the wave's tile at a time, so that each
    // lane stores whole 16-byte row segments.
    half_t* C = (half_t*)Cout;
    constexpr int SP = TN * 2 + 16;  // staging row pitch in bytes
    char* stage = smem + wave * 32 * SP;
    float wsv[FJ];
    half_t bv[FJ];
#pragma unroll
    for (int j = 0; j < FJ; j++) {
        const int n = n0 + wn * TN + j * 32 + (lane & 31);
        wsv[j] = EPI == PER_CHANNEL ? ws[n] : 0.f;
        bv[j] = bias ? bias[n] : (half_t)0;
    }
#pragma unroll
    for (int i = 0; i < FI; i++) {
        const int mb = m0 + wm * TM + i * 32;
        f4 asv[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            // Rows 8q + 4 (l / 32) + e, e < 4, of this 32-row block.
            const int mm = mb + 8 * q + 4 * (lane >> 5);
            if (mm + 3 < M) asv[q] = *(const f4*)(as + mm);
            else {
#pragma unroll
                for (int e = 0; e < 4; e++) asv[q][e] = mm + e < M ? as[mm + e] : 0.f;
            }
        }
#pragma unroll
        for (int j = 0; j < FJ; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const float s = asv[r >> 2][r & 3];
                float y;
                if (EPI == PER_CHANNEL) {
                    y = (float)acc[i][j][r] * s * wsv[j];
                    if (bias) y = y + (float)bv[j];
                } else {
                    y = yacc[i][j][r] * s;
                    if (bias) y = y + (float)bv[j];
                }
                const int rr = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                *(half_t*)(stage + rr * SP + (j * 32 + (lane & 31)) * 2) = to_half(y);
            }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        constexpr int CPR = TN / 8;  // 16-byte chunks per staged row
#pragma unroll
        for (int p = 0; p < 32 * CPR / 64; p++) {
            const int q = lane + p * 64, rr = q / CPR, cc = q % CPR;
            const int m = mb + rr, n = n0 + wn * TN + cc * 8;
            h8 y = *(const h8*)(stage + rr * SP + cc * 16);
            if (m < M) {
                const size_t at = (size_t)m * N + n;
                if (R) {
                    const h8 res = *(const h8*)(R + at), gate = *(const h8*)(G + (size_t)(m / L) * N + n);
#pragma unroll
                    for (int e = 0; e < 8; e++) y[e] = to_half((float)res[e] + r16((float)gate[e] * (float)y[e]));
                }
                *(h8*)(C + at) = y;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

template <int BM, int BN, int WM, int WN, bool W4, int EPI>
static int launch_gemm(const void* a, const void* w, const float* as, const float* ws, const void* gs, const void* bias, void* c, int M, int N, int K,
                       int group, const void* R, const void* G, int L, void* stream) {
    const size_t lds = (size_t)2 * (BM + BN) * PITCH;
    auto kern = gemm_kernel<BM, BN, WM, WN, W4, EPI>;
    static bool configured = false;
    if (!configured) {
        const hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return (int)e;
        configured = true;
    }
    hipLaunchKernelGGL(kern, dim3(N / BN, (M + BM - 1) / BM), dim3(GT), lds, (hipStream_t)stream, (const int8_t*)a, (const int8_t*)w, as, ws,
                       (const half_t*)gs, (const half_t*)bias, c, M, N, K, group, (const half_t*)R, (const half_t*)G, L);
    return (int)hipGetLastError();
}

template <bool W4, int EPI>
static int dispatch(const void* a, const void* w, const float* as, const float* ws, const void* gs, const void* bias, void* c, int M, int N, int K,
                    int group, const void* R, const void* G, int L, void* stream) {
    if (M <= 0 || N <= 0 || K <= 0 || N % 64 != 0 || K % BK != 0) return RDA_ERR_INVALID;
    if (R && (!G || L <= 0)) return RDA_ERR_INVALID;
    if constexpr (EPI == GROUP_SCALED) {
        if (group <= 0 || group % BK != 0 || K % group != 0) return RDA_ERR_INVALID;
        if (N % 256 == 0) return launch_gemm<128, 256, 2, 2, W4, EPI>(a, w, as, ws, gs, bias, c, M, N, K, group, R, G, L, stream);
        return launch_gemm<256, 64, 4, 1, W4, EPI>(a, w, as, ws, gs, bias, c, M, N, K, group, R, G, L, stream);
    } else {
    if (N % 256 == 0) return launch_gemm<256, 256, 2, 2, W4, EPI>(a, w, as, ws, gs, bias, c, M, N, K, group, R, G, L, stream);
    if (N % 128 == 0) return launch_gemm<256, 128, 2, 2, W4, EPI>(a, w, as, ws, gs, bias, c, M, N, K, group, R, G, L, stream);
    return launch_gemm<256, 64, 4, 1, W4, EPI>(a, w, as, ws, gs, bias, c, M, N, K, group, R, G, L, stream);
    }
}

extern "C" {

int rda_gemm(const void* a_q, const void* w, const float* a_scale, const float* w_scale, const void* bias, void* c, int M, int N, int K, const void* res,
             const void* res_gate, int L, void* stream) {
    return dispatch<false, PER_CHANNEL>(a_q, w, a_scale, w_scale, nullptr, bias, c, M, N, K, 0, res, res_gate, L, stream);
}

int rda_gemm_i4(const void* a_q, const void* w_packed, const float* a_scale, const float* w_scale, const void* bias, void* c, int M, int N, int K,
                void* stream) {
    if (K % 128 != 0) return RDA_ERR_INVALID;
    return dispatch<true, PER_CHANNEL>(a_q, w_packed, a_scale, w_scale, nullptr, bias, c, M, N, K, 0, nullptr, nullptr, 1, stream);
}

int rda_gemm_w4a8(const void* a_q, const void* w_packed, const float* a_scale, const void* group_scales, const void* bias, void* c, int M, int N, int K,
                  int group, void* stream) {
    if (K % 128 != 0) return RDA_ERR_INVALID;
    return dispatch<true, GROUP_SCALED>(a_q, w_packed, a_scale, nullptr, group_scales, bias, c, M, N, K, group, nullptr, nullptr, 1, stream);
}

int rda_gemm_acc(const void* a_q, const void* w, int w_int4, void* acc, int M, int N, int K, void* stream) {
    if (w_int4) {
        if (K % 128 != 0) return RDA_ERR_INVALID;
        return dispatch<true, RAW_ACC>(a_q, w, nullptr, nullptr, nullptr, nullptr, acc, M, N, K, 0, nullptr, nullptr, 1, stream);
    }
    return dispatch<false, RAW_ACC>(a_q, w, nullptr, nullptr, nullptr, nullptr, acc, M, N, K, 0, nullptr, nullptr, 1, stream);
}

}  // extern "C"
