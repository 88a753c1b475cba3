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
#include <type_traits>

#include "common.h"

enum Epi { PER_CHANNEL = 0, GROUP_SCALED = 1, RAW_ACC = 2 };

#define BK 64
#define PITCH 80
#define GT 256

// Dequantizing epilogue of one wave's (32 FI) x (32 FJ) tile at rows mw.., columns nw..: int32 accumulators
// (or the fp32 group sums for GROUP_SCALED) -> fp16 C, staged through the wave's LDS area `stage`
// (32 rows of 64 FJ + 16 bytes) so that every lane stores whole 16-byte row segments; RAW_ACC stores the
// int32 accumulators themselves.
template <int FI, int FJ, int EPI>
__device__ __forceinline__ void epilogue(const i16v (&acc)[FI][FJ], const f16v (&yacc)[EPI == GROUP_SCALED ? FI : 1][EPI == GROUP_SCALED ? FJ : 1],
                                         char* stage, int lane, int mw, int nw, int M, int N, const float* __restrict__ as,
                                         const float* __restrict__ ws, const half_t* __restrict__ bias, void* __restrict__ Cout,
                                         const half_t* __restrict__ R, const half_t* __restrict__ G, int L) {
    constexpr int TN = FJ * 32;
    if (EPI == RAW_ACC) {
        int* C = (int*)Cout;
#pragma unroll
        for (int i = 0; i < FI; i++)
#pragma unroll
            for (int j = 0; j < FJ; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int m = mw + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    const int n = nw + j * 32 + (lane & 31);
                    if (m < M) C[(size_t)m * N + n] = acc[i][j][r];
                }
        return;
    }

    // fp16 epilogue staged through LDS, 32 rows of the wave's tile at a time, so that each
    // lane stores whole 16-byte row segments.
    half_t* C = (half_t*)Cout;
    constexpr int SP = TN * 2 + 16;  // staging row pitch in bytes
    float wsv[FJ];
    half_t bv[FJ];
#pragma unroll
    for (int j = 0; j < FJ; j++) {
        const int n = nw + j * 32 + (lane & 31);
        wsv[j] = EPI == PER_CHANNEL ? ws[n] : 0.f;
        bv[j] = bias ? bias[n] : (half_t)0;
    }
#pragma unroll
    for (int i = 0; i < FI; i++) {
        const int mb = mw + i * 32;
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
            const int m = mb + rr, n = nw + cc * 8;
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

    epilogue<FI, FJ, EPI>(acc, yacc, smem + wave * 32 * (TN * 2 + 16), lane, m0 + wm * TM, n0 + wn * TN, M, N, as, ws, bias, Cout, R, G, L);
}

// Epilogue for accumulators holding C^T blocks (the GEMM computed W A^T): in block (i, j), lane l owns
// row mw + 32 i + l % 32 of C and register r holds column nw + 32 j + 8 (r / 4) + 4 (l / 32) + r % 4, so
// each group of four registers is four consecutive columns of one row: they are dequantized and stored
// as 8-byte fp16 (16-byte int32) row segments, with no staging.
template <int FI, int FJ, int EPI>
__device__ __forceinline__ void epilogue_rows(const i16v (&acc)[FI][FJ], int lane, int mw, int nw, int M, int N, const float* __restrict__ as,
                                              const float* __restrict__ ws, const half_t* __restrict__ bias, void* __restrict__ Cout,
                                              const half_t* __restrict__ R, const half_t* __restrict__ G, int L) {
    const int lq = lane & 31, g = lane >> 5;
#pragma unroll
    for (int i = 0; i < FI; i++) {
        const int m = mw + i * 32 + lq;
        if (m >= M) continue;
        const float s = EPI == RAW_ACC ? 0.f : as[m];
#pragma unroll
        for (int j = 0; j < FJ; j++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int n = nw + j * 32 + 8 * q + 4 * g;
                const size_t at = (size_t)m * N + n;
                if (EPI == RAW_ACC) {
                    *(i4v*)((int*)Cout + at) = (i4v){acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
                    continue;
                }
                const f4 wv = *(const f4*)(ws + n);
                h4v bv = {};
                if (bias) bv = *(const h4v*)(bias + n);
                h4v y;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    float v = (float)acc[i][j][4 * q + e] * s * wv[e];
                    if (bias) v = v + (float)bv[e];
                    y[e] = to_half(v);
                }
                if (R) {
                    const h4v res = *(const h4v*)(R + at), gate = *(const h4v*)(G + (size_t)(m / L) * N + n);
#pragma unroll
                    for (int e = 0; e < 4; e++) y[e] = to_half((float)res[e] + r16((float)gate[e] * (float)y[e]));
                }
                *(h4v*)((half_t*)Cout + at) = y;
            }
    }
}

// Epilogue of the whole BM x BN block through LDS: every wave dequantizes its C^T accumulators
// (epilogue_rows' register layout; scales and biases from the scale block `sc` in LDS; GROUP_SCALED: the
// fp32 group sums yacc, times as) into an fp16 tile in LDS, then all 256 threads store it in 16-byte
// chunks, consecutive lanes covering consecutive bytes of a row, so each store instruction writes whole
// 128-byte lines (the register layout would touch 32 rows per instruction). R and G are read the same way.
// Bytes of the bias area of the scale block: BN halfs, copied in 256-byte instructions.
constexpr int SC_BIAS(int bn) { return (bn * 2 + 255) / 256 * 256; }
template <int BM, int BN, int FI, int FJ, int EPI, int NT>
__device__ __forceinline__ void epilogue_block(const i16v (&acc)[FI][FJ], const f16v (&yacc)[EPI == GROUP_SCALED ? FI : 1][EPI == GROUP_SCALED ? FJ : 1],
                                               char* tile, const char* sc, int t, int lane, int wm, int wn, int m0, int n0, int M, int N,
                                               const float* __restrict__ as, const float* __restrict__ ws, const half_t* __restrict__ bias,
                                               half_t* __restrict__ C, const half_t* __restrict__ R, const half_t* __restrict__ G, int L) {
    constexpr int TM = FI * 32, TN = FJ * 32, TP = BN * 2 + 16, CPR = BN / 8;  // tile row pitch (bytes), 16-byte chunks per row
    const int lq = lane & 31, g = lane >> 5;
    // The block's column scales, biases and row scales were copied into LDS at the kernel's start.
    const float* ws_s = (const float*)sc;
    const half_t* bias_s = (const half_t*)(sc + BN * 4);
    const float* as_s = (const float*)(sc + BN * 4 + SC_BIAS(BN));
    auto dequantize = [&](auto has_bias) {
        constexpr bool HB = decltype(has_bias)::value;
#pragma unroll
        for (int j = 0; j < FJ; j++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int c = wn * TN + j * 32 + 8 * q + 4 * g;
                const f4 wv = EPI == PER_CHANNEL ? *(const f4*)(ws_s + c) : (f4){};
                const h4v bv = HB ? *(const h4v*)(bias_s + c) : (h4v){};
#pragma unroll
                for (int i = 0; i < FI; i++) {
                    const int r = wm * TM + i * 32 + lq;
                    const float sv = as_s[r];
                    h4v y;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        float v;
                        if constexpr (EPI == PER_CHANNEL) v = (float)acc[i][j][4 * q + e] * sv * wv[e];
                        else v = yacc[EPI == GROUP_SCALED ? i : 0][EPI == GROUP_SCALED ? j : 0][4 * q + e] * sv;
                        if (HB) v = v + (float)bv[e];
                        y[e] = to_half(v);
                    }
                    *(h4v*)(tile + r * TP + c * 2) = y;
                }
            }
    };
    constexpr int ITER = BM * CPR / NT;  // 16-byte chunks per thread (the tile is a whole number of them)
    static_assert(BM * CPR % NT == 0, "whole chunks per thread");
    if (!R) {
        if (bias) dequantize(std::integral_constant<bool, true>{});
        else dequantize(std::integral_constant<bool, false>{});
        __syncthreads();
#pragma unroll 4
        for (int it = 0; it < ITER; it++) {
            const int idx = t + it * NT, r = idx / CPR, c = (idx % CPR) * 8, m = m0 + r;
            if (m < M) *(h8*)(C + (size_t)m * N + n0 + c) = *(const h8*)(tile + r * TP + c * 2);
        }
        return;
    }
    // Gated residual: R and G are read in batches of RB chunks per thread, double-buffered, with row indices
    // clamped in bounds so that no load sits under a branch; the first batch goes out before the dequantization
    // pass, whose LDS work then covers its latency. (One load per chunk, each awaited before its store, left
    // the epilogue latency-bound: +17 us on 4096 x 3072 x 3072.)
    // A batch is 16 VGPRs per chunk, and the first is in flight while the accumulators are live: eight-wave tiles of
    // 64 x 128 (128 accumulator VGPRs of a 256 budget) take batches of 4.
    constexpr int RBMAX = NT >= 512 && FI * FJ >= 8 ? 4 : 8;
    constexpr int RB = ITER % RBMAX == 0 ? RBMAX : ITER % 4 == 0 ? 4 : 1, NBATCH = ITER / RB;
    h8 res[2][RB], gat[2][RB];
    auto load = [&](int b, int slot) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < RB; k++) {
            const int idx = t + (b * RB + k) * NT, r = idx / CPR, c = (idx % CPR) * 8, m = min(m0 + r, M - 1);
            res[slot][k] = *(const h8*)(R + (size_t)m * N + n0 + c);
            gat[slot][k] = *(const h8*)(G + (size_t)(m / L) * N + n0 + c);
        }
    };
    load(0, 0);
    if (bias) dequantize(std::integral_constant<bool, true>{});
    else dequantize(std::integral_constant<bool, false>{});
    __syncthreads();
#pragma unroll
    for (int b = 0; b < NBATCH; b++) {
        if (b + 1 < NBATCH) load(b + 1, (b + 1) & 1);
#pragma unroll
        for (int k = 0; k < RB; k++) {
            const int idx = t + (b * RB + k) * NT, r = idx / CPR, c = (idx % CPR) * 8, m = m0 + r;
            h8 y = *(const h8*)(tile + r * TP + c * 2);
#pragma unroll
            for (int e = 0; e < 8; e++) y[e] = to_half((float)res[b & 1][k][e] + r16((float)gat[b & 1][k][e] * (float)y[e]));
            if (m < M) *(h8*)(C + (size_t)m * N + n0 + c) = y;
        }
    }
}

// int8 GEMM with direct global->LDS copies, for int8 or packed int4 weights (PER_CHANNEL, GROUP_SCALED and
// RAW_ACC epilogues). A workgroup of NW wave64s (4 or 8) computes a BM x BN tile, the waves WGM x (NW / WGM)
// over it (each a BM / WGM x BN / (NW / WGM) sub-tile: with four waves a BM/2 x BN/2 quarter, or with WGM = 1 all
// BM rows and BN/4 columns) in 32x32 blocks (the products compute W A^T, so each lane ends up owning row
// segments of C). K advances in slices of KB8
// values through NS LDS stages: the copies of slice k + NS go out during the last k step of slice k. A stage
// holds the slice's BM A rows (KB8 bytes each), then its BN W rows (KB8 bytes, or KB8 / 2 packed int4
// bytes), with 16-byte chunk c of row r at c ^ ((r / RPL) % CPR) (RPL rows per 256-byte bank line, CPR
// chunks per row): the fragment reads of 16 consecutive rows then hit 16 distinct bank groups, and one
// 1 KiB copy instruction (lane i -> bytes 16 i) fills whole rows. int4 fragments are read as 8 bytes, first
// in each k step, and widened after the step's last product to 16 int8 with each nibble in the high half of
// its byte, i.e. as 16 times its signed value (two ANDs and a shift, then v_perm interleaves the even-k low
// nibbles with the odd-k high nibbles); the accumulators then hold exactly 16 times the products, which the
// kernel undoes after the K loop (an arithmetic shift of the int32 sums, a factor 1/16 on the fp32 group
// sums: both exact). The host keeps K <= 65536 on this path so that 16 times the sums fits in 32 bits.
//
// GROUP_SCALED (group == KB8 == 128): the first product of each slice starts from zero and after the slice
// the int32 partials are folded into fp32 sums, y = fma((float)p, gs[n, slice], y), in group order; the
// block's group scales are staged in LDS as [group][column] at the start, and each lane reads its slice's
// scales at the slice's first product.
//
// One wave per SIMD (two with MINB = 2), so little else hides the issue time of copies and LDS reads: every
// copy and fragment read is issued in the shadow of a product, spread evenly over its 32-wide k step
// (sched_barrier pins the order). Fragments of the next k step are read during the current one; the
// slice's barrier sits before its last k step, so the next slice's first reads start right after it.
template <int BM, int BN, int KB8, int NS, bool W4, int EPI, int MINB, int WGM, int NW, bool IL>
__global__ __launch_bounds__(64 * NW, MINB) void gemm8_kernel(const int8_t* __restrict__ A, const int8_t* __restrict__ W, const float* __restrict__ as,
                                                      const float* __restrict__ ws, const half_t* __restrict__ gs, const half_t* __restrict__ bias,
                                                      void* __restrict__ Cout, int M, int N, int K, const half_t* __restrict__ R,
                                                      const half_t* __restrict__ G, int L) {
    constexpr int NT = 64 * NW, WGN = NW / WGM, TM = BM / WGM, TN = BN / WGN, FI = TM / 32, FJ = TN / 32, NF = FI * FJ, NR = FI + FJ;
    constexpr bool GRP = EPI == GROUP_SCALED;
    constexpr int KS = KB8 / 32;                                      // 32-wide k steps per slice
    constexpr int CPR = KB8 / 16, RPI = 1024 / KB8, RPL = 256 / KB8;  // A rows: chunks per row, rows per copy, rows per bank line
    constexpr int WB = W4 ? KB8 / 2 : KB8;                            // W row bytes per slice
    constexpr int CPRB = WB / 16, RPIB = 1024 / WB, RPLB = 256 / WB;
    constexpr int STAGE = BM * KB8 + BN * WB;
    constexpr int AI = BM / (NW * RPI), BI = BN / (NW * RPIB), NI = AI + BI;  // copy instructions per wave per slice
    static_assert((BM == 256 || BM == 128) && (WGM == 1 || WGM == 2 || WGM == 4) && NW % WGM == 0 && BN % 64 == 0 && TN % 32 == 0 && (KB8 == 64 || KB8 == 128) && BN % (NW * RPIB) == 0 &&
                  BM % (NW * RPI) == 0, "tile");
    static_assert(!GRP || KB8 == 128, "one group per slice");
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int t = threadIdx.x, lane = t & 63, lq = lane & 31, g = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6), wm = wave / WGN, wn = wave % WGN;

    // Tile order: block ids go round-robin to the 8 XCDs. When the grid allows it, XCD x gets the tiles of
    // one (gy / 2) x (gx / 4) sub-grid, so each A row panel is read by 4 XCDs' L2s and each W panel by 2
    // (round-robin order has every XCD read every A panel). Within the sub-grid the tiles go row by row; the
    // eight-wave W4A8 kernel (one block per CU, 32 at a time per XCD) takes them in strips four tiles tall, column
    // by column, so the blocks an XCD runs together cover 4 x 8 tiles rather than ~3 x 12 and read fewer panels
    // (W4A8 4096 x 12288 x 3072: fetched bytes -13.5%, time unchanged). Sub-grids under 8 tiles wide keep rows.
    int bx = blockIdx.x, by = blockIdx.y;
    {
        const int gx = gridDim.x, gy = gridDim.y;
        if (gx % 4 == 0 && gy % 2 == 0) {
            const int id = by * gx + bx, x = id % 8, r = id / 8, sx = gx / 4, sy = gy / 2;
            if (NW == 8 && GRP && sy % 4 == 0 && sx >= 8) {
                const int strip = r / (4 * sx), w = r % (4 * sx);
                bx = (x % 4) * sx + w / 4;
                by = (x / 4) * sy + strip * 4 + w % 4;
            } else {
                bx = (x % 4) * sx + r % sx;
                by = (x / 4) * sy + r / sx;
            }
        }
    }
    const int m0 = by * BM, n0 = bx * BN;
    const int wrow = W4 ? K / 2 : K;  // bytes per W row in memory

    // Copy instruction j of a wave fills rows (4 j + wave) RPI .. + RPI - 1 of A (or of W, with RPIB): lane i
    // takes row (4 j + wave) RPI + i / CPR at physical chunk i % CPR, i.e. logical chunk cchunk (the swizzle
    // term is the same for every j). A rows past M re-read row M - 1 (their results are not stored); the
    // clamp is folded into the per-lane offsets, taken from a clamped group base so that they are never
    // negative (they are the unsigned 32-bit voffset of the copy).
    const int crow = wave * RPI + lane / CPR, cchunk = (lane % CPR) ^ ((crow / RPL) % CPR);
    const int brow = wave * RPIB + lane / CPRB, bchunk = (lane % CPRB) ^ ((brow / RPLB) % CPRB);
    const u32 boff = (u32)brow * wrow + bchunk * 16;
    int arow[AI];
    u32 aoff[AI];
#pragma unroll
    for (int c = 0; c < AI; c++) {
        arow[c] = min(m0 + NW * RPI * c, M - 1);
        aoff[c] = (u32)(min(m0 + NW * RPI * c + crow, M - 1) - arow[c]) * K + cchunk * 16;
    }
    auto stage = [&](int kt) -> const char* { return smem + (kt % NS) * STAGE; };
    // The epilogue's scales go to a scale block: ws[n0 .. n0 + BN) (BN / 64 copies of 64 floats), bias[n0 ..)
    // (256-byte copies, lanes past BN / 2 re-read the last pair) and as[m0 .. m0 + BM) (rows past M re-read
    // row M - 1), each copy issued by one wave. (A static LDS array of its own: the compiler can then tell the
    // epilogue's scale reads from its tile writes.)
    __shared__ __attribute__((aligned(16))) char sc[BN * 4 + SC_BIAS(BN) + BM * 4];
    if (EPI != RAW_ACC) {
        constexpr int NWS = EPI == PER_CHANNEL ? BN / 64 : 0, NB = SC_BIAS(BN) / 256;
#pragma unroll
        for (int c = 0; c < NWS + NB + BM / 64; c++) {
            if (c % NW != wave) continue;
            if (c < NWS) {
                dma4(ws + n0 + 64 * c, lane * 4, sc + c * 256);
            } else if (c < NWS + NB) {
                if (bias) dma4(bias + n0, (u32)min(64 * (c - NWS) + lane, BN / 2 - 1) * 4, sc + BN * 4 + (c - NWS) * 256);
            } else {
                const int i = c - NWS - NB, mb = min(m0 + 64 * i, M - 1);
                dma4(as + mb, (u32)(min(m0 + 64 * i + lane, M - 1) - mb) * 4, sc + BN * 4 + SC_BIAS(BN) + i * 256);
            }
        }
    }
    // GROUP_SCALED: the block's group scales, transposed to [group][column] (one group per slice), past the
    // stages and the staged output tile.
    constexpr int GS_OFF = ((NS * STAGE > BM * (BN * 2 + 16) ? NS * STAGE : BM * (BN * 2 + 16)) + 15) / 16 * 16;
    half_t* gsl = (half_t*)(smem + GS_OFF);
    if (GRP) {
        const int groups = K / KB8;
        // The block's scales are BN consecutive rows of gs ([N][groups], contiguous): read them in 16-byte pieces (all
        // of a thread's pieces in flight together), then transpose them into LDS.
        const half_t* src = gs + (size_t)n0 * groups;
        const int pieces = BN * groups / 8;
        for (int ch = t; ch < pieces; ch += NT) {
            const h8 v = *(const h8*)(src + (size_t)ch * 8);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int idx = ch * 8 + e, c = idx / groups, gi = idx - c * groups;
                gsl[gi * BN + c] = v[e];
            }
        }
    }
    auto copy = [&](int kt, int c) {  // copy instruction c (< NI) of slice kt
        const char* st = stage(kt);
        if (c < AI) dma16(A + (size_t)arow[c] * K + kt * KB8, aoff[c], st + (NW * c + wave) * 1024);
        else dma16(W + (size_t)(n0 + NW * RPIB * (c - AI)) * wrow + kt * WB, boff, st + BM * KB8 + (NW * (c - AI) + wave) * 1024);
    };

    // Fragment f (< FI: A block f, else W block f - FI) of k step kk: row base + lq, k values 32 kk + 16 g ..
    // + 15, i.e. chunk 2 kk + g of an A row, the half g of chunk kk of a packed int4 W row. A packed int4
    // fragment is read as its 8 bytes (wraw) and widened later (widen), so that products, not the widening,
    // wait for the read.
    const int fx = (lq / RPL) % CPR, fxb = (lq / RPLB) % CPRB;
    auto frag = [&](const char* st, int kk, int f) -> i4v {
        if (f < FI) return *(const i4v*)(st + (wm * TM + f * 32 + lq) * KB8 + (((2 * kk + g) ^ fx) << 4));
        return *(const i4v*)(st + BM * KB8 + (wn * TN + (f - FI) * 32 + lq) * WB + (((2 * kk + g) ^ fxb) << 4));
    };
    auto wraw = [&](const char* st, int kk, int j) -> u2v {
        return *(const u2v*)(st + BM * KB8 + (wn * TN + j * 32 + lq) * WB + ((kk ^ fxb) << 4) + 8 * g);
    };
    // IL: the activations are stored k-interleaved (each 8 values of k as the even ones, then the odd ones), so the
    // even-k and odd-k bytes are the fragment's words as they are, with no interleave.
    auto widen = [](u2v p) -> i4v {
        u4v o;
#pragma unroll
        for (int d = 0; d < 2; d++) {
            const u32 lo = (p[d] << 4) & 0xf0f0f0f0u, hi = p[d] & 0xf0f0f0f0u;  // 16 x (signed nibble) per byte
            if constexpr (IL) {
                o[2 * d] = lo;
                o[2 * d + 1] = hi;
            } else {
                o[2 * d] = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
                o[2 * d + 1] = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
            }
        }
        return as_i4(o);
    };
    i16v acc[FI][FJ];
    f16v yacc[GRP ? FI : 1][GRP ? FJ : 1];
#pragma unroll
    for (int i = 0; i < FI; i++)
#pragma unroll
        for (int j = 0; j < FJ; j++) acc[i][j] = (i16v){};
    if (GRP)
#pragma unroll
        for (int i = 0; i < FI; i++)
#pragma unroll
            for (int j = 0; j < FJ; j++) yacc[GRP ? i : 0][GRP ? j : 0] = (f16v){};
    // W4A8 with a wave over 128 rows x 32 columns (four A blocks, one W block) runs the block-major slice below.
    constexpr bool PIPE = GRP && W4 && FI == 4 && FJ == 1 && KS == 4;
    i4v fr[2][NR];            // fragments of the current and the next k step
    u2v fw[W4 ? FJ : 1];      // packed int4 W fragments of the next k step, before widening

    // Copy schedule: a slice's stage is free once the barrier before the slice's last k step has passed
    // (every wave has then read its fragments of the slice), so the copies of slice k + NS go out during
    // that last k step, into that stage, NS - 1 slices of products before they are needed. (Spreading the
    // copies of slice k + NS - 1 over slice k instead left the last of them one k step to land.)
    const int KT = K / KB8;
#pragma unroll
    for (int kt = 0; kt < NS; kt++)
        if (kt < KT)
#pragma unroll
            for (int c = 0; c < NI; c++) copy(kt, c);
    // Slice 0 must have landed; up to NS - 1 later slices may still be in flight.
    if (KT >= NS) wait_copies_but<(NS - 1) * NI>();
    else wait_copies();
    __syncthreads();
#pragma unroll
    for (int f = 0; f < NR; f++) {
        if (PIPE) break;
        fr[0][f] = W4 && f >= FI ? widen(wraw(stage(0), 0, f - FI)) : frag(stage(0), 0, f);
    }
    // PIPE (below): the first three products' A fragments, slice 0's packed W fragments, the first one widened. (These
    // arrays have one element in the other instantiations, which never use them; indices there are written `PIPE ? i : 0`
    // so that those instantiations compile without out-of-range constants.)
    i4v afr[PIPE ? 4 : 1], wf[PIPE ? 4 : 1];
    u2v wr[PIPE ? 4 : 1];
    h4v gva[PIPE ? 4 : 1][4];  // [0]: scales of the slice's blocks 0, 1 fold; [1]: of its blocks 2, 3 (folded in the next slice)
    if constexpr (PIPE) {
#pragma unroll
        for (int P = 0; P < 3; P++) afr[P] = frag(stage(0), (P >> 1) & 3, (P >> 3) * 2 + (P & 1));
#pragma unroll
        for (int ks = 0; ks < 4; ks++) wr[ks] = wraw(stage(0), ks, 0);
        wf[0] = widen(wr[0]);
#pragma unroll
        for (int q = 0; q < 4; q++) gva[1][q] = (h4v){};  // slice 0 folds the zero partials of blocks 2, 3 with zero scales
    }

    // Copies that may still be in flight at the barrier of slice k once slice k + 1 has landed: the NS - 2
    // slices after it.
    constexpr int LEFT = (NS - 2) * NI;
    // Order of the next step's fragment reads over the products: int4 W fragments first, so that they have
    // landed when they are widened after the step's last product.
    constexpr auto RD = [](int f) { return W4 ? (f >= FI ? f - FI : f + FJ) : f; };
    // GROUP_SCALED: each lane's group scales of a slice, read at its first product, used by its fold. The
    // per-lane offset is held opaque so the slice's reads are one base plus immediate offsets.
    u32 goff = 0;
    if constexpr (GRP) {
        goff = (u32)(GS_OFF + (wn * TN + 4 * g) * 2);
        asm volatile("" : "+v"(goff));
    }
    // One slice. AHEAD: slice kt + NS exists and is copied during this slice's last k step (then slices
    // kt + 2 .. kt + NS - 1 exist too); MORE: slice kt + 1 exists; SI >= 0: kt % NS, known at compile time,
    // so the slice's LDS reads take their stage as an immediate offset.
    // GROUP_SCALED fold of block p's partial (one group: one slice) into its fp32 sums, with the group scales in gv.
    // Register r of block (i, j) is column wn TN + 32 j + 8 (r / 4) + 4 g + r % 4.
    h4v gv[GRP ? FJ : 1][4];
    auto fold = [&](int p) __attribute__((always_inline)) {
        const int i = p / FJ, j = p % FJ;
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int e = 0; e < 4; e++)
                yacc[GRP ? i : 0][GRP ? j : 0][4 * q + e] =
                    __builtin_fmaf((float)acc[i][j][4 * q + e], (float)gv[GRP ? j : 0][q][e], yacc[GRP ? i : 0][GRP ? j : 0][4 * q + e]);
    };
    auto slice = [&](int kt, auto ahead, auto more, auto si) {
        constexpr bool AHEAD = decltype(ahead)::value, MORE = decltype(more)::value;
        constexpr int SI = decltype(si)::value;
        const char* st = SI >= 0 ? smem + SI * STAGE : stage(kt);
        const char* sn = SI >= 0 ? smem + (SI + 1) % NS * STAGE : stage(kt + 1);
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            if (ks == KS - 1) {
                if (AHEAD) wait_copies_but<LEFT>();  // slice kt + 1 has landed
                else wait_copies();
                __syncthreads();
            }
            const int cur = ks & 1, nxt = cur ^ 1;
            const bool last = ks == KS - 1;
#pragma unroll
            for (int p = 0; p < NF; p++) {
                // GROUP_SCALED: the previous slice's partial of block p is folded just before the block's first
                // product of this slice restarts it, in the shadow of the other blocks' products (issued between
                // them), rather than all at the end of the slice with the matrix cores idle.
                if (GRP && ks == 0 && kt > 0) fold(p);
                const i16v c0 = GRP && ks == 0 ? (i16v){} : acc[p / FJ][p % FJ];
                acc[p / FJ][p % FJ] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fr[cur][FI + p % FJ], fr[cur][p / FJ], c0, 0, 0, 0);
                if (AHEAD && ks == KS - 1)
#pragma unroll
                    for (int c = 0; c < NI; c++)
                        if (c * NF / NI == p) copy(kt + NS, c);
                if (GRP && ks == 0 && p == NF - 1)  // this slice's scales, once the previous slice's are used
#pragma unroll
                    for (int j = 0; j < FJ; j++)
#pragma unroll
                        for (int q = 0; q < 4; q++) gv[GRP ? j : 0][q] = *(const h4v*)(smem + goff + kt * BN * 2 + (j * 32 + 8 * q) * 2);
                if (!last || MORE) {
#pragma unroll
                    for (int f = 0; f < NR; f++) {
                        if ((RD(f) * NF + NF / 2) / NR != p) continue;
                        if (W4 && f >= FI) fw[W4 ? f - FI : 0] = last ? wraw(sn, 0, f - FI) : wraw(st, ks + 1, f - FI);
                        else fr[nxt][f] = last ? frag(sn, 0, f) : frag(st, ks + 1, f);
                    }
                    if (W4 && p == NF - 1)
#pragma unroll
                        for (int j = 0; j < FJ; j++) fr[nxt][FI + j] = widen(fw[W4 ? j : 0]);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };
    // PIPE: one slice as 16 products P = 0 .. 15, block-major: block (P / 8) * 2 + P % 2 at k step (P / 2) % 4 (blocks
    // 0 and 1 alternate over the four k steps, then blocks 2 and 3), so each block's partial is complete eight
    // products before the block restarts it. Its fold (16 conversions and 16 FMAs) is then spread over those
    // products, a quarter (8 vector instructions) beside each: blocks 0 and 1 of this slice beside products 8-15,
    // blocks 2 and 3 of the previous slice beside products 0-7 -- few enough per product that the vector ALU runs
    // in the matrix cores' shadow (a burst of 32 before a product left the matrix cores idle). A fragments are read
    // three products ahead (ring of four); the slice's four int4 W fragments are widened once and held, their
    // packed bytes read after the barrier of the slice before. The barrier sits before product 13, once every read
    // of the slice's stage has been issued; the copies of slice kt + NS follow it, beside products 13-15. The group
    // scales are read twice per slice (before product 5 for blocks 0, 1; at 13 for blocks 2, 3), each set then held
    // until its last fold.
    auto slice_g = [&](int kt, auto ahead, auto more, auto si) __attribute__((always_inline)) {
        constexpr bool AHEAD = decltype(ahead)::value, MORE = decltype(more)::value;
        constexpr int SI = decltype(si)::value;
        const char* st = SI >= 0 ? smem + SI * STAGE : stage(kt);
        const char* sn = SI >= 0 ? smem + (SI + 1) % NS * STAGE : stage(kt + 1);
        const u32 gk = goff + (u32)(kt * BN * 2);
#pragma unroll
        for (int P = 0; P < 16; P++) {
            if (P == 13) {
                if (AHEAD) wait_copies_but<LEFT>();  // slice kt + 1 has landed
                else wait_copies();
                __syncthreads();
            }
            const int b = (P >> 3) * 2 + (P & 1), ks = (P >> 1) & 3;
            const i16v c0 = ks == 0 ? (i16v){} : acc[PIPE ? b : 0][0];
            acc[PIPE ? b : 0][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf[PIPE ? ks : 0], afr[PIPE ? P & 3 : 0], c0, 0, 0, 0);
            {  // a quarter of one block's fold
                const int fb = P < 8 ? 2 + (P >> 2) : (P - 8) >> 2, q = P & 3, set = P < 8 ? 1 : 0;
#pragma unroll
                for (int e = 0; e < 4; e++)
                    yacc[PIPE ? fb : 0][0][4 * q + e] =
                        __builtin_fmaf((float)acc[PIPE ? fb : 0][0][4 * q + e], (float)gva[PIPE ? set : 0][q][e], yacc[PIPE ? fb : 0][0][4 * q + e]);
            }
            {  // the A fragment three products ahead
                const int n = P + 3, nb = ((n & 15) >> 3) * 2 + (n & 1), nk = (n >> 1) & 3;
                if (n < 16) afr[PIPE ? n & 3 : 0] = frag(st, nk, nb);
                else if (MORE) afr[PIPE ? n & 3 : 0] = frag(sn, nk, nb);
            }
            if (P <= 2) wf[PIPE ? P + 1 : 0] = widen(wr[PIPE ? P + 1 : 0]);  // this slice's k steps 1-3
            if (MORE && P == 13) {
                wr[0] = wraw(sn, 0, 0);
                wr[PIPE ? 1 : 0] = wraw(sn, 1, 0);
            }
            if (MORE && P == 14) {
                wr[PIPE ? 2 : 0] = wraw(sn, 2, 0);
                wr[PIPE ? 3 : 0] = wraw(sn, 3, 0);
            }
            if (MORE && P == 15) wf[0] = widen(wr[0]);  // the next slice's first k step
            if (P == 5 || P == 13)
#pragma unroll
                for (int q = 0; q < 4; q++) gva[PIPE ? (P == 5 ? 0 : 1) : 0][q] = *(const h4v*)(smem + gk + 16 * q);
            if (AHEAD && P >= 13)
#pragma unroll
                for (int c = 0; c < NI; c++)
                    if (13 + c * 3 / NI == P) copy(kt + NS, c);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    using yes = std::integral_constant<bool, true>;
    using no = std::integral_constant<bool, false>;
    using any = std::integral_constant<int, -1>;
    int kt = 0;
    // int4 weights (vector-ALU bound: the widening, and the folds of GROUP_SCALED): NS slices per iteration,
    // starting at a multiple of NS, so slice kt + j is in stage j (18 fewer vector instructions per W4A8
    // slice). With int8 weights the unrolled loop measured the same and ran short of scalar registers.
    static_assert(NS >= 2 && NS <= 4, "stages");
    auto run = [&](int k, auto ahead, auto more, auto si) __attribute__((always_inline)) {
        if constexpr (PIPE) slice_g(k, ahead, more, si);
        else slice(k, ahead, more, si);
    };
    if constexpr (W4) {
        for (; kt + 2 * NS - 1 < KT; kt += NS) {
            run(kt, yes{}, yes{}, std::integral_constant<int, 0>{});
            run(kt + 1, yes{}, yes{}, std::integral_constant<int, 1>{});
            if constexpr (NS > 2) run(kt + 2, yes{}, yes{}, std::integral_constant<int, 2>{});
            if constexpr (NS > 3) run(kt + 3, yes{}, yes{}, std::integral_constant<int, 3>{});
        }
    }
    for (; kt + NS < KT; kt++) run(kt, yes{}, yes{}, any{});
    for (; kt + 1 < KT; kt++) run(kt, no{}, yes{}, any{});
    run(kt, no{}, no{}, any{});
    if constexpr (PIPE) {  // the last slice's blocks 2 and 3
#pragma unroll
        for (int fb = 2; fb < 4; fb++)
#pragma unroll
            for (int r = 0; r < 16; r++)
                yacc[PIPE ? fb : 0][0][r] = __builtin_fmaf((float)acc[PIPE ? fb : 0][0][r], (float)gva[PIPE ? 1 : 0][r >> 2][r & 3], yacc[PIPE ? fb : 0][0][r]);
    } else if constexpr (GRP) {  // the last slice's partials
#pragma unroll
        for (int p = 0; p < NF; p++) fold(p);
    }
    if constexpr (W4) {  // the int4 operands were 16 times their values: undo it (exactly)
        if constexpr (GRP) {
#pragma unroll
            for (int i = 0; i < FI; i++)
#pragma unroll
                for (int j = 0; j < FJ; j++) yacc[GRP ? i : 0][GRP ? j : 0] *= 0.0625f;
        } else {
#pragma unroll
            for (int i = 0; i < FI; i++)
#pragma unroll
                for (int j = 0; j < FJ; j++) acc[i][j] >>= 4;
        }
    }
    if constexpr (EPI == RAW_ACC) {
        epilogue_rows<FI, FJ, EPI>(acc, lane, m0 + wm * TM, n0 + wn * TN, M, N, as, ws, bias, Cout, R, G, L);
    } else {
        __syncthreads();  // the staged tile overlaps the stages
        epilogue_block<BM, BN, FI, FJ, EPI, NT>(acc, yacc, smem, sc, t, lane, wm, wn, m0, n0, M, N, as, ws, bias, (half_t*)Cout, R, G, L);
    }
}

template <int BM, int BN, int KB8, int NS, bool W4, int EPI, int MINB = 1, int WGM = 2, int NW = 4, bool IL = false>
static int launch_gemm8(const void* a, const void* w, const float* as, const float* ws, const void* gs, const void* bias, void* c, int M, int N, int K,
                        const void* R, const void* G, int L, void* stream) {
    const size_t stage = (size_t)BM * KB8 + (size_t)BN * (W4 ? KB8 / 2 : KB8);
    const size_t stages = NS * stage, tile = (size_t)BM * (BN * 2 + 16);
    size_t lds = EPI == RAW_ACC || stages > tile ? stages : tile;  // dynamic part; the scale block is static
    if (EPI == GROUP_SCALED) lds = (lds + 15) / 16 * 16 + (size_t)BN * (K / KB8) * 2;
    if (lds > 160 * 1024 / MINB - (size_t)(BN * 4 + SC_BIAS(BN) + BM * 4)) return -1;
    auto kern = gemm8_kernel<BM, BN, KB8, NS, W4, EPI, MINB, WGM, NW, IL>;
    static std::atomic<size_t> configured[RDA_MAX_DEVICES];
    if (const int e = ensure_dynamic_lds((const void*)kern, lds, configured)) return e;
    hipLaunchKernelGGL(kern, dim3(N / BN, (M + BM - 1) / BM), dim3(64 * NW), lds, (hipStream_t)stream, (const int8_t*)a, (const int8_t*)w, as, ws,
                       (const half_t*)gs, (const half_t*)bias, c, M, N, K, (const half_t*)R, (const half_t*)G, L);
    return (int)hipGetLastError();
}

// Tile width for the direct-copy kernel: the one of 256, 192, 128 that divides N and leaves the fewest idle
// CU slots in the last round of 256-CU waves (ties to the wider tile); 0 if none divides N.
static int gemm8_width(int M, int N) {
    int best = 0;
    double best_util = 0.0;
    for (int bn : {256, 192, 128}) {
        if (N % bn != 0) continue;
        const long tiles = (long)((M + 255) / 256) * (N / bn);
        const double util = (double)tiles / (double)(((tiles + 255) / 256) * 256);
        if (util > best_util + 1e-9) {
            best = bn;
            best_util = util;
        }
    }
    return best;
}

// The direct-copy kernel for this call, or -1 when the call does not fit it (the caller then uses gemm_kernel).
template <bool W4, int EPI, bool IL = false>
static int dispatch8(const void* a, const void* w, const float* as, const float* ws, const void* gs, const void* bias, void* c, int M, int N, int K,
                     int group, const void* R, const void* G, int L, void* stream) {
    if (K >= (1 << 24)) return -1;  // per-lane copy offsets (< 64 K) must fit the 32-bit voffset
    if (W4 && K > 65536) return -1;  // 16 x the int4 products, summed over K, must fit in int32
    // The row-segment epilogue reads ws as float4 and bias / R / G and writes C as 8-byte (int32: 16-byte) vectors.
    auto aligned = [](const void* p, uintptr_t al) { return ((uintptr_t)p & (al - 1)) == 0; };
    // A and W reach LDS by 16-byte global->LDS copies (rows stay aligned: K % 64 == 0).
    if (!aligned(a, 16) || !aligned(w, 16) || !aligned(c, 16) || !aligned(ws, 16) || !aligned(bias, 8) || !aligned(R, 8) || !aligned(G, 8)) return -1;
    if constexpr (EPI == GROUP_SCALED) {
        // One group per 128-wide slice. 128 x 128 blocks of four waves leave room for two blocks per CU, so one
        // block's group folds (vector ALU) overlap the other's products. Each wave takes all 128 rows and 32 columns:
        // one int4 fragment to widen per k step instead of two (as 64 x 64), for two more A fragment reads from LDS.
        // The block's group scales are staged whole (BN x K / 128 halves), so past K = 3456 two blocks no longer fit
        // a CU's LDS: there, with N % 256 == 0, one 128 x 256 block of eight waves per CU (each A panel serving 256
        // columns), else one 128 x 128 block, which holds the scales of K up to ~45000. In one process:
        // 4096 x 12288 x 3072 197.0 / 198.6 us two 128 x 128 blocks per CU, 200.9 / 202.3 one 128 x 256, 217.6 one
        // 128 x 128; 4096 x 3072 x 12288 210.8 one 128 x 256 (four stages 213.4 at two; one 128 x 128 234-239).
        if (group != 128 || K % 128 != 0 || N % 128 != 0 || !aligned(gs, 16)) return -1;
        {
            const int e = launch_gemm8<128, 128, 128, 3, W4, EPI, 2, 1, 4, IL>(a, w, as, ws, gs, bias, c, M, N, K, R, G, L, stream);
            if (e >= 0) return e;
        }
        if (N % 256 == 0) {
            const int e = launch_gemm8<128, 256, 128, 3, W4, EPI, 1, 1, 8, IL>(a, w, as, ws, gs, bias, c, M, N, K, R, G, L, stream);
            if (e >= 0) return e;
        }
        return launch_gemm8<128, 128, 128, 3, W4, EPI, 1, 1, 4, IL>(a, w, as, ws, gs, bias, c, M, N, K, R, G, L, stream);
    } else {
        // 128-value k slices when K allows (two stages, three for 128-wide tiles), else 64 in four stages.
        const bool wide = K % 128 == 0;
        if (W4 && !wide) return -1;
        switch (gemm8_width(M, N) * 2 + (wide ? 1 : 0)) {
            // int8 weights: eight waves of 64 x 128 (4096 x 8192 x 3072: 91.1-92.3 -> 88.4-90.0 us on one box).
            case 513:
                if constexpr (!W4) return launch_gemm8<256, 256, 128, 2, false, EPI, 1, 4, 8>(a, w, as, ws, gs, bias, c, M, N, K, R, G, L, stream);
                else return launch_gemm8<256, 256, 128, 2, W4, EPI>(a, w, as, ws, gs, bias, c, M, N, K, R, G, L, stream);
            // int8 weights: eight waves of 64 x 96 (two per SIMD, so one wave's fragment and copy waits are covered by the
            // other's products: 39.7 -> 38.6 us at 4096 x 3072 x 3072); int4 weights keep four waves of 128 x 96.
            case 385: return launch_gemm8<256, 192, 128, 2, W4, EPI, 1, (W4 ? 2 : 4), (W4 ? 4 : 8)>(a, w, as, ws, gs, bias, c, M, N, K, R, G, L, stream);
            case 257: return launch_gemm8<256, 128, 128, 3, W4, EPI>(a, w, as, ws, gs, bias, c, M, N, K, R, G, L, stream);
            case 512: if constexpr (!W4) return launch_gemm8<256, 256, 64, 4, false, EPI>(a, w, as, ws, gs, bias, c, M, N, K, R, G, L, stream); return -1;
            case 384: if constexpr (!W4) return launch_gemm8<256, 192, 64, 4, false, EPI>(a, w, as, ws, gs, bias, c, M, N, K, R, G, L, stream); return -1;
            case 256: if constexpr (!W4) return launch_gemm8<256, 128, 64, 4, false, EPI>(a, w, as, ws, gs, bias, c, M, N, K, R, G, L, stream); return -1;
            default: return -1;
        }
    }
}

template <int BM, int BN, int WM, int WN, bool W4, int EPI>
static int launch_gemm(const void* a, const void* w, const float* as, const float* ws, const void* gs, const void* bias, void* c, int M, int N, int K,
                       int group, const void* R, const void* G, int L, void* stream) {
    const size_t lds = (size_t)2 * (BM + BN) * PITCH;
    auto kern = gemm_kernel<BM, BN, WM, WN, W4, EPI>;
    static std::atomic<size_t> configured[RDA_MAX_DEVICES];
    if (const int e = ensure_dynamic_lds((const void*)kern, lds, configured)) return e;
    hipLaunchKernelGGL(kern, dim3(N / BN, (M + BM - 1) / BM), dim3(GT), lds, (hipStream_t)stream, (const int8_t*)a, (const int8_t*)w, as, ws,
                       (const half_t*)gs, (const half_t*)bias, c, M, N, K, group, (const half_t*)R, (const half_t*)G, L);
    return (int)hipGetLastError();
}

template <bool W4, int EPI>
static int dispatch(const void* a, const void* w, const float* as, const float* ws, const void* gs, const void* bias, void* c, int M, int N, int K,
                    int group, const void* R, const void* G, int L, void* stream) {
    if (M <= 0 || N <= 0 || K <= 0 || N % 64 != 0 || K % BK != 0) return RDA_ERR_INVALID;
    if (R && (!G || L <= 0)) return RDA_ERR_INVALID;
    // The activations, the output and the residual operands move in 16-byte vectors (the weight may sit anywhere).
    if (((uintptr_t)a | (uintptr_t)c | (uintptr_t)R | (uintptr_t)G) & 15) return RDA_ERR_INVALID;
    {
        const int e = dispatch8<W4, EPI>(a, w, as, ws, gs, bias, c, M, N, K, group, R, G, L, stream);
        if (e >= 0) return e;
    }
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

int rda_gemm_w4a8_il(const void* a_q, const void* w_packed, const float* a_scale, const void* group_scales, const void* bias, void* c, int M, int N,
                     int K, int group, void* stream) {
    if (M <= 0 || N <= 0 || K <= 0 || K % 128 != 0) return RDA_ERR_INVALID;
    if (((uintptr_t)a_q | (uintptr_t)c) & 15) return RDA_ERR_INVALID;
    // Only the direct-copy kernel reads k-interleaved activations: shapes it does not take are refused.
    const int e = dispatch8<true, GROUP_SCALED, true>(a_q, w_packed, a_scale, nullptr, group_scales, bias, c, M, N, K, group, nullptr, nullptr, 1, stream);
    return e >= 0 ? e : RDA_ERR_INVALID;
}

int rda_gemm_acc(const void* a_q, const void* w, int w_int4, void* acc, int M, int N, int K, void* stream) {
    if (w_int4) {
        if (K % 128 != 0) return RDA_ERR_INVALID;
        return dispatch<true, RAW_ACC>(a_q, w, nullptr, nullptr, nullptr, nullptr, acc, M, N, K, 0, nullptr, nullptr, 1, stream);
    }
    return dispatch<false, RAW_ACC>(a_q, w, nullptr, nullptr, nullptr, nullptr, acc, M, N, K, 0, nullptr, nullptr, 1, stream);
}

}  // extern "C"
