// Activation -> block Hadamard ("ConvRot") rotation -> per-token absmax quantization, one pass.
//
// One 256-thread workgroup (four wave64s) owns one row. A rotation group is split over
// lanes that each hold 16 consecutive values: the two fastest base-4 digits are H4 steps
// in registers, an LDS transpose per group brings the remaining digits into registers,
// and the rotated fp16 row stays in LDS until the row's absmax is known. The int8 codes
// are written row-major [M, K], which is what the GEMM's LDS stage reads.
//
// Arithmetic follows rot_quant (int8_gemm.hip:151-243) step for step: fp32 butterflies
// in digit order 1, 4, 16, 64, times 1/16, rounded to fp16, absmax over the fp16 values,
// scale = max(absmax / 127, 1e-30), q = clamp(floor(x / scale + 0.5), -128, 127).
#include "common.h"

enum Act { NO_ACT = 0, SITU = 1, SWIGLU = 2, GATE = 3, MOD = 4 };
struct ModArgs {
    const float* w;
    const half_t* s;
    const half_t* t;
    int L;
    float eps;
};

#define QT 256  // threads per row of the reference's kernels (rms_norm's summation order follows it)
#define MAX_LDS_K 16384  // longest row held in LDS (fp16, 32 KiB); rotations need it, plain quantization does not

// int8_gemm.hip:106-109
// s - 2 x as one FMA: 2 x is exact, so fma(-2, x, s) rounds s - 2 x once, exactly as the separate product and
// difference do.
__device__ __forceinline__ void h4(float& a, float& b, float& c, float& d) {
    const float s = a + b + c + d, a0 = a, b0 = b;
    a = __builtin_fmaf(-2.f, d, s);
    b = __builtin_fmaf(-2.f, c, s);
    c = __builtin_fmaf(-2.f, b0, s);
    d = __builtin_fmaf(-2.f, a0, s);
}
__device__ __forceinline__ void h16(float (&v)[16]) {
#pragma unroll
    for (int i = 0; i < 16; i += 4) h4(v[i], v[i + 1], v[i + 2], v[i + 3]);
#pragma unroll
    for (int i = 0; i < 4; i++) h4(v[i], v[i + 4], v[i + 8], v[i + 12]);
}

// int8_gemm.hip:118-127, with the exponentials of common.h.
__device__ __forceinline__ float soft_tanh(float x) {
    const float ax = fabsf(x), t = rda_exp2f(-2.885390082f * ax);
    float y = (1.f - t) / (1.f + t);
    if (ax < 0.02f) y = ax * (1.f - ax * ax * (1.f / 3.f - ax * ax * (2.f / 15.f)));
    return x < 0.f ? -y : y;
}
__device__ __forceinline__ float situ(float hidden, float gate) {
    const float sigmoid = 1.f / (1.f + rda_exp2f(-1.442695041f * gate));
    return r16(4.f * soft_tanh(gate * 0.25f) * sigmoid * 25.f * soft_tanh(hidden * 0.04f));
}
// The kernels round "r16(a * b)" and "r16(a + b)" of two fp16 values in pairs, as fp16 products and sums (v_pk_mul_f16,
// v_pk_add_f16): the fp32 product of two fp16 values is exact, so rounding it to fp16 gives the fp16 product; an fp32
// sum rounded again to fp16 is the correctly rounded fp16 sum too (a second rounding is harmless when the first keeps
// at least 2 x 11 + 2 significant bits, as fp32's 24 do). -ffp-contract=off keeps "a * s + t" two roundings.
__device__ __forceinline__ h2 to_half2(float a, float b) {
    asm("" : "+v"(a), "+v"(b));  // round to fp32 first, as in to_half
    return __builtin_convertvector((f2){a, b}, h2);
}
// SwiGLU (int8_gemm.hip:130-132): r16(r16(silu(g)) u) with silu(g) = g / (1 + rda_expf(-g)) in fp32; the sigmoid
// gate (int8_gemm.hip:135-137): r16(x r16(sigmoid(gate))), sigmoid(g) = 1 / (1 + rda_expf(-g)) in fp32.
// Both take a fast path -- hardware exp2 of a rounded argument and a hardware reciprocal -- whose value q lies
// within 11 fp32 ulps of the exact one over every fp16 input (measured on all 65536; <= 4 ulps for |g| < 4).
// round_sure rounds the two ends of [q (1 - d), q (1 + d)], d = 13 x 2^-23 (at least 12 ulps of q on either side
// after the ends' own fp32 rounding), to fp16: where both give the same fp16 value, every value between them rounds
// to it as well, the exact one included, and that is r16 of the exact value. This holds on fp16's subnormal grid
// and at the overflow threshold too, and values too small for fp32's normal range round to zero either way. The
// pairs where the ends differ (about 0.3% of values) take the exact formula; the SwiGLU and gate tests run every
// finite fp16 gate through the kernels and compare the codes, which then fix r16 of the value, with the oracle's.
__device__ __forceinline__ float silu_fast(float g) { return g * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-g * 1.44269504088896341f)); }
__device__ __forceinline__ float silu_exact(float g) { return g / (1.f + rda_expf(-g)); }
__device__ __forceinline__ float sigmoid_fast(float g) { return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-g * 1.44269504088896341f)); }
__device__ __forceinline__ float sigmoid_exact(float g) { return 1.f / (1.f + rda_expf(-g)); }
template <class Exact>
__device__ __forceinline__ h2 round_sure(float q0, float q1, Exact exact) {
    constexpr float lo_f = 1.f - 0x1.ap-20f, hi_f = 1.f + 0x1.ap-20f;  // 1 -+ 13 x 2^-23, both exact in fp32
    const h2 lo = to_half2(q0 * lo_f, q1 * lo_f), hi = to_half2(q0 * hi_f, q1 * hi_f);
    const u32 diff = __builtin_bit_cast(u32, lo) ^ __builtin_bit_cast(u32, hi);
    const bool unsure0 = (diff & 0xffffu) != 0, unsure1 = (diff >> 16) != 0;
    h2 r = lo;
    // Element by element, so that a wave runs the exact formula only for the elements some lane needs it for.
    if (__any(unsure0)) {
        if (unsure0) r[0] = to_half(exact(0));
    }
    if (__any(unsure1)) {
        if (unsure1) r[1] = to_half(exact(1));
    }
    return r;
}

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// (int)floorf(x) in one instruction (the compiler emits a floor and a truncation); x is finite here.
__device__ __forceinline__ int cvt_floor(float x) {
    int r;
    asm("v_cvt_flr_i32_f32 %0, %1" : "=v"(r) : "v"(x));
    return r;
}

// The low bytes of a, b, c, d as one word (a in the lowest byte): three byte permutes.
__device__ __forceinline__ u32 pack4(int a, int b, int c, int d) {
    const u32 ab = __builtin_amdgcn_perm((u32)b, (u32)a, 0x0c0c0400u), cd = __builtin_amdgcn_perm((u32)d, (u32)c, 0x0c0c0400u);
    return __builtin_amdgcn_perm(cd, ab, 0x05040100u);
}

// GROUP 256 or 128 rotates; GROUP 0 is quant_pack_a (no rotation, int8_gemm.hip:93-103). NW waves per row: the
// launcher sizes it to the row (K / 1024 waves, so that K = 3072 keeps every lane busy in both passes: the kernel
// is vector-ALU bound); MOD keeps 4 (QT threads), whose sum of squares follows the reference's thread order.
// IL: the codes k-interleaved (each 8 values of k stored as their 4 even ones, then their 4 odd ones).
// WL (the rotations other than MOD): each wave keeps the rotated fp16 values of its own passes (1024 values each) in an
// LDS region of its own -- pass p at SW_BYTES + 2048 p, the last pass inside its transpose buffer, free by then -- and
// quantizes them itself once the row maximum is known, so a row takes NW (SW_BYTES + 2048 (passes - 1)) bytes of LDS
// instead of 2 K + NW SW_BYTES (K = 3072: 13.1 against 19.2 KiB; more rows in flight per CU). MOD stages its input
// row in LDS for the sum of squares and rotates in place there.
#define SW_BYTES (64 * 17 * 4)  // a wave's transpose buffer: 17 floats per lane
template <int GROUP, int NW>
__host__ __device__ constexpr int rot_passes(int K) { return (K / GROUP + NW * (1024 / GROUP) - 1) / (NW * (1024 / GROUP)); }

template <int ACT, bool I4, int GROUP, int NW, bool IL>
__global__ __launch_bounds__(NW * 64) void rot_quant_kernel(const half_t* __restrict__ X, long ldx, const half_t* __restrict__ U,
                                                       int8_t* __restrict__ Aq, float* __restrict__ as, int K, ModArgs mod) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    __shared__ float red[8];
    constexpr bool WL = GROUP != 0 && ACT != MOD;
    half_t* rotated = (half_t*)smem;
    const int row = blockIdx.x, t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const half_t* x = X + (size_t)row * ldx;
    float mx = 0.f;

    // GROUP 0 stages the row in LDS when it fits (K <= MAX_LDS_K); longer rows are read again from global memory by
    // the quantization pass below, so quant_pack_a takes any K, as the reference's does.
    const bool staged = GROUP != 0 || K <= MAX_LDS_K;
    if constexpr (GROUP == 0) {
        for (int i = t; i < K / 8; i += NW * 64) {
            const h8 v = ((const h8*)x)[i];
            if (staged) ((h8*)rotated)[i] = v;
#pragma unroll
            for (int j = 0; j < 8; j++) mx = fmaxf(mx, fabsf((float)v[j]));
        }
    } else {
        float rstd = 0.f;
        if constexpr (ACT == MOD) {
            // The sum of squares in rms_norm_row's order (rms_norm.hip:19-37): thread t adds its chunks
            // t + 256c with FMAs, 32-lane butterflies, then the eight partial sums in order.
            float sum = 0.f;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int i = t + c * QT;
                if (i < K / 8) {
                    const h8 v = ((const h8*)x)[i];
                    ((h8*)rotated)[i] = v;
#pragma unroll
                    for (int j = 0; j < 8; j++) sum = __builtin_fmaf((float)v[j], (float)v[j], sum);
                }
            }
            sum = xor_butterfly_sum<32>(sum);
            static_assert(ACT != MOD || NW * 64 == QT, "the MOD sum of squares needs the reference's 256 threads");
            if ((t & 31) == 0) red[t >> 5] = sum;
            __syncthreads();
            float total = 0.f;
#pragma unroll
            for (int i = 0; i < 8; i++) total += red[i];
            rstd = 1.f / sqrtf(total / (float)K + mod.eps);
            __syncthreads();
        }
        constexpr int LPG = GROUP / 16;  // lanes per group, 16 values each
        constexpr int GPW = 64 / LPG;    // groups per wave per pass
        const int gl = lane / LPG, c = lane % LPG, groups = K / GROUP;
        const int passes = rot_passes<GROUP, NW>(K), wreg = SW_BYTES + 2048 * (passes - 1);  // WL: a wave's LDS region
        char* wbase = WL ? smem + (size_t)wave * wreg : smem + (size_t)K * 2 + (size_t)wave * SW_BYTES;
        float* sw = (float*)wbase + gl * LPG * 17;
        const size_t mrow = ACT == MOD ? (size_t)(row / mod.L) * K : 0;
        const half_t* ms = ACT == MOD ? mod.s + mrow : nullptr;
        const half_t* mt = ACT == MOD ? mod.t + mrow : nullptr;
        const float norm = GROUP == 256 ? 0.0625f : 0.0883883461356163025f;

        for (int g0 = wave * GPW; g0 < groups; g0 += NW * GPW) {
            const int g = g0 + gl;
            const bool active = g < groups;
            float v[16];
            if (active) {
                const int e0 = g * GROUP + c * 16;
                const half_t* src = ACT == MOD ? rotated : x;
                const h8 lo = *(const h8*)(src + e0), hi = *(const h8*)(src + e0 + 8);
                if (ACT == SITU) {
                    const h8 glo = *(const h8*)(x + K + e0), ghi = *(const h8*)(x + K + e0 + 8);
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        v[i] = situ((float)lo[i], (float)glo[i]);
                        v[8 + i] = situ((float)hi[i], (float)ghi[i]);
                    }
                } else if (ACT == SWIGLU) {
                    const half_t* u = U + (size_t)row * K;
                    const h8 ulo = *(const h8*)(u + e0), uhi = *(const h8*)(u + e0 + 8);
#pragma unroll
                    for (int i = 0; i < 16; i += 2) {
                        const float g0 = (float)(i < 8 ? lo[i] : hi[i - 8]), g1 = (float)(i < 8 ? lo[i + 1] : hi[i - 7]);
                        const h2 sg = round_sure(silu_fast(g0), silu_fast(g1), [&](int k) { return silu_exact(k ? g1 : g0); });
                        const h2 pr = sg * (h2){i < 8 ? ulo[i] : uhi[i - 8], i < 8 ? ulo[i + 1] : uhi[i - 7]};
                        v[i] = (float)pr[0];
                        v[i + 1] = (float)pr[1];
                    }
                } else if (ACT == GATE) {
                    const half_t* u = U + (size_t)row * K;
                    const h8 ulo = *(const h8*)(u + e0), uhi = *(const h8*)(u + e0 + 8);
#pragma unroll
                    for (int i = 0; i < 16; i += 2) {
                        const float g0 = (float)(i < 8 ? ulo[i] : uhi[i - 8]), g1 = (float)(i < 8 ? ulo[i + 1] : uhi[i - 7]);
                        const h2 sg = round_sure(sigmoid_fast(g0), sigmoid_fast(g1), [&](int k) { return sigmoid_exact(k ? g1 : g0); });
                        const h2 pr = (h2){i < 8 ? lo[i] : hi[i - 8], i < 8 ? lo[i + 1] : hi[i - 7]} * sg;
                        v[i] = (float)pr[0];
                        v[i + 1] = (float)pr[1];
                    }
                } else if (ACT == MOD) {
                    const h8 slo = *(const h8*)(ms + e0), shi = *(const h8*)(ms + e0 + 8);
                    const h8 tlo = *(const h8*)(mt + e0), thi = *(const h8*)(mt + e0 + 8);
                    const f4* w = (const f4*)(mod.w + e0);
                    const f4 w0 = w[0], w1 = w[1], w2 = w[2], w3 = w[3];
                    const float wv[16] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w, w2.x, w2.y, w2.z, w2.w, w3.x, w3.y, w3.z, w3.w};
#pragma unroll
                    for (int i = 0; i < 16; i += 2) {
                        // modulate (int8_gemm.hip:140-143): r16(r16(r16(x rstd (w + 1)) s) + t), two elements at a time.
                        const h8 &xs = i < 8 ? lo : hi, &ss = i < 8 ? slo : shi, &ts = i < 8 ? tlo : thi;
                        const int j = i & 7;
                        const h2 a = to_half2((float)xs[j] * rstd * (wv[i] + 1.f), (float)xs[j + 1] * rstd * (wv[i + 1] + 1.f));
                        const h2 m = a * (h2){ss[j], ss[j + 1]} + (h2){ts[j], ts[j + 1]};
                        v[i] = (float)m[0];
                        v[i + 1] = (float)m[1];
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        v[i] = (float)lo[i];
                        v[8 + i] = (float)hi[i];
                    }
                }
                h16(v);  // digits at strides 1 and 4
#pragma unroll
                for (int i = 0; i < 16; i++) sw[c * 17 + i] = v[i];
            }
            wave_sync();
            if (active) {
                if (GROUP == 256) {
                    // Lane c now holds elements c + 16i: digits at strides 16 and 64.
#pragma unroll
                    for (int i = 0; i < 16; i++) v[i] = sw[i * 17 + c];
                    h16(v);
                } else {
                    // Lane c takes the columns c and c + 8 (elements c + 16i, c + 8 + 16i, i < 8):
                    // an H4 over the stride-16 digit, then an H2 over the stride-64 digit.
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        v[i] = sw[i * 17 + c];
                        v[8 + i] = sw[i * 17 + c + 8];
                    }
#pragma unroll
                    for (int b = 0; b < 16; b += 4) h4(v[b], v[b + 1], v[b + 2], v[b + 3]);
#pragma unroll
                    for (int b = 0; b < 16; b += 8)
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const float p = v[b + i], q = v[b + i + 4];
                            v[b + i] = p + q;
                            v[b + i + 4] = p - q;
                        }
                }
            }
            // The row maximum is taken before the rounding to fp16 and rounded once at the end: rounding is monotonic,
            // so max(round |p|) = round(max |p|), one conversion per element fewer.
            const int p = (g0 - wave * GPW) / (NW * GPW);
            if (WL && p == passes - 1) wave_sync();  // the last pass reuses the transpose buffer: every lane has read it
            if (active) {
                half_t* dst = WL ? (half_t*)(wbase + (p == passes - 1 ? 0 : SW_BYTES + 2048 * p)) + gl * GROUP : rotated + g * GROUP;
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const float y = v[i] * norm;
                    // element of the group: c + 16 i (GROUP 256); c + 16 i and c + 8 + 16 (i - 8) (GROUP 128)
                    dst[GROUP == 256 ? c + 16 * i : c + (i < 8 ? 16 * i : 8 + 16 * (i - 8))] = to_half(y);
                    mx = fmaxf(mx, fabsf(y));
                }
            }
            wave_sync();
        }
    }
    mx = rows_max(row_max16(mx));  // the wave's maximum (exact in any order)
    __syncthreads();
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int w = 1; w < NW; w++) mx = fmaxf(mx, red[w]);
    if (GROUP != 0) mx = r16(mx);  // the largest |rotated fp16 value| (see the rotation pass)
    const float scale = I4 ? fmaxf(mx, 1e-10f) / 7.f : fmaxf(mx / 127.f, 1e-30f);
    if (t == 0) as[row] = scale;

    const float rcp = 1.f / scale;
    int8_t* out = Aq + (size_t)row * K;
    // The 16 codes of the row's chunk ch (values 16 ch ..) from its fp16 values lo, hi, stored in one 16-byte write.
    auto quant16 = [&](const h8 lo, const h8 hi, int ch) __attribute__((always_inline)) {
        const u4v wl = __builtin_bit_cast(u4v, lo), wh = __builtin_bit_cast(u4v, hi);
        int q[16];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float f = (float)(i < 8 ? lo[i] : hi[i - 8]);
            // f / scale as div_by_scale, its first product f * rcp taken straight from the fp16 value (one mixed-precision
            // FMA, + 0, in place of a conversion and a multiply: the same value, up to the sign of a zero, which the
            // code does not depend on).
            const u32 w = i < 8 ? wl[i >> 1] : wh[(i - 8) >> 1];
            float y;
            if (i & 1) asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(y) : "v"(w), "v"(rcp));
            else asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[1,0,0]" : "=v"(y) : "v"(w), "v"(rcp));
            const float d = __builtin_fmaf(__builtin_fmaf(-y, scale, f), rcp, y);
            // int8_gemm.hip:84 and :53. The clamp to [lo, hi] (integers) goes before the rounding: both orders give the same
            // code for every input, NaN included (-128 / -7), and floor then truncation fuse into one conversion.
            if (I4) q[i] = (int)rintf(fminf(fmaxf(d, -7.f), 7.f));
            else q[i] = cvt_floor(fminf(fmaxf(d + 0.5f, -128.f), 127.f));
        }
        u4v o;
        if constexpr (IL) {
#pragma unroll
            for (int d = 0; d < 4; d++) {
                const int b = (d >> 1) * 8 + (d & 1);
                o[d] = pack4(q[b], q[b + 2], q[b + 4], q[b + 6]);
            }
        } else {
#pragma unroll
            for (int d = 0; d < 4; d++) o[d] = pack4(q[d * 4], q[d * 4 + 1], q[d * 4 + 2], q[d * 4 + 3]);
        }
        *(u4v*)(out + ch * 16) = o;
    };
    if constexpr (WL) {
        // Each wave its own passes: lane l takes values 16 l .. of pass p's 1024 (chunk (wave + NW p) 64 + l of the row).
        const int passes = rot_passes<GROUP, NW>(K), wreg = SW_BYTES + 2048 * (passes - 1);
        for (int p = 0; p < passes; p++) {
            const int ch = (wave + NW * p) * 64 + lane;
            if (ch >= K / 16) break;  // past the row's groups (a wave's later passes may hold none)
            const h8* from = (const h8*)(smem + (size_t)wave * wreg + (p == passes - 1 ? 0 : SW_BYTES + 2048 * p)) + lane * 2;
            quant16(from[0], from[1], ch);
        }
    } else {
        const h8* src = staged ? (const h8*)rotated : (const h8*)x;
        for (int ch = t; ch < K / 16; ch += NW * 64) quant16(src[ch * 2], src[ch * 2 + 1], ch);
    }
}

template <int ACT, bool I4, int GROUP, int NW>
static int launch_rot_quant_nw(const void* x, long ldx, const void* u, void* aq, float* as, int M, int K, ModArgs mod, void* stream, int il) {
    const size_t lds = GROUP == 0 ? (K <= MAX_LDS_K ? (size_t)K * 2 : 0)
                       : ACT == MOD ? (size_t)K * 2 + NW * SW_BYTES
                                    : (size_t)NW * (SW_BYTES + 2048 * (rot_passes<GROUP ? GROUP : 16, NW>(K) - 1));
    if (il) {  // k-interleaved codes: the plain rotation only
        if constexpr (ACT == NO_ACT && !I4 && GROUP != 0)
            hipLaunchKernelGGL((rot_quant_kernel<ACT, I4, GROUP, NW, true>), dim3(M), dim3(NW * 64), lds, (hipStream_t)stream, (const half_t*)x, ldx,
                               (const half_t*)u, (int8_t*)aq, as, K, mod);
        else return RDA_ERR_INVALID;
    } else {
        hipLaunchKernelGGL((rot_quant_kernel<ACT, I4, GROUP, NW, false>), dim3(M), dim3(NW * 64), lds, (hipStream_t)stream, (const half_t*)x, ldx,
                           (const half_t*)u, (int8_t*)aq, as, K, mod);
    }
    return (int)hipGetLastError();
}

template <int ACT, bool I4, int GROUP>
static int launch_rot_quant(const void* x, long ldx, const void* u, void* aq, float* as, int M, int K, ModArgs mod, void* stream, int il = 0) {
    if (M <= 0 || K <= 0 || K % (GROUP ? GROUP : 16) != 0 || (GROUP != 0 && K > MAX_LDS_K)) return RDA_ERR_INVALID;
    // Rows are read (and the int8 rows written) in 16-byte vectors: every row must start on a 16-byte boundary.
    if (M > 1 && (ldx < (ACT == SITU ? 2L * K : (long)K) || ldx % 8 != 0)) return RDA_ERR_INVALID;
    if (((uintptr_t)x | (uintptr_t)u | (uintptr_t)aq | (uintptr_t)mod.w | (uintptr_t)mod.s | (uintptr_t)mod.t) & 15) return RDA_ERR_INVALID;
    if constexpr (ACT == MOD || GROUP == 0) {
        return launch_rot_quant_nw<ACT, I4, GROUP, 4>(x, ldx, u, aq, as, M, K, mod, stream, il);
    } else {
        // One wave per 1024 values, up to four: every lane has a chunk in both passes when K is a multiple of 1024.
        switch (K >= 4096 ? 4 : K <= 1024 ? 1 : K / 1024) {
        case 1: return launch_rot_quant_nw<ACT, I4, GROUP, 1>(x, ldx, u, aq, as, M, K, mod, stream, il);
        case 2: return launch_rot_quant_nw<ACT, I4, GROUP, 2>(x, ldx, u, aq, as, M, K, mod, stream, il);
        case 3: return launch_rot_quant_nw<ACT, I4, GROUP, 3>(x, ldx, u, aq, as, M, K, mod, stream, il);
        default: return launch_rot_quant_nw<ACT, I4, GROUP, 4>(x, ldx, u, aq, as, M, K, mod, stream, il);
        }
    }
}

template <int ACT, bool I4>
static int dispatch_group(int group, const void* x, long ldx, const void* u, void* aq, float* as, int M, int K, ModArgs mod, void* stream, int il = 0) {
    if (group == 256) return launch_rot_quant<ACT, I4, 256>(x, ldx, u, aq, as, M, K, mod, stream, il);
    if (group == 128) return launch_rot_quant<ACT, I4, 128>(x, ldx, u, aq, as, M, K, mod, stream, il);
    return RDA_ERR_INVALID;
}

extern "C" {

int rda_quant_pack_a(const void* x, long ldx, void* a_q, float* a_scale, int M, int K, void* stream) {
    return launch_rot_quant<NO_ACT, false, 0>(x, ldx, nullptr, a_q, a_scale, M, K, ModArgs{}, stream);
}

int rda_rot_quant_pack_a(const void* x, long ldx, void* a_q, float* a_scale, int M, int K, int group, void* stream) {
    return dispatch_group<NO_ACT, false>(group, x, ldx, nullptr, a_q, a_scale, M, K, ModArgs{}, stream);
}

int rda_rot_quant_pack_a_il(const void* x, long ldx, void* a_q, float* a_scale, int M, int K, int group, void* stream) {
    return dispatch_group<NO_ACT, false>(group, x, ldx, nullptr, a_q, a_scale, M, K, ModArgs{}, stream, 1);
}

int rda_situ_rot_quant_pack_a(const void* x, long ldx, void* a_q, float* a_scale, int M, int K, int group, void* stream) {
    return dispatch_group<SITU, false>(group, x, ldx, nullptr, a_q, a_scale, M, K, ModArgs{}, stream);
}

int rda_swiglu_rot_quant_pack_a(const void* gate, const void* up, void* a_q, float* a_scale, int M, int K, int group, void* stream) {
    return dispatch_group<SWIGLU, false>(group, gate, K, up, a_q, a_scale, M, K, ModArgs{}, stream);
}

int rda_gate_rot_quant_pack_a(const void* x, const void* gate, void* a_q, float* a_scale, int M, int K, int group, void* stream) {
    return dispatch_group<GATE, false>(group, x, K, gate, a_q, a_scale, M, K, ModArgs{}, stream);
}

int rda_mod_rot_quant_pack_a(const void* x, void* a_q, float* a_scale, int M, int K, const float* w, const void* s, const void* t, int L,
                             float eps, void* stream) {
    if (L <= 0 || K > 8192) return RDA_ERR_INVALID;
    return launch_rot_quant<MOD, false, 256>(x, K, nullptr, a_q, a_scale, M, K, ModArgs{w, (const half_t*)s, (const half_t*)t, L, eps}, stream);
}

int rda_rot_quant_pack_a_i4(const void* x, long ldx, void* a_q, float* a_scale, int M, int K, int group, void* stream) {
    return dispatch_group<NO_ACT, true>(group, x, ldx, nullptr, a_q, a_scale, M, K, ModArgs{}, stream);
}

}  // extern "C"
