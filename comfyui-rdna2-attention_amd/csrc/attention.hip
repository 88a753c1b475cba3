// Fused attention for head dim 128 on CDNA4 matrix cores: fp16 Q/K/V, fp32 accumulation,
// log2-domain online softmax, fp16 P for the PV product, fp16 output. The int8-QK variant
// quantizes Q per row inside the kernel and reads K quantized per key by pack_k_i8.
//
// Arithmetic follows attn / attn_i8 (hip_attention.hip:160-373): scores s in fp32; the running
// maximum m only moves when some row's block maximum exceeds m + 8 (the lazy rescale,
// hip_attention.hip:333-340); p = exp2(s * scale_log2 - m) (int8: exp2(s - m) with s already
// scaled); l sums the fp32 p; P is rounded to fp16 before PV; out = fp16(o * (1 / l)).
//
// Layout: a workgroup of four wave64s owns 128 query rows of one (batch, head); each wave owns
// 32 rows and keeps Q, O, l and m in registers. Key/value tiles of 64 keys are staged in
// double-buffered LDS: K row-major (pitch 272 B), V transposed to V^T[d][key] (pitch 136 B) so
// that the PV operand reads are k-contiguous. Scores are computed transposed, S^T = K Q^T, so a
// lane's accumulator registers all belong to its own query row (lane % 32) and the softmax needs
// one cross-lane exchange (lane ^ 32). O^T = V^T P^T then consumes P straight from registers.
#include "common.h"

#define AT 256   // threads per workgroup
#define QB 128   // query rows per workgroup (32 per wave)
#define KB 64    // keys per tile
#define KP 272   // fp16 K tile row pitch in bytes
#define K8P 144  // int8 K tile row pitch in bytes
#define VP 136   // V^T tile row pitch in bytes

struct AttnArgs {
    const half_t* q;
    const half_t* k;
    const half_t* v;
    half_t* o;
    const int8_t* k8;   // int8 K [B * Hkv][Lk_pad][128]
    const float* ks;    // per-key scales [B * Hkv][Lk_pad]
    int H, Hkv, Lq, Lk, Lk_pad;
    long sqb, sqh, sql, skb, skh, skl, svb, svh, svl, sob, soh, sol;
    float scale_log2;
};

template <bool I8>
struct Tile {
    static constexpr int K_BYTES = I8 ? KB * K8P + KB * 4 : KB * KP;
    static constexpr int BYTES = K_BYTES + 128 * VP;
};

template <bool I8>
__global__ __launch_bounds__(AT, 2) void attn_kernel(AttnArgs p) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    constexpr int TB = Tile<I8>::BYTES;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, g = lane >> 5, lq = lane & 31;
    const int bh = blockIdx.y, b = bh / p.H, h = bh % p.H, hk = h / (p.H / p.Hkv);
    const int q0 = blockIdx.x * QB + wave * 32;
    const int qrow = min(q0 + lq, p.Lq - 1);
    const half_t* qp = p.q + b * p.sqb + h * p.sqh + (long)qrow * p.sql;

    // Q as the B operand of S^T = K Q^T: k-step ks covers head dims [16 ks, 16 ks + 16) (fp16) or
    // [32 ks, 32 ks + 32) (int8); lane half g supplies the upper or lower half of each step.
    h8 qf[8];
    i4v q8f[4];
    float score_scale = p.scale_log2;
    if (!I8) {
#pragma unroll
        for (int ks = 0; ks < 8; ks++) qf[ks] = *(const h8*)(qp + ks * 16 + g * 8);
    } else {
        h8 raw[8];
        float qmax = 0.f;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            raw[2 * ks] = *(const h8*)(qp + ks * 32 + g * 16);
            raw[2 * ks + 1] = *(const h8*)(qp + ks * 32 + g * 16 + 8);
        }
#pragma unroll
        for (int i = 0; i < 8; i++)
#pragma unroll
            for (int e = 0; e < 8; e++) qmax = fmaxf(qmax, fabsf((float)raw[i][e]));
        qmax = fmaxf(qmax, __shfl_xor(qmax, 32, 64));
        const float q_scale = fmaxf(qmax / 127.f, 1e-30f);  // hip_attention.hip:183
        score_scale = q_scale * p.scale_log2;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            u4v w;
#pragma unroll
            for (int d = 0; d < 4; d++) {
                u32 x = 0;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int idx = d * 4 + e;
                    const float f = (float)raw[2 * ks + (idx >> 3)][idx & 7];
                    x |= (u32)((int)rintf(f / q_scale) & 255) << (e * 8);  // hip_attention.hip:192
                }
                w[d] = x;
            }
            q8f[ks] = as_i4(w);
        }
    }

    f16v o[4];
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] = (f16v){};
    float m = -1e30f, l = 0.f;

    const half_t* kbase = p.k + b * p.skb + hk * p.skh;
    const half_t* vbase = p.v + b * p.svb + hk * p.svh;
    const int bkv = b * p.Hkv + hk;
    const int8_t* k8base = I8 ? p.k8 + (size_t)bkv * p.Lk_pad * 128 : nullptr;
    const float* ksbase = I8 ? p.ks + (size_t)bkv * p.Lk_pad : nullptr;

    u4v rk[I8 ? 2 : 4], rv[4];
    f4 rks = {};
    // Global -> registers for the tile at key0.
    auto load = [&](int key0) {
        if (!I8) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int c = t + i * AT, key = c >> 4, dc = c & 15;
                rk[i] = key0 + key < p.Lk ? *(const u4v*)(kbase + (long)(key0 + key) * p.skl + dc * 8) : (u4v){};
            }
        } else {
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int c = t + i * AT, key = c >> 3, dc = c & 7;
                rk[i] = *(const u4v*)(k8base + (size_t)(key0 + key) * 128 + dc * 16);
            }
            if (t < 16) rks = *(const f4*)(ksbase + key0 + t * 4);
        }
        const int kq = t >> 4, dq = t & 15;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int key = key0 + kq * 4 + i;
            rv[i] = key < p.Lk ? *(const u4v*)(vbase + (long)key * p.svl + dq * 8) : (u4v){};
        }
    };
    // Registers -> LDS stage buf.
    auto store = [&](int buf) {
        char* st = smem + buf * TB;
        if (!I8) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int c = t + i * AT, key = c >> 4, dc = c & 15;
                *(u4v*)(st + key * KP + dc * 16) = rk[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int c = t + i * AT, key = c >> 3, dc = c & 7;
                *(u4v*)(st + key * K8P + dc * 16) = rk[i];
            }
            if (t < 16) *(f4*)(st + KB * K8P + t * 16) = rks;
        }
        // V^T: four keys x eight dims per thread -> eight 8-byte rows of four keys.
        char* vt = st + Tile<I8>::K_BYTES;
        const int kq = t >> 4, dq = t & 15;
        h8 v0 = __builtin_bit_cast(h8, rv[0]), v1 = __builtin_bit_cast(h8, rv[1]), v2 = __builtin_bit_cast(h8, rv[2]),
           v3 = __builtin_bit_cast(h8, rv[3]);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const h4v w = {v0[j], v1[j], v2[j], v3[j]};
            *(h4v*)(vt + (dq * 8 + j) * VP + kq * 8) = w;
        }
    };

    const int tiles = (p.Lk + KB - 1) / KB;
    load(0);
    store(0);
    __syncthreads();
    for (int it = 0; it < tiles; it++) {
        const int buf = it & 1, key0 = it * KB;
        if (it + 1 < tiles) load(key0 + KB);
        const char* st = smem + buf * TB;

        float s[2][16];
        if (!I8) {
#pragma unroll
            for (int kb = 0; kb < 2; kb++) {
                f16v acc = {};
#pragma unroll
                for (int ks = 0; ks < 8; ks++) {
                    const h8 a = *(const h8*)(st + (kb * 32 + lq) * KP + ks * 32 + g * 16);
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[ks], acc, 0, 0, 0);
                }
#pragma unroll
                for (int r = 0; r < 16; r++) s[kb][r] = acc[r];
            }
        } else {
            const float* kscale = (const float*)(st + KB * K8P);
#pragma unroll
            for (int kb = 0; kb < 2; kb++) {
                i16v acc = {};
#pragma unroll
                for (int ks = 0; ks < 4; ks++) {
                    const i4v a = *(const i4v*)(st + (kb * 32 + lq) * K8P + ks * 32 + g * 16);
                    acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, q8f[ks], acc, 0, 0, 0);
                }
#pragma unroll
                for (int r4 = 0; r4 < 4; r4++) {
                    const f4 sc = *(const f4*)(kscale + kb * 32 + 8 * r4 + 4 * g);
#pragma unroll
                    for (int e = 0; e < 4; e++) s[kb][r4 * 4 + e] = (float)acc[r4 * 4 + e] * score_scale * sc[e];  // hip_attention.hip:227
                }
            }
        }
        // Keys past Lk (hip_attention.hip:324-328).
        if (key0 + KB > p.Lk) {
#pragma unroll
            for (int kb = 0; kb < 2; kb++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                    if (key0 + kb * 32 + 8 * (r >> 2) + 4 * g + (r & 3) >= p.Lk) s[kb][r] = -1e30f;
        }
        float mx = s[0][0];
#pragma unroll
        for (int kb = 0; kb < 2; kb++)
#pragma unroll
            for (int r = 0; r < 16; r++) mx = fmaxf(mx, s[kb][r]);
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        if (!I8) mx *= p.scale_log2;
        if (__any(mx > m + 8.f)) {
            const float mn = fmaxf(m, mx), alpha = __builtin_amdgcn_exp2f(m - mn);
            m = mn;
            l *= alpha;
#pragma unroll
            for (int i = 0; i < 4; i++) o[i] *= alpha;
        }
        h8 pf[4];
#pragma unroll
        for (int kb = 0; kb < 2; kb++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const float e = I8 ? __builtin_amdgcn_exp2f(s[kb][r] - m) : __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][r], p.scale_log2, -m));
                l += e;
                pf[kb * 2 + (r >> 3)][r & 7] = (half_t)e;
            }

        // O^T += V^T P^T over four 16-key steps; step j takes registers 8 (j % 2) .. +8 of score
        // block j / 2, i.e. keys 32 (j / 2) + 16 (j % 2) + 8 (i / 4) + 4 g + i % 4 for item i.
        const char* vt = st + Tile<I8>::K_BYTES;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int base = (j >> 1) * 32 + (j & 1) * 16 + 4 * g;
#pragma unroll
            for (int dt = 0; dt < 4; dt++) {
                const char* row = vt + (dt * 32 + lq) * VP;
                const h4v a0 = *(const h4v*)(row + base * 2), a1 = *(const h4v*)(row + (base + 8) * 2);
                const h8 a = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pf[j], o[dt], 0, 0, 0);
            }
        }
        if (it + 1 < tiles) store(buf ^ 1);
        __syncthreads();
    }

    const int row = q0 + lq;
    const float l_row = l + __shfl_xor(l, 32, 64);  // the two lane halves hold disjoint keys of one row
    if (row < p.Lq) {
        const float inv = 1.f / l_row;
        half_t* op = p.o + b * p.sob + h * p.soh + (long)row * p.sol;
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int r4 = 0; r4 < 4; r4++) {
                const h4v w = {to_half(o[dt][r4 * 4] * inv), to_half(o[dt][r4 * 4 + 1] * inv), to_half(o[dt][r4 * 4 + 2] * inv),
                               to_half(o[dt][r4 * 4 + 3] * inv)};
                *(h4v*)(op + dt * 32 + 8 * r4 + 4 * g) = w;
            }
    }
}

// Per-key absmax int8 quantization of K (pack_kv_i8, hip_attention.hip:56-94): 16 lanes per key,
// 8 dims each; scale = max(absmax / 127, 1e-30); k8 = rint(k / scale). Rows past Lk up to the
// padded length are written as zeros.
__global__ __launch_bounds__(256) void pack_k_i8_kernel(const half_t* __restrict__ K, int8_t* __restrict__ K8, float* __restrict__ Ks, int Hkv,
                                                        int Lk, int Lk_pad, long skb, long skh, long skl) {
    const int t = threadIdx.x, key = blockIdx.x * 16 + (t >> 4), sub = t & 15, bkv = blockIdx.y;
    const int b = bkv / Hkv, hk = bkv % Hkv;
    float f[8];
    float mx = 0.f;
    if (key < Lk) {
        const h8 v = *(const h8*)(K + b * skb + hk * skh + (long)key * skl + sub * 8);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            f[i] = (float)v[i];
            mx = fmaxf(mx, fabsf(f[i]));
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++) f[i] = 0.f;
    }
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 16));
    const float scale = fmaxf(mx / 127.f, 1e-30f);
    u2v w;
#pragma unroll
    for (int d = 0; d < 2; d++) {
        u32 x = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) x |= (u32)((int)rintf(f[d * 4 + i] / scale) & 255) << (i * 8);
        w[d] = x;
    }
    if (key < Lk_pad) {
        *(u2v*)(K8 + ((size_t)bkv * Lk_pad + key) * 128 + sub * 8) = w;
        if (sub == 0) Ks[(size_t)bkv * Lk_pad + key] = scale;
    }
}

static AttnArgs make_args(const void* q, const void* k, const void* v, void* out, int H, int Hkv, int Lq, int Lk, const long* st, float scale) {
    AttnArgs a;
    a.q = (const half_t*)q;
    a.k = (const half_t*)k;
    a.v = (const half_t*)v;
    a.o = (half_t*)out;
    a.k8 = nullptr;
    a.ks = nullptr;
    a.H = H;
    a.Hkv = Hkv;
    a.Lq = Lq;
    a.Lk = Lk;
    a.Lk_pad = (Lk + KB - 1) / KB * KB;
    a.sqb = st[0]; a.sqh = st[1]; a.sql = st[2];
    a.skb = st[3]; a.skh = st[4]; a.skl = st[5];
    a.svb = st[6]; a.svh = st[7]; a.svl = st[8];
    a.sob = st[9]; a.soh = st[10]; a.sol = st[11];
    a.scale_log2 = scale * 1.4426950408889634f;
    return a;
}

template <bool I8>
static int launch_attn(const AttnArgs& a, int B, void* stream) {
    const size_t lds = 2 * (size_t)Tile<I8>::BYTES;
    static bool configured = false;
    if (!configured) {
        const hipError_t e = hipFuncSetAttribute((const void*)attn_kernel<I8>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return (int)e;
        configured = true;
    }
    hipLaunchKernelGGL(attn_kernel<I8>, dim3((a.Lq + QB - 1) / QB, B * a.H), dim3(AT), lds, (hipStream_t)stream, a);
    return (int)hipGetLastError();
}

static bool attn_shapes_ok(int B, int H, int Hkv, int Lq, int Lk) {
    return B > 0 && H > 0 && Hkv > 0 && H % Hkv == 0 && Lq > 0 && Lk > 0;
}

extern "C" {

size_t rda_attn_i8_workspace(int B, int Hkv, int Lk) {
    const size_t pad = (size_t)(Lk + KB - 1) / KB * KB;
    return (size_t)B * Hkv * pad * 128 + (size_t)B * Hkv * pad * 4;
}

int rda_attn(const void* q, const void* k, const void* v, void* out, int B, int H, int Hkv, int Lq, int Lk, const long* strides, float scale,
             void* stream) {
    if (!attn_shapes_ok(B, H, Hkv, Lq, Lk)) return RDA_ERR_INVALID;
    return launch_attn<false>(make_args(q, k, v, out, H, Hkv, Lq, Lk, strides, scale), B, stream);
}

int rda_pack_k_i8(const void* k, void* workspace, int B, int Hkv, int Lk, long skb, long skh, long skl, void* stream) {
    if (B <= 0 || Hkv <= 0 || Lk <= 0) return RDA_ERR_INVALID;
    const int pad = (Lk + KB - 1) / KB * KB;
    int8_t* k8 = (int8_t*)workspace;
    float* ks = (float*)(k8 + (size_t)B * Hkv * pad * 128);
    hipLaunchKernelGGL(pack_k_i8_kernel, dim3(pad / 16, B * Hkv), dim3(256), 0, (hipStream_t)stream, (const half_t*)k, k8, ks, Hkv, Lk, pad, skb,
                       skh, skl);
    return (int)hipGetLastError();
}

int rda_attn_i8(const void* q, const void* workspace, const void* v, void* out, int B, int H, int Hkv, int Lq, int Lk, const long* strides,
                float scale, void* stream) {
    if (!attn_shapes_ok(B, H, Hkv, Lq, Lk)) return RDA_ERR_INVALID;
    AttnArgs a = make_args(q, nullptr, v, out, H, Hkv, Lq, Lk, strides, scale);
    a.k8 = (const int8_t*)workspace;
    a.ks = (const float*)(a.k8 + (size_t)B * Hkv * a.Lk_pad * 128);
    return launch_attn<true>(a, B, stream);
}

}  // extern "C"
