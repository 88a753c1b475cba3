// Fused attention for head dim 128 on CDNA4 matrix cores: fp16 Q/K/V, fp32 accumulation,
// log2-domain online softmax, fp16 P for the PV product, fp16 output. The int8-QK variant
// quantizes Q per row inside the kernel and reads K quantized per key by pack_k_i8.
//
// Arithmetic follows attn / attn_i8 (hip_attention.hip:160-373): scores s in fp32; the running
// maximum m only moves when some row's block maximum exceeds m + 8 (the lazy rescale,
// hip_attention.hip:333-340); p = exp2(s * scale_log2 - m) (int8: exp2(s - m) with s already
// scaled); l sums the fp32 p; P is rounded to fp16 before PV; out = fp16(o * (1 / l)).
//
// Work split. A workgroup of four wave64s owns 128 query rows of one (batch, head). The waves
// form two pairs that walk the two halves of the key range; inside a pair each wave owns 64
// query rows and keeps Q, O, l and m for them in registers. At the end the second pair's
// (m, l, O) is merged into the first through LDS. With 128-row blocks the attention
// configuration (24 heads x 4096 rows) is 768 workgroups, three per CU, one resident at a time.
// Block ids are remapped so that the workgroups an XCD runs together belong to one head and
// share its K/V through that XCD's L2.
//
// Tiles. Each pair stages 64-key tiles in its own double-buffered LDS: K row-major (pitch
// 272 B, so the 16-byte reads of 16 consecutive keys hit distinct banks) and V transposed to
// V^T[d][key] (pitch 144 B). Inside every 16-key group of a V^T row the keys are stored in the
// order 0-3, 8-11, 4-7, 12-15: that is the order in which the S^T accumulator registers of
// lane half g hold them, so each PV operand is one 16-byte read.
//
// Products. Scores are computed transposed, S^T = K Q^T (32x32x16 fp16 MFMA; 32x32x32 int8 for
// int8-QK), so the accumulator registers of a lane all belong to its own query row (lane % 32)
// and the row statistics need one exchange with lane ^ 32. O^T = V^T P^T then takes P straight
// from those registers: in a 32x32 block lane l supplies row l % 32 of the A operand and column
// l % 32 of B, k-half l / 32, and receives C[8 (r / 4) + 4 (l / 32) + r % 4][l % 32] in register r.
#include "common.h"

#define AT 256   // threads per workgroup: two pairs of waves
#define PT 128   // threads per pair
#define QB 128   // query rows per workgroup (64 per wave)
#define KB 64    // keys per tile
#define KP 272   // fp16 K tile row pitch (bytes)
#define K8P 144  // int8 K tile row pitch
#define VP 144   // V^T tile row pitch

struct AttnArgs {
    const half_t* q;
    const half_t* k;
    const half_t* v;
    half_t* o;
    const int8_t* k8;  // int8 K [B * Hkv][Lk_pad][128]
    const float* ks;   // per-key scales [B * Hkv][Lk_pad]
    int H, Hkv, Lq, Lk, Lk_pad, qblocks, nblocks;
    long sqb, sqh, sql, skb, skh, skl, svb, svh, svl, sob, soh, sol;
    float scale_log2;
};

template <bool I8>
struct Tile {
    static constexpr int K_BYTES = I8 ? KB * K8P + KB * 4 : KB * KP;
    static constexpr int BYTES = K_BYTES + 128 * VP;  // one stage
    static constexpr int PAIR = 2 * BYTES;            // two stages per pair
    static constexpr int MERGE = 2 * 64 * 132 * 4;    // (O, m, l) of the second pair's two waves
    static constexpr int LDS = 2 * PAIR > MERGE ? 2 * PAIR : MERGE;
};

// Byte offset, inside a V^T row, of the 4-key group kq (keys 4 kq .. 4 kq + 3) of a tile.
__device__ __forceinline__ int vt_pos(int kq) { return (kq >> 2) * 32 + (kq & 1) * 16 + ((kq >> 1) & 1) * 8; }

template <bool I8>
__global__ __launch_bounds__(AT, 1) void attn_kernel(AttnArgs p) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    constexpr int TB = Tile<I8>::BYTES;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, g = lane >> 5, lq = lane & 31;
    const int pair = t >> 7, pt = t & (PT - 1), wq = wave & 1;

    // Block remap: consecutive block ids go round-robin to the 8 XCDs; give each XCD a contiguous run
    // of (head, q-block) work so its resident workgroups share K/V.
    int blk = blockIdx.x;
    if (p.nblocks % 8 == 0) blk = (blk % 8) * (p.nblocks / 8) + blk / 8;
    const int bh = blk / p.qblocks, qblk = blk % p.qblocks;
    const int b = bh / p.H, h = bh % p.H, hk = h / (p.H / p.Hkv);
    const int q0 = qblk * QB + wq * 64;

    // Q as the B operand of S^T = K Q^T, for the lane's two rows q0 + 32 qb + lq.
    h8 qf[2][8];
    i4v q8f[2][4];
    float score_scale[2] = {p.scale_log2, p.scale_log2};
#pragma unroll
    for (int qb = 0; qb < 2; qb++) {
        const int qrow = min(q0 + qb * 32 + lq, p.Lq - 1);
        const half_t* qp = p.q + b * p.sqb + h * p.sqh + (long)qrow * p.sql;
        if (!I8) {
#pragma unroll
            for (int ks = 0; ks < 8; ks++) qf[qb][ks] = *(const h8*)(qp + ks * 16 + g * 8);
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
            score_scale[qb] = q_scale * p.scale_log2;
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
                q8f[qb][ks] = as_i4(w);
            }
        }
    }

    f16v o[2][4];
#pragma unroll
    for (int qb = 0; qb < 2; qb++)
#pragma unroll
        for (int i = 0; i < 4; i++) o[qb][i] = (f16v){};
    float m[2] = {-1e30f, -1e30f}, l[2] = {0.f, 0.f};

    const half_t* kbase = p.k + b * p.skb + hk * p.skh;
    const half_t* vbase = p.v + b * p.svb + hk * p.svh;
    const int bkv = b * p.Hkv + hk;
    const int8_t* k8base = I8 ? p.k8 + (size_t)bkv * p.Lk_pad * 128 : nullptr;
    const float* ksbase = I8 ? p.ks + (size_t)bkv * p.Lk_pad : nullptr;

    const int tiles = (p.Lk + KB - 1) / KB, half = (tiles + 1) / 2;
    const int t_begin = pair * half, t_end = min(tiles, t_begin + half);
    char* pbuf = smem + pair * Tile<I8>::PAIR;

    u4v rk[I8 ? 4 : 8], rv[8];
    f4 rks = {};
    // Global -> registers -> LDS stage buf, by the 128 threads of this pair, in two halves (K, then V) so
    // that only one half of the next tile is held in registers at a time. Rows past Lk re-read row
    // Lk - 1: their scores are masked to -1e30, so P is 0 there and the (finite) values drop out.
    auto load_k = [&](int key0) {
        if (!I8) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int c = pt + i * PT, key = c >> 4, dc = c & 15;
                rk[i] = *(const u4v*)(kbase + (long)min(key0 + key, p.Lk - 1) * p.skl + dc * 8);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int c = pt + i * PT, key = c >> 3, dc = c & 7;
                rk[i] = *(const u4v*)(k8base + (size_t)(key0 + key) * 128 + dc * 16);
            }
            if (pt < 16) rks = *(const f4*)(ksbase + key0 + pt * 4);
        }
    };
    auto store_k = [&](int buf) {
        char* st = pbuf + buf * TB;
        if (!I8) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int c = pt + i * PT, key = c >> 4, dc = c & 15;
                *(u4v*)(st + key * KP + dc * 16) = rk[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int c = pt + i * PT, key = c >> 3, dc = c & 7;
                *(u4v*)(st + key * K8P + dc * 16) = rk[i];
            }
            if (pt < 16) *(f4*)(st + KB * K8P + pt * 16) = rks;
        }
    };
    // V: unit u = (4-key group kq = u % 16, 8-dim group dq = u / 16), two units per thread.
    auto load_v = [&](int key0) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int u = pt + j * PT, kq = u & 15, dq = u >> 4;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int key = min(key0 + kq * 4 + i, p.Lk - 1);
                rv[j * 4 + i] = *(const u4v*)(vbase + (long)key * p.svl + dq * 8);
            }
        }
    };
    auto store_v = [&](int buf) {
        char* vt = pbuf + buf * TB + Tile<I8>::K_BYTES;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int u = pt + j * PT, kq = u & 15, dq = u >> 4;
            const h8 v0 = __builtin_bit_cast(h8, rv[j * 4]), v1 = __builtin_bit_cast(h8, rv[j * 4 + 1]);
            const h8 v2 = __builtin_bit_cast(h8, rv[j * 4 + 2]), v3 = __builtin_bit_cast(h8, rv[j * 4 + 3]);
            char* col = vt + vt_pos(kq);
#pragma unroll
            for (int e = 0; e < 8; e++) *(h4v*)(col + (dq * 8 + e) * VP) = (h4v){v0[e], v1[e], v2[e], v3[e]};
        }
    };

    if (t_begin < t_end) {
        load_k(t_begin * KB);
        store_k(0);
        load_v(t_begin * KB);
        store_v(0);
    }
    __syncthreads();
    // Both pairs run the same number of iterations (the second may have one tile fewer) so that
    // every wave reaches every barrier.
    for (int it = 0; it < half; it++) {
        const int tile = t_begin + it;
        const bool active = tile < t_end, next = active && tile + 1 < t_end;
        const int buf = it & 1, key0 = tile * KB;
        if (active) {
            if (next) load_k(key0 + KB);
            __builtin_amdgcn_sched_barrier(0);
            const char* st = pbuf + buf * TB;
            float s[2][2][16];  // [qb][kb][r]
            if (!I8) {
#pragma unroll
                for (int kb = 0; kb < 2; kb++) {
                    f16v acc[2] = {};
#pragma unroll
                    for (int ks = 0; ks < 8; ks++) {
                        const h8 a = *(const h8*)(st + (kb * 32 + lq) * KP + ks * 32 + g * 16);
                        acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[0][ks], acc[0], 0, 0, 0);
                        acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[1][ks], acc[1], 0, 0, 0);
                    }
#pragma unroll
                    for (int qb = 0; qb < 2; qb++)
#pragma unroll
                        for (int r = 0; r < 16; r++) s[qb][kb][r] = acc[qb][r];
                }
            } else {
                const float* kscale = (const float*)(st + KB * K8P);
#pragma unroll
                for (int kb = 0; kb < 2; kb++) {
                    i16v acc[2] = {};
#pragma unroll
                    for (int ks = 0; ks < 4; ks++) {
                        const i4v a = *(const i4v*)(st + (kb * 32 + lq) * K8P + ks * 32 + g * 16);
                        acc[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, q8f[0][ks], acc[0], 0, 0, 0);
                        acc[1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, q8f[1][ks], acc[1], 0, 0, 0);
                    }
#pragma unroll
                    for (int r4 = 0; r4 < 4; r4++) {
                        const f4 sc = *(const f4*)(kscale + kb * 32 + 8 * r4 + 4 * g);
#pragma unroll
                        for (int qb = 0; qb < 2; qb++)
#pragma unroll
                            for (int e = 0; e < 4; e++)
                                s[qb][kb][r4 * 4 + e] = (float)acc[qb][r4 * 4 + e] * score_scale[qb] * sc[e];  // hip_attention.hip:227
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            if (next) store_k(buf ^ 1);
            // Keys past Lk (hip_attention.hip:324-328).
            if (key0 + KB > p.Lk) {
#pragma unroll
                for (int kb = 0; kb < 2; kb++)
#pragma unroll
                    for (int r = 0; r < 16; r++)
                        if (key0 + kb * 32 + 8 * (r >> 2) + 4 * g + (r & 3) >= p.Lk) {
                            s[0][kb][r] = -1e30f;
                            s[1][kb][r] = -1e30f;
                        }
            }
            float mx[2];
#pragma unroll
            for (int qb = 0; qb < 2; qb++) {
                float v = s[qb][0][0];
#pragma unroll
                for (int kb = 0; kb < 2; kb++)
#pragma unroll
                    for (int r = 0; r < 16; r++) v = fmaxf(v, s[qb][kb][r]);
                v = fmaxf(v, __shfl_xor(v, 32, 64));
                mx[qb] = I8 ? v : v * p.scale_log2;
            }
            if (__any(mx[0] > m[0] + 8.f || mx[1] > m[1] + 8.f)) {
#pragma unroll
                for (int qb = 0; qb < 2; qb++) {
                    const float mn = fmaxf(m[qb], mx[qb]), alpha = __builtin_amdgcn_exp2f(m[qb] - mn);
                    m[qb] = mn;
                    l[qb] *= alpha;
#pragma unroll
                    for (int i = 0; i < 4; i++) o[qb][i] *= alpha;
                }
            }
            // P, packed for the four 16-key steps: step j holds registers 8 (j % 2) .. +8 of block j / 2.
            h8 pf[2][4];
#pragma unroll
            for (int qb = 0; qb < 2; qb++)
#pragma unroll
                for (int kb = 0; kb < 2; kb++)
#pragma unroll
                    for (int r = 0; r < 16; r += 2) {
                        const float e0 = I8 ? __builtin_amdgcn_exp2f(s[qb][kb][r] - m[qb]) : __builtin_amdgcn_exp2f(__builtin_fmaf(s[qb][kb][r], p.scale_log2, -m[qb]));
                        const float e1 = I8 ? __builtin_amdgcn_exp2f(s[qb][kb][r + 1] - m[qb])
                                            : __builtin_amdgcn_exp2f(__builtin_fmaf(s[qb][kb][r + 1], p.scale_log2, -m[qb]));
                        l[qb] += e0 + e1;
                        const h2 pk = __builtin_convertvector((f2){e0, e1}, h2);
                        pf[qb][kb * 2 + (r >> 3)][r & 7] = pk[0];
                        pf[qb][kb * 2 + (r >> 3)][(r & 7) + 1] = pk[1];
                    }

            __builtin_amdgcn_sched_barrier(0);
            if (next) load_v(key0 + KB);
            // O^T += V^T P^T.
            const char* vt = st + Tile<I8>::K_BYTES;
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int dt = 0; dt < 4; dt++) {
                    const h8 a = *(const h8*)(vt + (dt * 32 + lq) * VP + j * 32 + g * 16);
                    o[0][dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pf[0][j], o[0][dt], 0, 0, 0);
                    o[1][dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pf[1][j], o[1][dt], 0, 0, 0);
                }
            if (next) store_v(buf ^ 1);
        }
        __syncthreads();
    }

    // Merge the second pair's (m, l, O) into the first pair's, then normalise and store.
    float* mb = (float*)smem + (wq * 64 + lane) * 132;
    if (pair == 1) {
#pragma unroll
        for (int qb = 0; qb < 2; qb++) {
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
#pragma unroll
                for (int r = 0; r < 16; r += 4) *(f4*)(mb + qb * 64 + dt * 16 + r) = (f4){o[qb][dt][r], o[qb][dt][r + 1], o[qb][dt][r + 2], o[qb][dt][r + 3]};
            mb[128 + qb * 2] = m[qb];
            mb[129 + qb * 2] = l[qb];
        }
    }
    __syncthreads();
    if (pair == 1) return;
#pragma unroll
    for (int qb = 0; qb < 2; qb++) {
        const float m1 = mb[128 + qb * 2], l1 = mb[129 + qb * 2];
        const float mn = fmaxf(m[qb], m1), a0 = __builtin_amdgcn_exp2f(m[qb] - mn), a1 = __builtin_amdgcn_exp2f(m1 - mn);
        const float lsum = l[qb] * a0 + l1 * a1;
        const float inv = 1.f / (lsum + __shfl_xor(lsum, 32, 64));  // the lane halves hold disjoint keys of one row
        const int row = q0 + qb * 32 + lq;
        half_t* op = p.o + b * p.sob + h * p.soh + (long)row * p.sol;
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int r4 = 0; r4 < 4; r4++) {
                const f4 o1 = *(const f4*)(mb + qb * 64 + dt * 16 + r4 * 4);
                h4v w;
#pragma unroll
                for (int e = 0; e < 4; e++) w[e] = to_half((o[qb][dt][r4 * 4 + e] * a0 + o1[e] * a1) * inv);
                if (row < p.Lq) *(h4v*)(op + dt * 32 + 8 * r4 + 4 * g) = w;
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
    *(u2v*)(K8 + ((size_t)bkv * Lk_pad + key) * 128 + sub * 8) = w;
    if (sub == 0) Ks[(size_t)bkv * Lk_pad + key] = scale;
}

static AttnArgs make_args(const void* q, const void* k, const void* v, void* out, int B, int H, int Hkv, int Lq, int Lk, const long* st, float scale) {
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
    a.qblocks = (Lq + QB - 1) / QB;
    a.nblocks = a.qblocks * B * H;
    a.sqb = st[0]; a.sqh = st[1]; a.sql = st[2];
    a.skb = st[3]; a.skh = st[4]; a.skl = st[5];
    a.svb = st[6]; a.svh = st[7]; a.svl = st[8];
    a.sob = st[9]; a.soh = st[10]; a.sol = st[11];
    a.scale_log2 = scale * 1.4426950408889634f;
    return a;
}

template <bool I8>
static int launch_attn(const AttnArgs& a, void* stream) {
    const size_t lds = Tile<I8>::LDS;
    static bool configured = false;
    if (!configured) {
        const hipError_t e = hipFuncSetAttribute((const void*)attn_kernel<I8>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return (int)e;
        configured = true;
    }
    hipLaunchKernelGGL(attn_kernel<I8>, dim3(a.nblocks), dim3(AT), lds, (hipStream_t)stream, a);
    return (int)hipGetLastError();
}

static bool attn_shapes_ok(int B, int H, int Hkv, int Lq, int Lk) {
    return B > 0 && H > 0 && Hkv > 0 && H % Hkv == 0 && Lq > 0 && Lk > 0 && (long)B * H * ((Lq + QB - 1) / QB) < (1L << 31);
}

extern "C" {

size_t rda_attn_i8_workspace(int B, int Hkv, int Lk) {
    const size_t pad = (size_t)(Lk + KB - 1) / KB * KB;
    return (size_t)B * Hkv * pad * 128 + (size_t)B * Hkv * pad * 4;
}

int rda_attn(const void* q, const void* k, const void* v, void* out, int B, int H, int Hkv, int Lq, int Lk, const long* strides, float scale,
             void* stream) {
    if (!attn_shapes_ok(B, H, Hkv, Lq, Lk)) return RDA_ERR_INVALID;
    return launch_attn<false>(make_args(q, k, v, out, B, H, Hkv, Lq, Lk, strides, scale), stream);
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
    AttnArgs a = make_args(q, nullptr, v, out, B, H, Hkv, Lq, Lk, strides, scale);
    a.k8 = (const int8_t*)workspace;
    a.ks = (const float*)(a.k8 + (size_t)B * Hkv * a.Lk_pad * 128);
    return launch_attn<true>(a, stream);
}

}  // extern "C"
