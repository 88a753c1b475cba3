// Single-token (decode) kernels: the ConvRot rotation of one activation row, the int8 and bf16
// GEMVs that read the weights straight from their stored form, and split-K GQA attention over a
// fixed-capacity KV cache. One row of activations makes the linears purely HBM-bound: weights
// are streamed once with 16-byte non-temporal loads, the activation row sits in LDS.
#include "common.h"

#define GV_WAVES 4  // waves per block of the bf16 logits GEMV
#define GI_WAVES 8  // waves per block of the int8 GEMV
#define SPLITS 32  // position chunks per (batch, kv head) in attn_decode
#define HEAD 128

// The sum of a value over the wave's 64 lanes, in every lane: DPP steps within each row of 16 lanes, then the lane
// swaps across rows -- no LDS round trip (a butterfly of shuffles would be six ds_bpermute). Every GEMV, fused or not,
// one matrix or several, reduces its lanes with this one order, so their outputs agree bit for bit.
__device__ __forceinline__ float lane_total(float x) { return rows_sum(row_sum16(x)); }
__device__ __forceinline__ float sbyte(u32 w, int i) { return (float)((int)(w << (24 - 8 * i)) >> 24); }

// Position in the GEMVs' LDS copy of x of its f4 number i (values 4i .. 4i + 3), in reading order: the f4 j of lane
// l in step s at (4s + j) * 64 + l, in the half step past the `steps` whole ones at 256 steps + 64 j + l.
__device__ __forceinline__ int gemv_pos(int i, int steps) {
    const int tail = i - steps * 256;
    return tail < 0 ? ((i >> 8) * 4 + (i & 3)) * 64 + ((i & 255) >> 2) : steps * 256 + (tail & 1) * 64 + (tail >> 1);
}

// One H4 step of the rotation on the four values i, i + s, i + 2s, i + 3s (elementwise for f4), in the sum order of
// int8_gemv.hip:41-46, so with its roundings.
template <typename T>
__device__ __forceinline__ void h4_step(T& a, T& b, T& c, T& d) {
    const T sum = a + b + c + d;
    const T na = sum - 2.0f * d, nb = sum - 2.0f * c, nc = sum - 2.0f * b, nd = sum - 2.0f * a;
    a = na;
    b = nb;
    c = nc;
    d = nd;
}

// The H4 step of stride 1 on the four consecutive values of one f4.
__device__ __forceinline__ f4 h4_step1(f4 x) {
    const float sum = x[0] + x[1] + x[2] + x[3];
    return (f4){sum - 2.0f * x[3], sum - 2.0f * x[2], sum - 2.0f * x[1], sum - 2.0f * x[0]};
}

// rotate (int8_gemv.hip:31-52): every group of G = 4^n fp32 values goes through one H4 step per base-4 digit of the
// value index, lowest digit first (strides 1, 4, 16, ... < G; each step with h4_step's sum order), then the factor
// 1 / sqrt(G), exact. A workgroup takes one group. The group is copied into LDS (coalesced), then rotated in passes
// of one base-16 digit: in pass k a thread takes sets of the 16 values that differ only in digit k -- set q holds
// hi 16^(k+1) + j 16^k + lo for j < 16, lo = q mod 16^k, hi = q / 16^k -- and runs both of the digit's H4 steps in
// registers (strides 16^k and 4 16^k: j's low and high base-4 digits); a last base-4 digit alone takes sets of 4.
// Then the group is copied out, scaled. LDS word of value p: p + p / 16, so that the sets of a wave's lanes fall in
// distinct banks in every pass. ceil(n / 2) + 1 barriers per group, against n + 1 for one step per barrier.
__host__ __device__ __forceinline__ int rot_word(int p) { return p + (p >> 4); }

__global__ __launch_bounds__(256) void rotate_group_kernel(const float* __restrict__ x, float* __restrict__ out, int group) {
    extern __shared__ float gs[];
    const float* in = x + (size_t)blockIdx.x * group;
    for (int p = threadIdx.x; p < group; p += 256) gs[rot_word(p)] = in[p];
    __syncthreads();
    const int digits = __builtin_ctz(group) / 2;  // n
    for (int k = 0, span = 1; 2 * k < digits; k++, span *= 16) {
        const int W = 2 * k + 1 < digits ? 16 : 4;  // values per set: two base-4 digits, or the last one alone
        for (int q = threadIdx.x; q < group / W; q += 256) {
            const int lo = q % span, hi = q / span, first = hi * W * span + lo;
            float v[16];
#pragma unroll
            for (int jj = 0; jj < 16; jj++)
                if (jj < W) v[jj] = gs[rot_word(first + jj * span)];
            if (W == 16) {
#pragma unroll
                for (int b = 0; b < 16; b += 4) h4_step(v[b], v[b + 1], v[b + 2], v[b + 3]);  // stride 16^k
#pragma unroll
                for (int m = 0; m < 4; m++) h4_step(v[m], v[m + 4], v[m + 8], v[m + 12]);  // stride 4 16^k
            } else {
                h4_step(v[0], v[1], v[2], v[3]);
            }
#pragma unroll
            for (int jj = 0; jj < 16; jj++)
                if (jj < W) gs[rot_word(first + jj * span)] = v[jj];
        }
        __syncthreads();
    }
    const float norm = 1.0f / sqrtf((float)group);
    float* o = out + (size_t)blockIdx.x * group;
    for (int p = threadIdx.x; p < group; p += 256) o[p] = gs[rot_word(p)] * norm;
}

// The fused ConvRot of the GEMVs' fp32 x (rotate_group_kernel's arithmetic, bit for bit) goes through two LDS layouts of
// one buffer (word = 4 bytes):
// * natural: value v at word nat_word(v) = v + 4 (v >> 4) + 16 (v >> 8) -- a thread's four f4s of 16 consecutive values
//   and the transposed words 256 b + 16 i + p (p = lane & 15, b = 4 consecutive blocks a wave) both fall in distinct
//   banks;
// * reading order: the f4 j of lane l in step s at ro_f4(s, j, l) = (4 s + j) RO_ROW + l + 4 (l >> 4), the half step
//   past the `steps` whole ones as step `steps` with j < 2 and 8 values per lane. RO_ROW is odd, so that a transposed
//   thread set's word writes land in 64 distinct banks, and a product read's 16-lane groups take consecutive f4s.
#define RO_ROW 77
__device__ __forceinline__ int ro_f4(int s, int j, int l) { return (4 * s + j) * RO_ROW + l + 4 * (l >> 4); }
__device__ __forceinline__ int ro_of_value(int v, int steps) {  // the f4 holding value v (a multiple of 4)
    if (v < steps * 1024) return ro_f4(v >> 10, (v >> 2) & 3, (v >> 4) & 63);
    const int t = v - steps * 1024;
    return ro_f4(steps, (t >> 2) & 1, t >> 3);
}
// Bytes of LDS of x in reading order for K values.
static inline size_t ro_lds_bytes(int K) { return (size_t)16 * RO_ROW * (4 * (K / 1024) + (K % 1024 ? 2 : 0)); }
// Bytes of LDS the fused rotation needs for K values: the larger of the two layouts.
static inline size_t rot_lds_bytes(int K) {
    const size_t nat = 4 * ((size_t)K + K / 4 + K / 16), ro = ro_lds_bytes(K);
    return nat > ro ? nat : ro;
}

// The NT threads of the workgroup take x in sets of 16 consecutive values, set q = thread + NT r (r < RS). rot_load
// issues the loads (before the weights'). rot_to_lds runs the H4 steps of strides 1 and 4 on a set's registers, writes
// the sets in natural order, and reads them back transposed -- thread u = q takes the 16 values 256 b + 16 i + p of
// b = u >> 4, p = u & 15 -- for the steps of strides 16 and 64 in registers, and writes the results times
// 1 / sqrt(group) in reading order once every thread has read: three LDS passes, three barriers with the caller's
// (groups of 4 and 16 write their sets in reading order straight away). With rot_out (nonzero in one workgroup) the
// rotated values are also stored there, in natural order. group is 4, 16, 64 or 256: larger groups
// would need LDS steps of their own (rotate_group_kernel then gemv_i8_kernel serve them). The caller waits at a barrier
// before reading xs.
template <int NT, int RS>
__device__ __forceinline__ void rot_load(const float* __restrict__ x, int K, f4 (&v)[RS][4]) {
#pragma unroll
    for (int r = 0; r < RS; r++) {
        const int q = threadIdx.x + NT * r;
        const f4* src = (const f4*)x + 4 * (q < K / 16 ? q : 0);  // sets past K / 16 re-read set 0 and are skipped
#pragma unroll
        for (int j = 0; j < 4; j++) v[r][j] = src[j];
    }
}

template <int NT, int RS>
__device__ __forceinline__ void rot_to_lds(f4 (&v)[RS][4], f4* xs, int K, int group, int steps, float* __restrict__ rot_out) {
    float* xw = (float*)xs;
    const int sets = K / 16;
    const float norm = 1.0f / sqrtf((float)group);
#pragma unroll
    for (int r = 0; r < RS; r++) {
#pragma unroll
        for (int j = 0; j < 4; j++) v[r][j] = h4_step1(v[r][j]);  // stride 1
        if (group >= 16) h4_step(v[r][0], v[r][1], v[r][2], v[r][3]);  // stride 4
    }
    if (group <= 16) {
#pragma unroll
        for (int r = 0; r < RS; r++) {
            const int q = threadIdx.x + NT * r;
            if (q < sets)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const f4 val = v[r][j] * norm;
                    xs[ro_of_value(16 * q + 4 * j, steps)] = val;
                    if (rot_out) ((f4*)rot_out)[4 * q + j] = val;
                }
        }
        return;
    }
#pragma unroll
    for (int r = 0; r < RS; r++) {
        const int q = threadIdx.x + NT * r;
        if (q < sets)
#pragma unroll
            for (int j = 0; j < 4; j++) *(f4*)(xw + 20 * q + 16 * (q >> 4) + 4 * j) = v[r][j];  // nat_word(16 q + 4 j)
    }
    __syncthreads();
    float y[RS][16];
#pragma unroll
    for (int r = 0; r < RS; r++) {
        const int u = threadIdx.x + NT * r;
        if (u < sets) {
            const float* src = xw + 336 * (u >> 4) + (u & 15);  // nat_word(256 b + p + 16 i) = 336 b + p + 20 i
#pragma unroll
            for (int i = 0; i < 16; i++) y[r][i] = src[20 * i];
#pragma unroll
            for (int k = 0; k < 4; k++) h4_step(y[r][4 * k], y[r][4 * k + 1], y[r][4 * k + 2], y[r][4 * k + 3]);  // stride 16
            if (group >= 256)
#pragma unroll
                for (int m = 0; m < 4; m++) h4_step(y[r][m], y[r][m + 4], y[r][m + 8], y[r][m + 12]);  // stride 64
        }
    }
    __syncthreads();  // every transposed read done: the reading order overwrites the buffer
    {
#pragma unroll
        for (int r = 0; r < RS; r++) {
            const int u = threadIdx.x + NT * r, b = u >> 4, p = u & 15;
            if (u < sets) {
                // value 256 b + 16 i + p: in a whole step s = b / 4, lane 16 (b & 3) + i, f4 p / 4, i.e. word
                // 4 ((4 s + p / 4) RO_ROW + 20 (b & 3)) + p % 4 + 4 i; in the half step (b >= 4 steps), lane
                // 32 (b - 4 steps) + 2 i + p / 8, f4 (p / 4) & 1, i.e. word 4 ((4 steps + (p / 4) & 1) RO_ROW
                // + 40 (b - 4 steps) + p / 8) + p % 4 + 8 i + 16 (i / 8). One formula for both (a wave's four
                // blocks lie all in whole steps or all in the half step): word0 + di i + dh (i / 8).
                const bool half = b >= 4 * steps;
                const int word0 = half ? 4 * ((4 * steps + ((p >> 2) & 1)) * RO_ROW + 40 * (b - 4 * steps) + (p >> 3)) + (p & 3)
                                       : 4 * ((4 * (b >> 2) + (p >> 2)) * RO_ROW + 20 * (b & 3)) + (p & 3);
                const int di = half ? 8 : 4, dh = half ? 16 : 0;
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const float val = y[r][i] * norm;
                    xw[word0 + di * i + dh * (i >> 3)] = val;
                    if (rot_out) rot_out[256 * b + 16 * i + p] = val;
                }
            }
        }
    }
}

// out[n] = scale[n] * sum_k w[n, k] x[k] (+ bias[n]) (int8_gemv.hip:54-85). Each wave owns one row
// and reads it in steps of 1024 values (16 per lane), plus a last half step of 512 (8 per lane) when
// TAIL (K % 1024 == 512). x is fp32 or fp16; out has the dtype of x. One row per wave and NW = 8 waves per
// block measured fastest on the decode shapes (K = 4096, N = 1024 .. 12288): more waves in flight per CU
// beat more rows per wave, and larger blocks (which read x fewer times) did not gain. Rotated rows of more
// than 8192 values (without a half step) take NW = 16, so that each thread holds one set of x.
//
// One memory round trip per launch: every load of the kernel is issued at the start, x and the row scale
// first, then the G steps of the row (the host picks G >= K / 1024). Loads complete in issue order, so
// staging x into LDS waits for x alone and the products of a step start as soon as that step's weights
// have arrived (sched_barrier keeps this issue order). No load sits under a branch (branches would make
// the compiler's wait counts assume the fewest loads in flight): steps past K / 1024 re-read an in-bounds
// chunk of the row and are skipped by the products, indices of x past K / 4 re-read x[0 .. 4).
// x sits in LDS in reading order, so that the 64 lanes of a b128 read touch consecutive addresses: the
// f4 j of lane l in step s at (4s + j) * 64 + l, and in the half step at 256 steps + 64 j + l.
// ROT: x (fp32) is first rotated in groups of `group` by the workgroup (rot_to_lds), bit for bit as rotate_group_kernel
// would, so that one launch replaces rotate + GEMV; its loads go out before the weights' as well; in ROT mode
// the LDS copy is in rot_to_lds's padded reading order (ro_f4).
template <int G, bool TAIL, bool XH, bool ROT, int NW>
__global__ __launch_bounds__(NW * 64) void gemv_i8_kernel(const void* __restrict__ xin, const int8_t* __restrict__ w, const float* __restrict__ scale,
                                                                 const float* __restrict__ bias, void* __restrict__ out, int N, int K, int group,
                                                                 float* __restrict__ rot_out) {
    constexpr int XS = ROT ? 1 : (4 * G + (TAIL ? 2 : 0) + NW - 1) / NW;  // float4s of x per thread: K / 4 <= 64 NW XS
    constexpr int RS = (64 * G + (TAIL ? 32 : 0) + NW * 64 - 1) / (NW * 64) < 2 ? 1 : 2;  // ROT: sets of 16 per thread, K <= 16384
    extern __shared__ f4 xs[];
    const int steps = K / 1024;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row = blockIdx.x * NW + wave;
    const bool active = row < N;
    const int8_t* base = w + (size_t)(active ? row : 0) * K;
    typedef typename std::conditional<XH, h4v, f4>::type xv_t;
    xv_t xr[XS];
    f4 xq[RS][4];
    if constexpr (ROT) {
        rot_load<NW * 64, RS>((const float*)xin, K, xq);
    } else {
#pragma unroll
        for (int j = 0; j < XS; j++) {
            const int i = threadIdx.x + j * NW * 64;
            xr[j] = ((const xv_t*)xin)[i < K / 4 ? i : 0];
        }
    }
    const float sc = scale[active ? row : 0];
    __builtin_amdgcn_sched_barrier(0);  // x and the scale go out before the weights
    u4v v[G];
    u2v vt;
#pragma unroll
    for (int g = 0; g < G; g++) {
        v[g] = __builtin_nontemporal_load((const u4v*)(base + min(g * 1024 + lane * 16, K - 16)));
        __builtin_amdgcn_sched_barrier(0);  // step order, the order of the products
    }
    if constexpr (TAIL) vt = __builtin_nontemporal_load((const u2v*)(base + steps * 1024 + lane * 8));
    __builtin_amdgcn_sched_barrier(0);

    if constexpr (ROT) {
        rot_to_lds<NW * 64, RS>(xq, xs, K, group, steps, blockIdx.x == 0 ? rot_out : nullptr);
    } else {
#pragma unroll
        for (int j = 0; j < XS; j++) {
            const int i = threadIdx.x + j * NW * 64;
            if (i < K / 4) {
                f4 x;
                if constexpr (XH) x = (f4){(float)xr[j][0], (float)xr[j][1], (float)xr[j][2], (float)xr[j][3]};
                else x = xr[j];
                xs[gemv_pos(i, steps)] = x;
            }
        }
    }
    __syncthreads();
    if (!active) return;
    float acc = 0.f;
#pragma unroll
    for (int g = 0; g < G; g++) {
        if (g >= steps) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const f4 xv = xs[ROT ? ro_f4(g, j, lane) : (g * 4 + j) * 64 + lane];
#pragma unroll
            for (int i = 0; i < 4; i++) acc = __builtin_fmaf(sbyte(v[g][j], i), xv[i], acc);
        }
    }
    if constexpr (TAIL) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const f4 xv = xs[ROT ? ro_f4(steps, j, lane) : steps * 256 + j * 64 + lane];
#pragma unroll
            for (int i = 0; i < 4; i++) acc = __builtin_fmaf(sbyte(vt[j], i), xv[i], acc);
        }
    }
    float sum = lane_total(acc) * sc;
    if (bias) sum = sum + bias[row];
    if (lane == 0) {
        if (XH) ((half_t*)out)[row] = to_half(sum);
        else ((float*)out)[row] = sum;
    }
}

// The same product with each row split over S waves (split K), for shapes with too few rows to give every CU its
// share of the weight stream (N = 1024: 128 blocks of one row per wave on 256 CUs). Wave w of a block takes row
// blockIdx.x * (GI_WAVES / S) + w / S and the G steps of 1024 values starting at step (w % S) G; its lanes load their
// 16 weights and 16 values of x per step straight into registers (no LDS copy of x: a wave reads only its own K / S
// slice of it). All loads of the wave are issued first, x then weights, in step order. The S partial sums of a row
// meet in LDS and are added in part order by the row's first wave. K == 1024 S G.
// ROT: x (fp32) is rotated in groups of `group` by the whole workgroup into LDS first (rot_to_lds, as in
// gemv_i8_kernel), and each wave reads its slice from there.
template <int S, int G, bool XH, bool ROT>
__global__ __launch_bounds__(GI_WAVES * 64) void gemv_i8_split_kernel(const void* __restrict__ xin, const int8_t* __restrict__ w,
                                                                       const float* __restrict__ scale, const float* __restrict__ bias,
                                                                       void* __restrict__ out, int N, int K, int group, float* __restrict__ rot_out) {
    constexpr int RPB = GI_WAVES / S;  // rows per block
    constexpr int RS = S * G * 64 > GI_WAVES * 64 ? 2 : 1;  // ROT: sets of 16 values per thread (K / 16 = 64 S G <= 1024)
    __shared__ float part_s[GI_WAVES];
    extern __shared__ f4 xs[];  // ROT: the rotated x in reading order (ro_f4)
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row = blockIdx.x * RPB + wave / S, part = wave % S;
    const bool active = row < N;
    const int8_t* base = w + (size_t)(active ? row : 0) * K + part * G * 1024 + lane * 16;
    const int k0 = part * G * 1024 + lane * 16;  // first of the lane's 16 values of x in step 0
    typedef typename std::conditional<XH, h8, f4>::type xv_t;
    constexpr int XV = XH ? 2 : 4;  // vectors of x per step: 16 values
    xv_t xr[ROT ? 1 : G][XV];
    f4 xq[RS][4];
    if constexpr (ROT) {
        rot_load<GI_WAVES * 64, RS>((const float*)xin, K, xq);
    } else {
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int j = 0; j < XV; j++) xr[g][j] = ((const xv_t*)xin)[(k0 + g * 1024) / (16 / XV) + j];
    }
    const float sc = scale[active ? row : 0];
    __builtin_amdgcn_sched_barrier(0);
    u4v v[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
        v[g] = __builtin_nontemporal_load((const u4v*)(base + g * 1024));
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (ROT) {
        rot_to_lds<GI_WAVES * 64, RS>(xq, xs, K, group, K / 1024, blockIdx.x == 0 ? rot_out : nullptr);
        __syncthreads();
    }
    float acc = 0.f;
#pragma unroll
    for (int g = 0; g < G; g++) {
        float xf[16];
        if constexpr (ROT) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const f4 xv = xs[ro_f4(part * G + g, j, lane)];  // values k0 + 1024 g + 4 j .. + 3
#pragma unroll
                for (int e = 0; e < 4; e++) xf[j * 4 + e] = xv[e];
            }
        } else {
#pragma unroll
            for (int j = 0; j < XV; j++)
#pragma unroll
                for (int e = 0; e < 16 / XV; e++) xf[j * (16 / XV) + e] = (float)xr[g][j][e];
        }
#pragma unroll
        for (int d = 0; d < 4; d++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc = __builtin_fmaf(sbyte(v[g][d], i), xf[d * 4 + i], acc);
    }
    const float sum = lane_total(acc);
    if (S > 1) {
        if (lane == 0) part_s[wave] = sum;
        __syncthreads();
    }
    if (!active || part != 0 || lane != 0) return;
    float total = sum;
#pragma unroll
    for (int p2 = 1; p2 < S; p2++) total += part_s[wave + p2];
    total *= sc;
    if (bias) total = total + bias[row];
    if (XH) ((half_t*)out)[row] = to_half(total);
    else ((float*)out)[row] = total;
}

// Several GEMVs over one input row in one launch: the linears that one parent forward applies to the same activation
// (q, k and v of an attention layer; gate and up of an MLP). Matrix i takes blocks first[i] .. first[i + 1] - 1 and
// splits its K over parts[i] waves per row -- the split gemv_i8_dispatch would choose for it alone -- so that each
// output is the one-matrix launch's, bit for bit: parts 1 is gemv_i8_kernel's arithmetic (one row per wave, every
// step in order, then the wave sum), parts 2 or 4 gemv_i8_split_kernel's (each wave its K / parts slice, the partial
// sums added in part order). x is staged once per workgroup in LDS in rot_to_lds's reading order (ro_f4), rotated
// there first when group is nonzero, and all the block's loads are issued before any arithmetic, x first.
#define MULTI_MAX 4
struct GemvTable {
    const int8_t* w[MULTI_MAX];
    const float* scale[MULTI_MAX];
    const float* bias[MULTI_MAX];
    void* out[MULTI_MAX];
    int n[MULTI_MAX];
    int parts[MULTI_MAX];
    int first[MULTI_MAX + 1];
    int count;
};

// The rows of matrix `mi` in block `blk` of its range, with S waves per row and RW rows per wave (row
// r GI_WAVES / S + wave / S of the block's RW GI_WAVES / S, part wave % S) and GW steps of 1024 per wave at most
// (steps past K / 1024 / S re-read an in-bounds chunk and are skipped). Split matrices take RW = S, so that every
// block holds GI_WAVES rows and each wave G loads, as a one-row-per-wave block does: a block rotates x once for 8
// rows rather than for 8 / S (q|k|v, K = 4096: 1536 -> 768 blocks). XS: float4s (fp16: 4-vectors) of x per thread
// without the rotation; RS: sets of 16 values per thread with it.
template <int GW, int S, int RW, bool TAIL, bool XH, bool ROT, int XS, int RS>
__device__ __forceinline__ void gemv_multi_rows(const void* __restrict__ xin, const GemvTable& t, int mi, int blk, int K, int group,
                                                float* __restrict__ rot_out, f4* xs, float* part_s) {
    constexpr int RPB = GI_WAVES / S * RW;
    const int steps = K / 1024, wsteps = steps / S;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row0 = blk * RPB + wave / S, part = wave % S;
    const int N = t.n[mi];
    auto row_of = [&](int r) { return row0 + r * (GI_WAVES / S); };
    bool active[RW];
    const int8_t* base[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) {
        const int row = row_of(r);
        active[r] = row < N;
        base[r] = t.w[mi] + (size_t)(active[r] ? row : 0) * K + part * wsteps * 1024;
    }
    typedef typename std::conditional<XH, h4v, f4>::type xv_t;
    xv_t xr[XS];
    f4 xq[RS][4];
    if constexpr (ROT) {
        rot_load<GI_WAVES * 64, RS>((const float*)xin, K, xq);
    } else {
#pragma unroll
        for (int j = 0; j < XS; j++) {
            const int i = threadIdx.x + j * GI_WAVES * 64;
            xr[j] = ((const xv_t*)xin)[i < K / 4 ? i : 0];
        }
    }
    float sc[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) sc[r] = t.scale[mi][active[r] ? row_of(r) : 0];
    __builtin_amdgcn_sched_barrier(0);  // x and the scales go out before the weights
    u4v v[RW][GW];
    u2v vt[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) {
#pragma unroll
        for (int g = 0; g < GW; g++) {
            v[r][g] = __builtin_nontemporal_load((const u4v*)(base[r] + (g < wsteps ? g * 1024 + lane * 16 : lane * 16)));
            __builtin_amdgcn_sched_barrier(0);  // row and step order, the order of the products
        }
        if constexpr (TAIL) vt[r] = __builtin_nontemporal_load((const u2v*)(base[r] + steps * 1024 + lane * 8));
    }
    __builtin_amdgcn_sched_barrier(0);

    if constexpr (ROT) {
        rot_to_lds<GI_WAVES * 64, RS>(xq, xs, K, group, steps, blockIdx.x == 0 ? rot_out : nullptr);
    } else {
#pragma unroll
        for (int j = 0; j < XS; j++) {
            const int i = threadIdx.x + j * GI_WAVES * 64;
            if (i < K / 4) {
                f4 x;
                if constexpr (XH) x = (f4){(float)xr[j][0], (float)xr[j][1], (float)xr[j][2], (float)xr[j][3]};
                else x = xr[j];
                xs[ro_of_value(4 * i, steps)] = x;
            }
        }
    }
    __syncthreads();
    float sum[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) {
        float acc = 0.f;
#pragma unroll
        for (int g = 0; g < GW; g++) {
            if (g >= wsteps) continue;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const f4 xv = xs[ro_f4(part * wsteps + g, j, lane)];
#pragma unroll
                for (int i = 0; i < 4; i++) acc = __builtin_fmaf(sbyte(v[r][g][j], i), xv[i], acc);
            }
        }
        if constexpr (TAIL) {
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const f4 xv = xs[ro_f4(steps, j, lane)];
#pragma unroll
                for (int i = 0; i < 4; i++) acc = __builtin_fmaf(sbyte(vt[r][j], i), xv[i], acc);
            }
        }
        sum[r] = lane_total(acc);
    }
    if constexpr (S > 1) {  // each row's parts meet in LDS and are added in part order by its first wave
#pragma unroll
        for (int r = 0; r < RW; r++)
            if (lane == 0) part_s[r * GI_WAVES + wave] = sum[r];
        __syncthreads();
        if (part != 0) return;
#pragma unroll
        for (int r = 0; r < RW; r++)
#pragma unroll
            for (int p2 = 1; p2 < S; p2++) sum[r] += part_s[r * GI_WAVES + wave + p2];
    }
#pragma unroll
    for (int r = 0; r < RW; r++) {
        const int row = row_of(r);
        if (active[r] && lane == 0) {
            float y = sum[r] * sc[r];
            const float* bias = t.bias[mi];
            if (bias) y = y + bias[row];
            if (XH) ((half_t*)t.out[mi])[row] = to_half(y);
            else ((float*)t.out[mi])[row] = y;
        }
    }
}

// G: steps of 1024 values in flight for a one-row-per-wave matrix, >= K / 1024 (4 or 8: K <= 8192). RW: rows per
// wave of the matrices that take one wave per row.
template <int G, int RW, bool TAIL, bool XH, bool ROT>
__global__ __launch_bounds__(GI_WAVES * 64) void gemv_multi_kernel(const void* __restrict__ xin, GemvTable t, int K, int group,
                                                                   float* __restrict__ rot_out) {
    constexpr int XS = ROT ? 1 : (4 * G + (TAIL ? 2 : 0) + GI_WAVES - 1) / GI_WAVES;
    constexpr int RS = (64 * G + (TAIL ? 32 : 0) + GI_WAVES * 64 - 1) / (GI_WAVES * 64) < 2 ? 1 : 2;
    extern __shared__ f4 xs[];
    __shared__ float part_s[4 * GI_WAVES];
    int mi = 0;
#pragma unroll
    for (int i = 1; i < MULTI_MAX; i++)
        if (i < t.count && (int)blockIdx.x >= t.first[i]) mi = i;
    const int blk = blockIdx.x - t.first[mi];
    switch (t.parts[mi]) {  // uniform over the workgroup
    case 4:
        if constexpr (!TAIL && G >= 4) gemv_multi_rows<G / 4, 4, 4, false, XH, ROT, XS, RS>(xin, t, mi, blk, K, group, rot_out, xs, part_s);
        break;
    case 2:
        if constexpr (!TAIL && G >= 2) gemv_multi_rows<G / 2, 2, 2, false, XH, ROT, XS, RS>(xin, t, mi, blk, K, group, rot_out, xs, part_s);
        break;
    default: gemv_multi_rows<G, 1, RW, TAIL, XH, ROT, XS, RS>(xin, t, mi, blk, K, group, rot_out, xs, part_s);
    }
}

// logits[n] = sum_k bf16(w[n, k]) x[k] (int8_gemv.hip:87-119): 8 weights per lane per step of 512, a
// last half step of 256 when K % 512 == 256.
__device__ __forceinline__ float bf16_dot4(u32 a, u32 b, f4 xv, float acc) {
    acc = __builtin_fmaf(__uint_as_float(a << 16), xv[0], acc);
    acc = __builtin_fmaf(__uint_as_float(a & 0xffff0000u), xv[1], acc);
    acc = __builtin_fmaf(__uint_as_float(b << 16), xv[2], acc);
    return __builtin_fmaf(__uint_as_float(b & 0xffff0000u), xv[3], acc);
}

template <int RW>
__global__ __launch_bounds__(GV_WAVES * 64) void gemv_bf16_kernel(const float* __restrict__ x, const u32* __restrict__ w, float* __restrict__ out, int N,
                                                                  int K) {
    extern __shared__ f4 xs[];
    const int steps = K / 512;
    // Reading order: f4 j of lane l in step s at (2s + j) * 64 + l; the half step's f4 of lane l at 128 steps + l.
    for (int i = threadIdx.x; i < K / 4; i += GV_WAVES * 64) {
        const int tail = i - steps * 128;
        xs[tail < 0 ? ((i >> 7) * 2 + (i & 1)) * 64 + ((i & 127) >> 1) : steps * 128 + tail] = ((const f4*)x)[i];
    }
    __syncthreads();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row = (blockIdx.x * GV_WAVES + wave) * RW;
    if (row >= N) return;
    float acc[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) acc[r] = 0.f;
    for (int s = 0; s < steps; s++) {
        u4v v[RW];
#pragma unroll
        for (int r = 0; r < RW; r++) v[r] = __builtin_nontemporal_load((const u4v*)(w + ((size_t)(row + r) * K + s * 512 + lane * 8) / 2));
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const f4 xv = xs[(s * 2 + j) * 64 + lane];
#pragma unroll
            for (int r = 0; r < RW; r++) acc[r] = bf16_dot4(v[r][j * 2], v[r][j * 2 + 1], xv, acc[r]);
        }
    }
    if (K % 512) {
        const int k0 = steps * 512 + lane * 4;
#pragma unroll
        for (int r = 0; r < RW; r++) {
            const u2v v = __builtin_nontemporal_load((const u2v*)(w + ((size_t)(row + r) * K + k0) / 2));
            acc[r] = bf16_dot4(v[0], v[1], xs[steps * 128 + lane], acc[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < RW; r++) {
        const float sum = lane_total(acc[r]);
        if (lane == 0) out[row + r] = sum;
    }
}

// attn_decode (int8_gemv.hip:121-180): one new token over the cache, split by position so that a few
// KV heads still fill the GPU. The grid is fixed and the length is read here, so a captured graph
// stays valid as the cache grows. Memory-level parallelism is the point: a wave takes 4 ITS positions at
// once (16 lanes per position, 8 dims per lane), issues all their K and V loads (non-temporal: the cache is
// read once per token) before any arithmetic, then folds the scores of each query head into its running
// (max, sum, acc) with one rescale per half. The REP query heads of the KV head share every load.
// Per REP, as measured (decode + merge, graph-replayed, B = 1, 2048 positions): one query head per KV head
// takes eight waves of 8 positions (9.9 -> 8.0 us), the others four waves of 16; the q.k and p.v products are
// FMA chains up to four heads (REP 2: 10.7 -> 8.6 us, REP 4: 10.1 -> 9.4 us) and separate multiplies and adds
// at eight (13.5 -> 13.0 us; with FMA chains, 13.5: more registers than the rescale schedule keeps).
template <int REP>
struct DecodeShape {
    static constexpr int W = REP == 1 ? 8 : 4, ITS = REP == 1 ? 2 : 4;  // waves; 4-position steps per round
    static constexpr bool FMA = REP <= 4;
};
template <int REP>
__global__ __launch_bounds__(DecodeShape<REP>::W * 64) void attn_decode_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                                              const float* __restrict__ v, const int* __restrict__ lengths,
                                                                              float* __restrict__ partial, float* __restrict__ stats, int capacity,
                                                                              int kv_heads, float scale) {
    constexpr int W = DecodeShape<REP>::W, ITS = DecodeShape<REP>::ITS, PW = 4 * ITS;  // positions per wave per round
    constexpr bool FMA = DecodeShape<REP>::FMA;
    __shared__ float acc_s[W][REP][HEAD];
    __shared__ float max_s[W][REP], sum_s[W][REP];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, pos = lane >> 4, sub = lane & 15;
    const int b = blockIdx.y / kv_heads, kv_head = blockIdx.y % kv_heads, split = blockIdx.x;
    const int length = min(max(lengths[b], 0), capacity);  // a length past the cache reads no row beyond it
    const int chunk = (length + SPLITS - 1) / SPLITS;
    const int begin = split * chunk, end = min(begin + chunk, length);
    const int first_head = (b * kv_heads + kv_head) * REP;

    f4 qv[REP][2], acc[REP][2];
    float mx[REP], sum[REP];
#pragma unroll
    for (int g = 0; g < REP; g++) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            qv[g][h] = ((const f4*)(q + (size_t)(first_head + g) * HEAD + sub * 8))[h] * scale;
            acc[g][h] = (f4){0.f, 0.f, 0.f, 0.f};
        }
        mx[g] = -1e30f;
        sum[g] = 0.f;
    }
    for (int base = begin + wave * PW; base < end; base += W * PW) {
        f4 kr[ITS][2], vr[ITS][2];
        bool valid[ITS];
        // Loads in the order the two halves of the round use them (K then V of the first half's steps, then of the
        // second half's), so the first half's arithmetic waits only for its own data and runs while the second half's
        // arrives.
#pragma unroll
        for (int half = 0; half < 2; half++) {
#pragma unroll
            for (int it = half * ITS / 2; it < (half + 1) * ITS / 2; it++) {
                const int j = base + it * 4 + pos;
                valid[it] = j < end;
                const size_t row = ((size_t)(b * capacity + (valid[it] ? j : base)) * kv_heads + kv_head) * HEAD + sub * 8;
                kr[it][0] = __builtin_nontemporal_load((const f4*)(k + row));
                kr[it][1] = __builtin_nontemporal_load((const f4*)(k + row + 4));
            }
#pragma unroll
            for (int it = half * ITS / 2; it < (half + 1) * ITS / 2; it++) {
                const int j = base + it * 4 + pos;
                const size_t row = ((size_t)(b * capacity + (valid[it] ? j : base)) * kv_heads + kv_head) * HEAD + sub * 8;
                vr[it][0] = __builtin_nontemporal_load((const f4*)(v + row));
                vr[it][1] = __builtin_nontemporal_load((const f4*)(v + row + 4));
            }
        }
#pragma unroll
        for (int half = 0; half < 2; half++)
#pragma unroll
            for (int g = 0; g < REP; g++) {
                constexpr int HI = ITS / 2;
                float s[HI];
                float top = -1e30f;
#pragma unroll
                for (int u = 0; u < HI; u++) {
                    const int it = half * HI + u;
                    float x;
                    if constexpr (FMA) {  // two chains of four
                        float e0 = qv[g][0][0] * kr[it][0][0], e1 = qv[g][0][1] * kr[it][0][1];
                        e0 = __builtin_fmaf(qv[g][0][2], kr[it][0][2], e0);
                        e1 = __builtin_fmaf(qv[g][0][3], kr[it][0][3], e1);
                        e0 = __builtin_fmaf(qv[g][1][0], kr[it][1][0], e0);
                        e1 = __builtin_fmaf(qv[g][1][1], kr[it][1][1], e1);
                        e0 = __builtin_fmaf(qv[g][1][2], kr[it][1][2], e0);
                        e1 = __builtin_fmaf(qv[g][1][3], kr[it][1][3], e1);
                        x = row_sum16(e0 + e1);
                    } else {
                        const f4 d = qv[g][0] * kr[it][0] + qv[g][1] * kr[it][1];
                        x = row_sum16((d[0] + d[1]) + (d[2] + d[3]));
                    }
                    s[u] = valid[it] ? x : -1e30f;
                    top = fmaxf(top, s[u]);
                }
                top = rows_max(top);
                const float next = fmaxf(mx[g], top), keep = __expf(mx[g] - next);
                float psum = 0.f;
                f4 a0 = acc[g][0] * keep, a1 = acc[g][1] * keep;
#pragma unroll
                for (int u = 0; u < HI; u++) {
                    const int it = half * HI + u;
                    const float p = valid[it] ? __expf(s[u] - next) : 0.f;
                    psum += p;
                    if constexpr (FMA) {
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            a0[e] = __builtin_fmaf(vr[it][0][e], p, a0[e]);
                            a1[e] = __builtin_fmaf(vr[it][1][e], p, a1[e]);
                        }
                    } else {
                        a0 += vr[it][0] * p;
                        a1 += vr[it][1] * p;
                    }
                }
                psum = rows_sum(psum);
                sum[g] = sum[g] * keep + psum;
                acc[g][0] = a0;
                acc[g][1] = a1;
                mx[g] = next;
            }
    }
    // The four position groups of the wave hold partial sums of the same dims: add them up.
#pragma unroll
    for (int g = 0; g < REP; g++)
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int e = 0; e < 4; e++) acc[g][h][e] = rows_sum(acc[g][h][e]);
#pragma unroll
    for (int g = 0; g < REP; g++) {
        if (pos == 0) {
            ((f4*)acc_s[wave][g])[sub * 2] = acc[g][0];
            ((f4*)acc_s[wave][g])[sub * 2 + 1] = acc[g][1];
        }
        if (lane == 0) {
            max_s[wave][g] = mx[g];
            sum_s[wave][g] = sum[g];
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < REP * HEAD; i += W * 64) {
        const int g = i / HEAD, d = i % HEAD;
        float top = max_s[0][g];
#pragma unroll
        for (int w = 1; w < W; w++) top = fmaxf(top, max_s[w][g]);
        float value = 0.f, total = 0.f;
#pragma unroll
        for (int w = 0; w < W; w++) {
            const float keep = __expf(max_s[w][g] - top);
            value += acc_s[w][g][d] * keep;
            total += sum_s[w][g] * keep;
        }
        const size_t at = (size_t)(first_head + g) * SPLITS + split;
        partial[at * HEAD + d] = value;
        if (d == 0) {
            stats[at * 2] = top;
            stats[at * 2 + 1] = total;
        }
    }
}

// attn_merge (int8_gemv.hip:182-195): joins the splits, one block per query head.
// Every load -- the splits' (max, sum) pairs and the thread's partial of each split -- is issued before any
// arithmetic, so the merge is one memory round trip rather than two.
__global__ __launch_bounds__(HEAD) void attn_merge_kernel(const float* __restrict__ partial, const float* __restrict__ stats, float* __restrict__ out) {
    const size_t head = blockIdx.x;
    const f2* st = (const f2*)(stats + head * SPLITS * 2);
    f2 ms[SPLITS];
    float pv[SPLITS];
#pragma unroll
    for (int s = 0; s < SPLITS; s++) ms[s] = st[s];
#pragma unroll
    for (int s = 0; s < SPLITS; s++) pv[s] = partial[(head * SPLITS + s) * HEAD + threadIdx.x];
    float top = ms[0][0];
#pragma unroll
    for (int s = 1; s < SPLITS; s++) top = fmaxf(top, ms[s][0]);
    float value = 0.f, total = 0.f;
#pragma unroll
    for (int s = 0; s < SPLITS; s++) {
        const float keep = __expf(ms[s][0] - top);
        value += pv[s] * keep;
        total += ms[s][1] * keep;
    }
    out[head * HEAD + threadIdx.x] = value / total;
}

template <int G, bool TAIL, bool XH, bool ROT>
static int launch_gemv(const void* x, const void* w, const float* scale, const float* bias, void* out, int N, int K, int group, float* rot_out, void* stream) {
    // rows past 8192 values with the rotation: 16 waves of one row each, so that a thread holds one set of x and the
    // registers leave a workgroup per CU; with a half step that shape would spill, and keeps 8 waves
    constexpr int NW = ROT && G >= 12 && !TAIL ? 16 : GI_WAVES;
    const size_t lds = ROT ? rot_lds_bytes(K) : (size_t)K * 4;
    if constexpr (ROT) {  // K > 12288: more than 64 KiB
        static std::atomic<size_t> done[RDA_MAX_DEVICES];
        if (const int e = ensure_dynamic_lds((const void*)gemv_i8_kernel<G, TAIL, XH, ROT, NW>, lds, done)) return e;
    }
    hipLaunchKernelGGL((gemv_i8_kernel<G, TAIL, XH, ROT, NW>), dim3((N + NW - 1) / NW), dim3(NW * 64), lds, (hipStream_t)stream, x,
                       (const int8_t*)w, scale, bias, out, N, K, group, rot_out);
    return (int)hipGetLastError();
}

template <int S, int G, bool ROT>
static int launch_gemv_split(const void* x, int x_half, const void* w, const float* scale, const float* bias, void* out, int N, int K, int group, float* rot_out,
                             void* stream) {
    constexpr int RPB = GI_WAVES / S;
    const dim3 grid((N + RPB - 1) / RPB), block(GI_WAVES * 64);
    const size_t lds = ROT ? rot_lds_bytes(K) : 0;
    if (x_half) {
        if constexpr (ROT) return RDA_ERR_INVALID;  // the rotation takes fp32 x only
        else hipLaunchKernelGGL((gemv_i8_split_kernel<S, G, true, false>), grid, block, 0, (hipStream_t)stream, x, (const int8_t*)w, scale, bias, out, N, K, 0, nullptr);
    } else {
        if constexpr (ROT) {  // K > 12288: more than 64 KiB
            static std::atomic<size_t> done[RDA_MAX_DEVICES];
            if (const int e = ensure_dynamic_lds((const void*)gemv_i8_split_kernel<S, G, false, true>, lds, done)) return e;
        }
        hipLaunchKernelGGL((gemv_i8_split_kernel<S, G, false, ROT>), grid, block, lds, (hipStream_t)stream, x, (const int8_t*)w, scale, bias, out, N, K,
                           group, rot_out);
    }
    return (int)hipGetLastError();
}

template <int G, bool ROT>
static int launch_gemv_g(const void* x, int x_half, const void* w, const float* scale, const float* bias, void* out, int N, int K, int group, float* rot_out,
                         void* stream) {
    if constexpr (ROT) {
        if (K % 1024) return launch_gemv<G, true, false, true>(x, w, scale, bias, out, N, K, group, rot_out, stream);
        return launch_gemv<G, false, false, true>(x, w, scale, bias, out, N, K, group, rot_out, stream);
    } else {
        switch ((K % 1024 ? 2 : 0) + (x_half ? 1 : 0)) {
        case 0: return launch_gemv<G, false, false, false>(x, w, scale, bias, out, N, K, 0, nullptr, stream);
        case 1: return launch_gemv<G, false, true, false>(x, w, scale, bias, out, N, K, 0, nullptr, stream);
        case 2: return launch_gemv<G, true, false, false>(x, w, scale, bias, out, N, K, 0, nullptr, stream);
        default: return launch_gemv<G, true, true, false>(x, w, scale, bias, out, N, K, 0, nullptr, stream);
        }
    }
}

// Waves per row of the GEMV of N rows of K values. Up to 2048 rows, split K: 4 waves per row up to 1024 rows, 2 up to
// 2048 (K = 4096: N = 1024 3.56 -> 3.01 us; from 4096 rows on, one row per wave already gives every CU two or more
// blocks and measured as fast or faster), where K / 1024 splits into the per-wave step counts the split kernel is
// built for; 1 otherwise. rda_gemv_i8_multi gives each of its matrices the same split.
static int gemv_parts(int N, int K) {
    if (K % 1024 != 0 || N > 2048) return 1;
    const int steps = K / 1024, S = N <= 1024 ? 4 : 2;
    if (steps % S != 0) return 1;
    const int g = steps / S;
    return g == 1 || g == 2 || g == 4 || (S == 2 && g == 8) ? S : 1;
}

// The GEMV launch of rda_gemv_i8 (ROT false) and rda_rotate_gemv_i8 (ROT true, fp32 x): arguments already checked.
template <bool ROT>
static int gemv_i8_dispatch(const void* x, int x_half, const void* w, const float* scale, const float* bias, void* out, int N, int K, int group, float* rot_out,
                            void* stream) {
    const int steps = K / 1024;
    if (const int S = gemv_parts(N, K); S > 1) {
        switch (S * 100 + steps / S) {
        case 401: return launch_gemv_split<4, 1, ROT>(x, x_half, w, scale, bias, out, N, K, group, rot_out, stream);
        case 402: return launch_gemv_split<4, 2, ROT>(x, x_half, w, scale, bias, out, N, K, group, rot_out, stream);
        case 404: return launch_gemv_split<4, 4, ROT>(x, x_half, w, scale, bias, out, N, K, group, rot_out, stream);
        case 201: return launch_gemv_split<2, 1, ROT>(x, x_half, w, scale, bias, out, N, K, group, rot_out, stream);
        case 202: return launch_gemv_split<2, 2, ROT>(x, x_half, w, scale, bias, out, N, K, group, rot_out, stream);
        case 204: return launch_gemv_split<2, 4, ROT>(x, x_half, w, scale, bias, out, N, K, group, rot_out, stream);
        case 208: return launch_gemv_split<2, 8, ROT>(x, x_half, w, scale, bias, out, N, K, group, rot_out, stream);
        default: return RDA_ERR_INVALID;  // gemv_parts returns only the splits listed here
        }
    }
    // fp16 x up to 4096 rows: one row per wave with the lane's x read straight into registers (the split kernel with
    // one part; K = 4096: N = 4096 5.43 -> 5.32 us, bit-identical; at N = 12288 the LDS copy of x is faster).
    if (!ROT && x_half && N <= 4096 && K % 1024 == 0) {
        switch (steps) {
        case 1: return launch_gemv_split<1, 1, false>(x, x_half, w, scale, bias, out, N, K, 0, nullptr, stream);
        case 2: return launch_gemv_split<1, 2, false>(x, x_half, w, scale, bias, out, N, K, 0, nullptr, stream);
        case 4: return launch_gemv_split<1, 4, false>(x, x_half, w, scale, bias, out, N, K, 0, nullptr, stream);
        default: break;
        }
    }
    // One row per wave. Steps in flight: the first of 4, 8, 12, 16 that covers K / 1024 (steps past it re-read a chunk
    // and are skipped: at K = 12288, 12 instead of 16 measured 13.0 against 13.6-14.6 us with the rotation and
    // 11.4-11.8 against 12.1 us without, N = 4096, bit-identical).
    if (steps <= 4) return launch_gemv_g<4, ROT>(x, x_half, w, scale, bias, out, N, K, group, rot_out, stream);
    if (steps <= 8) return launch_gemv_g<8, ROT>(x, x_half, w, scale, bias, out, N, K, group, rot_out, stream);
    if (steps <= 12) return launch_gemv_g<12, ROT>(x, x_half, w, scale, bias, out, N, K, group, rot_out, stream);
    return launch_gemv_g<16, ROT>(x, x_half, w, scale, bias, out, N, K, group, rot_out, stream);
}

extern "C" {

int rda_rotate(const float* x, float* out, int rows, int group, void* stream) {
    if (rows <= 0 || group < 4 || group > 16384 || (group & (group - 1)) != 0 || (__builtin_ctz(group) & 1)) return RDA_ERR_INVALID;
    const size_t lds = (size_t)rot_word(group) * 4;  // 16384 values: 68 KiB
    static std::atomic<size_t> done[RDA_MAX_DEVICES];
    if (const int e = ensure_dynamic_lds((const void*)rotate_group_kernel, lds, done)) return e;
    hipLaunchKernelGGL(rotate_group_kernel, dim3(rows), dim3(256), lds, (hipStream_t)stream, x, out, group);
    return (int)hipGetLastError();
}

// x_half: 0 for fp32 x and out, 1 for fp16 x and out.
int rda_gemv_i8(const void* x, int x_half, const void* w, const float* scale, const float* bias, void* out, int N, int K, void* stream) {
    if (N <= 0 || K <= 0 || K % 512 != 0 || K > 16384) return RDA_ERR_INVALID;
    if ((uintptr_t)x & 15) return RDA_ERR_INVALID;  // read in 16-byte vectors
    return gemv_i8_dispatch<false>(x, x_half, w, scale, bias, out, N, K, 0, nullptr, stream);
}

// rotate then gemv_i8 in one launch (fp32 x and out): the same outputs, bit for bit, as rda_rotate of x's K / group
// groups followed by rda_gemv_i8 of the result; `rotated` (K floats, or null) receives that rotation as well, written
// by the first workgroup.
int rda_rotate_gemv_i8(const float* x, int group, const void* w, const float* scale, const float* bias, float* out, float* rotated, int N, int K,
                       void* stream) {
    if (N <= 0 || K <= 0 || K % 512 != 0 || K > 16384) return RDA_ERR_INVALID;
    if (group != 4 && group != 16 && group != 64 && group != 256) return RDA_ERR_INVALID;
    if (((uintptr_t)x | (uintptr_t)rotated) & 15) return RDA_ERR_INVALID;  // read and written in 16-byte vectors
    // The first workgroup writes `rotated` while later ones may still be reading x: the two must not overlap.
    if (rotated && (uintptr_t)rotated < (uintptr_t)(x + K) && (uintptr_t)x < (uintptr_t)(rotated + K)) return RDA_ERR_INVALID;
    return gemv_i8_dispatch<true>(x, 0, w, scale, bias, out, N, K, group, rotated, stream);
}

int rda_gemv_i8_multi(const void* x, int x_half, int group, int count, const void* const* w, const float* const* scale, const float* const* bias,
                      void* const* out, const int* n, int K, float* rotated, void* stream) {
    if (count < 1 || count > MULTI_MAX || !w || !scale || !out || !n) return RDA_ERR_INVALID;
    if (K <= 0 || K % 512 != 0 || K > 8192) return RDA_ERR_INVALID;
    if (group != 0 && group != 4 && group != 16 && group != 64 && group != 256) return RDA_ERR_INVALID;
    if ((group != 0 && x_half) || (group == 0 && rotated)) return RDA_ERR_INVALID;  // the rotation takes fp32 x
    if (((uintptr_t)x | (uintptr_t)rotated) & 15) return RDA_ERR_INVALID;  // read and written in 16-byte vectors
    const char *xb = (const char*)x, *rb = (const char*)rotated;
    if (rotated && rb < xb + 4 * (size_t)K && xb < rb + 4 * (size_t)K) return RDA_ERR_INVALID;  // see rda_rotate_gemv_i8
    // Rows per wave of the one-row-per-wave matrices: 4 or 2 where that still leaves >= 768 of their blocks (a block
    // stages and rotates x once for all its rows: gate|up 2 x 12288 rows, K = 4096: 22.4 us at 1, 21.4 at 2, 20.3 at 4),
    // else 1 (q|k|v: 10.7 us at 1, 12.0 at 2; o: 6.5 at 1 or 2, 8.2 at 4).
    long rows1 = 0;
    for (int i = 0; i < count; i++)
        if (gemv_parts(n[i], K) == 1) rows1 += n[i] > 0 ? n[i] : 0;
    const int rw = rows1 >= 768L * GI_WAVES * 4 ? 4 : rows1 >= 768L * GI_WAVES * 2 ? 2 : 1;
    GemvTable t = {};
    t.count = count;
    long blocks = 0;
    for (int i = 0; i < count; i++) {
        if (n[i] <= 0 || !w[i] || !scale[i] || !out[i]) return RDA_ERR_INVALID;
        t.w[i] = (const int8_t*)w[i];
        t.scale[i] = scale[i];
        t.bias[i] = bias ? bias[i] : nullptr;
        t.out[i] = out[i];
        t.n[i] = n[i];
        t.parts[i] = gemv_parts(n[i], K);
        t.first[i] = (int)blocks;
        const int rpb = t.parts[i] > 1 ? GI_WAVES : GI_WAVES * rw;  // split rows: parts rows per wave
        blocks += (n[i] + rpb - 1) / rpb;
        if (blocks > 0x7fffffff) return RDA_ERR_INVALID;
    }
    for (int i = count; i <= MULTI_MAX; i++) t.first[i] = (int)blocks;
    const bool tail = K % 1024 != 0, big = K > 4096;
    const size_t lds = group ? rot_lds_bytes(K) : ro_lds_bytes(K);
    const dim3 grid((unsigned)blocks), block(GI_WAVES * 64);
    hipStream_t st = (hipStream_t)stream;
#define RDA_MULTI(G, T, XH, R)                                                                                                \
    do {                                                                                                                      \
        if (rw == 1) hipLaunchKernelGGL((gemv_multi_kernel<G, 1, T, XH, R>), grid, block, lds, st, x, t, K, group, rotated);  \
        else if (rw == 2) hipLaunchKernelGGL((gemv_multi_kernel<G, 2, T, XH, R>), grid, block, lds, st, x, t, K, group, rotated); \
        else hipLaunchKernelGGL((gemv_multi_kernel<G, 4, T, XH, R>), grid, block, lds, st, x, t, K, group, rotated);          \
    } while (0)
    if (group) {
        if (tail) RDA_MULTI(8, true, false, true);
        else if (big) RDA_MULTI(8, false, false, true);
        else RDA_MULTI(4, false, false, true);
    } else if (x_half) {
        if (tail) RDA_MULTI(8, true, true, false);
        else if (big) RDA_MULTI(8, false, true, false);
        else RDA_MULTI(4, false, true, false);
    } else {
        if (tail) RDA_MULTI(8, true, false, false);
        else if (big) RDA_MULTI(8, false, false, false);
        else RDA_MULTI(4, false, false, false);
    }
#undef RDA_MULTI
    return (int)hipGetLastError();
}

int rda_gemv_bf16(const float* x, const void* w, float* out, int N, int K, void* stream) {
    if (N <= 0 || K <= 0 || K % 256 != 0 || K > 16384 || N % (GV_WAVES * 2) != 0) return RDA_ERR_INVALID;
    hipLaunchKernelGGL(gemv_bf16_kernel<2>, dim3(N / (GV_WAVES * 2)), dim3(GV_WAVES * 64), (size_t)K * 4, (hipStream_t)stream, x, (const u32*)w, out, N,
                       K);
    return (int)hipGetLastError();
}

int rda_attn_decode(const float* q, const float* k, const float* v, const int* lengths, float* partial, float* stats, int B, int H, int Hkv,
                    int capacity, float scale, void* stream) {
    if (B <= 0 || Hkv <= 0 || H % Hkv != 0 || capacity <= 0) return RDA_ERR_INVALID;
    const int rep = H / Hkv;
    dim3 grid(SPLITS, B * Hkv);
    switch (rep) {
    case 1: hipLaunchKernelGGL(attn_decode_kernel<1>, grid, dim3(DecodeShape<1>::W * 64), 0, (hipStream_t)stream, q, k, v, lengths, partial, stats, capacity, Hkv, scale); break;
    case 2: hipLaunchKernelGGL(attn_decode_kernel<2>, grid, dim3(DecodeShape<2>::W * 64), 0, (hipStream_t)stream, q, k, v, lengths, partial, stats, capacity, Hkv, scale); break;
    case 4: hipLaunchKernelGGL(attn_decode_kernel<4>, grid, dim3(DecodeShape<4>::W * 64), 0, (hipStream_t)stream, q, k, v, lengths, partial, stats, capacity, Hkv, scale); break;
    case 8: hipLaunchKernelGGL(attn_decode_kernel<8>, grid, dim3(DecodeShape<8>::W * 64), 0, (hipStream_t)stream, q, k, v, lengths, partial, stats, capacity, Hkv, scale); break;
    default: return RDA_ERR_INVALID;
    }
    return (int)hipGetLastError();
}

int rda_attn_merge(const float* partial, const float* stats, float* out, int heads, void* stream) {
    if (heads <= 0) return RDA_ERR_INVALID;
    hipLaunchKernelGGL(attn_merge_kernel, dim3(heads), dim3(HEAD), 0, (hipStream_t)stream, partial, stats, out);
    return (int)hipGetLastError();
}

int rda_decode_splits(void) { return SPLITS; }

}  // extern "C"

// ---------------------------------------------------------------- decode attention without allocation
// For callers that cannot allocate device memory (code under HIP graph capture, tight serving loops): the split
// partials and statistics of rda_attn_decode live in `scratch`, a file-scope device array sized for
// NOALLOC_MAX_HEADS query heads (256 x 32 splits x (128 + 2) floats = 4.06 MiB), which every GPU the library runs
// on holds until the process ends. In host code `scratch` only names the symbol: its device address on the current
// GPU comes from hipGetSymbolAddress, once per device, and only that address is passed to the kernels. attn_decode
// writes every (head, split) slot of the partials and statistics it reads back, so nothing needs clearing between
// calls; calls that overlap on one GPU share the array and race.
#define NOALLOC_MAX_HEADS 256
static __device__ __align__(256) float scratch[NOALLOC_MAX_HEADS * SPLITS * (HEAD + 2)];
static std::atomic<float*> scratch_on[RDA_MAX_DEVICES];

// The device address of `scratch` on the current GPU (looked up on the first call for that GPU).
static int scratch_address(float** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= RDA_MAX_DEVICES) return (int)hipErrorInvalidDevice;
    float* p = scratch_on[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        void* addr = nullptr;
        e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        if (addr == nullptr) return (int)hipErrorInvalidSymbol;
        p = (float*)addr;
        scratch_on[dev].store(p, std::memory_order_release);
    }
    *out = p;
    return 0;
}

extern "C" int rda_attention_decode_noalloc(const float* q, const float* k, const float* v, const int* lengths, float* out, int B, int H, int Hkv,
                                            int capacity, float scale, void* stream) {
    if (B <= 0 || H <= 0 || (long)B * H > NOALLOC_MAX_HEADS) return RDA_ERR_INVALID;
    float* base = nullptr;
    if (const int e = scratch_address(&base)) return e;
    float* partial = base;                                              // (B H, SPLITS, HEAD)
    float* stats = base + (size_t)NOALLOC_MAX_HEADS * SPLITS * HEAD;    // (B H, SPLITS, 2)
    if (const int e = rda_attn_decode(q, k, v, lengths, partial, stats, B, H, Hkv, capacity, scale, stream)) return e;
    return rda_attn_merge(partial, stats, out, B * H, stream);
}
