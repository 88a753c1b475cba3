// Fused attention for head dim 128 on CDNA4 matrix cores: fp16 Q/K/V, fp32 accumulation,
// log2-domain online softmax, fp16 P for the PV product, fp16 output. The int8-QK variant
// quantizes Q per row inside the kernel and reads K quantized per key by pack_k_i8.
//
// Arithmetic follows attn / attn_i8 (hip_attention.hip:160-373): scores s in fp32; the running
// maximum m only moves when some row's block maximum exceeds m + 8 (the lazy rescale,
// hip_attention.hip:333-340; applied to the whole wave when any of its rows needs it); p =
// exp2(s * scale_log2 - m) (int8: s = the int32 score times the key's scale, and the row factor q_scale *
// scale_log2 multiplies it in the same FMA); P is rounded to fp16
// before PV and l sums those fp16 values (in fp32, by v_dot2 with ones, which halves the adds;
// the reference sums the fp32 p); out = fp16(o * (1 / l)). The block maximum is only computed
// when a tile's P, made first with the current m, shows that a row may need the rescale (see
// settle below): the outcome is the same as computing it for every tile.
//
// Work split. Each wave owns 32 query rows and walks the whole key range, keeping Q, O, l and m for
// its rows in registers (<= 168 VGPRs, three waves per SIMD). When every head has at least 384 query
// rows, a workgroup is twelve waves over 384 consecutive rows of the rows flattened over (batch,
// head, row), each head's padded to a multiple of 32, one workgroup per CU: the attention configuration (24 heads x
// 4096 rows) is 256 workgroups, one round, and each K/V tile is copied once for twelve waves rather
// than once per four (copies measured at ~8% of the kernel). A workgroup's rows then lie in one head
// or two; with two it keeps a second set of tiles, copied by waves 8-11 (waves 0-7 copy the first),
// and each wave reads the set of its own head. Otherwise a workgroup is four waves over 128 rows of
// one head, three to a CU. Block ids are remapped so that the workgroups an XCD runs together cover
// a contiguous range of heads and share their K/V through that XCD's L2.
//
// Tiles. Each workgroup keeps 32-key tiles of K and V (one or two sets) in three LDS stages. They are copied by
// direct global->LDS loads (global_load_lds_dwordx4: lane i of a wave writes the 16 bytes at LDS
// base + 16 i), issued one step ahead, so no register holds a tile in flight and the load
// latency hides behind a full step of work; the s_waitcnt before each step's closing barrier is
// where the copies are awaited. The loop is software-pipelined: step i computes the scores of
// tile i + 1 with exponentials of tile i between those products, then tile i's PV product with
// exponentials of tile i + 1 between its products (fp16: half of a tile's exponentials in each
// phase; int8: all beside the score products) -- so tiles i and i + 1 are read while tile i + 2
// arrives. Vector work issues beside the matrix products of the same SIMD, but not for free: a
// phase with a 6-instruction part beside every product slows its products down (the step
// schedule below). Both tiles are row-major, 256 bytes per key
// (int8 K: 128), with the 16-byte chunks of a row permuted by an XOR swizzle so that the
// reads below hit distinct banks: K chunk c of key r sits at c ^ (r & 15) (int8: c ^ (r & 7)),
// V chunk c at c ^ 4 (r & 3).
//
// Products. Scores are computed transposed, S^T = K Q^T (32x32x16 fp16 MFMA; 32x32x32 int8 for
// int8-QK), so the accumulator registers of a lane all belong to its own query row (lane % 32)
// and the row statistics need one exchange with lane ^ 32 (v_permlane32_swap). O^T = V^T P^T
// then takes P straight from those registers: in a 32x32 block lane l supplies row l % 32 of
// the A operand and column l % 32 of B, k-half l / 32, and receives C[8 (r / 4) + 4 (l / 32) +
// r % 4][l % 32] in register r. A lane's P operand for a 16-key step therefore holds keys
// 4 g + {0-3, 8-11} (g = l / 32); the V^T operand is gathered in the same order from the
// row-major V tile by two ds_read_b64_tr_b16, which hand lane i of each 16-lane group element
// i % 4 of the 8-byte read of lane 4 e + i / 4 as its element e.
#include "common.h"

#define QB 128         // query rows of a four-wave workgroup (32 per wave)
#define FLAT_ROWS 384  // query rows of a twelve-wave workgroup
#define KB 32          // keys per tile

struct AttnArgs {
    const half_t* q;
    const half_t* k;
    const half_t* v;
    half_t* o;
    const int8_t* k8;  // int8 K [B * Hkv][Lk_pad][128]
    const float* ks;   // per-key scales [B * Hkv][Lk_pad]
    int H, Hkv, Lq, Lk, Lk_pad, qblocks, nblocks;
    int Lq_pad;  // Lq rounded up to 32: the rows of a head in the flattened range
    long rows;   // B H Lq_pad, the query rows flattened over (batch, head, row)
    long sqb, sqh, sql, skb, skh, skl, svb, svh, svl, sob, soh, sol;
    float scale_log2;
};

template <bool I8>
struct Tile {
    static constexpr int K_ROW = I8 ? 128 : 256;
    static constexpr int SC_BYTES = I8 ? 256 : 0;  // int8 per-key scales: one 256-byte copy, KB floats used
    static constexpr int K_BYTES = KB * K_ROW + SC_BYTES;
    static constexpr int V_BYTES = KB * 256;
    static constexpr int BYTES = K_BYTES + V_BYTES;  // one tile: K, then V
};
// Three stages, each of one tile (four waves) or of two, one per head among the workgroup's rows (twelve waves).
template <bool I8, int NWV>
constexpr int attn_lds() { return 3 * (NWV == 12 ? 2 : 1) * Tile<I8>::BYTES; }

typedef __fp16 fp16x4_t __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef __attribute__((address_space(3))) fp16x4_t lds_fp16x4_t;

// LDS reads by 32-bit LDS offset (no generic pointers in the tile loop, so a stage's constant offset folds into the
// instruction's offset field): a 16-byte read, and the transposing 8-byte read (see the header).
typedef __attribute__((address_space(3))) h8 lds_h8_t;
__device__ __forceinline__ h8 lds_h8(u32 addr) { return *(const lds_h8_t*)(size_t)addr; }
__device__ __forceinline__ h4v read_tr(u32 addr) {
    return __builtin_bit_cast(h4v, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_fp16x4_t*)(size_t)addr));
}
// (x of lanes 0-31, x of lanes 32-63) for every lane: the two halves of a query row.
__device__ __forceinline__ f2 halves(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return (f2){__uint_as_float(r[0]), __uint_as_float(r[1])};
}

// The stage after `s` of the three: at compile time for a constant stage, at run time otherwise.
template <int N>
__device__ __forceinline__ constexpr std::integral_constant<int, (N + 1) % 3> next_stage(std::integral_constant<int, N>) { return {}; }
__device__ __forceinline__ int next_stage(int s) { return s == 2 ? 0 : s + 1; }

template <bool I8, int NWV>
__global__ __launch_bounds__(64 * NWV) __attribute__((amdgpu_waves_per_eu(3, 3))) void attn_kernel(AttnArgs p) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    using T = Tile<I8>;
    // LDS: the K tiles of the three stages, then their V tiles (stage s, set c: K at s KS + c K_BYTES, V at
    // VOFF + s VS + c V_BYTES), so that a stage's offset from the K or V base register fits the 16-bit offset field
    // of an LDS read in every stage (with K and V stages interleaved, the third began at 64 KiB and each of its reads
    // took a v_add).
    constexpr int NSET = NWV == 12 ? 2 : 1;
    constexpr int KS = NSET * T::K_BYTES, VS = NSET * T::V_BYTES, VOFF = 3 * KS;
    const int t = threadIdx.x, lane = t & 63, g = lane >> 5, lq = lane & 31;
    const int wq = __builtin_amdgcn_readfirstlane(t >> 6);  // scalar

    // Block remap: consecutive block ids go round-robin to the 8 XCDs; give each XCD a contiguous run
    // of (head, q-block) work so its resident workgroups share K/V through its L2.
    int blk = blockIdx.x;
    if (p.nblocks % 8 == 0) blk = (blk % 8) * (p.nblocks / 8) + blk / 8;
    // The wave's query rows q0 .. q0 + 31 of head h of batch b. Tile set c of the workgroup holds the K/V of batch
    // kvb[c], KV head kvh[c]; the wave reads set `set`. Four waves: one set, 128 rows of one head. Twelve waves: 384
    // consecutive rows of the (batch, head, row) range with each head's rows padded to a multiple of 32 (Lq_pad), i.e.
    // of one head or two (two sets, the second copied only when present); a wave's 32 rows lie in one head, padding
    // rows recompute row Lq - 1 and waves past the last row the last 32 rows, neither stored.
    int b, h, q0, set = 0, kvb[2], kvh[2];
    bool store = true, two = false;
    if constexpr (NWV == 4) {
        const int bh = blk / p.qblocks, qblk = blk % p.qblocks;
        b = bh / p.H;
        h = bh % p.H;
        q0 = qblk * QB + wq * 32;
        kvb[0] = kvb[1] = b;
        kvh[0] = kvh[1] = h / (p.H / p.Hkv);
    } else {
        const long g0 = (long)blk * FLAT_ROWS, gw = g0 + 32 * wq, gc = gw < p.rows ? gw : p.rows - 32;
        store = gw < p.rows;
        const int bh = (int)(gc / p.Lq_pad), bh0 = (int)(g0 / p.Lq_pad), bh1 = (int)((min(g0 + FLAT_ROWS, p.rows) - 1) / p.Lq_pad);
        b = bh / p.H;
        h = bh % p.H;
        q0 = (int)(gc % p.Lq_pad);
        set = bh - bh0;
        two = bh1 != bh0;
        kvb[0] = bh0 / p.H;
        kvh[0] = (bh0 % p.H) / (p.H / p.Hkv);
        kvb[1] = bh1 / p.H;
        kvh[1] = (bh1 % p.H) / (p.H / p.Hkv);
    }

    // Q as the B operand of S^T = K Q^T, for the lane's row q0 + lq.
    h8 qf[8];
    i4v q8f[4];
    float score_scale = p.scale_log2;
    {
        const int qrow = min(q0 + lq, p.Lq - 1);
        const half_t* qp = p.q + b * p.sqb + h * p.sqh + (long)qrow * p.sql;
        if (!I8) {
#pragma unroll
            for (int ks = 0; ks < 8; ks++) {
                qf[ks] = *(const h8*)(qp + ks * 16 + g * 8);
                asm volatile("" : "+v"(qf[ks]));  // the loads complete here, not inside the tile loop
            }
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
            const f2 qh = halves(qmax);
            qmax = fmaxf(qh[0], qh[1]);
            const float q_scale = fmaxf(qmax / 127.f, 1e-30f);  // hip_attention.hip:183
            score_scale = q_scale * p.scale_log2;
            const float q_rcp = 1.f / q_scale;
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
                        x |= (u32)((int)rintf(div_by_scale(f, q_scale, q_rcp)) & 255) << (e * 8);  // f / q_scale, hip_attention.hip:192
                    }
                    w[d] = x;
                }
                q8f[ks] = as_i4(w);
            }
        }
    }

    f16v o[4];
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] = (f16v){};
    float m = -1e30f, l = 0.f;

    // Copy duty: four waves copy the tile together; of twelve, waves 0-7 copy set 0 and waves 8-11 set 1 (if any).
    const int cset = NWV == 12 && wq >= 8 ? 1 : 0, cw = wq - 8 * cset;  // the wave's set and index among its copiers
    const bool copier = cset == 0 || two;
    const half_t* kbase = p.k + kvb[cset] * p.skb + kvh[cset] * p.skh;
    const half_t* vbase = p.v + kvb[cset] * p.svb + kvh[cset] * p.svh;
    const int bkv = kvb[cset] * p.Hkv + kvh[cset];
    const int8_t* k8base = I8 ? p.k8 + (size_t)bkv * p.Lk_pad * 128 : nullptr;
    const float* ksbase = I8 ? p.ks + (size_t)bkv * p.Lk_pad : nullptr;
    const int tiles = (p.Lk + KB - 1) / KB;

    // Copies the tile at key0 into stage st, each copying wave its part: DMA i (< 2) of a wave fills K (and V)
    // rows 16 i + row0 .. +3, row0 = 4 cw + lane / 16; the eight copiers of set 0 among twelve waves take one DMA
    // each, rows row0 .. + 3 (int8 K: one DMA for each of copiers 0-3, rows 8 cw + lane / 8, and copier 0 the
    // scales). Rows past Lk re-read row Lk - 1: their scores are masked to -1e30, so P is 0 there and the (finite)
    // values drop out. int8 K is zero-padded to a whole tile by pack_k_i8. Per-lane byte offsets are fixed; only the
    // tile base moves (the launcher keeps 32 rows of stride inside 2^31 bytes).
    constexpr bool ONE = NWV == 12;  // one K and one V DMA for the copiers of set 0 (two otherwise)
    const bool single = ONE && cset == 0;
    const int row0 = 4 * cw + (lane >> 4);
    const long skl2 = p.skl * 2, svl2 = p.svl * 2;
    const int kc = (lane & 15) ^ (row0 & 15), vc = (lane & 15) ^ ((lane >> 4) << 2);
    const u32 k_off = (u32)(row0 * skl2) + ((u32)kc << 4);
    const u32 v_off = (u32)(row0 * svl2) + ((u32)vc << 4);
    const u32 k8_off = (u32)((8 * cw + (lane >> 3)) * 128) + ((u32)((lane & 7) ^ (lane >> 3)) << 4);
    auto issue = [&](int key0, int stage) {
        if (!copier) return;
        const char* kst = smem + stage * KS + cset * T::K_BYTES;
        const char* vst = smem + VOFF + stage * VS + cset * T::V_BYTES;
        if (I8) {
            if (cw < 4) dma16((const char*)k8base + (size_t)key0 * 128, k8_off, kst + cw * 1024);
            if (cw == 0) dma4(ksbase + key0, (u32)min(lane, KB - 1) * 4, kst + KB * 128);
        }
        const char* kt = (const char*)kbase + key0 * skl2;
        const char* vt = (const char*)vbase + key0 * svl2;
        if (key0 + KB <= p.Lk) {
            if (single) {
                if (!I8) dma16(kt, k_off, kst + cw * 1024);
                dma16(vt, v_off, vst + cw * 1024);
            } else {
                if (!I8) {
#pragma unroll
                    for (int i = 0; i < 2; i++) dma16(kt + i * 16 * skl2, k_off, kst + (4 * i + cw) * 1024);
                }
#pragma unroll
                for (int i = 0; i < 2; i++) dma16(vt + i * 16 * svl2, v_off, vst + (4 * i + cw) * 1024);
            }
        } else {
            // The tile's base stays in SGPRs; the lane's row (clamped to Lk - 1) enters through its 32-bit offset. The
            // lane id is read again here (a volatile read the compiler cannot hoist), so that this branch, taken once,
            // holds no registers across the tile loop.
            u32 ln;
            asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
            const int r0 = 4 * cw + (int)(ln >> 4);
            const u32 kcl = ((ln & 15) ^ (u32)(r0 & 15)) << 4, vcl = ((ln & 15) ^ ((ln >> 4) << 2)) << 4;
#pragma unroll
            for (int i = 0; i < 2; i++) {
                if (single && i > 0) break;
                const int ri = single ? r0 : 16 * i + r0, di = single ? cw : 4 * i + cw;
                const u32 r = (u32)(min(key0 + ri, p.Lk - 1) - key0);
                if (!I8) dma16(kt, r * (u32)skl2 + kcl, kst + di * 1024);
                dma16(vt, r * (u32)svl2 + vcl, vst + di * 1024);
            }
        }
    };

    // LDS offsets of the lane's V^T reads (and int8 K reads) within a stage, fixed for the whole loop: the stage
    // enters as an immediate offset (the loop below is unrolled over the two stages), so the tile loop spends
    // no VALU on them. Kept opaque so that the compiler holds them in VGPRs rather than recomputing them.
    u32 k_rd[4];
    u32 ks_rd = 0;
    if (I8) {
#pragma unroll
        for (int ks = 0; ks < 4; ks++) k_rd[ks] = (u32)(set * T::K_BYTES + lq * 128 + (((2 * ks + g) ^ (lq & 7)) << 4));
        ks_rd = (u32)(set * T::K_BYTES + KB * 128 + 16 * g);
        asm volatile("" : "+v"(ks_rd));
    }
    const u32 smem_u = lds_addr(smem);  // the dynamic LDS base (0: no static LDS), folded into the per-lane offsets below
    // V^T reads: chunk 4 dt + c' of the lane's rows sits at 4 dt ^ vx, so its offset is v_base ^ 64 dt (v_base has
    // zeros in bits 4-7 besides vx << 4: the V region and its tiles start on 256-byte boundaries).
    u32 v_base;
    {
        const int sg = lane & 15;
        const u32 vt = smem_u + (u32)(VOFF + set * T::V_BYTES + (4 * g + (sg >> 2)) * 256 + (sg & 1) * 8);
        const int vx = (2 * ((lane >> 4) & 1) + ((sg & 3) >> 1)) ^ ((sg >> 2) << 2);
        v_base = vt + (u32)(vx << 4);
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
        if (I8) asm volatile("" : "+v"(k_rd[i]));
    asm volatile("" : "+v"(v_base));

    // The fp16 K reads of a lane: row lq of the stage, chunk 2 ks + g at (2 ks + g) ^ (lq & 15) = 2 ks ^ kx, i.e. byte
    // offset 256 lq + ((kx << 4) ^ 32 ks). The dynamic LDS starts at offset 0 (this kernel has no static LDS), so the
    // low eight bits of k_base are kx << 4 and the read for ks is k_base ^ 32 ks: one xor per read from one value.
    u32 k_base = smem_u + (u32)(set * T::K_BYTES + lq * 256) + (u32)(((lane & 15) ^ g) << 4);
    asm volatile("" : "+v"(k_base));

    // S^T of the tile in stage `stage` (a compile-time stage folds into the reads' offset fields; a runtime one is
    // added), scaled for int8, into out. hook(k) runs right after the k-th product is issued (eight fp16 products,
    // four int8 ones): the caller puts the previous tile's exponentials there, which the transcendental unit runs
    // while the matrix cores work on these products.
    // int8: the products of S^T (int32), and a quarter of their scaling -- scores times the per-key scales only; the
    // per-row factor (Q's scale times scale log2 e) enters the exponent's FMA (exps) and the slow path's maximum. The
    // steady steps run the scaling of the next tile's scores beside the PV products, where the vector ALU is idle.
    auto qk_raw = [&](auto stage, i16v& acc, auto&& hook) __attribute__((always_inline)) {
        const u32 st_u = (u32)((int)stage * KS);
        i4v ka[4];
#pragma unroll
        for (int ks = 0; ks < 4; ks++) ka[ks] = *(const i4v*)(smem + st_u + k_rd[ks]);
        __builtin_amdgcn_sched_barrier(0);
        acc = (i16v){};
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(ka[ks], q8f[ks], acc, 0, 0, 0);
            hook(ks);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto scale_part = [&](auto stage, const i16v& acc, float (&out)[16], int r4) __attribute__((always_inline)) {
        const u32 st_u = (u32)((int)stage * KS);
        const f4 sc = *(const f4*)(smem + st_u + ks_rd + 32 * r4);  // the scales of keys 8 r4 + 4 g .. + 3
#pragma unroll
        for (int e = 0; e < 4; e++) out[r4 * 4 + e] = (float)acc[r4 * 4 + e] * sc[e];  // hip_attention.hip:227
    };
    auto qk = [&](auto stage, float (&out)[16], auto&& hook) __attribute__((always_inline)) {
        const u32 st_u = (u32)((int)stage * KS);
        if constexpr (!I8) {
            // K operands of the first 64 dims go out before the products; each operand of the second 64 is read into
            // the registers the matching first-half product has just consumed. The base passes through an empty asm
            // in every tile, so the eight addresses are made where they are read (one xor each) rather than hoisted
            // out of the loop into eight more VGPRs.
            u32 kb = k_base;
            asm volatile("" : "+v"(kb));
            f16v acc = {};
            h8 ka[4];
#pragma unroll
            for (int k4 = 0; k4 < 4; k4++) ka[k4] = lds_h8((kb ^ (u32)(32 * k4)) + st_u);
            __builtin_amdgcn_sched_barrier(0);
            // A wave in this part (products interleaved with the previous tile's exponentials) issues ahead of the
            // waves of its SIMD in their PV products: 201.8 -> 199.9 us, bit-identical (a raised priority over the
            // PV products instead measured 4% slower).
            __builtin_amdgcn_s_setprio(1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int k4 = 0; k4 < 4; k4++) {
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[k4], qf[k4], acc, 0, 0, 0);
                ka[k4] = lds_h8((kb ^ (u32)(32 * (4 + k4))) + st_u);
                hook(k4);
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int k4 = 0; k4 < 4; k4++) {
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[k4], qf[4 + k4], acc, 0, 0, 0);
                hook(4 + k4);
                __builtin_amdgcn_sched_barrier(0);
            }
            __builtin_amdgcn_s_setprio(0);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int r = 0; r < 16; r++) out[r] = acc[r];
        } else {
            i16v acc;
            qk_raw(stage, acc, hook);
#pragma unroll
            for (int r4 = 0; r4 < 4; r4++) scale_part(stage, acc, out, r4);
        }
    };
    auto no_hook = [](int) {};
    // Keys past Lk (hip_attention.hip:324-328): only the last tile can reach past Lk. int8: -inf, since its scores are
    // scaled only in the exponent, by a factor that an all-zero Q row takes down to 1e-30 x scale log2 e.
    auto mask = [&](float (&x)[16], int key0) __attribute__((always_inline)) {
        if (key0 + KB > p.Lk) {
#pragma unroll
            for (int r = 0; r < 16; r++)
                if (key0 + 8 * (r >> 2) + 4 * g + (r & 3) >= p.Lk) x[r] = I8 ? -__builtin_inff() : -1e30f;
        }
    };

    // The online softmax of a tile with scores s: P = exp2(s * scale_log2 - m) (int8: exp2(s * score_scale - m)), rounded to fp16 into
    // pf, and l += the fp16 P (in fp32, by v_dot2 with ones). `exps(k)` does the k-th of eight (int8: four) equal parts.
    float s[16];
    h8 pf[2];  // P, packed for the two 16-key steps: step j holds registers 8 j .. 8 j + 7
    constexpr int PARTS = I8 ? 4 : 8, PER = 16 / PARTS;
    // Part k of the P of scores x into d0 (keys 0-15) and d1 (keys 16-31).
    auto exps_into = [&](const float (&x)[16], int k, h8& d0, h8& d1) __attribute__((always_inline)) {
#pragma unroll
        for (int r = k * PER; r < (k + 1) * PER; r += 2) {
            const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(x[r], I8 ? score_scale : p.scale_log2, -m));
            const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(x[r + 1], I8 ? score_scale : p.scale_log2, -m));
            const h2 pk = __builtin_convertvector((f2){e0, e1}, h2);
            l = __builtin_amdgcn_fdot2(pk, (h2){(_Float16)1.f, (_Float16)1.f}, l, false);  // l sums the fp16 P of PV
            h8& d = r < 8 ? d0 : d1;
            d[r & 7] = pk[0];
            d[(r & 7) + 1] = pk[1];
        }
    };
    auto exps = [&](int k) __attribute__((always_inline)) { exps_into(s, k, pf[0], pf[1]); };
    // fp16: part k (< 4: keys 0-15) of the next tile's P into registers of its own, pinned where it is issued (the
    // empty asm consumes the results: without it the parts placed beside the PV products sink past the step's
    // closing barrier to their first use).
    auto exps_to = [&](const float (&x)[16], int k, h8& d) __attribute__((always_inline)) {
        exps_into(x, k, d, d);
        asm volatile("" : "+v"(d), "+v"(l));
    };
    // The lazy rescale (hip_attention.hip:333-340): m moves only when some row's tile maximum exceeds m + 8. The tile's P
    // is first made with the current m; a row whose maximum exceeds m + 8 has a P of at least ~2^7.8 in one of its two
    // lanes, so a lane sum that grew by no more than 64 (and is not NaN) proves that no row needs the rescale, and the
    // P just made is the one the rule gives. Otherwise (always on the first tile, where m is -1e30 and P overflows,
    // rarely after) the scores are recomputed from the tile still in LDS, the rule is applied to their maxima, and P
    // and l are made again from the old l -- the same values, in the same order, as applying the rule first.
    auto settle = [&](auto stage, int key0, auto last, float l_old) __attribute__((always_inline)) {
        if (__builtin_expect(__any(!(l <= l_old + 64.f)), 0)) {
            qk(stage, s, no_hook);
            if constexpr (decltype(last)::value) mask(s, key0);
            // The maximum reads the products' results through compiler-visible operations: the compiler inserts
            // the wait states a VALU read of an MFMA result needs only for instructions it can see, not inline asm.
            float mx = s[0];
#pragma unroll
            for (int r = 1; r < 16; r++) mx = fmaxf(mx, s[r]);
            const f2 mh = halves(mx);
            mx = fmaxf(mh[0], mh[1]);
            mx *= I8 ? score_scale : p.scale_log2;
            l = l_old;
            if (__any(mx > m + 8.f)) {
                const float mn = fmaxf(m, mx), alpha = __builtin_amdgcn_exp2f(m - mn);
                m = mn;
                l *= alpha;
#pragma unroll
                for (int i = 0; i < 4; i++) o[i] *= alpha;
            }
#pragma unroll
            for (int k = 0; k < PARTS; k++) exps(k);
        }
    };
    // O^T += V^T P^T with the V tile of stage `stage` and P in pf. Each V^T operand of the second 16-key step is read
    // into the registers the matching first-step product has just consumed.
    auto pv = [&](auto stage, auto&& hook, auto&& hook2) __attribute__((always_inline)) {
        const u32 st_u = (u32)((int)stage * VS);
        u32 vb = v_base;
        asm volatile("" : "+v"(vb));
        auto read_v = [&](int j, int dt) __attribute__((always_inline)) {
            const u32 ra = (vb ^ (u32)(64 * dt)) + st_u + 16 * j * 256;
            return __builtin_shufflevector(read_tr(ra), read_tr(ra + 8 * 256), 0, 1, 2, 3, 4, 5, 6, 7);
        };
        h8 va[4];
#pragma unroll
        for (int dt = 0; dt < 4; dt++) va[dt] = read_v(0, dt);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
            o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[dt], pf[0], o[dt], 0, 0, 0);
            va[dt] = read_v(1, dt);
            hook(dt);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
            o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[dt], pf[1], o[dt], 0, 0, 0);
            hook2(dt);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // Tile loop, software-pipelined over three LDS stages. At the start of step i, tiles i and i + 1 are in LDS and
    // s holds tile i's scores (fp16: and tile i's P for keys 0-15). Step i issues the copies of tile i + 2 (into the
    // stage tile i - 1 left), computes tile i + 1's scores with tile i's (remaining) exponentials between the
    // products, settles the rescale, runs tile i's PV product (fp16: with tile i + 1's first exponentials between its
    // products), and awaits tile i + 2 at the barrier closing the step (which also retires every read of tile i's
    // stage before step i + 1 copies into it). Tile t sits in stage (t - tiles + 1) mod 3, so the last tile is in
    // stage 0 and the one before it in stage 2. The steady steps run six to a loop pass -- stages 2, 0, 1 twice,
    // which also returns the scores to the registers they started in (they alternate between two sets) -- after
    // 0-5 steps taken one at a time with the stage at run time. Kinds: 0 = steady; 1 = the step before the last
    // (next tile masked, nothing to copy); 2 = the last.
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    using Steady = std::integral_constant<int, 0>;
    using Penult = std::integral_constant<int, 1>;
    using Last = std::integral_constant<int, 2>;
    // fp16: a tile's exponentials run in two halves, keys 0-15 beside the previous tile's PV products (into registers
    // of their own, since those products still read the previous tile's P) and keys 16-31 beside the next tile's
    // score products, one part of four exponential pairs beside every other product in each phase. With all of them
    // beside the score products (the int8 layout), that phase was vector-ALU bound while the PV phase had almost no
    // vector work: 194.7 -> 188.1 us at B=1, H=24, S=4096, bit-identical, in one process (keys 0-15 beside only the
    // last four PV products, which do not read them, so no second P buffer: 190.1 us). l_old (l before the tile's
    // first half) then carries over from the step before.
    float l_old = 0.f;
    auto step = [&](int i, auto stage, auto kind) __attribute__((always_inline)) {
        constexpr int K = decltype(kind)::value;
        const auto next = next_stage(stage);
        if constexpr (K == 0) issue((i + 2) * KB, (int)next_stage(next));
        if constexpr (I8) l_old = l;
        if constexpr (K != 2) {
            float nxt[16];
            if constexpr (I8) {
                i16v raw;
                qk_raw(next, raw, exps);
                settle(stage, i * KB, std::false_type{}, l_old);
                pv(stage, [&](int dt) { scale_part(next, raw, nxt, dt); }, no_hook);
                if constexpr (K == 1) mask(nxt, (i + 1) * KB);
            } else {
                qk(next, nxt, [&](int k) { if (k & 1) exps(4 + (k >> 1)); });
                if constexpr (K == 1) mask(nxt, (i + 1) * KB);
                settle(stage, i * KB, std::false_type{}, l_old);
                l_old = l;
                h8 pn;
                pv(stage, [&](int dt) { if (dt & 1) exps_to(nxt, dt >> 1, pn); }, [&](int dt) { if (dt & 1) exps_to(nxt, 2 + (dt >> 1), pn); });
                pf[0] = pn;
            }
#pragma unroll
            for (int r = 0; r < 16; r++) s[r] = nxt[r];
        } else {
#pragma unroll
            for (int k = I8 ? 0 : PARTS / 2; k < PARTS; k++) exps(k);
            settle(stage, i * KB, std::true_type{}, l_old);
            pv(stage, no_hook, no_hook);
        }
        if constexpr (K == 0) {
            wait_copies();
            __syncthreads();
        }
    };
    const int first = ((1 - tiles) % 3 + 3) % 3;  // the stage of tile 0
    issue(0, first);
    if (tiles > 1) issue(KB, next_stage(first));
    wait_copies();
    __syncthreads();
    if (tiles == 1) {
        qk(S0{}, s, no_hook);
        mask(s, 0);
        if constexpr (!I8)
#pragma unroll
            for (int k = 0; k < PARTS / 2; k++) exps(k);
        step(0, S0{}, Last{});
    } else {
        qk(first, s, no_hook);
        if constexpr (!I8)
#pragma unroll
            for (int k = 0; k < PARTS / 2; k++) exps(k);
        const int steady = tiles - 2, peel = steady % 6;
        if (peel >= 5) step(peel - 5, S0{}, Steady{});
        if (peel >= 4) step(peel - 4, S1{}, Steady{});
        if (peel >= 3) step(peel - 3, S2{}, Steady{});
        if (peel >= 2) step(peel - 2, S0{}, Steady{});
        if (peel >= 1) step(peel - 1, S1{}, Steady{});
        for (int i = peel; i < steady; i += 6) {
            step(i, S2{}, Steady{});
            step(i + 1, S0{}, Steady{});
            step(i + 2, S1{}, Steady{});
            step(i + 3, S2{}, Steady{});
            step(i + 4, S0{}, Steady{});
            step(i + 5, S1{}, Steady{});
        }
        step(tiles - 2, S2{}, Penult{});
        step(tiles - 1, S0{}, Last{});
    }

    // Normalise and store: the lane halves hold disjoint keys of one row.
    const f2 lh = halves(l);
    const float inv = 1.f / (lh[0] + lh[1]);
    const int row = q0 + lq;
    half_t* op = p.o + b * p.sob + h * p.soh + (long)row * p.sol;
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int r4 = 0; r4 < 4; r4++) {
            h4v w;
#pragma unroll
            for (int e = 0; e < 4; e++) w[e] = to_half(o[dt][r4 * 4 + e] * inv);
            if (store && row < p.Lq) *(h4v*)(op + dt * 32 + 8 * r4 + 4 * g) = w;
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
    mx = row_max16(mx);  // over the key's 16 lanes
    const float scale = fmaxf(mx / 127.f, 1e-30f), rcp = 1.f / scale;
    u2v w;
#pragma unroll
    for (int d = 0; d < 2; d++) {
        u32 x = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) x |= (u32)((int)rintf(div_by_scale(f[d * 4 + i], scale, rcp)) & 255) << (i * 8);  // f / scale
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
    a.Lq_pad = (Lq + 31) / 32 * 32;
    a.rows = (long)B * H * a.Lq_pad;
    a.sqb = st[0]; a.sqh = st[1]; a.sql = st[2];
    a.skb = st[3]; a.skh = st[4]; a.skl = st[5];
    a.svb = st[6]; a.svh = st[7]; a.svl = st[8];
    a.sob = st[9]; a.soh = st[10]; a.sol = st[11];
    a.scale_log2 = scale * 1.4426950408889634f;
    return a;
}

template <bool I8, int NWV>
static int launch_attn_waves(const AttnArgs& a, void* stream) {
    constexpr size_t lds = attn_lds<I8, NWV>();
    static std::atomic<size_t> configured[RDA_MAX_DEVICES];
    if (const int e = ensure_dynamic_lds((const void*)attn_kernel<I8, NWV>, lds, configured)) return e;
    hipLaunchKernelGGL((attn_kernel<I8, NWV>), dim3(a.nblocks), dim3(64 * NWV), lds, (hipStream_t)stream, a);
    return (int)hipGetLastError();
}

// The current device's compute units, read once per device.
static int device_cus(int* cus) {
    static std::atomic<int> known[RDA_MAX_DEVICES];
    int dev = 0;
    if (const hipError_t e = hipGetDevice(&dev)) return (int)e;
    if (dev < 0 || dev >= RDA_MAX_DEVICES) return (int)hipErrorInvalidDevice;
    int n = known[dev].load(std::memory_order_relaxed);
    if (n <= 0) {
        if (const hipError_t e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev)) return (int)e;
        known[dev].store(n, std::memory_order_relaxed);
    }
    *cus = n;
    return 0;
}

// Workgroup layout: twelve waves over 384 rows of the (batch, head, row) range (every head of at least 384 query rows,
// so that a workgroup's rows span at most two heads), or four waves over 128 rows of one head. The twelve-wave grid
// has a third as many workgroups, one per CU: it is the faster one only when it still covers most of the chip. B = 1,
// H = 24, fp16, one process: 1024 rows per head (64 twelve-wave workgroups) 45.2 us twelve-wave against 24.6 us
// four-wave, 2048 (128) 77.7 / 62.4, 2560 (160) 96.0 / 84.5, 2816 (176) 108.6 / 120.1, 3072 (192) 121.1 / 134.7,
// 4096 (256) 193.0 / 199.6; int8-QK alike, and the outputs bit-identical. So twelve waves when their grid covers at
// least two thirds of the CUs. waves: 0 chooses so; 4 or 12 fixes the layout (12 needs Lq >= 384).
template <bool I8>
static int launch_attn(AttnArgs a, int waves, void* stream) {
    const long flat = (a.rows + FLAT_ROWS - 1) / FLAT_ROWS;
    if (waves == 0) {
        int cus = 0;
        if (const int e = device_cus(&cus)) return e;
        waves = a.Lq >= FLAT_ROWS && 3 * flat >= 2L * cus ? 12 : 4;
    }
    if (waves == 12 && a.Lq >= FLAT_ROWS && flat < (1L << 31)) {
        a.nblocks = (int)flat;
        return launch_attn_waves<I8, 12>(a, stream);
    }
    if (waves == 4) return launch_attn_waves<I8, 4>(a, stream);
    return RDA_ERR_INVALID;
}

// Row strides of K and V must keep a tile's 32 rows within 2^31 bytes (the kernel's 32-bit per-lane offsets).
// K and V reach LDS by 16-byte global->LDS copies: their base addresses and their (batch, head, row) strides must
// keep every row 16-byte aligned.
static bool dma_ready(const void* p, long sb, long sh, long sl) { return ((uintptr_t)p & 15) == 0 && sb % 8 == 0 && sh % 8 == 0 && sl % 8 == 0; }

static bool attn_shapes_ok(int B, int H, int Hkv, int Lq, int Lk, const long* st) {
    const bool rows_ok = st[5] >= 0 && st[5] < (1L << 24) && st[8] >= 0 && st[8] < (1L << 24);
    return B > 0 && H > 0 && Hkv > 0 && H % Hkv == 0 && Lq > 0 && Lk > 0 && (long)B * H * ((Lq + QB - 1) / QB) < (1L << 31) && rows_ok;
}

extern "C" {

size_t rda_attn_i8_workspace(int B, int Hkv, int Lk) {
    const size_t pad = (size_t)(Lk + KB - 1) / KB * KB;
    return (size_t)B * Hkv * pad * 128 + (size_t)B * Hkv * pad * 4;
}

int rda_attn_waves(const void* q, const void* k, const void* v, void* out, int B, int H, int Hkv, int Lq, int Lk, const long* strides, float scale,
                   int waves, void* stream) {
    if (!attn_shapes_ok(B, H, Hkv, Lq, Lk, strides)) return RDA_ERR_INVALID;
    if (!dma_ready(k, strides[3], strides[4], strides[5]) || !dma_ready(v, strides[6], strides[7], strides[8])) return RDA_ERR_INVALID;
    return launch_attn<false>(make_args(q, k, v, out, B, H, Hkv, Lq, Lk, strides, scale), waves, stream);
}

int rda_attn(const void* q, const void* k, const void* v, void* out, int B, int H, int Hkv, int Lq, int Lk, const long* strides, float scale,
             void* stream) {
    return rda_attn_waves(q, k, v, out, B, H, Hkv, Lq, Lk, strides, scale, 0, stream);
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

int rda_attn_i8_waves(const void* q, const void* workspace, const void* v, void* out, int B, int H, int Hkv, int Lq, int Lk, const long* strides,
                      float scale, int waves, void* stream) {
    if (!attn_shapes_ok(B, H, Hkv, Lq, Lk, strides)) return RDA_ERR_INVALID;
    if (((uintptr_t)workspace & 15) != 0 || !dma_ready(v, strides[6], strides[7], strides[8])) return RDA_ERR_INVALID;
    AttnArgs a = make_args(q, nullptr, v, out, B, H, Hkv, Lq, Lk, strides, scale);
    a.k8 = (const int8_t*)workspace;
    a.ks = (const float*)(a.k8 + (size_t)B * Hkv * a.Lk_pad * 128);
    return launch_attn<true>(a, waves, stream);
}

int rda_attn_i8(const void* q, const void* workspace, const void* v, void* out, int B, int H, int Hkv, int Lq, int Lk, const long* strides,
                float scale, void* stream) {
    return rda_attn_i8_waves(q, workspace, v, out, B, H, Hkv, Lq, Lk, strides, scale, 0, stream);
}

}  // extern "C"
