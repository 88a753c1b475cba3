// Shared device helpers for the gfx950 (CDNA4, wave64) kernels.
//
// All sources are compiled with -ffp-contract=off: a multiply and an add stay two
// IEEE operations unless the code calls __builtin_fmaf, so every rounding point
// is explicit and the CPU oracle can restate it bit for bit. fp32 division and
// square root are correctly rounded (hipcc's default), and fp32 denormals are kept.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 half_t;
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4v __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef int i4v __attribute__((ext_vector_type(4)));
typedef int i16v __attribute__((ext_vector_type(16)));
typedef unsigned u32;
typedef u32 u2v __attribute__((ext_vector_type(2)));
typedef u32 u4v __attribute__((ext_vector_type(4)));

#define RDA_ERR_INVALID 1  // hipErrorInvalidValue

#include <atomic>

#define RDA_MAX_DEVICES 64
// Raises kernel `fn`'s dynamic-LDS limit to at least `bytes` on the current device, once per device and size:
// `done` is the caller's record for that kernel (bytes configured per device; atomics, so that threads launching
// at the same time at most repeat the call). Returns a hipError_t.
static inline int ensure_dynamic_lds(const void* fn, size_t bytes, std::atomic<size_t> (&done)[RDA_MAX_DEVICES]) {
    int dev = 0;
    const hipError_t g = hipGetDevice(&dev);
    if (g != hipSuccess) return (int)g;
    if (dev < 0 || dev >= RDA_MAX_DEVICES) return (int)hipErrorInvalidDevice;
    if (done[dev].load(std::memory_order_relaxed) >= bytes) return 0;
    const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e != hipSuccess) return (int)e;
    size_t prev = done[dev].load(std::memory_order_relaxed);
    while (prev < bytes && !done[dev].compare_exchange_weak(prev, bytes, std::memory_order_relaxed)) {
    }
    return 0;
}

// fp32 -> fp16 (RNE) of a value that has been rounded to fp32 first. Without the register barrier the compiler
// folds a preceding fp32 multiply or FMA into v_fma_mixlo_f16, which rounds the exact product once, straight to
// fp16; every rounding point in these kernels is "round to fp32, then to fp16", as the arithmetic is written.
__device__ __forceinline__ half_t to_half(float x) {
    asm("" : "+v"(x));  // not volatile: the scheduler may still interleave independent conversions
    return (half_t)x;
}
// Rounds an fp32 value to fp16 and back.
__device__ __forceinline__ float r16(float x) { return (float)to_half(x); }

// exp(x): 2^n e^r with n = rint(x log2 e), r = x - n ln2 by a two-constant
// Cody-Waite reduction, e^r by a degree-7 Taylor polynomial in Horner form, and
// 2^n as two exact power-of-two factors. Below -88 it returns 0 (1 + e^x == 1
// there), above ln(FLT_MAX) +inf. Every step is an IEEE fp32 operation, so the
// CPU restatement reproduces it exactly.
__device__ __forceinline__ float pow2i(int n) { return __int_as_float((n + 127) << 23); }
__device__ __forceinline__ float scale2(float p, int n) {
    const int h = n / 2;
    return (p * pow2i(h)) * pow2i(n - h);
}
__device__ __forceinline__ float rda_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return __builtin_inff();
    if (x < -88.0f) return 0.0f;
    const float n = rintf(x * 1.44269504088896341f);
    float r = __builtin_fmaf(-n, 0.693145751953125f, x);
    r = __builtin_fmaf(-n, 1.42860682030941723e-6f, r);
    float p = 1.98412701138295233e-4f;
    p = __builtin_fmaf(p, r, 1.38888892251998186e-3f);
    p = __builtin_fmaf(p, r, 8.33333376795053482e-3f);
    p = __builtin_fmaf(p, r, 4.16666679084300995e-2f);
    p = __builtin_fmaf(p, r, 1.66666671633720398e-1f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return scale2(p, (int)n);
}
// 2^y = 2^n 2^f with n = rint(y), f = y - n (exact), 2^f by the polynomial of
// e^(f ln 2) with its coefficients multiplied through by powers of ln 2.
__device__ __forceinline__ float rda_exp2f(float y) {
    if (y != y) return y;
    if (y >= 128.0f) return __builtin_inff();
    if (y < -127.0f) return 0.0f;
    const float n = rintf(y);
    const float f = y - n;
    float p = 1.52527336467755958e-5f;
    p = __builtin_fmaf(p, f, 1.54035296873189509e-4f);
    p = __builtin_fmaf(p, f, 1.33335578721016645e-3f);
    p = __builtin_fmaf(p, f, 9.61812864989042282e-3f);
    p = __builtin_fmaf(p, f, 5.55041097104549408e-2f);
    p = __builtin_fmaf(p, f, 2.40226507186889648e-1f);
    p = __builtin_fmaf(p, f, 6.93147182464599609e-1f);
    p = __builtin_fmaf(p, f, 1.0f);
    return scale2(p, (int)n);
}

// x / s for an fp16 value x (as float) and a per-row quantization scale s, from rcp = 1 / s (one IEEE division
// per row): the product with the reciprocal, corrected by its exact residual. For every fp16 x with |x| <= a
// and s = max(a / 127, 1e-30) or s = max(a, 1e-10) / 7, a an fp16 absmax, this is the correctly rounded
// quotient (tests/exhaustive_div.c checks every such pair); only the sign of a zero quotient may differ, which
// no caller depends on. Three instructions instead of the ~10 of an IEEE division.
__device__ __forceinline__ float div_by_scale(float x, float s, float rcp) {
    const float y = x * rcp;
    return __builtin_fmaf(__builtin_fmaf(-y, s, x), rcp, y);
}

__device__ __forceinline__ i4v as_i4(u4v v) { return __builtin_bit_cast(i4v, v); }

// Cross-lane reductions on DPP and lane-swap instructions (one VALU op per step, no LDS round trip).
// Every lane of a group receives the same bits: partners always add the same two partial values.
template <int CTRL>
__device__ __forceinline__ float dpp(float x) { return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false)); }
// Over the 16 lanes of each row (lanes 16 r .. 16 r + 15): xor 1, xor 2 (quad_perm), then the half-row
// mirror (i <-> 7 - i) and the row mirror (i <-> 15 - i).
__device__ __forceinline__ float row_sum16(float x) {
    x += dpp<0xB1>(x);
    x += dpp<0x4E>(x);
    x += dpp<0x141>(x);
    x += dpp<0x140>(x);
    return x;
}
__device__ __forceinline__ float row_max16(float x) {
    x = fmaxf(x, dpp<0xB1>(x));
    x = fmaxf(x, dpp<0x4E>(x));
    x = fmaxf(x, dpp<0x141>(x));
    x = fmaxf(x, dpp<0x140>(x));
    return x;
}
// The value of lane l ^ 4 and of lane l ^ 8, by two mirrors each (half-row i <-> 7 - i, quad i <-> 3 - i, row
// i <-> 15 - i): exact partners, no LDS round trip.
__device__ __forceinline__ float lane_xor4(float x) { return dpp<0x1B>(dpp<0x141>(x)); }
__device__ __forceinline__ float lane_xor8(float x) { return dpp<0x141>(dpp<0x140>(x)); }
// sum += __shfl_xor(sum, o) for o = W / 2, ..., 2, 1 (W = 32 or 16), with the same partners, so the same bits (each
// step adds the same two values in every lane of a pair; IEEE addition is commutative).
template <int W>
__device__ __forceinline__ float xor_butterfly_sum(float x) {
    static_assert(W == 32 || W == 16, "32- or 16-lane butterflies");
    if constexpr (W == 32) {
        const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        x = __uint_as_float(a[0]) + __uint_as_float(a[1]);  // lanes l and l ^ 16
    }
    x += lane_xor8(x);
    x += lane_xor4(x);
    x += dpp<0x4E>(x);
    return x + dpp<0xB1>(x);
}
// Over the four rows (lanes l, l ^ 16, l ^ 32, l ^ 48).
__device__ __forceinline__ float rows_sum(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
__device__ __forceinline__ float rows_max(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

typedef __attribute__((address_space(3))) void lds_void_t;

// Direct global->LDS copies: 16 (4) bytes per lane from base + off (or from src), lane i writing LDS
// address lds + 16 i (4 i). They are issued from asm, which keeps them out of the compiler's wait
// bookkeeping: the compiler cannot tell the LDS stage they fill from the stage being read and would
// otherwise make every LDS read wait for the copies in flight. A kernel waits for its copies itself
// (wait_copies, wait_copies_but) before the barrier that hands a stage over.
// They set m0 (the copies' LDS base), a register the compiler reserves; clang warns that such a clobber may not
// be honoured. Nothing else in these kernels uses m0 (tests/test_abi.py checks the generated code: every m0
// reference is the s_mov_b32 of one of these copies), so the warning is silenced here.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ u32 lds_addr(const char* p) { return (u32)(uintptr_t)(const lds_void_t*)p; }
__device__ __forceinline__ void dma16(const void* base, u32 off, const char* lds) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds_addr(lds)) : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* base, u32 off, const char* lds) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(base), "s"(lds_addr(lds)) : "memory", "m0");
}
__device__ __forceinline__ void dma16_at(const void* src, const char* lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds_addr(lds)) : "memory", "m0");
}
#pragma clang diagnostic pop
__device__ __forceinline__ void wait_copies() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// Waits until at most N of this wave's copies are outstanding (they complete in issue order).
template <int N>
__device__ __forceinline__ void wait_copies_but() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }
