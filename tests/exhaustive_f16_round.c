// Exhaustive check of the packed fp16 rounding steps of the quantization passes (csrc/quant.hip, to_half2): the
// reference rounds r16(a * b) and r16(a + b) -- an fp32 product or sum of two fp16 values, rounded to fp16 -- and
// the kernels compute them as fp16 products and sums (v_pk_mul_f16, v_pk_add_f16), i.e. the exact result rounded
// once to fp16. For every pair of finite fp16 values (by symmetry: a >= 0, |b| <= a, both signs of b) this checks
// that the two roundings agree, signed zeros and overflow to infinity included.
// Build: gcc -O2 -fopenmp -ffp-contract=off exhaustive_f16_round.c -lm. Prints the mismatch counts; exit status 0
// when both are zero.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static double h2d(uint16_t h) {
    const int e = (h >> 10) & 31, m = h & 1023;
    const double v = e == 0 ? ldexp((double)m, -24) : ldexp((double)(1024 + m), e - 25);
    return (h & 0x8000u) ? -v : v;
}

// x (finite) rounded to the nearest fp16 value, ties to even; +-inf past the largest finite value's rounding range.
static double round_f16(double x) {
    const double ax = fabs(x);
    if (ax >= 65520.0) return copysign(INFINITY, x);
    int e;
    frexp(ax, &e);  // ax = f 2^e, f in [0.5, 1)
    const int q = ax < 0x1p-14 ? -24 : e - 11;  // the grid spacing of the binade (subnormals: 2^-24)
    const double r = ldexp(nearbyint(ldexp(ax, -q)), q);
    return copysign(r, x);
}

static int same(double u, double v) { return u == v && signbit(u) == signbit(v); }

int main(void) {
    long bad_mul = 0, bad_add = 0;
#pragma omp parallel for reduction(+ : bad_mul, bad_add) schedule(dynamic, 16)
    for (int ha = 0; ha < 0x7c00; ha++) {
        const double a = h2d((uint16_t)ha);
        const float af = (float)a;
        for (int hb = 0; hb <= ha; hb++) {
            for (int sgn = 0; sgn < 2; sgn++) {
                const double b = sgn ? -h2d((uint16_t)hb) : h2d((uint16_t)hb);
                const float bf = (float)b;
                const float pf = af * bf, sf = af + bf;  // the reference's fp32 operations
                if (!same(round_f16((double)pf), round_f16(a * b))) {  // a * b is exact in double
                    if (bad_mul < 5) printf("mul a=%a b=%a\n", a, b);
                    bad_mul++;
                }
                if (!same(round_f16((double)sf), round_f16(a + b))) {  // a + b is exact in double
                    if (bad_add < 5) printf("add a=%a b=%a\n", a, b);
                    bad_add++;
                }
            }
        }
    }
    printf("mismatches: mul %ld, add %ld\n", bad_mul, bad_add);
    return bad_mul || bad_add;
}
