// Exhaustive check of div_by_scale (csrc/common.h), the quotient the quantizers use: for every fp16 absmax
// a >= 0 and every fp16 x with |x| <= a, the reciprocal-and-correct sequence r = 1 / scale; y = x * r;
// e = fma(-y, scale, x); q = fma(e, r, y) equals the correctly rounded x / scale (the oracle's division), for
// scale = max(a / 127, 1e-30) (int8 codes) and scale = max(a, 1e-10) / 7 (int4 codes). A zero quotient may
// differ in sign only; the int8 / int4 codes derived from it must agree in every case.
// Build: gcc -O2 -fopenmp -ffp-contract=off exhaustive_div.c -lm. Prints the mismatch counts; exit status 0
// when both are zero.
#include <math.h>
#include <stdio.h>
#include <stdint.h>
#include <string.h>
static float h2f(uint16_t h) {
    uint32_t s = (h & 0x8000u) << 16, e = (h >> 10) & 31, m = h & 1023, u;
    if (e == 0) { if (!m) u = s; else { float f = ldexpf((float)m, -24); memcpy(&u, &f, 4); u |= s; } }
    else if (e == 31) u = s | 0x7f800000u | (m << 13);
    else u = s | ((e + 112) << 23) | (m << 13);
    float f; memcpy(&f, &u, 4); return f;
}
int main(void) {
    long bad[2] = {0, 0}, total = 0;
    for (int kind = 0; kind < 2; kind++) {
        #pragma omp parallel for reduction(+:bad[kind]) schedule(dynamic, 64)
        for (int ha = 0; ha < 0x7c00; ha++) {
            const float a = h2f((uint16_t)ha);
            const float scale = kind == 0 ? fmaxf(a / 127.f, 1e-30f) : fmaxf(a, 1e-10f) / 7.f;
            const float r = 1.f / scale;
            for (int hx = 0; hx <= ha; hx++) {
                for (int sgn = 0; sgn < 2; sgn++) {
                    const float x = sgn ? -h2f((uint16_t)hx) : h2f((uint16_t)hx);
                    const float ref = x / scale;
                    const float y = x * r, e = fmaf(-y, scale, x), q = fmaf(e, r, y);
                    const int qr = kind == 0 ? (int)fminf(fmaxf(floorf(ref + 0.5f), -128.f), 127.f) : (int)fminf(fmaxf(rintf(ref), -7.f), 7.f);
                    const int qq = kind == 0 ? (int)fminf(fmaxf(floorf(q + 0.5f), -128.f), 127.f) : (int)fminf(fmaxf(rintf(q), -7.f), 7.f);
                    if (qr != qq || (memcmp(&ref, &q, 4) != 0 && !(ref == 0.f && q == 0.f))) {
                        if (bad[kind] < 5) printf("kind %d a=%a x=%a ref=%a got=%a\n", kind, a, x, ref, q);
                        bad[kind]++;
                    }
                }
            }
        }
    }
    printf("mismatches: int8 scale %ld, int4 scale %ld\n", bad[0], bad[1]);
    return bad[0] || bad[1];
}
