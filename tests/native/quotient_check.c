/* The INT8 quantizer's quotient scheme (q8 in yanlongvla_amd/csrc/tcq_device.h) against IEEE division, on the host:
 * q = v * r (r = 1 / s correctly rounded), then twice e = fma(-q, s, v), q = fma(e, r, q). For scales s in [2^-90, 2^90]
 * the scheme must give the same round-half-even integer as v / s for every v with |v| <= 127 s (the quantizer's domain),
 * and the correctly rounded quotient itself whenever |v / s| >= 2^-12.
 * usage: quotient_check PAIRS STEP  -> random near-tie pairs, then every STEP-th FP32 pattern at six scales. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float scheme(float v, float s, float r) {
    float q = v * r;
    float e = fmaf(-q, s, v);
    q = fmaf(e, r, q);
    e = fmaf(-q, s, v);
    return fmaf(e, r, q);
}
static uint64_t state = 88172645463325252ull;
static uint32_t next(void) { state ^= state << 13; state ^= state >> 7; state ^= state << 17; return (uint32_t)state; }
static long bad_round = 0, bad_quot = 0, checked = 0;
static void check(float v, float s, float r) {
    if (!(fabsf(v) <= 127.f * s)) return;
    const float a = v / s, b = scheme(v, s, r);
    ++checked;
    if (rintf(a) != rintf(b)) ++bad_round;
    if (fabsf(a) >= 0x1p-12f && f2u(a) != f2u(b)) ++bad_quot;
}
int main(int argc, char** argv) {
    const long pairs = argc > 1 ? atol(argv[1]) : 1000000;
    const long step = argc > 2 ? atol(argv[2]) : 97;
    for (long i = 0; i < pairs; ++i) {
        float s;
        do { s = u2f(next() & 0x7fffffffu); } while (!(s >= 0x1p-90f && s <= 0x1p90f));
        const float r = 1.0f / s;
        const uint32_t m = next();
        float v = ((float)(int)(m % 255) - 127.0f + 0.5f) * s;                  /* a rounding tie, moved by -2 .. 2 ulp */
        v = u2f(f2u(v) + (int)(next() % 5) - 2);
        check(v, s, r);
        check(u2f(f2u(127.f * s) - (m % 0x7fffff)), s, r);                    /* the top of the row's range */
    }
    const float scales[6] = {0x1p-90f, 0x1.4cccccp-90f, 0.0078740157f, 3.14159f, 1.7e-9f, 0x1.ccccccp+89f};
    for (int k = 0; k < 6; ++k) {
        const float s = scales[k], r = 1.0f / s;
        for (uint64_t u = 0; u < (1ull << 32); u += step) check(u2f((uint32_t)u), s, r);
    }
    printf("checked %ld round-mismatches %ld quotient-mismatches %ld\n", checked, bad_round, bad_quot);
    return bad_round || bad_quot;
}
