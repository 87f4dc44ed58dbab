/* CPU check of the quantizers' quotient (kvq_decode_amd/csrc/quant.hip, quotient()):
 *   r = RN(1/s), q = RN(d r), rem = fma(-q, s, d), t = fma(rem, r, q)
 * must equal the IEEE quotient RN(d / s) bit for bit for every positive finite fp16 s and
 * every d = fl32(x - z) of fp16 x, z (0 or |d| >= 2^-24). Cases: random fp16 x, z for
 * every s, and d at and a few ulps around multiples of s / 2 (quotients at and near
 * half-integers). Exit status 0 = no difference. With argv[1] = "plain", t = RN(d r)
 * alone is checked instead, which must differ somewhere (the check's own sanity test). */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static float h2f(uint16_t h) { __fp16 x; memcpy(&x, &h, 2); return (float)x; }
static uint64_t rs = 0x9E3779B97F4A7C15ull;
static uint32_t rnd32(void) { rs ^= rs << 13; rs ^= rs >> 7; rs ^= rs << 17; return (uint32_t)(rs >> 16); }

static int plain;
static float quotient(float d, float s, float r) {
    const float q = d * r;
    if (plain) return q;
    const float rem = fmaf(-q, s, d);
    return fmaf(rem, r, q);
}

static long n, bad;
static void check(float d, float s, float r) {
    if (!isfinite(d) || (d != 0.f && fabsf(d) < 5.9604644775390625e-8f)) return;
    const float e = d / s, t = quotient(d, s, r);
    ++n;
    if (f2u(t) != f2u(e) && !(t == 0.f && e == 0.f)) {
        if (bad < 5) printf("s %a d %a: IEEE %a, quotient() %a\n", s, d, e, t);
        ++bad;
    }
}

int main(int argc, char** argv) {
    plain = argc > 1 && strcmp(argv[1], "plain") == 0;
    for (uint32_t sb = 1; sb < 0x7C00; ++sb) {
        const float s = h2f((uint16_t)sb), r = 1.f / s;
        for (int k = 0; k < 128; ++k) {
            const uint16_t xb = rnd32() & 0xFFFF, zb = rnd32() & 0xFFFF;
            if ((xb & 0x7C00) == 0x7C00 || (zb & 0x7C00) == 0x7C00) continue;
            check(h2f(xb) - h2f(zb), s, r);
        }
        for (int m = -64; m <= 64; ++m)
            for (int u = -2; u <= 2; ++u) check(u2f(f2u((float)m * s * 0.5f) + u), s, r);
    }
    printf("%ld cases, %ld differ from IEEE division\n", n, bad);
    return bad != 0;
}
