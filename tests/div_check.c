/* The norms' division by a shared divisor (div_shared in
 * gemma4-webgpu_amd/csrc/ref_math.h: q0 = a * y with y = 1.0f / b, then
 * fma(fma(-q0, b, a), y, q0); tiny, zero or non-finite dividends and divisors
 * of 2^32 or more take a / b) against the IEEE quotient a / b, bit for bit:
 *   - n random pairs: a of every exponent (denormals and zeros included) and
 *     either sign, b in [2^-60, 2^35) (a norm's rms is at least sqrt(eps));
 *   - every significand of b in [1, 2), each with 4 random dividends, +0, -0;
 *   - dividends next to the fast path's threshold 2^-64.
 * Quotients that overflow are skipped: a norm's quotient is at most 16 times
 * its weight (|x| <= 16 rms over 256 elements).
 * Prints the count of pairs tested and of mismatches; exits 1 on a mismatch.
 * Build: gcc -O2 -ffp-contract=off div_check.c -lm (contraction off: the
 * products and sums are rounded one by one, as on the device). */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static uint64_t state = 88172645463325252ull;
static uint64_t next(void) {
    state ^= state << 13;
    state ^= state >> 7;
    state ^= state << 17;
    return state;
}
static float from_bits(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static uint32_t to_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static float div_shared(float a, float b, float y) {
    if (!(fabsf(a) >= 0x1p-64f) || !(b < 0x1p32f)) return a / b;
    const float q0 = a * y;
    return fmaf(fmaf(-q0, b, a), y, q0);
}

static long tested, bad;
static void check(float a, float b) {
    const float want = a / b;
    if (isinf(want)) return;
    const float got = div_shared(a, b, 1.0f / b);
    tested++;
    if (to_bits(want) != to_bits(got)) {
        if (bad < 10) printf("mismatch: a=%a b=%a a/b=%a got %a\n", a, b, want, got);
        bad++;
    }
}

int main(int argc, char** argv) {
    const long n = argc > 1 ? atol(argv[1]) : 20000000L;
    for (long i = 0; i < n; i++) {
        const uint32_t be = 127 - 60 + (uint32_t)(next() % 95);
        const float b = from_bits((be << 23) | (uint32_t)(next() & 0x7fffff));
        const float a = from_bits(((uint32_t)(next() & 1) << 31) | ((uint32_t)(next() % 255) << 23) |
                                  (uint32_t)(next() & 0x7fffff));
        check(a, b);
    }
    for (uint32_t m = 0; m < (1u << 23); m++) {
        const float b = from_bits((127u << 23) | m);
        for (int k = 0; k < 4; k++)
            check(from_bits(((uint32_t)(next() & 1) << 31) | ((uint32_t)(90 + next() % 80) << 23) |
                            (uint32_t)(next() & 0x7fffff)), b);
        check(0.0f, b);
        check(-0.0f, b);
        check(nextafterf(0x1p-64f, 0.0f), b);
        check(0x1p-64f, b);
        check(-0x1p-64f, b);
    }
    printf("tested %ld pairs, mismatches %ld\n", tested, bad);
    return bad != 0;
}
