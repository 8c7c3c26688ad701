/*
 * CPU proof checks for the two arithmetic identities the pre-quant kernel
 * (kore_amd/csrc/norm.hip, quant_code) relies on.  Both use only IEEE
 * binary32 operations that the GPU executes identically (mul, fma, add,
 * truncating convert), so checking them here checks the kernel's math.
 *
 *  1. Markstein quotient: with y = RN(1/b), q0 = RN(a*y),
 *     r = fma(-b, q0, a), t = fma(r, y, q0)  ==>  t == RN(a/b).
 *     Checked on random (a, b) pairs drawn from the kernel's domain
 *     (b > 0 finite, |a| <= 127*b*(1+2^-23), plus 1e-8 <= b), on a grid of
 *     exponents, and on every a at a set of hard divisors.
 *  2. Ties-away rounding: trunc(t + copysign(0.5 - 2^-25, t)) == roundf(t)
 *     for EVERY float t with |t| < 2^23 (exhaustive over bit patterns).
 *  3. Bracketed fast code: with M = amax in [1e-8, 2^120) (or the 1.0
 *     guard), y = RN(1/M), c = RN(127*y), v = fma(xn, c, 0.5 - 2^-14):
 *     whenever fract(v) < 1 - 2^-13, floor(v) (v_cvt_flr_i32_f32, exact) is
 *     the reference code clamp(round_half_away(RN(RN(xn*127)/M))).  Checked
 *     on random (xn, M) with |xn| <= M, and on numerators placed within a
 *     few ulps of every tie k + 0.5.
 *
 * Exit status 0 when both hold; prints the first counterexample otherwise.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float bits2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f2bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static uint64_t rng = 0x9E3779B97F4A7C15ull;
static uint64_t next(void) {
    rng ^= rng << 13; rng ^= rng >> 7; rng ^= rng << 17; return rng;
}

static int check_div(float a, float b) {
    volatile float y = 1.0f / b;
    volatile float q0 = a * y;
    volatile float r = fmaf(-b, q0, a);
    volatile float t = fmaf(r, y, q0);
    volatile float ref = a / b;
    if (f2bits(t) != f2bits(ref) && !(t != t && ref != ref)) {
        printf("markstein mismatch: a=%a b=%a t=%a ref=%a\n", a, b, t, ref);
        return 1;
    }
    return 0;
}

static int check_round(float t) {
    volatile float bias = copysignf(0.49999997f, t);
    volatile float s = t + bias;
    int32_t c = (int32_t)truncf(s);
    int32_t ref = (int32_t)roundf(t);
    if (c != ref) {
        printf("round mismatch: t=%a (%.9g) got %d want %d\n", t, t, c, ref);
        return 1;
    }
    return 0;
}

static long n_ambiguous = 0;

/* The reference code of xn for absmax M (both finite, |xn| <= M). */
static int32_t ref_code(float xn, float M) {
    volatile float a = xn * 127.0f;
    volatile float t = a / M;
    float r = roundf(t);
    if (r != r) return 0;
    if (r < -128.0f) r = -128.0f;
    if (r > 127.0f) r = 127.0f;
    return (int32_t)r;
}

static int check_bracket(float xn, float M) {
    const float off = 0.5f - 6.103515625e-05f; /* 0.5 - 2^-14, exact */
    volatile float y = 1.0f / M;
    volatile float c = 127.0f * y;
    volatile float v = fmaf(xn, c, off);
    volatile float fl = floorf(v);
    volatile float fr = v - fl; /* exact: v_fract_f32 */
    if (!(fr < 0.99987793f)) { ++n_ambiguous; return 0; } /* 1 - 2^-13 */
    int32_t code = (int32_t)fl;
    int32_t ref = ref_code(xn, M);
    if (code != ref) {
        printf("bracket mismatch: xn=%a M=%a v=%a code=%d want %d\n", xn, M, v, code, ref);
        return 1;
    }
    return 0;
}

int main(int argc, char **argv) {
    long n_random = argc > 1 ? atol(argv[1]) : 50000000L;
    /* 2. exhaustive rounding over |t| < 2^23, both signs */
    const uint32_t lim = f2bits(8388608.0f);
    for (uint32_t u = 0; u < lim; ++u) {
        float t = bits2f(u);
        if (check_round(t) || check_round(-t)) return 1;
    }
    /* 1a. random pairs in the kernel's domain */
    for (long i = 0; i < n_random; ++i) {
        /* b: positive normal float, exponent spread over [1e-8, 1e30] */
        uint32_t eb = 100 + (uint32_t)(next() % 127);     /* biased exp 100..226 */
        float b = bits2f((eb << 23) | (uint32_t)(next() & 0x7FFFFF));
        /* a = xn*127 with |xn| <= b: build xn as b * u, u in [-1, 1] */
        double u = ((double)(next() >> 11) / 9007199254740992.0) * 2.0 - 1.0;
        float xn = (float)(b * u);
        if (fabsf(xn) > b) xn = copysignf(b, xn);
        float a = xn * 127.0f;
        if (check_div(a, b)) return 1;
        /* also a near-tie numerator: a = (k + 0.5) * b rounded */
        int k = (int)(next() % 128);
        float a2 = (float)(((double)k + 0.5) * (double)b);
        if (check_div(a2, b) || check_div(-a2, b)) return 1;
    }
    /* 1b. every numerator mantissa against a few divisors */
    const float divs[] = {1.0f, 3.0f, 127.0f, 1.5f, 1.99999988f, 1.00000012f, 0.1f, 7.0f, 1e-8f, 12345.678f};
    for (unsigned d = 0; d < sizeof(divs) / sizeof(divs[0]); ++d) {
        for (uint32_t m = 0; m < (1u << 23); m += 1) {
            float a = bits2f((127u << 23) | m) * 64.0f; /* [64,128) */
            if (check_div(a, divs[d]) || check_div(a * 0.5f, divs[d])) return 1;
        }
    }
    /* 3a. bracketed fast code on random (xn, M), M over the fast path's range */
    long n_br = 0;
    for (long i = 0; i < n_random; ++i) {
        uint32_t eb = 100 + (uint32_t)(next() % 147);      /* biased exp 100..246: M in [1e-8, 2^120) */
        float M = bits2f((eb << 23) | (uint32_t)(next() & 0x7FFFFF));
        if (M < 1e-8f) M = 1e-8f;
        double u = ((double)(next() >> 11) / 9007199254740992.0) * 2.0 - 1.0;
        float xn = (float)(M * u);
        if (fabsf(xn) > M) xn = copysignf(M, xn);
        if (check_bracket(xn, M) || check_bracket(M, M) || check_bracket(-M, M)) return 1;
        /* numerators at and around a tie: 127*xn/M ~ k + 0.5, stepped by ulps */
        int k = (int)(next() % 128);
        float xt = (float)(((double)k + 0.5) * (double)M / 127.0);
        for (int d = -6; d <= 6; ++d) {
            float v = bits2f(f2bits(xt) + (uint32_t)d);
            if (fabsf(v) <= M && (check_bracket(v, M) || check_bracket(-v, M))) return 1;
        }
        n_br += 29;
    }
    /* 3b. the guard (M = 1.0, every |xn| < 1e-8) and small/large exponents */
    for (long i = 0; i < 1000000; ++i) {
        float v = bits2f((uint32_t)(next() % 0x3229705Fu)); /* [0, 1e-8) */
        if (check_bracket(v, 1.0f) || check_bracket(-v, 1.0f)) return 1;
    }
    printf("ok: rounding exhaustive below 2^23, %ld random quotient pairs, %u divisor sweeps, "
           "%ld bracket checks (%ld ambiguous)\n", n_random,
           (unsigned)(sizeof(divs) / sizeof(divs[0])), n_br, n_ambiguous);
    return 0;
}
