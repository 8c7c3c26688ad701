/*
 * CPU check of the segmented exact fold used by the row kernels
 * (kore_amd/csrc/norm.hip): it must return, bit for bit, the left-to-right
 * f32 fold  s_0 = +0, s_i = RN(s_{i-1} + a_i)  of non-negative terms a_i
 * (squares), for every input -- including NaN/Inf, subnormals, overflow,
 * exact ties and adversarial binade crossings.
 *
 * The algorithm (one row, K segments of L consecutive terms):
 *   0. estimate the running sum at every segment start (any order);
 *   1. for segment j, guess the binade E of its true start from the estimate
 *      and fold the segment twice from artificial starts sigma_p, p in {0,1}:
 *      sigma_0 = 2^E, sigma_1 = 2^E + ulp (E = -126: 0 and 2^-149), giving
 *      increments d_p = w_p - sigma_p and ok_p = (w_p < 2^(E+1));
 *   2. resolve in order: with the exact start s of segment j, if s lies in
 *      binade E (the grid of ulp 2^(E-23)), p = lsb(bits(s)), ok_p and
 *      RN(s + d_p) < 2^(E+1), then the segment's true end is s + d_p;
 *      otherwise fold the segment sequentially from s.
 * Step 2 is exact because, inside one binade, s -> RN(s + a) commutes with a
 * shift of s by an even number of ulps (the only start-dependence is the
 * ties-to-even parity), and a walk whose shifted end stays below 2^(E+1)
 * never left the binade.  The estimate only decides how often step 2 falls
 * back; it never affects the result.
 *
 * This file restates the GPU algorithm in scalar C (same K, L, guesses and
 * checks) and compares it with the plain sequential fold.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

static float seq_fold(const float *a, int n, float s) {
    for (int i = 0; i < n; ++i) s = s + a[i];
    return s;
}

/* binade index of a non-negative float: -126 for [0, 2^-125), exponent
 * otherwise; 128 for Inf/NaN (matches no segment guess). */
static int binade(float s) {
    uint32_t u = f2u(s);
    int ex = (int)((u >> 23) & 0xff);
    if (ex == 0xff) return 128;
    if (ex == 0) return -126;
    return ex - 127;
}

static float pow2f(int e) { return e > 127 ? INFINITY : u2f((uint32_t)(e + 127) << 23); }

/* mirrors the kernel: guess E from an f32 estimate of the segment start */
static float sef_fold(const float *a, int n, int K, long *fallbacks) {
    int L = (n + K - 1) / K;
    float est = 0.0f;
    float s = 0.0f;
    for (int j = 0; j < K; ++j) {
        int lo = j * L, hi = lo + L < n ? lo + L : n;
        if (lo >= n) break;
        /* phase 0 (per lane, here in order): estimate = sum of earlier
         * segments' approximate sums */
        float seg_est = 0.0f;
        for (int i = lo; i < hi; ++i) seg_est += a[i];
        int E = binade(est);
        /* phase 1 */
        float d0 = 0, d1 = 0;
        int ok0 = 0, ok1 = 0;
        if (E <= 127) {
            float lo0 = E == -126 ? 0.0f : pow2f(E);
            float g = pow2f(E - 23 < -149 ? -149 : E - 23);
            if (E == -126) g = u2f(1); /* 2^-149 */
            float lo1 = lo0 + g;
            float top = pow2f(E + 1);
            float w0 = seq_fold(a + lo, hi - lo, lo0);
            float w1 = seq_fold(a + lo, hi - lo, lo1);
            ok0 = w0 < top;
            ok1 = w1 < top;
            d0 = w0 - lo0;
            d1 = w1 - lo1;
        }
        /* phase 2 */
        int done = 0;
        if (binade(s) == E && E <= 127) {
            int p = (int)(f2u(s) & 1u);
            float d = p ? d1 : d0;
            int ok = p ? ok1 : ok0;
            float t = s + d;
            if (ok && t < pow2f(E + 1)) {
                s = t;
                done = 1;
            }
        }
        if (!done) {
            ++*fallbacks;
            s = seq_fold(a + lo, hi - lo, s);
        }
        est = est + seg_est;
    }
    return s;
}

/* Scalar restatement of row_norm_kernel's fold (kore_amd/csrc/norm.hip):
 * 64 segments of sl4 float4 (sl4 = ceil(n4 / 64)), estimates from an
 * inclusive scan of pairwise segment sums, lane 0 folding from the exact
 * start, invalid walks encoded as NaN increments, empty segments as the
 * identity, and the resolve check s >= bot && s + d < top.  n % 4 == 0. */
static float kernel_fold(const float *a, int n, long *fallbacks) {
    const int n4 = n / 4;
    const int sl4 = (n4 + 63) / 64 ? (n4 + 63) / 64 : 1;
    const int nseg = (n4 + sl4 - 1) / sl4;
    const int sl = 4 * sl4;
    float d0[64], d1[64], bot[64], top[64], ssum[64];
    const float inf = INFINITY, qnan = NAN;
    for (int j = 0; j < 64; ++j) {
        ssum[j] = 0.0f;
        for (int k = 0; k < sl4; ++k) {
            int i = j * sl + 4 * k;
            float v[4];
            for (int q = 0; q < 4; ++q) v[q] = (i + q < n) ? a[i + q] : 0.0f;
            ssum[j] += (v[0] + v[1]) + (v[2] + v[3]);
        }
    }
    /* Hillis-Steele inclusive scan, as the __shfl_up loop computes it */
    float incl[64], tmp[64];
    for (int j = 0; j < 64; ++j) incl[j] = ssum[j];
    for (int d = 1; d < 64; d <<= 1) {
        for (int j = 0; j < 64; ++j) tmp[j] = (j >= d) ? incl[j] + incl[j - d] : incl[j];
        memcpy(incl, tmp, sizeof(incl));
    }
    for (int j = 0; j < 64; ++j) {
        float est = incl[j] - ssum[j];
        if (j >= nseg) { d0[j] = 0; d1[j] = 0; bot[j] = 0; top[j] = inf; continue; }
        float sig0, sig1, b, t;
        if (j == 0) { sig0 = 0; sig1 = 0; b = 0; t = inf; }
        else {
            uint32_t ef = f2u(est) >> 23;
            if (ef >= 255u) { sig0 = 0; sig1 = 0; b = inf; t = 0; }
            else if (ef <= 1u) { sig0 = 0; sig1 = u2f(1u); b = 0; t = u2f(2u << 23); }
            else { sig0 = u2f(ef << 23); sig1 = u2f((ef << 23) | 1u); b = sig0; t = u2f((ef + 1u) << 23); }
        }
        float w0 = sig0, w1 = sig1;
        for (int i = j * sl; i < j * sl + sl; ++i) {
            float v = i < n ? a[i] : 0.0f;
            w0 = w0 + v;
            w1 = w1 + v;
        }
        d0[j] = (w0 < t) ? w0 - sig0 : qnan;
        d1[j] = (j != 0 && w1 < t) ? w1 - sig1 : qnan;
        bot[j] = b;
        top[j] = t;
    }
    float s = 0.0f;
    for (int j = 0; j < nseg; ++j) {
        float d = (f2u(s) & 1u) ? d1[j] : d0[j];
        float t = s + d;
        if (s >= bot[j] && t < top[j]) {
            s = t;
        } else {
            ++*fallbacks;
            for (int i = j * sl; i < j * sl + sl; ++i) s = s + (i < n ? a[i] : 0.0f);
        }
    }
    return s;
}

static long rfb = 0;

/* Run-jumping resolve (row_norm_kernel's current form): consecutive valid
 * segments that share a binade form a run; for every segment j the exact
 * increment of [j, run end] is composed from the per-segment increments and
 * end parities (F_j(p) = lsb(w_p)).  The resolve runs on integers: inside a
 * binade [bot, top) of grid g the float bits are linear in the value, so a
 * run's increment D is stored as D/g = bits(bot + D) - bits(bot) (or
 * 0x7fffffff when bot + D >= top), and a jump is taken when the bits s of the
 * running sum satisfy max(s - lo, s + inc - lo) < width in wrapping unsigned
 * arithmetic (lo = bits(bot), width = bits(top) - lo; both s and s + inc in
 * [bot, top)); otherwise, or when segment j is outside every run (width 0),
 * segment j is folded alone from s.  Segment 0 is folded from +0 exactly. */
static uint32_t run_inc(float bot, float top, float d) {
    float e = bot + d;
    return (e < top) ? f2u(e) - f2u(bot) : 0x7fffffffu;
}

static float run_fold(const float *a, int n, long *steps) {
    const int n4 = n / 4;
    const int sl4 = (n4 + 63) / 64 ? (n4 + 63) / 64 : 1;
    const int nseg = (n4 + sl4 - 1) / sl4;
    const int sl = 4 * sl4;
    float d0[64], d1[64], bot[64], top[64], ssum[64], est[64], w0s[64];
    int f0[64], f1[64], key[64], valid[64];
    (void)f0; (void)f1;
    uint32_t efs[64];
    const float qnan = NAN;
    float total = 0.0f;
    for (int j = 0; j < 64; ++j) {
        ssum[j] = 0.0f;
        for (int i = j * sl; i < j * sl + sl; ++i) ssum[j] += (i < n) ? a[i] : 0.0f;
    }
    for (int j = 0; j < 64; ++j) { est[j] = total; total += ssum[j]; }
    for (int j = 0; j < 64; ++j) {
        float sig0, sig1;
        if (j >= nseg) { d0[j] = d1[j] = 0; bot[j] = 0; top[j] = INFINITY; f0[j] = 0; f1[j] = 1; key[j] = 1024; valid[j] = 1; efs[j] = 0; continue; }
        uint32_t ef = f2u(est[j]) >> 23;
        if (ef < 1u) ef = 1u;
        int bad = j != 0 && ef >= 255u;
        efs[j] = bad ? 0u : ef;
        if (ef == 1u) { sig0 = 0; sig1 = u2f(1u); } else { sig0 = u2f(ef << 23); sig1 = u2f((ef << 23) | 1u); }
        bot[j] = sig0;
        top[j] = u2f((ef + 1u) << 23);
        if (j == 0) { sig0 = 0; sig1 = 0; key[j] = 1025; } else key[j] = (int)ef;
        float w0 = sig0, w1 = sig1;
        for (int i = j * sl; i < j * sl + sl; ++i) { float v = i < n ? a[i] : 0.0f; w0 = w0 + v; w1 = w1 + v; }
        w0s[j] = w0;
        int ok0 = j == 0 || w0 < top[j], ok1 = j == 0 || w1 < top[j];
        int edge = j != 0 && (est[j] < bot[j] * 1.0009765625f || est[j] + ssum[j] >= top[j] * 0.9990234375f);
        valid[j] = ok0 && ok1 && !edge && !bad;
        d0[j] = ok0 ? w0 - sig0 : qnan;
        d1[j] = (j == 0) ? d0[j] : (ok1 ? w1 - sig1 : qnan);
        f0[j] = (int)(f2u(w0) & 1u);
        f1[j] = (j == 0) ? 0 : (int)(f2u(w1) & 1u);
        if (!valid[j] && j != 0) key[j] = 2048 + j;
    }
    /* Runs (the kernel's integer form): a valid segment whose two walks give
     * the same bit increment ("simple") maps every start in its binade to
     * s + inc; consecutive simple segments with one binade key form a run
     * whose entry is the sum of their increments.  Any other segment is a
     * run of its own and keeps both increments. */
    uint32_t I0[64], I1[64], inc0[64], inc1[64];
    int simple[64], rkey[64], next[64];
    for (int j = 0; j < 64; ++j) {
        inc0[j] = run_inc(bot[j], top[j], d0[j]);
        inc1[j] = run_inc(bot[j], top[j], d1[j]);
        simple[j] = j < nseg && j != 0 && valid[j] && inc0[j] == inc1[j];
        rkey[j] = j >= nseg ? 1024 : (j == 0 ? 1025 : (simple[j] ? (int)efs[j] : 2048 + j));
    }
    for (int j = 63; j >= 0; --j) {
        int end_here = (j == 63) || rkey[j + 1] != rkey[j];
        uint32_t own = simple[j] ? inc0[j] : 0u;
        uint32_t sum = end_here ? own : own + (I0[j + 1]);
        next[j] = end_here ? j + 1 : next[j + 1];
        I0[j] = simple[j] ? sum : inc0[j];
        I1[j] = simple[j] ? sum : inc1[j];
    }
    uint32_t s = f2u(w0s[0]);
    int j = 1;
    while (j < nseg) {
        ++*steps;
        uint32_t i0 = I0[j], i1 = I1[j];
        uint32_t lo = f2u(bot[j]), wd = valid[j] ? f2u(top[j]) - f2u(bot[j]) : 0u;
        uint32_t t = s + ((s & 1u) ? i1 : i0);
        uint32_t da = s - lo, db = t - lo;
        if (wd != 0u && (da > db ? da : db) < wd) { s = t; j = next[j]; }
        else {
            ++rfb;
            float acc = u2f(s);
            for (int i = j * sl; i < j * sl + sl; ++i) acc = acc + (i < n ? a[i] : 0.0f);
            s = f2u(acc);
            ++j;
        }
    }
    return u2f(s);
}

static uint64_t rs = 88172645463325252ull;
static uint64_t xr(void) { rs ^= rs << 13; rs ^= rs >> 7; rs ^= rs << 17; return rs; }
static double unif(void) { return (double)(xr() >> 11) / 9007199254740992.0; }
static double gauss(void) {
    double u = unif(), v = unif();
    if (u < 1e-300) u = 1e-300;
    return sqrt(-2 * log(u)) * cos(6.283185307179586 * v);
}

static long kfb = 0, krows = 0, rsteps = 0;
static int check(const float *a, int n, int K, long *fb, const char *what, long row) {
    float r0 = seq_fold(a, n, 0.0f);
    float r1 = sef_fold(a, n, K, fb);
    if (f2u(r0) != f2u(r1) && !(r0 != r0 && r1 != r1)) {
        printf("MISMATCH %s row %ld n=%d K=%d: seq=%a sef=%a\n", what, row, n, K, r0, r1);
        return 1;
    }
    if (n % 4 == 0) {
        float r2 = kernel_fold(a, n, &kfb);
        ++krows;
        if (f2u(r0) != f2u(r2) && !(r0 != r0 && r2 != r2)) {
            printf("MISMATCH kernel_fold %s row %ld n=%d: seq=%a kernel=%a\n", what, row, n, r0, r2);
            return 1;
        }
        float r3 = run_fold(a, n, &rsteps);
        if (f2u(r0) != f2u(r3) && !(r0 != r0 && r3 != r3)) {
            printf("MISMATCH run_fold %s row %ld n=%d: seq=%a run=%a\n", what, row, n, r0, r3);
            return 1;
        }
    }
    return 0;
}

int main(int argc, char **argv) {
    long rows = argc > 1 ? atol(argv[1]) : 200000;
    static float a[16384];
    long fb = 0, total_segs = 0;
    const int sizes[] = {1, 2, 3, 4, 7, 8, 40, 64, 100, 256, 260, 1000, 2048, 2560, 4096, 5000, 8192, 16384};
    const int Ks[] = {1, 4, 16, 64};
    for (long r = 0; r < rows; ++r) {
        int n = sizes[xr() % (sizeof(sizes) / sizeof(sizes[0]))];
        int K = Ks[xr() % 4];
        int kind = (int)(xr() % 10);
        for (int i = 0; i < n; ++i) {
            double x;
            switch (kind) {
                case 0: x = gauss(); break;                              /* N(0,1) */
                case 1: x = gauss() * (unif() < 0.01 ? 20 : 1); break;   /* outliers */
                case 2: x = gauss() * 1e-21; break;                      /* subnormal squares */
                case 3: x = gauss() * 1e19; break;                       /* overflow to Inf */
                case 4: x = (double)(int)(gauss() * 8); break;           /* small ints: many exact ties */
                case 5: x = ldexp(1.0, (int)(xr() % 40) - 20); break;   /* powers of two */
                case 6: x = (xr() % 3 == 0) ? 0.0 : gauss(); break;      /* zeros */
                case 7: x = sqrt((double)(xr() % 1000)) ; break;         /* near-integer squares */
                case 8: x = gauss() * ldexp(1.0, (int)(xr() % 60) - 30); break; /* mixed scales */
                default: x = (i == (int)(xr() % n)) ? gauss() * 1e3 : gauss() * 1e-3; break;
            }
            float xf = (float)x;
            a[i] = xf * xf;
        }
        if (kind == 9 && (xr() % 50) == 0) a[xr() % n] = NAN;
        if (kind == 9 && (xr() % 50) == 1) a[xr() % n] = INFINITY;
        total_segs += K;
        if (check(a, n, K, &fb, "random", r)) return 1;
    }
    printf("ok: %ld rows, fallback segments %ld of %ld; kernel mirror: %ld rows, %.2f fallbacks/row\n", rows, fb,
           total_segs, krows, krows ? (double)kfb / krows : 0.0);
    printf("run-jumping resolve: %.2f steps/row, %.2f fallbacks/row\n", krows ? (double)rsteps / krows : 0.0, krows ? (double)rfb / krows : 0.0);
    return 0;
}
