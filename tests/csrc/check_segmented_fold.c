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

/* The kernel's current form: every segment gets its own binade guess,
 * walks, validity and run entry.  Runs are maximal spans of "simple"
 * segments (valid, both walks giving the same bit increment) with one
 * binade key, whose entry is the sum of their increments; any other valid
 * segment is a run of its own with both increments.  Entries are jumpable
 * only when valid, outside the merged range [0, 2^-125), with
 * |inc1 - inc0| < 64 and an increment below 2^23; others (width 0) are
 * folded alone from s. */
/* automaton = 1 mirrors the kernel: runs of every valid segment of one
 * binade, composed by the 2-state parity automaton over integer increments
 * (parity after a span with entry parity p is (p + inc_p) & 1).
 * automaton = 0 is an alternative kept as a second check of the resolve:
 * runs of only the segments whose two walks give one increment, composed by
 * adding increments. */
static float run_fold_k(const float *a, int n, long *steps, int automaton) {
    const int n4 = n / 4;
    const int sl4 = (n4 + 63) / 64 ? (n4 + 63) / 64 : 1;
    const int nsubper = 1;
    const int sub4 = sl4 / nsubper;
    const int sl = 4 * sub4;               /* terms per sub-segment */
    const int nsub = (n4 + sub4 - 1) / sub4;
    const int U = 64 * nsubper;
    float ssub[128], est[128], w0s[128];
    uint32_t inc0[128], inc1[128], lo[128], wd[128], I0[128], I1[128], efs[128];
    int simple[128], rkey[128], next[128], valid[128];
    for (int u = 0; u < U; ++u) {
        ssub[u] = 0.0f;
        for (int i = u * sl; i < u * sl + sl; i += 4) {
            float v[4];
            for (int q = 0; q < 4; ++q) v[q] = (i + q < n) ? a[i + q] : 0.0f;
            ssub[u] += (v[0] + v[1]) + (v[2] + v[3]);
        }
    }
    /* segment-start estimates (any order: sequential here), then per half */
    float total = 0.0f;
    for (int j = 0; j < 64; ++j) {
        float e = total;
        for (int h = 0; h < nsubper; ++h) { est[j * nsubper + h] = e; e = e + ssub[j * nsubper + h]; }
        float ssum = ssub[j * nsubper];
        if (nsubper == 2) ssum += ssub[j * nsubper + 1];
        total += ssum;
    }
    for (int u = 0; u < U; ++u) {
        int empty = u >= nsub, first = u == 0 || empty;
        uint32_t ef = f2u(est[u]) >> 23;
        if (ef < 1u) ef = 1u;
        int subn = ef == 1u, bad = !first && ef >= 255u;
        float bot = subn ? 0.0f : u2f(ef << 23);
        float top = u2f((ef + 1u) << 23);
        float sig0 = first ? 0.0f : bot;
        float sig1 = first ? 0.0f : (subn ? u2f(1u) : u2f((ef << 23) | 1u));
        float w0 = sig0, w1 = sig1;
        for (int i = u * sl; i < u * sl + sl; ++i) { float v = i < n ? a[i] : 0.0f; w0 = w0 + v; w1 = w1 + v; }
        w0s[u] = w0;
        int edge = est[u] < bot * 1.0001220703125f || est[u] + ssub[u] >= top * 0.9998779296875f;
        valid[u] = !first && !subn && w0 < top && w1 < top && !edge && !bad;
        inc0[u] = f2u(w0) - f2u(bot);
        inc1[u] = f2u(w1) - f2u(bot) - 1u;
        simple[u] = valid[u] && inc0[u] == inc1[u];
        rkey[u] = empty ? 1024 : (u == 0 ? 1025 : (simple[u] ? (int)ef : 2048 + u));
        lo[u] = f2u(bot);
        /* two-walk sub-segments jump only with |inc1 - inc0| < 64 (7-bit field) */
        int32_t delta = (int32_t)(inc1[u] - inc0[u]);
        (void)delta;
        wd[u] = f2u(top) - f2u(bot);
        efs[u] = ef;
    }
    uint32_t run = 0, r0 = 0, r1 = 0;
    for (int u = U - 1; u >= 0; --u) {
        if (automaton) {
            int empty = u >= nsub;
            rkey[u] = empty ? 1024 : (u == 0 ? 1025 : (valid[u] ? (int)efs[u] : 2048 + u));
        }
    }
    for (int u = U - 1; u >= 0; --u) {
        int end_here = (u == U - 1) || rkey[u + 1] != rkey[u];
        next[u] = end_here ? u + 1 : next[u + 1];
        if (automaton) {
            /* x = this segment, y = the rest of its run */
            uint32_t x0 = valid[u] ? inc0[u] : 0u, x1 = valid[u] ? inc1[u] : 0u;
            uint32_t y0 = end_here ? 0u : r0, y1 = end_here ? 0u : r1;
            r0 = x0 + ((x0 & 1u) ? y1 : y0);
            r1 = x1 + (((1u + x1) & 1u) ? y1 : y0);
            I0[u] = r0;
            I1[u] = r1;
        } else {
            uint32_t own = simple[u] ? inc0[u] : 0u;
            run = end_here ? own : own + run;
            I0[u] = simple[u] ? run : inc0[u];
            I1[u] = simple[u] ? run : inc1[u];
        }
        {   /* jumpable: valid, |inc1 - inc0| < 64, entry increment below 2^23 */
            int32_t dl = (int32_t)(I1[u] - I0[u]);
            if (!(valid[u] && dl >= -64 && dl < 64 && I0[u] < 0x800000u)) wd[u] = 0u;
        }
    }
    uint32_t s = f2u(w0s[0]);
    int u = 1;
    while (u < nsub) {
        ++*steps;
        uint32_t t = s + ((s & 1u) ? I1[u] : I0[u]);
        uint32_t da = s - lo[u], db = t - lo[u];
        if (wd[u] != 0u && (da > db ? da : db) < wd[u]) { s = t; u = next[u]; }
        else {
            ++rfb;
            float acc = u2f(s);
            for (int i = u * sl; i < u * sl + sl; ++i) acc = acc + (i < n ? a[i] : 0.0f);
            s = f2u(acc);
            ++u;
        }
    }
    return u2f(s);
}

static float run_fold(const float *a, int n, long *steps) { return run_fold_k(a, n, steps, 1); }
static long asteps = 0;
static float run_fold_simple(const float *a, int n) { return run_fold_k(a, n, &asteps, 0); }

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
        float r4 = run_fold_simple(a, n);
        if (f2u(r0) != f2u(r4) && !(r0 != r0 && r4 != r4)) {
            printf("MISMATCH run_fold (simple-segment runs) %s row %ld n=%d: seq=%a run=%a\n", what, row, n, r0, r4);
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
    printf("run-jumping resolve (as the kernel): %.2f steps/row, %.2f fallbacks/row; simple-segment runs: %.2f steps/row\n",
           krows ? (double)rsteps / krows : 0.0, krows ? (double)rfb / krows : 0.0, krows ? (double)asteps / krows : 0.0);
    return 0;
}
