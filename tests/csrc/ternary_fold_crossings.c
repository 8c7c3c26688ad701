/*
 * Why the segmented exact fold of the row kernels (kore_amd/csrc/norm.hip)
 * is not used for the f32-activation ternary matmul's fold
 * (kore_amd/csrc/ternary.hip, ternary_f32_pipe_kernel; the reference's
 * compute_row, crates/kore-kernels/src/cpu_ternary_matmul.rs:105-124).
 *
 * The segmented fold jumps a segment in O(1) when the running sum stays in
 * one binade (and, for signed terms, one sign) across it; every segment that
 * leaves its start binade is folded term by term from the exact sum.  For
 * the squares of a row (non-negative terms) the sum crosses ~6 binades after
 * its first segment.  For t * b with trits t (BitLinear weights: w ~ U(-1, 1)
 * packed at threshold 0.3, as crates/kore-nn/src/bit_linear.rs:93-108
 * generates them) and N(0, 1) activations b, the sum is a random walk around
 * zero: this program measures, over seeded rows, how often the exact running
 * sum changes binade or sign, and how many of 64 equal segments leave their
 * start binade -- the segments such a resolve would fold one by one.
 *
 * Usage: ternary_fold_crossings [K] [rows]
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
static uint64_t rs = 88172645463325252ull;
static uint64_t xr(void) { rs ^= rs << 13; rs ^= rs >> 7; rs ^= rs << 17; return rs; }
static double unif(void) { return (double)(xr() >> 11) / 9007199254740992.0; }
static double gauss(void) { double u = unif(), v = unif(); if (u < 1e-300) u = 1e-300; return sqrt(-2 * log(u)) * cos(6.283185307179586 * v); }
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
/* binade key incl. sign: (sign, exponent) */
static int key(float s) { uint32_t u = f2u(s); return (int)(u >> 23); }
int main(int argc, char **argv) {
    int K = argc > 1 ? atoi(argv[1]) : 2560, rows = argc > 2 ? atoi(argv[2]) : 20000;
    double tot_changes = 0, tot_bad = 0, tot_runs = 0, tot_zero = 0;
    float w[8192], b[8192];
    for (int r = 0; r < rows; ++r) {
        float mx = 0;
        for (int i = 0; i < K; ++i) { w[i] = (float)(2 * unif() - 1); if (fabsf(w[i]) > mx) mx = fabsf(w[i]); }
        for (int i = 0; i < K; ++i) { float q = w[i] / mx; w[i] = q > 0.3f ? 1.f : (q < -0.3f ? -1.f : 0.f); b[i] = (float)gauss(); }
        float s = 0; int changes = 0, prev = key(0.0f);
        int L = (K + 63) / 64; int bad = 0, runs = 0, lastkey = -1;
        for (int j = 0; j < 64; ++j) {
            int k0 = key(s), same = 1;
            for (int i = j * L; i < (j + 1) * L && i < K; ++i) {
                if (w[i] != 0.f) s = s + w[i] * b[i];
                int kk = key(s);
                if (kk != prev) { ++changes; prev = kk; }
                if (kk != k0) same = 0;
                if (s == 0.f) ++tot_zero;
            }
            if (!same) ++bad; else if (k0 != lastkey) ++runs;
            lastkey = same ? k0 : -1;
        }
        tot_changes += changes; tot_bad += bad; tot_runs += runs;
    }
    printf("K=%d: %.1f binade/sign changes of the running sum per fold; 64 segments of %d terms: %.1f segments leave their start binade "
           "(folded), %.1f runs of in-binade segments -> ~%.1f resolve steps per fold (unsigned squares: ~6 folds, ~11 steps)\n",
           K, tot_changes / rows, (K + 63) / 64, tot_bad / rows, tot_runs / rows, (tot_bad + tot_runs) / rows);
    return 0;
}
