/*
 * kore_oracle.c -- CPU restatement of KORE's reference CPU path for the fused
 * layer ops.  TEST INFRASTRUCTURE ONLY (the parity checker and the CPU
 * baseline); the product library never links it.
 *
 * Build: see oracle/Makefile (gcc -O2 -ffp-contract=off -fno-fast-math
 * -fno-builtin, glibc libm).  Each function names the reference Rust function
 * it restates; the declarations in kore_oracle.h carry the file:line.
 */
#include "kore_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <pthread.h>
#include <string.h>

/* cpu_fused.rs:175-187: per row, sum_sq is `row.iter().map(|x| x*x).sum()`,
 * a left-to-right f32 fold; rms = sqrt(sum_sq / D + eps); inv = 1/rms;
 * y = row[i] * inv * g[i] evaluated as (row[i]*inv)*g[i]. */
void kore_oracle_rms_norm_f32(const float *x, const float *gamma, float *y,
                              size_t rows, size_t cols, float eps) {
    for (size_t r = 0; r < rows; ++r) {
        const float *row = x + r * cols;
        float *out = y + r * cols;
        float sum_sq = 0.0f;
        for (size_t i = 0; i < cols; ++i) {
            float sq = row[i] * row[i];
            sum_sq = sum_sq + sq;
        }
        float rms = sqrtf(sum_sq / (float)cols + eps);
        float inv_rms = 1.0f / rms;
        for (size_t i = 0; i < cols; ++i) {
            float t = row[i] * inv_rms;
            out[i] = t * gamma[i];
        }
    }
}

/* activations.rs:23-29.  FRAC_2_SQRT_PI * FRAC_1_SQRT_2 is a product of two
 * f32 constants, folded in f32 (0x3F4C422A); 0.044715*x*x*x associates left. */
void kore_oracle_gelu_f32(const float *x, float *y, size_t n) {
    const float frac_2_sqrt_pi = 1.12837916709551257390f;
    const float frac_1_sqrt_2 = 0.707106781186547524401f;
    const float k = frac_2_sqrt_pi * frac_1_sqrt_2;
    for (size_t i = 0; i < n; ++i) {
        float v = x[i];
        float cube = ((0.044715f * v) * v) * v;
        float inner = k * (v + cube);
        float half_x = 0.5f * v;
        y[i] = half_x * (1.0f + tanhf(inner));
    }
}

/* activations.rs:43: x / (1.0 + (-x).exp()). */
void kore_oracle_silu_f32(const float *x, float *y, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        float v = x[i];
        y[i] = v / (1.0f + expf(-v));
    }
}

struct mul_job {
    const float *a, *b;
    float *out;
    size_t lo, hi;
};

static void *mul_worker(void *arg) {
    struct mul_job *j = (struct mul_job *)arg;
    for (size_t i = j->lo; i < j->hi; ++i) j->out[i] = j->a[i] * j->b[i];
    return NULL;
}

/* arithmetic.rs:499-509: result[i] = a[i] * b[i], rayon-parallel above
 * PAR_THRESHOLD; element-wise, so the split never changes a bit. */
void kore_oracle_mul_f32(const float *a, const float *b, float *out, size_t n,
                         int nthreads) {
    if (nthreads <= 1 || n < 8192) {
        for (size_t i = 0; i < n; ++i) out[i] = a[i] * b[i];
        return;
    }
    if (nthreads > 256) nthreads = 256;
    pthread_t tid[256];
    struct mul_job jobs[256];
    size_t chunk = (n + (size_t)nthreads - 1) / (size_t)nthreads;
    int started = 0;
    for (int t = 0; t < nthreads; ++t) {
        size_t lo = (size_t)t * chunk, hi = lo + chunk;
        if (lo >= n) break;
        if (hi > n) hi = n;
        jobs[t].a = a; jobs[t].b = b; jobs[t].out = out;
        jobs[t].lo = lo; jobs[t].hi = hi;
        if (pthread_create(&tid[t], NULL, mul_worker, &jobs[t]) != 0) {
            mul_worker(&jobs[t]);
            tid[t] = 0;
        }
        started = t + 1;
    }
    for (int t = 0; t < started; ++t)
        if (tid[t]) pthread_join(tid[t], NULL);
}

/* engine.rs:633-643: silu(gate) into a fresh tensor, then Tensor::mul. */
void kore_oracle_swiglu_f32(const float *gate, const float *up, float *out,
                            float *tmp, size_t n, int mul_threads) {
    kore_oracle_silu_f32(gate, tmp, n);
    kore_oracle_mul_f32(tmp, up, out, n, mul_threads);
}

/* engine.rs:694-700: 1.0 / base.powf(2.0 * i as f32 / head_dim as f32). */
void kore_oracle_rope_inv_freq_f32(float *inv_freq, size_t head_dim, float base) {
    size_t half = head_dim / 2;
    for (size_t i = 0; i < half; ++i) {
        float e = (2.0f * (float)i) / (float)head_dim;
        inv_freq[i] = 1.0f / powf(base, e);
    }
}

/* rope.rs:18-35.  freq is recomputed per element with the same expression as
 * the inv_freq table above; angle = (start_pos + pos) as f32 * freq. */
void kore_oracle_rope_f32(float *data, size_t seq_len, size_t n_heads,
                          size_t head_dim, size_t start_pos, float base) {
    size_t half = head_dim / 2;
    for (size_t pos = 0; pos < seq_len; ++pos) {
        float abs_pos = (float)(start_pos + pos);
        for (size_t h = 0; h < n_heads; ++h) {
            size_t off = pos * n_heads * head_dim + h * head_dim;
            for (size_t i = 0; i < half; ++i) {
                float e = (2.0f * (float)i) / (float)head_dim;
                float freq = 1.0f / powf(base, e);
                float angle = abs_pos * freq;
                float c = cosf(angle);
                float s = sinf(angle);
                float x0 = data[off + i];
                float x1 = data[off + half + i];
                float a0 = x0 * c, b0 = x1 * s;
                float a1 = x0 * s, b1 = x1 * c;
                data[off + i] = a0 - b0;
                data[off + half + i] = a1 + b1;
            }
        }
    }
}

/* engine.rs:715-724, per head: pairs (2*pair, 2*pair+1) of each head vector,
 * angle = abs_pos * inv_freq[pair]. */
void kore_oracle_rope_interleaved_f32(float *data, size_t seq_len,
                                      size_t n_heads, size_t head_dim,
                                      size_t start_pos, const float *inv_freq) {
    size_t half = head_dim / 2;
    for (size_t pos = 0; pos < seq_len; ++pos) {
        float abs_pos = (float)(start_pos + pos);
        for (size_t h = 0; h < n_heads; ++h) {
            float *v = data + pos * n_heads * head_dim + h * head_dim;
            for (size_t p = 0; p < half; ++p) {
                float angle = abs_pos * inv_freq[p];
                float c = cosf(angle);
                float s = sinf(angle);
                float x0 = v[2 * p];
                float x1 = v[2 * p + 1];
                float a0 = x0 * c, b0 = x1 * s;
                float a1 = x0 * s, b1 = x1 * c;
                v[2 * p] = a0 - b0;
                v[2 * p + 1] = a1 + b1;
            }
        }
    }
}

/* embedding.rs (edge) :16-26: copy the row when id < vocab, else zeros. */
void kore_oracle_embedding_f32(const float *table, const uint32_t *ids,
                               float *out, size_t n_ids, size_t vocab,
                               size_t dim) {
    for (size_t t = 0; t < n_ids; ++t) {
        size_t id = (size_t)ids[t];
        float *dst = out + t * dim;
        if (id < vocab) {
            memcpy(dst, table + id * dim, dim * sizeof(float));
        } else {
            for (size_t i = 0; i < dim; ++i) dst[i] = 0.0f;
        }
    }
}

/* Rust `f32 as usize` (64-bit): saturating float-to-int cast, NaN -> 0. */
uint64_t kore_oracle_f32_as_usize(float v) {
    if (v != v) return 0;
    if (v <= 0.0f) return 0;
    if (v >= 18446744073709551616.0f) return UINT64_MAX;
    return (uint64_t)v; /* C truncates toward zero, in range here */
}

/* embedding.rs:91-98: ids.iter().map(|&v| v as usize), then lookup :55-72. */
void kore_oracle_embedding_forward_f32(const float *table, const float *ids,
                                       float *out, size_t n_ids, size_t vocab,
                                       size_t dim) {
    for (size_t t = 0; t < n_ids; ++t) {
        uint64_t id = kore_oracle_f32_as_usize(ids[t]);
        float *dst = out + t * dim;
        if (id < (uint64_t)vocab) {
            memcpy(dst, table + id * dim, dim * sizeof(float));
        } else {
            for (size_t i = 0; i < dim; ++i) dst[i] = 0.0f;
        }
    }
}

/* engine.rs:831-839: two branches on the sign of v. */
void kore_oracle_silu_stable_f32(const float *x, float *y, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        float v = x[i];
        if (v >= 0.0f) {
            y[i] = v / (1.0f + expf(-v));
        } else {
            float exp_v = expf(v);
            y[i] = (v * exp_v) / (1.0f + exp_v);
        }
    }
}

/* engine.rs:640-643: gate_activated = silu(&gate); gate_activated.mul(&up). */
void kore_oracle_swiglu_serve_f32(const float *gate, const float *up,
                                  float *out, size_t n) {
    kore_oracle_silu_stable_f32(gate, out, n);
    for (size_t i = 0; i < n; ++i) out[i] = out[i] * up[i];
}

/* ((xn * 127.0) / amax).round().clamp(-128.0, 127.0) as i8.
 * f32::round rounds half away from zero (= C roundf); f32::clamp keeps NaN;
 * `as i8` saturates and maps NaN to 0. */
int8_t kore_oracle_quant_code(float xn, float amax_guarded) {
    float t = (xn * 127.0f) / amax_guarded;
    float r = roundf(t);
    if (r != r) return 0;
    if (r < -128.0f) r = -128.0f;
    if (r > 127.0f) r = 127.0f;
    return (int8_t)(int)r;
}

/* f32::max: returns the non-NaN operand when exactly one is NaN. */
static float rust_fmax(float a, float b) {
    if (a != a) return b;
    if (b != b) return a;
    return a > b ? a : b;
}

void kore_oracle_rms_norm_quant_i8(const float *x, const float *gamma,
                                   int8_t *q, float *scale, size_t rows,
                                   size_t cols, float eps) {
    for (size_t r = 0; r < rows; ++r) {
        const float *row = x + r * cols;
        float sum_sq = 0.0f;
        for (size_t i = 0; i < cols; ++i) {
            float sq = row[i] * row[i];
            sum_sq = sum_sq + sq;
        }
        float rms = sqrtf(sum_sq / (float)cols + eps);
        float inv_rms = 1.0f / rms;
        float amax = 0.0f;
        for (size_t i = 0; i < cols; ++i) {
            float xn = (row[i] * inv_rms) * gamma[i];
            amax = rust_fmax(amax, fabsf(xn));
        }
        float a = amax < 1e-8f ? 1.0f : amax;
        for (size_t i = 0; i < cols; ++i) {
            float xn = (row[i] * inv_rms) * gamma[i];
            q[r * cols + i] = kore_oracle_quant_code(xn, a);
        }
        scale[r] = a / 127.0f;
    }
}

/* cpu_fused.rs:459-473: sum_sq fold, inv_rms = 1/sqrt(sum_sq/cols + eps),
 * x_hat = row[c]*inv_rms*gamma[c], y = x_hat * silu(z). */
void kore_oracle_rms_norm_silu_gate_f32(const float *x, const float *gamma,
                                        const float *z, float *y, size_t rows,
                                        size_t cols, float eps) {
    for (size_t r = 0; r < rows; ++r) {
        const float *row = x + r * cols;
        float sum_sq = 0.0f;
        for (size_t i = 0; i < cols; ++i) {
            float sq = row[i] * row[i];
            sum_sq = sum_sq + sq;
        }
        float rms = sqrtf(sum_sq / (float)cols + eps);
        float inv_rms = 1.0f / rms;
        for (size_t i = 0; i < cols; ++i) {
            float xh = (row[i] * inv_rms) * gamma[i];
            float zv = z[r * cols + i];
            float sz = zv / (1.0f + expf(-zv));
            y[r * cols + i] = xh * sz;
        }
    }
}

/* cpu_fused.rs:208-227. */
void kore_oracle_softmax_f32(const float *x, float *y, size_t rows, size_t cols) {
    for (size_t r = 0; r < rows; ++r) {
        const float *row = x + r * cols;
        float *out = y + r * cols;
        float max_val = -INFINITY;
        for (size_t i = 0; i < cols; ++i) max_val = rust_fmax(max_val, row[i]);
        float sum = 0.0f;
        for (size_t i = 0; i < cols; ++i) {
            float e = expf(row[i] - max_val);
            out[i] = e;
            sum = sum + e;
        }
        float inv_sum = 1.0f / sum;
        for (size_t i = 0; i < cols; ++i) out[i] = out[i] * inv_sum;
    }
}

/* softmax.cu:101-156 with sequential sums; fmaxf is IEEE maxNum like f32::max. */
void kore_oracle_softmax_causal_f32(const float *x, float *y, size_t rows,
                                    size_t cols, size_t seq_offset) {
    for (size_t r = 0; r < rows; ++r) {
        const float *row = x + r * cols;
        float *out = y + r * cols;
        size_t limit = seq_offset + r + 1;
        float max_val = -INFINITY;
        for (size_t c = 0; c < cols; ++c) {
            float v = c < limit ? row[c] : -INFINITY;
            max_val = rust_fmax(max_val, v);
        }
        float sum = 0.0f;
        for (size_t c = 0; c < cols; ++c) {
            float v = c < limit ? expf(row[c] - max_val) : 0.0f;
            out[c] = v;
            sum = sum + v;
        }
        float inv_sum = sum > 0.0f ? 1.0f / sum : 0.0f;
        for (size_t c = 0; c < cols; ++c) out[c] = out[c] * inv_sum;
    }
}

/* cpu_fused_backward.rs:102-112. */
void kore_oracle_softmax_backward_f32(const float *dy, const float *y,
                                      float *dx, size_t rows, size_t cols) {
    for (size_t r = 0; r < rows; ++r) {
        const float *yr = y + r * cols;
        const float *dyr = dy + r * cols;
        float dot = 0.0f;
        for (size_t i = 0; i < cols; ++i) dot = dot + yr[i] * dyr[i];
        for (size_t i = 0; i < cols; ++i) dx[r * cols + i] = yr[i] * (dyr[i] - dot);
    }
}

/* cpu_fused_backward.rs:43-78. */
void kore_oracle_rms_norm_backward_f32(const float *dy, const float *x,
                                       const float *gamma, float *dx,
                                       float *dgamma, size_t rows, size_t cols,
                                       float eps) {
    for (size_t i = 0; i < cols; ++i) dgamma[i] = 0.0f;
    for (size_t r = 0; r < rows; ++r) {
        const float *xr = x + r * cols;
        const float *gr = dy + r * cols;
        float sum_sq = 0.0f;
        for (size_t i = 0; i < cols; ++i) sum_sq = sum_sq + xr[i] * xr[i];
        float rms = sqrtf(sum_sq / (float)cols + eps);
        float inv_rms = 1.0f / rms;
        for (size_t i = 0; i < cols; ++i) dgamma[i] = dgamma[i] + (gr[i] * xr[i]) * inv_rms;
        float dot = 0.0f;
        for (size_t i = 0; i < cols; ++i) dot = dot + (xr[i] * gr[i]) * gamma[i];
        float coeff = (dot * inv_rms) / (sum_sq + eps * (float)cols);
        for (size_t i = 0; i < cols; ++i) {
            float a = (gamma[i] * inv_rms) * gr[i];
            float b = coeff * xr[i];
            dx[r * cols + i] = a - b;
        }
    }
}

/* Rust `f32 as usize`: NaN -> 0, negatives -> 0, truncation, saturating. */
static size_t rust_f32_as_usize(float t) {
    if (!(t >= 1.0f)) return 0;
    if (t >= 18446744073709551616.0f) return (size_t)-1;
    return (size_t)t;
}

/* cpu_fused_backward.rs:143-168. */
void kore_oracle_cross_entropy_backward_f32(const float *logits,
                                            const float *targets, float *grad,
                                            size_t batch, size_t num_classes) {
    float inv_batch = 1.0f / (float)batch;
    for (size_t b = 0; b < batch; ++b) {
        const float *row = logits + b * num_classes;
        float *g = grad + b * num_classes;
        size_t target_idx = rust_f32_as_usize(targets[b]);
        float max_val = -INFINITY;
        for (size_t i = 0; i < num_classes; ++i) max_val = rust_fmax(max_val, row[i]);
        float sum = 0.0f;
        for (size_t i = 0; i < num_classes; ++i) {
            float e = expf(row[i] - max_val);
            g[i] = e;
            sum = sum + e;
        }
        float inv_sum = 1.0f / sum;
        for (size_t i = 0; i < num_classes; ++i) g[i] = g[i] * (inv_sum * inv_batch);
        if (target_idx < num_classes) g[target_idx] = g[target_idx] - inv_batch;
    }
}

/* ------------------------------------------------------------ ternary */

void kore_oracle_decode_trits(uint8_t byte, int8_t out[5]) {
    /* crates/kore-btes/src/encoder.rs:50-70 (TERNARY_DECODE_LUT) and :89-95
     * (decode_trits): base-3 digits, least significant first, digit 0 ->
     * Neg, 1 -> Zero, 2 -> Pos; bytes 243..255 decode to five zeros. */
    if (byte >= 243) {
        for (int j = 0; j < 5; ++j) out[j] = 0;
        return;
    }
    unsigned v = byte;
    for (int j = 0; j < 5; ++j) {
        out[j] = (int8_t)((int)(v % 3u) - 1);
        v /= 3u;
    }
}

uint8_t kore_oracle_encode_trits(const int8_t t[5]) {
    /* crates/kore-btes/src/encoder.rs:73-86: digit (t + 1) times 3^j, with
     * the reference's u8 arithmetic (the sum of 5 digits <= 2*121 fits). */
    unsigned val = 0, mul = 1;
    for (int j = 0; j < 5; ++j) {
        val += (unsigned)(t[j] + 1) * mul;
        mul *= 3u;
    }
    return (uint8_t)val;
}

static float rust_fmax_t(float a, float b) {
    if (a != a) return b;
    if (b != b) return a;
    return a > b ? a : b;
}

void kore_oracle_pack_weights_ternary(const float *w, size_t m, size_t k,
                                      float threshold, uint8_t *packed,
                                      float *scales) {
    /* crates/kore-kernels/src/cpu_ternary_matmul.rs:198-240 */
    const size_t kp = (k + 4) / 5;
    for (size_t row = 0; row < m; ++row) {
        const float *rd = w + row * k;
        float abs_max = 0.0f;
        for (size_t i = 0; i < k; ++i) abs_max = rust_fmax_t(abs_max, fabsf(rd[i]));
        const float scale = abs_max < 1e-8f ? 1.0f : abs_max;
        scales[row] = scale;
        for (size_t b = 0; b < kp; ++b) {
            int8_t block[5] = {0, 0, 0, 0, 0};
            for (size_t j = 0; j < 5 && b * 5 + j < k; ++j) {
                const float nv = rd[b * 5 + j] / scale;
                block[j] = nv > threshold ? 1 : (nv < -threshold ? -1 : 0);
            }
            packed[row * kp + b] = kore_oracle_encode_trits(block);
        }
    }
}

/* unpack_row_trits (cpu_ternary_matmul.rs:91-101): decode every byte of
 * the packed row and keep the first k trits. */
static void unpack_row_trits(const uint8_t *row, size_t k, int8_t *out) {
    int8_t t5[5];
    for (size_t b = 0; b * 5 < k; ++b) {
        kore_oracle_decode_trits(row[b], t5);
        for (size_t j = 0; j < 5 && b * 5 + j < k; ++j) out[b * 5 + j] = t5[j];
    }
}

void kore_oracle_ternary_matmul_f32(const uint8_t *a_packed,
                                    const float *a_scales, const float *b,
                                    float *c, size_t m, size_t n, size_t k) {
    /* crates/kore-kernels/src/cpu_ternary_matmul.rs:29-124 (ternary_matmul:
     * unpack_row_trits :91-101, compute_row :105-124); the same loop is
     * crates/kore-edge/src/ops/matmul.rs:49-93.  Per output row: c = 0; for
     * each k in order, skip zero trits, c[col] += t * b[k, col]; then
     * c[col] *= scale. */
    const size_t kp = (k + 4) / 5;
    int8_t *tr = (int8_t *)malloc(k ? k : 1);
    for (size_t row = 0; row < m; ++row) {
        unpack_row_trits(a_packed + row * kp, k, tr);
        float *cr = c + row * n;
        for (size_t col = 0; col < n; ++col) cr[col] = 0.0f;
        for (size_t ki = 0; ki < k; ++ki) {
            const int8_t t = tr[ki];
            if (t == 0) continue;
            const float tf = (float)t;
            const float *br = b + ki * n;
            for (size_t col = 0; col < n; ++col) cr[col] = cr[col] + tf * br[col];
        }
        const float s = a_scales[row];
        for (size_t col = 0; col < n; ++col) cr[col] = cr[col] * s;
    }
    free(tr);
}

void kore_oracle_ternary_matmul_i8(const uint8_t *a_packed,
                                   const float *a_scales, const int8_t *q,
                                   const float *q_scales, float *c, size_t m,
                                   size_t n, size_t k) {
    /* The BitLinear matmul on pre-quant codes: integer dot products of the
     * decoded trits (unpacked once per row, cpu_ternary_matmul.rs:91-101)
     * with the int8 codes q[n, :] (exact in 64-bit), then the ternary-ternary
     * epilogue of crates/kore-kernels/src/cpu_ternary_matmul.rs:188
     * (ternary_ternary_matmul, `int_acc as f32 * a_scale * b_scale`) with the
     * code row's scale in place of b_scale. */
    const size_t kp = (k + 4) / 5;
    int8_t *tr = (int8_t *)malloc(k ? k : 1);
    for (size_t row = 0; row < m; ++row) {
        unpack_row_trits(a_packed + row * kp, k, tr);
        for (size_t col = 0; col < n; ++col) {
            const int8_t *qr = q + col * k;
            long long acc = 0;
            for (size_t ki = 0; ki < k; ++ki) acc += (long long)tr[ki] * (long long)qr[ki];
            c[row * n + col] = ((float)acc * a_scales[row]) * q_scales[col];
        }
    }
    free(tr);
}
