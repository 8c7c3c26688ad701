/*
 * kore_oracle.h -- CPU restatement of KORE's reference CPU path for the fused
 * layer ops (RMSNorm, SiLU/GELU/SwiGLU, RoPE, embedding gather, BitLinear
 * pre-quant).
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker and the CPU
 * baseline: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg load it.  The product (libkore_hip.so) never links or calls it.
 *
 * Every function follows one reference Rust function, statement for
 * statement, in IEEE binary32 with the same operation order; the file:line
 * of the function it restates is given beside each declaration (paths are
 * relative to the KidIkaros/KORE checkout).  Rust never contracts a*b+c into
 * an FMA and folds iterator sums left to right, so this file is built with
 * -ffp-contract=off -fno-fast-math -fno-builtin and calls glibc libm, which is
 * what Rust's f32::{exp,tanh,sin,cos,powf} resolve to on linux-gnu.
 */
#ifndef KORE_ORACLE_H
#define KORE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* crates/kore-kernels/src/cpu_fused.rs:160-190 (fused_rms_norm); identical
 * arithmetic in crates/kore-edge/src/ops/norm.rs:7-20. */
void kore_oracle_rms_norm_f32(const float *x, const float *gamma, float *y,
                              size_t rows, size_t cols, float eps);

/* crates/kore-nn/src/activations.rs:14-32 (gelu, tanh form). */
void kore_oracle_gelu_f32(const float *x, float *y, size_t n);

/* crates/kore-nn/src/activations.rs:35-45 (silu); same formula as
 * crates/kore-edge/src/ops/activation.rs:21-26. */
void kore_oracle_silu_f32(const float *x, float *y, size_t n);

/* crates/kore-core/src/ops/arithmetic.rs:482-509 (binary_op, same-shape fast
 * path, op = a*b).  nthreads > 1 splits the index range like rayon's
 * par_iter_mut; the result does not depend on the split. */
void kore_oracle_mul_f32(const float *a, const float *b, float *out, size_t n,
                         int nthreads);

/* SwiGLU as the reference composes it: silu(gate) (activations.rs:35-45)
 * followed by Tensor::mul (arithmetic.rs:76-95); see
 * crates/kore-serve/src/layered/engine.rs:633-643 and
 * crates/kore-edge/src/runtime.rs:253-255.  `tmp` holds the silu tensor. */
void kore_oracle_swiglu_f32(const float *gate, const float *up, float *out,
                            float *tmp, size_t n, int mul_threads);

/* crates/kore-serve/src/layered/engine.rs:694-700 (precompute_rope_inv_freq):
 * inv_freq[i] = 1 / base^(2i/head_dim), i < head_dim/2. */
void kore_oracle_rope_inv_freq_f32(float *inv_freq, size_t head_dim, float base);

/* crates/kore-edge/src/ops/rope.rs:9-36 (apply_rope, half-split pairs
 * (i, i+D/2), in place on [seq_len, n_heads, head_dim]). */
void kore_oracle_rope_f32(float *data, size_t seq_len, size_t n_heads,
                          size_t head_dim, size_t start_pos, float base);

/* crates/kore-serve/src/layered/engine.rs:706-727 (apply_rope, interleaved
 * pairs (2i, 2i+1), inv_freq table), applied in place to every head of a
 * [seq_len, n_heads, head_dim] buffer. */
void kore_oracle_rope_interleaved_f32(float *data, size_t seq_len,
                                      size_t n_heads, size_t head_dim,
                                      size_t start_pos, const float *inv_freq);

/* crates/kore-edge/src/ops/embedding.rs:8-27 and
 * crates/kore-nn/src/embedding.rs:55-72: out[t,:] = table[id_t,:] when
 * id_t < vocab (ids read as unsigned 32-bit), else a zero row. */
void kore_oracle_embedding_f32(const float *table, const uint32_t *ids,
                               float *out, size_t n_ids, size_t vocab,
                               size_t dim);

/* crates/kore-nn/src/embedding.rs:91-98 (Embedding::forward): ids arrive as
 * f32 and are converted with Rust's `v as usize` (truncation toward zero;
 * NaN and negatives saturate to 0, values >= 2^64 to usize::MAX), then
 * looked up as Embedding::lookup (:55-72): id < vocab copies the row, else a
 * zero row. */
void kore_oracle_embedding_forward_f32(const float *table, const float *ids,
                                       float *out, size_t n_ids, size_t vocab,
                                       size_t dim);

/* Rust's `v as usize` for an f32 on a 64-bit target (saturating cast). */
uint64_t kore_oracle_f32_as_usize(float v);

/* crates/kore-serve/src/layered/engine.rs:828-842 (the serving path's silu,
 * which apply_transformer_block :640 composes with Tensor::mul):
 * v >= 0: v / (1 + exp(-v)); else e = exp(v), (v * e) / (1 + e). */
void kore_oracle_silu_stable_f32(const float *x, float *y, size_t n);

/* engine.rs:640-643: silu_stable(gate) then Tensor::mul(up). */
void kore_oracle_swiglu_serve_f32(const float *gate, const float *up,
                                  float *out, size_t n);

/* BitLinear pre-quant.  The reference has no such function; this is the
 * composition the build defines:
 *   xn    = fused_rms_norm(x, gamma, eps)   (cpu_fused.rs:160-190)
 *   amax  = fold(0, f32::max) of |xn|       (kore-btes/src/quantize.rs:9)
 *   amax  = 1.0 if amax < 1e-8              (kore-btes/src/quantize.rs:10)
 *   q     = ((xn*127)/amax).round().clamp(-128,127) as i8
 *           (f32::round = ties away from zero; `as i8` saturates, NaN -> 0)
 *   scale = amax / 127                      (x ~= q * scale)            */
void kore_oracle_rms_norm_quant_i8(const float *x, const float *gamma,
                                   int8_t *q, float *scale, size_t rows,
                                   size_t cols, float eps);

/* RMSNorm with a SiLU gate, y = RMSNorm(x) * silu(z): the CPU definition of
 * fused_rms_norm_silu_gate_f32 in crates/kore-kernels/src/cpu_fused.rs:451-483
 * (x_hat = (x*inv)*g with the sequential sum of squares; silu(z) =
 * z/(1+exp(-z)); y = x_hat * silu(z)); the CUDA kernel is
 * crates/kore-kernels/src/cuda/kernels/fused_norm_proj.cu:204-253. */
void kore_oracle_rms_norm_silu_gate_f32(const float *x, const float *gamma,
                                        const float *z, float *y, size_t rows,
                                        size_t cols, float eps);

/* One element of the pre-quant code: the shared definition used above.  */
int8_t kore_oracle_quant_code(float xn, float amax_guarded);

/* crates/kore-kernels/src/cpu_fused.rs:195-231 (fused_softmax): max by an
 * f32::max fold from -inf (NaN elements skipped), e = exp(x - max), sum folded
 * left to right, y = e * (1 / sum). */
void kore_oracle_softmax_f32(const float *x, float *y, size_t rows, size_t cols);

/* crates/kore-kernels/src/cuda/kernels/softmax.cu:88-157 (softmax_causal_f32;
 * GPU-only in the reference, no CPU twin): row r keeps columns
 * c < seq_offset + r + 1, the rest are -inf in the max and 0 in the output;
 * inv_sum = sum > 0 ? 1/sum : 0.  Sums are folded left to right here (the CUDA
 * kernel uses a tree; both are within the f32 tolerance). */
void kore_oracle_softmax_causal_f32(const float *x, float *y, size_t rows,
                                    size_t cols, size_t seq_offset);

/* crates/kore-kernels/src/cpu_fused_backward.rs:86-115
 * (fused_softmax_backward): dot = sum(y*dy) folded left to right,
 * dx = y * (dy - dot). */
void kore_oracle_softmax_backward_f32(const float *dy, const float *y,
                                      float *dx, size_t rows, size_t cols);

/* crates/kore-kernels/src/cpu_fused_backward.rs:130-170
 * (fused_cross_entropy_backward): per row the softmax is formed as in
 * fused_softmax, grad = e * (inv_sum * inv_batch), inv_batch = 1/batch (f32),
 * then grad[t] -= inv_batch, t = targets[b] as usize (Rust's saturating
 * float-to-int cast).  Where the reference would panic (t >= num_classes)
 * this restatement, like the device op, subtracts nothing. */
void kore_oracle_cross_entropy_backward_f32(const float *logits,
                                            const float *targets, float *grad,
                                            size_t batch, size_t num_classes);

/* crates/kore-kernels/src/cpu_fused_backward.rs:20-81
 * (fused_rms_norm_backward): per row sum_sq, inv_rms = 1/sqrt(sum_sq/d + eps);
 * dgamma[i] += (go*x)*inv_rms (rows in order);
 * dot = sum((x*go)*g); coeff = (dot*inv_rms) / (sum_sq + eps*d);
 * dx = ((g*inv_rms)*go) - coeff*x.  dgamma is overwritten. */
void kore_oracle_rms_norm_backward_f32(const float *dy, const float *x,
                                       const float *gamma, float *dx,
                                       float *dgamma, size_t rows, size_t cols,
                                       float eps);


/* ---------------------------------------------------------------- ternary
 * Base-243 packed ternary weights: 5 trits per byte, least significant
 * base-3 digit first, digit 0/1/2 = -1/0/+1 (crates/kore-btes/src/encoder.rs). */

/* crates/kore-btes/src/encoder.rs:89-95 (decode_trits; LUT :50-70). */
void kore_oracle_decode_trits(uint8_t byte, int8_t out[5]);

/* crates/kore-btes/src/encoder.rs:73-86 (encode_trits). */
uint8_t kore_oracle_encode_trits(const int8_t t[5]);

/* crates/kore-kernels/src/cpu_ternary_matmul.rs:198-240
 * (pack_weights_ternary): per-row absmax scale (1.0 below 1e-8), trit =
 * sign(w/scale) where |w/scale| > threshold.  packed[m, ceil(k/5)]. */
void kore_oracle_pack_weights_ternary(const float *w, size_t m, size_t k,
                                      float threshold, uint8_t *packed,
                                      float *scales);

/* crates/kore-kernels/src/cpu_ternary_matmul.rs:29-124 (ternary_matmul) ==
 * crates/kore-edge/src/ops/matmul.rs:49-93 (matmul_ternary):
 * c[m, n] = scale[m] * sum_k trit[m, k] * b[k, n], b row-major [k, n],
 * summed in k order, zero trits skipped. */
void kore_oracle_ternary_matmul_f32(const uint8_t *a_packed,
                                    const float *a_scales, const float *b,
                                    float *c, size_t m, size_t n, size_t k);

/* BitLinear matmul on the pre-quant codes (no single reference function):
 * c[m, n] = ((float)(sum_k trit[m, k] * q[n, k]) * a_scales[m]) * q_scales[n],
 * the integer dot product exact, the epilogue of
 * crates/kore-kernels/src/cpu_ternary_matmul.rs:188 (ternary_ternary_matmul). */
void kore_oracle_ternary_matmul_i8(const uint8_t *a_packed,
                                   const float *a_scales, const int8_t *q,
                                   const float *q_scales, float *c, size_t m,
                                   size_t n, size_t k);

#ifdef __cplusplus
}
#endif

#endif /* KORE_ORACLE_H */
