/*
 * kore_hip.h -- C ABI of libkore_hip.so: KORE's fused layer ops as
 * hand-written gfx950 (MI355X) HIP kernels.
 *
 * Contract shared by every entry point:
 *   - All tensors are row-major, contiguous, little-endian, resident in device
 *     memory (hipMalloc or any allocator that hands out device pointers).  The
 *     caller owns every buffer: no entry point allocates, frees or copies
 *     between host and device, so nothing hidden lands in a timed region.
 *   - `stream` is a hipStream_t (NULL = the default stream).  Work is only
 *     enqueued; nothing synchronises.  The caller syncs before reading results.
 *   - Return value: 0 on success; a negative KORE_HIP_ERR_* code for a bad
 *     argument (checked on the host before anything is launched); a positive
 *     hipError_t value when the launch itself fails.  No entry point aborts.
 *   - A call with zero elements of work returns 0 and launches nothing, as the
 *     reference CPU ops return empty tensors.
 *   - Pointers that are not 16-byte aligned, or rows whose length is not a
 *     multiple of 4 floats, take a scalar path with identical results (the
 *     ternary matmuls read unaligned packed rows and code rows through
 *     dword windows in their vector kernels; only an output that is not
 *     4-byte aligned, or K = 0, takes their one-thread-per-output path).
 *   - Entry points are reentrant and keep no state between calls.
 *
 * Each declaration names the reference function it replaces (paths relative
 * to the KidIkaros/KORE tree) and what its results match: "bit-exact" means
 * byte-identical to the reference CPU function on the same input; "f32 tol"
 * means |gpu - ref| <= 1e-6 or <= 1e-5 * |ref| per element.
 */
#ifndef KORE_HIP_H
#define KORE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *kore_stream_t; /* hipStream_t */

#define KORE_HIP_OK 0
#define KORE_HIP_ERR_NULL_PTR (-1)  /* a required pointer is NULL        */
#define KORE_HIP_ERR_BAD_DIM (-2)   /* a dimension is invalid (odd head_dim, cols == 0 with rows > 0, ...) */
#define KORE_HIP_ERR_OVERFLOW (-3)  /* an element count overflows 64-bit or exceeds the kernel's index range */
#define KORE_HIP_ERR_ALIAS (-4)     /* input/output overlap the op does not allow */
#define KORE_HIP_ERR_SCRATCH (-5)   /* the work needs more scratch than the library's fixed array holds */

/* Library version as 10000*major + 100*minor + patch. */
int kore_hip_version(void);

/* Static text for a status code (never NULL). */
const char *kore_hip_status_string(int status);

/* ---------------------------------------------------------------- RMSNorm
 * out[r, :] = (x[r, :] * inv_rms_r) * weight[:],
 * inv_rms_r = 1 / sqrt((sum_i x[r,i]^2 summed left to right) / cols + eps).
 * Replaces cuda_rms_norm_f32 (crates/kore-kernels/src/cuda/ops.rs:517-541)
 * and is the device twin of kore_kernels::cpu_fused::fused_rms_norm
 * (crates/kore-kernels/src/cpu_fused.rs:160-190).  Bit-exact: the row sum
 * keeps the reference's sequential f32 order.  out may equal x. */
int kore_hip_rms_norm_f32(const float *x, const float *weight, float *out,
                          uint64_t rows, uint64_t cols, float eps,
                          kore_stream_t stream);

/* ------------------------------------------------------------ activations
 * out[i] = gelu_tanh(x[i]).  Replaces cuda_gelu_f32
 * (crates/kore-kernels/src/cuda/ops.rs:197-204); twin of
 * kore_nn::activations::gelu (crates/kore-nn/src/activations.rs:14-32).
 * f32 tol.  out may equal x. */
int kore_hip_gelu_f32(const float *x, float *out, uint64_t n,
                      kore_stream_t stream);

/* out[i] = x[i] / (1 + exp(-x[i])).  Replaces cuda_silu_f32
 * (crates/kore-kernels/src/cuda/ops.rs:206-213); twin of
 * kore_nn::activations::silu (crates/kore-nn/src/activations.rs:35-45).
 * f32 tol.  out may equal x. */
int kore_hip_silu_f32(const float *x, float *out, uint64_t n,
                      kore_stream_t stream);

/* out[i] = a[i] * b[i].  Replaces cuda_mul_f32
 * (crates/kore-kernels/src/cuda/ops.rs:100-108); twin of Tensor::mul's
 * same-shape path (crates/kore-core/src/ops/arithmetic.rs:482-509).
 * Bit-exact.  out may equal a or b. */
int kore_hip_mul_f32(const float *a, const float *b, float *out, uint64_t n,
                     kore_stream_t stream);

/* out[i] = silu(gate[i]) * up[i] in one HBM pass.  Replaces the reference's
 * two-op composition silu(gate) then mul(up)
 * (crates/kore-serve/src/layered/engine.rs:633-643,
 *  crates/kore-edge/src/runtime.rs:253-255).  f32 tol.  out may equal gate
 * or up. */
int kore_hip_swiglu_f32(const float *gate, const float *up, float *out,
                        uint64_t n, kore_stream_t stream);

/* ------------------------------------------------------------------- RoPE
 * Host helper (no device work): inv_freq[i] = 1 / base^((2i)/head_dim) for
 * i < head_dim/2, written to HOST memory.  The caller uploads it once per
 * (head_dim, base).  Same expression as precompute_rope_inv_freq
 * (crates/kore-serve/src/layered/engine.rs:694-700) and the per-element freq
 * of kore_edge::ops::rope::apply_rope (crates/kore-edge/src/ops/rope.rs:24);
 * it plays the role of cuda_rope_freqs_f32
 * (crates/kore-kernels/src/cuda/ops.rs:549-567). */
int kore_hip_rope_inv_freq_f32(float *inv_freq_host, uint32_t head_dim,
                               float base);

/* In-place rotary embedding of data[batch, seq_len, num_heads, head_dim] at
 * positions start_pos + s (the same for every batch entry).
 * interleaved = 0: pairs (i, i + head_dim/2), as kore_edge apply_rope
 *   (crates/kore-edge/src/ops/rope.rs:9-36) and the CUDA rope_f32 kernel
 *   (crates/kore-kernels/src/cuda/kernels/rope.cu:36-37);
 * interleaved = 1: pairs (2i, 2i+1), as kore-serve's apply_rope
 *   (crates/kore-serve/src/layered/engine.rs:706-727).
 * inv_freq: device buffer from kore_hip_rope_inv_freq_f32.  Replaces
 * cuda_rope_f32 (crates/kore-kernels/src/cuda/ops.rs:572-599).  f32 tol. */
int kore_hip_rope_f32(float *data, const float *inv_freq, uint64_t batch,
                      uint64_t seq_len, uint32_t num_heads, uint32_t head_dim,
                      uint64_t start_pos, int interleaved,
                      kore_stream_t stream);

/* Q and K of one attention layer (GQA: q_heads != k_heads allowed) rotated in
 * one launch; identical results to two kore_hip_rope_f32 calls. */
int kore_hip_rope_qk_f32(float *q, float *k, const float *inv_freq,
                         uint64_t batch, uint64_t seq_len, uint32_t q_heads,
                         uint32_t k_heads, uint32_t head_dim,
                         uint64_t start_pos, int interleaved,
                         kore_stream_t stream);

/* -------------------------------------------------------------- Embedding
 * out[t, :] = table[ids[t], :] if ids[t] < vocab, else zeros.  ids are read
 * as unsigned 32-bit (an int32 buffer is accepted as-is; negative ids are
 * out of range).  Twin of kore_nn::Embedding::lookup
 * (crates/kore-nn/src/embedding.rs:55-72) and kore_edge embedding_lookup
 * (crates/kore-edge/src/ops/embedding.rs:8-27).  Bit-exact. */
int kore_hip_embedding_f32(const float *table, const uint32_t *ids,
                           float *out, uint64_t n_ids, uint64_t vocab,
                           uint64_t dim, kore_stream_t stream);

/* Embedding::forward's entry (crates/kore-nn/src/embedding.rs:91-98): the ids
 * arrive as an f32 tensor and each is converted with Rust's `v as usize`
 * (truncation; NaN and values below 1 give row 0, values >= 2^64 give
 * usize::MAX), then looked up as kore_hip_embedding_f32 does: an index >=
 * vocab gives a zero row.  Bit-exact. */
int kore_hip_embedding_forward_f32(const float *table, const float *ids,
                                   float *out, uint64_t n_ids, uint64_t vocab,
                                   uint64_t dim, kore_stream_t stream);

/* ----------------------------------------------------- BitLinear pre-quant
 * Per row r: xn = RMSNorm(x[r,:]) exactly as kore_hip_rms_norm_f32;
 * amax = max_i |xn_i| (1.0 if amax < 1e-8); scale[r] = amax / 127;
 * q[r,i] = clamp(round_half_away((xn_i * 127) / amax), -128, 127) (NaN -> 0).
 * The reference has no such op (BitLinear::forward,
 * crates/kore-nn/src/bit_linear.rs:175-237, feeds f32 activations to the
 * ternary GEMM); it composes fused_rms_norm (cpu_fused.rs:160-190) with the
 * absmax convention of kore_btes::quantize (crates/kore-btes/src/quantize.rs:8-10).
 * One HBM pass.  Bit-exact codes and scales. */
int kore_hip_rms_norm_quant_i8(const float *x, const float *weight,
                               int8_t *q, float *scale, uint64_t rows,
                               uint64_t cols, float eps, kore_stream_t stream);

/* ------------------------------------------------- RMSNorm with SiLU gate
 * out[r, :] = RMSNorm(x)[r, :] * silu(z[r, :]), silu(v) = v / (1 + exp(-v)),
 * with the RMSNorm part computed exactly as kore_hip_rms_norm_f32.  Replaces
 * cuda_fused_rms_norm_silu_gate_f32 (crates/kore-kernels/src/cuda/ops.rs:717-751,
 * kernel crates/kore-kernels/src/cuda/kernels/fused_norm_proj.cu:204-253),
 * whose CPU definition is the test at crates/kore-kernels/src/cpu_fused.rs:451-483.
 * f32 tol.  out may equal x or z. */
int kore_hip_rms_norm_silu_gate_f32(const float *x, const float *weight,
                                    const float *z, float *out, uint64_t rows,
                                    uint64_t cols, float eps,
                                    kore_stream_t stream);

/* ---------------------------------------------------------------- Softmax
 * Row softmax over the last dimension of x[rows, cols]:
 * out[r, :] = e * (1 / sum(e)), e = exp(x[r, :] - max(x[r, :])), the max
 * skipping NaN like f32::max.  Replaces cuda_softmax_f32
 * (crates/kore-kernels/src/cuda/ops.rs:486-511, kernel
 * crates/kore-kernels/src/cuda/kernels/softmax.cu:26-86); twin of
 * fused_softmax (crates/kore-kernels/src/cpu_fused.rs:195-231).  f32 tol.
 * out may equal x. */
int kore_hip_softmax_f32(const float *x, float *out, uint64_t rows,
                         uint64_t cols, kore_stream_t stream);

/* Causal row softmax: row r (counting all rows of the call) keeps columns
 * c < seq_offset + r + 1; the others are excluded from the max and written as
 * 0; a row whose kept sum is not > 0 is scaled by 0.  Replaces the
 * softmax_causal_f32 kernel (crates/kore-kernels/src/cuda/kernels/softmax.cu:88-157),
 * which the reference launches from no host wrapper.  f32 tol.  out may
 * equal x. */
int kore_hip_softmax_causal_f32(const float *x, float *out, uint64_t rows,
                                uint64_t cols, uint64_t seq_offset,
                                kore_stream_t stream);

/* Softmax backward: grad_in[r, :] = out[r, :] * (grad_out[r, :] - dot_r),
 * dot_r = sum(out[r, :] * grad_out[r, :]).  Twin of fused_softmax_backward
 * (crates/kore-kernels/src/cpu_fused_backward.rs:86-115); the reference has
 * no GPU version.  f32 tol.  grad_in may equal out or grad_out. */
int kore_hip_softmax_backward_f32(const float *grad_out, const float *out,
                                  float *grad_in, uint64_t rows, uint64_t cols,
                                  kore_stream_t stream);

/* Cross-entropy backward from raw logits[batch, num_classes]:
 * grad[b, :] = e * (inv_sum * inv_batch), e = exp(logits[b, :] - max),
 * inv_sum = 1 / sum(e), inv_batch = 1 / batch; then
 * grad[b, t] -= inv_batch for t = targets[b] converted like Rust's
 * `f32 as usize` (truncation; NaN and negatives give 0).  A t >= num_classes
 * (the reference panics on the index) subtracts nothing.  Twin of
 * fused_cross_entropy_backward (crates/kore-kernels/src/cpu_fused_backward.rs:130-170,
 * also reached through fused_softmax_cross_entropy_backward :179-184); the
 * reference has no GPU version.  f32 tol.  grad_logits may equal logits. */
int kore_hip_cross_entropy_backward_f32(const float *logits,
                                        const float *targets,
                                        float *grad_logits, uint64_t batch,
                                        uint64_t num_classes,
                                        kore_stream_t stream);

/* --------------------------------------------------------- RMSNorm backward
 * For y = RMSNorm(x) * gamma (rows x cols), given grad_out = dL/dy:
 *   inv_r = 1 / sqrt(sum_i x^2 / cols + eps)
 *   grad_x[r, i]  = (gamma[i] * inv_r) * grad_out[r, i] - coeff_r * x[r, i],
 *   coeff_r = (sum_i (x * grad_out) * gamma * inv_r) / (sum_i x^2 + eps * cols)
 *   grad_gamma[i] = sum_r (grad_out[r, i] * x[r, i]) * inv_r   (overwritten)
 * Twin of fused_rms_norm_backward
 * (crates/kore-kernels/src/cpu_fused_backward.rs:20-81); the reference has no
 * GPU version.  f32 tol.  grad_gamma is deterministic (fixed reduction order).
 * workspace: device scratch of at least
 * kore_hip_rms_norm_backward_workspace_bytes(rows, cols) bytes (the dgamma
 * partial sums), else KORE_HIP_ERR_BAD_DIM.  grad_x must not overlap
 * grad_out or x (KORE_HIP_ERR_ALIAS).  rows == 0 zeroes grad_gamma. */
uint64_t kore_hip_rms_norm_backward_workspace_bytes(uint64_t rows, uint64_t cols);

int kore_hip_rms_norm_backward_f32(const float *grad_out, const float *x,
                                   const float *gamma, float *grad_x,
                                   float *grad_gamma, float *workspace,
                                   uint64_t workspace_bytes, uint64_t rows,
                                   uint64_t cols, float eps,
                                   kore_stream_t stream);

/* Allocation-free variant of kore_hip_rms_norm_backward_f32 (same kernels,
 * same results bit for bit).  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving/training loops, harnesses that forbid hipMalloc).  The dgamma
 * partials go to a library-held device array of
 * kore_hip_rms_norm_backward_noalloc_max_bytes() bytes (16 MiB per GPU, held
 * until the process ends) instead of a caller workspace; work whose
 * kore_hip_rms_norm_backward_workspace_bytes(rows, cols) exceeds it returns
 * KORE_HIP_ERR_SCRATCH.  Calls never allocate or free.  All calls on one GPU
 * share the array: calls that overlap in time on one GPU (other streams,
 * other threads) race. */
uint64_t kore_hip_rms_norm_backward_noalloc_max_bytes(void);

int kore_hip_rms_norm_backward_noalloc_f32(const float *grad_out,
                                           const float *x, const float *gamma,
                                           float *grad_x, float *grad_gamma,
                                           uint64_t rows, uint64_t cols,
                                           float eps, kore_stream_t stream);

/* ------------------------------------------------------ ternary (BitLinear)
 * Weights a_packed[m, ceil(k/5)] in the reference's base-243 format (five
 * trits per byte, least significant base-3 digit first, digit 0/1/2 =
 * -1/0/+1, bytes 243..255 = five zeros; crates/kore-btes/src/encoder.rs:50-95,
 * as written by pack_weights_ternary, crates/kore-kernels/src/
 * cpu_ternary_matmul.rs:198-240), per-row scales a_scales[m].
 *
 * BitLinear matmul on the pre-quant codes: q[n, k] int8 (one row per token,
 * as kore_hip_rms_norm_quant_i8 writes them) with q_scales[n]:
 *   c[m, n] = ((float)(sum_k trit[m, k] * q[n, k]) * a_scales[m]) * q_scales[n].
 * The reference has no single function for this step: the dot product is
 * the integer one of ternary_ternary_matmul and the epilogue its
 * `int_acc as f32 * a_scale * b_scale` (cpu_ternary_matmul.rs:131-193, :188),
 * which replaces ternary_matmul (cpu_ternary_matmul.rs:29-124) fed with
 * dequantised activations.  Exact integer sum: bit-exact.  k <= 2^24.
 * c must not overlap an input (KORE_HIP_ERR_ALIAS). */
int kore_hip_ternary_matmul_i8(const uint8_t *a_packed, const float *a_scales,
                               const int8_t *q, const float *q_scales,
                               float *c, uint64_t m, uint64_t n, uint64_t k,
                               kore_stream_t stream);

/* c[M,N] = (sum over k, in order, of t[m,k] * b[k,n]) * a_scales[m] with f32
 * activations b[K,N] row-major: replaces ternary_matmul
 * (crates/kore-kernels/src/cpu_ternary_matmul.rs:29-124; unpack_row_trits
 * :91-101, compute_row :105-124), which BitLinear::forward
 * (crates/kore-nn/src/bit_linear.rs:175-237) calls with the transposed input.
 * The sum is the reference's sequential f32 fold that skips zero trits, so c
 * is bit-exact.  c must not overlap the inputs (KORE_HIP_ERR_ALIAS). */
int kore_hip_ternary_matmul_f32(const uint8_t *a_packed, const float *a_scales,
                                const float *b, float *c, uint64_t m,
                                uint64_t n, uint64_t k, kore_stream_t stream);

/* BitLinear::forward (crates/kore-nn/src/bit_linear.rs:175-237) as one
 * launch: y[batch, out] = ternary_matmul(W, scales, x^T)^T + bias, with the
 * layer's input x[batch, in] as it is stored (token-major) and its output in
 * the layer's layout -- the transposes at :200 and :218 and the bias add at
 * :222 need no passes of their own.  y[b, o] is the f32 fold of
 * kore_hip_ternary_matmul_f32 for output row o and column b, rounded, then
 * + bias[o] (one f32 add, as Tensor::add does); bias may be NULL (a layer
 * without bias).  Bit-exact.  in_features <= 2^23.  y must not overlap the
 * inputs (KORE_HIP_ERR_ALIAS). */
int kore_hip_bit_linear_f32(const uint8_t *a_packed, const float *a_scales,
                            const float *x, const float *bias, float *y,
                            uint64_t out_features, uint64_t batch,
                            uint64_t in_features, kore_stream_t stream);

/* The same layer on pre-quant codes (kore_hip_rms_norm_quant_i8's q[batch,
 * in] and q_scales[batch]): y[b, o] = c[o, b] + bias[o] with c of
 * kore_hip_ternary_matmul_i8, in the layer's [batch, out] layout; bias may be
 * NULL.  Bit-exact.  in_features <= 2^24.  y must not overlap the inputs
 * (KORE_HIP_ERR_ALIAS). */
int kore_hip_bit_linear_i8(const uint8_t *a_packed, const float *a_scales,
                           const int8_t *q, const float *q_scales,
                           const float *bias, float *y, uint64_t out_features,
                           uint64_t batch, uint64_t in_features,
                           kore_stream_t stream);

/* Quantise f32 weights w[m, k] (row-major) to ternary with a per-row scale
 * and pack them base-243, the weight format both matmuls read: replaces
 * pack_weights_ternary (crates/kore-kernels/src/cpu_ternary_matmul.rs:198-240;
 * encode_trits crates/kore-btes/src/encoder.rs:72-86).  scales[row] =
 * max |w| of the row (NaN dropped; 1.0 below 1e-8); a weight's trit is +1 /
 * -1 / 0 as w / scale (IEEE quotient) is > threshold / < -threshold /
 * otherwise; packed[row, j] = sum over i < 5 of (trit[5 j + i] + 1) * 3^i,
 * zero trits past k.  Bit-exact.  packed [m, ceil(k/5)] and scales [m] must
 * not overlap w (KORE_HIP_ERR_ALIAS). */
int kore_hip_pack_weights_ternary(const float *w, uint64_t m, uint64_t k,
                                  float threshold, uint8_t *packed,
                                  float *scales, kore_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* KORE_HIP_H */
