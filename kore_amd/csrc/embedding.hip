// embedding.hip -- token-embedding gather  out[t, :] = table[ids[t], :].
//
// Roofline: HBM.  Bytes per token: dim*4 read + dim*4 written + 4 for the id.
// A pure copy, so results are bit-exact by construction; out-of-range ids
// (ids[t] >= vocab, ids read as uint32) produce a zero row, as
// crates/kore-nn/src/embedding.rs:63-68 and
// crates/kore-edge/src/ops/embedding.rs:18-25 do.
//
// Vector path: one float4 per thread over a (token, row chunk) grid; rows
// longer than 65535 chunks use a workgroup-per-token loop.  Table reads use
// the default cache policy (repeated ids hit L2/MALL); output stores are
// nontemporal.
#include "common.hpp"
#include "kore_hip_internal.hpp"

namespace kore {

// Token id -> row index.  u32 ids (Embedding::lookup, embedding_lookup) are
// used as they are.  f32 ids (Embedding::forward,
// crates/kore-nn/src/embedding.rs:91-98) go through Rust's `v as usize`:
// truncation toward zero, NaN and everything below 1 to 0 (row 0, a valid
// row), values >= 2^64 to usize::MAX (out of range).
__device__ __forceinline__ uint64_t row_index(uint32_t id) { return id; }
__device__ __forceinline__ uint64_t row_index(float v) {
    if (!(v >= 1.0f)) return 0;
    if (v >= 18446744073709551616.0f) return ~0ull;
    return (uint64_t)v;
}

constexpr int kEmbBlock = 256;      // per-token loop and scalar kernels
constexpr int kEmbMaxBlock = 1024;  // one-float4 kernel: blockDim chosen per call
constexpr int kEmbUnroll = 4;  // float4 per thread per pass (rows > 16M floats)

template <typename Id>
__global__ __launch_bounds__(kEmbBlock) void embedding_vec_kernel(const f32x4* __restrict__ table,
                                                                  const Id* __restrict__ ids,
                                                                  f32x4* __restrict__ out, uint64_t vocab,
                                                                  uint64_t dim4) {
    const uint64_t t = blockIdx.x;
    const uint64_t id = row_index(ids[t]);
    f32x4* dst = out + t * dim4;
    if (id >= vocab) {
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
        for (uint64_t i = threadIdx.x; i < dim4; i += kEmbBlock) st_stream(dst + i, z);
        return;
    }
    const f32x4* src = table + id * dim4;
    uint64_t i = threadIdx.x;
    for (; i + (kEmbUnroll - 1) * kEmbBlock < dim4; i += kEmbUnroll * kEmbBlock) {
        f32x4 v[kEmbUnroll];
#pragma unroll
        for (int u = 0; u < kEmbUnroll; ++u) v[u] = ld_cached(src + i + u * kEmbBlock);
#pragma unroll
        for (int u = 0; u < kEmbUnroll; ++u) st_stream(dst + i + u * kEmbBlock, v[u]);
    }
    for (; i < dim4; i += kEmbBlock) st_stream(dst + i, ld_cached(src + i));
}

// One float4 per thread: grid (token, chunk of blockDim float4), blockDim =
// the row's float4 count rounded up to a wave, at most 1024.  Short-lived
// workgroups that each move one contiguous row chunk keep the most
// independent requests in flight (measured on MI355X: a 1 GiB gather-copy
// runs at 74.6% of 8 TB/s with 256-thread chunks, 81.5% with 1024, and
// worse with several tokens per workgroup).  Table rows are read through the
// caches (repeated ids hit them); nontemporal table loads measured slower
// (8192 x 4096 from a 128256-row table: 43.6 -> 44.7 us).
template <typename Id>
__global__ __launch_bounds__(kEmbMaxBlock) void embedding_vec1_kernel(const f32x4* __restrict__ table,
                                                                      const Id* __restrict__ ids,
                                                                      f32x4* __restrict__ out, uint64_t vocab,
                                                                      uint64_t dim4) {
    const uint64_t t = blockIdx.x;
    const uint64_t i = (uint64_t)blockIdx.y * blockDim.x + threadIdx.x;
    if (i >= dim4) return;
    const uint64_t id = row_index(ids[t]);
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    const f32x4 v = (id < vocab) ? ld_cached(table + id * dim4 + i) : z;
    st_stream(out + t * dim4 + i, v);
}

// Scalar path: dim % 4 != 0 or unaligned table/out.
template <typename Id>
__global__ __launch_bounds__(kEmbBlock) void embedding_scalar_kernel(const float* __restrict__ table,
                                                                     const Id* __restrict__ ids,
                                                                     float* __restrict__ out, uint64_t vocab,
                                                                     uint64_t dim) {
    const uint64_t t = blockIdx.x;
    const uint64_t id = row_index(ids[t]);
    float* dst = out + t * dim;
    if (id >= vocab) {
        for (uint64_t i = threadIdx.x; i < dim; i += kEmbBlock) dst[i] = 0.0f;
        return;
    }
    const float* src = table + id * dim;
    for (uint64_t i = threadIdx.x; i < dim; i += kEmbBlock) dst[i] = src[i];
}

}  // namespace kore

using namespace kore;

template <typename Id>
static int embedding_launch(const float* table, const Id* ids, float* out, uint64_t n_ids,
                                      uint64_t vocab, uint64_t dim, kore_stream_t stream) {
    if (n_ids == 0 || dim == 0) return KORE_HIP_OK;
    if (!ids || !out || (vocab && !table)) return KORE_HIP_ERR_NULL_PTR;
    uint64_t out_elems, table_elems;
    if (!mul_ok(n_ids, dim, &out_elems) || !mul_ok(vocab, dim, &table_elems) || out_elems > kMaxElements ||
        table_elems > kMaxElements || n_ids > 0x7fffffffull)
        return KORE_HIP_ERR_OVERFLOW;
    hipStream_t s = (hipStream_t)stream;
    dim3 grid((uint32_t)n_ids), block(kEmbBlock);
    if (dim % 4 == 0 && aligned16(out) && (vocab == 0 || aligned16(table))) {
        const uint64_t dim4 = dim / 4;
        const uint32_t thr = dim4 >= (uint64_t)kEmbMaxBlock ? kEmbMaxBlock : (uint32_t)((dim4 + 63) / 64 * 64);
        const uint64_t chunks = (dim4 + thr - 1) / thr;
        if (chunks <= 65535) {
            hipLaunchKernelGGL(embedding_vec1_kernel<Id>, dim3((uint32_t)n_ids, (uint32_t)chunks), dim3(thr), 0, s,
                               reinterpret_cast<const f32x4*>(table), ids, reinterpret_cast<f32x4*>(out), vocab,
                               dim / 4);
            return launch_status();
        }
        hipLaunchKernelGGL(embedding_vec_kernel<Id>, grid, block, 0, s, reinterpret_cast<const f32x4*>(table), ids,
                           reinterpret_cast<f32x4*>(out), vocab, dim / 4);
    } else {
        hipLaunchKernelGGL(embedding_scalar_kernel<Id>, grid, block, 0, s, table, ids, out, vocab, dim);
    }
    return launch_status();
}

extern "C" int kore_hip_embedding_f32(const float* table, const uint32_t* ids, float* out, uint64_t n_ids,
                                      uint64_t vocab, uint64_t dim, kore_stream_t stream) {
    return embedding_launch(table, ids, out, n_ids, vocab, dim, stream);
}

extern "C" int kore_hip_embedding_forward_f32(const float* table, const float* ids, float* out, uint64_t n_ids,
                                              uint64_t vocab, uint64_t dim, kore_stream_t stream) {
    return embedding_launch(table, ids, out, n_ids, vocab, dim, stream);
}
