// rope.hip -- in-place rotary position embedding over [batch, seq, heads, D].
//
// Roofline: HBM.  Bytes per token (b, s): 2 * heads * D * 4 (read + write,
// in place); the inv_freq table (D/2 floats) stays in L2.
//
// D in {32, 64, 128, 256} (16-byte aligned): one float4 per thread, 128
// consecutive float4 of one token's Q or K row per workgroup, the half-split
// partner taken from another lane (rope_lane_kernel, below).  Other D: one
// workgroup per token (rope_vec_kernel).  Either way the first D/2 threads
// of a workgroup compute the token's
// (cos, sin) pairs once into LDS: angle = (start_pos + s) * inv_freq[i] is
// the reference's f32 product (crates/kore-edge/src/ops/rope.rs:22-26 /
// crates/kore-serve/src/layered/engine.rs:716-719) and sincosf is ocml's
// accurate version with full range reduction (angles reach ~2047 rad), never
// the __sinf fast path.  Every head of Q and K then reuses those pairs, so the
// transcendental cost is D/2 per token instead of heads*D/2.
//
// Half-split layout (pairs i, i+D/2): a task is a float4 at i and its partner
// float4 at i+D/2 -> D/8 tasks per head.  Interleaved (pairs 2p, 2p+1): a task
// is one float4 holding two pairs -> D/4 tasks per head.  Consecutive threads
// take consecutive tasks, so each wave-wide access is 16 contiguous 16-byte
// words per head segment.  Q/K are touched once, so loads and stores are
// nontemporal (measured 108.7 -> 106.5 us on the 8x2048x(32+8)x128 config).
//
// The rotation is the reference's: d[i] = x0*c - x1*s, d[j] = x0*s + x1*c,
// with every product rounded on its own (-ffp-contract=off).
#include "common.hpp"
#include "kore_hip_internal.hpp"

namespace kore {

constexpr int kRopeBlock = 128;      // scalar path
constexpr int kRopeMaxBlock = 1024;  // vector path: blockDim chosen per call
constexpr uint32_t kRopeMaxHeadDim = 4096;

struct RopeTensor {
    float* data;     // [batch*seq, heads, D]
    uint32_t heads;
};

__device__ __forceinline__ float2 rot(float x0, float x1, float c, float s) {
    float a0 = x0 * c, b0 = x1 * s;
    float a1 = x0 * s, b1 = x1 * c;
    return make_float2(a0 - b0, a1 + b1);
}

// Vector path: D % 8 == 0 and both tensors 16-byte aligned.  blockDim covers
// a token's tasks in at most kRopeBatch slots per thread (one float4 pair per
// slot: many short waves, as for the other streams); a pass issues all of its
// global loads first, so the token's sincos work (first pass only) and the
// barrier overlap the memory latency instead of delaying the loads.
constexpr int kRopeBatch = 2;


template <bool Interleaved>
__global__ __launch_bounds__(kRopeMaxBlock) void rope_vec_kernel(RopeTensor t0, RopeTensor t1,
                                                              const float* __restrict__ inv_freq,
                                                              uint64_t seq_len, uint32_t head_dim,
                                                              uint64_t start_pos) {
    extern __shared__ f32x4 cs_raw[];  // [D/2] (cos, sin), 16-byte aligned base
    float2* cs = reinterpret_cast<float2*>(cs_raw);
    const uint64_t token = blockIdx.x;
    const uint32_t half = head_dim >> 1;
    const uint32_t tasks_per_head = Interleaved ? (head_dim >> 2) : (head_dim >> 3);
    const uint32_t n0 = t0.heads * tasks_per_head;
    const uint32_t n_all = n0 + t1.heads * tasks_per_head;
    float* row0 = t0.data + token * (uint64_t)t0.heads * head_dim;
    float* row1 = t1.data + token * (uint64_t)t1.heads * head_dim;

    const uint32_t nthr = blockDim.x;
    for (uint32_t base = 0; base < n_all; base += kRopeBatch * nthr) {
        f32x4* p0[kRopeBatch];
        f32x4* p1[kRopeBatch];
        f32x4 x0[kRopeBatch], x1[kRopeBatch];
        uint32_t kk[kRopeBatch];
#pragma unroll
        for (int u = 0; u < kRopeBatch; ++u) {
            const uint32_t task = base + u * nthr + threadIdx.x;
            const bool ok = task < n_all;
            const bool first = task < n0;
            const uint32_t local = first ? task : task - n0;
            const uint32_t h = local / tasks_per_head;
            const uint32_t k = local - h * tasks_per_head;
            float* v = (first ? row0 : row1) + (uint64_t)h * head_dim;
            kk[u] = k;
            if (Interleaved) {
                p0[u] = reinterpret_cast<f32x4*>(v + 4 * k);
                p1[u] = p0[u];
                if (ok) x0[u] = ld_stream(p0[u]);
            } else {
                p0[u] = reinterpret_cast<f32x4*>(v + 4 * k);
                p1[u] = reinterpret_cast<f32x4*>(v + half + 4 * k);
                if (ok) {
                    x0[u] = ld_stream(p0[u]);
                    x1[u] = ld_stream(p1[u]);
                }
            }
        }
        if (base == 0) {
            const float pos = (float)(start_pos + token % seq_len);
            for (uint32_t i = threadIdx.x; i < half; i += nthr) {
                float angle = pos * inv_freq[i];
                float s, c;
                sincosf(angle, &s, &c);
                cs[i] = make_float2(c, s);
            }
            __syncthreads();
        }
#pragma unroll
        for (int u = 0; u < kRopeBatch; ++u) {
            const uint32_t task = base + u * nthr + threadIdx.x;
            if (task >= n_all) continue;
            const uint32_t k = kk[u];
            if (Interleaved) {
                const f32x4 csv = *reinterpret_cast<const f32x4*>(&cs[2 * k]);  // c0 s0 c1 s1
                float2 r0 = rot(x0[u].x, x0[u].y, csv.x, csv.y);
                float2 r1 = rot(x0[u].z, x0[u].w, csv.z, csv.w);
                f32x4 o;
                o.x = r0.x; o.y = r0.y; o.z = r1.x; o.w = r1.y;
                st_stream(p0[u], o);
            } else {
                const f32x4 ca = *reinterpret_cast<const f32x4*>(&cs[4 * k]);      // c0 s0 c1 s1
                const f32x4 cb = *reinterpret_cast<const f32x4*>(&cs[4 * k + 2]);  // c2 s2 c3 s3
                float2 r0 = rot(x0[u].x, x1[u].x, ca.x, ca.y);
                float2 r1 = rot(x0[u].y, x1[u].y, ca.z, ca.w);
                float2 r2 = rot(x0[u].z, x1[u].z, cb.x, cb.y);
                float2 r3 = rot(x0[u].w, x1[u].w, cb.z, cb.w);
                f32x4 o0, o1;
                o0.x = r0.x; o0.y = r1.x; o0.z = r2.x; o0.w = r3.x;
                o1.x = r0.y; o1.y = r1.y; o1.z = r2.y; o1.w = r3.y;
                st_stream(p0[u], o0);
                st_stream(p1[u], o1);
            }
        }
    }
}

// Lane path: D in {32, 64, 128, 256} (a head is D/4 <= 64 float4, so a
// pair's two halves lie in one wave), both tensors 16-byte aligned.  One
// float4 per thread: a workgroup covers 128 consecutive float4 of one token's
// Q or K row (whole heads), which streams at the copy's rate (measured: one
// float4 per thread in 128-256 thread groups ~84% of HBM peak for an
// in-place update; two per thread in 640-thread groups ~80%; 128 threads
// 0.4-1.6% faster than 256 on the headline).  Half-split:
// lane L holds float4 j = L % (D/4) of its head and takes its partner (the
// float4 D/8 away) from lane L ^ (D/8) by a cross-lane swizzle; with x its
// own and p the partner's values, the first half stores x*c - p*s and the
// second half p*s + x*c, written as x*c + p*(-s) and x*c + p*s (negation is
// exact and a single addition commutes), the reference's products and sum.
constexpr int kRopeLaneBlock = 128;

__device__ __forceinline__ float lane_xor(float v, uint32_t m) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((int)((threadIdx.x ^ m) << 2), __builtin_bit_cast(int, v)));
}

template <bool Interleaved>
__global__ __launch_bounds__(kRopeLaneBlock) void rope_lane_kernel(RopeTensor t0, RopeTensor t1,
                                                                const float* __restrict__ inv_freq,
                                                                uint64_t seq_len, uint32_t head_dim,
                                                                uint64_t start_pos, uint32_t blocks0,
                                                                uint32_t blocks_tok) {
    extern __shared__ f32x4 cs_raw[];  // [D/2] (cos, sin)
    float2* cs = reinterpret_cast<float2*>(cs_raw);
    const uint64_t token = blockIdx.x / blocks_tok;
    const uint32_t bt = blockIdx.x % blocks_tok;
    const bool first_t = bt < blocks0;
    const RopeTensor& tt = first_t ? t0 : t1;
    const uint32_t row4 = tt.heads * (head_dim >> 2);  // float4 per token row
    const uint32_t f = (first_t ? bt : bt - blocks0) * kRopeLaneBlock + threadIdx.x;
    f32x4* row = reinterpret_cast<f32x4*>(tt.data + token * (uint64_t)tt.heads * head_dim);
    const bool ok = f < row4;
    f32x4 x = {0.f, 0.f, 0.f, 0.f};
    if (ok) x = ld_stream(row + f);
    const uint32_t half = head_dim >> 1;
    {
        const float pos = (float)(start_pos + token % seq_len);
        for (uint32_t i = threadIdx.x; i < half; i += kRopeLaneBlock) {
            float angle = pos * inv_freq[i];
            float sn, c;
            sincosf(angle, &sn, &c);
            cs[i] = make_float2(c, sn);
        }
        __syncthreads();
    }
    const uint32_t j = f & ((head_dim >> 2) - 1);  // float4 within the head
    f32x4 o;
    if (Interleaved) {
        const f32x4 csv = *reinterpret_cast<const f32x4*>(&cs[2 * j]);  // c0 s0 c1 s1
        const float2 r0 = rot(x.x, x.y, csv.x, csv.y);
        const float2 r1 = rot(x.z, x.w, csv.z, csv.w);
        o.x = r0.x; o.y = r0.y; o.z = r1.x; o.w = r1.y;
    } else {
        const uint32_t q8 = head_dim >> 3;  // float4 per half head
        f32x4 p;
        p.x = lane_xor(x.x, q8);
        p.y = lane_xor(x.y, q8);
        p.z = lane_xor(x.z, q8);
        p.w = lane_xor(x.w, q8);
        const uint32_t jj = j & (q8 - 1);
        const f32x4 ca = *reinterpret_cast<const f32x4*>(&cs[4 * jj]);      // c0 s0 c1 s1
        const f32x4 cb = *reinterpret_cast<const f32x4*>(&cs[4 * jj + 2]);  // c2 s2 c3 s3
        const bool lo = j < q8;
        const float s0 = lo ? -ca.y : ca.y, s1 = lo ? -ca.w : ca.w, s2 = lo ? -cb.y : cb.y, s3 = lo ? -cb.w : cb.w;
        float a, b;
        a = x.x * ca.x; b = p.x * s0; o.x = a + b;
        a = x.y * ca.z; b = p.y * s1; o.y = a + b;
        a = x.z * cb.x; b = p.z * s2; o.z = a + b;
        a = x.w * cb.z; b = p.w * s3; o.w = a + b;
    }
    if (ok) st_stream(row + f, o);
}

// Scalar path: any even D, any 4-byte alignment.  One task per pair.
template <bool Interleaved>
__global__ __launch_bounds__(kRopeBlock) void rope_scalar_kernel(RopeTensor t0, RopeTensor t1,
                                                                 const float* __restrict__ inv_freq,
                                                                 uint64_t seq_len, uint32_t head_dim,
                                                                 uint64_t start_pos) {
    extern __shared__ f32x4 cs_raw[];
    float2* cs = reinterpret_cast<float2*>(cs_raw);
    const uint64_t token = blockIdx.x;
    const uint32_t half = head_dim >> 1;
    const float pos = (float)(start_pos + token % seq_len);
    for (uint32_t i = threadIdx.x; i < half; i += kRopeBlock) {
        float angle = pos * inv_freq[i];
        float s, c;
        sincosf(angle, &s, &c);
        cs[i] = make_float2(c, s);
    }
    __syncthreads();
    const uint32_t n0 = t0.heads * half;
    const uint32_t n_all = n0 + t1.heads * half;
    for (uint32_t task = threadIdx.x; task < n_all; task += kRopeBlock) {
        const bool first = task < n0;
        const uint32_t local = first ? task : task - n0;
        const uint32_t heads = first ? t0.heads : t1.heads;
        float* row = (first ? t0.data : t1.data) + token * (uint64_t)heads * head_dim;
        const uint32_t h = local / half;
        const uint32_t i = local - h * half;
        float* v = row + (uint64_t)h * head_dim;
        const uint32_t j0 = Interleaved ? 2 * i : i;
        const uint32_t j1 = Interleaved ? 2 * i + 1 : i + half;
        float2 r = rot(v[j0], v[j1], cs[i].x, cs[i].y);
        v[j0] = r.x;
        v[j1] = r.y;
    }
}

static int rope_launch(float* q, uint32_t q_heads, float* k, uint32_t k_heads, const float* inv_freq,
                       uint64_t batch, uint64_t seq_len, uint32_t head_dim, uint64_t start_pos,
                       int interleaved, hipStream_t s) {
    uint64_t tokens;
    if (!mul_ok(batch, seq_len, &tokens)) return KORE_HIP_ERR_OVERFLOW;
    const uint64_t heads_all = (uint64_t)q_heads + k_heads;
    if (tokens == 0 || heads_all == 0 || head_dim == 0) return KORE_HIP_OK;
    if ((head_dim & 1u) || head_dim > kRopeMaxHeadDim) return KORE_HIP_ERR_BAD_DIM;
    if (!inv_freq || (q_heads && !q) || (k_heads && !k)) return KORE_HIP_ERR_NULL_PTR;
    uint64_t elems;
    if (!mul_ok(tokens, (uint64_t)heads_all * head_dim, &elems) || elems > kMaxElements ||
        tokens > 0x7fffffffull)
        return KORE_HIP_ERR_OVERFLOW;
    if ((uint64_t)heads_all * (head_dim / 2) > 0xffffffffull) return KORE_HIP_ERR_OVERFLOW;
    if (start_pos + seq_len < start_pos) return KORE_HIP_ERR_OVERFLOW;
    if (q && k && q_heads && k_heads) {
        // Overlapping Q and K would rotate shared elements twice.
        const char* q0 = (const char*)q;
        const char* q1 = q0 + tokens * (uint64_t)q_heads * head_dim * 4;
        const char* k0 = (const char*)k;
        const char* k1 = k0 + tokens * (uint64_t)k_heads * head_dim * 4;
        if (q0 < k1 && k0 < q1) return KORE_HIP_ERR_ALIAS;
    }
    RopeTensor t0{q_heads ? q : k, q_heads ? q_heads : k_heads};
    RopeTensor t1{q_heads ? k : nullptr, q_heads ? k_heads : 0u};
    const bool vec = (head_dim % 8 == 0) && aligned16(t0.data) && (t1.heads == 0 || aligned16(t1.data));
    const size_t lds = ((size_t)(head_dim / 2) * sizeof(float2) + 15) & ~(size_t)15;
    dim3 grid((uint32_t)tokens), block(kRopeBlock);
    const bool lane_ok = vec && (head_dim == 32 || head_dim == 64 || head_dim == 128 || head_dim == 256);
    if (lane_ok) {
        const uint64_t b0 = ((uint64_t)t0.heads * (head_dim / 4) + kRopeLaneBlock - 1) / kRopeLaneBlock;
        const uint64_t b1 = ((uint64_t)t1.heads * (head_dim / 4) + kRopeLaneBlock - 1) / kRopeLaneBlock;
        const uint64_t blocks = tokens * (b0 + b1);
        if (blocks > 0x7fffffffull) return KORE_HIP_ERR_OVERFLOW;
        const dim3 gl((uint32_t)blocks), bl(kRopeLaneBlock);
        if (interleaved)
            hipLaunchKernelGGL(rope_lane_kernel<true>, gl, bl, lds, s, t0, t1, inv_freq, seq_len, head_dim, start_pos,
                               (uint32_t)b0, (uint32_t)(b0 + b1));
        else
            hipLaunchKernelGGL(rope_lane_kernel<false>, gl, bl, lds, s, t0, t1, inv_freq, seq_len, head_dim, start_pos,
                               (uint32_t)b0, (uint32_t)(b0 + b1));
        return launch_status();
    }
    if (vec) {
        // Threads per token: the token's tasks in at most kRopeBatch slots,
        // rounded to whole waves, capped at kRopeMaxBlock.
        const uint64_t tasks = heads_all * (interleaved ? head_dim / 4 : head_dim / 8);
        uint64_t thr = (tasks + kRopeBatch - 1) / kRopeBatch;
        if (tasks <= (uint64_t)kRopeMaxBlock) thr = tasks;
        thr = (thr + 63) / 64 * 64;
        block = dim3((uint32_t)(thr > (uint64_t)kRopeMaxBlock ? kRopeMaxBlock : thr));
        if (interleaved)
            hipLaunchKernelGGL(rope_vec_kernel<true>, grid, block, lds, s, t0, t1, inv_freq, seq_len, head_dim,
                               start_pos);
        else
            hipLaunchKernelGGL(rope_vec_kernel<false>, grid, block, lds, s, t0, t1, inv_freq, seq_len, head_dim,
                               start_pos);
    } else {
        if (interleaved)
            hipLaunchKernelGGL(rope_scalar_kernel<true>, grid, block, lds, s, t0, t1, inv_freq, seq_len,
                               head_dim, start_pos);
        else
            hipLaunchKernelGGL(rope_scalar_kernel<false>, grid, block, lds, s, t0, t1, inv_freq, seq_len,
                               head_dim, start_pos);
    }
    return launch_status();
}

}  // namespace kore

using namespace kore;

extern "C" int kore_hip_rope_f32(float* data, const float* inv_freq, uint64_t batch, uint64_t seq_len,
                                 uint32_t num_heads, uint32_t head_dim, uint64_t start_pos, int interleaved,
                                 kore_stream_t stream) {
    return rope_launch(data, num_heads, nullptr, 0, inv_freq, batch, seq_len, head_dim, start_pos, interleaved,
                       (hipStream_t)stream);
}

extern "C" int kore_hip_rope_qk_f32(float* q, float* k, const float* inv_freq, uint64_t batch,
                                    uint64_t seq_len, uint32_t q_heads, uint32_t k_heads, uint32_t head_dim,
                                    uint64_t start_pos, int interleaved, kore_stream_t stream) {
    return rope_launch(q, q_heads, k, k_heads, inv_freq, batch, seq_len, head_dim, start_pos, interleaved,
                       (hipStream_t)stream);
}
