// activation.hip -- element-wise streams: GELU (tanh form), SiLU, mul and the
// fused SwiGLU  out = silu(gate) * up.
//
// Roofline: HBM.  Bytes per element: 8 (GELU, SiLU), 12 (mul, SwiGLU).
// Layout: flat f32 arrays.  Each thread owns kEwUnroll float4 slots spaced
// one block-width apart, so every wave-wide global_load_dwordx4 covers 1 KiB
// of contiguous memory.  Loads and stores carry the nontemporal hint: each
// byte is touched once.
//
// Arithmetic follows the reference op order (crates/kore-nn/src/activations.rs
// :23-29 for GELU, :43 for SiLU) so that only the transcendental differs; the
// library is compiled with -ffp-contract=off so no a*b+c is fused.
#include "common.hpp"
#include "kore_hip_internal.hpp"

namespace kore {

// tanh on the GELU path.  Only its absolute error matters there: GELU uses
// t through (1 + t), so an absolute error d in t moves y by 0.5*|x|*d.
//   tanh(|u|) = 1 - 2 / (exp(2|u|) + 1),  sign restored with copysign.
// v_exp_f32 and v_rcp_f32 are each within ~1 ulp, giving |d| < 2e-7 over
// all inputs (inf/NaN: exp overflows to inf -> t = 1; NaN propagates).
// This replaces ocml's branchy tanhf, which costs ~3x the VALU slots.
__device__ __forceinline__ float tanh_gelu(float u) {
    float a = fabsf(u);
    float e = __builtin_amdgcn_exp2f(a * 2.88539008f);  // 2*log2(e)
    float t = 1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f);
    return copysignf(t, u);
}

// tanh-form GELU, statement for statement as activations.rs:23-29:
//   inner = (FRAC_2_SQRT_PI * FRAC_1_SQRT_2) * (x + 0.044715*x*x*x)
//   y     = 0.5*x * (1 + tanh(inner))
// The constant product is folded in f32 (0x3F4C422A).
struct GeluOp {
    __device__ __forceinline__ float operator()(float x) const {
        const float k = __int_as_float(0x3F4C422A);
        float cube = ((0.044715f * x) * x) * x;
        float inner = k * (x + cube);
        float half_x = 0.5f * x;
        return half_x * (1.0f + tanh_gelu(inner));
    }
};

struct SiluOp {
    __device__ __forceinline__ float operator()(float x) const { return silu_f(x); }
};

struct MulOp {
    __device__ __forceinline__ float operator()(float a, float b) const { return a * b; }
};

// silu(gate) then Tensor::mul (arithmetic.rs:499-509: result = a*b with a the
// silu tensor).
struct SwigluOp {
    __device__ __forceinline__ float operator()(float g, float u) const { return silu_f(g) * u; }
};

// One float4 per thread per operand: on MI355X many short waves keep more
// independent requests in flight than fewer threads with unrolled loads
// (a plain copy reaches ~82% of 8 TB/s this way, ~76% at 4 float4/thread),
// and 128-thread workgroups measured faster than 256 (GELU 16384 x 14336
// 283.2 -> 278.4 us, SwiGLU 428.1 -> 425.9 us; 512 slower).
constexpr int kEwBlock = 128;
constexpr int kEwUnroll = 1;  // float4 per thread

constexpr uint64_t kEwTile = (uint64_t)kEwBlock * kEwUnroll;  // float4 per block

// One block's tile.  Full = true drops every bounds check (all blocks but the
// last), so the loads issue back to back as one clause.
template <class Op, bool Full>
__device__ __forceinline__ void unary_tile(const f32x4* __restrict__ x, f32x4* __restrict__ out,
                                           uint64_t base, uint64_t n4) {
    Op op;
    f32x4 v[kEwUnroll];
#pragma unroll
    for (int u = 0; u < kEwUnroll; ++u) {
        uint64_t i = base + (uint64_t)u * kEwBlock;
        if (Full || i < n4) v[u] = ld_stream(x + i);
    }
#pragma unroll
    for (int u = 0; u < kEwUnroll; ++u) {
        uint64_t i = base + (uint64_t)u * kEwBlock;
        if (Full || i < n4) {
            f32x4 r;
            r.x = op(v[u].x);
            r.y = op(v[u].y);
            r.z = op(v[u].z);
            r.w = op(v[u].w);
            st_stream(out + i, r);
        }
    }
}

template <class Op, bool Full>
__device__ __forceinline__ void binary_tile(const f32x4* __restrict__ a, const f32x4* __restrict__ b,
                                            f32x4* __restrict__ out, uint64_t base, uint64_t n4) {
    Op op;
    f32x4 va[kEwUnroll], vb[kEwUnroll];
#pragma unroll
    for (int u = 0; u < kEwUnroll; ++u) {
        uint64_t i = base + (uint64_t)u * kEwBlock;
        if (Full || i < n4) {
            va[u] = ld_stream(a + i);
            vb[u] = ld_stream(b + i);
        }
    }
#pragma unroll
    for (int u = 0; u < kEwUnroll; ++u) {
        uint64_t i = base + (uint64_t)u * kEwBlock;
        if (Full || i < n4) {
            f32x4 r;
            r.x = op(va[u].x, vb[u].x);
            r.y = op(va[u].y, vb[u].y);
            r.z = op(va[u].z, vb[u].z);
            r.w = op(va[u].w, vb[u].w);
            st_stream(out + i, r);
        }
    }
}

template <class Op>
__global__ __launch_bounds__(kEwBlock) void unary_vec_kernel(const f32x4* __restrict__ x,
                                                             f32x4* __restrict__ out, uint64_t n4,
                                                             const float* __restrict__ xs,
                                                             float* __restrict__ outs, uint32_t tail) {
    const uint64_t blk = (uint64_t)blockIdx.x * kEwTile;
    const uint64_t base = blk + threadIdx.x;
    if (blk + kEwTile <= n4)
        unary_tile<Op, true>(x, out, base, n4);
    else
        unary_tile<Op, false>(x, out, base, n4);
    // The n % 4 trailing elements go to the first threads of block 0.
    if (blockIdx.x == 0 && threadIdx.x < tail) {
        Op op;
        uint64_t j = n4 * 4 + threadIdx.x;
        outs[j] = op(xs[j]);
    }
}

// The binary streams give each XCD one contiguous range of tiles
// (xcd_tile): SwiGLU 16384 x
// 14336 433 -> 426 us (81.3 -> 82.8% of 8 TB/s, two runs alike).  The
// unary streams keep the plain order (GELU 276 -> 282 us with it).

template <class Op>
__global__ __launch_bounds__(kEwBlock) void binary_vec_kernel(const f32x4* __restrict__ a,
                                                              const f32x4* __restrict__ b,
                                                              f32x4* __restrict__ out, uint64_t n4,
                                                              const float* __restrict__ as,
                                                              const float* __restrict__ bs,
                                                              float* __restrict__ outs, uint32_t tail) {
    const uint64_t blk = xcd_tile(blockIdx.x, gridDim.x) * kEwTile;
    const uint64_t base = blk + threadIdx.x;
    if (blk + kEwTile <= n4)
        binary_tile<Op, true>(a, b, out, base, n4);
    else
        binary_tile<Op, false>(a, b, out, base, n4);
    if (blockIdx.x == 0 && threadIdx.x < tail) {
        Op op;
        uint64_t j = n4 * 4 + threadIdx.x;
        outs[j] = op(as[j], bs[j]);
    }
}

// Scalar path for pointers that are not 16-byte aligned (sub-tensor views).
template <class Op>
__global__ __launch_bounds__(kEwBlock) void unary_scalar_kernel(const float* __restrict__ x,
                                                                float* __restrict__ out, uint64_t n) {
    Op op;
    const uint64_t stride = (uint64_t)gridDim.x * kEwBlock;
    for (uint64_t i = (uint64_t)blockIdx.x * kEwBlock + threadIdx.x; i < n; i += stride) out[i] = op(x[i]);
}

template <class Op>
__global__ __launch_bounds__(kEwBlock) void binary_scalar_kernel(const float* __restrict__ a,
                                                                 const float* __restrict__ b,
                                                                 float* __restrict__ out, uint64_t n) {
    Op op;
    const uint64_t stride = (uint64_t)gridDim.x * kEwBlock;
    for (uint64_t i = (uint64_t)blockIdx.x * kEwBlock + threadIdx.x; i < n; i += stride)
        out[i] = op(a[i], b[i]);
}

// In-place use (out == input) is safe: every element is read and written by
// the same thread, read first.  __restrict__ above only promises that no
// *other* thread's stores alias this thread's loads.
template <class Op>
static int launch_unary(const float* x, float* out, uint64_t n, hipStream_t s) {
    if (n == 0) return KORE_HIP_OK;
    if (!x || !out) return KORE_HIP_ERR_NULL_PTR;
    if (n > kMaxElements) return KORE_HIP_ERR_OVERFLOW;
    if (aligned16(x) && aligned16(out)) {
        uint64_t n4 = n / 4;
        uint32_t tail = (uint32_t)(n % 4);
        uint64_t blocks = (n4 + kEwTile - 1) / kEwTile;
        if (blocks == 0) blocks = 1;
        hipLaunchKernelGGL(unary_vec_kernel<Op>, dim3((uint32_t)blocks), dim3(kEwBlock), 0, s,
                           reinterpret_cast<const f32x4*>(x), reinterpret_cast<f32x4*>(out), n4, x, out,
                           tail);
    } else {
        uint64_t blocks = (n + kEwBlock - 1) / kEwBlock;
        if (blocks > 65536) blocks = 65536;
        hipLaunchKernelGGL(unary_scalar_kernel<Op>, dim3((uint32_t)blocks), dim3(kEwBlock), 0, s, x, out, n);
    }
    return launch_status();
}

template <class Op>
static int launch_binary(const float* a, const float* b, float* out, uint64_t n, hipStream_t s) {
    if (n == 0) return KORE_HIP_OK;
    if (!a || !b || !out) return KORE_HIP_ERR_NULL_PTR;
    if (n > kMaxElements) return KORE_HIP_ERR_OVERFLOW;
    if (aligned16(a) && aligned16(b) && aligned16(out)) {
        uint64_t n4 = n / 4;
        uint32_t tail = (uint32_t)(n % 4);
        uint64_t blocks = (n4 + kEwTile - 1) / kEwTile;
        if (blocks == 0) blocks = 1;
        hipLaunchKernelGGL(binary_vec_kernel<Op>, dim3((uint32_t)blocks), dim3(kEwBlock), 0, s,
                           reinterpret_cast<const f32x4*>(a), reinterpret_cast<const f32x4*>(b),
                           reinterpret_cast<f32x4*>(out), n4, a, b, out, tail);
    } else {
        uint64_t blocks = (n + kEwBlock - 1) / kEwBlock;
        if (blocks > 65536) blocks = 65536;
        hipLaunchKernelGGL(binary_scalar_kernel<Op>, dim3((uint32_t)blocks), dim3(kEwBlock), 0, s, a, b, out,
                           n);
    }
    return launch_status();
}

}  // namespace kore

using namespace kore;

extern "C" int kore_hip_gelu_f32(const float* x, float* out, uint64_t n, kore_stream_t stream) {
    return launch_unary<GeluOp>(x, out, n, (hipStream_t)stream);
}

extern "C" int kore_hip_silu_f32(const float* x, float* out, uint64_t n, kore_stream_t stream) {
    return launch_unary<SiluOp>(x, out, n, (hipStream_t)stream);
}

extern "C" int kore_hip_mul_f32(const float* a, const float* b, float* out, uint64_t n, kore_stream_t stream) {
    return launch_binary<MulOp>(a, b, out, n, (hipStream_t)stream);
}

extern "C" int kore_hip_swiglu_f32(const float* gate, const float* up, float* out, uint64_t n,
                                   kore_stream_t stream) {
    return launch_binary<SwigluOp>(gate, up, out, n, (hipStream_t)stream);
}
