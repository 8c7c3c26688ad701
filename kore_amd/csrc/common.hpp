// common.hpp -- shared device helpers for the gfx950 fused layer kernels.
//
// Everything here is written for CDNA4 (gfx950): wave64, 128-bit vector
// memory operations, LDS, DPP/ds_swizzle cross-lane moves.  The fused layer
// ops are bound by HBM bandwidth and use no MFMA; only the BitLinear int8 x
// ternary matmul (ternary.hip) is a contraction on the int8 MFMA units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kore {

// Native 128-bit vector types (clang ext_vector_type maps 1:1 onto a
// global_load_dwordx4 / global_store_dwordx4 operand).
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

__device__ __forceinline__ int lane_id() { return __lane_id(); }

// Streaming loads/stores: data touched once.  The nontemporal hint keeps
// the 2+ GB element-wise streams from evicting reusable lines in L2/MALL.
// Workgroups are dispatched to the 8 XCDs round-robin by index, so block b
// runs on XCD b % 8.  xcd_tile(b, nb) gives XCD x one contiguous range of the
// nb tiles: [x q + min(x, r), ...) of its share q + (x < r), q = nb / 8,
// r = nb % 8 -- a bijection on [0, nb).
__device__ __forceinline__ uint64_t xcd_tile(uint64_t b, uint64_t nb) {
    const uint64_t x = b % 8u, q = nb / 8u, r = nb % 8u;
    return x * q + (x < r ? x : r) + b / 8u;
}

__device__ __forceinline__ f32x4 ld_stream(const f32x4* p) {
    return __builtin_nontemporal_load(p);
}
__device__ __forceinline__ void st_stream(f32x4* p, f32x4 v) {
    __builtin_nontemporal_store(v, p);
}
__device__ __forceinline__ f32x4 ld_cached(const f32x4* p) { return *p; }

// Exact wave-wide max.  max is order-free, so any reduction tree gives the
// same bits; NaN operands are dropped like Rust's f32::max.
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Wave64 sum through DPP (row_shr 1/2/4/8 within each row of 16 lanes, then
// row_bcast 15/31 carry the row totals forward; lane 63 ends with the total,
// which is read into every lane).  Lanes without a DPP source contribute 0.
// A fixed-shape tree: the same inputs give the same bits on every call.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ float dpp_zero_src(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, kRowMask, 0xf, false));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += dpp_zero_src<0x111, 0xf>(v);  // row_shr:1
    v += dpp_zero_src<0x112, 0xf>(v);  // row_shr:2
    v += dpp_zero_src<0x114, 0xf>(v);  // row_shr:4
    v += dpp_zero_src<0x118, 0xf>(v);  // row_shr:8
    v += dpp_zero_src<0x142, 0xa>(v);  // row_bcast:15 -> rows 1, 3
    v += dpp_zero_src<0x143, 0xc>(v);  // row_bcast:31 -> rows 2, 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), kWave - 1));
}

// Read lane `src`'s value of v into every lane (v_readlane -> SGPR).
__device__ __forceinline__ float read_lane(float v, int src) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src));
}

// SiLU as the reference writes it (crates/kore-nn/src/activations.rs:43):
// x / (1 + exp(-x)) with ocml's accurate expf and IEEE division.
__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Orders this wave's LDS accesses across lanes.  A lane reading what another
// lane of the same wave wrote (or overwriting what another lane read) needs
// it: the compiler reasons per thread, sees different addresses, and would
// otherwise move the load above the store.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

}  // namespace kore
