// diag.hip -- measurement probes (no counterpart in the reference): the
// floors the fused kernels are compared against in the benchmark.
//
//   kore_hip_diag_empty        one empty workgroup: the launch floor of a
//                              dependent kernel on a stream;
//   kore_hip_diag_stream_rows  the pre-quant kernel's memory traffic with a
//                              trivial body: one wave per row reads the
//                              row's f32 values with the same coalesced,
//                              nontemporal 16-byte loads (all in flight) and
//                              writes one byte per value plus one f32 per
//                              row, in the same launch geometry (four waves
//                              per workgroup).  Its duration is the streaming
//                              ceiling of that shape.
#include "common.hpp"
#include "kore_hip_internal.hpp"

namespace kore {

__global__ __launch_bounds__(64) void diag_empty_kernel() {}

template <int NCH>
__global__ __launch_bounds__(256) void diag_stream_rows_kernel(const f32x4* __restrict__ x, uint32_t* __restrict__ q,
                                                               float* __restrict__ scale, uint64_t rows) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
    const uint64_t row = (uint64_t)blockIdx.x * 4 + wave;
    if (row >= rows) return;
    const f32x4* xr = x + row * (uint64_t)(NCH * kWave);
    f32x4 v[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) v[c] = ld_stream(xr + c * kWave + lane);
    uint32_t* qr = q + row * (uint64_t)(NCH * kWave);
    float m = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const f32x4 a = v[c];
        // a byte per value (bits of the float, not a quantisation)
        const uint32_t b = (__float_as_uint(a.x) >> 24) | ((__float_as_uint(a.y) >> 24) << 8) |
                           ((__float_as_uint(a.z) >> 24) << 16) | ((__float_as_uint(a.w) >> 24) << 24);
        __builtin_nontemporal_store(b, qr + c * kWave + lane);
        m = fmaxf(m, a.x);
    }
    if (lane == 0) scale[row] = m;
}

}  // namespace kore

using namespace kore;

extern "C" int kore_hip_diag_empty(kore_stream_t stream) {
    hipLaunchKernelGGL(diag_empty_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream);
    return launch_status();
}

extern "C" int kore_hip_diag_stream_rows(const float* x, int8_t* q, float* scale, uint64_t rows, uint64_t cols,
                                         kore_stream_t stream) {
    if (rows == 0) return KORE_HIP_OK;
    if (!x || !q || !scale) return KORE_HIP_ERR_NULL_PTR;
    if (cols != 2048 && cols != 2560) return KORE_HIP_ERR_BAD_DIM;
    if (!aligned16(x) || (reinterpret_cast<uintptr_t>(q) & 3u)) return KORE_HIP_ERR_BAD_DIM;
    const uint64_t blocks = (rows + 3) / 4;
    if (blocks > 0x7fffffffull || rows > kMaxElements / cols) return KORE_HIP_ERR_OVERFLOW;
    hipStream_t s = (hipStream_t)stream;
    if (cols == 2560)
        hipLaunchKernelGGL(diag_stream_rows_kernel<10>, dim3((uint32_t)blocks), dim3(256), 0, s,
                           reinterpret_cast<const f32x4*>(x), reinterpret_cast<uint32_t*>(q), scale, rows);
    else
        hipLaunchKernelGGL(diag_stream_rows_kernel<8>, dim3((uint32_t)blocks), dim3(256), 0, s,
                           reinterpret_cast<const f32x4*>(x), reinterpret_cast<uint32_t*>(q), scale, rows);
    return launch_status();
}
