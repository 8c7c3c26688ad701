// softmax.hip -- row softmax (plain and causal) and its backward.
//
// Roofline: HBM.  Bytes per row: forward 8*cols (x read, y written);
// backward 12*cols (y and dy read, dx written).
//
// Definitions (the reference's, with the f32 tolerance of its CUDA twin):
//   forward  crates/kore-kernels/src/cpu_fused.rs:195-231 (fused_softmax):
//            m = max over the row (NaN skipped, as f32::max / fmaxf),
//            e = exp(x - m), y = e * (1 / sum(e));
//   causal   crates/kore-kernels/src/cuda/kernels/softmax.cu:88-157
//            (softmax_causal_f32): row r keeps columns c < seq_offset + r + 1
//            (r counts over all rows of the call); the rest are -inf in the
//            max and 0 in the output; inv = sum > 0 ? 1/sum : 0;
//   backward crates/kore-kernels/src/cpu_fused_backward.rs:86-115
//            (fused_softmax_backward): dx = y * (dy - sum(y * dy));
//   cross-entropy backward cpu_fused_backward.rs:130-170
//            (fused_cross_entropy_backward): g = e * (inv_sum * inv_batch),
//            inv_batch = 1 / rows, then g[t] -= inv_batch at t = targets[r]
//            cast like Rust's `as usize` (truncation, NaN and negatives -> 0);
//            a t >= cols (the reference panics) subtracts nothing.
// The sums are tree reductions (lane partials, then a wave butterfly), so
// results are within the f32 tolerance of the reference's left fold, as its
// own CUDA kernel is.  exp(d) is evaluated on the reference's d = x - m
// (rounded the same way) as the hardware exp2(d * log2(e)); see exp_diff.
//
// Shapes: a row of up to 1024 floats, or of 2049-4096, is held in one wave's
// registers (one wave per row, 4 rows per workgroup); 1025-2048 floats and
// up to 16384 in one workgroup's (256 threads; 512 for the 1025-2048
// backward); longer rows (vocab-sized) stream through a workgroup in three
// passes.  Unaligned views and cols % 4 != 0 use the looped kernel with
// scalar accesses.  Every kernel reads a row fully before writing it, so out
// may alias an input.
#include "common.hpp"
#include "kore_hip_internal.hpp"

namespace kore {

enum class SmKind : int { Fwd = 0, Causal = 1, Bwd = 2, CeBwd = 3 };

struct SmArgs {
    const float* a;  // x (forward) or y (backward)
    const float* b;  // dy (backward), targets[rows] (cross-entropy), unused otherwise
    float* out;
    uint64_t rows;
    uint64_t cols;
    uint64_t seq_offset;
};

constexpr int kSmBlock = 256;
constexpr int kSmWaves = kSmBlock / kWave;

__device__ __forceinline__ float f4_get(const f32x4& v, int k) {
    return k == 0 ? v.x : (k == 1 ? v.y : (k == 2 ? v.z : v.w));
}
__device__ __forceinline__ void f4_set(f32x4& v, int k, float s) {
    if (k == 0) v.x = s; else if (k == 1) v.y = s; else if (k == 2) v.z = s; else v.w = s;
}

// Rust `f32 as usize`: NaN and negatives -> 0, truncation toward zero,
// saturating; returned as a column index, or UINT64_MAX when >= cols.
__device__ __forceinline__ uint64_t target_index(float t, uint64_t cols) {
    if (!(t >= 1.0f)) return cols > 0 ? 0 : ~0ull;  // NaN, negative, [0, 1)
    if (t >= 18446744073709551616.0f) return ~0ull;
    const uint64_t i = (uint64_t)t;
    return i < cols ? i : ~0ull;
}

// exp(d) for d = x - max <= 0 as v_exp_f32(d * log2(e)): 2 VALU ops instead
// of ~12 for ocml expf.  Rounding d*log2(e) perturbs the result by at most
// |d| * 2^-24 * ln 2 relative (< 1e-6 for d >= -16, where e^d > 1e-7 still
// matters next to the row's largest term e^0 = 1); v_exp_f32 adds ~1 ulp.
// Below that the absolute error is < 1e-7 * e^d.  exp(-inf) = 0 and
// exp(NaN) = NaN as in the reference.  (Measured: 87.2 -> 85.3 us on the
// 32768 x 2048 softmax.)
__device__ __forceinline__ float exp_diff(float d) { return __builtin_amdgcn_exp2f(d * 1.44269504f); }

// Number of leading columns of `row` that take part (causal mask).
template <SmKind K>
__device__ __forceinline__ uint64_t row_limit(const SmArgs& a, uint64_t row) {
    if (K != SmKind::Causal) return a.cols;
    const uint64_t lim = a.seq_offset + row + 1;  // host checked: no overflow
    return lim < a.cols ? lim : a.cols;
}

// Block-wide reduction of one value per wave through LDS, combined in wave
// order (deterministic).  `red` holds kSmWaves floats.
template <bool IsMax, int Waves = kSmWaves>
__device__ __forceinline__ float block_combine(float v, float* red) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    __syncthreads();  // previous readers of red are done
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int w = 1; w < Waves; ++w) r = IsMax ? fmaxf(r, red[w]) : r + red[w];
    return r;
}

// Row in registers.  Wave mode (Block = false): one wave per row, element f4
// index = c*64 + lane, 4 rows per 256-thread workgroup.  Block mode: one
// workgroup of BS threads per row, index = c*BS + tid.
template <SmKind K, int NCH, bool Block, int BS = kSmBlock>
__global__ __launch_bounds__(BS) void softmax_reg_kernel(SmArgs a) {
    constexpr int kWavesB = BS / kWave;
    __shared__ float red[kWavesB];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const uint64_t row = Block ? (uint64_t)blockIdx.x : (uint64_t)blockIdx.x * kSmWaves + wave;
    if (!Block && row >= a.rows) return;  // uniform per wave; no block barrier in wave mode
    const int step = Block ? BS : kWave;
    const int me = Block ? (int)threadIdx.x : lane;
    const uint32_t cols4 = (uint32_t)(a.cols >> 2);      // <= 4096 here
    const uint32_t lim = (uint32_t)row_limit<K>(a, row);  // <= cols
    const f32x4* ar = reinterpret_cast<const f32x4*>(a.a) + row * cols4;
    const f32x4* br = reinterpret_cast<const f32x4*>(a.b) + row * cols4;
    f32x4* orow = reinterpret_cast<f32x4*>(a.out) + row * cols4;
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};

    f32x4 v[NCH], g[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const uint32_t f = (uint32_t)(c * step + me);
        v[c] = f < cols4 ? ld_stream(ar + f) : zero;
        if (K == SmKind::Bwd) g[c] = f < cols4 ? ld_stream(br + f) : zero;
    }

    if (K == SmKind::Bwd) {
        // dot = sum(y * dy); dx = y * (dy - dot)
        float dot = 0.0f;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const f32x4 p = v[c] * g[c];
            dot += (p.x + p.y) + (p.z + p.w);
        }
        dot = wave_sum(dot);
        if (Block) dot = block_combine<false, kWavesB>(dot, red);
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const uint32_t f = (uint32_t)(c * step + me);
            if (f < cols4) st_stream(orow + f, v[c] * (g[c] - dot));
        }
        return;
    }

    const float ninf = -__builtin_inff();
    float m = ninf;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const uint32_t f = (uint32_t)(c * step + me);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const bool in = 4 * f + k < lim;
            m = fmaxf(m, in ? f4_get(v[c], k) : ninf);
        }
    }
    m = wave_max(m);
    if (Block) m = block_combine<true, kWavesB>(m, red);
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const uint32_t f = (uint32_t)(c * step + me);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const bool in = 4 * f + k < lim;
            const float e = in ? exp_diff(f4_get(v[c], k) - m) : 0.0f;
            f4_set(v[c], k, e);
            s += e;
        }
    }
    s = wave_sum(s);
    if (Block) s = block_combine<false, kWavesB>(s, red);
    const float inv = (K == SmKind::Causal) ? (s > 0.0f ? 1.0f / s : 0.0f) : 1.0f / s;
    if (K == SmKind::CeBwd) {
        const float inv_batch = 1.0f / (float)a.rows;
        const float scale = inv * inv_batch;
        const uint64_t t = target_index(a.b[row], a.cols);
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const uint32_t f = (uint32_t)(c * step + me);
            f32x4 o = v[c] * scale;
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if ((uint64_t)(4 * f + k) == t) f4_set(o, k, f4_get(o, k) - inv_batch);
            if (f < cols4) st_stream(orow + f, o);
        }
        return;
    }
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const uint32_t f = (uint32_t)(c * step + me);
        if (f < cols4) st_stream(orow + f, v[c] * inv);
    }
}

// Any row length and alignment: one workgroup per row, the row streamed
// three times (max, sum, write) -- or twice for the backward.  Vec = float4
// accesses (cols % 4 == 0 and aligned views), else scalar.
template <SmKind K, bool Vec>
__global__ __launch_bounds__(kSmBlock) void softmax_loop_kernel(SmArgs a) {
    __shared__ float red[kSmWaves];
    const uint64_t row = blockIdx.x;
    const uint64_t lim = row_limit<K>(a, row);
    const float* ar = a.a + row * a.cols;
    const float* br = a.b + row * a.cols;
    float* orow = a.out + row * a.cols;
    const uint64_t n = Vec ? a.cols >> 2 : a.cols;
    const float ninf = -__builtin_inff();

    if (K == SmKind::Bwd) {
        float dot = 0.0f;
        for (uint64_t i = threadIdx.x; i < n; i += kSmBlock) {
            if (Vec) {
                const f32x4 p = reinterpret_cast<const f32x4*>(ar)[i] * reinterpret_cast<const f32x4*>(br)[i];
                dot += (p.x + p.y) + (p.z + p.w);
            } else {
                dot += ar[i] * br[i];
            }
        }
        dot = block_combine<false>(wave_sum(dot), red);
        for (uint64_t i = threadIdx.x; i < n; i += kSmBlock) {
            if (Vec) {
                const f32x4 y = reinterpret_cast<const f32x4*>(ar)[i];
                const f32x4 g = reinterpret_cast<const f32x4*>(br)[i];
                st_stream(reinterpret_cast<f32x4*>(orow) + i, y * (g - dot));
            } else {
                orow[i] = ar[i] * (br[i] - dot);
            }
        }
        return;
    }

    float m = ninf;
    for (uint64_t i = threadIdx.x; i < n; i += kSmBlock) {
        if (Vec) {
            const f32x4 v = reinterpret_cast<const f32x4*>(ar)[i];
#pragma unroll
            for (int k = 0; k < 4; ++k) m = fmaxf(m, 4 * i + k < lim ? f4_get(v, k) : ninf);
        } else {
            m = fmaxf(m, i < lim ? ar[i] : ninf);
        }
    }
    m = block_combine<true>(wave_max(m), red);
    float s = 0.0f;
    for (uint64_t i = threadIdx.x; i < n; i += kSmBlock) {
        if (Vec) {
            const f32x4 v = reinterpret_cast<const f32x4*>(ar)[i];
#pragma unroll
            for (int k = 0; k < 4; ++k) s += 4 * i + k < lim ? exp_diff(f4_get(v, k) - m) : 0.0f;
        } else {
            s += i < lim ? exp_diff(ar[i] - m) : 0.0f;
        }
    }
    s = block_combine<false>(wave_sum(s), red);
    const float inv = (K == SmKind::Causal) ? (s > 0.0f ? 1.0f / s : 0.0f) : 1.0f / s;
    const float inv_batch = 1.0f / (float)a.rows;
    const float scale = (K == SmKind::CeBwd) ? inv * inv_batch : inv;
    const uint64_t t = (K == SmKind::CeBwd) ? target_index(a.b[row], a.cols) : ~0ull;
    for (uint64_t i = threadIdx.x; i < n; i += kSmBlock) {
        if (Vec) {
            f32x4 v = reinterpret_cast<const f32x4*>(ar)[i];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                float o = (4 * i + k < lim ? exp_diff(f4_get(v, k) - m) : 0.0f) * scale;
                if (K == SmKind::CeBwd && 4 * i + k == t) o = o - inv_batch;
                f4_set(v, k, o);
            }
            st_stream(reinterpret_cast<f32x4*>(orow) + i, v);
        } else {
            float o = (i < lim ? exp_diff(ar[i] - m) : 0.0f) * scale;
            if (K == SmKind::CeBwd && i == t) o = o - inv_batch;
            orow[i] = o;
        }
    }
}

template <SmKind K, int NCH>
static void launch_wave(const SmArgs& a, hipStream_t s) {
    const uint64_t blocks = (a.rows + kSmWaves - 1) / kSmWaves;
    hipLaunchKernelGGL((softmax_reg_kernel<K, NCH, false>), dim3((uint32_t)blocks), dim3(kSmBlock), 0, s, a);
}

template <SmKind K>
static int softmax_launch(const SmArgs& a, hipStream_t s) {
    if (a.rows == 0 || a.cols == 0) return KORE_HIP_OK;
    if (!a.a || !a.out || ((K == SmKind::Bwd || K == SmKind::CeBwd) && !a.b)) return KORE_HIP_ERR_NULL_PTR;
    uint64_t elems;
    if (!mul_ok(a.rows, a.cols, &elems) || elems > kMaxElements || a.rows > 0x7fffffffull)
        return KORE_HIP_ERR_OVERFLOW;
    if (K == SmKind::Causal && a.seq_offset + a.rows < a.seq_offset) return KORE_HIP_ERR_OVERFLOW;
    const bool vec = (a.cols % 4 == 0) && aligned16(a.a) && aligned16(a.out) &&
                     (K != SmKind::Bwd || aligned16(a.b));
    const uint64_t cols4 = a.cols / 4;
    if (vec && cols4 <= 64) launch_wave<K, 1>(a, s);
    else if (vec && cols4 <= 128) launch_wave<K, 2>(a, s);
    else if (vec && cols4 <= 256) launch_wave<K, 4>(a, s);
    else if (vec && cols4 <= 512) {
        // 1025-2048 columns: one workgroup per row streams faster than one
        // wave per row (measured at 32768 x 2048: forward 85.8 -> 83.3 us
        // with 256 threads x 2 float4, backward 129.3 -> 121.7 us with 512
        // threads x 1 float4 each of y and dy)
        if (K == SmKind::Bwd)
            hipLaunchKernelGGL((softmax_reg_kernel<K, 1, true, 512>), dim3((uint32_t)a.rows), dim3(512), 0, s, a);
        else
            hipLaunchKernelGGL((softmax_reg_kernel<K, 2, true>), dim3((uint32_t)a.rows), dim3(kSmBlock), 0, s, a);
    }
    else if (vec && cols4 <= 1024) launch_wave<K, 16>(a, s);
    else if (vec && cols4 <= 2048)
        hipLaunchKernelGGL((softmax_reg_kernel<K, 8, true>), dim3((uint32_t)a.rows), dim3(kSmBlock), 0, s, a);
    else if (vec && cols4 <= 4096)
        hipLaunchKernelGGL((softmax_reg_kernel<K, 16, true>), dim3((uint32_t)a.rows), dim3(kSmBlock), 0, s, a);
    else if (vec)
        hipLaunchKernelGGL((softmax_loop_kernel<K, true>), dim3((uint32_t)a.rows), dim3(kSmBlock), 0, s, a);
    else
        hipLaunchKernelGGL((softmax_loop_kernel<K, false>), dim3((uint32_t)a.rows), dim3(kSmBlock), 0, s, a);
    return launch_status();
}

}  // namespace kore

using namespace kore;

extern "C" int kore_hip_softmax_f32(const float* x, float* out, uint64_t rows, uint64_t cols,
                                    kore_stream_t stream) {
    SmArgs a{x, nullptr, out, rows, cols, 0};
    return softmax_launch<SmKind::Fwd>(a, (hipStream_t)stream);
}

extern "C" int kore_hip_softmax_causal_f32(const float* x, float* out, uint64_t rows, uint64_t cols,
                                           uint64_t seq_offset, kore_stream_t stream) {
    SmArgs a{x, nullptr, out, rows, cols, seq_offset};
    return softmax_launch<SmKind::Causal>(a, (hipStream_t)stream);
}

extern "C" int kore_hip_softmax_backward_f32(const float* grad_out, const float* out, float* grad_in,
                                             uint64_t rows, uint64_t cols, kore_stream_t stream) {
    SmArgs a{out, grad_out, grad_in, rows, cols, 0};
    return softmax_launch<SmKind::Bwd>(a, (hipStream_t)stream);
}

extern "C" int kore_hip_cross_entropy_backward_f32(const float* logits, const float* targets, float* grad_logits,
                                                   uint64_t batch, uint64_t num_classes, kore_stream_t stream) {
    SmArgs a{logits, targets, grad_logits, batch, num_classes, 0};
    return softmax_launch<SmKind::CeBwd>(a, (hipStream_t)stream);
}
