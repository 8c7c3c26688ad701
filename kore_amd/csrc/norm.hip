// norm.hip -- RMSNorm (f32 out) and the BitLinear pre-quant (RMSNorm + per-row
// absmax int8), bit-exact against the reference CPU path.
//
// Roofline: HBM.  Bytes per row: cols*4 read, plus cols*4 written (RMSNorm)
// or cols + 4 written (pre-quant); the weight vector stays in L2.
//
// Why a "row engine" instead of a tree reduction: the reference sums x^2 with
// a left-to-right f32 fold (crates/kore-kernels/src/cpu_fused.rs:180).  A tree
// sum lands a few ulps away, which moves inv_rms and flips int8 codes that sit
// on a rounding boundary.  The engine reproduces the fold exactly and still
// keeps every HBM access coalesced:
//
//   * one wave owns kRowsPerWave rows.  It loads them with wave-wide
//     global_load_dwordx4 (64 lanes x 16 B = 256 columns of one row per
//     instruction), all loads in flight before the first use, and keeps the
//     values in VGPRs until the output is written (one HBM read per byte);
//   * per 256-column chunk, every lane squares its float4s and writes them to
//     the wave's private LDS tile [kRowsPerWave][256 + pad];
//   * lane r of the wave then walks row r of the tile in column order adding
//     one square at a time -- the reference's exact fold -- with the tile read
//     as ds_read_b128.  The pad (4 floats) puts the rows' reads on disjoint
//     banks;
//   * inv_rms = 1 / sqrt(ss / cols + eps) with IEEE sqrt and division (the
//     library is built with correctly rounded f32 divide/sqrt), broadcast with
//     v_readlane; the epilogue is element-parallel over all 64 lanes.
//
// A wave's LDS traffic never crosses waves, so there is no barrier: LDS
// operations from one wave complete in issue order.
//
// Pre-quant epilogue (one pass, codes bit-exact):
//   xn   = (x * inv) * w                          (cpu_fused.rs:185)
//   amax = max |xn| (wave max: order-free, exact); 1.0 if amax < 1e-8
//   t    = (xn * 127) / amax                      IEEE quotient, obtained with
//          y = 1/amax (IEEE), q0 = a*y, r = fma(-amax, q0, a), t = fma(r, y, q0)
//          (Markstein's correction: with y the correctly rounded reciprocal,
//          t is the correctly rounded quotient -- checked exhaustively against
//          IEEE division on the CPU by the test suite)
//   code = trunc(t + copysign(0.5 - 2^-25, t)), then clamp to [-128, 127];
//          equal to round-half-away(t) for |t| < 2^23 (also checked on the
//          CPU over every float in range); v_cvt_i32_f32 maps NaN to 0 and
//          saturates, like Rust's `as i8` after clamp.
#include "common.hpp"
#include "kore_hip_internal.hpp"

namespace kore {

constexpr int kRowsPerWave = 4;
constexpr int kWavesPerBlock = 4;
constexpr int kNormBlock = kWave * kWavesPerBlock;
constexpr int kChunk = 256;                 // columns per wave-wide float4 load
constexpr int kPitch = kChunk + 4;          // LDS row pitch (floats)
constexpr int kTileFloats = kRowsPerWave * kPitch;

enum class NormOut { F32, I8 };

struct NormArgs {
    const float* x;
    const float* w;
    float* y;        // NormOut::F32
    int8_t* q;       // NormOut::I8
    float* scale;    // NormOut::I8
    uint64_t rows;
    uint32_t cols;
    float eps;
};

__device__ __forceinline__ int32_t cvt_i32_sat(float v) {
    // v_cvt_i32_f32: round toward zero, saturating, NaN -> 0.  Written as asm
    // because a C++ float->int cast of NaN is undefined.
    int32_t r;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(v));
    return r;
}

// int8 code of one normalised value; see the header comment for the proof
// obligations (both are exercised by the CPU test suite).
__device__ __forceinline__ uint32_t quant_code(float xn, float amax, float rcp_amax) {
    float a = xn * 127.0f;
    float q0 = a * rcp_amax;
    float r = __builtin_fmaf(-amax, q0, a);
    float t = __builtin_fmaf(r, rcp_amax, q0);
    float b = t + __builtin_copysignf(0.49999997f, t);
    int32_t c = cvt_i32_sat(b);
    c = c < -128 ? -128 : (c > 127 ? 127 : c);
    return (uint32_t)c & 0xffu;
}

__device__ __forceinline__ float abs_max4(float m, f32x4 v) {
    m = fmaxf(m, fabsf(v.x));
    m = fmaxf(m, fabsf(v.y));
    m = fmaxf(m, fabsf(v.z));
    m = fmaxf(m, fabsf(v.w));
    return m;
}

// Adds the 256 squares of this lane's tile row to ss in column order.  The
// reads are issued in blocks of 8 float4 ahead of the adds that consume them.
__device__ __forceinline__ float fold_tile_row(const f32x4* __restrict__ tp, float ss) {
    constexpr int kBlk = 8;
    constexpr int kN = kChunk / 4;  // 64 float4
    f32x4 a[kBlk], b[kBlk];
#pragma unroll
    for (int j = 0; j < kBlk; ++j) a[j] = tp[j];
    // Rolled loop: a fully unrolled fold lets the scheduler hoist all 64
    // reads (256 VGPRs) above the adds and evict the row cache to AGPRs.
#pragma unroll 1
    for (int blk = 0; blk < kN / kBlk; blk += 2) {
#pragma unroll
        for (int j = 0; j < kBlk; ++j) b[j] = tp[(blk + 1) * kBlk + j];
#pragma unroll
        for (int j = 0; j < kBlk; ++j) {
            ss = ss + a[j].x;
            ss = ss + a[j].y;
            ss = ss + a[j].z;
            ss = ss + a[j].w;
        }
        if (blk + 2 < kN / kBlk) {
#pragma unroll
            for (int j = 0; j < kBlk; ++j) a[j] = tp[(blk + 2) * kBlk + j];
        }
#pragma unroll
        for (int j = 0; j < kBlk; ++j) {
            ss = ss + b[j].x;
            ss = ss + b[j].y;
            ss = ss + b[j].z;
            ss = ss + b[j].w;
        }
    }
    return ss;
}

// Vector path: cols % 4 == 0, cols <= NCH * 256, x/w/y 16-byte aligned and q
// 4-byte aligned.  Grid: one block per kWavesPerBlock * kRowsPerWave rows.
template <NormOut Out, int NCH>
__global__ __launch_bounds__(kNormBlock) void row_norm_kernel(NormArgs args) {
    __shared__ f32x4 lds[kWavesPerBlock * kTileFloats / 4];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const uint64_t row0 = ((uint64_t)blockIdx.x * kWavesPerBlock + wave) * kRowsPerWave;
    if (row0 >= args.rows) return;  // uniform per wave; no block barrier follows
    const uint64_t left = args.rows - row0;
    const int nrows = left < (uint64_t)kRowsPerWave ? (int)left : kRowsPerWave;
    const uint32_t cols = args.cols;
    const uint32_t cols4 = cols >> 2;
    const int nch = (int)((cols4 + kWave - 1) / kWave);
    float* tile = reinterpret_cast<float*>(lds) + wave * kTileFloats;
    const f32x4* x4 = reinterpret_cast<const f32x4*>(args.x) + row0 * cols4;
    const f32x4* w4 = reinterpret_cast<const f32x4*>(args.w);
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};

    // All HBM reads of the wave, chunk-major so chunk 0 of every row lands
    // first and the fold can start while the rest streams in.
    f32x4 xv[NCH][kRowsPerWave];
    f32x4 wv[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const uint32_t c4 = (uint32_t)c * kWave + lane;
        const bool in_row = c < nch && c4 < cols4;
#pragma unroll
        for (int r = 0; r < kRowsPerWave; ++r)
            xv[c][r] = (in_row && r < nrows) ? ld_stream(x4 + (uint64_t)r * cols4 + c4) : zero;
        wv[c] = in_row ? ld_cached(w4 + c4) : zero;
    }

    // Sequential sum of squares, lane r <-> row r.  Columns past the end are
    // zero: adding +0.0 to a non-negative running sum leaves it bit-identical.
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        if (c < nch) {
#pragma unroll
            for (int r = 0; r < kRowsPerWave; ++r) {
                f32x4 v = xv[c][r];
                *reinterpret_cast<f32x4*>(tile + r * kPitch + 4 * lane) = v * v;
            }
            if (lane < nrows) ss = fold_tile_row(reinterpret_cast<const f32x4*>(tile + lane * kPitch), ss);
        }
    }

    // cpu_fused.rs:181-182 with IEEE sqrt and division.
    float inv_lane = 0.0f;
    if (lane < nrows) {
        float rms = sqrtf(ss / (float)cols + args.eps);
        inv_lane = 1.0f / rms;
    }
    float inv[kRowsPerWave];
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r) inv[r] = read_lane(inv_lane, r);

    if (Out == NormOut::F32) {
        f32x4* y4 = reinterpret_cast<f32x4*>(args.y) + row0 * cols4;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const uint32_t c4 = (uint32_t)c * kWave + lane;
            if (c < nch && c4 < cols4) {
#pragma unroll
                for (int r = 0; r < kRowsPerWave; ++r)
                    if (r < nrows) st_stream(y4 + (uint64_t)r * cols4 + c4, (xv[c][r] * inv[r]) * wv[c]);
            }
        }
    } else {
        float amax[kRowsPerWave];
#pragma unroll
        for (int r = 0; r < kRowsPerWave; ++r) amax[r] = 0.0f;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
#pragma unroll
            for (int r = 0; r < kRowsPerWave; ++r) {
                f32x4 xn = (xv[c][r] * inv[r]) * wv[c];
                xv[c][r] = xn;
                amax[r] = abs_max4(amax[r], xn);
            }
        }
        float rcp[kRowsPerWave];
#pragma unroll
        for (int r = 0; r < kRowsPerWave; ++r) {
            float m = wave_max(amax[r]);
            m = m < 1e-8f ? 1.0f : m;  // kore-btes/src/quantize.rs:10
            amax[r] = m;
            rcp[r] = 1.0f / m;
        }
        float my_amax = amax[0];
#pragma unroll
        for (int r = 1; r < kRowsPerWave; ++r) my_amax = lane == r ? amax[r] : my_amax;
        if (lane < nrows) args.scale[row0 + lane] = my_amax / 127.0f;
        uint32_t* q4 = reinterpret_cast<uint32_t*>(args.q) + row0 * cols4;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const uint32_t c4 = (uint32_t)c * kWave + lane;
            if (c < nch && c4 < cols4) {
#pragma unroll
                for (int r = 0; r < kRowsPerWave; ++r) {
                    if (r < nrows) {
                        const f32x4 v = xv[c][r];
                        uint32_t p = quant_code(v.x, amax[r], rcp[r]) | (quant_code(v.y, amax[r], rcp[r]) << 8) |
                                     (quant_code(v.z, amax[r], rcp[r]) << 16) |
                                     (quant_code(v.w, amax[r], rcp[r]) << 24);
                        q4[(uint64_t)r * cols4 + c4] = p;
                    }
                }
            }
        }
    }
}

// Scalar path for any shape/alignment: one thread per row, the reference loop
// verbatim.  Used for cols % 4 != 0, unaligned views and very long rows.
template <NormOut Out>
__global__ __launch_bounds__(64) void row_norm_scalar_kernel(NormArgs args) {
    const uint64_t row = (uint64_t)blockIdx.x * 64 + threadIdx.x;
    if (row >= args.rows) return;
    const uint32_t cols = args.cols;
    const float* xr = args.x + row * cols;
    float ss = 0.0f;
    for (uint32_t i = 0; i < cols; ++i) {
        float sq = xr[i] * xr[i];
        ss = ss + sq;
    }
    float rms = sqrtf(ss / (float)cols + args.eps);
    float inv = 1.0f / rms;
    if (Out == NormOut::F32) {
        float* yr = args.y + row * cols;
        for (uint32_t i = 0; i < cols; ++i) yr[i] = (xr[i] * inv) * args.w[i];
    } else {
        float m = 0.0f;
        for (uint32_t i = 0; i < cols; ++i) m = fmaxf(m, fabsf((xr[i] * inv) * args.w[i]));
        m = m < 1e-8f ? 1.0f : m;
        float rc = 1.0f / m;
        int8_t* qr = args.q + row * cols;
        for (uint32_t i = 0; i < cols; ++i) qr[i] = (int8_t)quant_code((xr[i] * inv) * args.w[i], m, rc);
        args.scale[row] = m / 127.0f;
    }
}

template <NormOut Out>
static int norm_launch(const NormArgs& a, hipStream_t s) {
    if (a.rows == 0) return KORE_HIP_OK;
    if (a.cols == 0) return KORE_HIP_ERR_BAD_DIM;
    if (!a.x || !a.w) return KORE_HIP_ERR_NULL_PTR;
    if (Out == NormOut::F32 && !a.y) return KORE_HIP_ERR_NULL_PTR;
    if (Out == NormOut::I8 && (!a.q || !a.scale)) return KORE_HIP_ERR_NULL_PTR;
    uint64_t elems;
    if (!mul_ok(a.rows, a.cols, &elems) || elems > kMaxElements) return KORE_HIP_ERR_OVERFLOW;
    const uint32_t cols4 = a.cols / 4;
    const int nch = (int)((cols4 + kWave - 1) / kWave);
    bool vec = a.cols % 4 == 0 && aligned16(a.x) && aligned16(a.w) && nch <= 16;
    if (Out == NormOut::F32) vec = vec && aligned16(a.y);
    else vec = vec && (reinterpret_cast<uintptr_t>(a.q) & 3u) == 0;
    if (!vec) {
        uint64_t blocks = (a.rows + 63) / 64;
        if (blocks > 0x7fffffffull) return KORE_HIP_ERR_OVERFLOW;
        hipLaunchKernelGGL(row_norm_scalar_kernel<Out>, dim3((uint32_t)blocks), dim3(64), 0, s, a);
        return launch_status();
    }
    const uint64_t rows_per_block = (uint64_t)kWavesPerBlock * kRowsPerWave;
    const uint64_t blocks = (a.rows + rows_per_block - 1) / rows_per_block;
    if (blocks > 0x7fffffffull) return KORE_HIP_ERR_OVERFLOW;
    dim3 grid((uint32_t)blocks), block(kNormBlock);
#define KORE_NORM_CASE(N)                                                           \
    if (nch <= N) {                                                                 \
        hipLaunchKernelGGL((row_norm_kernel<Out, N>), grid, block, 0, s, a);         \
        return launch_status();                                                     \
    }
    KORE_NORM_CASE(1)
    KORE_NORM_CASE(2)
    KORE_NORM_CASE(4)
    KORE_NORM_CASE(8)
    KORE_NORM_CASE(10)
    KORE_NORM_CASE(12)
    KORE_NORM_CASE(16)
#undef KORE_NORM_CASE
    return KORE_HIP_ERR_BAD_DIM;
}

}  // namespace kore

using namespace kore;

extern "C" int kore_hip_rms_norm_f32(const float* x, const float* weight, float* out, uint64_t rows,
                                     uint64_t cols, float eps, kore_stream_t stream) {
    if (cols > 0xffffffffull) return KORE_HIP_ERR_OVERFLOW;
    NormArgs a{x, weight, out, nullptr, nullptr, rows, (uint32_t)cols, eps};
    return norm_launch<NormOut::F32>(a, (hipStream_t)stream);
}

extern "C" int kore_hip_rms_norm_quant_i8(const float* x, const float* weight, int8_t* q, float* scale,
                                          uint64_t rows, uint64_t cols, float eps, kore_stream_t stream) {
    if (cols > 0xffffffffull) return KORE_HIP_ERR_OVERFLOW;
    NormArgs a{x, weight, nullptr, q, scale, rows, (uint32_t)cols, eps};
    return norm_launch<NormOut::I8>(a, (hipStream_t)stream);
}
