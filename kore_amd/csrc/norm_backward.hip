// norm_backward.hip -- RMSNorm backward: dx and dgamma in one pass over the
// rows plus a small deterministic column reduction.
//
// Definition: crates/kore-kernels/src/cpu_fused_backward.rs:20-81
// (fused_rms_norm_backward), per row r with d = cols:
//   sum_sq = sum_i x^2;  inv = 1 / sqrt(sum_sq / d + eps)
//   dgamma[i] += (dy[i] * x[i]) * inv                 (accumulated over rows)
//   dot = sum_i (x[i] * dy[i]) * g[i]
//   coeff = (dot * inv) / (sum_sq + eps * d)
//   dx[i] = (g[i] * inv) * dy[i] - coeff * x[i]
// Sums are tree reductions (f32 tolerance; the reference has no GPU version).
//
// Roofline: HBM.  Algorithmic bytes: x and dy read once, dx written once
// (12 * rows * cols), plus gamma and dgamma.  The dgamma partials add
// 2 * P * cols * 4 bytes (P = the workgroup count, ~512 for large batches:
// 2% of the traffic at 16384 x 2048).
//
// Vector path (cols % 4 == 0, 16-byte aligned, cols <= 4096):
//   1. rms_bwd_rows_kernel: a row is split over S = 1, 2 or 4 waves (at
//      most 4 float4 columns per wave and operand); a workgroup of 4 waves
//      runs up to 16 row iterations with the next row's loads in flight;
//      gamma is staged in LDS; each wave's dgamma partial stays in
//      registers; the row slots' partials are added in a fixed order through
//      LDS and written as workspace row p = the block index.
//   2. rms_bwd_reduce_kernel: 8 float4 columns x 64 row slots per block;
//      every slot adds its partial rows in order (16 loads in flight), then
//      a fixed-shape tree adds the slots -> dgamma (deterministic).
// Generic path (any shape): one workgroup per row writes dx and inv[r] to the
// workspace; then one thread per column folds its dgamma over the rows in
// the reference's order.
#include <mutex>

#include "common.hpp"
#include "kore_hip_internal.hpp"

namespace kore {

constexpr int kBwBlock = 256;
constexpr int kBwWaves = kBwBlock / kWave;

struct BwArgs {
    const float* dy;
    const float* x;
    const float* g;
    float* dx;
    float* dgamma;
    float* ws;
    uint64_t rows;
    uint64_t cols;
    float eps;
    uint32_t rpw;       // row iterations per workgroup (vector path)
    uint64_t partials;  // P
};

__device__ __forceinline__ float sum4(f32x4 a) { return (a.x + a.y) + (a.z + a.w); }

// A row is split over S waves (wave w: row slot j = w / S, column part
// q = w % S, float4 columns (q*NCHW + k)*64 + lane, k < NCHW), so a wave holds
// at most 4 float4 per operand.  Iteration it of workgroup b takes row
// (it * P + b) * (4/S) + j (P = the grid size), so each iteration of the grid
// sweeps one contiguous band of rows (measured 89 -> 80 us at 16384 x 2048
// against giving each workgroup a contiguous block of rows).  Per row, the S waves' partial sums meet in LDS (slot
// parity double-buffered, one barrier per iteration) and are added in q
// order.  Each wave keeps its dgamma partial in registers; at the end the
// row slots' partials are added in j order through LDS and written as
// workspace row b.
template <int NCHW, int S>
__global__ __launch_bounds__(kBwBlock) __attribute__((amdgpu_waves_per_eu(4))) void rms_bwd_rows_kernel(BwArgs a) {
    constexpr int kSlots = kBwWaves / S;
    extern __shared__ f32x4 part[];  // [cols4] dgamma combine, then [cols4] gamma
    f32x4* gam = part + (a.cols >> 2);
    __shared__ float red[2][kBwWaves][2];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int j = wave / S, q = wave % S;
    const uint32_t cols4 = (uint32_t)(a.cols >> 2);
    const float fcols = (float)a.cols;
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    // iteration it of block b: row (it * P + b) * slots + j -- the grid sweeps
    // one contiguous band of rows per iteration.
    const uint64_t rstride = (uint64_t)gridDim.x * kSlots;
    const uint64_t rbase = (uint64_t)blockIdx.x * kSlots;

    f32x4 acc[NCHW];
#pragma unroll
    for (int k = 0; k < NCHW; ++k) acc[k] = zero;
    // Row loads are double-buffered: iteration it + 1's x and dy are in
    // flight while iteration it reduces, synchronises and stores.
    f32x4 xv[NCHW], dv[NCHW];
    auto load_row = [&](uint32_t it, f32x4* xo, f32x4* dout) {
        const uint64_t r = rbase + (uint64_t)it * rstride + j;
        const bool live = it < a.rpw && r < a.rows;
        const uint64_t rr = live ? r : 0;
        const f32x4* xr = reinterpret_cast<const f32x4*>(a.x) + rr * cols4;
        const f32x4* dr = reinterpret_cast<const f32x4*>(a.dy) + rr * cols4;
#pragma unroll
        for (int k = 0; k < NCHW; ++k) {
            const uint32_t f = (uint32_t)(q * NCHW + k) * kWave + lane;
            xo[k] = (live && f < cols4) ? ld_stream(xr + f) : zero;
            dout[k] = (live && f < cols4) ? ld_stream(dr + f) : zero;
        }
    };
    load_row(0, xv, dv);
    // gamma lives in LDS for the whole sweep: its reads are LDS operations,
    // so they neither hold registers nor make a wait for them also wait for
    // the prefetched row.
    for (uint32_t f = threadIdx.x; f < cols4; f += kBwBlock) gam[f] = reinterpret_cast<const f32x4*>(a.g)[f];
    __syncthreads();
    for (uint32_t it = 0; it < a.rpw; ++it) {
        const uint64_t r = rbase + (uint64_t)it * rstride + j;
        const bool live = r < a.rows;
        f32x4 xn[NCHW], dn[NCHW];
        load_row(it + 1, xn, dn);
        float ss = 0.0f, dot = 0.0f;
#pragma unroll
        for (int k = 0; k < NCHW; ++k) {
            const uint32_t f = (uint32_t)(q * NCHW + k) * kWave + lane;
            ss += sum4(xv[k] * xv[k]);
            dot += sum4((xv[k] * dv[k]) * gam[f < cols4 ? f : 0]);
        }
        ss = wave_sum_dpp(ss);
        dot = wave_sum_dpp(dot);
        if (S > 1) {
            const int par = it & 1;
            if (lane == 0) {
                red[par][wave][0] = ss;
                red[par][wave][1] = dot;
            }
            __syncthreads();
            ss = red[par][j * S][0];
            dot = red[par][j * S][1];
#pragma unroll
            for (int t = 1; t < S; ++t) {
                ss += red[par][j * S + t][0];
                dot += red[par][j * S + t][1];
            }
        }
        const float inv = 1.0f / sqrtf(ss / fcols + a.eps);
        const float coeff = (dot * inv) / (ss + a.eps * fcols);
        if (live) {
            f32x4* orow = reinterpret_cast<f32x4*>(a.dx) + r * cols4;
#pragma unroll
            for (int k = 0; k < NCHW; ++k) {
                const uint32_t f = (uint32_t)(q * NCHW + k) * kWave + lane;
                if (f < cols4) st_stream(orow + f, (gam[f] * inv) * dv[k] - coeff * xv[k]);
                acc[k] = acc[k] + (dv[k] * xv[k]) * inv;
            }
        }
#pragma unroll
        for (int k = 0; k < NCHW; ++k) {
            xv[k] = xn[k];
            dv[k] = dn[k];
        }
    }
    // Row slots' partials added in j order through LDS, then one partial row.
#pragma unroll 1
    for (int jj = 0; jj < kSlots; ++jj) {
        if (j == jj) {
#pragma unroll
            for (int k = 0; k < NCHW; ++k) {
                const uint32_t f = (uint32_t)(q * NCHW + k) * kWave + lane;
                if (f < cols4) part[f] = (jj == 0) ? acc[k] : part[f] + acc[k];
            }
        }
        __syncthreads();
    }
    f32x4* wrow = reinterpret_cast<f32x4*>(a.ws) + (uint64_t)blockIdx.x * cols4;
    for (uint32_t f = threadIdx.x; f < cols4; f += kBwBlock) wrow[f] = part[f];
}

// dgamma = sum of the P partial rows, deterministic: block = 8 float4
// columns (128 contiguous bytes of a partial row) x 64 row slots; thread
// (slot, c) adds rows slot, slot+64, ... in order, with 16 loads in flight;
// the 64 slot sums are then added by a fixed-shape tree in LDS.  The order
// depends only on P, so repeated calls give identical bits.
constexpr int kRedCols = 8;
constexpr int kRedSlots = 64;
constexpr int kRedBatch = 16;
__global__ __launch_bounds__(kRedCols * kRedSlots) void rms_bwd_reduce_kernel(BwArgs a) {
    __shared__ f32x4 red[kRedSlots][kRedCols];
    const uint64_t cols4 = a.cols >> 2;
    const int c = threadIdx.x % kRedCols;
    const int slot = threadIdx.x / kRedCols;
    const uint64_t col = (uint64_t)blockIdx.x * kRedCols + c;
    const f32x4* w4 = reinterpret_cast<const f32x4*>(a.ws);
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    f32x4 t = zero;
    if (col < cols4) {
        for (uint64_t p0 = slot; p0 < a.partials; p0 += kRedBatch * kRedSlots) {
            f32x4 v[kRedBatch];
#pragma unroll
            for (int u = 0; u < kRedBatch; ++u) {
                const uint64_t p = p0 + (uint64_t)u * kRedSlots;
                v[u] = p < a.partials ? w4[p * cols4 + col] : zero;
            }
#pragma unroll
            for (int u = 0; u < kRedBatch; ++u) {
                if (p0 + (uint64_t)u * kRedSlots < a.partials) t = t + v[u];
            }
        }
    }
    red[slot][c] = t;
    __syncthreads();
#pragma unroll
    for (int w = kRedSlots / 2; w >= 1; w >>= 1) {
        if (slot < w) red[slot][c] = red[slot][c] + red[slot + w][c];
        __syncthreads();
    }
    if (slot == 0 && col < cols4) reinterpret_cast<f32x4*>(a.dgamma)[col] = red[0][c];
}

// ---- generic path
__global__ __launch_bounds__(kBwBlock) void rms_bwd_row_generic_kernel(BwArgs a) {
    __shared__ float red[2][kBwWaves];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const uint64_t r = blockIdx.x;
    const float* xr = a.x + r * a.cols;
    const float* dr = a.dy + r * a.cols;
    float ss = 0.0f, dot = 0.0f;
    for (uint64_t i = threadIdx.x; i < a.cols; i += kBwBlock) {
        const float xv = xr[i];
        ss += xv * xv;
        dot += (xv * dr[i]) * a.g[i];
    }
    ss = wave_sum(ss);
    dot = wave_sum(dot);
    if (lane == 0) {
        red[0][wave] = ss;
        red[1][wave] = dot;
    }
    __syncthreads();
    ss = red[0][0];
    dot = red[1][0];
#pragma unroll
    for (int w = 1; w < kBwWaves; ++w) {
        ss += red[0][w];
        dot += red[1][w];
    }
    const float fcols = (float)a.cols;
    const float inv = 1.0f / sqrtf(ss / fcols + a.eps);
    const float coeff = (dot * inv) / (ss + a.eps * fcols);
    for (uint64_t i = threadIdx.x; i < a.cols; i += kBwBlock)
        a.dx[r * a.cols + i] = (a.g[i] * inv) * dr[i] - coeff * xr[i];
    if (threadIdx.x == 0) a.ws[r] = inv;
}

// One thread per column: dgamma[c] = sum over rows, in row order.
__global__ __launch_bounds__(kBwBlock) void rms_bwd_col_generic_kernel(BwArgs a) {
    const uint64_t c = (uint64_t)blockIdx.x * kBwBlock + threadIdx.x;
    if (c >= a.cols) return;
    float acc = 0.0f;
    for (uint64_t r = 0; r < a.rows; ++r) acc = acc + (a.dy[r * a.cols + c] * a.x[r * a.cols + c]) * a.ws[r];
    a.dgamma[c] = acc;
}

__global__ __launch_bounds__(kBwBlock) void fill_zero_kernel(float* p, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * kBwBlock + threadIdx.x;
    if (i < n) p[i] = 0.0f;
}

static bool bwd_vec(uint64_t cols) { return cols % 4 == 0 && cols / 4 <= 1024; }

// Waves per row for the vector path: each wave holds <= 4 float4 columns.
static uint32_t bwd_split(uint64_t cols) {
    const uint64_t c4 = cols / 4;
    return c4 <= 256 ? 1u : (c4 <= 512 ? 2u : 4u);
}


// Row iterations per workgroup: ~512 workgroups (4 waves each, two per SIMD,
// with the next row's loads in flight) -- measured against 256, 384, 768 and
// 1024 at 16384 x 2048: fewer partial rows to reduce, and enough waves to keep
// HBM busy (70.0 vs 72.7 us at 1024); at most 16 iterations so that large
// batches keep few partial rows.
static uint32_t bwd_iters(uint64_t rows, uint32_t split) {
    const uint64_t per_iter = kBwWaves / split;
    uint64_t it = (rows + 512 * per_iter - 1) / (512 * per_iter);
    if (it < 1) it = 1;
    if (it > 16) it = 16;
    return (uint32_t)it;
}

// Workspace floats for the vector and generic plans (the larger is required).
static uint64_t bwd_ws_floats(uint64_t rows, uint64_t cols, uint64_t* partials, uint32_t* iters) {
    const uint32_t split = bwd_split(cols);
    const uint32_t it = bwd_iters(rows, split);
    const uint64_t rpb = (uint64_t)it * (kBwWaves / split);  // rows per block = per partial row
    const uint64_t p = (rows + rpb - 1) / rpb;
    if (partials) *partials = p;
    if (iters) *iters = it;
    const uint64_t vec = bwd_vec(cols) ? p * cols : 0;
    return vec > rows ? vec : rows;
}

template <int NCHW, int S>
static void launch_rows(const BwArgs& a, hipStream_t s) {
    const size_t lds = 2 * (a.cols / 4) * sizeof(f32x4);
    hipLaunchKernelGGL((rms_bwd_rows_kernel<NCHW, S>), dim3((uint32_t)a.partials), dim3(kBwBlock), lds, s, a);
}

// Library-held scratch for the allocation-free entry point: the dgamma
// partial rows (vector path) or the per-row inv (generic path), at most
// kBwScratchBytes.  Each GPU holds its own copy for the life of the process.
// Every call fully writes the part it reads back, so nothing needs clearing;
// calls that overlap on one GPU share the array and race.
constexpr uint64_t kBwScratchBytes = 16ull << 20;
static __device__ __align__(256) float rms_bwd_scratch[kBwScratchBytes / sizeof(float)];

// Device address of rms_bwd_scratch on the current device, looked up once per
// device with that device current.  In host code the array's name is only a
// host-side stand-in; kernels get this address instead.
constexpr int kMaxScratchDevices = 64;
static std::mutex g_bw_scratch_mu;
static float* g_bw_scratch[kMaxScratchDevices];

static int bwd_scratch_ptr(float** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= kMaxScratchDevices) return KORE_HIP_ERR_BAD_DIM;
    std::lock_guard<std::mutex> lock(g_bw_scratch_mu);
    if (!g_bw_scratch[dev]) {
        // The first call on a device may come from code under stream capture.
        // The lookup enqueues nothing, but a strict capture mode can refuse
        // runtime calls it does not know to be safe: this thread switches to
        // relaxed mode for the lookup and restores its mode afterwards.
        hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
        e = hipThreadExchangeStreamCaptureMode(&mode);
        if (e != hipSuccess) return (int)e;
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(rms_bwd_scratch));
        const hipError_t r = hipThreadExchangeStreamCaptureMode(&mode);
        if (e != hipSuccess) return (int)e;
        if (r != hipSuccess) return (int)r;
        g_bw_scratch[dev] = static_cast<float*>(p);
    }
    *out = g_bw_scratch[dev];
    return KORE_HIP_OK;
}

}  // namespace kore

using namespace kore;

extern "C" uint64_t kore_hip_rms_norm_backward_workspace_bytes(uint64_t rows, uint64_t cols) {
    if (rows == 0 || cols == 0) return 0;
    uint64_t elems;
    if (!mul_ok(rows, cols, &elems) || elems > kMaxElements) return 0;
    return bwd_ws_floats(rows, cols, nullptr, nullptr) * sizeof(float);
}

// The whole entry point once the workspace is known.  ws == nullptr asks for
// the library's own scratch array (the allocation-free entry point); it is
// looked up only after every argument check has passed.
static int rms_bwd_run(const float* grad_out, const float* x, const float* gamma, float* grad_x,
                       float* grad_gamma, float* workspace, uint64_t workspace_bytes, bool own_scratch,
                       uint64_t rows, uint64_t cols, float eps, hipStream_t s) {
    if (cols == 0) return KORE_HIP_OK;
    if (!grad_gamma || !gamma) return KORE_HIP_ERR_NULL_PTR;
    if (rows == 0) {  // dgamma of an empty batch is zero (the reference's vec![0.0; d])
        if (cols > kMaxElements) return KORE_HIP_ERR_OVERFLOW;
        // A fill kernel rather than hipMemsetAsync, so the call can be captured in a graph.
        hipLaunchKernelGGL(fill_zero_kernel, dim3((uint32_t)((cols + kBwBlock - 1) / kBwBlock)), dim3(kBwBlock), 0, s,
                           grad_gamma, cols);
        return launch_status();
    }
    if (!grad_out || !x || !grad_x || (!own_scratch && !workspace)) return KORE_HIP_ERR_NULL_PTR;
    uint64_t elems;
    if (!mul_ok(rows, cols, &elems) || elems > kMaxElements || rows > 0x7fffffffull) return KORE_HIP_ERR_OVERFLOW;
    BwArgs a{grad_out, x, gamma, grad_x, grad_gamma, workspace, rows, cols, eps, 0, 0};
    const uint64_t need = bwd_ws_floats(rows, cols, &a.partials, &a.rpw) * sizeof(float);
    if (own_scratch) {
        if (need > kBwScratchBytes) return KORE_HIP_ERR_SCRATCH;
        workspace_bytes = kBwScratchBytes;
    } else if (workspace_bytes < need) {
        return KORE_HIP_ERR_BAD_DIM;
    }
    // grad_x must not overlap the inputs (the row pass reads a row ahead).
    const char* o0 = (const char*)grad_x;
    const char* o1 = o0 + elems * sizeof(float);
    for (const float* in : {grad_out, x}) {
        const char* i0 = (const char*)in;
        if (i0 < o1 && o0 < i0 + elems * sizeof(float)) return KORE_HIP_ERR_ALIAS;
    }
    if (own_scratch) {
        const int st = bwd_scratch_ptr(&a.ws);
        if (st != KORE_HIP_OK) return st;
        workspace = a.ws;
    }
    const bool vec = bwd_vec(cols) && aligned16(grad_out) && aligned16(x) && aligned16(gamma) &&
                     aligned16(grad_x) && aligned16(grad_gamma) && aligned16(workspace);
    if (vec) {
        const uint64_t cols4 = cols / 4;
        if (cols4 <= 64) launch_rows<1, 1>(a, s);
        else if (cols4 <= 128) launch_rows<2, 1>(a, s);
        else if (cols4 <= 256) launch_rows<4, 1>(a, s);
        else if (cols4 <= 512) launch_rows<4, 2>(a, s);
        else launch_rows<4, 4>(a, s);
        hipLaunchKernelGGL(rms_bwd_reduce_kernel, dim3((uint32_t)((cols4 + kRedCols - 1) / kRedCols)),
                           dim3(kRedCols * kRedSlots), 0, s, a);
    } else {
        hipLaunchKernelGGL(rms_bwd_row_generic_kernel, dim3((uint32_t)rows), dim3(kBwBlock), 0, s, a);
        hipLaunchKernelGGL(rms_bwd_col_generic_kernel, dim3((uint32_t)((cols + kBwBlock - 1) / kBwBlock)),
                           dim3(kBwBlock), 0, s, a);
    }
    return launch_status();
}

extern "C" int kore_hip_rms_norm_backward_f32(const float* grad_out, const float* x, const float* gamma,
                                              float* grad_x, float* grad_gamma, float* workspace,
                                              uint64_t workspace_bytes, uint64_t rows, uint64_t cols, float eps,
                                              kore_stream_t stream) {
    return rms_bwd_run(grad_out, x, gamma, grad_x, grad_gamma, workspace, workspace_bytes, false, rows, cols, eps,
                       (hipStream_t)stream);
}

extern "C" uint64_t kore_hip_rms_norm_backward_noalloc_max_bytes(void) { return kBwScratchBytes; }

extern "C" int kore_hip_rms_norm_backward_noalloc_f32(const float* grad_out, const float* x, const float* gamma,
                                                      float* grad_x, float* grad_gamma, uint64_t rows,
                                                      uint64_t cols, float eps, kore_stream_t stream) {
    return rms_bwd_run(grad_out, x, gamma, grad_x, grad_gamma, nullptr, 0, true, rows, cols, eps,
                       (hipStream_t)stream);
}
