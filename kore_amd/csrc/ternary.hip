// ternary.hip -- BitLinear matmuls on base-243 packed ternary weights.
//
// Weights: a_packed[M, Kp] bytes, Kp = ceil(K/5); byte b holds trits
// t_j = digit_j(b) - 1 (base 3, least significant digit first, j < 5) for
// columns 5*i + j; bytes 243..255 decode to zeros (crates/kore-btes/src/
// encoder.rs:50-95).  a_scales[M] per-row scales.
//
// kore_hip_ternary_matmul_i8: the matmul on the pre-quant codes,
//   c[m, n] = ((float)(sum_k t[m, k] * q[n, k]) * a_scales[m]) * q_scales[n]
// with q[N, K] int8 (one row per token, as kore_hip_rms_norm_quant_i8 writes
// them) and c[M, N] f32; the dot product is exact in int32 and the epilogue
// is the reference's ternary_ternary_matmul one
// (crates/kore-kernels/src/cpu_ternary_matmul.rs:188), so the result is
// bit-exact.
//
// Roofline: MFMA int8 (v_mfma_i32_32x32x32_i8, 5.0 POP/s dense): 2*M*N*K
// operations; the f32 output (4*M*N bytes) is the largest HBM stream.
//
// Vector path (K % 16 == 0, q 16-byte aligned, c 4-byte aligned; packed rows
// are read as 16-byte vectors when Kp % 16 == 0, else byte by byte):
//   workgroup = 4 waves, 128 (m) x 128 (n) outputs, each wave 64 x 64 as
//   2 x 2 MFMA tiles of 32 x 32; K advances 160 columns (32 packed bytes =
//   five 32-deep MFMA steps) per iteration.  Per iteration every thread
//   decodes 16 packed bytes into 80 trit bytes through a 256-entry LDS table
//   (byte -> five int8 trits) and stages 5 x 16 bytes of q; both tiles sit
//   in LDS at a 176-byte row pitch (44 dwords: 16 lanes reading 16 bytes at
//   consecutive rows hit 16 distinct bank groups).  The next iteration's
//   global loads are in flight while the current one computes.
//   MFMA operands: lane l reads row l % 32 and 16 bytes at k = 16 * (l / 32)
//   of a 32-deep step from both tiles (the k order inside an MFMA is the
//   same for both operands, so any assignment gives the same sum);
//   accumulator register r of lane l is row 8*(r/4) + 4*(l/32) + r%4,
//   column l % 32.
// n <= 8: the small-n path (dot4 on decoded windows, no MFMA); 8 < n <= 64:
// the skinny path (32 weight rows per workgroup, K split over its waves and
// summed exactly in LDS); at least 144 tiles of 256 x 256: the wide kernel
// (below); few output tiles beyond that: the tile kernel over
// K ranges, summed with exact int32 atomics into the output (zeroed first,
// finished in place).  Code rows that are not 16-byte aligned (K % 16 != 0
// or an unaligned q) take the tile kernel with dword-window loads.
// Generic path (K = 0, or an output not 4-byte aligned): one thread per
// output, the reference loop order.
//
// kore_hip_ternary_matmul_f32: the reference's f32-activation ternary_matmul,
// a sequential fold per output (at the end): ternary_f32_mfma_kernel (fp32
// matrix cores, 16 x 16 x 1) for prefill-sized shapes,
// ternary_f32_mf4_kernel (4 x 4 x 1) for the layer's token-major input at
// 41-192 tokens, ternary_f32_rows_kernel for five columns and more,
// ternary_f32_pipe_kernel for one to four columns, ternary_f32_seq_kernel for
// K = 0 and matrices of fewer than 20 packed bytes.
#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "kore_hip_internal.hpp"

namespace kore {

typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kTmBlock = 256;
constexpr int kTmM = 128, kTmN = 128;  // workgroup tile; each wave 64 x 64
constexpr int kTmK = 160;          // trit columns per iteration
constexpr int kTmKp = kTmK / 5;    // packed bytes per iteration
constexpr int kTmPitch = 176;      // LDS row pitch in bytes
constexpr uint32_t kZeroByte = 121;  // encodes five zero trits
constexpr uint32_t kXcds = 8;        // MI355X: 8 XCDs, one L2 each
constexpr uint32_t kGroupM = 8;      // m-tiles per tile group

struct TernArgs {
    const uint8_t* a;   // packed [M, Kp]
    const float* sa;    // [M]
    const int8_t* q;    // [N, K]
    const float* sq;    // [N]
    float* c;           // [M, N], or [N, M] with trans
    uint32_t m, n, k, kp;
    uint32_t splits, kt_per;  // split-K: K-tile ranges of kt_per per workgroup
    const float* bias;  // [M] added to every output of row m, or null
    uint32_t trans;     // 1: output (m, n) at c[n * M + m] (BitLinear::forward's layout)
};

// Index of output (m, n) in c, and the layer's bias add: the output is
// rounded first, then the bias is added to it (bit_linear.rs:220-224 adds
// the bias to the finished matmul output).
__device__ __forceinline__ uint64_t out_idx(const TernArgs& p, uint32_t m, uint32_t n) {
    return p.trans ? (uint64_t)n * p.m + m : (uint64_t)m * p.n + n;
}
__device__ __forceinline__ float add_bias(const float* bias, float v, uint32_t m) { return bias ? v + bias[m] : v; }

// An MFMA with the weight and code operands in either order: kTrans puts
// the codes first, so that accumulator rows run over n and lanes over m --
// the transposed output's contiguous dimension.  The int32 sums are the same
// either way (exact integer arithmetic).
template <bool kTrans>
__device__ __forceinline__ i32x16 mfma_wq(i32x4 w, i32x4 q, i32x16 acc) {
    return kTrans ? __builtin_amdgcn_mfma_i32_32x32x32_i8(q, w, acc, 0, 0, 0)
                  : __builtin_amdgcn_mfma_i32_32x32x32_i8(w, q, acc, 0, 0, 0);
}

// Sixteen bytes at a dword boundary: global loads need dword alignment only.
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

// Five trits of byte b as int8 in the low 40 bits (byte j = trit j).
__device__ __forceinline__ uint64_t trit_lut_entry(uint32_t b) {
    if (b >= 243u) return 0;
    uint64_t v = 0;
#pragma unroll
    for (int j = 0; j < 5; ++j) {
        const uint32_t d = b % 3u;
        b /= 3u;
        v |= (uint64_t)(uint8_t)(int8_t)((int)d - 1) << (8 * j);
    }
    return v;
}

// kAlignedA: packed rows are 16-byte aligned (Kp % 16 == 0) and read as
// dwordx4; otherwise as the five dwords around the 16 bytes, shifted into
// place (a row's last partial piece, and the matrix's last bytes, byte by
// byte).
// kSplit: the workgroup covers K-tiles [split * kt_per, (split + 1) * kt_per)
// of its output tile and adds its int32 sums into c (zeroed, read as int32)
// with integer atomics -- exact and order-free, so the result is the same on
// every run; ternary_i8_finish_kernel then applies the epilogue in place.
template <bool kAlignedA, bool kAlignedB, bool kSplit, bool kTrans>
__global__ __launch_bounds__(kTmBlock) void ternary_i8_mfma_kernel(TernArgs p) {
    __shared__ uint64_t lut[256];
    __shared__ __attribute__((aligned(16))) uint8_t As[kTmM * kTmPitch];
    __shared__ __attribute__((aligned(16))) uint8_t Bs[kTmN * kTmPitch];
    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const int wave = t / kWave;
    const int wm = wave >> 1, wn = wave & 1;
    // Tile order: workgroups are dispatched round-robin over the 8 XCDs
    // (block b runs on XCD b % 8), each with its own L2.  XCD x takes the
    // contiguous range [x * per, (x + 1) * per) of a grouped tile order
    // (groups of kGroupM m-tiles, m fastest inside a group), so the tiles a
    // CU's neighbours work on share weights and codes in that XCD's L2.
    const uint32_t tm_n = (p.m + kTmM - 1) / kTmM, tn_n = (p.n + kTmN - 1) / kTmN;
    const uint32_t ntiles = tm_n * tn_n;
    const uint32_t nwork = ntiles * (kSplit ? p.splits : 1u);
    const uint32_t per = (nwork + kXcds - 1) / kXcds;
    const uint32_t work = (blockIdx.x % kXcds) * per + blockIdx.x / kXcds;
    if (work >= nwork) return;  // whole workgroup: no barrier reached yet
    const uint32_t lin = kSplit ? work / p.splits : work;
    const uint32_t kt_lo = kSplit ? (work % p.splits) * p.kt_per : 0u;
    const uint32_t grp = lin / (kGroupM * tn_n);
    const uint32_t first_m = grp * kGroupM;
    const uint32_t gsz = min(tm_n - first_m, (uint32_t)kGroupM);
    const uint32_t in_grp = lin % (kGroupM * tn_n);
    const uint32_t m0 = (first_m + in_grp % gsz) * kTmM, n0 = (in_grp / gsz) * kTmN;
    lut[t] = trit_lut_entry((uint32_t)t);

    // A staging: thread t decodes packed bytes [16h, 16h + 16) of tile row r.
    const int ar = t >> 1, ah = t & 1;
    const bool arow_ok = m0 + ar < p.m;
    const uint8_t* arow8 = p.a + (uint64_t)(arow_ok ? m0 + ar : 0) * p.kp;
    const u32x4* arow = reinterpret_cast<const u32x4*>(arow8);
    // B staging: 16-byte pieces c = t + 256u (u < 5) of the 128 x 160 tile.
    const uint32_t nkt_all = (p.k + kTmK - 1) / kTmK;
    const uint32_t nkt = kSplit ? min(nkt_all, kt_lo + p.kt_per) : nkt_all;
    const u32x4 zero_bytes = {kZeroByte * 0x01010101u, kZeroByte * 0x01010101u, kZeroByte * 0x01010101u,
                              kZeroByte * 0x01010101u};
    const u32x4 zero4 = {0u, 0u, 0u, 0u};

    const uintptr_t a_hi = reinterpret_cast<uintptr_t>(p.a) + (uintptr_t)p.m * p.kp;
    const uintptr_t q_hi = reinterpret_cast<uintptr_t>(p.q) + (uintptr_t)p.n * p.k;
    // Unaligned rows (packed weights) and code rows (K % 16 != 0 or an
    // unaligned q): each 16-byte piece is loaded as the 20 bytes from the
    // dword boundary below it (x and its fifth dword e) and shifted into
    // place only when it is staged, after the barrier that waits for the
    // loads anyway: a shift right after the loads would wait on every load
    // in flight.  The shift is fixed per piece slot (pieces start at
    // multiples of 16 bytes of a row).  Only where the 20 bytes would pass a
    // matrix's end are they read byte by byte.  Code bytes at columns >= k
    // (and code rows past n, read clamped to row n - 1) are zeroed at
    // staging; weight bytes past a row's end meet only those zero codes.
    auto load20 = [&](uintptr_t w0, uintptr_t hi, u32x4& x, uint32_t& e) {
        if (__builtin_expect(w0 + 20u <= hi, 1)) {
            x = *reinterpret_cast<const u32x4_a4*>(w0);
            e = *reinterpret_cast<const uint32_t*>(w0 + 16);
        } else {
            uint32_t w[5];
#pragma unroll
            for (int d = 0; d < 5; ++d) {
                w[d] = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uintptr_t o = w0 + 4 * d + j;
                    w[d] |= (o < hi ? (uint32_t)*reinterpret_cast<const uint8_t*>(o) : 0u) << (8 * j);
                }
            }
            x = u32x4{w[0], w[1], w[2], w[3]};
            e = w[4];
        }
    };
    auto shift20 = [](const u32x4& x, uint32_t e, uint32_t sh) {
        return u32x4{__builtin_amdgcn_alignbyte(x[1], x[0], sh), __builtin_amdgcn_alignbyte(x[2], x[1], sh),
                     __builtin_amdgcn_alignbyte(x[3], x[2], sh), __builtin_amdgcn_alignbyte(e, x[3], sh)};
    };
    const uint32_t sh_a = (uint32_t)(reinterpret_cast<uintptr_t>(arow8) & 3u);
    uint32_t sh_b[5];
    const int8_t* brow[5];
#pragma unroll
    for (int u = 0; u < 5; ++u) {
        const int c = t + kTmBlock * u;
        const uint32_t rowc = min(n0 + (uint32_t)(c / 10), p.n - 1u);
        brow[u] = p.q + (uint64_t)rowc * p.k + 16u * (uint32_t)(c % 10);
        sh_b[u] = (uint32_t)(reinterpret_cast<uintptr_t>(brow[u]) & 3u);
    }
    auto load_b = [&](uint32_t kt, u32x4* bv, uint32_t* be) {
#pragma unroll
        for (int u = 0; u < 5; ++u) {
            const int c = t + kTmBlock * u;
            const int row = c / 10, piece = c % 10;
            const uint32_t kb = kt * kTmK + 16u * piece;
            if (kAlignedB) {
                const bool ok = n0 + row < p.n && kb < p.k;
                bv[u] = ok ? *reinterpret_cast<const u32x4*>(p.q + (uint64_t)(n0 + row) * p.k + kb) : zero4;
                continue;
            }
            load20(reinterpret_cast<uintptr_t>(brow[u] + kt * kTmK) & ~(uintptr_t)3, q_hi, bv[u], be[u]);
        }
    };
    auto load_tile = [&](uint32_t kt, u32x4& av, uint32_t& ae, u32x4* bv, uint32_t* be) {
        const uint32_t ab = kt * kTmKp + 16u * ah;  // packed byte offset
        if (kAlignedA)
            av = (arow_ok && ab < p.kp) ? arow[ab >> 4] : zero_bytes;
        else
            load20(reinterpret_cast<uintptr_t>(arow8 + ab) & ~(uintptr_t)3, a_hi, av, ae);
        load_b(kt, bv, be);
    };

    i32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

    u32x4 av, bv[5];
    uint32_t ae = 0u, be[5] = {0u, 0u, 0u, 0u, 0u};
    load_tile(kt_lo, av, ae, bv, be);
    for (uint32_t kt = kt_lo; kt < nkt; ++kt) {
        __syncthreads();  // previous tile's MFMA reads (and the LUT fill) are done
        if (!kAlignedA) av = shift20(av, ae, sh_a);
        if (!kAlignedB) {
#pragma unroll
            for (int u = 0; u < 5; ++u) {
                const int c = t + kTmBlock * u;
                const int row = c / 10, piece = c % 10;
                // bytes of the piece to keep: columns below k of a row below n
                const int keep = n0 + row < p.n ? (int)p.k - (int)(kt * kTmK + 16u * piece) : 0;
                u32x4 x = shift20(bv[u], be[u], sh_b[u]);
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const int kd = keep - 4 * d;
                    x[d] &= kd >= 4 ? 0xffffffffu : (kd <= 0 ? 0u : (0xffffffffu >> (8 * (4 - kd))));
                }
                bv[u] = x;
            }
        }
        // decode 16 packed bytes -> 80 trit bytes, little-endian in 20 dwords
        uint32_t out[20];
#pragma unroll
        for (int d = 0; d < 20; ++d) out[d] = 0;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t b = (av[i >> 2] >> (8 * (i & 3))) & 0xffu;
            const uint64_t v = lut[b];
            const int off = 5 * i, d = off >> 2, sh = (off & 3) * 8;
            out[d] |= (uint32_t)(v << sh);
            out[d + 1] |= (uint32_t)(v >> (32 - sh));
        }
        u32x4* adst = reinterpret_cast<u32x4*>(As + ar * kTmPitch + ah * 80);
#pragma unroll
        for (int w = 0; w < 5; ++w) {
            const u32x4 o = {out[4 * w], out[4 * w + 1], out[4 * w + 2], out[4 * w + 3]};
            adst[w] = o;
        }
#pragma unroll
        for (int u = 0; u < 5; ++u) {
            const int c = t + kTmBlock * u;
            const int row = c / 10, piece = c % 10;
            *reinterpret_cast<u32x4*>(Bs + row * kTmPitch + 16 * piece) = bv[u];
        }
        __syncthreads();
        if (kt + 1 < nkt) load_tile(kt + 1, av, ae, bv, be);
#pragma unroll
        for (int s = 0; s < 5; ++s) {
            const int koff = 32 * s + 16 * (lane >> 5);
            i32x4 a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                a[i] = *reinterpret_cast<const i32x4*>(As + (wm * 64 + i * 32 + (lane & 31)) * kTmPitch + koff);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                b[j] = *reinterpret_cast<const i32x4*>(Bs + (wn * 64 + j * 32 + (lane & 31)) * kTmPitch + koff);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = mfma_wq<kTrans>(a[i], b[j], acc[i][j]);
        }
    }

    // epilogue: ((float)acc * sa[m]) * sq[n] (+ bias[m]).  Register r of
    // lane l is row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32 of its
    // 32 x 32 tile: rows over m and columns over n, or (kTrans) the reverse,
    // so that the lanes of a store always run along the output's rows.
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t rr = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3), cc = lane & 31;
                const uint32_t m = m0 + wm * 64 + i * 32 + (kTrans ? cc : rr);
                const uint32_t n = n0 + wn * 64 + j * 32 + (kTrans ? rr : cc);
                if (n < p.n && m < p.m) {
                    const uint64_t o = out_idx(p, m, n);
                    if (kSplit) {
                        atomicAdd(reinterpret_cast<int*>(p.c) + o, acc[i][j][r]);
                    } else {
                        const float v = ((float)acc[i][j][r] * p.sa[m]) * p.sq[n];
                        __builtin_nontemporal_store(add_bias(p.bias, v, m), p.c + o);
                    }
                }
            }
        }
    }
}

// Wide path (at least 144 output tiles, code rows 16-byte aligned (K % 16 == 0), packed rows of any alignment): the
// workgroup owns a 256 (m) x 256 (n) output tile; wave w owns weight rows
// [64 w, 64 w + 64) of it against all 256 code rows: 2 x 8 MFMA tiles of
// 32 x 32 (256 int32 accumulators per lane), one workgroup per CU.
//   * Weights never pass through LDS as data: each lane decodes its own
//     rows' 16 packed bytes per 160-column K step (lane half h owns columns
//     [80 h, 80 h + 80)) straight into the operands of five 32-deep MFMA
//     steps (step s: columns 80 h + 16 s .. + 16, natural order), through a
//     byte -> five-trit table held in 32 copies, copy c serving lanes c and
//     c + 32 and laid out so that every entry of copy c lies in the same two
//     LDS banks: a half-wave's 32 lanes read 32 distinct bank pairs whatever
//     bytes they decode.  The next K step's weights are decoded while the
//     current step's MFMAs run (a fifth of the bytes per MFMA step).
//   * Codes reach LDS by direct global -> LDS loads (no registers), into a
//     double-buffered tile with a 176-byte row pitch (16 lanes reading 16
//     bytes of 16 consecutive rows hit 16 distinct bank groups); the tile of
//     step kt + 1 is loaded into the other buffer during step kt's first
//     MFMA groups; one barrier per step.  Code rows past n are clamped to
//     row n - 1 (their outputs are not stored); columns past k are clamped
//     to the step's first 16 bytes and the weights' trits there are zeroed
//     instead.
//   * The output tile leaves through LDS, 32 rows of a wave at a time, as
//     whole 1 KB rows per store instruction.
// LDS traffic per MFMA is ~0.7 KB (operand reads 0.5, table reads 0.2)
// against the ~1 KB one CU delivers per MFMA of each of its four SIMDs.
constexpr int kWdM = 256, kWdN = 256;
// The wide kernel runs one workgroup per CU; below 144 tiles of 256 x 256
// the 128 x 128 kernel (more, smaller workgroups) is faster: measured wide
// against 128 x 128 at 4096 x 2048 x 2560 (128 tiles) 45.9 vs 39.7 us, and at
// 3072 x 3072 x 2560 (144) 41.2 vs 49.0, 2560 x 4096 x 6912 (160, unaligned
// rows) 107.1 vs 133.6, 6912 x 2048 (216) 49.7 vs 73.7.
constexpr uint64_t kWdMinTiles = 144;
constexpr uint64_t kCus = 256;  // MI355X compute units
constexpr int kWdPitch = 176;
constexpr int kWdCopies = 32;
// A tile of NJ 32-column groups (NJ = 8: 256 columns; 6: 192): its code
// buffer, LDS, and 16-byte code slots and loads per wave and step (the last
// load covering only the slots left).
template <int NJ> struct WideTile {
    static constexpr int kN = 32 * NJ;
    static constexpr size_t kBBytes = (size_t)kN * kWdPitch;
    // the K loop's buffers and table, or the epilogue's four 32-row slabs of
    // 264 floats, whichever is larger
    static constexpr size_t kLoop = 2 * kBBytes + 256 * kWdCopies * 8;
    static constexpr size_t kEpi = (size_t)4 * 32 * 264 * 4;
    static constexpr size_t kLds = kLoop > kEpi ? kLoop : kEpi;
    static constexpr int kSlots = (int)(kBBytes / 16 / 4);
    static constexpr int kDma = (kSlots + kWave - 1) / kWave;
};

typedef __attribute__((address_space(3))) void* lds_vptr;
typedef __attribute__((address_space(1))) void* glb_vptr;

// Trits of byte b of a 16-byte packed window: b's five trits go to bytes
// 5b .. 5b + 4 of the 80-byte (20-dword) decoded window.
__device__ __forceinline__ void splice_trits(uint32_t (&out)[20], int b, uint64_t v) {
    const int off = 5 * b, d = off >> 2, sh = (off & 3) * 8;
    out[d] |= (uint32_t)(v << sh);
    out[d + 1] |= (uint32_t)(v >> (32 - sh));
}

template <bool kAlignedA, int NJ, bool kTrans>
__global__ __launch_bounds__(256, 1) void ternary_i8_wide_kernel(TernArgs p) {
    using Tile = WideTile<NJ>;
    constexpr int kN = Tile::kN;
    constexpr size_t kBB = Tile::kBBytes;
    static_assert(Tile::kLds >= Tile::kEpi && Tile::kLds <= 160 * 1024, "wide kernel LDS");
    constexpr int kSl = Tile::kSlots, kDm = Tile::kDma;
    extern __shared__ __attribute__((aligned(16))) uint8_t wlds[];
    uint64_t* lut = reinterpret_cast<uint64_t*>(wlds + 2 * kBB);
    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
    const int r = lane & 31, h = lane >> 5;
    // Tile order: block b runs on XCD b % 8 and XCD x takes the contiguous
    // range [x * per, (x + 1) * per) of a panel order: panels of pw =
    // ceil(tn / 8) n-tiles, m-major inside a panel.  One XCD then holds about
    // one panel (its code rows once in its L2), and the workgroups it runs at
    // the same time share weight rows pairwise instead of each fetching its own.
    const uint32_t tm_n = (p.m + kWdM - 1) / kWdM, tn_n = (p.n + kN - 1) / kN;
    const uint32_t ntiles = tm_n * tn_n;
    const uint32_t per = (ntiles + kXcds - 1) / kXcds;
    const uint32_t work = (blockIdx.x % kXcds) * per + blockIdx.x / kXcds;
    if (work >= ntiles) return;  // whole workgroup: no barrier reached yet
    const uint32_t pw = (tn_n + kXcds - 1) / kXcds;
    const uint32_t panel = work / (tm_n * pw), within = work % (tm_n * pw);
    const uint32_t pwid = min(pw, tn_n - panel * pw);
    const uint32_t m0 = (within / pwid) * kWdM, n0 = (panel * pw + within % pwid) * kN;

    // Table: entry e, copy c at u64 index e * 32 + c (bank pair 2c).  Thread
    // e fills its entry's copies in a rotated order so that the 64 lanes of a
    // write hit distinct bank pairs.
    {
        const uint64_t v = trit_lut_entry((uint32_t)t);
#pragma unroll 8
        for (int c2 = 0; c2 < kWdCopies; ++c2) lut[t * kWdCopies + ((c2 + t) & (kWdCopies - 1))] = v;
    }
    const uint64_t* lut_lane = lut + r;

    const uint32_t nkt = (p.k + kTmK - 1) / kTmK;
    // This lane's two weight rows (fragments i = 0, 1); rows past m read row
    // m - 1 (their outputs are not stored).
    const uint8_t* arow[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t m = min(m0 + 64 * wave + 32 * i + r, p.m - 1u);
        arow[i] = p.a + (uint64_t)m * p.kp;
    }
    const uintptr_t a_hi = reinterpret_cast<uintptr_t>(p.a) + (uintptr_t)p.m * p.kp;
    // A window past kp (the second half of a last step) reads the row's
    // first window: it lies wholly past k, so its trits are zeroed below.
    // Unaligned rows: the 20 bytes from the dword boundary below the window
    // (av and ae), shifted into place by the row's byte offset sh only where
    // the step decodes them (align_a), so that no wait on these loads -- whose
    // counter the code tiles' loads share -- lands in the step that issues
    // them.  A window that straddles the row's end (last step only) takes the
    // next row's bytes, at columns >= k, zeroed below as well; only where the
    // 20 bytes would pass the matrix's end are they read one by one.
    uint32_t sh[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) sh[i] = (uint32_t)(reinterpret_cast<uintptr_t>(arow[i]) & 3u);
    auto load_a = [&](uint32_t kt, u32x4 (&av)[2], uint32_t (&ae)[2]) {
        const uint32_t ab = kt * kTmKp + 16u * h;
        const uint32_t abc = ab < p.kp ? ab : 0u;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            if (kAlignedA) {
                av[i] = *reinterpret_cast<const u32x4*>(arow[i] + abc);
                continue;
            }
            const uintptr_t w0 = reinterpret_cast<uintptr_t>(arow[i] + abc) & ~(uintptr_t)3;
            if (__builtin_expect(w0 + 20u <= a_hi, 1)) {
                av[i] = *reinterpret_cast<const u32x4_a4*>(w0);
                ae[i] = *reinterpret_cast<const uint32_t*>(w0 + 16);
            } else {
                uint32_t w[5];
#pragma unroll
                for (int q = 0; q < 5; ++q) {
                    w[q] = 0;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uintptr_t o = w0 + 4 * q + e;
                        w[q] |= (o < a_hi ? (uint32_t)*reinterpret_cast<const uint8_t*>(o) : 0u) << (8 * e);
                    }
                }
                av[i] = u32x4{w[0], w[1], w[2], w[3]};
                ae[i] = w[4];
            }
        }
    };
    auto align_a = [&](const u32x4 (&av)[2], const uint32_t (&ae)[2], u32x4 (&aa)[2]) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            if (kAlignedA) {
                aa[i] = av[i];
                continue;
            }
            aa[i] = u32x4{__builtin_amdgcn_alignbyte(av[i][1], av[i][0], sh[i]),
                          __builtin_amdgcn_alignbyte(av[i][2], av[i][1], sh[i]),
                          __builtin_amdgcn_alignbyte(av[i][3], av[i][2], sh[i]),
                          __builtin_amdgcn_alignbyte(ae[i], av[i][3], sh[i])};
        }
    };
    // Code slots of this wave: slot s (16 bytes) of a tile is row s / 11,
    // piece s % 11 (piece 10: the row's padding, filled with piece 0).
    uint32_t boff[kDm], bp16[kDm];
#pragma unroll
    for (int g = 0; g < kDm; ++g) {
        const int slot = kSl * wave + kWave * g + lane;
        const int row = slot / 11, piece = slot % 11;
        const uint32_t rowc = min(n0 + (uint32_t)row, p.n - 1u);
        bp16[g] = piece < 10 ? 16u * piece : 0u;
        boff[g] = rowc * p.k + bp16[g];
    }
    const bool k_tail = p.k % kTmK != 0;
    // Code load g (0 .. kDm - 1) of step kt into buffer buf (the last one
    // only for the lanes whose slot exists).
    auto dma_one = [&](uint32_t kt, uint32_t buf, int g) {
        const int8_t* base = p.q + (uint64_t)kt * kTmK;
        const uint32_t rem = p.k - kt * kTmK;  // >= 16 bytes of this step per row
        uint8_t* dst = wlds + buf * kBB + (size_t)kSl * 16 * wave + kWave * 16 * g;
        uint32_t off = boff[g];
        if (k_tail && bp16[g] >= rem) off -= bp16[g];
        if (kSl % kWave == 0 || g < kDm - 1 || kWave * g + lane < kSl)
            __builtin_amdgcn_global_load_lds((glb_vptr)(base + off), (lds_vptr)dst, 16, 0, 0);
    };
    auto dma_b = [&](uint32_t kt, uint32_t buf) {
#pragma unroll
        for (int g = 0; g < kDm; ++g) dma_one(kt, buf, g);
    };

    i32x16 acc[2][NJ];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[i][j][q] = 0;

    // Trits past k (last step only): zero the decoded bytes at columns >= k.
    auto mask_tail = [&](uint32_t kt, uint32_t (&dec)[2][20]) {
        const int rem = (int)p.k - (int)(kt * kTmK) - 80 * h;  // valid trits of this lane's window
#pragma unroll
        for (int d = 0; d < 20; ++d) {
            const int keep = rem - 4 * d;  // bytes of dword d to keep
            const uint32_t msk = keep >= 4 ? 0xffffffffu : (keep <= 0 ? 0u : (0xffffffffu >> (8 * (4 - keep))));
#pragma unroll
            for (int i = 0; i < 2; ++i) dec[i][d] &= msk;
        }
    };

    // Software pipeline, per K step kt (buffer kt & 1 holds its code tile):
    //   * the code tile of step kt + 1 is loaded into the other buffer (freed
    //     by the barrier that ended step kt - 1) over the first three MFMA
    //     groups, the weights of step kt + 2 into registers before the fourth;
    //   * the weights of step kt + 1 are decoded while the MFMAs of step kt
    //     run; code operands are read one MFMA group ahead;
    //   * a barrier ends the step once this wave's code loads have landed;
    //     the reads of the next step's first operands go out right after it,
    //     covered by the second half of the step's last MFMA group.
    // Steps are unrolled in pairs so that the double-buffered registers swap
    // names instead of being copied.
    auto read_b = [&](uint32_t buf, int s, i32x4 (&bf)[NJ]) {
        const uint8_t* bb = wlds + buf * kBB + r * kWdPitch + 80 * h + 16 * s;
#pragma unroll
        for (int j = 0; j < NJ; ++j) bf[j] = *reinterpret_cast<const i32x4*>(bb + 32 * j * kWdPitch);
    };
    auto decode_all = [&](const u32x4 (&av)[2], uint32_t (&dec)[2][20]) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
            for (int d = 0; d < 20; ++d) dec[i][d] = 0;
#pragma unroll
            for (int b = 0; b < 16; ++b) {
                const uint32_t byte = (av[i][b >> 2] >> (8 * (b & 3))) & 0xffu;
                splice_trits(dec[i], b, lut_lane[byte * kWdCopies]);
            }
        }
    };
    // One MFMA group: operands of group s from bc (read one group earlier),
    // the next group's operands into bn, table reads and splices of the
    // next step's weight bytes [kBy[s], kBy[s + 1]).
    // The code loads of step kt + 1 are spread over groups 0 .. 2 (four,
    // four, three), one after each of the group's first MFMAs: issued as one
    // burst they stall this wave's instruction stream for the time the vector
    // memory unit takes to accept them; issued in group 3 they have not
    // landed by the end of the step.
    // the code loads spread over MFMA groups 0 .. 2 (11 = 4 + 4 + 3; 9 = 3 + 3 + 3)
    constexpr int kDmaAt[5] = {0, (kDm + 2) / 3, 2 * ((kDm + 2) / 3), kDm, kDm};
    auto mgroup = [&](auto S_, uint32_t kt, const uint32_t (&cur)[2][20], uint32_t (&nxt)[2][20],
                      const i32x4 (&bc)[NJ], i32x4 (&bn)[NJ], const u32x4 (&av)[2]) {
        constexpr int s = decltype(S_)::value;
        constexpr int dlo = s < 4 ? kDmaAt[s] : 0, dhi = s < 4 ? kDmaAt[s + 1] : 0;
        const bool dma = kt + 1 < nkt;
        constexpr int kBy[6] = {0, 7, 14, 20, 26, 32};
        constexpr int lo = kBy[s], hi = kBy[s + 1];
        uint64_t tv[hi - lo];
#pragma unroll
        for (int b = lo; b < hi; ++b) {
            const int i = b >> 4, bi = b & 15;
            const uint32_t byte = (av[i][bi >> 2] >> (8 * (bi & 3))) & 0xffu;
            tv[b - lo] = lut_lane[byte * kWdCopies];
        }
        if constexpr (s < 4) read_b(kt & 1u, s + 1, bn);
        __builtin_amdgcn_sched_barrier(0);
        constexpr int ni = s < 4 ? 2 : 1;
#pragma unroll
        for (int i = 0; i < ni; ++i) {
            const i32x4 af = {(int)cur[i][4 * s], (int)cur[i][4 * s + 1], (int)cur[i][4 * s + 2],
                              (int)cur[i][4 * s + 3]};
#pragma unroll
            for (int j = 0; j < NJ; ++j)
                acc[i][j] = mfma_wq<kTrans>(af, bc[j], acc[i][j]);
        }
#pragma unroll
        for (int b = lo; b < hi; ++b) splice_trits(nxt[b >> 4], b & 15, tv[b - lo]);
        if (dma) {
#pragma unroll
            for (int g = dlo; g < dhi; ++g) dma_one(kt + 1, (kt + 1) & 1u, g);
        }
#pragma unroll
        for (int g = 0; g < NJ * ni; ++g) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (g < dhi - dlo) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    using S3 = std::integral_constant<int, 3>;
    using S4 = std::integral_constant<int, 4>;
    auto kstep = [&](uint32_t kt, const uint32_t (&cur)[2][20], uint32_t (&nxt)[2][20], i32x4 (&bx)[NJ],
                     i32x4 (&by)[NJ], const u32x4 (&avr)[2], const uint32_t (&aer)[2], u32x4 (&av2)[2],
                     uint32_t (&ae2)[2]) {
        u32x4 av[2];
        align_a(avr, aer, av);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int d = 0; d < 20; ++d) nxt[i][d] = 0;
        mgroup(S0(), kt, cur, nxt, bx, by, av);
        mgroup(S1(), kt, cur, nxt, by, bx, av);
        mgroup(S2(), kt, cur, nxt, bx, by, av);
        if (kt + 2 < nkt) load_a(kt + 2, av2, ae2);
        mgroup(S3(), kt, cur, nxt, by, bx, av);
        mgroup(S4(), kt, cur, nxt, bx, by, av);
        if (k_tail && kt + 2 == nkt) mask_tail(kt + 1, nxt);
        // This wave's code loads for step kt + 1 have landed and every wave
        // is done reading buffer kt & 1 before anyone passes the barrier.
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        read_b((kt + 1) & 1u, 0, by);
        const i32x4 af = {(int)cur[1][16], (int)cur[1][17], (int)cur[1][18], (int)cur[1][19]};
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[1][j] = mfma_wq<kTrans>(af, bx[j], acc[1][j]);
    };

    u32x4 ava[2], avb[2];
    uint32_t aea[2] = {0u, 0u}, aeb[2] = {0u, 0u};
    load_a(0, ava, aea);
    dma_b(0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // table filled, first code tile staged
    uint32_t cura[2][20], curb[2][20];
    {
        u32x4 a0[2];
        align_a(ava, aea, a0);
        decode_all(a0, cura);
    }
    if (k_tail && nkt == 1) mask_tail(0, cura);
    if (nkt > 1) load_a(1, ava, aea);
    i32x4 bfx[NJ], bfy[NJ];
    read_b(0, 0, bfx);
    uint32_t kt = 0;
    for (; kt + 1 < nkt; kt += 2) {
        kstep(kt, cura, curb, bfx, bfy, ava, aea, avb, aeb);
        kstep(kt + 1, curb, cura, bfy, bfx, avb, aeb, ava, aea);
    }
    if (kt < nkt) kstep(kt, cura, curb, bfx, bfy, ava, aea, avb, aeb);

    // Epilogue: ((float)acc * sa[m]) * sq[n] (+ bias[m]).  Accumulator
    // register q of lane l holds row 8 (q / 4) + 4 (l / 32) + q % 4, column
    // l % 32 of its 32 x 32 tile.  Each wave stages its results in its own
    // LDS region and writes them back as whole output rows, 16 bytes per lane:
    //   * c[m, n]: one 32-row slab (fragment i: 32 m x kN n, row pitch 264
    //     floats: the two row groups of a write land on disjoint banks) at a
    //     time, a 1 KB output row per store instruction;
    //   * c[n, m] (kTrans, the MFMA operands swapped: rows over n, columns
    //     over m): one 32-row slab per column group j (32 n x the wave's 64 m,
    //     row pitch 72 floats), four 256-byte output rows per store
    //     instruction; the slab holds (float)acc * sa[m], and sq[n] is applied
    //     as it is read back.
    constexpr int kEpPitch = 264;
    __syncthreads();  // every wave is done with the code tiles
    if constexpr (kTrans) {
        constexpr int kTp = 72;
        float* slab = reinterpret_cast<float*>(wlds) + wave * 32 * kTp;
        // the tile's sq[n0 .. n0 + kN), read per output row in the store phase
        float* sqs = reinterpret_cast<float*>(wlds) + 4 * 32 * kTp;
        if (t < kN) sqs[t] = p.sq[min(n0 + (uint32_t)t, p.n - 1u)];
        __syncthreads();
        const uint32_t mw = m0 + 64 * wave;  // this wave's 64 rows of m
        float sam[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) sam[i] = p.sa[min(mw + 32 * i + r, p.m - 1u)];
        // store phase: lane l writes m = mw + 4 (l % 16) .. + 3 of row 4 it + l / 16
        const uint32_t mc = mw + 4 * (lane & 15);
        const bool vec_out = (p.m & 3u) == 0 && (reinterpret_cast<uintptr_t>(p.c) & 15u) == 0;
        f32x4 bias4 = {0.f, 0.f, 0.f, 0.f};
        if (p.bias) {
#pragma unroll
            for (int u = 0; u < 4; ++u) bias4[u] = p.bias[min(mc + u, p.m - 1u)];
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int row = 8 * (q >> 2) + 4 * h + (q & 3);
#pragma unroll
                for (int i = 0; i < 2; ++i) slab[row * kTp + 32 * i + r] = (float)acc[i][j][q] * sam[i];
            }
            wave_lds_sync();
#pragma unroll
            for (int it = 0; it < 8; ++it) {
                const int row = 4 * it + (lane >> 4);
                const uint32_t n = n0 + 32 * j + row;
                if (n >= p.n) continue;
                const float sqn = sqs[32 * j + row];
                f32x4 v = *reinterpret_cast<const f32x4*>(slab + row * kTp + 4 * (lane & 15));
                v = v * sqn;
                if (p.bias) v = v + bias4;
                float* crow = p.c + (uint64_t)n * p.m;
                if (vec_out && mc + 3 < p.m) {
                    __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(crow + mc));
                } else {
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        if (mc + u < p.m) crow[mc + u] = v[u];
                }
            }
            wave_lds_sync();  // the slab is rewritten for the next j
        }
        return;
    }
    float sqn[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) sqn[j] = p.sq[min(n0 + 32 * j + r, p.n - 1u)];
    float* slab = reinterpret_cast<float*>(wlds) + wave * 32 * kEpPitch;
    const bool vec_out = (p.n & 3u) == 0 && (reinterpret_cast<uintptr_t>(p.c) & 15u) == 0;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t mb = m0 + 64 * wave + 32 * i;
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const int row = 8 * (q >> 2) + 4 * h + (q & 3);
            const float sam = p.sa[min(mb + row, p.m - 1u)];
#pragma unroll
            for (int j = 0; j < NJ; ++j) slab[row * kEpPitch + 32 * j + r] = ((float)acc[i][j][q] * sam) * sqn[j];
        }
        __syncthreads();
        // kN / 4 lanes cover a row: 256-wide tiles store one row per
        // instruction; 192-wide ones a block of four rows in three
        // instructions (lane L of instruction s takes floats 256 s + 4 L of
        // the block: 48 lanes per row, every lane busy)
        constexpr int kLpr = kN / 4;                  // lanes per row
        constexpr int kRows = kWave % kLpr == 0 ? kWave / kLpr : 4;  // rows per block
        constexpr int kIns = kRows * kLpr / kWave;    // store instructions per block
        for (int rb = 0; rb < 32; rb += kRows) {
#pragma unroll
            for (int s = 0; s < kIns; ++s) {
                const int f = s * kWave + lane;  // 4-float group of the block
                const int row = rb + f / kLpr, col = 4 * (f % kLpr);
                const uint32_t m = mb + row;
                if (m >= p.m) continue;
                f32x4 v = *reinterpret_cast<const f32x4*>(slab + row * kEpPitch + col);
                if (p.bias) v = v + p.bias[m];
                float* crow = p.c + (uint64_t)m * p.n;
                const uint32_t nc = n0 + col;
                if (vec_out && nc + 3 < p.n) {
                    __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(crow + nc));
                } else {
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        if (nc + u < p.n) crow[nc + u] = v[u];
                }
            }
        }
        __syncthreads();
    }
}

// Skinny path (8 < n <= 64, the vector path's alignment): a decode batch
// against a tall weight matrix.  A workgroup owns 32 weight rows and every
// code row (NT tiles of 32); its kWaves waves split K (160-column blocks kb =
// w, w + kWaves, ...), and their exact int32 partials meet in LDS, each wave
// adding one slice of the accumulators over all waves in wave order -- no
// atomics, no zero / finish launches.  A lane decodes its own weight row's
// 16 packed bytes per block straight into MFMA operands: the k order inside a
// block is permuted the same way for both operands (step s, lane half h ->
// columns 80 h + 16 s .. + 16), which leaves each 32-deep MFMA's sum
// unchanged.  The block's codes are read coalesced (10 lanes per 160-byte row
// piece) into the wave's LDS tile, then read back as operands with that
// mapping.  The next block's loads are in flight during the current block's
// MFMAs.
constexpr int kSkRows = 32;
constexpr uint64_t kSkMaxN = 64;
constexpr int kSkPitch = 176;  // LDS bytes per code row of a block (160 + 16)

template <int NT, bool kAlignedA, int kWaves, bool kTrans>
__global__ __launch_bounds__(kWaves * kWave) void ternary_i8_skinny_kernel(TernArgs p) {
    constexpr int kRowsB = 32 * NT;                   // code rows of the workgroup
    constexpr int kPieces = kRowsB * 10 / kWave;     // 16-byte code pieces per lane and block
    constexpr int kTileB = kRowsB * kSkPitch;        // bytes of one wave's code tile
    constexpr int kPart = NT * kWave * 64;           // bytes of one wave's partial sums
    constexpr int kRegion = kTileB > kPart ? kTileB : kPart;
    __shared__ uint64_t lut[256];
    __shared__ __attribute__((aligned(16))) uint8_t smem[kWaves * kRegion];
    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const int wave = t / kWave;
    const int r = lane & 31, h = lane >> 5;
    uint8_t* region = smem + wave * kRegion;
    if (t < 256) lut[t] = trit_lut_entry((uint32_t)t);
    const uint32_t m0 = blockIdx.x * kSkRows;
    const bool row_ok = m0 + r < p.m;
    const uint8_t* arow8 = p.a + (uint64_t)(row_ok ? m0 + r : 0) * p.kp;
    const uintptr_t a_hi = reinterpret_cast<uintptr_t>(p.a) + (uintptr_t)p.m * p.kp;
    const uint32_t nkb = (p.k + kTmK - 1) / kTmK;
    const u32x4 zero_bytes = {kZeroByte * 0x01010101u, kZeroByte * 0x01010101u, kZeroByte * 0x01010101u,
                              kZeroByte * 0x01010101u};
    const u32x4 zero4 = {0u, 0u, 0u, 0u};
    // Unaligned rows: the 20 bytes from the dword boundary below the 16
    // (x and its fifth dword e), shifted into place by the row's byte offset
    // only when the block is decoded -- a shift right after the loads would
    // wait for them (and the code loads behind them) before the MFMAs that
    // are meant to cover them.  Bytes past a row's end meet only zero codes
    // (code pieces at columns >= k are zero); only where the 20 bytes would
    // pass the matrix's end are they read byte by byte.
    const uint32_t sh_a = (uint32_t)(reinterpret_cast<uintptr_t>(arow8) & 3u);
    auto load_a = [&](uint32_t kb, uint32_t& e) -> u32x4 {
        const uint32_t ab = kb * kTmKp + 16u * h;
        if (kAlignedA) return (row_ok && ab < p.kp) ? *reinterpret_cast<const u32x4*>(arow8 + ab) : zero_bytes;
        const uintptr_t w0 = reinterpret_cast<uintptr_t>(arow8 + ab) & ~(uintptr_t)3;
        if (__builtin_expect(w0 + 20u <= a_hi, 1)) {
            e = *reinterpret_cast<const uint32_t*>(w0 + 16);
            return *reinterpret_cast<const u32x4_a4*>(w0);
        }
        uint32_t w[5];
#pragma unroll
        for (int d = 0; d < 5; ++d) {
            w[d] = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uintptr_t o = w0 + 4 * d + j;
                w[d] |= (o < a_hi ? (uint32_t)*reinterpret_cast<const uint8_t*>(o) : 0u) << (8 * j);
            }
        }
        e = w[4];
        return u32x4{w[0], w[1], w[2], w[3]};
    };
    // piece u of this lane: row (u * 64 + lane) / 10, 16-byte piece % 10
    auto load_b = [&](uint32_t kb, u32x4 (&bv)[kPieces]) {
#pragma unroll
        for (int u = 0; u < kPieces; ++u) {
            const uint32_t pc = (uint32_t)(u * kWave + lane);
            const uint32_t n = pc / 10u, c = kb * kTmK + 16u * (pc % 10u);
            const bool ok = n < p.n && c < p.k;
            const u32x4 v = *reinterpret_cast<const u32x4*>(p.q + (ok ? (uint64_t)n * p.k + c : 0u));
            bv[u] = ok ? v : zero4;
        }
    };

    i32x16 acc[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int q = 0; q < 16; ++q) acc[j][q] = 0;
    __syncthreads();  // table filled
    uint32_t kb = (uint32_t)wave;
    u32x4 av = zero_bytes;
    uint32_t ae = 0u;
    u32x4 bv[kPieces];
    if (kb < nkb) {
        av = load_a(kb, ae);
        load_b(kb, bv);
    }
    for (; kb < nkb; kb += kWaves) {
        // this block's codes into the wave's tile (after the last block's reads)
        wave_lds_sync();
#pragma unroll
        for (int u = 0; u < kPieces; ++u) {
            const uint32_t pc = (uint32_t)(u * kWave + lane);
            *reinterpret_cast<u32x4*>(region + (pc / 10u) * kSkPitch + 16u * (pc % 10u)) = bv[u];
        }
        // decode this block's 16 packed bytes into 80 trits (20 dwords)
        uint32_t out[20];
#pragma unroll
        for (int d = 0; d < 20; ++d) out[d] = 0;
        if (!kAlignedA)
            av = u32x4{__builtin_amdgcn_alignbyte(av[1], av[0], sh_a), __builtin_amdgcn_alignbyte(av[2], av[1], sh_a),
                       __builtin_amdgcn_alignbyte(av[3], av[2], sh_a), __builtin_amdgcn_alignbyte(ae, av[3], sh_a)};
        uint64_t lv[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) lv[i] = lut[(av[i >> 2] >> (8 * (i & 3))) & 0xffu];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int off = 5 * i, d = off >> 2, sh = (off & 3) * 8;
            out[d] |= (uint32_t)(lv[i] << sh);
            out[d + 1] |= (uint32_t)(lv[i] >> (32 - sh));
        }
        const uint32_t kn = kb + kWaves;
        if (kn < nkb) {
            av = load_a(kn, ae);
            load_b(kn, bv);
        }
        wave_lds_sync();
#pragma unroll
        for (int s = 0; s < 5; ++s) {
            const i32x4 a = {(int)out[4 * s], (int)out[4 * s + 1], (int)out[4 * s + 2], (int)out[4 * s + 3]};
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                const i32x4 b = *reinterpret_cast<const i32x4*>(region + (32 * j + r) * kSkPitch + 80 * h + 16 * s);
                acc[j] = mfma_wq<kTrans>(a, b, acc[j]);
            }
        }
    }
    // every wave stores its partial sums; wave w then adds accumulator
    // registers [w * kSlice, (w + 1) * kSlice) over all waves, in wave order
    // (exact), and applies the epilogue to them
    __syncthreads();  // all waves are done with their code tiles
    i32x4* mypart = reinterpret_cast<i32x4*>(region);
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4)
            mypart[(j * 4 + q4) * kWave + lane] = i32x4{acc[j][4 * q4], acc[j][4 * q4 + 1], acc[j][4 * q4 + 2],
                                                        acc[j][4 * q4 + 3]};
    __syncthreads();
    constexpr int kQuads = NT * 4;  // 4-register groups per lane
    for (int g = wave; g < kQuads; g += kWaves) {
        i32x4 sum = {0, 0, 0, 0};
#pragma unroll
        for (int w = 0; w < kWaves; ++w) sum += reinterpret_cast<const i32x4*>(smem + w * kRegion)[g * kWave + lane];
        const int j = g / 4, q4 = g % 4;
        if (kTrans) {
            // accumulator rows over n, lanes over m: stores run along c[n, m]'s rows
            const uint32_t m = m0 + (uint32_t)r;
            if (m < p.m) {
                const float sam = p.sa[m];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t n = (uint32_t)j * 32u + 8u * q4 + 4u * h + e;  // register 4 q4 + e
                    if (n < p.n) p.c[out_idx(p, m, n)] = add_bias(p.bias, ((float)sum[e] * sam) * p.sq[n], m);
                }
            }
            continue;
        }
        const uint32_t n = (uint32_t)j * 32u + (uint32_t)r;
        if (n < p.n) {
            const float sqn = p.sq[n];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t m = m0 + 8 * q4 + 4 * h + e;  // register 4 q4 + e
                if (m < p.m) p.c[out_idx(p, m, n)] = add_bias(p.bias, ((float)sum[e] * p.sa[m]) * sqn, m);
            }
        }
    }
}

// Split-K helpers: zero c as int32 (a kernel, not hipMemsetAsync, so the
// call can be captured in a graph), then turn the int32 sums into
// ((float)acc * a_scale) * q_scale in place.
__global__ __launch_bounds__(kTmBlock) void ternary_i8_zero_kernel(int32_t* c, uint64_t total) {
    const uint64_t i = (uint64_t)blockIdx.x * kTmBlock + threadIdx.x;
    if (i < total) c[i] = 0;
}

__global__ __launch_bounds__(kTmBlock) void ternary_i8_finish_kernel(TernArgs p) {
    const uint64_t i = (uint64_t)blockIdx.x * kTmBlock + threadIdx.x;
    if (i >= (uint64_t)p.m * p.n) return;
    const uint32_t m = (uint32_t)(p.trans ? i % p.m : i / p.n), n = (uint32_t)(p.trans ? i / p.m : i % p.n);
    const int32_t acc = reinterpret_cast<const int32_t*>(p.c)[i];
    p.c[i] = add_bias(p.bias, ((float)acc * p.sa[m]) * p.sq[n], m);
}

// Small-n path (n <= 8, k % 8 == 0, 8-byte aligned codes): a group of waves
// owns 4 weight rows and every lane a 40-column window of them (8 packed
// bytes per row), decoded through the LDS table and reused for up to 4 code
// rows at a time: 10 v_dot4_i32_i8 per row and code row, then exact integer
// wave sums (DPP) and the same epilogue.  K is walked in chunks of 2560
// columns (512 packed bytes) shared by the group's waves.  Bound by the
// packed weights' bytes (m * ceil(k/5)) and latency where the MFMA tiles
// would waste most of their columns.
constexpr int kGvRows = 4;     // weight rows per wave group
constexpr int kGvChunk = 2560; // columns per lane-window sweep (64 lanes x 40)
// Largest n the small-n path takes, by measured crossover against the
// split-K MFMA tiles: n = 8 is faster here (6912 x 8 x 2560: 10.4 vs 10.7 us;
// 2560 x 8 x 6912: 13.6 vs 15.9 us), n = 16 is not (6912 x 16 x 2560: 18.5
// vs 10.4 us).  It also spares k % 16 == 8 shapes the one-thread-per-output
// kernel (2560 x 8 x 6920: 12.5 vs 334 us).
constexpr uint64_t kGvMaxN = 8;

__device__ __forceinline__ int32_t wave_sum_i32(int32_t v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
    return __builtin_amdgcn_readlane(v, kWave - 1);
}

// kAligned8: packed rows start 8-byte aligned (a and Kp), so a lane's window
// (8 bytes at a multiple of 8) is one load.
// W: waves per group of kGvRows weight rows.  With K longer than one chunk
// the W waves of a group take chunks ks, ks + W, ... (ks = wave % W) so that
// their loads are in flight together; their exact int32 sums meet in LDS and
// the group's first wave adds them (fixed order) and applies the epilogue.
template <int NT, bool kAligned8, int W>
__global__ __launch_bounds__(kTmBlock) void ternary_i8_gemv_kernel(TernArgs p) {
    constexpr int kWaves = kTmBlock / kWave;
    __shared__ uint64_t lut[256];
    __shared__ int32_t part[kWaves][kGvRows][NT];
    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const int wave = t / kWave;
    const int ks = wave % W;
    lut[t] = trit_lut_entry((uint32_t)t);
    __syncthreads();
    const uint32_t mrow0 = (blockIdx.x * (kWaves / W) + wave / W) * kGvRows;
    const bool live = mrow0 < p.m;  // uniform per wave; every wave reaches the barriers
    // bounds of the packed matrix for the unaligned path's dword reads
    const uintptr_t a_lo = reinterpret_cast<uintptr_t>(p.a);
    const uintptr_t a_hi = a_lo + (uintptr_t)p.m * p.kp;
    // code rows in groups of NT (the last one partial); each group re-walks K
    for (uint32_t n0 = 0; n0 < p.n; n0 += NT) {
    int32_t acc[kGvRows][NT];
#pragma unroll
    for (int r = 0; r < kGvRows; ++r)
#pragma unroll
        for (int n = 0; n < NT; ++n) acc[r][n] = 0;
    for (uint32_t k0 = (uint32_t)ks * kGvChunk; live && k0 < p.k; k0 += (uint32_t)W * kGvChunk) {
        const uint32_t kw = k0 + 40u * lane;  // this lane's first column
        const uint32_t pb = kw / 5u;          // its first packed byte
        // the 8 packed bytes of each row (one 8-byte load when the row and
        // the window allow it; bytes past the row read as five zero trits),
        // all rows in flight before any is decoded
        uint32_t pk[kGvRows][2];
#pragma unroll
        for (int r = 0; r < kGvRows; ++r) {
            const uint32_t m = mrow0 + r;
            const uint8_t* ar = p.a + (uint64_t)(m < p.m ? m : 0) * p.kp;
            const uintptr_t wa = reinterpret_cast<uintptr_t>(ar + pb);  // window address
            const uintptr_t w0 = wa & ~(uintptr_t)3;
            if (kAligned8 && m < p.m && pb + 8u <= p.kp) {
                const uint2 v = *reinterpret_cast<const uint2*>(ar + pb);
                pk[r][0] = v.x;
                pk[r][1] = v.y;
            } else if (!kAligned8 && m < p.m && pb + 8u <= p.kp && w0 >= a_lo && w0 + 12u <= a_hi) {
                // unaligned row: the three dwords around the window, shifted
                const uint3 v = *reinterpret_cast<const uint3*>(w0);
                const uint32_t sh = (uint32_t)(wa & 3u);
                pk[r][0] = __builtin_amdgcn_alignbyte(v.y, v.x, sh);
                pk[r][1] = __builtin_amdgcn_alignbyte(v.z, v.y, sh);
            } else if (m >= p.m || pb >= p.kp) {
                pk[r][0] = pk[r][1] = kZeroByte * 0x01010101u;  // window past the row
            } else {
                // byte by byte; out-of-row bytes load byte 0 of the row (always
                // valid) and are replaced, so every load issues unconditionally
                pk[r][0] = pk[r][1] = 0;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const uint32_t o = pb + i;
                    const bool ok = m < p.m && o < p.kp;
                    const uint32_t b = ar[ok ? o : 0u];
                    pk[r][i >> 2] |= (ok ? b : kZeroByte) << (8 * (i & 3));
                }
            }
        }
        // every code row's 40-column window, also in flight; 8-column pieces
        // past k read the row's first 8 codes instead (in bounds), which meet
        // the zeroed trits below
        uint32_t qw[NT][10];
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            const uint32_t nn = n0 + n < p.n ? n0 + n : 0u;
            const int8_t* qr = p.q + (uint64_t)nn * p.k;
#pragma unroll
            for (int h = 0; h < 5; ++h) {
                const uint32_t c = kw + 8u * h;
                const uint2 v = *reinterpret_cast<const uint2*>(qr + (c < p.k ? c : 0u));
                qw[n][2 * h] = v.x;
                qw[n][2 * h + 1] = v.y;
            }
        }
        // decode -> 40 trits in 10 dwords per row (all table reads issued
        // first), dot with the code windows
        uint64_t lv[kGvRows][8];
#pragma unroll
        for (int r = 0; r < kGvRows; ++r)
#pragma unroll
            for (int i = 0; i < 8; ++i) lv[r][i] = lut[(pk[r][i >> 2] >> (8 * (i & 3))) & 0xffu];
#pragma unroll
        for (int r = 0; r < kGvRows; ++r) {
            uint32_t out[10];
#pragma unroll
            for (int d = 0; d < 10; ++d) out[d] = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint64_t v = lv[r][i];
                const int off = 5 * i, d = off >> 2, sh = (off & 3) * 8;
                out[d] |= (uint32_t)(v << sh);
                if (d + 1 < 10) out[d + 1] |= (uint32_t)(v >> (32 - sh));
            }
            // trits of columns >= k (a last byte's padding) are not in the
            // sum (k % 4 == 0: whole dwords)
#pragma unroll
            for (int d = 0; d < 10; ++d) out[d] = kw + 4u * d < p.k ? out[d] : 0u;
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                int32_t a = acc[r][n];
#pragma unroll
                for (int d = 0; d < 10; ++d) a = __builtin_amdgcn_sdot4((int)out[d], (int)qw[n][d], a, false);
                acc[r][n] = a;
            }
        }
    }
    // exact integer sums over the wave (and the group's W waves), then
    // ((float)acc * sa[m]) * sq[n]
    int32_t tot[kGvRows][NT];
#pragma unroll
    for (int r = 0; r < kGvRows; ++r)
#pragma unroll
        for (int n = 0; n < NT; ++n) tot[r][n] = wave_sum_i32(acc[r][n]);
    if (W > 1) {
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < kGvRows; ++r)
#pragma unroll
                for (int n = 0; n < NT; ++n) part[wave][r][n] = tot[r][n];
        }
        __syncthreads();
        if (ks == 0) {
#pragma unroll
            for (int r = 0; r < kGvRows; ++r)
#pragma unroll
                for (int n = 0; n < NT; ++n) {
                    int32_t v = 0;
#pragma unroll
                    for (int j = 0; j < W; ++j) v += part[wave + j][r][n];
                    tot[r][n] = v;
                }
        }
        __syncthreads();  // part is rewritten by the next code-row group
    }
    if (ks == 0 && live && lane == 0) {
#pragma unroll
        for (int r = 0; r < kGvRows; ++r) {
            const uint32_t m = mrow0 + r;
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                if (n0 + n >= p.n || m >= p.m) continue;
                p.c[out_idx(p, m, n0 + n)] = add_bias(p.bias, ((float)tot[r][n] * p.sa[m]) * p.sq[n0 + n], m);
            }
        }
    }
    }
}

template <int NT, bool kAligned8>
static void launch_gemv(const TernArgs& p, uint64_t m, uint64_t k, hipStream_t s) {
    const uint64_t chunks = (k + kGvChunk - 1) / kGvChunk;
    const int w = chunks >= 3 ? 4 : (chunks == 2 ? 2 : 1);
    const uint64_t rows_per_block = (uint64_t)(kTmBlock / kWave / w) * kGvRows;
    const dim3 g((uint32_t)((m + rows_per_block - 1) / rows_per_block)), b(kTmBlock);
    if (w == 4) hipLaunchKernelGGL((ternary_i8_gemv_kernel<NT, kAligned8, 4>), g, b, 0, s, p);
    else if (w == 2) hipLaunchKernelGGL((ternary_i8_gemv_kernel<NT, kAligned8, 2>), g, b, 0, s, p);
    else hipLaunchKernelGGL((ternary_i8_gemv_kernel<NT, kAligned8, 1>), g, b, 0, s, p);
}

// Generic path: one thread per output, integer accumulation in k order.
__global__ __launch_bounds__(kTmBlock) void ternary_i8_generic_kernel(TernArgs p) {
    __shared__ uint64_t lut[256];
    lut[threadIdx.x] = trit_lut_entry(threadIdx.x);
    __syncthreads();
    const uint64_t idx = (uint64_t)blockIdx.x * kTmBlock + threadIdx.x;
    if (idx >= (uint64_t)p.m * p.n) return;
    const uint32_t m = (uint32_t)(p.trans ? idx % p.m : idx / p.n), n = (uint32_t)(p.trans ? idx / p.m : idx % p.n);
    const uint8_t* ar = p.a + (uint64_t)m * p.kp;
    const int8_t* qr = p.q + (uint64_t)n * p.k;
    int32_t acc = 0;
    for (uint32_t k = 0; k < p.k; ++k) {
        const uint64_t v = lut[ar[k / 5]];
        const int8_t tr = (int8_t)(uint8_t)(v >> (8 * (k % 5)));
        acc += (int32_t)tr * (int32_t)qr[k];
    }
    p.c[idx] = add_bias(p.bias, ((float)acc * p.sa[m]) * p.sq[n], m);
}

// ---------------------------------------------------------------------------
// f32 activations (the reference's ternary_matmul, cpu_ternary_matmul.rs:29-124,
// which BitLinear::forward calls): c[m, col] = (sum over ki in order of
// t[m, ki] * b[ki, col]) * a_scales[m] with b[K, N] f32 and the sum a
// sequential f32 fold that skips zero trits (compute_row :105-124).  Every
// lane owns one output and folds its K terms in the reference's order, so the
// result is bit-exact: acc = fma(t, b, acc) is fl(acc + t*b) (t*b = +-b is
// exact), and a zero trit adds +-0, which leaves acc unchanged (acc is never
// -0: it starts at +0 and an exact-zero sum rounds to +0) -- except when b is
// Inf or NaN (0 * Inf = NaN), so chunks holding such a b skip zero trits
// explicitly.  Bound by the K chain: per term one fma, and per 5 terms two
// LDS reads of b and two of the trit table; with one column (decode) the
// table reads of 64 different rows' bytes dominate.
//
// Block: 4 waves; a wave's 64 lanes are CT columns x 64/CT row slots, each
// lane R rows of its column.  Per chunk of KC columns of K (640, 320 or 160
// as CT is 1, 2 or wider) the block stages b[kc.., col0..col0+CT) in LDS,
// per column as groups of 8 floats (the 5 terms of one packed byte), and
// every lane loads its rows' packed bytes of the chunk.

struct TernF32Args {
    const uint8_t* a;   // packed [M, Kp]
    const float* sa;    // [M]
    const float* b;     // element (k, col) at b[k * bk + col * bn]: [K, N] (bk = N, bn = 1) or token-major [N, K]
    float* c;           // [M, N], or [N, M] with trans
    uint32_t m, n, k, kp;
    uint64_t bk, bn;
    const float* bias;  // [M] added to every output of row m, or null
    uint32_t trans;     // 1: output (m, col) at c[col * ldt + m]
    uint64_t ldt;       // row stride of the transposed output (the full M)
};

__device__ __forceinline__ uint64_t out_idx(const TernF32Args& p, uint32_t m, uint32_t n) {
    return p.trans ? (uint64_t)n * p.ldt + m : (uint64_t)m * p.n + n;
}

template <int CT, int R, int kW, bool kAligned16>
__global__ __launch_bounds__(kW * kWave) void ternary_f32_seq_kernel(TernF32Args p) {
    constexpr int kThreads = kW * kWave;
    constexpr int kSlots = kW * (kWave / CT);  // row slots per block
    constexpr int RB = kSlots * R;             // rows per block
    constexpr int kSub = 8 / R;  // packed bytes whose operands are read ahead of their fmas
    // K columns per chunk: longer for narrow column tiles (few b values per
    // chunk), so that a chunk's folds outlast the next chunk's loads
    constexpr int KC = CT == 1 ? 640 : (CT == 2 ? 320 : 160);
    constexpr int NB = KC / 5;  // packed bytes per chunk
    __shared__ __attribute__((aligned(16))) float flut[256 * 8];  // byte -> 5 trits as floats
    __shared__ __attribute__((aligned(16))) float lut9[9 * 2];      // b % 9  -> trits 0, 1
    __shared__ __attribute__((aligned(16))) float lut27[27 * 4];    // b / 9 -> trits 2, 3, 4
    // b of the chunk, per column c: 32 groups of 8 floats (the 5 columns of K
    // one packed byte covers, padded), so a lane reads its 5 terms as one
    // 16-byte and one 4-byte read; odd pitch in 16-byte units
    constexpr int kPitch = NB * 8 + 4;
    __shared__ __attribute__((aligned(16))) float bs[CT * kPitch];
    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const int wave = t / kWave;
    {
        uint32_t v = (uint32_t)t;
        const bool pad = v >= 243u;
#pragma unroll
        for (int j = 0; j < 5; ++j) {
            flut[t * 8 + j] = pad ? 0.0f : (float)((int)(v % 3u) - 1);
            v /= 3u;
        }
        if (t < 9) {
            lut9[2 * t] = (float)((int)(t % 3) - 1);
            lut9[2 * t + 1] = (float)((int)(t / 3) - 1);
        }
        if (t < 27) {
            lut27[4 * t] = (float)((int)(t % 3) - 1);
            lut27[4 * t + 1] = (float)((int)(t / 3 % 3) - 1);
            lut27[4 * t + 2] = (float)((int)(t / 9) - 1);
            lut27[4 * t + 3] = 0.0f;
        }
    }
    const uint32_t col0 = blockIdx.y * CT;
    const int cl = lane % CT;
    const uint32_t col = col0 + cl;
    const uint32_t slot = (uint32_t)(wave * (kWave / CT) + lane / CT);
    // this lane's R rows (independent folds, interleaved so that each hides
    // the others' latency)
    uint32_t rows[R];
    const uint8_t* arow[R];
    bool live[R];
    bool any_live = false;
#pragma unroll
    for (int i = 0; i < R; ++i) {
        rows[i] = blockIdx.x * RB + slot + (uint32_t)i * kSlots;
        live[i] = rows[i] < p.m && col < p.n;
        any_live |= live[i];
        arow[i] = p.a + (uint64_t)(rows[i] < p.m ? rows[i] : 0) * p.kp;
    }
    const uintptr_t a_hi = reinterpret_cast<uintptr_t>(p.a) + (uintptr_t)p.m * p.kp;
    // b is loaded one chunk ahead into registers, then staged in LDS for the
    // chunk's folds; the rows' packed bytes are loaded at the chunk's start
    // (small, their latency overlaps the barrier and the staging).  Every load
    // is unconditional, at a clamped in-bounds index, so none waits for
    // another.
    constexpr int kStage = (KC * CT + kThreads - 1) / kThreads;  // b elements per thread
    uint32_t pbn[R][NB / 4];  // packed bytes, 4 per register
    float bvn[kStage];
    auto load_pb = [&](uint32_t kc) {
        const uint32_t pb0 = kc / 5u;
        // each row's NB packed bytes of the chunk: 16-byte loads (aligned
        // rows), NB/4 + 1 dwords shifted into place (unaligned rows), or
        // bytes (the row's end)
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const uintptr_t wa = reinterpret_cast<uintptr_t>(arow[i] + pb0);
            const uintptr_t w0 = wa & ~(uintptr_t)3;
            if (kAligned16 && pb0 + NB <= p.kp) {
#pragma unroll
                for (int q = 0; q < NB / 16; ++q) {
                    const u32x4 x = *reinterpret_cast<const u32x4*>(arow[i] + pb0 + 16 * q);
                    pbn[i][4 * q] = x[0]; pbn[i][4 * q + 1] = x[1]; pbn[i][4 * q + 2] = x[2]; pbn[i][4 * q + 3] = x[3];
                }
            } else if (!kAligned16 && pb0 + NB <= p.kp && w0 + NB + 4u <= a_hi) {
                uint32_t d[NB / 4 + 1];
#pragma unroll
                for (int q = 0; q <= NB / 4; ++q) d[q] = reinterpret_cast<const uint32_t*>(w0)[q];
                const uint32_t sh = (uint32_t)(wa & 3u);
#pragma unroll
                for (int q = 0; q < NB / 4; ++q) pbn[i][q] = __builtin_amdgcn_alignbyte(d[q + 1], d[q], sh);
            } else {
#pragma unroll
                for (int q = 0; q < NB / 4; ++q) pbn[i][q] = 0;
#pragma unroll
                for (int j = 0; j < NB; ++j) {
                    const uint32_t o = pb0 + j;
                    pbn[i][j >> 2] |= (uint32_t)arow[i][o < p.kp ? o : 0u] << (8 * (j & 3));
                }
            }
        }
    };
    auto load_b = [&](uint32_t kc) {
        const uint32_t kn = min((uint32_t)KC, p.k - kc);
#pragma unroll
        for (int u = 0; u < kStage; ++u) {
            const uint32_t e = (uint32_t)t + kThreads * u;
            const uint32_t ki = e / CT, c = e % CT;
            const bool ok = e < kn * CT && col0 + c < p.n;
            const float v = p.b[ok ? (uint64_t)(kc + ki) * p.bk + (uint64_t)(col0 + c) * p.bn : 0u];
            bvn[u] = ok ? v : 0.0f;
        }
    };
    float acc[R];
#pragma unroll
    for (int i = 0; i < R; ++i) acc[i] = 0.0f;
    if (p.k > 0) load_b(0);
    for (uint32_t kc = 0; kc < p.k; kc += KC) {
        const uint32_t kn = min((uint32_t)KC, p.k - kc);
        load_pb(kc);  // small; its latency overlaps the barrier and the staging
        __syncthreads();  // the previous chunk's b reads are done (and the table is filled)
        bool bad = false;
#pragma unroll
        for (int u = 0; u < kStage; ++u) {
            const uint32_t e = (uint32_t)t + kThreads * u;
            const uint32_t ki = e / CT, c = e % CT;
            if (e < (uint32_t)(KC * CT)) bs[c * kPitch + (ki / 5u) * 8u + ki % 5u] = bvn[u];
            bad |= !__builtin_isfinite(bvn[u]);
        }
        const uint32_t pb0 = kc / 5u;
        const bool skip_zero = __syncthreads_or(bad);
        if (kc + KC < p.k) load_b(kc + KC);
        auto& pb = pbn;
        if (!any_live) continue;
        const float* bc = bs + cl * kPitch;
        if (CT == 1 && kn == (uint32_t)KC && !skip_zero) {
            // One column: the 64 lanes hold 64 different rows, whose reads of
            // the 256-entry table would conflict.  A byte b < 243 is instead
            // split as b = 9 h + l: trits 0-1 from a 9-entry table indexed by
            // l, trits 2-4 from a 27-entry one indexed by h (both small enough
            // that the reads are broadcasts or distinct banks); bytes >= 243
            // decode as 121 (five zero trits).  b is read uniformly from LDS.
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const f32x4 b4 = *reinterpret_cast<const f32x4*>(bc + 8 * j);
                const float b5 = bc[8 * j + 4];
#pragma unroll
                for (int i = 0; i < R; ++i) {
                    uint32_t byte = (pb[i][j >> 2] >> (8 * (j & 3))) & 0xffu;
                    byte = byte >= 243u ? 121u : byte;
                    const uint32_t h = (byte * 57u) >> 9;  // byte / 9 for byte < 256
                    const uint32_t l = byte - 9u * h;
                    const float2 tl = *reinterpret_cast<const float2*>(lut9 + 2 * l);
                    const f32x4 th = *reinterpret_cast<const f32x4*>(lut27 + 4 * h);
                    acc[i] = __builtin_fmaf(tl.x, b4.x, acc[i]);
                    acc[i] = __builtin_fmaf(tl.y, b4.y, acc[i]);
                    acc[i] = __builtin_fmaf(th.x, b4.z, acc[i]);
                    acc[i] = __builtin_fmaf(th.y, b4.w, acc[i]);
                    acc[i] = __builtin_fmaf(th.z, b5, acc[i]);
                }
            }
        } else if (kn == (uint32_t)KC && !skip_zero) {
#pragma unroll
            for (int j0 = 0; j0 < NB; j0 += kSub) {
                f32x4 b4[kSub], t4[R][kSub];
                float b5[kSub], t5[R][kSub];
#pragma unroll
                for (int jj = 0; jj < kSub; ++jj) {
                    const int j = j0 + jj;
                    b4[jj] = *reinterpret_cast<const f32x4*>(bc + 8 * j);
                    b5[jj] = bc[8 * j + 4];
#pragma unroll
                    for (int i = 0; i < R; ++i) {
                        const uint32_t byte = (pb[i][j >> 2] >> (8 * (j & 3))) & 0xffu;
                        t4[i][jj] = *reinterpret_cast<const f32x4*>(flut + byte * 8);
                        t5[i][jj] = flut[byte * 8 + 4];
                    }
                }
#pragma unroll
                for (int jj = 0; jj < kSub; ++jj)
#pragma unroll
                    for (int i = 0; i < R; ++i) {
                        acc[i] = __builtin_fmaf(t4[i][jj].x, b4[jj].x, acc[i]);
                        acc[i] = __builtin_fmaf(t4[i][jj].y, b4[jj].y, acc[i]);
                        acc[i] = __builtin_fmaf(t4[i][jj].z, b4[jj].z, acc[i]);
                        acc[i] = __builtin_fmaf(t4[i][jj].w, b4[jj].w, acc[i]);
                        acc[i] = __builtin_fmaf(t5[i][jj], b5[jj], acc[i]);
                    }
            }
        } else {
            // last partial chunk, or Inf/NaN in b: bounds and zero trits checked
#pragma unroll
            for (int i = 0; i < R; ++i) {
                for (uint32_t ki = 0; ki < kn; ++ki) {
                    const uint32_t o = pb0 + ki / 5u;
                    const float tr = flut[(uint32_t)arow[i][o < p.kp ? o : 0u] * 8 + ki % 5u];
                    if (tr != 0.0f) acc[i] = __builtin_fmaf(tr, bc[(ki / 5u) * 8u + ki % 5u], acc[i]);
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < R; ++i)
        if (live[i]) p.c[out_idx(p, rows[i], col)] = add_bias(p.bias, acc[i] * p.sa[rows[i]], rows[i]);
}

// One to four columns (K = 0 or fewer than 20 packed bytes): one fold per
// lane, 4 waves.
template <bool kAligned16>
static void launch_f32_seq(int ct, dim3 g, hipStream_t s, const TernF32Args& p) {
#define KORE_F32_SEQ(C) \
    hipLaunchKernelGGL((ternary_f32_seq_kernel<C, 1, 4, kAligned16>), g, dim3(4 * kWave), 0, s, p)
    if (ct == 1) KORE_F32_SEQ(1);
    else if (ct == 2) KORE_F32_SEQ(2);
    else KORE_F32_SEQ(4);
#undef KORE_F32_SEQ
}

// 16 bytes per lane from a range-checked resource straight into LDS (lane
// L's at dst + 16 L; dst wave-uniform).
__device__ __forceinline__ void lds_load16(__amdgpu_buffer_rsrc_t r, lds_vptr dst, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, voff, soff, 0, 0);
}

constexpr uint32_t kRowsW = 4;            // waves per workgroup (b[K, N])
// Token-major b (the layer's input as stored): a staged chunk is a 320-byte
// piece of every column, which straddles cache lines, so every workgroup's
// share of L2 reads grows; eight waves share each staged chunk instead of
// four (measured at 6912 x 64 x 2560: 82.3 -> 71.1 us; 16 columns 25.6 ->
// 23.1 us).
constexpr uint32_t kRowsWTm = 8;
constexpr int kBufWord3 = 0x00020000;     // buffer resource word 3 (raw dword access)
constexpr uint64_t kRowsMinWaves = 1536;  // 1.5 per SIMD of 256 CUs
constexpr uint64_t kSimds = 1024;         // 256 CUs x 4
// From five columns the row-broadcast kernel; narrower, the fold-wave kernel
// (measured: 6912 x 4 x 2560 21.1 against 24.8 us, 6912 x 5 26.4 against 32.3).
constexpr uint64_t kRowsMinCols = 5;
// Five columns and more, any alignment: a wave is 64 / CT row slots of CT
// columns (CT = 16, 32 or 64, one column per lane), and slot s owns R rows,
// so a row's trit at each K is the same for all CT lanes of its slot.  The
// per-lane kernel above reads each such trit from LDS as a broadcast
// returned to all 64 lanes, which leaves it LDS-bound (about 2.5 LDS cycles
// per fma cycle).  Here lane L decodes byte L % 16 of the chunk's 16 packed
// bytes of each of its slot's rows (so every 16-lane row of the wave holds
// the 80 trits of the chunk of its slot's rows, 5 per lane, from a table in
// LDS), and each fma takes its trit from lane j of its own 16-lane row
// through the DPP operand modifier row_newbcast:j: the vector unit issues one
// fma per term, and LDS serves b and 5 table reads per row and chunk.  A slot
// is at least one 16-lane row, so 5-15 columns leave lanes idle.
//
// Terms and zero trits as in the per-lane kernel: fma(t, b, acc) is the
// reference's step for finite b; a chunk whose b holds an Inf or NaN (and
// the last partial chunk) skips zero trits explicitly.
template <int J>
__device__ __forceinline__ float fmac_trit(float acc, float t, float b) {
    // acc = fma(t from lane J of this lane's 16-lane row, b, acc)
    asm("v_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf" : "+v"(acc) : "v"(t), "v"(b), "i"(J));
    return acc;
}

template <int CT, int R, int W, bool TM>
__global__ __launch_bounds__(W * kWave) void ternary_f32_rows_kernel(TernF32Args p) {
    constexpr int KC = 80;                 // K columns per chunk
    constexpr int NB = KC / 5;             // packed bytes per row and chunk (one per lane of a 16-lane row)
    constexpr int kPitch = KC + 4;         // floats per column of the staged b: 21 x 16 bytes
    constexpr int kSlots = kWave / CT;     // row slots of a wave (CT lanes each)
    constexpr int kThreads = W * kWave;
    constexpr int kGroups = KC / 4 * CT;   // 4-float groups of b per chunk
    constexpr int kStage = (kGroups + kThreads - 1) / kThreads;
    static_assert(NB == 16 && CT % 16 == 0 && kWave % CT == 0, "chunk split");
    static_assert(kGroups % kWave == 0, "staging is wave-uniform");
    __shared__ __attribute__((aligned(16))) float bs[2][CT * kPitch];  // b of a chunk, [column][k]
    __shared__ float tlut[5 * 256];  // digit d of byte v -> trit as float at [d * 256 + v]; v >= 243: 0
    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane(t / kWave);
    for (int v = t; v < 256; v += kThreads) {
        uint32_t x = (uint32_t)v;
#pragma unroll
        for (int d = 0; d < 5; ++d) {
            tlut[d * 256 + v] = v >= 243 ? 0.0f : (float)((int)(x % 3u) - 1);
            x /= 3u;
        }
    }
    __syncthreads();  // the table is read before the first chunk's barrier
    const uint32_t col0 = blockIdx.y * CT;
    const uint32_t col = col0 + (uint32_t)(lane % CT);
    // row slot lane / CT of the wave owns rows row0 .. row0 + R - 1
    const uint32_t row0 = ((blockIdx.x * W + wave) * kSlots + (uint32_t)(lane / CT)) * R;
    // b staging: group g of a chunk is k = 4 (g / CT) .. + 3 of column g % CT,
    // one 16-byte LDS write at [column][k].  Buffer loads from a resource
    // based at the chunk's first k of the tile's first column, with byte
    // offsets fixed for the whole kernel; an offset past any range returns
    // zeros for columns past N.  b[K, N] (TM false): four coalesced loads (a
    // row of CT columns each), and the hardware range check returns zeros
    // past K.  Token-major b[N, K] (TM true: the layer's input x as it is
    // stored): the four k of a group are consecutive in one column, and the
    // last chunk zeroes k >= K itself (those offsets lie in the next column).
    // Token-major groups run along k (cl = g / 20, k4 = 4 (g % 20)), so that
    // consecutive lanes read consecutive bytes of one column.
    uint32_t boff[kStage][4];
    uint32_t bk4[kStage];
    auto g_col = [](uint32_t g) { return TM ? g / (KC / 4) : g % CT; };
    auto g_k4 = [](uint32_t g) { return TM ? 4u * (g % (KC / 4)) : 4u * (g / CT); };
#pragma unroll
    for (int u = 0; u < kStage; ++u) {
        const uint32_t g = (uint32_t)t + kThreads * u;
        const uint32_t cl = g_col(g), k4 = g_k4(g);
        bk4[u] = k4;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            boff[u][q] = col0 + cl < p.n ? (TM ? (cl * p.k + k4 + q) * 4u : ((k4 + q) * p.n + cl) * 4u) : 0x80000000u;
    }
    auto load_b = [&](uint32_t kc, f32x4 (&bv)[kStage]) {
        const uint64_t left = TM ? ((uint64_t)(p.n - col0) * p.k - kc) * 4u : ((uint64_t)(p.k - kc) * p.n - col0) * 4u;
        const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(p.b + (uint64_t)kc * p.bk + (uint64_t)col0 * p.bn), (short)0,
            (int)(left < 0x7fffffffull ? left : 0x7fffffffull), kBufWord3);
        const uint32_t kleft = p.k - kc;
#pragma unroll
        for (int u = 0; u < kStage; ++u) {
            if (kGroups % kThreads != 0 && u == kStage - 1 && t >= kGroups % kThreads) break;
            float v[4];
            if (TM) {
                // the group's four k are consecutive in its column: one
                // 16-byte load (global loads need dword alignment only) in a
                // whole chunk, single elements checked against K in the last
                const float* src = p.b + (boff[u][0] == 0x80000000u ? 0u : (uint64_t)boff[u][0] / 4u + kc +
                                                                              (uint64_t)col0 * p.k);
                if (kleft >= (uint32_t)KC) {
                    const u32x4 wu = boff[u][0] == 0x80000000u ? u32x4{0u, 0u, 0u, 0u}
                                                               : (u32x4)*reinterpret_cast<const u32x4_a4*>(src);
                    const f32x4 w = __builtin_bit_cast(f32x4, wu);
                    v[0] = w[0]; v[1] = w[1]; v[2] = w[2]; v[3] = w[3];
                } else {
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        v[q] = (boff[u][0] != 0x80000000u && bk4[u] + q < kleft) ? src[q] : 0.0f;
                }
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    v[q] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rb, boff[u][q], 0, 0));
            }
            bv[u] = f32x4{v[0], v[1], v[2], v[3]};
        }
    };
    // byte lane % 16 of the chunk for each row.  Past the row's end the byte
    // is the next row's (or 0 past the matrix, by the range check): its
    // trits meet only b past K, which is zero, and fma(t, 0, acc) = acc.
    const int a_bytes = (int)((uint64_t)p.m * p.kp);  // below 2^31 (checked by the launcher)
    uint32_t aoff[R];
#pragma unroll
    for (int i = 0; i < R; ++i) aoff[i] = min(row0 + i, p.m - 1) * p.kp + (uint32_t)(lane & (NB - 1));
    auto load_pb = [&](uint32_t kc, uint32_t (&pb)[R]) {
        const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void*)p.a, (short)0, a_bytes, kBufWord3);
#pragma unroll
        for (int i = 0; i < R; ++i) pb[i] = __builtin_amdgcn_raw_buffer_load_b8(ra, aoff[i] + kc / 5u, 0, 0);
    };
    f32x4 bvn[kStage];
    uint32_t pbn[R];
    float acc[R];
#pragma unroll
    for (int i = 0; i < R; ++i) acc[i] = 0.0f;
    if (p.k > 0) {
        load_b(0, bvn);
        load_pb(0, pbn);
    }
    bool slow = false;  // wave-uniform: a row's sum is Inf or NaN
    uint32_t buf = 0;
    for (uint32_t kc = 0; kc < p.k; kc += KC, buf ^= 1u) {
        float* bb = bs[buf];
#pragma unroll
        for (int u = 0; u < kStage; ++u) {
            if (kGroups % kThreads != 0 && u == kStage - 1 && t >= kGroups % kThreads) break;
            const uint32_t g = (uint32_t)t + kThreads * u;
            *reinterpret_cast<f32x4*>(bb + g_col(g) * kPitch + g_k4(g)) = bvn[u];
        }
        // this chunk's trits: lane L holds the five of byte L % 16 of each row
        uint32_t pbc[R];
        float tr[R][5];
#pragma unroll
        for (int i = 0; i < R; ++i) {
            pbc[i] = pbn[i];
#pragma unroll
            for (int d = 0; d < 5; ++d) tr[i][d] = tlut[d * 256 + pbn[i]];
        }
        if (kc + KC < p.k) {
            load_b(kc + KC, bvn);
            load_pb(kc + KC, pbn);
        }
        // one barrier per chunk: this chunk's b written before it is read,
        // and the previous chunk's reads of the other buffer done before the
        // next chunk overwrites it
        __syncthreads();
        const f32x4* bc = reinterpret_cast<const f32x4*>(bb + (lane % CT) * kPitch);
        if (!slow) {
            // K advances 20 columns (4 bytes, 5 float4 of b) per group; the
            // next group's b is read before this group's fmas
            float saved[R];
#pragma unroll
            for (int i = 0; i < R; ++i) saved[i] = acc[i];
            f32x4 bcur[5], bnxt[5];
#pragma unroll
            for (int q = 0; q < 5; ++q) bcur[q] = bc[q];
            auto group = [&](auto gc) {
                constexpr int G = decltype(gc)::value;
                if (G < 3) {
#pragma unroll
                    for (int q = 0; q < 5; ++q) bnxt[q] = bc[5 * (G + 1) + q];
                }
                __builtin_amdgcn_sched_barrier(0);
                const float* bf = reinterpret_cast<const float*>(bcur);
                auto byte = [&](auto jc) {
                    constexpr int j = decltype(jc)::value;  // byte of the group
#pragma unroll
                    for (int d = 0; d < 5; ++d)
#pragma unroll
                        for (int i = 0; i < R; ++i) acc[i] = fmac_trit<4 * G + j>(acc[i], tr[i][d], bf[5 * j + d]);
                };
                byte(std::integral_constant<int, 0>{});
                byte(std::integral_constant<int, 1>{});
                byte(std::integral_constant<int, 2>{});
                byte(std::integral_constant<int, 3>{});
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int q = 0; q < 5; ++q) bcur[q] = bnxt[q];
            };
            group(std::integral_constant<int, 0>{});
            group(std::integral_constant<int, 1>{});
            group(std::integral_constant<int, 2>{});
            group(std::integral_constant<int, 3>{});
            // An Inf or NaN b turns the sum it enters Inf or NaN (fma(0, Inf,
            // acc) included), and so does an overflow: redo the chunk with
            // zero trits skipped from the saved sums, and keep doing so.
            bool nf = false;
#pragma unroll
            for (int i = 0; i < R; ++i) nf |= !__builtin_isfinite(acc[i]);
            if (__builtin_expect(__ballot(nf) != 0, 0)) {
                slow = true;
#pragma unroll
                for (int i = 0; i < R; ++i) acc[i] = saved[i];
            }
        }
        if (slow) {
            const uint32_t kn = min((uint32_t)KC, p.k - kc);
            const float* bf = bb + (lane % CT) * kPitch;
            for (uint32_t ki = 0; ki < kn; ++ki) {
                const float bv = bf[ki];
#pragma unroll
                for (int i = 0; i < R; ++i) {
                    // byte ki / 5 of the row, held by lane ki / 5 of this lane's 16-lane row
                    const uint32_t byte = (uint32_t)__shfl((int)pbc[i], (lane & ~15) + (int)(ki / 5u), kWave);
                    const float trv = tlut[(ki % 5u) * 256u + byte];
                    if (trv != 0.0f) acc[i] = __builtin_fmaf(trv, bv, acc[i]);
                }
            }
        }
    }
    if (col < p.n) {
        // c[n, m] with four rows per lane: the lane's rows are four
        // consecutive floats of one output row, stored as one 16-byte write
        if (R == 4 && p.trans && row0 + 3 < p.m && (p.ldt & 3u) == 0 &&
            (reinterpret_cast<uintptr_t>(p.c) & 15u) == 0) {
            f32x4 v;
#pragma unroll
            for (int i = 0; i < R && i < 4; ++i) v[i] = add_bias(p.bias, acc[i] * p.sa[row0 + i], row0 + i);
            *reinterpret_cast<f32x4*>(p.c + out_idx(p, row0, col)) = v;
            return;
        }
#pragma unroll
        for (int i = 0; i < R; ++i)
            if (row0 + i < p.m) p.c[out_idx(p, row0 + i, col)] = add_bias(p.bias, acc[i] * p.sa[row0 + i], row0 + i);
    }
}

// The row-broadcast kernel with token-major b loaded straight into LDS
// (three tiles, chunk c + 2's loads issued in chunk c); the rest as in
// ternary_f32_rows_kernel above.
template <int CT, int R, int W>
__global__ __launch_bounds__(W * kWave) void ternary_f32_rows_dma_kernel(TernF32Args p) {
    constexpr bool DMA = true;
    constexpr int KC = 80;                 // K columns per chunk
    constexpr int NB = KC / 5;             // packed bytes per row and chunk (one per lane of a 16-lane row)
    constexpr int kPitch = KC + 4;         // floats per column of the staged b: 21 x 16 bytes
    constexpr int kSlots = kWave / CT;     // row slots of a wave (CT lanes each)
    constexpr int kThreads = W * kWave;
    static_assert(NB == 16 && CT % 16 == 0 && kWave % CT == 0, "chunk split");
    // DMA: token-major b (the layer's input) goes straight into LDS: three
    // tiles, each a whole number of 1 KB loads (64 lanes x 16 bytes); see
    // below.
    constexpr int kDmaRows = (CT * kPitch / 4 + kWave - 1) / kWave;  // 1 KB loads per chunk
    constexpr int kTileF = DMA ? kDmaRows * kWave * 4 : CT * kPitch;  // floats per tile
    // b of a chunk, [column][k]: separate arrays, so that with the loop
    // unrolled over them the compiler sees which one a read and a load into
    // LDS touch (a read waits only for loads into its own tile)
    __shared__ __attribute__((aligned(16))) float bs0[kTileF];
    __shared__ __attribute__((aligned(16))) float bs1[kTileF];
    __shared__ __attribute__((aligned(16))) float bs2[kTileF];
    __shared__ float tlut[5 * 256];  // digit d of byte v -> trit as float at [d * 256 + v]; v >= 243: 0
    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane(t / kWave);
    for (int v = t; v < 256; v += kThreads) {
        uint32_t x = (uint32_t)v;
#pragma unroll
        for (int d = 0; d < 5; ++d) {
            tlut[d * 256 + v] = v >= 243 ? 0.0f : (float)((int)(x % 3u) - 1);
            x /= 3u;
        }
    }
    __syncthreads();  // the table is read before the first chunk's barrier
    const uint32_t col0 = blockIdx.y * CT;
    const uint32_t col = col0 + (uint32_t)(lane % CT);
    // row slot lane / CT of the wave owns rows row0 .. row0 + R - 1
    const uint32_t row0 = ((blockIdx.x * W + wave) * kSlots + (uint32_t)(lane / CT)) * R;
    // DMA staging (token-major b): slot s of a tile (16 bytes) holds column
    // s / 21, K columns 4 (s % 21) .. + 3 of the chunk ([column][84 floats],
    // the layout above; entry 20 of a column, its padding, reloads entry
    // 19, and slots past the tile's columns read zeros).  Wave w issues the
    // loads of rows w, w + W, ... of the tile through a resource based at the
    // tile's first column, at 32-bit offsets fixed for the kernel plus a
    // per-chunk scalar offset (the launcher takes this path where the tile's
    // 64 columns hold below 2^31 bytes).  Past K a column reads the next one's values: the partial
    // last chunk's trits past K are masked to zero instead.  Chunk c + 2's
    // loads are issued in chunk c (into the tile chunk c - 1 used; issued
    // past K too, into a tile no chunk reads) and waited for, with an
    // explicit vmcnt, before the barrier that ends chunk c + 1.
    // Every wave issues kDmaMax loads per chunk (a wave short of rows
    // reloads another wave's row: the same bytes to the same place), so that
    // the compiler's count of the loads in flight is the same on every path.
    constexpr int kDmaMax = (kDmaRows + W - 1) / W;
    auto dma_row = [&](int u) { return (uint32_t)(((int)wave + W * u) % kDmaRows); };
    uint32_t doff[kDmaMax];
    const uint32_t tile_cols = p.n - col0 < (uint32_t)CT ? p.n - col0 : (uint32_t)CT;
    const __amdgpu_buffer_rsrc_t rbd = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.b + (DMA ? (uint64_t)col0 * p.k : 0u)), (short)0, DMA ? (int)(tile_cols * p.k * 4u) : 0, kBufWord3);
    if constexpr (DMA) {
#pragma unroll
        for (int u = 0; u < kDmaMax; ++u) {
            const uint32_t sl = (uint32_t)kWave * dma_row(u) + (uint32_t)lane;
            const uint32_t cl = sl / (uint32_t)(kPitch / 4), j = sl % (uint32_t)(kPitch / 4);
            doff[u] = cl < tile_cols ? (cl * p.k + 4u * (j < 20u ? j : 19u)) * 4u : 0x80000000u;
        }
    }
    auto dma_chunk = [&](uint32_t kc, float* tile) {
#pragma unroll
        for (int u = 0; u < kDmaMax; ++u)
            lds_load16(rbd, (lds_vptr)(reinterpret_cast<char*>(tile) + 1024u * dma_row(u)), doff[u], 4u * kc);
    };
    // byte lane % 16 of the chunk for each row.  Past the row's end the byte
    // is the next row's (or 0 past the matrix, by the range check): its
    // trits meet only b past K, which is zero, and fma(t, 0, acc) = acc.
    const int a_bytes = (int)((uint64_t)p.m * p.kp);  // below 2^31 (checked by the launcher)
    uint32_t aoff[R];
#pragma unroll
    for (int i = 0; i < R; ++i) aoff[i] = min(row0 + i, p.m - 1) * p.kp + (uint32_t)(lane & (NB - 1));
    auto load_pb = [&](uint32_t kc, uint32_t (&pb)[R]) {
        const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void*)p.a, (short)0, a_bytes, kBufWord3);
#pragma unroll
        for (int i = 0; i < R; ++i) pb[i] = __builtin_amdgcn_raw_buffer_load_b8(ra, aoff[i] + kc / 5u, 0, 0);
    };
    uint32_t pbn[R];
    float acc[R];
#pragma unroll
    for (int i = 0; i < R; ++i) acc[i] = 0.0f;
    if (p.k > 0) {
        load_pb(0, pbn);
        dma_chunk(0, bs0);
        dma_chunk(KC, bs1);
        __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt(0): chunks 0 and 1
        __builtin_amdgcn_s_barrier();
    }
    bool slow = false;  // wave-uniform: a row's sum is Inf or NaN
    // one chunk: its b in tile bb; with DMA, chunk c + 2's loads into tile nb2
    auto chunk = [&](uint32_t kc, float* bb, float* nb2) {
        // this chunk's trits: lane L holds the five of byte L % 16 of each row
        uint32_t pbc[R];
        float tr[R][5];
#pragma unroll
        for (int i = 0; i < R; ++i) {
            pbc[i] = pbn[i];
#pragma unroll
            for (int d = 0; d < 5; ++d) tr[i][d] = tlut[d * 256 + pbn[i]];
        }
        if (DMA && kc + KC > p.k) {
            // the partial last chunk: trits past K are zero (b there is the
            // next column's)
            const uint32_t k0 = kc + 5u * (uint32_t)(lane & (NB - 1));
#pragma unroll
            for (int i = 0; i < R; ++i)
#pragma unroll
                for (int d = 0; d < 5; ++d) tr[i][d] = k0 + d < p.k ? tr[i][d] : 0.0f;
        }
        if constexpr (DMA) {
            // issued for every chunk, past K too (range-checked reads into a
            // tile no chunk reads), so that the waits count only the loads
            // they are for
            load_pb(kc + KC, pbn);
            dma_chunk(kc + 2 * KC, nb2);
        }
        const f32x4* bc = reinterpret_cast<const f32x4*>(bb + (lane % CT) * kPitch);
        if (!slow) {
            // K advances 20 columns (4 bytes, 5 float4 of b) per group; the
            // next group's b is read before this group's fmas
            float saved[R];
#pragma unroll
            for (int i = 0; i < R; ++i) saved[i] = acc[i];
            f32x4 bcur[5], bnxt[5];
#pragma unroll
            for (int q = 0; q < 5; ++q) bcur[q] = bc[q];
            auto group = [&](auto gc) {
                constexpr int G = decltype(gc)::value;
                if (G < 3) {
#pragma unroll
                    for (int q = 0; q < 5; ++q) bnxt[q] = bc[5 * (G + 1) + q];
                }
                __builtin_amdgcn_sched_barrier(0);
                const float* bf = reinterpret_cast<const float*>(bcur);
                auto byte = [&](auto jc) {
                    constexpr int j = decltype(jc)::value;  // byte of the group
#pragma unroll
                    for (int d = 0; d < 5; ++d)
#pragma unroll
                        for (int i = 0; i < R; ++i) acc[i] = fmac_trit<4 * G + j>(acc[i], tr[i][d], bf[5 * j + d]);
                };
                byte(std::integral_constant<int, 0>{});
                byte(std::integral_constant<int, 1>{});
                byte(std::integral_constant<int, 2>{});
                byte(std::integral_constant<int, 3>{});
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int q = 0; q < 5; ++q) bcur[q] = bnxt[q];
            };
            group(std::integral_constant<int, 0>{});
            group(std::integral_constant<int, 1>{});
            group(std::integral_constant<int, 2>{});
            group(std::integral_constant<int, 3>{});
            // An Inf or NaN b turns the sum it enters Inf or NaN (fma(0, Inf,
            // acc) included), and so does an overflow: redo the chunk with
            // zero trits skipped from the saved sums, and keep doing so.
            bool nf = false;
#pragma unroll
            for (int i = 0; i < R; ++i) nf |= !__builtin_isfinite(acc[i]);
            if (__builtin_expect(__ballot(nf) != 0, 0)) {
                slow = true;
#pragma unroll
                for (int i = 0; i < R; ++i) acc[i] = saved[i];
            }
        }
        if (slow) {
            const uint32_t kn = min((uint32_t)KC, p.k - kc);
            const float* bf = bb + (lane % CT) * kPitch;
            for (uint32_t ki = 0; ki < kn; ++ki) {
                const float bv = bf[ki];
#pragma unroll
                for (int i = 0; i < R; ++i) {
                    // byte ki / 5 of the row, held by lane ki / 5 of this lane's 16-lane row
                    const uint32_t byte = (uint32_t)__shfl((int)pbc[i], (lane & ~15) + (int)(ki / 5u), kWave);
                    const float trv = tlut[(ki % 5u) * 256u + byte];
                    if (trv != 0.0f) acc[i] = __builtin_fmaf(trv, bv, acc[i]);
                }
            }
        }
        if constexpr (DMA) {
            // chunk c + 1's loads (and the packed bytes) landed for every
            // wave, and this chunk's tile read by all, before the next chunk;
            // no release fence (it would wait for chunk c + 2's loads too)
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(0xF70 | kDmaMax);  // all but chunk c + 2's loads
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    if constexpr (DMA) {
        // unrolled over the three tiles: chunk c in tile c % 3
        for (uint32_t kc = 0; kc < p.k; kc += 3 * KC) {
            chunk(kc, bs0, bs2);
            if (kc + KC >= p.k) break;
            chunk(kc + KC, bs1, bs0);
            if (kc + 2 * KC >= p.k) break;
            chunk(kc + 2 * KC, bs2, bs1);
        }
    }
    // no LDS load may still be in flight when the workgroup's LDS is released
    if constexpr (DMA) __builtin_amdgcn_s_waitcnt(0xF70);
    if (col < p.n) {
        // c[n, m] with four rows per lane: the lane's rows are four
        // consecutive floats of one output row, stored as one 16-byte write
        if (R == 4 && p.trans && row0 + 3 < p.m && (p.ldt & 3u) == 0 &&
            (reinterpret_cast<uintptr_t>(p.c) & 15u) == 0) {
            f32x4 v;
#pragma unroll
            for (int i = 0; i < R && i < 4; ++i) v[i] = add_bias(p.bias, acc[i] * p.sa[row0 + i], row0 + i);
            *reinterpret_cast<f32x4*>(p.c + out_idx(p, row0, col)) = v;
            return;
        }
#pragma unroll
        for (int i = 0; i < R; ++i)
            if (row0 + i < p.m) p.c[out_idx(p, row0 + i, col)] = add_bias(p.bias, acc[i] * p.sa[row0 + i], row0 + i);
    }
}

// Rows per lane: 4 for 64-column tiles and 2 for narrower ones (b read from
// LDS once per R rows; measured: 16- and 32-column tiles ran 6-12% slower
// with 4 than with 2 at every m tried, 64-column tiles 8-20% faster) while
// that leaves at least 1.5 waves per SIMD, else fewer.
template <int CT, bool TM>
static int launch_f32_rows(uint64_t m, uint64_t n, hipStream_t s, const TernF32Args& p) {
    constexpr uint64_t kSlots = kWave / CT;
    const uint64_t gy = (n + CT - 1) / CT;
    uint32_t r = CT == 64 ? 4 : 2;
    if (r == 4 && (m + 4 * kSlots - 1) / (4 * kSlots) * gy < kRowsMinWaves) r = 2;
    if (r == 4) {
        // Many rows: the SIMDs run the waves in rounds, so R rows per wave
        // cost R * ceil(waves / 1024); 5 or 7 rows where that is lower and
        // still leaves two rounds (one wave alone on a SIMD hides less
        // latency).  Measured: 13824 x 64 x 2560 111.5 (R = 4) against 104.1
        // (5) and 99.7 us (7); 6912 x 64 x 2560 65.8 (4) against 67.3 (7,
        // one round).
        uint64_t best = 0;
        for (const uint32_t rr : {4u, 5u, 7u}) {
            const uint64_t rounds = ((m + rr - 1) / rr * gy + kSimds - 1) / kSimds;
            if (rr > 4 && rounds < 2) continue;
            if (best == 0 || rr * rounds < best) best = rr * rounds, r = rr;
        }
    }
    if ((m + 2 * kSlots - 1) / (2 * kSlots) * gy < kRowsMinWaves) r = 1;
    constexpr uint32_t W = TM ? kRowsWTm : kRowsW;
    const uint64_t rows = r * kSlots * W;  // rows per workgroup
    const uint64_t bx = (m + rows - 1) / rows;
    if (bx > 0x7fffffffull || gy > 65535) return KORE_HIP_ERR_OVERFLOW;
    const dim3 gr((uint32_t)bx, (uint32_t)gy), blk(W * kWave);
    // token-major b straight into LDS where a 64-column tile of it holds
    // below 2^31 bytes (the kernel's 32-bit offsets)
    const bool dma = TM && (uint64_t)CT * p.k * 4u < 0x80000000ull;
#define KORE_ROWS_LAUNCH(RR)                                                                   \
    do {                                                                                       \
        if (dma) hipLaunchKernelGGL((ternary_f32_rows_dma_kernel<CT, RR, W>), gr, blk, 0, s, p);        \
        else hipLaunchKernelGGL((ternary_f32_rows_kernel<CT, RR, W, TM>), gr, blk, 0, s, p);            \
    } while (0)
    if constexpr (CT == 64) {
        if (r == 4) KORE_ROWS_LAUNCH(4);
        else if (r == 5) KORE_ROWS_LAUNCH(5);
        else if (r == 7) KORE_ROWS_LAUNCH(7);
        if (r >= 4) return launch_status();
    }
    if (r == 2) KORE_ROWS_LAUNCH(2);
    else KORE_ROWS_LAUNCH(1);
#undef KORE_ROWS_LAUNCH
    return launch_status();
}

// Many columns on the fp32 matrix cores.  v_mfma_f32_16x16x1_4b_f32 takes
// one K column: each of its 64 x 16 products is added to its accumulator as
// one fused multiply-add with a single rounding (checked on the GPU against
// fmaf on 5 million random operands including denormals, infinities, NaN
// and signed zeros, and on 3000-step chains: no difference), and a
// dependent MFMA that directly follows the one it depends on issues back to
// back at the full rate (32 cycles for 1024 fmas; any instruction between
// the two costs ~14 cycles, measured).  So a chain of them over k is the
// reference's fold, acc = acc + t * b in k order, for every output at once,
// at twice the vector fma rate, with the vector unit left for the operands.
//
// A wave owns 64 weight rows x 16 columns.  Operand a is lane L's row
// m0 + L (block g = L / 16 holds rows 16g .. 16g + 15); operand b is the
// 16 columns, broadcast from one 16-lane group to all four blocks by the
// BLGP field (4 + q: group q), so one b register carries four K columns:
// lane 16q + j holds b(k0 + 4q + r, n0 + j) in register r of a group of 16
// columns of K.  Trits come from a 256-entry LDS table (byte -> five
// floats).  A workgroup is four such waves on consecutive row blocks of the
// same 16 columns: b is staged once per workgroup in LDS (three buffers,
// two chunks ahead), each wave's packed bytes are loaded one chunk ahead,
// and one barrier per chunk orders the staging, over LDS only so that it
// does not wait for the loads in flight.  K advances 160 columns (32 packed
// bytes per row) per chunk (80-column chunks: 1223 against 1182 us at 6912 x
// 4096 x 2560, 119 against 107 at 256 columns).
//
// The accumulator of output (m0 + 16(v / 4) + 4(L / 16) + v % 4, n0 + L % 16)
// is register v of lane L.  Zero trits: fma(0, b, acc) = acc for finite b
// (acc is never -0); a chunk whose b holds an Inf or NaN in this wave's
// columns is done instead on the vector unit, element by element, with zero
// trits skipped (the reference's step, bit for bit).
constexpr int kMfK = 160;            // K columns per chunk
constexpr int kMfB = kMfK / 5;       // packed bytes per row and chunk
constexpr int kMfG = kMfK / 16;      // groups of 16 K columns (one b register of four per lane group)
constexpr int kMfW = kMfB / 4 + 1;   // dwords around a row's bytes of a chunk
static_assert(kMfK % 80 == 0, "whole bytes and b groups per chunk");
constexpr int kMfWaves = 4;
constexpr int kMfThreads = kMfWaves * kWave;
constexpr int kMfStage = (kMfG * 4 * 16 + kMfThreads - 1) / kMfThreads;  // 16-byte b groups per thread and chunk

struct MfBytes {
    uint32_t w[kMfB / 4];
};

// A chunk whose b holds an Inf or NaN, element by element on the vector
// unit with zero trits skipped (the reference's step).  Output v of lane L is
// row 16 (v / 4) + 4 (L / 16) + v % 4 of the wave's block, whose trit is that
// lane's a operand, and column L % 16, whose b is in lanes 16 q' + L % 16.
// Kept out of line: it runs only for such chunks.
// kmajor: the chunk's b as [K][16 columns] floats instead of [g][q][j]
// entries.
__device__ __noinline__ f32x16 mf_slow_chunk(f32x16 acc, const float* tl, const f32x4* bsb, MfBytes by, int lane,
                                             bool kmajor) {
    const int q = lane >> 4, j = lane & 15;
    for (int jb = 0; jb < kMfB; ++jb) {
        const uint32_t bv = (by.w[jb >> 2] >> (8 * (jb & 3))) & 0xffu;
        for (int d = 0; d < 5; ++d) {
            const int kk = 5 * jb + d;
            const float tv = tl[8 * bv + d];
            const int g = kk >> 4, qq = (kk >> 2) & 3, r = kk & 3;
            float bk;
            if (kmajor) {
                bk = reinterpret_cast<const float*>(bsb)[16 * kk + j];
            } else {
                const f32x4 bgv = bsb[(g * 4 + q) * 16 + j];
                float bsel = 0.0f;
#pragma unroll
                for (int rr = 0; rr < 4; ++rr)
                    if (rr == r) bsel = bgv[rr];
                bk = __shfl(bsel, 16 * qq + j, kWave);
            }
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const float te = __shfl(tv, 16 * (v >> 2) + 4 * q + (v & 3), kWave);
                if (te != 0.0f) acc[v] = __builtin_fmaf(te, bk, acc[v]);
            }
        }
    }
    return acc;
}

template <bool TM, bool DMA>
__global__ __launch_bounds__(kMfThreads) void ternary_f32_mfma_kernel(TernF32Args p) {
    // byte v -> its five trits as floats at [8 v + d] (bytes >= 243: zero
    // trits).  Measured faster than int8 entries converted on the vector
    // unit, even replicated against bank conflicts (6912 x 4096 x 2560:
    // 1239 against 1401 us): the conversions cost MFMA issue slots.
    __shared__ __attribute__((aligned(16))) float tl[256 * 8];
    // b of a chunk, three buffers (chunk c in c % 3, staged two chunks
    // ahead so that the next chunk's entries can be read before the
    // barrier that ends a chunk): group g (16 columns of K), lane group
    // q, column j -> b(kc + 16 g + 4 q + r, n0 + j) for r = 0..3 as one
    // 16-byte entry at [g][q][j] (a lane reads its own entry: conflict-free)
    __shared__ f32x4 bst[3][kMfG][4][16];
    __shared__ uint32_t bbad[3][kMfWaves];  // per wave: its staged b held an Inf or NaN
    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane(t / kWave);
    {
        uint32_t x = (uint32_t)t;
        float* e = tl + 8 * t;
#pragma unroll
        for (int d = 0; d < 5; ++d) {
            e[d] = t >= 243 ? 0.0f : (float)((int)(x % 3u) - 1);
            x /= 3u;
        }
        e[5] = e[6] = e[7] = 0.0f;
    }
    const uint32_t m0 = (blockIdx.x * kMfWaves + wave) * kWave;
    const uint32_t n0 = blockIdx.y * 16;
    const int q = lane >> 4, j = lane & 15;
    const uint32_t col = n0 + (uint32_t)j;
    // b staging: entry e = [g][qq][jj] of the chunk; thread t takes entries
    // t, t + 256 (320 per chunk)
    auto stage_load = [&](uint32_t kc, f32x4 (&v)[kMfStage]) {
        const bool full = kc + kMfK <= p.k;
#pragma unroll
        for (int u = 0; u < kMfStage; ++u) {
            const int e = t + kMfThreads * u;
            v[u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            if (e < kMfG * 4 * 16) {
                const int g = e >> 6, qq = (e >> 4) & 3, jj = e & 15;
                const uint32_t k4 = kc + 16u * g + 4u * qq, cl = n0 + (uint32_t)jj;
                if (cl < p.n) {
                    if (TM) {
                        const float* src = p.b + (uint64_t)cl * p.bn + (full || k4 < p.k ? k4 : 0u);
                        if (full) {
                            v[u] = __builtin_bit_cast(f32x4, (u32x4)*reinterpret_cast<const u32x4_a4*>(src));
                        } else {
#pragma unroll
                            for (int r = 0; r < 4; ++r) v[u][r] = k4 + r < p.k ? src[r] : 0.0f;
                        }
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const uint32_t kk = k4 + r;
                            v[u][r] = (full || kk < p.k) ? p.b[(uint64_t)kk * p.bk + cl] : 0.0f;
                        }
                    }
                }
            }
        }
    };
    auto stage_store = [&](int buf, const f32x4 (&v)[kMfStage]) {
        bool bad = false;
#pragma unroll
        for (int u = 0; u < kMfStage; ++u) {
            const int e = t + kMfThreads * u;
            if (e < kMfG * 4 * 16) {
                reinterpret_cast<f32x4*>(bst[buf])[e] = v[u];
#pragma unroll
                for (int r = 0; r < 4; ++r) bad |= !__builtin_isfinite(v[u][r]);
            }
        }
        const uint64_t bl = __ballot(bad);
        if (lane == 0) bbad[buf][wave] = bl != 0 ? 1u : 0u;
    };
    // DMA: the chunk's b straight into LDS, 10 loads of 1 KB (64 lanes x 16
    // bytes), wave w issuing loads w, w + 4, w + 8, from a range-checked
    // resource at 32-bit offsets fixed for the kernel (plus a per-chunk
    // scalar offset).  Token-major b (K % 4 == 0, b below 2 GB): entry e =
    // 64 g + 16 qq + jj is lane e % 64 of load g; columns past n and
    // entries past K (all four of their K columns, as K % 4 == 0) read
    // zeros.  [K, N] b (its offsets below 2^31 up to K + 320): the chunk as
    // [K][16 columns] floats, load g holding K columns 16 g .. + 15, lane l
    // K column 16 g + l / 4 and columns 4 (l % 4) .. + 3; K columns past K
    // read zeros, and a lane's last columns past n read the next K row's
    // first values (columns whose outputs are not stored).  Chunk c + 2's loads are issued
    // at the start of chunk c, into the buffer chunk c - 1 used; the release
    // fence before the barrier that ends chunk c waits for them (a chunk
    // lasts far longer than the loads).  No registers, no LDS stores, no
    // staging flags: Inf/NaN are found from the sums after each chunk.
    constexpr int kMfDmaRows = kMfG;                            // 1 KB loads per chunk
    constexpr int kMfDmaMax = (kMfDmaRows + kMfWaves - 1) / kMfWaves;
    constexpr uint32_t kOutOff = 0x80000000u;                    // an offset past any b this path takes
    uint32_t doff[kMfDmaMax], dk4[kMfDmaMax];
    const __amdgpu_buffer_rsrc_t rbd = __builtin_amdgcn_make_buffer_rsrc(
        (void*)p.b, (short)0, DMA ? (int)((uint64_t)p.n * p.k * 4u) : 0, kBufWord3);
    if constexpr (DMA) {
#pragma unroll
        for (int u = 0; u < kMfDmaMax; ++u) {
            const uint32_t g = wave + (uint32_t)(kMfWaves * u);
            if (TM) {
                const uint32_t cl = n0 + (uint32_t)(lane & 15);
                dk4[u] = 16u * g + 4u * (uint32_t)(lane >> 4);  // K column of the entry within its chunk
                doff[u] = cl < p.n ? (cl * p.k + dk4[u]) * 4u : kOutOff;
            } else {
                const uint32_t c4 = n0 + 4u * (uint32_t)(lane & 3);
                dk4[u] = 0u;
                doff[u] = c4 < p.n ? ((16u * g + (uint32_t)(lane >> 2)) * p.n + c4) * 4u : kOutOff;
            }
        }
    }
    auto dma_chunk = [&](uint32_t kc, uint32_t buf) {
#pragma unroll
        for (int u = 0; u < kMfDmaMax; ++u) {
            const uint32_t g = wave + (uint32_t)(kMfWaves * u);
            if (u < kMfDmaMax - 1 || g < (uint32_t)kMfDmaRows)
                lds_load16(rbd, (lds_vptr)(reinterpret_cast<char*>(&bst[buf][0][0][0]) + 1024u * g),
                           !TM || kc + dk4[u] < p.k ? doff[u] : kOutOff, TM ? 4u * kc : 4u * kc * p.n);
        }
    };
    // packed bytes of row m0 + lane: the kMfB bytes of a chunk from the
    // dword boundary below them (kMfW dwords, shifted); bytes past the row meet b = 0
    // (k >= K); the range check returns zeros past the matrix, and the
    // matrix's partial last dword is read byte by byte
    const int a_bytes = (int)((uint64_t)p.m * p.kp);  // below 2^31 (checked by the launcher)
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void*)p.a, (short)0, a_bytes, kBufWord3);
    const uint32_t arow = min(m0 + (uint32_t)lane, p.m - 1u) * p.kp;
    auto load_a = [&](uint32_t kc, uint32_t (&w)[kMfW]) {
        const uint32_t o4 = (arow + kc / 5u) & ~3u;
        if (o4 + 4u * kMfW <= (uint32_t)a_bytes) {
#pragma unroll
            for (int h = 0; h < kMfB / 16; ++h) {
                const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, o4 + 16u * h, 0, 0));
                w[4 * h] = v[0]; w[4 * h + 1] = v[1]; w[4 * h + 2] = v[2]; w[4 * h + 3] = v[3];
            }
            w[kMfW - 1] = __builtin_amdgcn_raw_buffer_load_b32(ra, o4 + 16u * (kMfB / 16), 0, 0);
        } else {
#pragma unroll
            for (int i = 0; i < kMfW; ++i) {
                const uint32_t o = o4 + 4u * i;
                uint32_t v = 0;
#pragma unroll
                for (int b = 0; b < 4; ++b) v |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(ra, o + b, 0, 0) << (8 * b);
                w[i] = v;
            }
        }
    };
    f32x16 acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
    uint32_t wn[kMfW] = {};
    f32x4 sv[kMfStage];
    if (p.k > 0) {
        if constexpr (DMA) {
            dma_chunk(0, 0);
            dma_chunk(kMfK, 1);
            load_a(0, wn);
        } else {
            stage_load(0, sv);
            stage_store(0, sv);
            stage_load(kMfK, sv);
            stage_store(1, sv);
            load_a(0, wn);
            stage_load(2 * kMfK, sv);  // past K: zeros
        }
    }
    __syncthreads();  // the table and the b of chunks 0 and 1
    // Waves past M still stage b and meet every barrier; they skip the MFMAs.
    const bool live = m0 < p.m;
    // chunk c's operands, read before the barrier that ends chunk c - 1:
    // its first b entry, its kMfB bytes and the trits of its first two
    // bytes.  Byte jb's trits are read two bytes ahead of its MFMAs and a b
    // group's entry one group ahead, each read placed between MFMAs.
    f32x4 bq[2];  // b entries of groups g (bq[g % 2]) and g + 1
    // b(kc + 16 g + 4 q + r, n0 + j) for r = 0..3 from chunk buffer bufc
    auto b_entry = [&](uint32_t bufc, int g) -> f32x4 {
        if (TM || !DMA) return bst[bufc][g][q][j];
        const float* bk = reinterpret_cast<const float*>(&bst[bufc][0][0][0]) + 16 * (16 * g + 4 * q) + j;
        return f32x4{bk[0], bk[16], bk[32], bk[48]};
    };
    uint32_t by[kMfB / 4];
    f32x4 tq[3];  // trits 0..3 of byte jb in tq[jb % 3], trit 4 in t4[jb % 3]
    float t4[3];
    auto issue = [&](int jb) {
        const uint32_t v = (by[jb >> 2] >> (8 * (jb & 3))) & 0xffu;
        tq[jb % 3] = *reinterpret_cast<const f32x4*>(tl + 8 * v);
        t4[jb % 3] = tl[8 * v + 4];
    };
    auto prep = [&](uint32_t kc, uint32_t bufc) {
        bq[0] = b_entry(bufc, 0);
        const uint32_t sh = (arow + kc / 5u) & 3u;
#pragma unroll
        for (int i = 0; i < kMfB / 4; ++i) by[i] = __builtin_amdgcn_alignbyte(wn[i + 1], wn[i], sh);
        issue(0);
        issue(1);
    };
    if (p.k > 0) prep(0, 0);
    uint32_t buf = 0;
    bool stuck = false;  // DMA: the wave's sums are no longer all finite
    for (uint32_t kc = 0; kc < p.k; kc += kMfK, buf = buf == 2u ? 0u : buf + 1u) {
        if constexpr (DMA) {
            if (kc + 2 * kMfK < p.k) dma_chunk(kc + 2 * kMfK, buf == 0u ? 2u : buf - 1u);
        }
        if (kc + kMfK < p.k) load_a(kc + kMfK, wn);
        const bool bad = DMA ? stuck : (bbad[buf][0] | bbad[buf][1] | bbad[buf][2] | bbad[buf][3]) != 0u;
        f32x16 saved;
        if constexpr (DMA) saved = acc;
        if (live && !bad) {
#pragma unroll
            for (int jb = 0; jb < kMfB; ++jb) {
#pragma unroll
                for (int d = 0; d < 5; ++d) {
                    const int kk = 5 * jb + d;  // column of the chunk
                    const float tv = d < 4 ? tq[jb % 3][d] : t4[jb % 3];
                    const int g = kk >> 4, qq = (kk >> 2) & 3, r = kk & 3;
                    const float bv = bq[g & 1][r];
                    __builtin_amdgcn_sched_barrier(0);
                    switch (qq) {
                        case 0: acc = __builtin_amdgcn_mfma_f32_16x16x1f32(tv, bv, acc, 0, 0, 4); break;
                        case 1: acc = __builtin_amdgcn_mfma_f32_16x16x1f32(tv, bv, acc, 0, 0, 5); break;
                        case 2: acc = __builtin_amdgcn_mfma_f32_16x16x1f32(tv, bv, acc, 0, 0, 6); break;
                        default: acc = __builtin_amdgcn_mfma_f32_16x16x1f32(tv, bv, acc, 0, 0, 7); break;
                    }
                    __builtin_amdgcn_sched_barrier(0);
                    if ((kk & 15) == 0 && g + 1 < kMfG) bq[(g + 1) & 1] = b_entry(buf, g + 1);
                    if (d == 0 && jb + 2 < kMfB) issue(jb + 2);
                }
            }
        }
        if constexpr (DMA) {
            // the chain adds the zero-trit terms too: a finite sum is left
            // unchanged by them, but an Inf or NaN b makes it NaN, so a
            // chunk after which some sum is not finite is folded again from
            // the saved sums with zero trits skipped
            bool nf = false;
#pragma unroll
            for (int v = 0; v < 16; ++v) nf |= !__builtin_isfinite(acc[v]);
            if (live && !bad && __ballot(nf) != 0) {
                acc = saved;
                stuck = true;
            }
        }
        if (live && (DMA ? stuck : bad)) {
            MfBytes bb;
#pragma unroll
            for (int i = 0; i < kMfB / 4; ++i) bb.w[i] = by[i];
            acc = mf_slow_chunk(acc, tl, &bst[buf][0][0][0], bb, lane, !TM && DMA);
            if constexpr (DMA) {
                bool nf = false;
#pragma unroll
                for (int v = 0; v < 16; ++v) nf |= !__builtin_isfinite(acc[v]);
                stuck = __ballot(nf) != 0;
            }
        }
        // chunk c + 2's b into its buffer (read after the barrier), chunk
        // c + 3's loads, and chunk c + 1's operands (its buffer was written
        // before the last barrier)
        if (!DMA && kc + 2 * kMfK < p.k) {
            stage_store(buf == 0u ? 2u : buf - 1u, sv);  // buffer (c + 2) % 3
            stage_load(kc + 3 * kMfK, sv);
        }
        if (kc + kMfK < p.k) prep(kc + kMfK, buf == 2u ? 0u : buf + 1u);
        // a barrier over LDS only: the global loads in flight are this
        // thread's own registers
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    }
    if (!live || col >= p.n) return;
#pragma unroll
    for (int gb = 0; gb < 4; ++gb) {
        const uint32_t mr = m0 + 16u * gb + 4u * q;  // rows mr .. mr + 3: registers 4 gb .. 4 gb + 3
        if (p.trans && mr + 3 < p.m && (p.ldt & 3u) == 0 && (reinterpret_cast<uintptr_t>(p.c) & 15u) == 0) {
            f32x4 o;
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = add_bias(p.bias, acc[4 * gb + i] * p.sa[mr + i], mr + i);
            *reinterpret_cast<f32x4*>(p.c + out_idx(p, mr, col)) = o;
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (mr + i < p.m) p.c[out_idx(p, mr + i, col)] = add_bias(p.bias, acc[4 * gb + i] * p.sa[mr + i], mr + i);
        }
    }
}

// The matrix-core kernel where its waves (64 rows x 16 columns each, one
// dependent chain of k MFMAs) give most SIMDs one: with fewer, the vector
// kernel's shorter chains win (measured: 6912 x 128 x 2560 83 against
// 103 us, 6912 x 64 x 2560 76-82 against 68-70, 2560 x 256 x 6912 214
// against 209; from 1024 columns about 2x).
constexpr uint64_t kMfMinWaves = 768;
static bool f32_use_mfma(uint64_t m, uint64_t n, uint64_t k) {
    return k > 0 && k < (1ull << 31) && ((m + 63) / 64) * ((n + 15) / 16) >= kMfMinWaves;
}

template <bool TM>
static int launch_f32_mfma(uint64_t m, uint64_t n, hipStream_t s, const TernF32Args& p) {
    const uint64_t bx = (m + kMfWaves * kWave - 1) / (kMfWaves * kWave), by = (n + 15) / 16;
    if (bx > 0x7fffffffull || by > 65535) return KORE_HIP_ERR_OVERFLOW;
    // b straight into LDS: token-major b where K % 4 == 0 (no entry
    // straddles K) and b is below 2 GB, [K, N] b where its offsets stay below
    // 2^31 up to two chunks past K (32-bit offsets)
    const bool dma = TM ? p.k % 4u == 0 && (uint64_t)p.n * p.k * 4u < 0x7fffffffull
                        : (uint64_t)p.n * (p.k + 2u * kMfK) * 4u < 0x7fffffffull;
    if (dma)
        hipLaunchKernelGGL((ternary_f32_mfma_kernel<TM, true>), dim3((uint32_t)bx, (uint32_t)by), dim3(kMfWaves * kWave), 0, s, p);
    else
        hipLaunchKernelGGL((ternary_f32_mfma_kernel<TM, false>), dim3((uint32_t)bx, (uint32_t)by), dim3(kMfWaves * kWave), 0, s, p);
    return launch_status();
}

// Decode batches (a few dozen columns) on the fp32 matrix cores with the
// 4 x 4 x 1 form: v_mfma_f32_4x4x1_16b_f32 runs 16 blocks of 4 x 4 outputs,
// each output one fused multiply-add with a single rounding per K column,
// like the 16 x 16 form (checked on the GPU against fmaf chains of 3000
// steps on random operands with denormals: no difference).  A dependent
// chain of them issues one step per ~15 cycles (measured back to back; an
// instruction between two steps of a chain costs ~13 more; two chains
// interleaved, ~10 per step each), so a wave owning 4 weight rows x 64
// columns per chain has a chain 4x shorter per K column than the 64 x 16
// waves of the 16 x 16 form, and a decode batch gets more chains to spread
// over the SIMDs.
//
// Operands (lane L, block L / 4; layout measured on the GPU): b = b(k, n0 +
// L); output register v of lane L is (row v of the chain, n0 + L).  The
// trits need no data movement: per 80-column chunk lane 4 j + r decodes
// packed byte j of the chunk of the chain's row r (its five trits as
// floats, one LDS table entry), and the MFMA of column 5 j + d takes trit d
// from block j's lanes for all 16 blocks (CBSZ = 4, ABID = j).  CH chains
// per wave (rows m0 .. m0 + 4 CH - 1) share each b read.  A workgroup is
// W waves on 4 CH W consecutive rows of the same 64 columns.  Its rows'
// packed bytes (one contiguous range) are copied into LDS at the start; b is
// staged per chunk in LDS (per column, K contiguous, pitch 84 floats: a
// lane's 16-byte reads of its own column hit 16 distinct bank groups per 16
// lanes; the staging schedule is described in the kernel).  A chunk runs as
// four bursts of 20 K columns with nothing between the MFMAs; the next
// burst's b entries are read before the current burst, the next chunk's
// trits and first b entries during the chunk.  Inf and NaN b are found
// from the sums after each chunk (see the kernel).
constexpr int kM4K = 80;                 // K columns per chunk
constexpr int kM4Rows = 32;              // rows per workgroup
constexpr int kM4Pitch4 = kM4K / 4 + 1;  // 16-byte entries per staged column
constexpr int kM4Pieces = kWave * kM4K / 4;  // 16-byte pieces of b per chunk
constexpr uint32_t kM4MaxSlice = 48 * 1024;  // bytes of packed rows a workgroup holds in LDS

// One step of a 4 x 4 x 1 chain whose trit operand is block j's (CBSZ = 4,
// ABID = j: one block's four lanes broadcast to all sixteen).
__device__ __forceinline__ f32x4 mf4_step(float a, float b, f32x4 c, int j) {
    switch (j) {
        case 0: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 0, 0);
        case 1: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 1, 0);
        case 2: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 2, 0);
        case 3: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 3, 0);
        case 4: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 4, 0);
        case 5: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 5, 0);
        case 6: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 6, 0);
        case 7: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 7, 0);
        case 8: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 8, 0);
        case 9: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 9, 0);
        case 10: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 10, 0);
        case 11: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 11, 0);
        case 12: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 12, 0);
        case 13: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 13, 0);
        case 14: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 14, 0);
        default: return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, 15, 0);
    }
}

template <bool TM, int CH, int W>
__global__ __launch_bounds__(W * kWave) void ternary_f32_mf4_kernel(TernF32Args p) {
    constexpr int kRows = 4 * CH * W;  // rows per workgroup
    constexpr int kThreads = W * kWave;
    constexpr int kStage = (kM4Pieces + kThreads - 1) / kThreads;
    __shared__ __attribute__((aligned(16))) float tl[256 * 8];
    constexpr uint32_t kBufs = TM ? 4u : 3u;  // b tiles in LDS
    __shared__ f32x4 bs[kBufs][kWave][kM4Pitch4];
    extern __shared__ uint32_t araw[];  // the workgroup's packed rows, from a dword boundary
    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane(t / kWave);
    const uint32_t r0 = blockIdx.x * kRows;  // the workgroup's first row
    const uint32_t m0 = r0 + 4u * CH * wave;   // the wave's first row
    const uint32_t n0 = blockIdx.y * kWave;
    const uint32_t col = n0 + (uint32_t)lane;
    // the packed rows r0 .. r0 + 31 (past the matrix: zeros)
    const int a_bytes = (int)((uint64_t)p.m * p.kp);
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void*)p.a, (short)0, a_bytes, kBufWord3);
    const uint32_t s_beg = r0 * p.kp, d0 = s_beg & ~3u, s_off = s_beg - d0;
    // (+ 4 words: the last chunk's trit reads of row 31 reach up to 15 bytes
    // past the slice; past the matrix they read zeros)
    const uint32_t nwords = (s_off + kRows * p.kp + 3u) / 4u + 4u;
    // The copy into araw (after the b loads of the first chunks are issued,
    // below): the words of a batch are all loaded before any is stored, so
    // the batch costs one load latency (a loop storing each word after its
    // own load paid one per word).  Words past the matrix read zeros from
    // the range-checked resource; the word that straddles its end would too,
    // so its owner thread reads its bytes one by one up front.
    const uint32_t i_s = (a_bytes & 3) != 0 ? ((uint32_t)a_bytes - d0) / 4u : 0xffffffffu;
    // One batch, no loop: nwords <= 12288 (48 KB), 24 words per thread; the
    // loads past nwords read words that are not stored.  The straddling
    // word's bytes are loaded after the batch's words, so that waiting for
    // them (loads complete in order) costs nothing beyond the batch.
    auto copy_rows = [&]() {
        constexpr int kCopyU = (int)((kM4MaxSlice / 4u + kThreads - 1) / kThreads);
        uint32_t v[kCopyU];
#pragma unroll
        for (int u = 0; u < kCopyU; ++u)
            v[u] = __builtin_amdgcn_raw_buffer_load_b32(ra, d0 + 4u * ((uint32_t)t + (uint32_t)(kThreads * u)), 0, 0);
        uint32_t w_s = 0;
        if (i_s < nwords && (uint32_t)t == i_s % (uint32_t)kThreads) {
#pragma unroll
            for (int b = 0; b < 4; ++b)
                w_s |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(ra, d0 + 4u * i_s + (uint32_t)b, 0, 0) << (8 * b);
        }
#pragma unroll
        for (int u = 0; u < kCopyU; ++u) {
            const uint32_t i = (uint32_t)t + (uint32_t)(kThreads * u);
            if (i < nwords) araw[i] = i == i_s ? w_s : v[u];
        }
    };
    auto build_table = [&]() {
        for (int i = t; i < 256; i += kThreads) {
            uint32_t x = (uint32_t)i;
            float* e = tl + 8 * i;
#pragma unroll
            for (int d = 0; d < 5; ++d) {
                e[d] = i >= 243 ? 0.0f : (float)((int)(x % 3u) - 1);
                x /= 3u;
            }
            e[5] = e[6] = e[7] = 0.0f;
        }
    };
    // b staging.  b is below 6 MB here (n <= 192, k <= 7680) and loads
    // through a range-checked resource at 32-bit byte offsets fixed for the
    // kernel: a column past n sits past the end of b and reads zeros, and
    // the resource checks each dword.
    //  - token-major b: the LDS tile is [column][21 entries of 16 bytes]
    //    (20 used), i.e. 21 rows of 64 16-byte slots per chunk, and slot s
    //    holds column s / 21, K columns 4 (s % 21) .. + 3 of the chunk (the
    //    unused entry reloads entry 19).  Wave w loads rows w, w + W, w + 2W
    //    straight into LDS (buffer loads with the LDS bit: no registers, no
    //    LDS stores).  Four tiles: chunk c + 3's loads are issued in chunk c
    //    (into the tile chunk c - 1 used) and waited for, by an explicit
    //    vmcnt, before the barrier that ends chunk c + 1, so that they have
    //    landed for every wave when chunk c + 1's last burst reads chunk
    //    c + 2's first b entries.
    //  - [K, N] b: piece e = column e % 64, K columns 4 (e / 64) .. + 3 (four
    //    loads, each a wave-wide 256-byte piece of a row of b), through
    //    registers into the same tile layout, loaded four chunks ahead and
    //    stored into LDS two chunks ahead (three tiles).  (Loading [K, N] b
    //    straight into LDS needs a [K][column] tile, read as two
    //    ds_read2st64_b32 per four K columns: measured 5% slower.)
    // Past K: [K, N] b lies past the end of b (zeros); token-major b reads
    // the next column's values, whose trits are zero (masked for the partial
    // last chunk).  Every chunk issues the same loads, chunks past K
    // included, so the waits count only the loads they are for.
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc((void*)p.b, (short)0, (int)((uint64_t)p.n * p.k * 4u), kBufWord3);
    constexpr uint32_t kOut = 0x80000000u;  // an offset past any b this kernel takes
    constexpr int kTmRows = kM4Pitch4;      // LDS-DMA rows of 64 slots per chunk
    constexpr int kDmaMax = (kTmRows + W - 1) / W;
    const int ndma = (kTmRows - (int)wave + W - 1) / W;  // this wave's rows (wave-uniform)
    uint32_t boff[TM ? kDmaMax : kStage];
    if constexpr (TM) {
#pragma unroll
        for (int u = 0; u < kDmaMax; ++u) {
            const uint32_t sl = (uint32_t)(kWave * ((int)wave + W * u) + lane);
            const uint32_t cl = n0 + sl / (uint32_t)kM4Pitch4, j = sl % (uint32_t)kM4Pitch4;
            boff[u] = cl < p.n ? (cl * p.k + 4u * (j < 20u ? j : 19u)) * 4u : kOut;
        }
    } else {
#pragma unroll
        for (int u = 0; u < kStage; ++u) {
            const int e = t + kThreads * u;
            const uint32_t cl = n0 + (uint32_t)(e % kWave), q4 = 4u * (uint32_t)(e / kWave);
            boff[u] = e < kM4Pieces && cl < p.n ? (q4 * p.n + cl) * 4u : kOut;
        }
    }
    auto dma_chunk = [&](uint32_t kc, uint32_t buf) {
#pragma unroll
        for (int u = 0; u < kDmaMax; ++u) {
            if (u < kDmaMax - 1 || u < ndma) {
                lds_load16(rb, (lds_vptr)((char*)&bs[buf][0][0] + 1024 * ((int)wave + W * u)), boff[u], 4u * kc);
            }
        }
    };
    // the wait for the LDS loads of all but the last `pending` chunks issued
    auto dma_wait = [&](bool pending) {
        if (!pending) {
            __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt(0)
        } else if (ndma == kDmaMax) {
            __builtin_amdgcn_s_waitcnt(0xF70 | kDmaMax);
        } else {
            __builtin_amdgcn_s_waitcnt(0xF70 | (kDmaMax - 1));
        }
    };
    auto stage_load = [&](uint32_t kc, f32x4 (&v)[kStage]) {
#pragma unroll
        for (int u = 0; u < kStage; ++u)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                v[u][r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rb, boff[u] + 4u * (kc + r) * p.n, 0, 0));
    };
    auto stage_store = [&](uint32_t buf, const f32x4 (&v)[kStage]) {
#pragma unroll
        for (int u = 0; u < kStage; ++u) {
            const int e = t + kThreads * u;
            if (e < kM4Pieces) bs[buf][e % kWave][e / kWave] = v[u];
        }
    };
    f32x4 acc[CH];
#pragma unroll
    for (int h = 0; h < CH; ++h) acc[h] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 sv0[TM ? 1 : kStage], sv1[TM ? 1 : kStage];
    // the b of the first chunks, then the packed rows and the table while
    // those loads are in flight
    if constexpr (TM) {
        dma_chunk(0, 0);
        dma_chunk(kM4K, 1);
        dma_chunk(2 * kM4K, 2);
    } else {
        stage_load(0, sv0);
        stage_load(kM4K, sv1);
    }
    copy_rows();
    build_table();
    if constexpr (TM) {
        dma_wait(true);  // chunks 0 and 1 (chunk 2's: by the end of chunk 0)
    } else {
        stage_store(0, sv0);
        stage_store(1, sv1);
        stage_load(2 * kM4K, sv0);  // stored by chunk 0 where chunk 2 exists
        stage_load(3 * kM4K, sv1);
    }
    // the table, the packed rows and the b of chunks 0 and 1 (token-major b:
    // no release fence, which would wait for chunk 2's loads too; the
    // table and the packed rows are LDS stores, waited for by lgkmcnt(0))
    if constexpr (TM) {
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
    } else {
        __syncthreads();
    }
    const bool live = m0 < p.m;
    // lane 4 j + r: byte j of the chunk of chain h's row r
    const uint8_t* abytes = reinterpret_cast<const uint8_t*>(araw);
    const uint32_t aoff = s_off + (4u * CH * wave + (uint32_t)(lane & 3)) * p.kp + (uint32_t)(lane >> 2);
    f32x4 tq[CH], tqn[CH];  // trits 0..3 of this lane's byte, per chain (this chunk, the next)
    float t4[CH], t4n[CH];  // trit 4
    auto trit_bytes = [&](uint32_t kc, uint32_t (&v)[CH]) {
#pragma unroll
        for (int h = 0; h < CH; ++h) v[h] = abytes[aoff + 4u * h * p.kp + kc / 5u];
    };
    // the trits of chunk kc (zero past K: the packed matrix's last byte of a
    // row may hold any digits there, and token-major b is not zero there)
    auto trit_table = [&](uint32_t kc, const uint32_t (&v)[CH], f32x4 (&q)[CH], float (&q4)[CH]) {
#pragma unroll
        for (int h = 0; h < CH; ++h) {
            q[h] = *reinterpret_cast<const f32x4*>(tl + 8 * v[h]);
            q4[h] = tl[8 * v[h] + 4];
        }
        if (kc + kM4K > p.k) {
            const uint32_t k0 = kc + 5u * (uint32_t)(lane >> 2);
#pragma unroll
            for (int h = 0; h < CH; ++h) {
#pragma unroll
                for (int d = 0; d < 4; ++d) q[h][d] = k0 + d < p.k ? q[h][d] : 0.0f;
                q4[h] = k0 + 4 < p.k ? q4[h] : 0.0f;
            }
        }
    };
    auto nonfinite = [&]() {
        bool nf = false;
#pragma unroll
        for (int h = 0; h < CH; ++h)
#pragma unroll
            for (int r = 0; r < 4; ++r) nf |= !__builtin_isfinite(acc[h][r]);
        return __ballot(nf) != 0;
    };
    f32x4 bq[2][5];  // b entries of a burst (20 K columns)
    auto read_b = [&](f32x4 (&q)[5], uint32_t buf, int bi) {
#pragma unroll
        for (int g = 0; g < 5; ++g) q[g] = bs[buf][lane][5 * bi + g];
    };
    // The reference's step over chunk buf, element by element: output v of
    // lane L is row v of chain h, whose trit d of byte j lane 4 j + v holds.
    auto slow_chunk = [&](uint32_t buf) {
        for (int kk = 0; kk < kM4K; ++kk) {
            const int j = kk / 5, d = kk % 5;
            const float bk = bs[buf][lane][kk >> 2][kk & 3];
#pragma unroll
            for (int h = 0; h < CH; ++h) {
                float tv = t4[h];
#pragma unroll
                for (int dd = 0; dd < 4; ++dd)
                    if (dd == d) tv = tq[h][dd];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float te = __shfl(tv, 4 * j + r, kWave);
                    if (te != 0.0f) acc[h][r] = __builtin_fmaf(te, bk, acc[h][r]);
                }
            }
        }
    };
    // Inf and NaN: the matrix-core chain adds the zero-trit terms too, which
    // leave a finite sum unchanged (fma(0, b, s) = s for finite b; s is
    // never -0) but make it NaN for an infinite or NaN b.  So a chunk after
    // which some sum of the wave is not finite is folded again from the saved
    // sums, element by element with zero trits skipped (the reference's step;
    // a sum that overflowed gives the same result either way), and a wave
    // whose sums are no longer finite stays on that path.
    bool stuck = false;
    if (p.k > 0) {
        uint32_t tb[CH];
        trit_bytes(0, tb);
        trit_table(0, tb, tq, t4);
        read_b(bq[0], 0, 0);
    }
    // One chunk: its four bursts and, spread over them so that no LDS wait
    // stands before a burst's MFMAs, the staging of a later chunk into the
    // tile chunk c - 1 used (last read before the last barrier; token-major:
    // chunk c + 3's LDS loads, burst 0; [K, N]: chunk c + 2's LDS stores from
    // the registers loaded two chunks ago, burst 3), chunk c + 1's trit bytes
    // (burst 0), its trits from the table (burst 2) and its first b entries
    // (burst 3); then the Inf/NaN check, chunk c + 4's [K, N] loads, the
    // wait for chunk c + 2's token-major loads and a barrier over LDS only.  On the last chunk the
    // next-chunk reads re-read this chunk's (valid addresses, results
    // unused), so that no branch joins before a burst.
    auto chunk = [&](uint32_t kc, uint32_t buf, f32x4 (&svc)[TM ? 1 : kStage]) {
        const uint32_t nbuf = buf + 1u == kBufs ? 0u : buf + 1u, sbuf = buf == 0u ? kBufs - 1u : buf - 1u;
        const uint32_t kahead = TM ? 3u : 2u;  // the chunk staged into sbuf
        const uint32_t kn = kc + kM4K < p.k ? kc + kM4K : kc;
        const bool store = kc + kahead * kM4K < p.k;
        uint32_t tb[CH];
        if (live && !stuck) {
            f32x4 saved[CH];
#pragma unroll
            for (int h = 0; h < CH; ++h) saved[h] = acc[h];
#pragma unroll
            for (int bi = 0; bi < 4; ++bi) {
                if (bi < 3) read_b(bq[(bi + 1) & 1], buf, bi + 1);
                if (bi == 0) {
                    if constexpr (TM) {
                        if (store) dma_chunk(kc + kahead * kM4K, sbuf);
                    }
                    trit_bytes(kn, tb);
                }
                if (bi == 2) trit_table(kn, tb, tqn, t4n);
                if (bi == 3) {
                    if constexpr (!TM) {
                        if (store) stage_store(sbuf, svc);
                    }
                    read_b(bq[0], nbuf, 0);
                }
                const f32x4(&q)[5] = bq[bi & 1];
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int u = 0; u < 4; ++u) {
#pragma unroll
                    for (int d = 0; d < 5; ++d) {
                        const int kk = 5 * u + d;
#pragma unroll
                        for (int h = 0; h < CH; ++h)
                            acc[h] = mf4_step(d < 4 ? tq[h][d] : t4[h], q[kk >> 2][kk & 3], acc[h], 4 * bi + u);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            if (nonfinite()) {
#pragma unroll
                for (int h = 0; h < CH; ++h) acc[h] = saved[h];
                slow_chunk(buf);
                stuck = nonfinite();
            }
        } else {
            if (live) {
                slow_chunk(buf);
                stuck = nonfinite();
            }
            if constexpr (TM) {
                if (store) dma_chunk(kc + kahead * kM4K, sbuf);
            } else {
                if (store) stage_store(sbuf, svc);
            }
            trit_bytes(kn, tb);
            trit_table(kn, tb, tqn, t4n);
            read_b(bq[0], nbuf, 0);
        }
        if constexpr (!TM) stage_load(kc + 4 * kM4K, svc);
#pragma unroll
        for (int h = 0; h < CH; ++h) {
            tq[h] = tqn[h];
            t4[h] = t4n[h];
        }
        if constexpr (TM) {
            // no release fence: it would wait for the LDS loads still in
            // flight for chunk c + 3; this wave's reads of buffer c have
            // all been consumed, and no wave writes LDS but by those loads
            __builtin_amdgcn_sched_barrier(0);
            dma_wait(store);
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
        } else {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        }
    };
    uint32_t buf = 0;
    for (uint32_t kc = 0; kc < p.k; kc += 2 * kM4K) {
        chunk(kc, buf, sv0);
        buf = buf + 1u == kBufs ? 0u : buf + 1u;
        if (kc + kM4K >= p.k) break;
        chunk(kc + kM4K, buf, sv1);
        buf = buf + 1u == kBufs ? 0u : buf + 1u;
    }
    if (!live || col >= p.n) return;
#pragma unroll
    for (int h = 0; h < CH; ++h) {
        const uint32_t mr = m0 + 4u * h;
        if (mr >= p.m) break;
        if (p.trans && mr + 3 < p.m && (p.ldt & 3u) == 0 && (reinterpret_cast<uintptr_t>(p.c) & 15u) == 0) {
            f32x4 out;
#pragma unroll
            for (int r = 0; r < 4; ++r) out[r] = add_bias(p.bias, acc[h][r] * p.sa[mr + r], mr + r);
            *reinterpret_cast<f32x4*>(p.c + out_idx(p, mr, col)) = out;
        } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (mr + r < p.m) p.c[out_idx(p, mr + r, col)] = add_bias(p.bias, acc[h][r] * p.sa[mr + r], mr + r);
        }
    }
}

// Bytes of the packed-row slice a workgroup copies into LDS (0: too long for
// this kernel).
static uint32_t f32_mf4_slice(uint64_t kp) {
    const uint64_t words = (3u + kM4Rows * kp + 3u) / 4u + 4u;
    return words * 4u <= kM4MaxSlice ? (uint32_t)(words * 4u) : 0u;
}

// Where the 4 x 4 kernel runs: 41 to 192 columns, K from 2560 (its fixed
// costs -- the packed-row copy, the staging prologue -- spread over enough
// chunks), no 16 x 16 launch for the shape, and at least 640 waves of 4
// rows x 64 columns with token-major b (the layer), 1024 with [K, N] b (the
// plain ternary_matmul).  Up to 1024 waves a SIMD runs one wave, whose
// chain time does not shrink with m, so below that the row-broadcast
// kernel, whose time does, wins at some m.  Measured (HIP events; the
// row-broadcast kernel on the same box; layer, then [K, N]):
//   6912 x 64 x 2560 (1728 waves): 42.2 and 46.0 us against 70 and 66;
//   6912 x 96 x 2560: 81 and 90 against 107 and 102;
//   2560 x {96, 192} x 6912 (1280-1920 waves): 105-110 and 116-125 against
//   143-195;
//   2560 x 64 x 6912 (640 waves): 104 and 114 against 116 and 104;
//   3500 x 64 x 4096 (875 waves): 64 and 71 against 67 and 71;
//   3000 x 64 x 2560 (750 waves): 40.5 and 45.1 against 45.4 and 42.1;
//   2048 x 64 x 6912 (512 waves): 104 and 114 against 80 and 80;
//   24 and 32 columns: 47-49 against 38-39 us at 6912 x 2560 (the 64-column
//   waves half empty).
// Two chains per wave (8 rows, each b read shared by both; 864 waves at
// 6912 x 64) measured 5% slower, and workgroups of 7 waves (247 instead of
// 216 workgroups at 6912 rows, one per CU) 6% slower.
static bool f32_use_mf4(uint64_t m, uint64_t n, uint64_t k, uint64_t kp, bool tm) {
    if (n < 41 || n > 192 || k < 2560 || f32_use_mfma(m, n, k) || f32_mf4_slice(kp) == 0) return false;
    return (m + 3) / 4 * ((n + kWave - 1) / kWave) >= (tm ? 640u : 1024u);
}

template <bool TM, int CH, int W>
static int launch_f32_mf4_w(uint64_t m, uint64_t n, hipStream_t s, const TernF32Args& p) {
    const uint64_t bx = (m + 4 * CH * W - 1) / (4 * CH * W), by = (n + kWave - 1) / kWave;
    if (bx > 0x7fffffffull || by > 65535) return KORE_HIP_ERR_OVERFLOW;
    const uint32_t lds = f32_mf4_slice(p.kp);
    if (lds == 0) return KORE_HIP_ERR_BAD_DIM;
    hipLaunchKernelGGL((ternary_f32_mf4_kernel<TM, CH, W>), dim3((uint32_t)bx, (uint32_t)by), dim3(W * kWave), lds, s, p);
    return launch_status();
}

template <bool TM>
static int launch_f32_mf4(uint64_t m, uint64_t n, hipStream_t s, const TernF32Args& p) {
    return launch_f32_mf4_w<TM, 1, 8>(m, n, s, p);
}

// One to four columns (decode steps), any row alignment.  The
// fold is a chain of k dependent f32 operations per output, so its floor is k
// times the latency of one dependent vector operation (about 8 cycles for a
// single wave); the per-lane kernel above also puts the decode, the table and
// the b reads into that chain's wave.  Here a workgroup owns 64 rows: six
// waves decode, and one fold wave per column runs the chain.  With one
// column the decoders form the terms t * b in LDS and the fold wave adds
// them, nothing else in its instruction stream but the 16-byte LDS reads of
// the terms (with more columns, see the kernel).
//
// A term is fl(t * b) = +-b exactly for a nonzero trit and +-0 for a zero
// one, and acc + (+-0) = acc (acc is never -0): acc + term is the
// reference's acc + t * b with zero trits skipped, bit for bit.  Where b is
// Inf or NaN, 0 * b would be NaN: in such a step the terms are selected
// instead (+0 for a zero trit).  The decode is f32 arithmetic, no tables: with
// c the f32 just above 1/3^i, floor(byte * c) is byte / 3^i for every byte <
// 243 (exhaustively true), and the base-3 digits u follow exactly as
// q_i - 3 q_(i+1); the term is fma(u, b, -b) = (u - 1) * b, exact.
//
// K advances in steps of 240 columns (48 packed bytes per row; decoder d
// takes bytes [8 d, 8 d + 8) = columns [40 d, 40 d + 40)), double-buffered:
// in iteration s the decoders write the terms of step s (and stage b of step
// s + 1) while the fold wave reads the terms of step s - 1; one barrier per
// iteration separates them.  The decoders keep the packed bytes and b of the
// next kPfDepth steps in flight.
constexpr int kPfStep = 240;               // K columns per step
constexpr int kPfDec = 6;                  // decoding waves
constexpr int kDecB = kPfStep / 5 / kPfDec;  // packed bytes per decoder and step
constexpr int kDecQ = kDecB * 5 / 4;         // ... as groups of 4 terms
static_assert(kDecB * kPfDec * 5 == kPfStep && kDecB % 4 == 0, "decoder split");
constexpr int kPfQuads = kPfStep / 4;      // 16-byte groups of 4 terms per step
constexpr int kPfDepth = 2;                // steps of loads in flight

// One workgroup per CU (its LDS); the launch bound (7 to 10 waves, 2 or 3
// per SIMD) caps the registers.
//
// CT = 1: the decoders write the terms t * b and the fold wave adds them.
// CT = 2 or 4 columns (decode batches of 2-4 tokens): the decoders write the
// trits once (as floats) and fold wave c of the CT computes
// acc = fma(t, b[., c], acc), b read from LDS (the same address in every
// lane); a step whose column-c b holds an Inf or NaN skips zero trits
// explicitly.
template <int CT>
__global__ __launch_bounds__((kPfDec + CT) * kWave)
void ternary_f32_pipe_kernel(TernF32Args p) {
    constexpr int kStageN = (CT * kPfStep + kPfDec * kWave - 1) / (kPfDec * kWave);  // b elements per decoder lane
    // terms (CT = 1) or trits of the step per group of 4 K columns,
    // lane-major (a lane reads and writes 16 consecutive bytes:
    // conflict-free); 120 KB
    __shared__ f32x4 tb[2][kPfQuads][kWave];
    // b of a step per column, zero past k and n; three buffers: in iteration
    // s the decoders write step s + 1 while the fold waves read step s - 1
    // (and the decoders, for one column, step s)
    __shared__ f32x4 bb[3][CT][kPfQuads];
    __shared__ uint32_t bflag[2][kPfDec];   // per decoder: columns whose staged b holds an Inf or NaN
    __shared__ uint32_t tmask[2];           // the same for the step whose trits are in tb[buf]
    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const int wave = t / kWave;
    const uint32_t row = blockIdx.x * kWave + lane;
    const uint32_t col0 = blockIdx.y * CT;
    const uint32_t steps = (p.k + kPfStep - 1) / kPfStep;
    // the decoders run whole rounds of kPfDepth steps (the ones past K decode
    // zeros), so that every round issues and waits for its loads alike
    const uint32_t steps_p = (steps + kPfDepth - 1) / kPfDepth * kPfDepth;
    // b staging: decoder lane e takes elements e + h * (decoder lanes) of the
    // step's CT x 240 (K-major, as b[K, N] is stored)
    const int e = (wave - CT) * kWave + lane;
    constexpr int kSL = kPfDec * kWave;
    auto b_ok = [&](uint32_t s, int h) {
        const int i = e + kSL * h;
        return i < CT * kPfStep && s * kPfStep + (uint32_t)(i / CT) < p.k && col0 + (uint32_t)(i % CT) < p.n;
    };
    auto b_idx = [&](uint32_t s, int h) {
        const int i = e + kSL * h;
        return b_ok(s, h) ? (uint64_t)(s * kPfStep + (uint32_t)(i / CT)) * p.bk + (uint64_t)(col0 + (uint32_t)(i % CT)) * p.bn
                          : 0u;
    };
    float bv[kPfDepth][kStageN];
    // stage b of step s into bb[s % 3]; bflag[buf][d]: the columns in which
    // decoder d staged an Inf or NaN
    auto stage_b = [&](uint32_t s, int buf, const float (&v)[kStageN]) {
        const uint32_t bbuf = s % 3u;
        uint32_t bad = 0;
#pragma unroll
        for (int h = 0; h < kStageN; ++h) {
            const int i = e + kSL * h;
            if (i < CT * kPfStep) {
                const float x = b_ok(s, h) ? v[h] : 0.0f;
                reinterpret_cast<float*>(bb[bbuf][i % CT])[i / CT] = x;
                bad |= __builtin_isfinite(x) ? 0u : 1u << (i % CT);
            }
        }
        uint32_t mask = 0;
#pragma unroll
        for (int c = 0; c < CT; ++c) mask |= __any((bad >> c) & 1u) ? 1u << c : 0u;
        if (lane == 0) bflag[buf][wave - CT] = mask;
    };
    if (wave >= CT) {
        float v[kStageN];
#pragma unroll
        for (int h = 0; h < kStageN; ++h) v[h] = p.b[b_idx(0, h)];
        stage_b(0, 0, v);
    }
    __syncthreads();  // b of step 0
    if (wave < CT) {
        // fold wave of column col0 + wave
        const int c = wave;
        float acc = 0.0f;
        for (uint32_t s = 0; s <= steps_p; ++s) {
            if (s > 0 && s <= steps) {
                const int buf = (s - 1) & 1;
                const uint32_t bbuf = (s - 1) % 3u;
                // batches of kFb groups, the next batch's reads in flight
                // during a batch's operations
                constexpr int kFb = CT == 1 ? 6 : 4;
                if (CT == 1 || ((tmask[buf] >> c) & 1u) == 0u) {
                    f32x4 tq[2][kFb], bq[2][kFb];
                    auto rd = [&](int slot, int g0) {
#pragma unroll
                        for (int i = 0; i < kFb; ++i) {
                            tq[slot][i] = tb[buf][g0 + i][lane];
                            if (CT > 1) bq[slot][i] = bb[bbuf][c][g0 + i];
                        }
                    };
                    rd(0, 0);
#pragma unroll
                    for (int bt = 0; bt < kPfQuads / kFb; ++bt) {
                        const int cur = bt & 1;
                        if (bt + 1 < kPfQuads / kFb) rd(cur ^ 1, (bt + 1) * kFb);
#pragma unroll
                        for (int i = 0; i < kFb; ++i)
#pragma unroll
                            for (int j = 0; j < 4; ++j) {
                                if (CT == 1) acc += tq[cur][i][j];
                                else acc = __builtin_fmaf(tq[cur][i][j], bq[cur][i][j], acc);
                            }
                    }
                } else {
                    for (int g = 0; g < kPfQuads; ++g) {
                        const f32x4 t4 = tb[buf][g][lane];
                        const f32x4 b4 = bb[bbuf][c][g];
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            if (t4[j] != 0.0f) acc = __builtin_fmaf(t4[j], b4[j], acc);
                    }
                }
            }
            __syncthreads();
        }
        if (row < p.m && col0 + c < p.n) p.c[out_idx(p, row, col0 + c)] = add_bias(p.bias, acc * p.sa[row], row);
        return;
    }
    const int d = wave - CT;
    const uint8_t* arow = p.a + (uint64_t)(row < p.m ? row : 0u) * p.kp;
    // Loads are unconditional, at clamped in-bounds addresses; what lies
    // past the row or past k is replaced when the step is used (a select
    // right after a load would wait for it).  A decoder's 8 bytes of a step
    // come from the three dwords around them (any row alignment), the first
    // at floor4(address), clamped to the dwords wholly inside the matrix,
    // [ceil4(start), floor4(end)) (the host launches this kernel for
    // m * kp >= 20 only, so that span holds at least three dwords); the bytes
    // are then at offset o = address - first dword.  A step whose bytes reach
    // into the matrix's partial first or last dword (unaligned matrices only)
    // reads those bytes one by one instead.
    static_assert(kDecB == 8, "three-dword window");
    const uintptr_t a_lo = reinterpret_cast<uintptr_t>(p.a);
    const uintptr_t a_hi = a_lo + (uintptr_t)p.m * p.kp;
    const uintptr_t a_lo4 = (a_lo + 3u) & ~(uintptr_t)3, a_hi4 = a_hi & ~(uintptr_t)3;
    auto pb_of = [&](uint32_t s) { return s * (kPfStep / 5) + (uint32_t)(kDecB * d); };
    auto addr_of = [&](uint32_t s) {
        return reinterpret_cast<uintptr_t>(arow) + (pb_of(s) < p.kp ? pb_of(s) : 0u);
    };
    auto first_of = [&](uintptr_t a) { return min(max(a & ~(uintptr_t)3, a_lo4), a_hi4 - 12u); };
    uint32_t pk[kPfDepth][3];
    auto load = [&](uint32_t s, int r) {
        const uint32_t* w = reinterpret_cast<const uint32_t*>(first_of(addr_of(s)));
#pragma unroll
        for (int i = 0; i < 3; ++i) pk[r][i] = w[i];
#pragma unroll
        for (int h = 0; h < kStageN; ++h) bv[r][h] = p.b[b_idx(s + 1, h)];
        // keep every step's loads in one order (prologue and loop alike), so
        // that each step waits only for its own
        __builtin_amdgcn_sched_barrier(0);
    };
#pragma unroll
    for (int r = 0; r < kPfDepth; ++r) load((uint32_t)r, r);
    for (uint32_t s0 = 0; s0 < steps_p; s0 += kPfDepth) {
#pragma unroll
        for (int r = 0; r < kPfDepth; ++r) {
            const uint32_t s = s0 + r;
            const int buf = s & 1;
            const f32x4* bq = bb[s % 3u][0] + kDecQ * d;
            uint32_t any_bad = 0;
#pragma unroll
            for (int i = 0; i < kPfDec; ++i) any_bad |= bflag[buf][i];
            if (CT > 1 && d == 0 && lane == 0) tmask[buf] = any_bad;
            const bool safe = any_bad == 0u;
            // b of step s + 1 into the other buffer (read after the barrier)
            stage_b(s + 1, buf ^ 1, bv[r]);
            // the slice's b first (one column), then the digits, the terms
            // and the stores
            f32x4 bx[kDecQ];
            if (CT == 1) {
#pragma unroll
                for (int q = 0; q < kDecQ; ++q) bx[q] = bq[q];
            }
            // the step's 8 bytes (bytes past the row: 121, five zero trits)
            uint32_t wd[2];
            {
                const uintptr_t a = addr_of(s);
                const uint32_t o = (uint32_t)(a - first_of(a));
                const uint32_t o4 = o >> 2, sh = o & 3u;
                const uint32_t e0 = o4 == 0 ? pk[r][0] : (o4 == 1 ? pk[r][1] : pk[r][2]);
                const uint32_t e1 = o4 == 0 ? pk[r][1] : (o4 == 1 ? pk[r][2] : 0u);
                const uint32_t e2 = o4 == 0 ? pk[r][2] : 0u;
                wd[0] = __builtin_amdgcn_alignbyte(e1, e0, sh);
                wd[1] = __builtin_amdgcn_alignbyte(e2, e1, sh);
                const uint32_t pb = pb_of(s);
                const uint32_t nvalid = pb < p.kp ? min(p.kp - pb, (uint32_t)kDecB) : 0u;  // step-uniform
                if (a < a_lo4 || a + nvalid > a_hi4) {  // the matrix's partial first or last dword
                    const uint8_t* ab = reinterpret_cast<const uint8_t*>(a);
#pragma unroll
                    for (int j = 0; j < kDecB; ++j) {
                        const uint32_t v = (uint32_t)j < nvalid ? ab[j] : kZeroByte;
                        wd[j / 4] = (wd[j / 4] & ~(0xffu << (8 * (j % 4)))) | (v << (8 * (j % 4)));
                    }
                }
                if (nvalid < (uint32_t)kDecB) {
#pragma unroll
                    for (int j = 0; j < kDecB; ++j)
                        if ((uint32_t)j >= nvalid)
                            wd[j / 4] = (wd[j / 4] & ~(0xffu << (8 * (j % 4)))) | (kZeroByte << (8 * (j % 4)));
                }
            }
            // base-3 digits u = t + 1 of each byte; bytes >= 243 decode as
            // 121 (all zero trits).  Each stage runs over all the bytes
            // before the next, so that no operation waits on the one just
            // issued.
            float x[kDecB], q[4][kDecB], u[kDecB * 5];
#pragma unroll
            for (int j = 0; j < kDecB; ++j) {
                const uint32_t w = wd[j / 4];
                x[j] = (float)((w >> (8 * (j % 4))) & 0xffu);
            }
#pragma unroll
            for (int j = 0; j < kDecB; ++j) x[j] = x[j] >= 243.0f ? 121.0f : x[j];
            constexpr float kInv3[4] = {0x1.555558p-2f, 0x1.c71c74p-4f, 0x1.2f684ep-5f, 0x1.948b12p-7f};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < kDecB; ++j) q[i][j] = x[j] * kInv3[i];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < kDecB; ++j) q[i][j] = __builtin_floorf(q[i][j]);
#pragma unroll
            for (int j = 0; j < kDecB; ++j) {
                u[5 * j] = __builtin_fmaf(q[0][j], -3.0f, x[j]);
                u[5 * j + 1] = __builtin_fmaf(q[1][j], -3.0f, q[0][j]);
                u[5 * j + 2] = __builtin_fmaf(q[2][j], -3.0f, q[1][j]);
                u[5 * j + 3] = __builtin_fmaf(q[3][j], -3.0f, q[2][j]);
                u[5 * j + 4] = q[3][j];
            }
            if (CT > 1) {
                // the trits t = u - 1
#pragma unroll
                for (int q = 0; q < kDecQ; ++q)
                    tb[buf][kDecQ * d + q][lane] =
                        f32x4{u[4 * q] - 1.0f, u[4 * q + 1] - 1.0f, u[4 * q + 2] - 1.0f, u[4 * q + 3] - 1.0f};
            } else if (safe) {
                // term = (u - 1) * b: fma(u, b, -b) is exact (-b, +0 or b)
                // for finite b; otherwise selected, +0 for a zero trit
#pragma unroll
                for (int q = 0; q < kDecQ; ++q) {
                    f32x4 v;
#pragma unroll
                    for (int c = 0; c < 4; ++c) v[c] = __builtin_fmaf(u[4 * q + c], bx[q][c], -bx[q][c]);
                    tb[buf][kDecQ * d + q][lane] = v;
                }
            } else {
#pragma unroll
                for (int q = 0; q < kDecQ; ++q) {
                    f32x4 v;
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        v[c] = u[4 * q + c] == 1.0f ? 0.0f : (u[4 * q + c] == 0.0f ? -bx[q][c] : bx[q][c]);
                    tb[buf][kDecQ * d + q][lane] = v;
                }
            }
            // unconditional (in bounds past the last step too), so that the
            // wait for each step's loads is a fixed count
            load(s + kPfDepth, r);
            __syncthreads();
        }
    }
    __syncthreads();  // the fold of the last step
}


// ---------------------------------------------------------------------------
// Weight packing, the weight-side format of the matmuls above
// (pack_weights_ternary, cpu_ternary_matmul.rs:198-240; encode_trits,
// kore-btes/src/encoder.rs:72-86): per row, scale = max |w| (f32::max drops
// NaN; 1.0 below 1e-8), trit = +1 / -1 / 0 for w / scale (the IEEE quotient)
// > threshold / < -threshold / otherwise (NaN: 0), and byte j = sum over i of
// (trit[5 j + i] + 1) * 3^i, zero trits past k.  HBM-bound: 4 m k bytes
// read, m ceil(k/5) + 4 m written.
//
// Vector path (k % 4 == 0, 16-byte aligned rows): one wave per row for
// k <= 1280, a workgroup of two waves per row for k <= 2560, else of four
// (k <= 40960), the waves' row maxima meeting in LDS; a lane holds its 20-float
// chunks in registers, so the row is read once; a chunk packs into 4 bytes
// (one dword store where the packed rows are dword-aligned).  Otherwise the
// generic path reads the row twice (max, then one byte per lane and step).
constexpr int kPackWaves = 4;

// The next float above (up) or below x, for finite x.
__device__ __forceinline__ float float_next(float x, bool up) {
    if (x == 0.0f) return up ? 0x1p-149f : -0x1p-149f;
    const uint32_t b = __builtin_bit_cast(uint32_t, x);
    return __builtin_bit_cast(float, (x > 0.0f) == up ? b + 1u : b - 1u);
}

__device__ __forceinline__ uint32_t trit_digit(float x, float scale, float threshold) {
    const float nv = x / scale;
    return nv > threshold ? 2u : (nv < -threshold ? 0u : 1u);
}

// RB: a workgroup per row (long rows): wave w takes the 64-chunk slices w,
// w + 4, ..., and the row max meets in LDS.
template <int NC, bool RB, int W = kPackWaves>
__global__ __launch_bounds__(W * kWave) void ternary_pack_vec_kernel(const float* __restrict__ w, uint64_t m,
                                                                              uint32_t k, float threshold,
                                                                              uint8_t* __restrict__ packed,
                                                                              float* __restrict__ scales) {
    // per wave: 64 chunks of 20 floats, staged to turn coalesced loads into
    // each lane's own chunk
    __shared__ f32x4 stage[W][5 * kWave];
    __shared__ float red[W];
    const int lane = threadIdx.x & (kWave - 1);
    const int wv = threadIdx.x / kWave;
    const uint64_t row = RB ? (uint64_t)blockIdx.x : (uint64_t)blockIdx.x * W + wv;
    if (!RB && row >= m) return;  // whole waves; only wave-local LDS sync below
    auto slice = [&](int c) { return RB ? wv + W * c : c; };  // this wave's c-th 64-chunk slice
    const uint32_t n4 = k / 4;  // float4s in the row
    const f32x4* rd = reinterpret_cast<const f32x4*>(w + row * k);
    // coalesced loads: iteration c, step q -> float4 320 c + 64 q + lane
    f32x4 g[NC][5];
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int q = 0; q < 5; ++q) {
            const uint32_t i = (uint32_t)(320 * slice(c) + 64 * q + lane);
            g[c][q] = ld_stream(rd + (i < n4 ? i : 0u));  // clamped, in-bounds
        }
    float amax = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int q = 0; q < 5; ++q)
            if ((uint32_t)(320 * slice(c) + 64 * q + lane) < n4)
#pragma unroll
                for (int e = 0; e < 4; ++e) amax = fmaxf(amax, fabsf(g[c][q][e]));
    amax = wave_max(amax);
    if (RB) {
        if (lane == 0) red[wv] = amax;
        __syncthreads();
#pragma unroll
        for (int i = 0; i < W; ++i) amax = fmaxf(amax, red[i]);
    }
    const float scale = amax < 1e-8f ? 1.0f : amax;
    if (lane == 0 && (!RB || wv == 0)) scales[row] = scale;
    // The comparisons as bounds on w: fl(w / scale) is monotone in w and odd,
    // so with xh the largest float whose quotient is <= threshold,
    // quotient > threshold <=> w > xh and quotient < -threshold <=> w < -xh
    // (NaN: neither).  xh is found from fl(threshold * scale), within a few
    // ulps, by stepping with IEEE divisions (the same for every lane; each
    // quotient computed once, stepping stops at the bound).  If
    // that fails (an infinite scale or threshold, a NaN threshold), each
    // weight is divided instead, as w * (1 / scale) -- within 3 ulp of the
    // quotient -- with the IEEE division for values within 2^-20 (relative)
    // of +-threshold (below 2^-100 for a zero threshold).
    float xh = threshold * scale;
    float qx = xh / scale;
    for (int it = 0; it < 4 && qx > threshold; ++it) {
        xh = float_next(xh, false);
        qx = xh / scale;
    }
    float xn = float_next(xh, true), qn = xn / scale;
    for (int it = 0; it < 4 && qn <= threshold; ++it) {
        xh = xn;
        qx = qn;
        xn = float_next(xh, true);
        qn = xn / scale;
    }
    const bool bounds = __builtin_isfinite(xh) && qx <= threshold && !(qn <= threshold);
    const float rcp = 1.0f / scale;
    const float tt = fabsf(threshold);
    const float tol = fmaxf(tt * 0x1p-20f, 0x1p-100f);
    auto digit = [&](float x) -> uint32_t {
        if (bounds) return x > xh ? 2u : (x < -xh ? 0u : 1u);
        float nv = x * rcp;
        if (fabsf(fabsf(nv) - tt) <= tol) nv = x / scale;
        return nv > threshold ? 2u : (nv < -threshold ? 0u : 1u);
    };
    const uint32_t chunks = (k + 19) / 20;  // the last one partial when k % 20 != 0
    const uint32_t kp = (k + 4) / 5;
    uint8_t* pr = packed + row * kp;
    const bool word_stores = kp % 4 == 0 && (reinterpret_cast<uintptr_t>(packed) & 3u) == 0;
    f32x4* st = stage[wv];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        if ((uint32_t)(kWave * slice(c)) >= chunks) break;  // wave-uniform
#pragma unroll
        for (int q = 0; q < 5; ++q) st[64 * q + lane] = g[c][q];
        wave_lds_sync();
        f32x4 v[5];
#pragma unroll
        for (int q = 0; q < 5; ++q) v[q] = st[5 * lane + q];  // chunk 64 c + lane
        wave_lds_sync();
        const uint32_t ch = (uint32_t)lane + kWave * slice(c);
        if (ch < chunks) {
            uint32_t word = 0;
#pragma unroll
            for (int bq = 0; bq < 4; ++bq) {
                uint32_t val = 0, mul = 1;
#pragma unroll
                for (int j = 0; j < 5; ++j) {
                    const int f = 5 * bq + j;
                    val += (20u * ch + (uint32_t)f < k ? digit(v[f / 4][f % 4]) : 1u) * mul;  // zero trits past k
                    mul *= 3u;
                }
                word |= val << (8 * bq);
            }
            if (word_stores && 4u * ch + 4u <= kp) {
                reinterpret_cast<uint32_t*>(pr)[ch] = word;
            } else {
#pragma unroll
                for (int bq = 0; bq < 4; ++bq)
                    if (4u * ch + (uint32_t)bq < kp) pr[4u * ch + bq] = (uint8_t)(word >> (8 * bq));
            }
        }
    }
}

__global__ __launch_bounds__(kPackWaves * kWave) void ternary_pack_kernel(const float* __restrict__ w, uint64_t m,
                                                                          uint32_t k, uint32_t kp, float threshold,
                                                                          uint8_t* __restrict__ packed,
                                                                          float* __restrict__ scales) {
    const int lane = threadIdx.x & (kWave - 1);
    const uint64_t row = (uint64_t)blockIdx.x * kPackWaves + threadIdx.x / kWave;
    if (row >= m) return;  // whole waves; no barriers below
    const float* rd = w + row * k;
    float amax = 0.0f;
    for (uint32_t i = (uint32_t)lane; i < k; i += kWave) amax = fmaxf(amax, fabsf(rd[i]));
    amax = wave_max(amax);
    const float scale = amax < 1e-8f ? 1.0f : amax;
    if (lane == 0) scales[row] = scale;
    uint8_t* pr = packed + row * kp;
    for (uint32_t b = (uint32_t)lane; b < kp; b += kWave) {
        uint32_t val = 0, mul = 1;
#pragma unroll
        for (int j = 0; j < 5; ++j) {
            const uint32_t i = 5u * b + (uint32_t)j;
            val += (i < k ? trit_digit(rd[i], scale, threshold) : 1u) * mul;  // zero trits past k
            mul *= 3u;
        }
        pr[b] = (uint8_t)val;
    }
}

}  // namespace kore

namespace kore {
template <bool kSplit, bool kTrans>
static void launch_mfma_t(bool aligned_a, bool aligned_b, dim3 grid, hipStream_t s, const TernArgs& p) {
    if (aligned_a && aligned_b)
        hipLaunchKernelGGL((ternary_i8_mfma_kernel<true, true, kSplit, kTrans>), grid, dim3(kTmBlock), 0, s, p);
    else if (aligned_b)
        hipLaunchKernelGGL((ternary_i8_mfma_kernel<false, true, kSplit, kTrans>), grid, dim3(kTmBlock), 0, s, p);
    else if (aligned_a)
        hipLaunchKernelGGL((ternary_i8_mfma_kernel<true, false, kSplit, kTrans>), grid, dim3(kTmBlock), 0, s, p);
    else hipLaunchKernelGGL((ternary_i8_mfma_kernel<false, false, kSplit, kTrans>), grid, dim3(kTmBlock), 0, s, p);
}
template <bool kSplit>
static void launch_mfma(bool aligned_a, bool aligned_b, dim3 grid, hipStream_t s, const TernArgs& p) {
    if (p.trans) launch_mfma_t<kSplit, true>(aligned_a, aligned_b, grid, s, p);
    else launch_mfma_t<kSplit, false>(aligned_a, aligned_b, grid, s, p);
}
// Two-workgroups-per-CU path (the wide path's shapes): a workgroup owns a
// 256 (m) x 128 (n) output tile, wave w its weight rows [64 w, 64 w + 64)
// against the tile's 128 code rows: 2 x 4 MFMA tiles of 32 x 32 (128 int32
// accumulators per lane), 128 VGPRs + 128 AGPRs, so that each SIMD runs one
// wave of each of two workgroups.  A v_mfma_i32_32x32x32_i8 issues every 32
// cycles, but the vector and LDS instructions a wave issues between its own
// MFMAs (the trit decode, operand reads, code loads) delay its next one
// (measured: one wave per SIMD with three VALU and one LDS read per MFMA
// reaches 2.4 POP/s, two waves 3.2): with two waves per SIMD one wave's
// MFMAs cover the other's operand work, and one workgroup's epilogue the
// other's K loop.  Per 160-column K step a wave first decodes its two rows'
// 32 packed bytes into the step's A operands (the other wave on its SIMD
// runs MFMAs meanwhile), then runs 40 MFMAs with the code operands read one
// group ahead and the next step's code tile loaded into the other buffer by
// direct global -> LDS loads; one barrier per step.  The byte -> five-trit
// table is held in 16 copies (copy c for lanes c, c + 16, c + 32, c + 48).
// Code tile, K order, masking of trits past k, the alignment of packed rows
// and the output layouts as in the wide path.
constexpr int kW2N = 128;
constexpr int kW2NJ = kW2N / 32;
constexpr int kW2Copies = 16;
constexpr size_t kW2BBytes = (size_t)kW2N * kWdPitch;                      // one code tile
constexpr size_t kW2Loop = 2 * kW2BBytes + 256 * kW2Copies * 8;           // code tiles + table
constexpr int kW2EpPitch = kW2N + 8;                                      // epilogue slab pitch (floats)
constexpr size_t kW2Epi = (size_t)4 * 32 * kW2EpPitch * 4;
constexpr size_t kW2Lds = kW2Loop > kW2Epi ? kW2Loop : kW2Epi;
constexpr int kW2Slots = (int)(kW2BBytes / 16 / 4);                       // 16-byte code slots per wave
constexpr int kW2Dma = (kW2Slots + kWave - 1) / kWave;
constexpr uint64_t kW2MaxSteps = 16;  // K steps up to which it beats the wide path
static_assert(kW2Lds * 2 <= 160 * 1024, "two workgroups per CU");

template <bool kAlignedA, bool kTrans>
__global__ __launch_bounds__(256, 2) void ternary_i8_w2_kernel(TernArgs p) {
    constexpr int NJ = kW2NJ, kN = kW2N;
    constexpr size_t kBB = kW2BBytes;
    constexpr int kSl = kW2Slots, kDm = kW2Dma;
    extern __shared__ __attribute__((aligned(16))) uint8_t wlds[];
    uint64_t* lut = reinterpret_cast<uint64_t*>(wlds + 2 * kBB);
    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
    const int r = lane & 31, h = lane >> 5;
    // tile order as in the wide path (panels of n-tiles per XCD)
    const uint32_t tm_n = (p.m + kWdM - 1) / kWdM, tn_n = (p.n + kN - 1) / kN;
    const uint32_t ntiles = tm_n * tn_n;
    const uint32_t per = (ntiles + kXcds - 1) / kXcds;
    const uint32_t work = (blockIdx.x % kXcds) * per + blockIdx.x / kXcds;
    if (work >= ntiles) return;  // whole workgroup: no barrier reached yet
    const uint32_t pw = (tn_n + kXcds - 1) / kXcds;
    const uint32_t panel = work / (tm_n * pw), within = work % (tm_n * pw);
    const uint32_t pwid = min(pw, tn_n - panel * pw);
    const uint32_t m0 = (within / pwid) * kWdM, n0 = (panel * pw + within % pwid) * kN;

    // table: entry e, copy c at u64 index e * 16 + c, filled in a rotated order
    {
        const uint64_t v = trit_lut_entry((uint32_t)t);
#pragma unroll 4
        for (int c2 = 0; c2 < kW2Copies; ++c2) lut[t * kW2Copies + ((c2 + t) & (kW2Copies - 1))] = v;
    }
    const uint64_t* lut_lane = lut + (lane & (kW2Copies - 1));

    const uint32_t nkt = (p.k + kTmK - 1) / kTmK;
    const uint8_t* arow[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t m = min(m0 + 64 * wave + 32 * i + r, p.m - 1u);
        arow[i] = p.a + (uint64_t)m * p.kp;
    }
    const uintptr_t a_hi = reinterpret_cast<uintptr_t>(p.a) + (uintptr_t)p.m * p.kp;
    uint32_t sh[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) sh[i] = (uint32_t)(reinterpret_cast<uintptr_t>(arow[i]) & 3u);
    // this lane's 16 packed bytes of step kt per row (the 20 bytes from the
    // dword boundary below them for unaligned rows; byte by byte only where
    // they would pass the matrix's end)
    auto load_a = [&](uint32_t kt, u32x4 (&av)[2], uint32_t (&ae)[2]) {
        const uint32_t ab = kt * kTmKp + 16u * h;
        const uint32_t abc = ab < p.kp ? ab : 0u;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            if (kAlignedA) {
                av[i] = *reinterpret_cast<const u32x4*>(arow[i] + abc);
                continue;
            }
            const uintptr_t w0 = reinterpret_cast<uintptr_t>(arow[i] + abc) & ~(uintptr_t)3;
            if (__builtin_expect(w0 + 20u <= a_hi, 1)) {
                av[i] = *reinterpret_cast<const u32x4_a4*>(w0);
                ae[i] = *reinterpret_cast<const uint32_t*>(w0 + 16);
            } else {
                uint32_t w[5];
#pragma unroll
                for (int q = 0; q < 5; ++q) {
                    w[q] = 0;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uintptr_t o = w0 + 4 * q + e;
                        w[q] |= (o < a_hi ? (uint32_t)*reinterpret_cast<const uint8_t*>(o) : 0u) << (8 * e);
                    }
                }
                av[i] = u32x4{w[0], w[1], w[2], w[3]};
                ae[i] = w[4];
            }
        }
    };
    // code slots of this wave: slot s (16 bytes) of a tile is row s / 11,
    // piece s % 11 (piece 10: the row's padding, filled with piece 0)
    // (the piece's byte offset bp16 is recomputed where it is used: registers)
    uint32_t boff[kDm];
    auto bp16_of = [&](int g) {
        const int piece = (kSl * wave + kWave * g + lane) % 11;
        return piece < 10 ? 16u * (uint32_t)piece : 0u;
    };
#pragma unroll
    for (int g = 0; g < kDm; ++g) {
        const int slot = kSl * wave + kWave * g + lane;
        const uint32_t rowc = min(n0 + (uint32_t)(slot / 11), p.n - 1u);
        boff[g] = rowc * p.k + bp16_of(g);
    }
    const bool k_tail = p.k % kTmK != 0;
    auto dma_one = [&](uint32_t kt, uint32_t buf, int g) {
        const int8_t* base = p.q + (uint64_t)kt * kTmK;
        const uint32_t rem = p.k - kt * kTmK;
        uint8_t* dst = wlds + buf * kBB + (size_t)kSl * 16 * wave + kWave * 16 * g;
        uint32_t off = boff[g];
        if (k_tail) {
            const uint32_t b16 = bp16_of(g);
            if (b16 >= rem) off -= b16;
        }
        if (kSl % kWave == 0 || g < kDm - 1 || kWave * g + lane < kSl)
            __builtin_amdgcn_global_load_lds((glb_vptr)(base + off), (lds_vptr)dst, 16, 0, 0);
    };

    i32x16 acc[2][NJ];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[i][j][q] = 0;

    auto read_b = [&](uint32_t buf, int s, i32x4 (&bf)[NJ]) {
        const uint8_t* bb = wlds + buf * kBB + r * kWdPitch + 80 * h + 16 * s;
#pragma unroll
        for (int j = 0; j < NJ; ++j) bf[j] = *reinterpret_cast<const i32x4*>(bb + 32 * j * kWdPitch);
    };
    // step kt's A operands: its bytes decoded into five 32-deep MFMA steps
    // (lane half h: columns 80 h .. 80 h + 79), trits past k zeroed
    auto decode = [&](uint32_t kt, const u32x4 (&avr)[2], const uint32_t (&aer)[2], uint32_t (&dec)[2][20]) {
        u32x4 av[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            if (kAlignedA) {
                av[i] = avr[i];
            } else {
                av[i] = u32x4{__builtin_amdgcn_alignbyte(avr[i][1], avr[i][0], sh[i]),
                              __builtin_amdgcn_alignbyte(avr[i][2], avr[i][1], sh[i]),
                              __builtin_amdgcn_alignbyte(avr[i][3], avr[i][2], sh[i]),
                              __builtin_amdgcn_alignbyte(aer[i], avr[i][3], sh[i])};
            }
        }
        // eight table reads in flight at a time (registers: two waves per SIMD)
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
            for (int d = 0; d < 20; ++d) dec[i][d] = 0;
#pragma unroll
            for (int b0 = 0; b0 < 16; b0 += 8) {
                uint64_t tv[8];
#pragma unroll
                for (int b = 0; b < 8; ++b) {
                    const uint32_t byte = (av[i][(b0 + b) >> 2] >> (8 * ((b0 + b) & 3))) & 0xffu;
                    tv[b] = lut_lane[byte * kW2Copies];
                }
#pragma unroll
                for (int b = 0; b < 8; ++b) splice_trits(dec[i], b0 + b, tv[b]);
            }
        }
        if (k_tail && kt + 1 == nkt) {
            const int rem = (int)p.k - (int)(kt * kTmK) - 80 * h;
#pragma unroll
            for (int d = 0; d < 20; ++d) {
                const int keep = rem - 4 * d;
                const uint32_t msk = keep >= 4 ? 0xffffffffu : (keep <= 0 ? 0u : (0xffffffffu >> (8 * (4 - keep))));
#pragma unroll
                for (int i = 0; i < 2; ++i) dec[i][d] &= msk;
            }
        }
    };
    // the next step's code loads spread over MFMA groups 0 .. 2 (2 + 2 + 2)
    constexpr int kDmaAt[6] = {0, (kDm + 2) / 3, 2 * ((kDm + 2) / 3), kDm, kDm, kDm};
    // (the code operands are read at the start of their group, not a group
    // ahead: registers; the other wave on the SIMD covers the wait)
    auto mgroup = [&](auto S_, uint32_t kt, const uint32_t (&cur)[2][20]) {
        constexpr int s = decltype(S_)::value;
        constexpr int dlo = kDmaAt[s], dhi = kDmaAt[s + 1];
        i32x4 bc[NJ];
        read_b(kt & 1u, s, bc);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const i32x4 af = {(int)cur[i][4 * s], (int)cur[i][4 * s + 1], (int)cur[i][4 * s + 2],
                              (int)cur[i][4 * s + 3]};
#pragma unroll
            for (int j = 0; j < NJ; ++j) acc[i][j] = mfma_wq<kTrans>(af, bc[j], acc[i][j]);
        }
        if (kt + 1 < nkt) {
#pragma unroll
            for (int g = dlo; g < dhi; ++g) dma_one(kt + 1, (kt + 1) & 1u, g);
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    using S3 = std::integral_constant<int, 3>;
    using S4 = std::integral_constant<int, 4>;
    uint32_t cur[2][20];
    auto kstep = [&](uint32_t kt, u32x4 (&av)[2], uint32_t (&ae)[2]) {
        decode(kt, av, ae, cur);
        if (kt + 2 < nkt) load_a(kt + 2, av, ae);
        mgroup(S0(), kt, cur);
        mgroup(S1(), kt, cur);
        mgroup(S2(), kt, cur);
        mgroup(S3(), kt, cur);
        mgroup(S4(), kt, cur);
        // this wave's code loads for step kt + 1 have landed and every wave
        // is done reading buffer kt & 1 before anyone passes the barrier
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    };

    u32x4 ava[2], avb[2];
    uint32_t aea[2] = {0u, 0u}, aeb[2] = {0u, 0u};
    load_a(0, ava, aea);
    if (nkt > 1) load_a(1, avb, aeb);
#pragma unroll
    for (int g = 0; g < kDm; ++g) dma_one(0, 0, g);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // table filled, first code tile staged
    uint32_t kt = 0;
    for (; kt + 1 < nkt; kt += 2) {
        kstep(kt, ava, aea);
        kstep(kt + 1, avb, aeb);
    }
    if (kt < nkt) kstep(kt, ava, aea);

    // Epilogue as in the wide path: ((float)acc * sa[m]) * sq[n] (+ bias[m])
    // through per-wave LDS slabs, whole output rows per store instruction.
    if constexpr (kTrans) {
        constexpr int kTp = 72;
        float* slab = reinterpret_cast<float*>(wlds) + wave * 32 * kTp;
        float* sqs = reinterpret_cast<float*>(wlds) + 4 * 32 * kTp;
        if (t < kN) sqs[t] = p.sq[min(n0 + (uint32_t)t, p.n - 1u)];
        __syncthreads();
        const uint32_t mw = m0 + 64 * wave;
        float sam[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) sam[i] = p.sa[min(mw + 32 * i + r, p.m - 1u)];
        const uint32_t mc = mw + 4 * (lane & 15);
        const bool vec_out = (p.m & 3u) == 0 && (reinterpret_cast<uintptr_t>(p.c) & 15u) == 0;
        f32x4 bias4 = {0.f, 0.f, 0.f, 0.f};
        if (p.bias) {
#pragma unroll
            for (int u = 0; u < 4; ++u) bias4[u] = p.bias[min(mc + u, p.m - 1u)];
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int row = 8 * (q >> 2) + 4 * h + (q & 3);
#pragma unroll
                for (int i = 0; i < 2; ++i) slab[row * kTp + 32 * i + r] = (float)acc[i][j][q] * sam[i];
            }
            wave_lds_sync();
#pragma unroll
            for (int it = 0; it < 8; ++it) {
                const int row = 4 * it + (lane >> 4);
                const uint32_t n = n0 + 32 * j + row;
                if (n >= p.n) continue;
                const float sqn = sqs[32 * j + row];
                f32x4 v = *reinterpret_cast<const f32x4*>(slab + row * kTp + 4 * (lane & 15));
                v = v * sqn;
                if (p.bias) v = v + bias4;
                float* crow = p.c + (uint64_t)n * p.m;
                if (vec_out && mc + 3 < p.m) {
                    __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(crow + mc));
                } else {
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        if (mc + u < p.m) crow[mc + u] = v[u];
                }
            }
            wave_lds_sync();  // the slab is rewritten for the next j
        }
        return;
    }
    float sqn[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) sqn[j] = p.sq[min(n0 + 32 * j + r, p.n - 1u)];
    float* slab = reinterpret_cast<float*>(wlds) + wave * 32 * kW2EpPitch;
    const bool vec_out = (p.n & 3u) == 0 && (reinterpret_cast<uintptr_t>(p.c) & 15u) == 0;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t mb = m0 + 64 * wave + 32 * i;
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const int row = 8 * (q >> 2) + 4 * h + (q & 3);
            const float sam = p.sa[min(mb + row, p.m - 1u)];
#pragma unroll
            for (int j = 0; j < NJ; ++j) slab[row * kW2EpPitch + 32 * j + r] = ((float)acc[i][j][q] * sam) * sqn[j];
        }
        wave_lds_sync();
        // 32 lanes cover a 128-float row: two rows per store instruction
        for (int rb = 0; rb < 32; rb += 2) {
            const int row = rb + (lane >> 5), col = 4 * (lane & 31);
            const uint32_t m = mb + row;
            if (m >= p.m) continue;
            f32x4 v = *reinterpret_cast<const f32x4*>(slab + row * kW2EpPitch + col);
            if (p.bias) v = v + p.bias[m];
            float* crow = p.c + (uint64_t)m * p.n;
            const uint32_t nc = n0 + col;
            if (vec_out && nc + 3 < p.n) {
                __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(crow + nc));
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (nc + u < p.n) crow[nc + u] = v[u];
            }
        }
        wave_lds_sync();
    }
}

template <bool kTrans>
static void launch_w2_t(bool aligned_a, dim3 g, hipStream_t s, const TernArgs& p) {
    if (aligned_a) hipLaunchKernelGGL((ternary_i8_w2_kernel<true, kTrans>), g, dim3(256), kW2Lds, s, p);
    else hipLaunchKernelGGL((ternary_i8_w2_kernel<false, kTrans>), g, dim3(256), kW2Lds, s, p);
}

template <int NJ, bool kTrans>
static void launch_wide_t(bool aligned_a, dim3 g, hipStream_t s, const TernArgs& p) {
    if (aligned_a)
        hipLaunchKernelGGL((ternary_i8_wide_kernel<true, NJ, kTrans>), g, dim3(256), WideTile<NJ>::kLds, s, p);
    else hipLaunchKernelGGL((ternary_i8_wide_kernel<false, NJ, kTrans>), g, dim3(256), WideTile<NJ>::kLds, s, p);
}
template <int NJ>
static void launch_wide(bool aligned_a, dim3 g, hipStream_t s, const TernArgs& p) {
    if (p.trans) launch_wide_t<NJ, true>(aligned_a, g, s, p);
    else launch_wide_t<NJ, false>(aligned_a, g, s, p);
}
}  // namespace kore

using namespace kore;

// The int8 matmul with the output in either layout (trans: c[n, m]) and an
// optional bias per weight row.
static int ternary_i8_run(const uint8_t* a_packed, const float* a_scales, const int8_t* q, const float* q_scales,
                          const float* bias, float* c, uint64_t m, uint64_t n, uint64_t k, bool trans,
                          hipStream_t s) {
    if (m == 0 || n == 0) return KORE_HIP_OK;
    if (!c || !a_scales || !q_scales) return KORE_HIP_ERR_NULL_PTR;
    if (k > 0 && (!a_packed || !q)) return KORE_HIP_ERR_NULL_PTR;
    // |sum| <= 127 * k must stay exact in int32 and every index in 32 bits.
    if (m > 0x7fffffffull || n > 0x7fffffffull || k > (1ull << 24)) return KORE_HIP_ERR_OVERFLOW;
    uint64_t mn, nk;
    if (!mul_ok(m, n, &mn) || mn > kMaxElements || !mul_ok(n, k, &nk) || nk > kMaxElements)
        return KORE_HIP_ERR_OVERFLOW;
    const uint64_t kp = (k + 4) / 5;
    // c is written (and, with split-K, zeroed first) while the inputs are
    // read: it must not overlap any of them.
    {
        const char* c0 = reinterpret_cast<const char*>(c);
        const char* c1 = c0 + mn * sizeof(float);
        const struct { const void* p; uint64_t bytes; } ins[] = {
            {a_packed, m * kp}, {q, nk}, {a_scales, m * sizeof(float)}, {q_scales, n * sizeof(float)},
            {bias, bias ? m * sizeof(float) : 0u}};
        for (const auto& in : ins) {
            const char* i0 = reinterpret_cast<const char*>(in.p);
            if (in.p && in.bytes && i0 < c1 && c0 < i0 + in.bytes) return KORE_HIP_ERR_ALIAS;
        }
    }
    TernArgs p{a_packed, a_scales, q,  q_scales, c, (uint32_t)m, (uint32_t)n, (uint32_t)k, (uint32_t)kp, 1u, 0u,
               bias,     trans ? 1u : 0u};
    const bool c_ok = (reinterpret_cast<uintptr_t>(c) & 3u) == 0;
    if (n <= kGvMaxN && k > 0 && k % 8 == 0 && (reinterpret_cast<uintptr_t>(q) & 7u) == 0 && c_ok) {
        // grid: at most m / 4 blocks of one wave group (m < 2^31)
        const bool al8 = kp % 8 == 0 && (reinterpret_cast<uintptr_t>(a_packed) & 7u) == 0;
        if (al8) {
            if (n <= 1) launch_gemv<1, true>(p, m, k, s);
            else if (n <= 2) launch_gemv<2, true>(p, m, k, s);
            else launch_gemv<4, true>(p, m, k, s);
        } else {
            if (n <= 1) launch_gemv<1, false>(p, m, k, s);
            else if (n <= 2) launch_gemv<2, false>(p, m, k, s);
            else launch_gemv<4, false>(p, m, k, s);
        }
        return launch_status();
    }
    const bool vec = k > 0 && k % 16 == 0 && aligned16(q) && c_ok;
    if (vec && n <= kSkMaxN) {
        const uint64_t blocks = (m + kSkRows - 1) / kSkRows;
        if (blocks > 0x7fffffffull) return KORE_HIP_ERR_OVERFLOW;
        const bool al = kp % 16 == 0 && aligned16(a_packed);
        const dim3 g((uint32_t)blocks);
        const int nt = (int)((n + 31) / 32);
#define KORE_SKINNY(NT, AL, TR) hipLaunchKernelGGL((ternary_i8_skinny_kernel<NT, AL, 8, TR>), g, dim3(8 * kWave), 0, s, p)
        if (trans) {
            if (al) { if (nt == 1) KORE_SKINNY(1, true, true); else KORE_SKINNY(2, true, true); }
            else { if (nt == 1) KORE_SKINNY(1, false, true); else KORE_SKINNY(2, false, true); }
        } else {
            if (al) { if (nt == 1) KORE_SKINNY(1, true, false); else KORE_SKINNY(2, true, false); }
            else { if (nt == 1) KORE_SKINNY(1, false, false); else KORE_SKINNY(2, false, false); }
        }
#undef KORE_SKINNY
        return launch_status();
    }
    const uint64_t wide_tiles = ((m + kWdM - 1) / kWdM) * ((n + kWdN - 1) / kWdN);
    if (vec && wide_tiles >= kWdMinTiles && nk < (1ull << 31)) {
        // Many output tiles: the wide kernel (one 256 x 256 tile per CU), or
        // 256 x 192 tiles where the rounds of 256 CUs they need, at ~0.8 of a
        // 256 x 256 tile's time each, are fewer.
        const uint64_t t192 = ((m + kWdM - 1) / kWdM) * ((n + 191) / 192);
        const uint64_t r192 = (t192 + kCus - 1) / kCus, r256 = (wide_tiles + kCus - 1) / kCus;
        // (measured: 2560 x 8192 x 6912 215 -> 182 us, 2560 x 4096 x 6912 113 ->
        // 103; with few K steps the narrower tile loses: 2600 x 4000 x 336
        // 20.1 -> 22.3)
        const bool n192 = 4 * r192 < 5 * r256 && (k + kTmK - 1) / kTmK >= 8;  // 0.8 r192 < r256
        const uint64_t tiles = n192 ? t192 : wide_tiles;
        const uint64_t per = (tiles + kXcds - 1) / kXcds;
        if (per * kXcds > 0x7fffffffull) return KORE_HIP_ERR_OVERFLOW;
        const dim3 g((uint32_t)(per * kXcds));
        const bool al = kp % 16 == 0 && aligned16(a_packed);
        // Few K steps on 256 x 256 tiles: 256 x 128 tiles, two workgroups per
        // CU, so one workgroup's epilogue (an HBM write burst of a whole tile)
        // and its first K step overlap the other's matrix-core work.
        // (measured: 6912 x 4096 x 2560 106 -> 92 us, 8192 x 8192 x 2560 203
        // -> 177, 6912 x 4096 x 640 44.7 -> 35.4; at 26 K steps no gain:
        // 4096 x 4096 x 4096 74.5 -> 76.5; on 192-wide tiles a loss:
        // 2560 x 4096 x 6912 92 -> 105)
        if (!n192 && (k + kTmK - 1) / kTmK <= kW2MaxSteps) {
            const uint64_t per2 = (((m + kWdM - 1) / kWdM) * ((n + kW2N - 1) / kW2N) + kXcds - 1) / kXcds;
            if (per2 * kXcds > 0x7fffffffull) return KORE_HIP_ERR_OVERFLOW;
            const dim3 g2((uint32_t)(per2 * kXcds));
            if (p.trans) launch_w2_t<true>(al, g2, s, p);
            else launch_w2_t<false>(al, g2, s, p);
            return launch_status();
        }
        if (n192) launch_wide<6>(al, g, s, p);
        else launch_wide<8>(al, g, s, p);
        return launch_status();
    }
    if (k > 0 && c_ok) {
        // codes 16-byte aligned row by row (vec) or not
        const uint64_t tiles = ((m + kTmM - 1) / kTmM) * ((n + kTmN - 1) / kTmN);
        const uint64_t nkt = (k + kTmK - 1) / kTmK;
        // Few output tiles (small m * n): split K so that ~512 workgroups run,
        // each over at least two K-tiles.
        uint64_t splits = 1;
        if (tiles < 128 && nkt >= 4) {
            splits = std::min<uint64_t>(nkt / 2, (512 + tiles - 1) / tiles);
            const uint64_t kt_per = (nkt + splits - 1) / splits;
            splits = (nkt + kt_per - 1) / kt_per;
            p.splits = (uint32_t)splits;
            p.kt_per = (uint32_t)kt_per;
        }
        const uint64_t work = tiles * splits;
        const uint64_t per = (work + kXcds - 1) / kXcds;
        if (per * kXcds > 0x7fffffffull) return KORE_HIP_ERR_OVERFLOW;
        const dim3 grid((uint32_t)(per * kXcds));
        const bool al = kp % 16 == 0 && aligned16(a_packed);
        if (splits > 1) {
            const dim3 eg((uint32_t)((mn + kTmBlock - 1) / kTmBlock));
            hipLaunchKernelGGL(ternary_i8_zero_kernel, eg, dim3(kTmBlock), 0, s, reinterpret_cast<int32_t*>(c), mn);
            launch_mfma<true>(al, vec, grid, s, p);
            hipLaunchKernelGGL(ternary_i8_finish_kernel, eg, dim3(kTmBlock), 0, s, p);
        } else {
            launch_mfma<false>(al, vec, grid, s, p);
        }
    } else {
        const uint64_t blocks = (mn + kTmBlock - 1) / kTmBlock;
        if (blocks > 0x7fffffffull) return KORE_HIP_ERR_OVERFLOW;
        hipLaunchKernelGGL(ternary_i8_generic_kernel, dim3((uint32_t)blocks), dim3(kTmBlock), 0, s, p);
    }
    return launch_status();
}

extern "C" int kore_hip_ternary_matmul_i8(const uint8_t* a_packed, const float* a_scales, const int8_t* q,
                                          const float* q_scales, float* c, uint64_t m, uint64_t n, uint64_t k,
                                          kore_stream_t stream) {
    return ternary_i8_run(a_packed, a_scales, q, q_scales, nullptr, c, m, n, k, false, (hipStream_t)stream);
}

extern "C" int kore_hip_bit_linear_i8(const uint8_t* a_packed, const float* a_scales, const int8_t* q,
                                      const float* q_scales, const float* bias, float* y, uint64_t out_features,
                                      uint64_t batch, uint64_t in_features, kore_stream_t stream) {
    return ternary_i8_run(a_packed, a_scales, q, q_scales, bias, y, out_features, batch, in_features, true,
                          (hipStream_t)stream);
}

// The f32-activation matmul with b either [K, N] or token-major [N, K]
// (tm), the output in either layout (trans: c[n, m]) and an optional bias.
static int ternary_f32_run(const uint8_t* a_packed, const float* a_scales, const float* b, const float* bias,
                           float* c, uint64_t m, uint64_t n, uint64_t k, bool tm, bool trans, hipStream_t s) {
    if (m == 0 || n == 0) return KORE_HIP_OK;
    if (!c || !a_scales) return KORE_HIP_ERR_NULL_PTR;
    if (k > 0 && (!a_packed || !b)) return KORE_HIP_ERR_NULL_PTR;
    if (m > 0x7fffffffull || n > 0x7fffffffull || k > 0x7fffffffull) return KORE_HIP_ERR_OVERFLOW;
    uint64_t mn, kn;
    if (!mul_ok(m, n, &mn) || mn > kMaxElements || !mul_ok(k, n, &kn) || kn > kMaxElements)
        return KORE_HIP_ERR_OVERFLOW;
    const uint64_t kp = (k + 4) / 5;
    uint64_t mkp;
    if (!mul_ok(m, kp, &mkp) || mkp > kMaxElements) return KORE_HIP_ERR_OVERFLOW;
    {
        const char* c0 = reinterpret_cast<const char*>(c);
        const char* c1 = c0 + mn * sizeof(float);
        const struct { const void* p; uint64_t bytes; } ins[] = {
            {a_packed, mkp}, {b, kn * sizeof(float)}, {a_scales, m * sizeof(float)},
            {bias, bias ? m * sizeof(float) : 0u}};
        for (const auto& in : ins) {
            const char* i0 = reinterpret_cast<const char*>(in.p);
            if (in.p && in.bytes && i0 < c1 && c0 < i0 + in.bytes) return KORE_HIP_ERR_ALIAS;
        }
    }
    // token-major b: the rows kernel's buffer offsets (column x K x 4 bytes
    // within a 64-column tile) stay below 2^31
    if (tm && k > (1ull << 23)) return KORE_HIP_ERR_OVERFLOW;
    TernF32Args p{a_packed, a_scales, b, c, (uint32_t)m, (uint32_t)n, (uint32_t)k, (uint32_t)kp,
                  tm ? 1u : n, tm ? k : 1u, bias, trans ? 1u : 0u, m};
    int ct = 64;
    while (ct > 1 && (uint64_t)(ct / 2) >= n) ct /= 2;  // smallest power of two >= n (<= 64)
    // Five columns and more: the row-broadcast kernel (any row alignment) in
    // 16-, 32- or 64-column tiles, over row ranges of less than 2 GiB of
    // packed weights each (its buffer offsets are 31-bit).
    if (n >= kRowsMinCols) {
        const uint64_t span = kp ? std::min<uint64_t>(m, 0x7fffffffull / kp) : m;  // rows per launch
        for (uint64_t r0 = 0; r0 < m; r0 += span) {
            TernF32Args q = p;
            q.a += r0 * kp;
            q.sa += r0;
            q.m = (uint32_t)std::min<uint64_t>(span, m - r0);
            q.c += trans ? r0 : r0 * n;  // c[n, m]: columns r0 .. of every row, row stride m
            if (bias) q.bias += r0;
            if (f32_use_mf4(q.m, n, k, kp, tm)) {
                const int st = tm ? launch_f32_mf4<true>(q.m, n, s, q) : launch_f32_mf4<false>(q.m, n, s, q);
                if (st != KORE_HIP_OK) return st;
                continue;
            }
            if (f32_use_mfma(q.m, n, k)) {
                const int st = tm ? launch_f32_mfma<true>(q.m, n, s, q) : launch_f32_mfma<false>(q.m, n, s, q);
                if (st != KORE_HIP_OK) return st;
                continue;
            }
            const int st = tm ? (ct <= 16 ? launch_f32_rows<16, true>(q.m, n, s, q)
                                 : ct == 32 ? launch_f32_rows<32, true>(q.m, n, s, q)
                                            : launch_f32_rows<64, true>(q.m, n, s, q))
                              : (ct <= 16 ? launch_f32_rows<16, false>(q.m, n, s, q)
                                 : ct == 32 ? launch_f32_rows<32, false>(q.m, n, s, q)
                                            : launch_f32_rows<64, false>(q.m, n, s, q));
            if (st != KORE_HIP_OK) return st;
        }
        return KORE_HIP_OK;
    }
    // One to four columns: the fold-wave kernel; the per-lane kernel for K = 0
    // and for matrices of fewer than 20 packed bytes (the fold-wave kernel's
    // 8-byte windows).
    if (k > 0 && mkp >= 20) {
        const dim3 gp((uint32_t)((m + kWave - 1) / kWave));
        if (n == 1) hipLaunchKernelGGL(ternary_f32_pipe_kernel<1>, gp, dim3((kPfDec + 1) * kWave), 0, s, p);
        else if (n == 2) hipLaunchKernelGGL(ternary_f32_pipe_kernel<2>, gp, dim3((kPfDec + 2) * kWave), 0, s, p);
        else hipLaunchKernelGGL(ternary_f32_pipe_kernel<4>, gp, dim3((kPfDec + 4) * kWave), 0, s, p);
        return launch_status();
    }
    const dim3 g((uint32_t)((m + 4 * (kWave / ct) - 1) / (4 * (kWave / ct))));  // 4 waves of 64 / ct rows
    if (kp % 16 == 0 && aligned16(a_packed)) launch_f32_seq<true>(ct, g, s, p);
    else launch_f32_seq<false>(ct, g, s, p);
    return launch_status();
}

extern "C" int kore_hip_ternary_matmul_f32(const uint8_t* a_packed, const float* a_scales, const float* b, float* c,
                                           uint64_t m, uint64_t n, uint64_t k, kore_stream_t stream) {
    return ternary_f32_run(a_packed, a_scales, b, nullptr, c, m, n, k, false, false, (hipStream_t)stream);
}

extern "C" int kore_hip_bit_linear_f32(const uint8_t* a_packed, const float* a_scales, const float* x,
                                       const float* bias, float* y, uint64_t out_features, uint64_t batch,
                                       uint64_t in_features, kore_stream_t stream) {
    return ternary_f32_run(a_packed, a_scales, x, bias, y, out_features, batch, in_features, true, true,
                           (hipStream_t)stream);
}

extern "C" int kore_hip_pack_weights_ternary(const float* w, uint64_t m, uint64_t k, float threshold,
                                             uint8_t* packed, float* scales, kore_stream_t stream) {
    if (m == 0) return KORE_HIP_OK;
    if (!scales || (k > 0 && (!w || !packed))) return KORE_HIP_ERR_NULL_PTR;
    uint64_t mk;
    if (k > 0xffffffffull - 4 || !mul_ok(m, k, &mk) || mk > kMaxElements) return KORE_HIP_ERR_OVERFLOW;
    const uint64_t kp = (k + 4) / 5;
    // the outputs are written while w is read: no overlap
    {
        const char* w0 = reinterpret_cast<const char*>(w);
        const char* w1 = w0 + mk * sizeof(float);
        const struct { const void* p; uint64_t bytes; } outs[] = {{packed, m * kp}, {scales, m * sizeof(float)}};
        for (const auto& o : outs) {
            const char* o0 = reinterpret_cast<const char*>(o.p);
            if (w && mk && o.p && o.bytes && o0 < w1 && w0 < o0 + o.bytes) return KORE_HIP_ERR_ALIAS;
        }
    }
    const uint64_t blocks = (m + kPackWaves - 1) / kPackWaves;
    if (blocks > 0x7fffffffull) return KORE_HIP_ERR_OVERFLOW;
    const dim3 g((uint32_t)blocks), blk(kPackWaves * kWave);
    hipStream_t s = (hipStream_t)stream;
    const uint64_t slices = ((k + 19) / 20 + kWave - 1) / kWave;  // 64-chunk slices of 20 floats per row
    // Two slices: a workgroup of two waves per row, one slice each (measured
    // 6912 x 2560 15.65 -> 15.17 us against one wave per row); one slice: a
    // wave per row.
    if (k > 0 && k % 4 == 0 && aligned16(w) && slices == 2 && m <= 0x7fffffffull) {
        hipLaunchKernelGGL((ternary_pack_vec_kernel<1, true, 2>), dim3((uint32_t)m), dim3(2 * kWave), 0, s, w, m,
                           (uint32_t)k, threshold, packed, scales);
        return launch_status();
    }
    if (k > 0 && k % 4 == 0 && aligned16(w) && slices <= 2) {
        if (slices <= 1) hipLaunchKernelGGL((ternary_pack_vec_kernel<1, false>), g, blk, 0, s, w, m, (uint32_t)k, threshold, packed, scales);
        else hipLaunchKernelGGL((ternary_pack_vec_kernel<2, false>), g, blk, 0, s, w, m, (uint32_t)k, threshold, packed, scales);
    } else if (k > 0 && k % 4 == 0 && aligned16(w) && slices <= 8 * kPackWaves) {
        // long rows: a workgroup per row (m < 2^31 blocks)
        if (m > 0x7fffffffull) return KORE_HIP_ERR_OVERFLOW;
        const dim3 gr((uint32_t)m);
        const uint64_t per_wave = (slices + kPackWaves - 1) / kPackWaves;
        if (per_wave <= 1) hipLaunchKernelGGL((ternary_pack_vec_kernel<1, true>), gr, blk, 0, s, w, m, (uint32_t)k, threshold, packed, scales);
        else if (per_wave <= 2) hipLaunchKernelGGL((ternary_pack_vec_kernel<2, true>), gr, blk, 0, s, w, m, (uint32_t)k, threshold, packed, scales);
        else if (per_wave <= 4) hipLaunchKernelGGL((ternary_pack_vec_kernel<4, true>), gr, blk, 0, s, w, m, (uint32_t)k, threshold, packed, scales);
        else hipLaunchKernelGGL((ternary_pack_vec_kernel<8, true>), gr, blk, 0, s, w, m, (uint32_t)k, threshold, packed, scales);
    } else {
        hipLaunchKernelGGL(ternary_pack_kernel, g, blk, 0, s, w, m, (uint32_t)k, (uint32_t)kp, threshold, packed,
                           scales);
    }
    return launch_status();
}
