// norm.hip -- RMSNorm (f32 out) and the BitLinear pre-quant (RMSNorm + per-row
// absmax int8), bit-exact against the reference CPU path.
//
// Roofline: HBM.  Bytes per row: cols*4 read, plus cols*4 written (RMSNorm)
// or cols + 4 written (pre-quant); the weight vector stays in L2.
//
// The reference sums x^2 with a left-to-right f32 fold
// (crates/kore-kernels/src/cpu_fused.rs:180).  A tree sum lands a few ulps
// away, which moves inv_rms and flips int8 codes on rounding boundaries, so
// the fold must be reproduced exactly.  A plain sequential walk costs one
// dependent add (~8 cycles on gfx950) per element -- ~8.5 us for a 2560-wide
// row, longer than the whole HBM budget of the pre-quant config.  The engine
// below computes the same bits with a *segmented exact fold*:
//
//   Row split into 64 contiguous segments, segment j owned by lane j.
//   phase 0  every lane sums its segment (any order) and a wave scan turns the
//            sums into an estimate of the running sum at its segment start;
//   phase 1  the estimate names a binade E = [2^E, 2^(E+1)) (grid g = 2^(E-23));
//            the lane folds its segment twice, from sigma_0 = 2^E and
//            sigma_1 = 2^E + g (E = -126: from 0 and 2^-149), giving increments
//            d_p = w_p - sigma_p (NaN if the walk left the binade);
//   resolve  walk the segments in order with the exact running sum s: if s is
//            in the segment's binade, p = lsb(s), and t = s + d_p < 2^(E+1),
//            the segment's true end is t; otherwise fold it sequentially from
//            s.
// Exactness: inside one binade s -> RN(s + a) commutes with a shift of s by
// an even number of ulps (round-half-even only looks at the last bit), so the
// walk from s is the walk from sigma_p shifted by s - sigma_p, as long as it
// stays below 2^(E+1) -- which t < 2^(E+1) certifies.  Lane 0 folds from the
// true start 0, so its result is exact with no condition.  The estimate only
// decides how often the resolve falls back (binade crossings: ~log2(sum)
// segments per row); it never affects a bit of the result.  The algorithm is
// checked against the plain fold on adversarial rows by the CPU test suite
// (tests/csrc/check_segmented_fold.c restates this kernel in scalar C).
//
// Data movement per wave (one row per wave, four waves per workgroup):
//   * the row is loaded with wave-wide global_load_dwordx4 (coalesced, 1 KiB
//     per instruction), all in flight before first use, and kept in VGPRs
//     for the epilogue: one HBM read per byte;
//   * its squares pass through a wave-private LDS tile (half a row at a time)
//     to put segment j into lane 63 - j (odd float4 pitch: conflict-free
//     ds_read_b128);
//   * runs of segments in one binade are composed by a segmented DPP scan
//     (the parity automaton over integer increments), so each lane holds
//     its segment's run entry (increments for both entry parities, binade,
//     next segment) and its squares in registers;
//   * the resolve runs on the scalar unit in integers: inside one binade the
//     float bits are linear in the value, so a run's exact increment is an
//     integer added to the bits of the running sum, and the binade window
//     checks are unsigned compares.  It reads entry j from lane 63 - j with
//     v_readlane, jumps whole runs, and when a segment falls back the owning
//     lane's fold of its own registers is broadcast.  No LDS, no re-read of
//     global memory.
// A wave's LDS traffic never crosses waves, so there are no barriers: LDS
// operations from one wave complete in issue order.

// Epilogue (element-parallel over all 64 lanes, coalesced layout):
//   inv  = 1 / sqrt(ss / cols + eps)   IEEE sqrt and division (cpu_fused.rs:181-182)
//   xn   = (x * inv) * w                                      (cpu_fused.rs:185)
// Pre-quant additionally:
//   amax = max |xn| (wave max: order-free, exact, NaN dropped); 1.0 if
//          amax < 1e-8 (kore-btes/src/quantize.rs:10)
//   code = clamp(round_half_away((xn * 127) / amax), -128, 127), the
//          quotient correctly rounded.  For rows with amax < 2^120 each code
//          comes from one fma and one floor conversion, with a bracket test
//          that sends the rare undecided element (and any NaN) to the exact
//          Markstein quotient (quant_code); other rows take the exact path
//          throughout.  Both are checked on the CPU by the test suite.
#include "common.hpp"
#include "kore_hip_internal.hpp"

namespace kore {

constexpr int kWavesPerBlock = 4;
constexpr int kSegs = kWave;  // segments per row: one per lane

// F32: y = RMSNorm(x); I8: pre-quant codes + scales; SiluGate: y = RMSNorm(x)
// * silu(z) (the Mamba input-path gate).
enum class NormOut { F32, I8, SiluGate };

struct NormArgs {
    const float* x;
    const float* w;
    float* y;        // NormOut::F32
    int8_t* q;       // NormOut::I8
    float* scale;    // NormOut::I8
    const float* z;  // NormOut::SiluGate
    uint64_t rows;
    uint32_t cols;
    float eps;
};

// Transpose tile geometry.  Segment j (SL4 consecutive float4 of the row)
// starts at float4 j*P of the tile, with an odd pitch P: 16 lanes reading
// float4 k of 16 consecutive segments then hit 16 distinct 16-byte bank
// groups.  For even SL4 with four waves per workgroup the tile holds half a
// row (32 segments = SL4/2 whole load chunks) and is filled in two passes;
// odd SL4, and one wave per workgroup (launches of few rows, where LDS is
// plentiful and the second pass's round trip is on the row's chain), take
// one pass.
__host__ __device__ constexpr int seg_pitch4(int sl4) { return (sl4 & 1) ? sl4 : sl4 + 1; }
__host__ __device__ constexpr int tile_segs(int sl4, int wpb) { return (sl4 & 1) || wpb == 1 ? kSegs : kSegs / 2; }
__host__ __device__ constexpr uint32_t wave_lds_f4(int sl4, int wpb) {
    return (uint32_t)(tile_segs(sl4, wpb) * seg_pitch4(sl4));
}


__device__ __forceinline__ int32_t cvt_i32_sat(float v) {
    // v_cvt_i32_f32: round toward zero, saturating, NaN -> 0.  Written as asm
    // because a C++ float->int cast of NaN is undefined.
    int32_t r;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(v));
    return r;
}

// Code of one normalised value xn of a row with absmax amax (>= every |xn|
// of the row, or 1.0 when the row's absmax is below 1e-8), exactly as the
// reference computes clamp(round((xn * 127) / amax), -128, 127) as i8:
// t is the IEEE quotient (Markstein: with y = RN(1/amax), q0 = RN(a*y),
// r = fma(-amax, q0, a), t = fma(r, y, q0) is RN(a/amax) -- checked on the
// CPU by the test suite), rounded half away from zero.  An infinite
// numerator (|xn| * 127 above FLT_MAX) over a finite amax gives an infinite
// quotient, which saturates; NaN (NaN inputs, or a NaN quotient from an
// infinite amax) converts to 0.
__device__ __forceinline__ int32_t quant_code(float xn, float amax, float rcp_amax) {
    float a = xn * 127.0f;
    float q0 = a * rcp_amax;
    float r = __builtin_fmaf(-amax, q0, a);
    float t = __builtin_fmaf(r, rcp_amax, q0);
    if (__builtin_isinf(a) && __builtin_isfinite(amax)) t = a;
    float b = t + __builtin_copysignf(0.49999997f, t);
    const int32_t c = cvt_i32_sat(b);
    return c < -128 ? -128 : (c > 127 ? 127 : c);
}

// Fast codes for rows whose absmax M lies in [1e-8, 2^120) (or is the 1.0
// guard).  With c = RN(127 * RN(1/M)) and e = 2^-14, v = fma(xn, c, 0.5 - e)
// satisfies v < t + 0.5 < v + 2e for the reference quotient t
// (|fma(xn, c, 0) - t| < 3.1e-5 < e), so when fract(v) < 1 - 2e the code
// round-half-away(t) = floor(t + 0.5) is floor(v); an exact tie t = k + 0.5
// puts the integer k + 1 inside (v, v + 2e) and always fails the test.
// v_cvt_flr_i32_f32 computes floor exactly and its SDWA form writes the low
// byte into byte B of the destination, so four codes pack with four
// instructions.  The largest fract of a float4 is kept as integer bits (a
// max of non-negative floats), where a NaN or infinite xn (NaN fract) sorts
// above every threshold: those lanes, and the ~1 element in 8000 whose
// fract is too close to 1, are recomputed with quant_code.  The identity is
// checked on the CPU by the test suite.
constexpr float kCodeEps = 6.103515625e-05f;             // 2^-14
constexpr float kCodeOff = 0.5f - kCodeEps;              // exact in f32
constexpr uint32_t kFractLimit = 0x3f7ff800u;            // bits of 1 - 2^-13
constexpr float kFastAmaxLimit = 1.329227995784916e36f;  // 2^120

template <int B>
__device__ __forceinline__ uint32_t flr_byte(uint32_t d, float v) {
    if (B == 0) {
        asm("v_cvt_flr_i32_f32_sdwa %0, %1 dst_sel:BYTE_0 dst_unused:UNUSED_PAD src0_sel:DWORD" : "=v"(d) : "v"(v));
    } else if (B == 1) {
        asm("v_cvt_flr_i32_f32_sdwa %0, %1 dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:DWORD" : "+v"(d) : "v"(v));
    } else if (B == 2) {
        asm("v_cvt_flr_i32_f32_sdwa %0, %1 dst_sel:BYTE_2 dst_unused:UNUSED_PRESERVE src0_sel:DWORD" : "+v"(d) : "v"(v));
    } else {
        asm("v_cvt_flr_i32_f32_sdwa %0, %1 dst_sel:BYTE_3 dst_unused:UNUSED_PRESERVE src0_sel:DWORD" : "+v"(d) : "v"(v));
    }
    return d;
}

__device__ __forceinline__ uint32_t fract_bits(float v) { return __float_as_uint(__builtin_amdgcn_fractf(v)); }

__device__ __forceinline__ uint32_t max3_u32(uint32_t a, uint32_t b, uint32_t c) {
    uint32_t r;
    asm("v_max3_u32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// Four bracketed codes of xn (see above) and the largest fract bits among them.
__device__ __forceinline__ uint32_t flr_pack4(f32x4 xn, float c, uint32_t& fmax) {
    const float v0 = __builtin_fmaf(xn.x, c, kCodeOff), v1 = __builtin_fmaf(xn.y, c, kCodeOff);
    const float v2 = __builtin_fmaf(xn.z, c, kCodeOff), v3 = __builtin_fmaf(xn.w, c, kCodeOff);
    uint32_t d = 0;
    d = flr_byte<0>(d, v0);
    d = flr_byte<1>(d, v1);
    d = flr_byte<2>(d, v2);
    d = flr_byte<3>(d, v3);
    fmax = max3_u32(fract_bits(v0), fract_bits(v1), max3_u32(fract_bits(v2), fract_bits(v3), 0u));
    return d;
}

// Four codes -> one dword, byte k = code k (v_perm_b32 byte selects).
__device__ __forceinline__ uint32_t pack4(int32_t c0, int32_t c1, int32_t c2, int32_t c3) {
    const uint32_t lo = __builtin_amdgcn_perm((uint32_t)c1, (uint32_t)c0, 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm((uint32_t)c3, (uint32_t)c2, 0x0c0c0400u);
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

__device__ __forceinline__ float abs_max4(float m, f32x4 v) {
    m = fmaxf(m, fabsf(v.x));
    m = fmaxf(m, fabsf(v.y));
    m = fmaxf(m, fabsf(v.z));
    m = fmaxf(m, fabsf(v.w));
    return m;
}

__device__ __forceinline__ float fold4(float s, f32x4 a) {
    s = s + a.x;
    s = s + a.y;
    s = s + a.z;
    s = s + a.w;
    return s;
}

__device__ __forceinline__ float sum4(f32x4 a) { return (a.x + a.y) + (a.z + a.w); }

// DPP move of v with lanes that have no source reading 0 (bound_ctrl off,
// old = 0).  ctrl/row_mask follow the gfx9 DPP encoding.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ float dpp0(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, kRowMask, 0xf, false));
}

// Inclusive wave64 prefix sum in DPP: row_shr 1/2/4/8 within each row of 16
// lanes, then row_bcast:15 and row_bcast:31 carry the row totals forward.
// Used only for the segment-start estimates, so its summation order is free.
__device__ __forceinline__ float wave_incl_scan(float v) {
    v += dpp0<0x111, 0xf>(v);  // row_shr:1
    v += dpp0<0x112, 0xf>(v);  // row_shr:2
    v += dpp0<0x114, 0xf>(v);  // row_shr:4
    v += dpp0<0x118, 0xf>(v);  // row_shr:8
    v += dpp0<0x142, 0xa>(v);  // row_bcast:15 -> rows 1, 3
    v += dpp0<0x143, 0xc>(v);  // row_bcast:31 -> rows 2, 3
    return v;
}

// Segmented inclusive scan composing run entries with the 2-state parity
// automaton: (i0, i1) are a span's exact increments in grid units for entry
// parity 0 / 1, so its exit parity is (p + i_p) & 1, and the span x followed
// by the span y has increments x_p + y_(exit parity of x).  The head flag
// (the span already reaches its run's end) rides in bit 31 of i0.  Lanes
// without a DPP source read (0, 0), the identity.  Lane L combines with the
// lane below it, which holds a later segment.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ void auto_scan_step(uint32_t& a, uint32_t& b) {
    const uint32_t la = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)a, kCtrl, kRowMask, 0xf, false);
    const uint32_t lb = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)b, kCtrl, kRowMask, 0xf, false);
    if ((int32_t)a >= 0) {
        const uint32_t y0 = la & 0x7fffffffu;
        const uint32_t na = a + ((a & 1u) ? lb : y0);
        b = b + (((b + 1u) & 1u) ? lb : y0);
        a = na | (la & 0x80000000u);
    }
}
__device__ __forceinline__ void auto_scan(uint32_t& a, uint32_t& b) {
    auto_scan_step<0x111, 0xf>(a, b);  // row_shr:1
    auto_scan_step<0x112, 0xf>(a, b);  // row_shr:2
    auto_scan_step<0x114, 0xf>(a, b);  // row_shr:4
    auto_scan_step<0x118, 0xf>(a, b);  // row_shr:8
    auto_scan_step<0x142, 0xa>(a, b);  // row_bcast:15 -> rows 1, 3
    auto_scan_step<0x143, 0xc>(a, b);  // row_bcast:31 -> rows 2, 3
}

// Vector path: cols % 4 == 0, x/w/y 16-byte aligned, q 4-byte aligned,
// ceil(cols/4 / 64) <= SL4.  Segment j covers float4 [j*SL4, (j+1)*SL4).
// Grid: one block per WPB rows (one row per wave); dynamic LDS =
// WPB * wave_lds_f4(SL4, WPB) float4 (the transpose tiles).
// silu(z) = z / (1 + e^-z) from the hardware exp2 and reciprocal (5 VALU
// instead of ~25 for expf + IEEE division).  Error: v_exp_f32 and v_rcp_f32
// are 1 ulp each; rounding z*log2(e) to f32 perturbs e^-z by |z|*2^-24*ln2
// relative, i.e. < 6e-6 at |z| = 87 (beyond it e^-z overflows and the result
// is z*0 = -0, as the reference's z / inf).  The gated output is therefore
// within 1e-5 relative of the reference; the RMSNorm factor stays bit-exact.
// Special values follow the reference: silu(-inf) = NaN, silu(+inf) = +inf.
__device__ __forceinline__ float silu_fast(float z) {
    const float e = __builtin_amdgcn_exp2f(z * -1.44269504f);
    return z * __builtin_amdgcn_rcpf(1.0f + e);
}

// Inclusive wave64 max-scan in DPP (row_shr 1/2/4/8, then row_bcast 15/31);
// lane 63 ends with the wave's max.  Lanes without a DPP source read 0, the
// identity for the non-negative values it is used on; fmaxf drops NaN like
// Rust's f32::max.
__device__ __forceinline__ float wave_max_nonneg(float v) {
    v = fmaxf(v, dpp0<0x111, 0xf>(v));
    v = fmaxf(v, dpp0<0x112, 0xf>(v));
    v = fmaxf(v, dpp0<0x114, 0xf>(v));
    v = fmaxf(v, dpp0<0x118, 0xf>(v));
    v = fmaxf(v, dpp0<0x142, 0xa>(v));
    v = fmaxf(v, dpp0<0x143, 0xc>(v));
    return read_lane(v, kWave - 1);
}

// FULL: cols == 256*SL4 exactly (every chunk and segment complete, no bounds
// checks).  Otherwise rows are ragged: loads past the end read 0, segments
// past the end are empty.
template <NormOut Out, int SL4, bool FULL, int WPB>
__global__ __launch_bounds__(kWave * WPB) void row_norm_kernel(NormArgs args) {
    constexpr int NCH = SL4;  // 64*SL4 float4 cover the row: SL4 wave-wide chunks
    constexpr int P = seg_pitch4(SL4);
    constexpr int TS = tile_segs(SL4, WPB);
    constexpr int NPASS = kSegs / TS;
    constexpr int CPP = NCH / NPASS;  // load chunks per tile pass
    constexpr uint32_t kWaveF4 = wave_lds_f4(SL4, WPB);
    extern __shared__ f32x4 lds4[];
    const int lane = threadIdx.x & (kWave - 1);
    // Wave index as a scalar: row addresses then live in SGPRs and every
    // load and store takes the scalar-base form with a lane offset.
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
    const uint64_t row = (uint64_t)blockIdx.x * WPB + wave;
    if (row >= args.rows) return;  // uniform per wave; no block barrier follows
    const uint32_t cols4 = FULL ? (uint32_t)(kWave * SL4) : (args.cols >> 2);
    const int nseg = FULL ? kSegs : (int)((cols4 + SL4 - 1) / SL4);
    f32x4* tile = lds4 + (size_t)wave * kWaveF4;
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    const f32x4* w4 = reinterpret_cast<const f32x4*>(args.w);

    // ---- HBM reads: coalesced, chunk-major, all in flight.
    const f32x4* xr = reinterpret_cast<const f32x4*>(args.x) + row * cols4;
    f32x4 xv[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const uint32_t f = (uint32_t)c * kWave + lane;
        xv[c] = (FULL || f < cols4) ? ld_stream(xr + f) : zero;
    }

    // Wave priority rises with a row's progress (its loads issued: 1; its
    // walks: 2; the scalar resolve, the latency-critical chain: 3) and drops
    // to 0 for the element-parallel epilogue, so that on a SIMD shared by
    // four rows the dependent chains of rows further along issue first.
    // Measured at 4096 x 2560 pre-quant: 14.0 -> 13.2 us.
    __builtin_amdgcn_s_setprio(1);
    // Lane L holds segment j = 63 - L, so a forward (lane-increasing) scan
    // composes each segment with the segments after it.
    const int seg_id = kSegs - 1 - lane;
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));

    // ---- transpose the squares through the wave's tile: float4 f of the row
    // (segment q = f / SL4, offset f % SL4) goes to q*P + f % SL4 = f + (P -
    // SL4)*q, minus the pass's base; segment reads use constant offsets.
    f32x4 seg[SL4];
#pragma unroll
    for (int h = 0; h < NPASS; ++h) {
        if (h) wave_lds_sync();  // previous tile reads precede these writes
#pragma unroll
        for (int cc = 0; cc < CPP; ++cc) {
            const int c = h * CPP + cc;
            const int f = c * kWave + lane;
            const int q = f / SL4;
            tile[f + (P - SL4) * q - h * TS * P] = xv[c] * xv[c];  // zero past the end
        }
        wave_lds_sync();
        const int my = seg_id - h * TS;
        if (NPASS == 1 || (my >= 0 && my < TS)) {
#pragma unroll
            for (int k = 0; k < SL4; ++k) seg[k] = tile[my * P + k];
        }
    }

    __builtin_amdgcn_s_setprio(2);
    const bool empty = !FULL && seg_id >= nseg;
    float ssum = 0.0f;
#pragma unroll
    for (int k = 0; k < SL4; ++k) ssum += sum4(seg[k]);
    // Estimate of the running sum at this segment's start = sum over the
    // segments before it = lanes above this one (any summation order).
    const float incl = wave_incl_scan(ssum);
    const float est = read_lane(incl, kWave - 1) - incl;

    // Binade of the estimate (exponent field ef; ef <= 1 is the uniform grid
    // [0, 2^-125) of step 2^-149), selected branch-free.  Segment 0 folds
    // from its true start +0; an Inf/NaN estimate makes the segment
    // non-jumpable so that it always falls back.
    const uint32_t ef_raw = __float_as_uint(est) >> 23;  // est >= 0
    const uint32_t ef = ef_raw < 1u ? 1u : ef_raw;
    const bool sub = ef == 1u;
    const bool first = seg_id == 0 || empty;
    const bool bad = ef >= 255u;
    const float bot = sub ? 0.0f : __uint_as_float(ef << 23);
    const float top = __uint_as_float((ef + 1u) << 23);  // ef + 1 == 255 -> +Inf
    const float sig0 = first ? 0.0f : bot;
    const float sig1 = first ? 0.0f : (sub ? __uint_as_float(1u) : __uint_as_float((ef << 23) | 1u));
    float w0 = sig0, w1 = sig1;
#pragma unroll
    for (int k = 0; k < SL4; ++k) {
        const f32x4 a = seg[k];
        w0 = w0 + a.x; w1 = w1 + a.x;
        w0 = w0 + a.y; w1 = w1 + a.y;
        w0 = w0 + a.z; w1 = w1 + a.z;
        w0 = w0 + a.w; w1 = w1 + a.w;
    }
    // A segment whose estimated span touches a binade edge (within 2^-13
    // relative; the estimate and the fold differ by ~sqrt(cols) * 2^-24
    // relative on typical rows) will most likely cross it: keep it out of
    // runs so that it is folded alone instead of breaking a jump.  A
    // heuristic only: any start is checked by the resolve.  (2^-10 measured
    // 1-2% slower: more segments left out of runs.)
    const bool edge = est < bot * 1.0001220703125f || est + ssum >= top * 0.9998779296875f;
    // The merged range [0, 2^-125) is not jumped (its window would not be
    // one exponent field); sums there are folded.
    const bool valid = !first && !sub && w0 < top && w1 < top && !edge && !bad;
    // Exact increments in grid units for entry parity 0 / 1: inside the
    // binade the float bits are linear in the value, sig1 one grid step
    // above sig0 = bot.  Meaningful for valid segments only.
    const uint32_t inc0 = __float_as_uint(w0) - __float_as_uint(bot);
    const uint32_t inc1 = __float_as_uint(w1) - __float_as_uint(bot) - 1u;
    // Runs: maximal spans of valid segments with one binade key, composed by
    // the parity automaton; any other segment is a run of its own.  (Runs of
    // only the segments whose two walks agree, composed by a plain integer
    // sum, make a lighter scan but more resolve steps: measured slower at
    // every size.)  This lane's segment ends its run when the next segment
    // (lane - 1, moved here by wave_shr:1) has another key.
    const int key_me = empty ? 1024 : (seg_id == 0 ? 1025 : (valid ? (int)ef : 2048 + seg_id));
    const int key_next = __builtin_amdgcn_update_dpp(key_me, key_me, 0x138, 0xf, 0xf, false);
    const bool ends_here = lane == 0 || key_next != key_me;
    const uint64_t ends = __ballot(ends_here);
    // Run increments from this segment to the run's end (a forward scan
    // composes the later segments, held by lower lanes).
    uint32_t run_i0 = (valid ? inc0 : 0u) | (ends_here ? 0x80000000u : 0u);
    uint32_t run_i1 = valid ? inc1 : 0u;
    auto_scan(run_i0, run_i1);
    run_i0 &= 0x7fffffffu;
    // The run of lane L ends at the highest lane <= L with its bit set; the
    // segment after it is 64 - that lane.
    const uint64_t below = ends & (lt_mask | (1ull << lane));
    const uint32_t next_seg = (uint32_t)(kSegs - (63 - __builtin_clzll(below)));
    // Run entry packed in two words, read with two lane reads:
    //   word 0: increment for entry parity 0 (24 bits; a run below one binade
    //           top never reaches 2^23) | exponent field of the binade << 24;
    //   word 1: segment after the run | parity-1 increment minus parity-0
    //           increment (7-bit signed) << 8 | jumpable << 15.
    // Runs whose parity-0 and parity-1 increments differ by 64 grid steps or
    // more, runs whose increment reaches a whole binade (no start could stay
    // inside it), and invalid segments are not jumpable: the resolve folds
    // them.
    const int32_t delta = (int32_t)(run_i1 - run_i0);
    const uint32_t e_inc = run_i0;
    const bool jumpable = valid && delta >= -64 && delta < 64 && e_inc < 0x800000u;
    const uint32_t e_w0 = (e_inc & 0xffffffu) | (ef << 24);
    const uint32_t e_w1 = next_seg | (((uint32_t)delta & 0x7fu) << 8) | (jumpable ? 0x8000u : 0u);

    // ---- resolve on the scalar unit.  s holds the bits of the exact running
    // sum (non-negative, so unsigned order is float order and NaN/Inf sort
    // above every window).  Segment 0 was folded from +0 and is exact.  The
    // entry of segment j lives in lane 63 - j.  A jumpable entry applies when
    // s lies in its binade [lo, lo + 2^23 grid steps) and the jump lands
    // inside it too: s moves by the increment for its parity (the lsb of s's
    // bits is its parity on the binade grid).  With t = s + inc >= s both
    // tests are max(s - lo, t - lo) < 2^23 in wrapping unsigned arithmetic
    // (s < lo wraps to a huge value).  Otherwise the owner lane folds the
    // segment alone from s and broadcasts the sum.  The next entry's lane
    // reads are issued before the test so that they overlap it.
    __builtin_amdgcn_s_setprio(3);
    uint32_t s = __builtin_amdgcn_readlane(__float_as_uint(w0), kWave - 1);
    int j = 1;
    uint32_t c0 = (uint32_t)__builtin_amdgcn_readlane((int)e_w0, kSegs - 2);
    uint32_t c1 = (uint32_t)__builtin_amdgcn_readlane((int)e_w1, kSegs - 2);
    while (j < nseg) {
        const int nj = (int)(c1 & 0xffu);
        const uint32_t n0 = (uint32_t)__builtin_amdgcn_readlane((int)e_w0, (kSegs - 1 - nj) & (kWave - 1));
        const uint32_t n1 = (uint32_t)__builtin_amdgcn_readlane((int)e_w1, (kSegs - 1 - nj) & (kWave - 1));
        const int32_t dp = (int32_t)(c1 << 17) >> 25;
        const uint32_t t = s + (c0 & 0xffffffu) + ((s & 1u) ? (uint32_t)dp : 0u);
        const uint32_t lo = (c0 >> 24) << 23;
        const uint32_t da = s - lo, db = t - lo;
        if ((c1 & 0x8000u) && (da > db ? da : db) < 0x800000u) {
            s = t;
            j = nj;
            c0 = n0;
            c1 = n1;
            continue;
        }
        // Fold segment j alone.  The entry of segment j + 1 is read first so
        // that its latency hides under the fold chain.  Every lane folds its
        // own segment from s (same cost as one lane under an exec mask,
        // without the mask changes); lane 63 - j's sum is the one kept.
        const int L = kSegs - 1 - j;
        c0 = (uint32_t)__builtin_amdgcn_readlane((int)e_w0, (L - 1) & (kWave - 1));
        c1 = (uint32_t)__builtin_amdgcn_readlane((int)e_w1, (L - 1) & (kWave - 1));
        float acc = __uint_as_float(s);
#pragma unroll
        for (int k = 0; k < SL4; ++k) acc = fold4(acc, seg[k]);
        s = (uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(acc), L);
        ++j;
    }
    const float ss = __uint_as_float(s);
    __builtin_amdgcn_s_setprio(0);

    // Weights for the epilogue (L2 hits), loaded after the resolve so their
    // registers are free while it runs (staging them in LDS at the start was
    // measured slower: 14.0 -> 14.4 us at 4096 x 2560).
    f32x4 wv[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const uint32_t f = (uint32_t)c * kWave + lane;
        wv[c] = (FULL || f < cols4) ? ld_cached(w4 + f) : zero;
    }

    // cpu_fused.rs:181-182 with IEEE sqrt and division (ss is uniform).
    const float inv = 1.0f / sqrtf(ss / (float)args.cols + args.eps);

    if (Out == NormOut::F32) {
        f32x4* yr = reinterpret_cast<f32x4*>(args.y) + row * cols4;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const uint32_t f = (uint32_t)c * kWave + lane;
            if (FULL || f < cols4) st_stream(yr + f, (xv[c] * inv) * wv[c]);
        }
    } else if (Out == NormOut::SiluGate) {
        // cpu_fused.rs:466-471: x_hat = (x*inv)*g; y = x_hat * silu(z).
        const f32x4* zr = reinterpret_cast<const f32x4*>(args.z) + row * cols4;
        f32x4* yr = reinterpret_cast<f32x4*>(args.y) + row * cols4;
        // x_hat first, so that the weights are dead before z is loaded
        // (keeps the 2560-column kernel within 128 VGPRs: four waves a SIMD)
#pragma unroll
        for (int c = 0; c < NCH; ++c) xv[c] = (xv[c] * inv) * wv[c];
        f32x4 zv[NCH];
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const uint32_t f = (uint32_t)c * kWave + lane;
            zv[c] = (FULL || f < cols4) ? ld_stream(zr + f) : zero;
        }
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const uint32_t f = (uint32_t)c * kWave + lane;
            if (FULL || f < cols4) {
                const f32x4 xh = xv[c];
                f32x4 g;
                g.x = silu_fast(zv[c].x);
                g.y = silu_fast(zv[c].y);
                g.z = silu_fast(zv[c].z);
                g.w = silu_fast(zv[c].w);
                st_stream(yr + f, xh * g);
            }
        }
    } else {
#pragma unroll
        for (int c = 0; c < NCH; ++c) xv[c] = (xv[c] * inv) * wv[c];
        // amax: the reference's fold(0, f32::max) of |xn| (NaN dropped).
        float amax = 0.0f;
#pragma unroll
        for (int c = 0; c < NCH; ++c) amax = abs_max4(amax, xv[c]);
        amax = wave_max_nonneg(amax);
        uint32_t* qr = reinterpret_cast<uint32_t*>(args.q) + row * cols4;
        if (amax < kFastAmaxLimit) {
            amax = amax < 1e-8f ? 1.0f : amax;  // kore-btes/src/quantize.rs:10
            const float rcp = 1.0f / amax;
            const float c127 = 127.0f * rcp;
            if (lane == 0) args.scale[row] = amax / 127.0f;
            uint64_t redo[NCH];
            uint64_t any = 0;
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                const uint32_t f = (uint32_t)c * kWave + lane;
                uint32_t fm = 0;
                const uint32_t d = flr_pack4(xv[c], c127, fm);
                redo[c] = __ballot((FULL || f < cols4) && fm >= kFractLimit);
                any |= redo[c];
                if (FULL || f < cols4) qr[f] = d;
            }
            if (any) {
                // Rare: exact codes for the lanes whose brackets failed (they
                // overwrite the stores above, in program order).
#pragma unroll
                for (int c = 0; c < NCH; ++c) {
                    if ((redo[c] >> lane) & 1u) {
                        const f32x4 v = xv[c];
                        qr[(uint32_t)c * kWave + lane] =
                            pack4(quant_code(v.x, amax, rcp), quant_code(v.y, amax, rcp),
                                  quant_code(v.z, amax, rcp), quant_code(v.w, amax, rcp));
                    }
                }
            }
        } else {
            // An absmax of 2^120 or more, infinite, or NaN (every xn NaN):
            // exact codes.
            amax = amax < 1e-8f ? 1.0f : amax;  // kore-btes/src/quantize.rs:10
            const float rcp = 1.0f / amax;
            if (lane == 0) args.scale[row] = amax / 127.0f;
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                const uint32_t f = (uint32_t)c * kWave + lane;
                if (FULL || f < cols4) {
                    const f32x4 v = xv[c];
                    qr[f] = pack4(quant_code(v.x, amax, rcp), quant_code(v.y, amax, rcp),
                                  quant_code(v.z, amax, rcp), quant_code(v.w, amax, rcp));
                }
            }
        }
    }
}

// Scalar path for any shape/alignment: one thread per row, the reference loop
// verbatim.  Used for cols % 4 != 0, unaligned views and rows longer than
// the vector path's register budget.
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
    } else if (Out == NormOut::SiluGate) {
        float* yr = args.y + row * cols;
        const float* zr = args.z + row * cols;
        for (uint32_t i = 0; i < cols; ++i) yr[i] = ((xr[i] * inv) * args.w[i]) * silu_f(zr[i]);
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

template <NormOut Out, int SL4, int WPB>
static int launch_vec_wpb(NormArgs a, hipStream_t s) {
    const size_t lds = (size_t)WPB * wave_lds_f4(SL4, WPB) * sizeof(f32x4);
    const uint64_t blocks = (a.rows + WPB - 1) / WPB;
    if (blocks > 0x7fffffffull) return KORE_HIP_ERR_OVERFLOW;
    if (a.cols == (uint32_t)(4 * kWave * SL4))
        hipLaunchKernelGGL((row_norm_kernel<Out, SL4, true, WPB>), dim3((uint32_t)blocks), dim3(kWave * WPB), lds, s, a);
    else
        hipLaunchKernelGGL((row_norm_kernel<Out, SL4, false, WPB>), dim3((uint32_t)blocks), dim3(kWave * WPB), lds, s,
                           a);
    return launch_status();
}

// One wave per workgroup (its tile holds the whole row: one LDS pass) for
// launches of up to kSmallRows rows (decode batches: the workgroups spread
// over more dispatchers and start sooner; 32 x 2048 RMSNorm 4.4 -> 4.0 us,
// 64 x 2560 gate 6.0 -> 5.6 us) and, at any row count, for the row lengths
// where the whole-row tiles still leave the register-bound occupancy: up to
// 2048 columns, and 4096 or 8192 (RMSNorm 16384 x 2048 47.2 -> 46.0 us,
// 8192 x 2048 26.5 -> 24.5, 16384 x 4096 94.7 -> 90.6, 16384 x 8192 202 ->
// 182, pre-quant 4096 x 8192 54.7 -> 46.9; ties within 1% elsewhere).  For
// SL4 = 10, 12 and 24 (2560, 3072 and 6144 columns) the whole-row tiles cap
// a CU below the waves its registers allow, and four waves per workgroup
// sharing half-row tiles are faster (pre-quant 4096 x 2560 13.0 against
// 15.1 us, RMSNorm 4096 x 3072 16.3 against 21.4).
constexpr uint64_t kSmallRows = 256;

template <NormOut Out, int SL4>
static int launch_vec(NormArgs a, hipStream_t s) {
    if constexpr (SL4 == 10 || SL4 == 12 || SL4 == 24) {
        if (a.rows > kSmallRows) return launch_vec_wpb<Out, SL4, kWavesPerBlock>(a, s);
    }
    return launch_vec_wpb<Out, SL4, 1>(a, s);
}

template <NormOut Out>
static int launch_sl4(NormArgs a, uint32_t nch, hipStream_t s) {
    if (nch <= 1) return launch_vec<Out, 1>(a, s);
    if (nch <= 2) return launch_vec<Out, 2>(a, s);
    if (nch <= 4) return launch_vec<Out, 4>(a, s);
    if (nch <= 6) return launch_vec<Out, 6>(a, s);
    if (nch <= 8) return launch_vec<Out, 8>(a, s);
    if (nch <= 10) return launch_vec<Out, 10>(a, s);
    if (nch <= 12) return launch_vec<Out, 12>(a, s);
    if (nch <= 16) return launch_vec<Out, 16>(a, s);
    if (nch <= 24) return launch_vec<Out, 24>(a, s);
    return launch_vec<Out, 32>(a, s);
}

// One row per wave: with the half-row tile a wave needs ~8 KB of LDS and
// ~110 VGPRs (2560 columns), so four waves share each SIMD and hide each
// other's latency -- measured faster than amortising the resolve over two or
// four rows per wave at lower occupancy, and than splitting a row over two
// waves that meet through block barriers (4096 x 2560 pre-quant 14.4 vs
// 16.4 us).
template <NormOut Out>
static int norm_launch(NormArgs a, hipStream_t s) {
    if (a.rows == 0) return KORE_HIP_OK;
    if (a.cols == 0) return KORE_HIP_ERR_BAD_DIM;
    if (!a.x || !a.w) return KORE_HIP_ERR_NULL_PTR;
    if (Out != NormOut::I8 && !a.y) return KORE_HIP_ERR_NULL_PTR;
    if (Out == NormOut::SiluGate && !a.z) return KORE_HIP_ERR_NULL_PTR;
    if (Out == NormOut::I8 && (!a.q || !a.scale)) return KORE_HIP_ERR_NULL_PTR;
    uint64_t elems;
    if (!mul_ok(a.rows, a.cols, &elems) || elems > kMaxElements) return KORE_HIP_ERR_OVERFLOW;
    const uint32_t cols4 = a.cols / 4;
    const uint32_t nch = (cols4 + kWave - 1) / kWave;
    bool vec = a.cols % 4 == 0 && aligned16(a.x) && aligned16(a.w) && nch <= 32;
    if (Out == NormOut::F32) vec = vec && aligned16(a.y);
    else if (Out == NormOut::SiluGate) vec = vec && aligned16(a.y) && aligned16(a.z);
    else vec = vec && (reinterpret_cast<uintptr_t>(a.q) & 3u) == 0;
    if (!vec) {
        uint64_t blocks = (a.rows + 63) / 64;
        if (blocks > 0x7fffffffull) return KORE_HIP_ERR_OVERFLOW;
        hipLaunchKernelGGL(row_norm_scalar_kernel<Out>, dim3((uint32_t)blocks), dim3(64), 0, s, a);
        return launch_status();
    }
    return launch_sl4<Out>(a, nch, s);
}

}  // namespace kore

using namespace kore;

extern "C" int kore_hip_rms_norm_f32(const float* x, const float* weight, float* out, uint64_t rows,
                                     uint64_t cols, float eps, kore_stream_t stream) {
    if (cols > 0xffffffffull) return KORE_HIP_ERR_OVERFLOW;
    NormArgs a{x, weight, out, nullptr, nullptr, nullptr, rows, (uint32_t)cols, eps};
    return norm_launch<NormOut::F32>(a, (hipStream_t)stream);
}

extern "C" int kore_hip_rms_norm_quant_i8(const float* x, const float* weight, int8_t* q, float* scale,
                                          uint64_t rows, uint64_t cols, float eps, kore_stream_t stream) {
    if (cols > 0xffffffffull) return KORE_HIP_ERR_OVERFLOW;
    NormArgs a{x, weight, nullptr, q, scale, nullptr, rows, (uint32_t)cols, eps};
    return norm_launch<NormOut::I8>(a, (hipStream_t)stream);
}

extern "C" int kore_hip_rms_norm_silu_gate_f32(const float* x, const float* weight, const float* z, float* out,
                                               uint64_t rows, uint64_t cols, float eps, kore_stream_t stream) {
    if (cols > 0xffffffffull) return KORE_HIP_ERR_OVERFLOW;
    NormArgs a{x, weight, out, nullptr, nullptr, z, rows, (uint32_t)cols, eps};
    return norm_launch<NormOut::SiluGate>(a, (hipStream_t)stream);
}
