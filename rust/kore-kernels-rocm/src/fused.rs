//! Fused layer ops on MI355X through `libkore_hip.so` (hand-written gfx950
//! kernels behind the C ABI of `include/kore_hip.h`).
//!
//! Drop-in module for KORE: copy this file to
//! `crates/kore-kernels/src/rocm/fused.rs` and add `pub mod fused;` to
//! `crates/kore-kernels/src/rocm/mod.rs`.  It needs nothing beyond what the
//! `rocm` feature already enables (`libloading`, crates/kore-kernels/Cargo.toml)
//! and the backend's own `context` and `memory` modules, and follows their
//! pattern: runtime loading like rocm/ffi.rs:90-133, `HipBuffer` outputs like
//! `cuda_rms_norm_f32` (cuda/ops.rs:527-529), `RocmError`
//! (rocm/context.rs:95-117), the null stream (rocm/launch.rs:190).
//!
//! Not compiled in this repository: the build image has no Rust toolchain.
use std::ffi::{c_char, c_int, c_void, CStr};
use std::sync::OnceLock;

use libloading::Library;

use super::context::{set_device, RocmError};
use super::memory::HipBuffer;

type Stream = *mut c_void;
type FnRmsNorm = unsafe extern "C" fn(*const f32, *const f32, *mut f32, u64, u64, f32, Stream) -> c_int;
type FnUnary = unsafe extern "C" fn(*const f32, *mut f32, u64, Stream) -> c_int;
type FnBinary = unsafe extern "C" fn(*const f32, *const f32, *mut f32, u64, Stream) -> c_int;
type FnInvFreq = unsafe extern "C" fn(*mut f32, u32, f32) -> c_int;
type FnRope = unsafe extern "C" fn(*mut f32, *const f32, u64, u64, u32, u32, u64, c_int, Stream) -> c_int;
type FnRopeQk =
    unsafe extern "C" fn(*mut f32, *mut f32, *const f32, u64, u64, u32, u32, u32, u64, c_int, Stream) -> c_int;
type FnEmbed = unsafe extern "C" fn(*const f32, *const u32, *mut f32, u64, u64, u64, Stream) -> c_int;
type FnEmbedF32Ids = unsafe extern "C" fn(*const f32, *const f32, *mut f32, u64, u64, u64, Stream) -> c_int;
type FnPreQuant = unsafe extern "C" fn(*const f32, *const f32, *mut i8, *mut f32, u64, u64, f32, Stream) -> c_int;
type FnSiluGate =
    unsafe extern "C" fn(*const f32, *const f32, *const f32, *mut f32, u64, u64, f32, Stream) -> c_int;
type FnSoftmax = unsafe extern "C" fn(*const f32, *mut f32, u64, u64, Stream) -> c_int;
type FnSoftmaxCausal = unsafe extern "C" fn(*const f32, *mut f32, u64, u64, u64, Stream) -> c_int;
type FnSoftmaxBwd = unsafe extern "C" fn(*const f32, *const f32, *mut f32, u64, u64, Stream) -> c_int;
type FnRmsBwdWs = unsafe extern "C" fn(u64, u64) -> u64;
type FnRmsBwd = unsafe extern "C" fn(*const f32, *const f32, *const f32, *mut f32, *mut f32, *mut f32, u64, u64,
                                     u64, f32, Stream) -> c_int;
type FnRmsBwdNoAlloc = unsafe extern "C" fn(*const f32, *const f32, *const f32, *mut f32, *mut f32, u64, u64, f32,
                                            Stream) -> c_int;
type FnMaxBytes = unsafe extern "C" fn() -> u64;
type FnTernaryI8 = unsafe extern "C" fn(*const u8, *const f32, *const i8, *const f32, *mut f32, u64, u64, u64,
                                        Stream) -> c_int;
type FnTernaryF32 = unsafe extern "C" fn(*const u8, *const f32, *const f32, *mut f32, u64, u64, u64,
                                         Stream) -> c_int;
type FnBitLinearF32 = unsafe extern "C" fn(*const u8, *const f32, *const f32, *const f32, *mut f32, u64, u64, u64,
                                          Stream) -> c_int;
type FnBitLinearI8 = unsafe extern "C" fn(*const u8, *const f32, *const i8, *const f32, *const f32, *mut f32, u64,
                                         u64, u64, Stream) -> c_int;
type FnPackTernary = unsafe extern "C" fn(*const f32, u64, u64, f32, *mut u8, *mut f32, Stream) -> c_int;
type FnStatus = unsafe extern "C" fn(c_int) -> *const c_char;

struct FusedApi {
    _lib: Library,
    rms_norm: FnRmsNorm,
    gelu: FnUnary,
    silu: FnUnary,
    mul: FnBinary,
    swiglu: FnBinary,
    rope_inv_freq: FnInvFreq,
    rope: FnRope,
    rope_qk: FnRopeQk,
    embedding: FnEmbed,
    embedding_forward: FnEmbedF32Ids,
    prequant: FnPreQuant,
    silu_gate: FnSiluGate,
    softmax: FnSoftmax,
    softmax_causal: FnSoftmaxCausal,
    softmax_bwd: FnSoftmaxBwd,
    ce_bwd: FnSoftmaxBwd,
    rms_bwd_ws: FnRmsBwdWs,
    rms_bwd: FnRmsBwd,
    rms_bwd_noalloc: FnRmsBwdNoAlloc,
    rms_bwd_noalloc_max: FnMaxBytes,
    ternary_i8: FnTernaryI8,
    ternary_f32: FnTernaryF32,
    bit_linear_f32: FnBitLinearF32,
    bit_linear_i8: FnBitLinearI8,
    pack_ternary: FnPackTernary,
    status: FnStatus,
}
unsafe impl Send for FusedApi {}
unsafe impl Sync for FusedApi {}

static API: OnceLock<Option<FusedApi>> = OnceLock::new();

fn api() -> Result<&'static FusedApi, RocmError> {
    API.get_or_init(|| unsafe {
        let path = std::env::var("KORE_HIP_LIB").unwrap_or_else(|_| "libkore_hip.so".into());
        let lib = Library::new(path).ok()?;
        Some(FusedApi {
            rms_norm: *lib.get(b"kore_hip_rms_norm_f32\0").ok()?,
            gelu: *lib.get(b"kore_hip_gelu_f32\0").ok()?,
            silu: *lib.get(b"kore_hip_silu_f32\0").ok()?,
            mul: *lib.get(b"kore_hip_mul_f32\0").ok()?,
            swiglu: *lib.get(b"kore_hip_swiglu_f32\0").ok()?,
            rope_inv_freq: *lib.get(b"kore_hip_rope_inv_freq_f32\0").ok()?,
            rope: *lib.get(b"kore_hip_rope_f32\0").ok()?,
            rope_qk: *lib.get(b"kore_hip_rope_qk_f32\0").ok()?,
            embedding: *lib.get(b"kore_hip_embedding_f32\0").ok()?,
            embedding_forward: *lib.get(b"kore_hip_embedding_forward_f32\0").ok()?,
            prequant: *lib.get(b"kore_hip_rms_norm_quant_i8\0").ok()?,
            silu_gate: *lib.get(b"kore_hip_rms_norm_silu_gate_f32\0").ok()?,
            softmax: *lib.get(b"kore_hip_softmax_f32\0").ok()?,
            softmax_causal: *lib.get(b"kore_hip_softmax_causal_f32\0").ok()?,
            softmax_bwd: *lib.get(b"kore_hip_softmax_backward_f32\0").ok()?,
            ce_bwd: *lib.get(b"kore_hip_cross_entropy_backward_f32\0").ok()?,
            rms_bwd_ws: *lib.get(b"kore_hip_rms_norm_backward_workspace_bytes\0").ok()?,
            rms_bwd: *lib.get(b"kore_hip_rms_norm_backward_f32\0").ok()?,
            rms_bwd_noalloc: *lib.get(b"kore_hip_rms_norm_backward_noalloc_f32\0").ok()?,
            rms_bwd_noalloc_max: *lib.get(b"kore_hip_rms_norm_backward_noalloc_max_bytes\0").ok()?,
            ternary_i8: *lib.get(b"kore_hip_ternary_matmul_i8\0").ok()?,
            ternary_f32: *lib.get(b"kore_hip_ternary_matmul_f32\0").ok()?,
            bit_linear_f32: *lib.get(b"kore_hip_bit_linear_f32\0").ok()?,
            bit_linear_i8: *lib.get(b"kore_hip_bit_linear_i8\0").ok()?,
            pack_ternary: *lib.get(b"kore_hip_pack_weights_ternary\0").ok()?,
            status: *lib.get(b"kore_hip_status_string\0").ok()?,
            _lib: lib,
        })
    })
    .as_ref()
    .ok_or(RocmError::NotAvailable)
}

/// Status -> RocmError, as `check_hip` does for HIP codes (rocm/ffi.rs:211-220).
fn check(code: c_int, context: &str) -> Result<(), RocmError> {
    if code == 0 {
        return Ok(());
    }
    let text = unsafe { CStr::from_ptr((api()?.status)(code)) }.to_string_lossy().into_owned();
    if code > 0 {
        Err(RocmError::HipError { code, context: format!("{context}: {text}") })
    } else {
        Err(RocmError::LaunchError(format!("{context}: {text}")))
    }
}

/// The product of a buffer's dimensions, or a MemoryError where it overflows usize (an oversized
/// shape must not wrap around to a small byte count and pass the size checks).
fn prod(dims: &[usize]) -> Result<usize, RocmError> {
    dims.iter()
        .try_fold(1usize, |acc, &d| acc.checked_mul(d))
        .ok_or_else(|| RocmError::MemoryError(format!("shape {dims:?}: byte count overflows usize")))
}

fn need(buf: &HipBuffer, bytes: usize, what: &str) -> Result<(), RocmError> {
    if buf.len() < bytes {
        return Err(RocmError::MemoryError(format!("{what}: {} bytes < {bytes}", buf.len())));
    }
    Ok(())
}

/// Mirrors `cuda_rms_norm_f32` (cuda/ops.rs:517-541); bit-exact vs `fused_rms_norm`.
pub fn rocm_rms_norm_f32(dev: usize, input: &HipBuffer, weight: &HipBuffer, rows: usize, cols: usize,
                         eps: f32) -> Result<HipBuffer, RocmError> {
    need(input, prod(&[rows, cols, 4])?, "rms_norm input")?;
    need(weight, prod(&[cols, 4])?, "rms_norm weight")?;
    set_device(dev)?;
    let out = HipBuffer::zeros(dev, prod(&[rows, cols, 4])?)?;
    check(unsafe { (api()?.rms_norm)(input.as_device_ptr() as _, weight.as_device_ptr() as _,
                                     out.as_device_ptr() as _, rows as u64, cols as u64, eps,
                                     std::ptr::null_mut()) }, "rms_norm_f32")?;
    Ok(out)
}

/// Mirrors `cuda_gelu_f32` / `cuda_silu_f32` (cuda/ops.rs:197-213).
pub fn rocm_gelu_f32(dev: usize, a: &HipBuffer, n: usize) -> Result<HipBuffer, RocmError> {
    unary(dev, a, n, api()?.gelu, "gelu_f32")
}
pub fn rocm_silu_f32(dev: usize, a: &HipBuffer, n: usize) -> Result<HipBuffer, RocmError> {
    unary(dev, a, n, api()?.silu, "silu_f32")
}
fn unary(dev: usize, a: &HipBuffer, n: usize, f: FnUnary, ctx: &str) -> Result<HipBuffer, RocmError> {
    need(a, prod(&[n, 4])?, ctx)?;
    set_device(dev)?;
    let out = HipBuffer::zeros(dev, prod(&[n, 4])?)?;
    check(unsafe { f(a.as_device_ptr() as _, out.as_device_ptr() as _, n as u64, std::ptr::null_mut()) }, ctx)?;
    Ok(out)
}

/// `cuda_mul_f32` (cuda/ops.rs:100-108) and the fused silu(gate)*up.
pub fn rocm_mul_f32(dev: usize, a: &HipBuffer, b: &HipBuffer, n: usize) -> Result<HipBuffer, RocmError> {
    binary(dev, a, b, n, api()?.mul, "mul_f32")
}
pub fn rocm_swiglu_f32(dev: usize, gate: &HipBuffer, up: &HipBuffer, n: usize) -> Result<HipBuffer, RocmError> {
    binary(dev, gate, up, n, api()?.swiglu, "swiglu_f32")
}
fn binary(dev: usize, a: &HipBuffer, b: &HipBuffer, n: usize, f: FnBinary, ctx: &str)
          -> Result<HipBuffer, RocmError> {
    need(a, prod(&[n, 4])?, ctx)?;
    need(b, prod(&[n, 4])?, ctx)?;
    set_device(dev)?;
    let out = HipBuffer::zeros(dev, prod(&[n, 4])?)?;
    check(unsafe { f(a.as_device_ptr() as _, b.as_device_ptr() as _, out.as_device_ptr() as _, n as u64,
                     std::ptr::null_mut()) }, ctx)?;
    Ok(out)
}

/// Plays the role of `cuda_rope_freqs_f32` (cuda/ops.rs:549-567): the
/// per-dimension inverse-frequency table, computed on the host, uploaded once.
pub fn rocm_rope_inv_freq_f32(dev: usize, head_dim: usize, theta: f32) -> Result<HipBuffer, RocmError> {
    let mut host = vec![0f32; head_dim / 2];
    check(unsafe { (api()?.rope_inv_freq)(host.as_mut_ptr(), head_dim as u32, theta) }, "rope_inv_freq_f32")?;
    let bytes = unsafe { std::slice::from_raw_parts(host.as_ptr() as *const u8, host.len() * 4) };
    HipBuffer::from_host(dev, bytes)
}

/// `cuda_rope_f32` (cuda/ops.rs:572-599), in place on [batch, seq, heads, head_dim].
pub fn rocm_rope_f32(dev: usize, data: &HipBuffer, inv_freq: &HipBuffer, batch: usize, seq_len: usize,
                     num_heads: usize, head_dim: usize, start_pos: usize, interleaved: bool)
                     -> Result<(), RocmError> {
    need(data, prod(&[batch, seq_len, num_heads, head_dim, 4])?, "rope data")?;
    need(inv_freq, head_dim / 2 * 4, "rope inv_freq")?;
    set_device(dev)?;
    check(unsafe { (api()?.rope)(data.as_device_ptr() as _, inv_freq.as_device_ptr() as _, batch as u64,
                                 seq_len as u64, num_heads as u32, head_dim as u32, start_pos as u64,
                                 interleaved as c_int, std::ptr::null_mut()) }, "rope_f32")
}

/// `Embedding::lookup` (crates/kore-nn/src/embedding.rs:55-72) on the device.
pub fn rocm_embedding_f32(dev: usize, table: &HipBuffer, ids: &HipBuffer, n_ids: usize, vocab: usize,
                          dim: usize) -> Result<HipBuffer, RocmError> {
    need(table, prod(&[vocab, dim, 4])?, "embedding table")?;
    need(ids, prod(&[n_ids, 4])?, "embedding ids")?;
    set_device(dev)?;
    let out = HipBuffer::zeros(dev, prod(&[n_ids, dim, 4])?)?;
    check(unsafe { (api()?.embedding)(table.as_device_ptr() as _, ids.as_device_ptr() as _,
                                      out.as_device_ptr() as _, n_ids as u64, vocab as u64, dim as u64,
                                      std::ptr::null_mut()) }, "embedding_f32")?;
    Ok(out)
}

/// Q and K of one attention layer (GQA: q_heads != k_heads) rotated in one launch; the same
/// results as two `rocm_rope_f32` calls.
pub fn rocm_rope_qk_f32(dev: usize, q: &HipBuffer, k: &HipBuffer, inv_freq: &HipBuffer, batch: usize,
                        seq_len: usize, q_heads: usize, k_heads: usize, head_dim: usize, start_pos: usize,
                        interleaved: bool) -> Result<(), RocmError> {
    need(q, prod(&[batch, seq_len, q_heads, head_dim, 4])?, "rope q")?;
    need(k, prod(&[batch, seq_len, k_heads, head_dim, 4])?, "rope k")?;
    need(inv_freq, head_dim / 2 * 4, "rope inv_freq")?;
    set_device(dev)?;
    check(unsafe { (api()?.rope_qk)(q.as_device_ptr() as _, k.as_device_ptr() as _, inv_freq.as_device_ptr() as _,
                                    batch as u64, seq_len as u64, q_heads as u32, k_heads as u32,
                                    head_dim as u32, start_pos as u64, interleaved as c_int,
                                    std::ptr::null_mut()) }, "rope_qk_f32")
}

/// `Module::forward` of `Embedding` (crates/kore-nn/src/embedding.rs:91-98): the ids arrive as an
/// f32 tensor and are converted with Rust's `v as usize` on the device (NaN and values below 1 ->
/// row 0, saturating), then looked up as `lookup` does.
pub fn rocm_embedding_forward_f32(dev: usize, table: &HipBuffer, ids: &HipBuffer, n_ids: usize, vocab: usize,
                                  dim: usize) -> Result<HipBuffer, RocmError> {
    need(table, prod(&[vocab, dim, 4])?, "embedding table")?;
    need(ids, prod(&[n_ids, 4])?, "embedding ids")?;
    set_device(dev)?;
    let out = HipBuffer::zeros(dev, prod(&[n_ids, dim, 4])?)?;
    check(unsafe { (api()?.embedding_forward)(table.as_device_ptr() as _, ids.as_device_ptr() as _,
                                              out.as_device_ptr() as _, n_ids as u64, vocab as u64, dim as u64,
                                              std::ptr::null_mut()) }, "embedding_forward_f32")?;
    Ok(out)
}

/// RMSNorm + per-row absmax int8 (the BitLinear pre-quant): (codes, scales).
pub fn rocm_rms_norm_quant_i8(dev: usize, input: &HipBuffer, weight: &HipBuffer, rows: usize, cols: usize,
                              eps: f32) -> Result<(HipBuffer, HipBuffer), RocmError> {
    need(input, prod(&[rows, cols, 4])?, "prequant input")?;
    need(weight, prod(&[cols, 4])?, "prequant weight")?;
    set_device(dev)?;
    let q = HipBuffer::zeros(dev, prod(&[rows, cols])?)?;
    let s = HipBuffer::zeros(dev, prod(&[rows, 4])?)?;
    check(unsafe { (api()?.prequant)(input.as_device_ptr() as _, weight.as_device_ptr() as _,
                                     q.as_device_ptr() as _, s.as_device_ptr() as _, rows as u64,
                                     cols as u64, eps, std::ptr::null_mut()) }, "rms_norm_quant_i8")?;
    Ok((q, s))
}

/// Mirrors `cuda_fused_rms_norm_silu_gate_f32` (cuda/ops.rs:717-751): y = RMSNorm(x) * silu(z).
pub fn rocm_fused_rms_norm_silu_gate_f32(dev: usize, input: &HipBuffer, gamma: &HipBuffer, gate: &HipBuffer,
                                         rows: usize, cols: usize, eps: f32) -> Result<HipBuffer, RocmError> {
    need(input, prod(&[rows, cols, 4])?, "silu_gate input")?;
    need(gamma, prod(&[cols, 4])?, "silu_gate gamma")?;
    need(gate, prod(&[rows, cols, 4])?, "silu_gate gate")?;
    set_device(dev)?;
    let out = HipBuffer::zeros(dev, prod(&[rows, cols, 4])?)?;
    check(unsafe { (api()?.silu_gate)(input.as_device_ptr() as _, gamma.as_device_ptr() as _,
                                      gate.as_device_ptr() as _, out.as_device_ptr() as _, rows as u64,
                                      cols as u64, eps, std::ptr::null_mut()) }, "rms_norm_silu_gate_f32")?;
    Ok(out)
}

/// Mirrors `cuda_softmax_f32` (cuda/ops.rs:486-511); `fused_softmax` semantics.
pub fn rocm_softmax_f32(dev: usize, a: &HipBuffer, rows: usize, cols: usize) -> Result<HipBuffer, RocmError> {
    need(a, prod(&[rows, cols, 4])?, "softmax input")?;
    set_device(dev)?;
    let out = HipBuffer::zeros(dev, prod(&[rows, cols, 4])?)?;
    check(unsafe { (api()?.softmax)(a.as_device_ptr() as _, out.as_device_ptr() as _, rows as u64, cols as u64,
                                    std::ptr::null_mut()) }, "softmax_f32")?;
    Ok(out)
}

/// The `softmax_causal_f32` kernel (cuda/kernels/softmax.cu:88-157), which the
/// reference never wraps: row r keeps columns < seq_offset + r + 1.
pub fn rocm_softmax_causal_f32(dev: usize, a: &HipBuffer, rows: usize, cols: usize, seq_offset: usize)
                               -> Result<HipBuffer, RocmError> {
    need(a, prod(&[rows, cols, 4])?, "softmax_causal input")?;
    set_device(dev)?;
    let out = HipBuffer::zeros(dev, prod(&[rows, cols, 4])?)?;
    check(unsafe { (api()?.softmax_causal)(a.as_device_ptr() as _, out.as_device_ptr() as _, rows as u64,
                                           cols as u64, seq_offset as u64, std::ptr::null_mut()) },
          "softmax_causal_f32")?;
    Ok(out)
}

/// `fused_softmax_backward` (cpu_fused_backward.rs:86-115) on the device.
pub fn rocm_softmax_backward_f32(dev: usize, grad_output: &HipBuffer, output: &HipBuffer, rows: usize,
                                 cols: usize) -> Result<HipBuffer, RocmError> {
    need(grad_output, prod(&[rows, cols, 4])?, "softmax_backward grad_output")?;
    need(output, prod(&[rows, cols, 4])?, "softmax_backward output")?;
    set_device(dev)?;
    let dx = HipBuffer::zeros(dev, prod(&[rows, cols, 4])?)?;
    check(unsafe { (api()?.softmax_bwd)(grad_output.as_device_ptr() as _, output.as_device_ptr() as _,
                                        dx.as_device_ptr() as _, rows as u64, cols as u64,
                                        std::ptr::null_mut()) }, "softmax_backward_f32")?;
    Ok(dx)
}

/// `fused_cross_entropy_backward` (cpu_fused_backward.rs:130-170): targets are
/// f32 class indices, as in the reference.
pub fn rocm_cross_entropy_backward_f32(dev: usize, logits: &HipBuffer, targets: &HipBuffer, batch: usize,
                                       classes: usize) -> Result<HipBuffer, RocmError> {
    need(logits, prod(&[batch, classes, 4])?, "cross_entropy_backward logits")?;
    need(targets, prod(&[batch, 4])?, "cross_entropy_backward targets")?;
    set_device(dev)?;
    let g = HipBuffer::zeros(dev, prod(&[batch, classes, 4])?)?;
    check(unsafe { (api()?.ce_bwd)(logits.as_device_ptr() as _, targets.as_device_ptr() as _,
                                   g.as_device_ptr() as _, batch as u64, classes as u64,
                                   std::ptr::null_mut()) }, "cross_entropy_backward_f32")?;
    Ok(g)
}

/// `fused_rms_norm_backward` (cpu_fused_backward.rs:20-81): (grad_input, grad_gamma).
/// The dgamma partial sums need a workspace; this wrapper allocates it.
pub fn rocm_rms_norm_backward_f32(dev: usize, grad_output: &HipBuffer, input: &HipBuffer, gamma: &HipBuffer,
                                  rows: usize, cols: usize, eps: f32)
                                  -> Result<(HipBuffer, HipBuffer), RocmError> {
    need(grad_output, prod(&[rows, cols, 4])?, "rms_norm_backward grad_output")?;
    need(input, prod(&[rows, cols, 4])?, "rms_norm_backward input")?;
    need(gamma, prod(&[cols, 4])?, "rms_norm_backward gamma")?;
    set_device(dev)?;
    let dx = HipBuffer::zeros(dev, prod(&[rows, cols, 4])?)?;
    let dg = HipBuffer::zeros(dev, prod(&[cols, 4])?)?;
    let wsb = unsafe { (api()?.rms_bwd_ws)(rows as u64, cols as u64) } as usize;
    let ws = HipBuffer::zeros(dev, wsb.max(16))?;
    check(unsafe { (api()?.rms_bwd)(grad_output.as_device_ptr() as _, input.as_device_ptr() as _,
                                    gamma.as_device_ptr() as _, dx.as_device_ptr() as _, dg.as_device_ptr() as _,
                                    ws.as_device_ptr() as _, ws.len() as u64, rows as u64, cols as u64, eps,
                                    std::ptr::null_mut()) }, "rms_norm_backward_f32")?;
    Ok((dx, dg))
}

/// The same op for callers that cannot allocate device memory (graph capture, tight loops): no
/// counterpart in the reference.  The caller owns grad_input and grad_gamma; the dgamma partial
/// sums go to the library's fixed per-GPU scratch array (`rocm_rms_norm_backward_noalloc_max_bytes`);
/// calls that overlap on one GPU race.  `stream` is the HIP stream the kernels are enqueued on:
/// the capturing stream under graph capture (the legacy null stream cannot be captured), or null.
pub fn rocm_rms_norm_backward_noalloc_f32(dev: usize, grad_output: &HipBuffer, input: &HipBuffer,
                                          gamma: &HipBuffer, grad_input: &HipBuffer, grad_gamma: &HipBuffer,
                                          rows: usize, cols: usize, eps: f32, stream: Stream)
                                          -> Result<(), RocmError> {
    need(grad_output, prod(&[rows, cols, 4])?, "rms_norm_backward grad_output")?;
    need(input, prod(&[rows, cols, 4])?, "rms_norm_backward input")?;
    need(gamma, prod(&[cols, 4])?, "rms_norm_backward gamma")?;
    need(grad_input, prod(&[rows, cols, 4])?, "rms_norm_backward grad_input")?;
    need(grad_gamma, prod(&[cols, 4])?, "rms_norm_backward grad_gamma")?;
    set_device(dev)?;
    check(unsafe { (api()?.rms_bwd_noalloc)(grad_output.as_device_ptr() as _, input.as_device_ptr() as _,
                                            gamma.as_device_ptr() as _, grad_input.as_device_ptr() as _,
                                            grad_gamma.as_device_ptr() as _, rows as u64, cols as u64, eps,
                                            stream) }, "rms_norm_backward_noalloc_f32")
}

/// Bytes of the fixed scratch array behind `rocm_rms_norm_backward_noalloc_f32`.
pub fn rocm_rms_norm_backward_noalloc_max_bytes() -> Result<usize, RocmError> {
    Ok(unsafe { (api()?.rms_bwd_noalloc_max)() } as usize)
}

/// BitLinear matmul on pre-quant codes: c[m, n] = ((f32)(sum_k trit[m, k] * q[n, k]) * a_scales[m])
/// * q_scales[n], with `BitLinear`'s base-243 weights (pack_weights_ternary,
/// cpu_ternary_matmul.rs:198-240) and the ternary_ternary_matmul epilogue (:188).  Bit-exact.
/// `q`, `q_scales` are what `rocm_rms_norm_quant_i8` returns for the layer input.
pub fn rocm_ternary_matmul_i8(dev: usize, a_packed: &HipBuffer, a_scales: &HipBuffer, q: &HipBuffer,
                              q_scales: &HipBuffer, m: usize, n: usize, k: usize)
                              -> Result<HipBuffer, RocmError> {
    need(a_packed, prod(&[m, k.div_ceil(5)])?, "ternary weights")?;
    need(a_scales, prod(&[m, 4])?, "ternary scales")?;
    need(q, prod(&[n, k])?, "ternary codes")?;
    need(q_scales, prod(&[n, 4])?, "ternary code scales")?;
    set_device(dev)?;
    let c = HipBuffer::zeros(dev, prod(&[m, n, 4])?)?;
    check(unsafe { (api()?.ternary_i8)(a_packed.as_device_ptr() as _, a_scales.as_device_ptr() as _,
                                       q.as_device_ptr() as _, q_scales.as_device_ptr() as _,
                                       c.as_device_ptr() as _, m as u64, n as u64, k as u64,
                                       std::ptr::null_mut()) }, "ternary_matmul_i8")?;
    Ok(c)
}

/// `ternary_matmul` (cpu_ternary_matmul.rs:29-124) on the device: c[m, n] = (sum over k in order of
/// trit[m, k] * b[k, n]) * a_scales[m] with f32 activations b[K, N] (BitLinear::forward passes the
/// transposed input).  The sum is the reference's sequential f32 fold, so c is bit-exact.
pub fn rocm_ternary_matmul_f32(dev: usize, a_packed: &HipBuffer, a_scales: &HipBuffer, b: &HipBuffer,
                               m: usize, n: usize, k: usize) -> Result<HipBuffer, RocmError> {
    need(a_packed, prod(&[m, k.div_ceil(5)])?, "ternary weights")?;
    need(a_scales, prod(&[m, 4])?, "ternary scales")?;
    need(b, prod(&[k, n, 4])?, "ternary activations")?;
    set_device(dev)?;
    let c = HipBuffer::zeros(dev, prod(&[m, n, 4])?)?;
    check(unsafe { (api()?.ternary_f32)(a_packed.as_device_ptr() as _, a_scales.as_device_ptr() as _,
                                        b.as_device_ptr() as _, c.as_device_ptr() as _, m as u64, n as u64,
                                        k as u64, std::ptr::null_mut()) }, "ternary_matmul_f32")?;
    Ok(c)
}

/// `BitLinear::forward` (bit_linear.rs:175-237) in one launch: the layer's input x[batch, in] as
/// stored, output y[batch, out] = ternary_matmul(W, scales, x^T)^T + bias in the layer's layout
/// (the transposes and the bias add of :200-224 need no passes of their own).  Bit-exact.
pub fn rocm_bit_linear_f32(dev: usize, a_packed: &HipBuffer, a_scales: &HipBuffer, x: &HipBuffer,
                           bias: Option<&HipBuffer>, out_features: usize, batch: usize, in_features: usize)
                           -> Result<HipBuffer, RocmError> {
    need(a_packed, prod(&[out_features, in_features.div_ceil(5)])?, "ternary weights")?;
    need(a_scales, prod(&[out_features, 4])?, "ternary scales")?;
    need(x, prod(&[batch, in_features, 4])?, "layer input")?;
    if let Some(b) = bias {
        need(b, prod(&[out_features, 4])?, "bias")?;
    }
    set_device(dev)?;
    let y = HipBuffer::zeros(dev, prod(&[batch, out_features, 4])?)?;
    let bp = bias.map_or(std::ptr::null(), |b| b.as_device_ptr() as *const f32);
    check(unsafe { (api()?.bit_linear_f32)(a_packed.as_device_ptr() as _, a_scales.as_device_ptr() as _,
                                           x.as_device_ptr() as _, bp, y.as_device_ptr() as _,
                                           out_features as u64, batch as u64, in_features as u64,
                                           std::ptr::null_mut()) }, "bit_linear_f32")?;
    Ok(y)
}

/// The BitLinear layer on pre-quant codes (`rocm_rms_norm_quant_i8`'s q[batch, in], q_scales):
/// y[b, o] = c[o, b] + bias[o] with c of `rocm_ternary_matmul_i8`, in the layer's [batch, out]
/// layout.  Bit-exact.
pub fn rocm_bit_linear_i8(dev: usize, a_packed: &HipBuffer, a_scales: &HipBuffer, q: &HipBuffer,
                          q_scales: &HipBuffer, bias: Option<&HipBuffer>, out_features: usize, batch: usize,
                          in_features: usize) -> Result<HipBuffer, RocmError> {
    need(a_packed, prod(&[out_features, in_features.div_ceil(5)])?, "ternary weights")?;
    need(a_scales, prod(&[out_features, 4])?, "ternary scales")?;
    need(q, prod(&[batch, in_features])?, "codes")?;
    need(q_scales, prod(&[batch, 4])?, "code scales")?;
    if let Some(b) = bias {
        need(b, prod(&[out_features, 4])?, "bias")?;
    }
    set_device(dev)?;
    let y = HipBuffer::zeros(dev, prod(&[batch, out_features, 4])?)?;
    let bp = bias.map_or(std::ptr::null(), |b| b.as_device_ptr() as *const f32);
    check(unsafe { (api()?.bit_linear_i8)(a_packed.as_device_ptr() as _, a_scales.as_device_ptr() as _,
                                          q.as_device_ptr() as _, q_scales.as_device_ptr() as _, bp,
                                          y.as_device_ptr() as _, out_features as u64, batch as u64,
                                          in_features as u64, std::ptr::null_mut()) }, "bit_linear_i8")?;
    Ok(y)
}

/// `pack_weights_ternary` (cpu_ternary_matmul.rs:198-240) on the device: f32 weights [m, k] ->
/// (base-243 bytes [m, ceil(k/5)], per-row scales [m]), bit-identical to the CPU function.
pub fn rocm_pack_weights_ternary(dev: usize, w: &HipBuffer, m: usize, k: usize, threshold: f32)
                                 -> Result<(HipBuffer, HipBuffer), RocmError> {
    need(w, prod(&[m, k, 4])?, "weights")?;
    set_device(dev)?;
    let packed = HipBuffer::zeros(dev, prod(&[m, k.div_ceil(5)])?)?;
    let scales = HipBuffer::zeros(dev, prod(&[m, 4])?)?;
    check(unsafe { (api()?.pack_ternary)(w.as_device_ptr() as _, m as u64, k as u64, threshold,
                                         packed.as_device_ptr() as _, scales.as_device_ptr() as _,
                                         std::ptr::null_mut()) }, "pack_weights_ternary")?;
    Ok((packed, scales))
}
