"""Host-side mirror of KORE's ``kore_kernels::rocm`` op API over libkore_hip.so.

The reference's ROCm backend hands raw device buffers (``HipBuffer``,
crates/kore-kernels/src/rocm/memory.rs:15-19) to ``rocm_*`` dispatch functions
that mirror the ``cuda_*`` signatures (crates/kore-kernels/src/rocm/ops.rs:49-70,
crates/kore-kernels/src/cuda/ops.rs).  This module is that layer for the fused
layer ops: the same names, the same argument meaning (device index, buffers,
explicit dims), the same ownership (each op allocates and returns its output
buffer, like ``cuda_rms_norm_f32`` at cuda/ops.rs:527-529) and the same error
type (:class:`RocmError`, crates/kore-kernels/src/rocm/context.rs:95-117).

Device memory and streams come from PyTorch-ROCm (plumbing only); every
computation runs in libkore_hip.so.  Every op also takes an optional ``out=``
buffer so that timed loops allocate nothing.

Sizes are validated on the host before any launch: a buffer smaller than the
dims imply raises ``RocmError.MemoryError`` instead of reaching the GPU.
"""
from __future__ import annotations

from typing import Optional, Tuple

import numpy as np

from . import _lib

try:  # torch is the device-memory provider; importing it is cheap to defer
    import torch
except ImportError:  # pragma: no cover
    torch = None


class RocmError(RuntimeError):
    """Mirror of ``RocmError`` (rocm/context.rs:95-117).

    ``kind`` is one of ``NotAvailable``, ``HipError``, ``LaunchError``,
    ``MemoryError``; ``code`` carries the C status for ``HipError`` /
    ``LaunchError``.
    """

    def __init__(self, kind: str, message: str, code: Optional[int] = None):
        super().__init__(f"{kind}: {message}" + (f" (code {code})" if code is not None else ""))
        self.kind = kind
        self.code = code


def _check(status: int, context: str) -> None:
    """``check_hip`` (rocm/ffi.rs:211-220): map a C status to RocmError."""
    if status == _lib.KORE_HIP_OK:
        return
    text = _lib.status_string(status)
    if status > 0:
        raise RocmError("HipError", f"{context}: {text}", status)
    raise RocmError("LaunchError", f"{context}: {text}", status)


def _require_device(device_idx: int):
    if torch is None or not torch.cuda.is_available():
        raise RocmError("NotAvailable", "no ROCm device visible to this process")
    if device_idx < 0 or device_idx >= torch.cuda.device_count():
        raise RocmError("NotAvailable", f"device {device_idx} does not exist")
    _lib.load()  # fail loudly if the native library is missing
    return torch.device("cuda", device_idx)


class HipBuffer:
    """Raw bytes on one HIP device (``HipBuffer``, rocm/memory.rs:15-146).

    Backed by a torch uint8 tensor, so the caching allocator owns the
    allocation and frees it when the buffer is dropped.
    """

    __slots__ = ("_t", "device_idx")

    def __init__(self, tensor, device_idx: int):
        self._t = tensor
        self.device_idx = device_idx

    # -- constructors (memory.rs:27-91) ------------------------------------
    @classmethod
    def zeros(cls, device_idx: int, nbytes: int) -> "HipBuffer":
        dev = _require_device(device_idx)
        return cls(torch.zeros(int(nbytes), dtype=torch.uint8, device=dev), device_idx)

    @classmethod
    def empty(cls, device_idx: int, nbytes: int) -> "HipBuffer":
        dev = _require_device(device_idx)
        return cls(torch.empty(int(nbytes), dtype=torch.uint8, device=dev), device_idx)

    @classmethod
    def from_host(cls, device_idx: int, data) -> "HipBuffer":
        dev = _require_device(device_idx)
        arr = np.ascontiguousarray(data)
        host = torch.from_numpy(arr.view(np.uint8).reshape(-1).copy())
        return cls(host.to(dev), device_idx)

    @classmethod
    def from_tensor(cls, t) -> "HipBuffer":
        """Wrap an existing contiguous device tensor (no copy)."""
        if not t.is_cuda or not t.is_contiguous():
            raise RocmError("MemoryError", "from_tensor needs a contiguous device tensor")
        return cls(t.view(-1).view(torch.uint8), t.device.index)

    # -- accessors ---------------------------------------------------------
    @property
    def nbytes(self) -> int:
        return self._t.numel()

    @property
    def ptr(self) -> int:
        return self._t.data_ptr() if self._t.numel() else 0

    def tensor(self, dtype=None):
        """View of the bytes as a torch tensor of ``dtype`` (no copy)."""
        return self._t if dtype is None else self._t.view(dtype)

    def to_host(self, dtype=np.uint8) -> np.ndarray:
        """Synchronous D2H copy (``HipBuffer::to_host``)."""
        return self._t.cpu().numpy().view(dtype)


def _stream(device_idx: int) -> int:
    return torch.cuda.current_stream(device_idx).cuda_stream


def _need(buf: HipBuffer, nbytes: int, what: str) -> None:
    if buf.nbytes < nbytes:
        raise RocmError("MemoryError", f"{what}: buffer holds {buf.nbytes} bytes, op needs {nbytes}")


def _out(device_idx: int, out: Optional[HipBuffer], nbytes: int, what: str) -> HipBuffer:
    if out is None:
        return HipBuffer.empty(device_idx, nbytes)
    _need(out, nbytes, what)
    return out


# ---------------------------------------------------------------- RMSNorm
def rocm_rms_norm_f32(device_idx: int, input: HipBuffer, weight: HipBuffer, rows: int, cols: int,
                      eps: float, out: Optional[HipBuffer] = None) -> HipBuffer:
    """``cuda_rms_norm_f32`` (cuda/ops.rs:517-541); bit-exact twin of
    ``fused_rms_norm`` (crates/kore-kernels/src/cpu_fused.rs:160-190)."""
    _require_device(device_idx)
    n = rows * cols * 4
    _need(input, n, "rms_norm input")
    _need(weight, cols * 4, "rms_norm weight")
    o = _out(device_idx, out, n, "rms_norm out")
    _check(_lib.load().kore_hip_rms_norm_f32(input.ptr, weight.ptr, o.ptr, rows, cols, eps,
                                             _stream(device_idx)), "rms_norm_f32")
    return o


def rocm_fused_rms_norm_silu_gate_f32(device_idx: int, input: HipBuffer, gamma: HipBuffer, gate: HipBuffer,
                                      rows: int, cols: int, eps: float,
                                      out: Optional[HipBuffer] = None) -> HipBuffer:
    """``cuda_fused_rms_norm_silu_gate_f32`` (cuda/ops.rs:717-751):
    y = RMSNorm(x) * silu(z), RMSNorm bit-exact as ``rocm_rms_norm_f32``."""
    _require_device(device_idx)
    n = rows * cols * 4
    _need(input, n, "rms_norm_silu_gate input")
    _need(gamma, cols * 4, "rms_norm_silu_gate gamma")
    _need(gate, n, "rms_norm_silu_gate gate")
    o = _out(device_idx, out, n, "rms_norm_silu_gate out")
    _check(_lib.load().kore_hip_rms_norm_silu_gate_f32(input.ptr, gamma.ptr, gate.ptr, o.ptr, rows, cols, eps,
                                                       _stream(device_idx)), "rms_norm_silu_gate_f32")
    return o


# ------------------------------------------------------------ activations
def _unary(name: str, device_idx: int, a: HipBuffer, n: int, out: Optional[HipBuffer]) -> HipBuffer:
    _require_device(device_idx)
    _need(a, n * 4, f"{name} input")
    o = _out(device_idx, out, n * 4, f"{name} out")
    _check(getattr(_lib.load(), f"kore_hip_{name}_f32")(a.ptr, o.ptr, n, _stream(device_idx)), f"{name}_f32")
    return o


def rocm_gelu_f32(device_idx: int, a: HipBuffer, n: int, out: Optional[HipBuffer] = None) -> HipBuffer:
    """``cuda_gelu_f32`` (cuda/ops.rs:197-204); twin of ``kore_nn::activations::gelu``."""
    return _unary("gelu", device_idx, a, n, out)


def rocm_silu_f32(device_idx: int, a: HipBuffer, n: int, out: Optional[HipBuffer] = None) -> HipBuffer:
    """``cuda_silu_f32`` (cuda/ops.rs:206-213); twin of ``kore_nn::activations::silu``."""
    return _unary("silu", device_idx, a, n, out)


def _binary(name: str, device_idx: int, a: HipBuffer, b: HipBuffer, n: int,
            out: Optional[HipBuffer]) -> HipBuffer:
    _require_device(device_idx)
    _need(a, n * 4, f"{name} a")
    _need(b, n * 4, f"{name} b")
    o = _out(device_idx, out, n * 4, f"{name} out")
    _check(getattr(_lib.load(), f"kore_hip_{name}_f32")(a.ptr, b.ptr, o.ptr, n, _stream(device_idx)),
           f"{name}_f32")
    return o


def rocm_mul_f32(device_idx: int, a: HipBuffer, b: HipBuffer, n: int,
                 out: Optional[HipBuffer] = None) -> HipBuffer:
    """``cuda_mul_f32`` (cuda/ops.rs:100-108); twin of ``Tensor::mul``."""
    return _binary("mul", device_idx, a, b, n, out)


def rocm_swiglu_f32(device_idx: int, gate: HipBuffer, up: HipBuffer, n: int,
                    out: Optional[HipBuffer] = None) -> HipBuffer:
    """silu(gate) * up in one pass (the reference composes silu then mul,
    crates/kore-serve/src/layered/engine.rs:633-643)."""
    return _binary("swiglu", device_idx, gate, up, n, out)


# ------------------------------------------------------------------- RoPE
def rope_inv_freq_host(head_dim: int, theta: float) -> np.ndarray:
    """Host table 1/theta^(2i/D) (engine.rs:694-700), computed by the library."""
    half = head_dim // 2
    arr = np.zeros(max(half, 1), dtype=np.float32)
    _check(_lib.load().kore_hip_rope_inv_freq_f32(arr.ctypes.data, head_dim, theta), "rope_inv_freq_f32")
    return arr[:half]


def rocm_rope_inv_freq_f32(device_idx: int, head_dim: int, theta: float) -> HipBuffer:
    """Plays the role of ``cuda_rope_freqs_f32`` (cuda/ops.rs:549-567): the
    per-dimension table the rope kernel consumes, uploaded once."""
    return HipBuffer.from_host(device_idx, rope_inv_freq_host(head_dim, theta))


def rocm_rope_f32(device_idx: int, data: HipBuffer, inv_freq: HipBuffer, batch: int, seq_len: int,
                  num_heads: int, head_dim: int, start_pos: int = 0, interleaved: bool = False) -> None:
    """``cuda_rope_f32`` (cuda/ops.rs:572-599), in place on
    [batch, seq_len, num_heads, head_dim]; half-split pairs by default
    (crates/kore-edge/src/ops/rope.rs:9-36), interleaved pairs as
    kore-serve's ``apply_rope`` (engine.rs:706-727)."""
    _require_device(device_idx)
    _need(data, batch * seq_len * num_heads * head_dim * 4, "rope data")
    _need(inv_freq, (head_dim // 2) * 4, "rope inv_freq")
    _check(_lib.load().kore_hip_rope_f32(data.ptr, inv_freq.ptr, batch, seq_len, num_heads, head_dim,
                                         start_pos, int(bool(interleaved)), _stream(device_idx)), "rope_f32")


def rocm_rope_qk_f32(device_idx: int, q: HipBuffer, k: HipBuffer, inv_freq: HipBuffer, batch: int,
                     seq_len: int, q_heads: int, k_heads: int, head_dim: int, start_pos: int = 0,
                     interleaved: bool = False) -> None:
    """Q and K of one layer rotated in one launch (same results as two
    ``rocm_rope_f32`` calls)."""
    _require_device(device_idx)
    _need(q, batch * seq_len * q_heads * head_dim * 4, "rope q")
    _need(k, batch * seq_len * k_heads * head_dim * 4, "rope k")
    _need(inv_freq, (head_dim // 2) * 4, "rope inv_freq")
    _check(_lib.load().kore_hip_rope_qk_f32(q.ptr, k.ptr, inv_freq.ptr, batch, seq_len, q_heads, k_heads,
                                            head_dim, start_pos, int(bool(interleaved)), _stream(device_idx)),
           "rope_qk_f32")


# -------------------------------------------------------------- Embedding
def rocm_embedding_f32(device_idx: int, table: HipBuffer, ids: HipBuffer, n_ids: int, vocab: int, dim: int,
                       out: Optional[HipBuffer] = None) -> HipBuffer:
    """``Embedding::lookup`` (crates/kore-nn/src/embedding.rs:55-72) on the
    device: ids are u32/i32, out-of-range ids give zero rows."""
    _require_device(device_idx)
    _need(table, vocab * dim * 4, "embedding table")
    _need(ids, n_ids * 4, "embedding ids")
    o = _out(device_idx, out, n_ids * dim * 4, "embedding out")
    _check(_lib.load().kore_hip_embedding_f32(table.ptr, ids.ptr, o.ptr, n_ids, vocab, dim, _stream(device_idx)),
           "embedding_f32")
    return o


def rocm_embedding_forward_f32(device_idx: int, table: HipBuffer, ids: HipBuffer, n_ids: int, vocab: int,
                               dim: int, out: Optional[HipBuffer] = None) -> HipBuffer:
    """``Embedding::forward`` (crates/kore-nn/src/embedding.rs:91-98) on the
    device: ids are an f32 buffer converted like Rust's ``v as usize`` (NaN
    and values below 1 -> 0, saturating), then looked up as ``lookup``."""
    _require_device(device_idx)
    _need(table, vocab * dim * 4, "embedding table")
    _need(ids, n_ids * 4, "embedding ids")
    o = _out(device_idx, out, n_ids * dim * 4, "embedding out")
    _check(_lib.load().kore_hip_embedding_forward_f32(table.ptr, ids.ptr, o.ptr, n_ids, vocab, dim,
                                                      _stream(device_idx)), "embedding_forward_f32")
    return o


# ----------------------------------------------------- BitLinear pre-quant
def rocm_rms_norm_quant_i8(device_idx: int, input: HipBuffer, weight: HipBuffer, rows: int, cols: int,
                           eps: float, out_q: Optional[HipBuffer] = None,
                           out_scale: Optional[HipBuffer] = None) -> Tuple[HipBuffer, HipBuffer]:
    """RMSNorm + per-row absmax int8 in one pass; returns (q int8[rows, cols],
    scale f32[rows]) with x ~= q * scale."""
    _require_device(device_idx)
    _need(input, rows * cols * 4, "prequant input")
    _need(weight, cols * 4, "prequant weight")
    q = _out(device_idx, out_q, rows * cols, "prequant q")
    s = _out(device_idx, out_scale, rows * 4, "prequant scale")
    _check(_lib.load().kore_hip_rms_norm_quant_i8(input.ptr, weight.ptr, q.ptr, s.ptr, rows, cols, eps,
                                                  _stream(device_idx)), "rms_norm_quant_i8")
    return q, s


__all__ = [
    "RocmError", "HipBuffer", "rocm_rms_norm_f32", "rocm_gelu_f32", "rocm_silu_f32", "rocm_mul_f32",
    "rocm_swiglu_f32", "rope_inv_freq_host", "rocm_rope_inv_freq_f32", "rocm_rope_f32", "rocm_rope_qk_f32",
    "rocm_embedding_f32", "rocm_embedding_forward_f32", "rocm_rms_norm_quant_i8", "rocm_fused_rms_norm_silu_gate_f32",
]


# ---------------------------------------------------------------- softmax
def rocm_softmax_f32(device_idx: int, a: HipBuffer, rows: int, cols: int,
                     out: Optional[HipBuffer] = None) -> HipBuffer:
    """``cuda_softmax_f32`` (cuda/ops.rs:486-511); twin of ``fused_softmax``
    (cpu_fused.rs:195-231)."""
    _require_device(device_idx)
    n = rows * cols * 4
    _need(a, n, "softmax input")
    o = _out(device_idx, out, n, "softmax out")
    _check(_lib.load().kore_hip_softmax_f32(a.ptr, o.ptr, rows, cols, _stream(device_idx)), "softmax_f32")
    return o


def rocm_softmax_causal_f32(device_idx: int, a: HipBuffer, rows: int, cols: int, seq_offset: int = 0,
                            out: Optional[HipBuffer] = None) -> HipBuffer:
    """The ``softmax_causal_f32`` kernel (cuda/kernels/softmax.cu:88-157): row r
    keeps columns < seq_offset + r + 1."""
    _require_device(device_idx)
    n = rows * cols * 4
    _need(a, n, "softmax_causal input")
    o = _out(device_idx, out, n, "softmax_causal out")
    _check(_lib.load().kore_hip_softmax_causal_f32(a.ptr, o.ptr, rows, cols, seq_offset, _stream(device_idx)),
           "softmax_causal_f32")
    return o


def rocm_softmax_backward_f32(device_idx: int, grad_output: HipBuffer, output: HipBuffer, rows: int, cols: int,
                              out: Optional[HipBuffer] = None) -> HipBuffer:
    """``fused_softmax_backward`` (cpu_fused_backward.rs:86-115) on the device:
    grad_input = y * (dy - sum(y * dy))."""
    _require_device(device_idx)
    n = rows * cols * 4
    _need(grad_output, n, "softmax_backward grad_output")
    _need(output, n, "softmax_backward output")
    o = _out(device_idx, out, n, "softmax_backward grad_input")
    _check(_lib.load().kore_hip_softmax_backward_f32(grad_output.ptr, output.ptr, o.ptr, rows, cols,
                                                     _stream(device_idx)), "softmax_backward_f32")
    return o


def rocm_cross_entropy_backward_f32(device_idx: int, logits: HipBuffer, targets: HipBuffer, batch: int,
                                    num_classes: int, out: Optional[HipBuffer] = None) -> HipBuffer:
    """``fused_cross_entropy_backward`` (cpu_fused_backward.rs:130-170) on the
    device: (softmax(logits) - one_hot(targets)) / batch; targets are f32."""
    _require_device(device_idx)
    n = batch * num_classes * 4
    _need(logits, n, "cross_entropy_backward logits")
    _need(targets, batch * 4, "cross_entropy_backward targets")
    o = _out(device_idx, out, n, "cross_entropy_backward grad")
    _check(_lib.load().kore_hip_cross_entropy_backward_f32(logits.ptr, targets.ptr, o.ptr, batch, num_classes,
                                                           _stream(device_idx)), "cross_entropy_backward_f32")
    return o


# ------------------------------------------------------- RMSNorm backward
def rocm_rms_norm_backward_workspace_bytes(rows: int, cols: int) -> int:
    """Device scratch ``rocm_rms_norm_backward_f32`` needs for (rows, cols)."""
    return int(_lib.load().kore_hip_rms_norm_backward_workspace_bytes(rows, cols))


def rocm_rms_norm_backward_f32(device_idx: int, grad_output: HipBuffer, input: HipBuffer, gamma: HipBuffer,
                               rows: int, cols: int, eps: float, workspace: Optional[HipBuffer] = None,
                               grad_input: Optional[HipBuffer] = None, grad_gamma: Optional[HipBuffer] = None):
    """``fused_rms_norm_backward`` (cpu_fused_backward.rs:20-81) on the device
    -> (grad_input, grad_gamma).  The workspace is allocated when not given."""
    _require_device(device_idx)
    n = rows * cols * 4
    _need(grad_output, n, "rms_norm_backward grad_output")
    _need(input, n, "rms_norm_backward input")
    _need(gamma, cols * 4, "rms_norm_backward gamma")
    gx = _out(device_idx, grad_input, n, "rms_norm_backward grad_input")
    gg = _out(device_idx, grad_gamma, cols * 4, "rms_norm_backward grad_gamma")
    wsb = rocm_rms_norm_backward_workspace_bytes(rows, cols)
    ws = workspace if workspace is not None else HipBuffer.empty(device_idx, max(wsb, 16))
    _check(_lib.load().kore_hip_rms_norm_backward_f32(grad_output.ptr, input.ptr, gamma.ptr, gx.ptr, gg.ptr, ws.ptr,
                                                      ws.nbytes, rows, cols, eps, _stream(device_idx)),
           "rms_norm_backward_f32")
    return gx, gg


# ------------------------------------------------------- ternary (BitLinear)
def rocm_ternary_matmul_i8(device_idx: int, a_packed: HipBuffer, a_scales: HipBuffer, q: HipBuffer,
                           q_scales: HipBuffer, m: int, n: int, k: int,
                           out: Optional[HipBuffer] = None) -> HipBuffer:
    """BitLinear matmul on pre-quant codes: c[m, n] = ((float)(sum_k trit[m, k]
    * q[n, k]) * a_scales[m]) * q_scales[n], with the base-243 weights of
    ``pack_weights_ternary`` (cpu_ternary_matmul.rs:198-240) and the epilogue
    of ``ternary_ternary_matmul`` (cpu_ternary_matmul.rs:188)."""
    _require_device(device_idx)
    _need(a_packed, m * ((k + 4) // 5), "ternary weights")
    _need(a_scales, m * 4, "ternary scales")
    _need(q, n * k, "ternary codes")
    _need(q_scales, n * 4, "ternary code scales")
    c = _out(device_idx, out, m * n * 4, "ternary out")
    _check(_lib.load().kore_hip_ternary_matmul_i8(a_packed.ptr, a_scales.ptr, q.ptr, q_scales.ptr, c.ptr, m, n, k,
                                                  _stream(device_idx)), "ternary_matmul_i8")
    return c


def rocm_ternary_matmul_f32(device_idx: int, a_packed: HipBuffer, a_scales: HipBuffer, b: HipBuffer, m: int,
                            n: int, k: int, out: Optional[HipBuffer] = None) -> HipBuffer:
    """``ternary_matmul`` (cpu_ternary_matmul.rs:29-124, as ``BitLinear::forward``
    calls it): c[m, n] = (sum over k in order of trit[m, k] * b[k, n]) *
    a_scales[m] with f32 activations b[K, N], the sum the reference's
    sequential f32 fold (bit-exact)."""
    _require_device(device_idx)
    _need(a_packed, m * ((k + 4) // 5), "ternary weights")
    _need(a_scales, m * 4, "ternary scales")
    _need(b, k * n * 4, "ternary activations")
    c = _out(device_idx, out, m * n * 4, "ternary out")
    _check(_lib.load().kore_hip_ternary_matmul_f32(a_packed.ptr, a_scales.ptr, b.ptr, c.ptr, m, n, k,
                                                   _stream(device_idx)), "ternary_matmul_f32")
    return c


def rocm_bit_linear_f32(device_idx: int, a_packed: HipBuffer, a_scales: HipBuffer, x: HipBuffer,
                        bias: Optional[HipBuffer], out_features: int, batch: int, in_features: int,
                        out: Optional[HipBuffer] = None) -> HipBuffer:
    """``BitLinear::forward`` (bit_linear.rs:175-237) in one launch: y[batch,
    out] = ternary_matmul(W, scales, x^T)^T + bias with the layer's input
    x[batch, in] as stored and the output in the layer's layout; bias None for
    a layer without bias (bit-exact)."""
    _require_device(device_idx)
    _need(a_packed, out_features * ((in_features + 4) // 5), "ternary weights")
    _need(a_scales, out_features * 4, "ternary scales")
    _need(x, batch * in_features * 4, "layer input")
    if bias is not None:
        _need(bias, out_features * 4, "bias")
    y = _out(device_idx, out, batch * out_features * 4, "layer output")
    _check(_lib.load().kore_hip_bit_linear_f32(a_packed.ptr, a_scales.ptr, x.ptr, bias.ptr if bias else None, y.ptr,
                                               out_features, batch, in_features, _stream(device_idx)),
           "bit_linear_f32")
    return y


def rocm_bit_linear_i8(device_idx: int, a_packed: HipBuffer, a_scales: HipBuffer, q: HipBuffer, q_scales: HipBuffer,
                       bias: Optional[HipBuffer], out_features: int, batch: int, in_features: int,
                       out: Optional[HipBuffer] = None) -> HipBuffer:
    """The BitLinear layer on pre-quant codes q[batch, in] / q_scales[batch]:
    y[b, o] = c[o, b] + bias[o] with c of ``rocm_ternary_matmul_i8``, in the
    layer's [batch, out] layout (bit-exact)."""
    _require_device(device_idx)
    _need(a_packed, out_features * ((in_features + 4) // 5), "ternary weights")
    _need(a_scales, out_features * 4, "ternary scales")
    _need(q, batch * in_features, "codes")
    _need(q_scales, batch * 4, "code scales")
    if bias is not None:
        _need(bias, out_features * 4, "bias")
    y = _out(device_idx, out, batch * out_features * 4, "layer output")
    _check(_lib.load().kore_hip_bit_linear_i8(a_packed.ptr, a_scales.ptr, q.ptr, q_scales.ptr,
                                              bias.ptr if bias else None, y.ptr, out_features, batch, in_features,
                                              _stream(device_idx)), "bit_linear_i8")
    return y


def rocm_pack_weights_ternary(device_idx: int, w: HipBuffer, m: int, k: int, threshold: float,
                              packed: Optional[HipBuffer] = None,
                              scales: Optional[HipBuffer] = None) -> Tuple[HipBuffer, HipBuffer]:
    """``pack_weights_ternary`` (cpu_ternary_matmul.rs:198-240): f32 weights
    w[m, k] -> (base-243 packed bytes [m, ceil(k/5)], per-row scales [m]),
    bit-exact."""
    _require_device(device_idx)
    _need(w, m * k * 4, "weights")
    kp = (k + 4) // 5
    p = _out(device_idx, packed, m * kp, "packed weights")
    sc = _out(device_idx, scales, m * 4, "weight scales")
    _check(_lib.load().kore_hip_pack_weights_ternary(w.ptr, m, k, threshold, p.ptr, sc.ptr, _stream(device_idx)),
           "pack_weights_ternary")
    return p, sc


__all__ += ["rocm_ternary_matmul_i8", "rocm_ternary_matmul_f32", "rocm_bit_linear_f32", "rocm_bit_linear_i8",
            "rocm_pack_weights_ternary"]
