"""numpy front end of the C oracle (kore_oracle.c).  TEST INFRASTRUCTURE ONLY.

Each wrapper names the reference function the C code restates; see
kore_oracle.h for file:line citations.  Inputs are converted to contiguous
float32 / uint32 arrays; outputs are new arrays.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "libkore_oracle.so")

_c = ctypes
_sz = _c.c_size_t
_p = _c.c_void_p
_f = _c.c_float
_i = _c.c_int

_SIGS = {
    "kore_oracle_rms_norm_f32": (None, [_p, _p, _p, _sz, _sz, _f]),
    "kore_oracle_gelu_f32": (None, [_p, _p, _sz]),
    "kore_oracle_silu_f32": (None, [_p, _p, _sz]),
    "kore_oracle_mul_f32": (None, [_p, _p, _p, _sz, _i]),
    "kore_oracle_swiglu_f32": (None, [_p, _p, _p, _p, _sz, _i]),
    "kore_oracle_rope_inv_freq_f32": (None, [_p, _sz, _f]),
    "kore_oracle_rope_f32": (None, [_p, _sz, _sz, _sz, _sz, _f]),
    "kore_oracle_rope_interleaved_f32": (None, [_p, _sz, _sz, _sz, _sz, _p]),
    "kore_oracle_embedding_f32": (None, [_p, _p, _p, _sz, _sz, _sz]),
    "kore_oracle_embedding_forward_f32": (None, [_p, _p, _p, _sz, _sz, _sz]),
    "kore_oracle_f32_as_usize": (_c.c_uint64, [_f]),
    "kore_oracle_silu_stable_f32": (None, [_p, _p, _sz]),
    "kore_oracle_swiglu_serve_f32": (None, [_p, _p, _p, _sz]),
    "kore_oracle_rms_norm_quant_i8": (None, [_p, _p, _p, _p, _sz, _sz, _f]),
    "kore_oracle_quant_code": (_c.c_int8, [_f, _f]),
    "kore_oracle_rms_norm_silu_gate_f32": (None, [_p, _p, _p, _p, _sz, _sz, _f]),
    "kore_oracle_softmax_f32": (None, [_p, _p, _sz, _sz]),
    "kore_oracle_softmax_causal_f32": (None, [_p, _p, _sz, _sz, _sz]),
    "kore_oracle_softmax_backward_f32": (None, [_p, _p, _p, _sz, _sz]),
    "kore_oracle_cross_entropy_backward_f32": (None, [_p, _p, _p, _sz, _sz]),
    "kore_oracle_rms_norm_backward_f32": (None, [_p, _p, _p, _p, _p, _sz, _sz, _f]),
    "kore_oracle_decode_trits": (None, [_c.c_uint8, _p]),
    "kore_oracle_encode_trits": (_c.c_uint8, [_p]),
    "kore_oracle_pack_weights_ternary": (None, [_p, _sz, _sz, _f, _p, _p]),
    "kore_oracle_ternary_matmul_f32": (None, [_p, _p, _p, _p, _sz, _sz, _sz]),
    "kore_oracle_ternary_matmul_i8": (None, [_p, _p, _p, _p, _p, _sz, _sz, _sz]),
}

_lib = None


def build() -> None:
    """Compile the oracle with its Makefile (gcc, no FMA contraction)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        l = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def rms_norm(x, gamma, eps: float) -> np.ndarray:
    """fused_rms_norm (crates/kore-kernels/src/cpu_fused.rs:160-190) over the last axis."""
    x = _f32(x)
    g = _f32(gamma)
    cols = x.shape[-1]
    rows = x.size // cols if cols else 0
    y = np.empty_like(x)
    lib().kore_oracle_rms_norm_f32(_ptr(x), _ptr(g), _ptr(y), rows, cols, eps)
    return y


def gelu(x) -> np.ndarray:
    """kore_nn::activations::gelu (crates/kore-nn/src/activations.rs:14-32)."""
    x = _f32(x)
    y = np.empty_like(x)
    lib().kore_oracle_gelu_f32(_ptr(x), _ptr(y), x.size)
    return y


def silu(x) -> np.ndarray:
    """kore_nn::activations::silu (crates/kore-nn/src/activations.rs:35-45)."""
    x = _f32(x)
    y = np.empty_like(x)
    lib().kore_oracle_silu_f32(_ptr(x), _ptr(y), x.size)
    return y


def mul(a, b, threads: int = 1) -> np.ndarray:
    """Tensor::mul same-shape path (crates/kore-core/src/ops/arithmetic.rs:482-509)."""
    a = _f32(a)
    b = _f32(b)
    out = np.empty_like(a)
    lib().kore_oracle_mul_f32(_ptr(a), _ptr(b), _ptr(out), a.size, threads)
    return out


def swiglu(gate, up, threads: int = 1) -> np.ndarray:
    """silu(gate) then Tensor::mul(up) (crates/kore-serve/src/layered/engine.rs:633-643)."""
    g = _f32(gate)
    u = _f32(up)
    out = np.empty_like(g)
    tmp = np.empty_like(g)
    lib().kore_oracle_swiglu_f32(_ptr(g), _ptr(u), _ptr(out), _ptr(tmp), g.size, threads)
    return out


def rope_inv_freq(head_dim: int, base: float) -> np.ndarray:
    """precompute_rope_inv_freq (crates/kore-serve/src/layered/engine.rs:694-700)."""
    out = np.zeros(max(head_dim // 2, 1), dtype=np.float32)
    lib().kore_oracle_rope_inv_freq_f32(_ptr(out), head_dim, base)
    return out[: head_dim // 2]


def rope(data, start_pos: int, base: float, interleaved: bool = False) -> np.ndarray:
    """RoPE on data[..., seq, heads, head_dim] (leading axes = batch, same
    positions per batch entry).  Half-split: kore_edge apply_rope
    (crates/kore-edge/src/ops/rope.rs:9-36); interleaved: kore-serve apply_rope
    (crates/kore-serve/src/layered/engine.rs:706-727)."""
    d = _f32(data).copy()
    seq, heads, hd = d.shape[-3:]
    batch = d.size // (seq * heads * hd) if d.size else 0
    inv = rope_inv_freq(hd, base)
    stride = seq * heads * hd
    for b in range(batch):
        view = d.reshape(-1)[b * stride:(b + 1) * stride]
        ptr = view.ctypes.data
        if interleaved:
            lib().kore_oracle_rope_interleaved_f32(ptr, seq, heads, hd, start_pos, _ptr(inv))
        else:
            lib().kore_oracle_rope_f32(ptr, seq, heads, hd, start_pos, base)
    return d


def embedding(table, ids) -> np.ndarray:
    """Embedding::lookup (crates/kore-nn/src/embedding.rs:55-72) /
    embedding_lookup (crates/kore-edge/src/ops/embedding.rs:8-27)."""
    t = _f32(table)
    vocab, dim = t.shape
    i = np.ascontiguousarray(ids).astype(np.int64).astype(np.uint32)  # i32 -> u32 bit pattern
    out = np.empty((i.size, dim), dtype=np.float32)
    lib().kore_oracle_embedding_f32(_ptr(t), _ptr(i), _ptr(out), i.size, vocab, dim)
    return out


def embedding_forward(table, ids_f32) -> np.ndarray:
    """Embedding::forward (crates/kore-nn/src/embedding.rs:91-98): f32 ids
    cast with Rust's ``as usize``, then ``lookup``."""
    t = _f32(table)
    vocab, dim = t.shape
    i = _f32(ids_f32).reshape(-1)
    out = np.empty((i.size, dim), dtype=np.float32)
    lib().kore_oracle_embedding_forward_f32(_ptr(t), _ptr(i), _ptr(out), i.size, vocab, dim)
    return out


def f32_as_usize(v: float) -> int:
    """Rust ``v as usize`` for one f32 (64-bit target)."""
    return int(lib().kore_oracle_f32_as_usize(v))


def silu_stable(x) -> np.ndarray:
    """kore-serve's two-branch silu (crates/kore-serve/src/layered/engine.rs:828-842)."""
    a = _f32(x)
    y = np.empty_like(a)
    lib().kore_oracle_silu_stable_f32(_ptr(a), _ptr(y), a.size)
    return y


def swiglu_serve(gate, up) -> np.ndarray:
    """silu_stable(gate) * up, as apply_transformer_block composes it
    (crates/kore-serve/src/layered/engine.rs:640-643)."""
    g, u = _f32(gate), _f32(up)
    y = np.empty_like(g)
    lib().kore_oracle_swiglu_serve_f32(_ptr(g), _ptr(u), _ptr(y), g.size)
    return y


def rms_norm_quant_i8(x, gamma, eps: float):
    """fused_rms_norm + per-row absmax int8 (composition defined in kore_oracle.h)."""
    x = _f32(x)
    g = _f32(gamma)
    cols = x.shape[-1]
    rows = x.size // cols if cols else 0
    q = np.empty(x.shape, dtype=np.int8)
    s = np.empty(x.shape[:-1], dtype=np.float32)
    lib().kore_oracle_rms_norm_quant_i8(_ptr(x), _ptr(g), _ptr(q), _ptr(s), rows, cols, eps)
    return q, s


def rms_norm_silu_gate(x, gamma, z, eps: float) -> np.ndarray:
    """RMSNorm(x) * silu(z) (crates/kore-kernels/src/cpu_fused.rs:451-483)."""
    x = _f32(x)
    g = _f32(gamma)
    zz = _f32(z)
    cols = x.shape[-1]
    rows = x.size // cols if cols else 0
    y = np.empty_like(x)
    lib().kore_oracle_rms_norm_silu_gate_f32(_ptr(x), _ptr(g), _ptr(zz), _ptr(y), rows, cols, eps)
    return y


def quant_code(xn: float, amax: float) -> int:
    return int(lib().kore_oracle_quant_code(xn, amax))


__all__ = ["build", "lib", "rms_norm", "gelu", "silu", "mul", "swiglu", "rope_inv_freq", "rope", "embedding",
           "embedding_forward", "f32_as_usize", "silu_stable", "swiglu_serve",
           "rms_norm_quant_i8", "rms_norm_silu_gate", "quant_code", "softmax", "softmax_causal",
           "softmax_backward", "rms_norm_backward", "cross_entropy_backward", "decode_trits", "encode_trits",
           "pack_weights_ternary", "ternary_matmul", "ternary_matmul_i8", "unpack_trits", "bit_linear_forward",
           "bit_linear_i8"]


def _rows_cols(x: np.ndarray):
    cols = x.shape[-1] if x.ndim else 1
    return (x.size // cols if cols else 0), cols


def softmax(x) -> np.ndarray:
    """cpu_fused.rs:195-231 (fused_softmax) over the last dimension."""
    x = _f32(x)
    y = np.empty_like(x)
    rows, cols = _rows_cols(x)
    lib().kore_oracle_softmax_f32(_ptr(x), _ptr(y), rows, cols)
    return y


def softmax_causal(x, seq_offset: int = 0) -> np.ndarray:
    """softmax.cu:88-157 (softmax_causal_f32): row r keeps columns < seq_offset + r + 1."""
    x = _f32(x)
    y = np.empty_like(x)
    rows, cols = _rows_cols(x)
    lib().kore_oracle_softmax_causal_f32(_ptr(x), _ptr(y), rows, cols, seq_offset)
    return y


def softmax_backward(dy, y) -> np.ndarray:
    """cpu_fused_backward.rs:86-115: dx = y * (dy - sum(y*dy))."""
    dy, y = _f32(dy), _f32(y)
    dx = np.empty_like(y)
    rows, cols = _rows_cols(y)
    lib().kore_oracle_softmax_backward_f32(_ptr(dy), _ptr(y), _ptr(dx), rows, cols)
    return dx


def rms_norm_backward(dy, x, gamma, eps: float):
    """cpu_fused_backward.rs:20-81 -> (dx, dgamma)."""
    dy, x, gamma = _f32(dy), _f32(x), _f32(gamma)
    rows, cols = _rows_cols(x)
    dx = np.empty_like(x)
    dgamma = np.empty(cols, np.float32)
    lib().kore_oracle_rms_norm_backward_f32(_ptr(dy), _ptr(x), _ptr(gamma), _ptr(dx), _ptr(dgamma), rows, cols, eps)
    return dx, dgamma


def cross_entropy_backward(logits, targets) -> np.ndarray:
    """cpu_fused_backward.rs:130-170: (softmax(logits) - one_hot(targets)) / batch."""
    l, t = _f32(logits), _f32(targets)
    batch, classes = l.shape
    g = np.empty_like(l)
    lib().kore_oracle_cross_entropy_backward_f32(_ptr(l), _ptr(t), _ptr(g), batch, classes)
    return g


# ------------------------------------------------------------------ ternary
def decode_trits(byte: int) -> np.ndarray:
    """encoder.rs:89-95: base-243 byte -> 5 trits in {-1, 0, 1}."""
    out = np.zeros(5, np.int8)
    lib().kore_oracle_decode_trits(int(byte), _ptr(out))
    return out


def encode_trits(trits) -> int:
    """encoder.rs:73-86: 5 trits -> base-243 byte."""
    t = np.ascontiguousarray(trits, dtype=np.int8)
    return int(lib().kore_oracle_encode_trits(_ptr(t)))


def pack_weights_ternary(w, threshold: float):
    """cpu_ternary_matmul.rs:198-240 -> (packed uint8[m, ceil(k/5)], scales f32[m])."""
    w = _f32(w)
    m, k = w.shape
    packed = np.empty((m, (k + 4) // 5), np.uint8)
    scales = np.empty(m, np.float32)
    lib().kore_oracle_pack_weights_ternary(_ptr(w), m, k, threshold, _ptr(packed), _ptr(scales))
    return packed, scales


def ternary_matmul(packed, scales, b, m: int, n: int, k: int) -> np.ndarray:
    """cpu_ternary_matmul.rs:29-124: c[m, n] = scale[m] * sum_k trit[m, k] * b[k, n]."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    scales, b = _f32(scales), _f32(b)
    c = np.empty((m, n), np.float32)
    lib().kore_oracle_ternary_matmul_f32(_ptr(packed), _ptr(scales), _ptr(b), _ptr(c), m, n, k)
    return c


def ternary_matmul_i8(packed, scales, q, q_scales, m: int, n: int, k: int) -> np.ndarray:
    """c[m, n] = ((float)(sum_k trit[m, k] * q[n, k]) * scales[m]) * q_scales[n]
    (integer dot exact; epilogue of cpu_ternary_matmul.rs:188)."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    q = np.ascontiguousarray(q, dtype=np.int8)
    scales, q_scales = _f32(scales), _f32(q_scales)
    c = np.empty((m, n), np.float32)
    lib().kore_oracle_ternary_matmul_i8(_ptr(packed), _ptr(scales), _ptr(q), _ptr(q_scales), _ptr(c), m, n, k)
    return c


def bit_linear_forward(packed, scales, x, bias, out_features: int, batch: int, in_features: int) -> np.ndarray:
    """BitLinear::forward (crates/kore-nn/src/bit_linear.rs:175-237) composed
    as the reference composes it: input_t = x^T made contiguous (:200),
    output = ternary_matmul(packed, scales, input_t, out, batch, in) (:202-209),
    transposed back to [batch, out] (:213), then output.add(bias) (:217-219),
    an f32 add per element broadcasting bias[out] over the batch."""
    xt = np.ascontiguousarray(_f32(x).reshape(batch, in_features).T)
    y = np.ascontiguousarray(ternary_matmul(packed, scales, xt, out_features, batch, in_features).T)
    if bias is not None:
        y = (y + _f32(bias).reshape(1, out_features)).astype(np.float32)
    return y


def bit_linear_i8(packed, scales, q, q_scales, bias, out_features: int, batch: int, in_features: int) -> np.ndarray:
    """The BitLinear layer on pre-quant codes, composed like bit_linear_forward
    with ternary_matmul_i8 in place of ternary_matmul: y = c^T + bias."""
    y = np.ascontiguousarray(ternary_matmul_i8(packed, scales, q, q_scales, out_features, batch, in_features).T)
    if bias is not None:
        y = (y + _f32(bias).reshape(1, out_features)).astype(np.float32)
    return y


def unpack_trits(packed, k: int) -> np.ndarray:
    """All rows of a packed matrix as int8 trits [m, k] (decode_trits per byte, truncated to k)."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    lut = np.stack([decode_trits(b) for b in range(256)])
    return lut[packed].reshape(packed.shape[0], -1)[:, :k]
