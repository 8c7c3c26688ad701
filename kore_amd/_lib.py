"""ctypes binding of libkore_hip.so (the C ABI declared in include/kore_hip.h).

The library is built in-tree by ``kore_amd/csrc/Makefile`` (``__graft_entry__.build``).
There is no fallback: if the shared object is missing or fails to load, every
op raises :class:`KoreLibraryError` -- the device path never silently routes
to CPU code.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("KORE_HIP_LIB", os.path.join(_HERE, "libkore_hip.so"))

KORE_HIP_OK = 0
KORE_HIP_ERR_NULL_PTR = -1
KORE_HIP_ERR_BAD_DIM = -2
KORE_HIP_ERR_OVERFLOW = -3
KORE_HIP_ERR_ALIAS = -4
KORE_HIP_ERR_SCRATCH = -5

_u64 = ctypes.c_uint64
_u32 = ctypes.c_uint32
_f32 = ctypes.c_float
_ptr = ctypes.c_void_p
_int = ctypes.c_int

# name -> argtypes (all return int status)
SIGNATURES = {
    "kore_hip_version": [],
    "kore_hip_rms_norm_f32": [_ptr, _ptr, _ptr, _u64, _u64, _f32, _ptr],
    "kore_hip_gelu_f32": [_ptr, _ptr, _u64, _ptr],
    "kore_hip_silu_f32": [_ptr, _ptr, _u64, _ptr],
    "kore_hip_mul_f32": [_ptr, _ptr, _ptr, _u64, _ptr],
    "kore_hip_swiglu_f32": [_ptr, _ptr, _ptr, _u64, _ptr],
    "kore_hip_rope_inv_freq_f32": [_ptr, _u32, _f32],
    "kore_hip_rope_f32": [_ptr, _ptr, _u64, _u64, _u32, _u32, _u64, _int, _ptr],
    "kore_hip_rope_qk_f32": [_ptr, _ptr, _ptr, _u64, _u64, _u32, _u32, _u32, _u64, _int, _ptr],
    "kore_hip_embedding_f32": [_ptr, _ptr, _ptr, _u64, _u64, _u64, _ptr],
    "kore_hip_embedding_forward_f32": [_ptr, _ptr, _ptr, _u64, _u64, _u64, _ptr],
    "kore_hip_rms_norm_quant_i8": [_ptr, _ptr, _ptr, _ptr, _u64, _u64, _f32, _ptr],
    "kore_hip_rms_norm_silu_gate_f32": [_ptr, _ptr, _ptr, _ptr, _u64, _u64, _f32, _ptr],
    "kore_hip_softmax_f32": [_ptr, _ptr, _u64, _u64, _ptr],
    "kore_hip_softmax_causal_f32": [_ptr, _ptr, _u64, _u64, _u64, _ptr],
    "kore_hip_softmax_backward_f32": [_ptr, _ptr, _ptr, _u64, _u64, _ptr],
    "kore_hip_cross_entropy_backward_f32": [_ptr, _ptr, _ptr, _u64, _u64, _ptr],
    "kore_hip_rms_norm_backward_f32": [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _u64, _u64, _u64, _f32, _ptr],
    "kore_hip_rms_norm_backward_noalloc_f32": [_ptr, _ptr, _ptr, _ptr, _ptr, _u64, _u64, _f32, _ptr],
    "kore_hip_ternary_matmul_i8": [_ptr, _ptr, _ptr, _ptr, _ptr, _u64, _u64, _u64, _ptr],
    "kore_hip_ternary_matmul_f32": [_ptr, _ptr, _ptr, _ptr, _u64, _u64, _u64, _ptr],
    "kore_hip_bit_linear_f32": [_ptr, _ptr, _ptr, _ptr, _ptr, _u64, _u64, _u64, _ptr],
    "kore_hip_bit_linear_i8": [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _u64, _u64, _u64, _ptr],
    "kore_hip_pack_weights_ternary": [_ptr, _u64, _u64, _f32, _ptr, _ptr, _ptr],
}

# Entry points whose return type is not int.
RESTYPES = {
    "kore_hip_rms_norm_backward_workspace_bytes": ([_u64, _u64], _u64),
    "kore_hip_rms_norm_backward_noalloc_max_bytes": ([], _u64),
}


class KoreLibraryError(RuntimeError):
    """libkore_hip.so is missing or does not export the C ABI."""


_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Load libkore_hip.so once and bind every entry point's signature."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise KoreLibraryError(
                f"{LIB_PATH} not found: build it with `python -c 'import __graft_entry__ as g; g.build()'`"
            )
        try:
            lib = ctypes.CDLL(LIB_PATH)
        except OSError as e:  # pragma: no cover - depends on the box
            raise KoreLibraryError(f"cannot load {LIB_PATH}: {e}") from e
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name, None)
            if fn is None:
                raise KoreLibraryError(f"{LIB_PATH} does not export {name}")
            fn.argtypes = argtypes
            fn.restype = _int
        for name, (argtypes, restype) in RESTYPES.items():
            fn = getattr(lib, name, None)
            if fn is None:
                raise KoreLibraryError(f"{LIB_PATH} does not export {name}")
            fn.argtypes = argtypes
            fn.restype = restype
        lib.kore_hip_status_string.argtypes = [_int]
        lib.kore_hip_status_string.restype = ctypes.c_char_p
        _lib = lib
        return lib


def status_string(status: int) -> str:
    return load().kore_hip_status_string(int(status)).decode()
