"""The C ABI library loads, exports every entry point include/kore_hip.h
declares, and rejects bad arguments on the host (no GPU needed: argument
checks run before anything is enqueued)."""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle
from kore_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "kore_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kore_hip_\w+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    lib = _lib.load()
    names = declared_symbols()
    assert len(names) >= 12
    for n in names:
        assert hasattr(lib, n), n
    # the ctypes binding covers every compute entry point
    assert set(names) - {"kore_hip_status_string"} == set(_lib.SIGNATURES) | set(_lib.RESTYPES)


def test_version_and_status_text():
    lib = _lib.load()
    assert lib.kore_hip_version() == 100
    assert _lib.status_string(0) == "ok"
    assert "null" in _lib.status_string(-1)
    assert "HIP" in _lib.status_string(700)


P = 0x1000  # a fake, never-dereferenced non-null pointer


def test_argument_errors_are_reported_on_host():
    lib = _lib.load()
    s = None
    # zero work: OK and nothing launched, even with null pointers
    assert lib.kore_hip_gelu_f32(None, None, 0, s) == 0
    assert lib.kore_hip_rms_norm_f32(None, None, None, 0, 128, 1e-6, s) == 0
    assert lib.kore_hip_embedding_f32(None, None, None, 0, 10, 4, s) == 0
    # null pointers with work
    assert lib.kore_hip_gelu_f32(None, P, 16, s) == _lib.KORE_HIP_ERR_NULL_PTR
    assert lib.kore_hip_swiglu_f32(P, None, P, 16, s) == _lib.KORE_HIP_ERR_NULL_PTR
    assert lib.kore_hip_rms_norm_f32(P, None, P, 4, 128, 1e-6, s) == _lib.KORE_HIP_ERR_NULL_PTR
    assert lib.kore_hip_rms_norm_quant_i8(P, P, P, None, 4, 128, 1e-6, s) == _lib.KORE_HIP_ERR_NULL_PTR
    assert lib.kore_hip_embedding_f32(P, None, P, 3, 10, 4, s) == _lib.KORE_HIP_ERR_NULL_PTR
    assert lib.kore_hip_embedding_forward_f32(P, None, P, 3, 10, 4, s) == _lib.KORE_HIP_ERR_NULL_PTR
    assert lib.kore_hip_embedding_forward_f32(None, None, None, 0, 10, 4, s) == 0
    assert lib.kore_hip_rope_f32(P, None, 1, 4, 2, 8, 0, 0, s) == _lib.KORE_HIP_ERR_NULL_PTR
    # bad dims
    assert lib.kore_hip_rope_f32(P, P, 1, 4, 2, 7, 0, 0, s) == _lib.KORE_HIP_ERR_BAD_DIM
    assert lib.kore_hip_rms_norm_f32(P, P, P, 4, 0, 1e-6, s) == _lib.KORE_HIP_ERR_BAD_DIM
    assert lib.kore_hip_rope_inv_freq_f32(P, 7, 10000.0) == _lib.KORE_HIP_ERR_BAD_DIM
    # overflow
    assert lib.kore_hip_gelu_f32(P, P, 2**62, s) == _lib.KORE_HIP_ERR_OVERFLOW
    assert lib.kore_hip_rms_norm_f32(P, P, P, 2**40, 2**40, 1e-6, s) == _lib.KORE_HIP_ERR_OVERFLOW
    assert lib.kore_hip_embedding_f32(P, P, P, 2**33, 2**33, 4, s) == _lib.KORE_HIP_ERR_OVERFLOW
    # overlapping Q and K
    assert lib.kore_hip_rope_qk_f32(P, P + 64, P, 1, 4, 2, 2, 8, 0, 0, s) == _lib.KORE_HIP_ERR_ALIAS
    # softmax family
    assert lib.kore_hip_softmax_f32(None, None, 0, 16, s) == 0
    assert lib.kore_hip_softmax_f32(None, P, 4, 16, s) == _lib.KORE_HIP_ERR_NULL_PTR
    assert lib.kore_hip_softmax_backward_f32(P, None, P, 4, 16, s) == _lib.KORE_HIP_ERR_NULL_PTR
    assert lib.kore_hip_softmax_f32(P, P, 2**40, 2**40, s) == _lib.KORE_HIP_ERR_OVERFLOW
    assert lib.kore_hip_softmax_causal_f32(P, P, 4, 16, 2**64 - 2, s) == _lib.KORE_HIP_ERR_OVERFLOW
    # RMSNorm backward: workspace, aliasing, nulls
    ws = lib.kore_hip_rms_norm_backward_workspace_bytes
    need = ws(16, 64)
    assert need > 0
    assert lib.kore_hip_rms_norm_backward_f32(P, P, P, P + 2**20, P, None, need, 16, 64, 1e-5, s) == \
        _lib.KORE_HIP_ERR_NULL_PTR
    assert lib.kore_hip_rms_norm_backward_f32(P, P + 2**20, P, P + 2**21, P, P, need - 4, 16, 64, 1e-5, s) == \
        _lib.KORE_HIP_ERR_BAD_DIM
    assert lib.kore_hip_rms_norm_backward_f32(P, P + 2**20, P, P + 64, P, P, need, 16, 64, 1e-5, s) == \
        _lib.KORE_HIP_ERR_ALIAS


def test_ternary_argument_errors_are_reported_on_host():
    lib = _lib.load()
    for f in (lambda *a: lib.kore_hip_ternary_matmul_f32(a[0], a[1], a[2], a[3], *a[4:]),):
        assert f(None, None, None, None, 0, 4, 16, None) == 0
        assert f(None, None, None, None, 4, 0, 16, None) == 0
        assert f(P, None, P, P + 4096, 4, 4, 16, None) == _lib.KORE_HIP_ERR_NULL_PTR
        assert f(None, P, None, P + 4096, 4, 4, 16, None) == _lib.KORE_HIP_ERR_NULL_PTR
        assert f(P, P, P, P, 2**32, 2**32, 16, None) == _lib.KORE_HIP_ERR_OVERFLOW
        # the output may not overlap the weights, scales or activations
        assert f(P, P + 2**20, P + 2**21, P + 2**21 + 64, 4, 4, 16, None) == _lib.KORE_HIP_ERR_ALIAS
    assert lib.kore_hip_ternary_matmul_i8(P, None, P, P, P + 4096, 4, 4, 16, None) == _lib.KORE_HIP_ERR_NULL_PTR
    # BitLinear::forward entry points: same checks, the bias (optional) included
    blf, bli = lib.kore_hip_bit_linear_f32, lib.kore_hip_bit_linear_i8
    assert blf(None, None, None, None, None, 0, 4, 16, None) == 0
    assert bli(None, None, None, None, None, None, 4, 0, 16, None) == 0
    assert blf(P, P, P, None, None, 4, 4, 16, None) == _lib.KORE_HIP_ERR_NULL_PTR
    assert bli(P, P, None, P, None, P + 4096, 4, 4, 16, None) == _lib.KORE_HIP_ERR_NULL_PTR
    assert blf(P, P, P, None, P, 2**32, 2**32, 16, None) == _lib.KORE_HIP_ERR_OVERFLOW
    assert blf(P, P + 2**30, P + 2**31, None, P + 2**40, 4, 4, 2**24, None) == _lib.KORE_HIP_ERR_OVERFLOW  # in > 2^23
    # the output may not overlap the bias
    assert blf(P, P + 2**20, P + 2**21, P + 2**22, P + 2**22 + 8, 4, 4, 16, None) == _lib.KORE_HIP_ERR_ALIAS
    assert bli(P, P + 2**20, P + 2**21, P + 2**21 + 4096, P + 2**22, P + 2**22 + 8, 4, 4, 16, None) == \
        _lib.KORE_HIP_ERR_ALIAS
    pack = lib.kore_hip_pack_weights_ternary
    assert pack(None, 0, 16, 0.3, None, None, None) == 0
    assert pack(P, 4, 16, 0.3, P + 4096, None, None) == _lib.KORE_HIP_ERR_NULL_PTR
    assert pack(None, 4, 16, 0.3, P + 4096, P + 8192, None) == _lib.KORE_HIP_ERR_NULL_PTR
    assert pack(P, 2**32, 2**32, 0.3, P, P, None) == _lib.KORE_HIP_ERR_OVERFLOW
    # packed bytes or scales inside the weights
    assert pack(P, 4, 16, 0.3, P + 64, P + 4096, None) == _lib.KORE_HIP_ERR_ALIAS
    assert pack(P, 4, 16, 0.3, P + 4096, P + 60, None) == _lib.KORE_HIP_ERR_ALIAS


def test_rms_norm_backward_noalloc_host_checks():
    # host-side only: a size beyond the fixed scratch array, null pointers and
    # empty work are answered before any device call
    lib = _lib.load()
    cap = lib.kore_hip_rms_norm_backward_noalloc_max_bytes()
    assert cap == 16 << 20
    f = lib.kore_hip_rms_norm_backward_noalloc_f32
    assert f(P, P + 2**40, P, P + 2**41, P, cap // 4 + 1, 3, 1e-5, None) == _lib.KORE_HIP_ERR_SCRATCH
    assert f(P, None, P, P, P, 16, 64, 1e-5, None) == _lib.KORE_HIP_ERR_NULL_PTR
    assert f(None, None, None, None, None, 16, 0, 1e-5, None) == 0
    assert _lib.status_string(_lib.KORE_HIP_ERR_SCRATCH).startswith("work exceeds")


def test_rms_norm_backward_workspace_size():
    ws = _lib.load().kore_hip_rms_norm_backward_workspace_bytes
    assert ws(0, 128) == 0 and ws(128, 0) == 0 and ws(2**40, 2**40) == 0
    # vector plan: a row split over S = 1/2/4 waves (cols <= 1024/2048/4096),
    # 4/S rows per iteration, iters = clamp(ceil(rows / (512 * 4/S)), 1, 16),
    # P = ceil(rows / (iters * 4/S)) partial rows of cols floats;
    # generic plan: one float per row.
    assert ws(16384, 2048) == 512 * 2048 * 4
    assert ws(100, 256) == 25 * 256 * 4
    assert ws(1 << 20, 4096) == 65536 * 4096 * 4
    assert ws(16384, 2050) == 16384 * 4       # cols % 4 != 0 -> generic
    assert ws(4, 8192) == 4 * 4               # cols > 4096 -> generic


@pytest.mark.parametrize("head_dim", [2, 8, 64, 128, 256])
@pytest.mark.parametrize("base", [10000.0, 500000.0, 10.0])
def test_rope_inv_freq_table_matches_oracle_bit_exact(head_dim, base):
    half = head_dim // 2
    got = np.zeros(half, np.float32)
    assert _lib.load().kore_hip_rope_inv_freq_f32(got.ctypes.data, head_dim, base) == 0
    want = oracle.rope_inv_freq(head_dim, base)
    assert got.tobytes() == want.tobytes()


def test_rust_binding_names_match_the_header():
    """rust/kore-kernels-rocm/src/fused.rs (the drop-in KORE module, not
    compiled here) loads only symbols that include/kore_hip.h declares, and
    binds every entry point."""
    import re

    rs = open(os.path.join(ROOT, "rust", "kore-kernels-rocm", "src", "fused.rs")).read()
    loaded = set(re.findall(r'lib\.get\(b"(kore_hip_[a-z0-9_]+)\\0"\)', rs))
    declared = set(declared_symbols())
    assert loaded, "no symbols found in fused.rs"
    assert loaded <= declared, loaded - declared
    expected = {d for d in declared if d != "kore_hip_version"}
    assert expected <= loaded, expected - loaded
