"""Pins the CPU oracle (oracle/kore_oracle.c) before anything is compared with it.

Three kinds of check, chosen so that a plausible restatement mistake -- a
dropped term, a wrong sign or index, pairwise instead of sequential summation,
half-split vs interleaved pairing, ties-to-even instead of ties-away -- fails
at least one of them:

  * the reference's own known-answer tests, tightened where the answer is
    exact (file:line of each);
  * closed forms / invariants / f64 recomputations of the mathematics;
  * an independent library (torch, f64) for the transcendental formulas.
"""
import math
import struct

import numpy as np
import pytest

import oracle
from inputs import normal, rmsnorm_inputs


def f32_bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


# --------------------------------------------------------------- embedding
def test_embedding_reference_kat():
    # crates/kore-edge/src/ops/embedding.rs:33-41 (exact assert_eq)
    w = np.array([1, 2, 3, 4, 5, 6], np.float32).reshape(3, 2)
    out = oracle.embedding(w, np.array([0, 2, 1], np.uint32))
    assert out.ravel().tolist() == [1.0, 2.0, 5.0, 6.0, 3.0, 4.0]


def test_embedding_out_of_range_reference_kat():
    # crates/kore-edge/src/ops/embedding.rs:44-50 and kore-nn embedding.rs:146-151
    w = np.array([1, 2, 3, 4], np.float32).reshape(2, 2)
    assert oracle.embedding(w, np.array([10], np.uint32)).ravel().tolist() == [0.0, 0.0]


def test_embedding_brute_force_and_negative_ids():
    table = normal((50, 7), 3)
    ids = np.array([0, 49, 50, -1, 3, 3, 2**31 - 1, -(2**31)], np.int64).astype(np.int32)
    out = oracle.embedding(table, ids)
    for t, i in enumerate(ids):
        u = int(np.uint32(np.int64(i) & 0xFFFFFFFF))
        want = table[u] if u < 50 else np.zeros(7, np.float32)
        assert out[t].tobytes() == want.tobytes()


def _rust_as_usize(v: float) -> int:
    # Rust reference semantics of `f32 as usize` (saturating since Rust 1.45):
    # NaN -> 0, below 0 -> 0, above usize::MAX -> usize::MAX, else truncate.
    if math.isnan(v):
        return 0
    if math.isinf(v):
        return 0 if v < 0 else 2**64 - 1
    return min(max(math.trunc(v), 0), 2**64 - 1)


def test_f32_as_usize_brute_force():
    specials = [float("nan"), -float("inf"), float("inf"), -1.5, -0.0, 0.0, 0.4, 0.9, 1.0, 1.5, 2.999999,
                3.0, 16777217.0, 1e19, 1.8446744e19, 2.0**64, 1e30, -1e30]
    vals = np.concatenate([np.array(specials, np.float32), normal((5000,), 21) * 1000,
                           np.float32(2.0) ** np.arange(-10, 70, dtype=np.float32)])
    for v in vals.tolist():
        assert oracle.f32_as_usize(v) == _rust_as_usize(np.float32(v).item()), v


def test_embedding_forward_cast_then_lookup():
    # crates/kore-nn/src/embedding.rs:91-98: forward = lookup(ids as usize);
    # kore-nn's own test (:152-158) feeds [0.0, 3.0, 7.0] and checks the shape
    table = normal((50, 7), 4)
    assert oracle.embedding_forward(table, np.array([0.0, 3.0, 7.0], np.float32)).shape == (3, 7)
    ids = np.array([0.0, 2.0, 1.0, float("nan"), -1.5, 0.9, 1e30, 49.0, 50.0, 51.0, 49.99, -0.0,
                    float("inf"), -float("inf")], np.float32)
    out = oracle.embedding_forward(table, ids)
    for t, v in enumerate(ids.tolist()):
        u = _rust_as_usize(v)
        want = table[u] if u < 50 else np.zeros(7, np.float32)
        assert out[t].tobytes() == want.tobytes(), (t, v)


# ----------------------------------------------------------------- RMSNorm
def test_rms_norm_unit_input_reference_kat():
    # crates/kore-nn/src/rms_norm.rs:193-202 (ones -> 1.0 within 1e-3)
    y = oracle.rms_norm(np.ones((2, 8), np.float32), np.ones(8, np.float32), 1e-6)
    assert np.allclose(y, 1.0, atol=1e-3)
    # exact f32 closed form: sum = 8 -> 8/8 + eps, inv = 1/sqrt(1+1e-6)
    inv = np.float32(1.0) / np.sqrt(np.float32(1.0) + np.float32(1e-6))
    assert (y == np.float32(1.0) * inv).all()


def test_rms_norm_123_closed_form():
    # crates/kore-edge/src/ops/norm.rs:44-52 ([1,2,3]: rms = sqrt(14/3))
    y = oracle.rms_norm(np.array([[1, 2, 3]], np.float32), np.ones(3, np.float32), 1e-5)
    rms = math.sqrt(14.0 / 3.0 + 1e-5)
    assert np.allclose(y[0], np.array([1, 2, 3]) / rms, rtol=1e-6)
    assert 0 < y[0, 0] < 1 and y[0, 2] > 1


def test_rms_norm_sum_is_sequential():
    # Squares [2^24, 1, 1, ...]: a left-to-right f32 fold absorbs every +1
    # (2^24 + 1 rounds back to 2^24), a pairwise/f64 sum would not.  This pins
    # the reference's sequential `row.iter().map(|x| x*x).sum()` (cpu_fused.rs:180).
    cols = 64
    x = np.ones((1, cols), np.float32)
    x[0, 0] = 4096.0
    y = oracle.rms_norm(x, np.ones(cols, np.float32), 0.0)
    ss = np.float32(2.0**24)
    inv = np.float32(1.0) / np.sqrt(ss / np.float32(cols))
    assert y[0, 1] == np.float32(1.0) * inv
    pairwise = np.float32(1.0) / np.sqrt(np.float32((2.0**24 + cols - 1) / cols))
    assert y[0, 1] != pairwise


def test_rms_norm_weight_and_order():
    # y_i = (x_i * inv) * g_i: scaling g by 2 scales y exactly by 2; the
    # invariant mean((y/g)^2) ~= 1 holds to f32 precision; f64 recomputation.
    x, g = rmsnorm_inputs(16, 256, seed=5)
    y = oracle.rms_norm(x, g, 1e-6)
    y2 = oracle.rms_norm(x, 2 * g, 1e-6)
    assert (y2 == 2 * y).all()
    assert np.allclose(((y / g) ** 2).mean(axis=1), 1.0, atol=1e-5)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64**2).mean(axis=1, keepdims=True) + 1e-6) * g
    assert np.max(np.abs(y - ref) / np.abs(ref)) < 2e-6


# ------------------------------------------------------------- activations
def test_gelu_constant_bits():
    # FRAC_2_SQRT_PI * FRAC_1_SQRT_2 folded in f32 (activations.rs:25-26) ==
    # edge's 0.797_884_6 (activation.rs:12) == 0x3F4C422A
    k = np.float32(1.12837916709551257390) * np.float32(0.707106781186547524401)
    assert f32_bits(float(k)) == 0x3F4C422A == f32_bits(0.7978846)


def test_gelu_reference_kat_and_torch():
    # crates/kore-nn/src/activations.rs:152-159: gelu(0)=0, gelu(1)>0.8, gelu(-1)<0
    y = oracle.gelu(np.array([0.0, 1.0, -1.0], np.float32))
    assert abs(y[0]) < 1e-4 and y[1] > 0.8 and y[2] < 0
    torch = pytest.importorskip("torch")
    x = np.concatenate([normal((20000,), 11) * 3, np.linspace(-10, 10, 2001, dtype=np.float32)])
    ref = torch.nn.functional.gelu(torch.from_numpy(x.astype(np.float64)), approximate="tanh").numpy()
    got = oracle.gelu(x)
    assert np.max(np.abs(got - ref)) < 2e-6  # f32 evaluation vs f64 library


def test_silu_reference_kat_and_torch():
    # crates/kore-serve/src/layered/engine.rs:877-886: silu(1)~0.7311, silu(-1)~-0.2689
    y = oracle.silu(np.array([1.0, -1.0], np.float32))
    assert abs(y[0] - 0.7311) < 1e-3 and abs(y[1] + 0.2689) < 1e-3
    torch = pytest.importorskip("torch")
    x = np.concatenate([normal((20000,), 12) * 4, np.linspace(-30, 30, 3001, dtype=np.float32)])
    ref = torch.nn.functional.silu(torch.from_numpy(x.astype(np.float64))).numpy()
    got = oracle.silu(x)
    rel = np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30)
    assert np.max(rel[np.abs(ref) > 1e-30]) < 1e-6


def test_silu_stable_serve_kat_and_torch():
    # crates/kore-serve/src/layered/engine.rs:877-886 (its own KAT), then the
    # two-branch formula of :828-842 against torch f64 on both branches
    y = oracle.silu_stable(np.array([0.0, 1.0, -1.0], np.float32))
    assert abs(y[0]) < 1e-5 and abs(y[1] - 0.7311) < 1e-3 and abs(y[2] + 0.2689) < 1e-3
    torch = pytest.importorskip("torch")
    x = np.concatenate([normal((20000,), 13) * 4, np.linspace(-120, 30, 3001, dtype=np.float32)])
    ref = torch.nn.functional.silu(torch.from_numpy(x.astype(np.float64))).numpy()
    got = oracle.silu_stable(x).astype(np.float64)
    ok = (np.abs(got - ref) <= 1e-6) | (np.abs(got - ref) <= 1e-6 * np.abs(ref))
    assert ok.all()
    # the branch for v < 0 is not the kore-nn formula: below -88.7 the
    # kore-nn silu is v / inf = -0 while the serve form keeps a subnormal
    far = np.array([-95.0], np.float32)
    assert oracle.silu(far)[0] == 0.0 and np.signbit(oracle.silu(far)[0])
    assert oracle.silu_stable(far)[0] < 0.0
    # specials: -inf and NaN give NaN in both forms, +inf gives +inf
    sp = oracle.silu_stable(np.array([-np.inf, np.nan, np.inf], np.float32))
    assert np.isnan(sp[0]) and np.isnan(sp[1]) and sp[2] == np.inf
    # swiglu_serve is silu_stable(gate) * up, rounded once per op
    a, b = normal((4001,), 14), normal((4001,), 15)
    assert (oracle.swiglu_serve(a, b) == oracle.silu_stable(a) * b).all()


def test_mul_and_swiglu_composition():
    a, b = normal((10001,), 1), normal((10001,), 2)
    assert (oracle.mul(a, b) == a * b).all()  # IEEE f32 product, bit-exact
    assert (oracle.mul(a, b, threads=4) == a * b).all()
    s = oracle.swiglu(a, b, threads=3)
    assert (s == oracle.silu(a) * b).all()


# -------------------------------------------------------------------- RoPE
def test_rope_identity_at_position_zero():
    # crates/kore-edge/src/ops/rope.rs:43-51
    d = np.array([1, 2, 3, 4], np.float32).reshape(1, 1, 4)
    assert (oracle.rope(d, 0, 10000.0) == d).all()
    assert (oracle.rope(d, 0, 10000.0, interleaved=True) == d).all()


def test_rope_changes_values_and_preserves_pair_norm():
    # rope.rs:53-74 (values change at pos 5; pair (0, 2) norm preserved at pos 7)
    d = np.array([3, 4, 1, 2], np.float32).reshape(1, 1, 4)
    assert (np.abs(oracle.rope(d, 5, 10000.0) - d) > 1e-5).any()
    r = oracle.rope(d, 7, 10000.0)[0, 0]
    assert abs(math.hypot(r[0], r[2]) - math.hypot(3, 1)) < 1e-5


def test_rope_f64_closed_form_both_pairings():
    seq, heads, hd, start = 37, 3, 16, 1000
    x = normal((seq, heads, hd), 21)
    inv = oracle.rope_inv_freq(hd, 10000.0)
    # inv_freq table is 1/base^(2i/D): check against f64
    assert np.allclose(inv, 1.0 / 10000.0 ** (np.arange(hd // 2) * 2.0 / hd), rtol=1e-6)
    pos = (start + np.arange(seq)).astype(np.float32)
    ang = (pos[:, None] * inv[None, :]).astype(np.float64)  # the reference's f32 product
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    x64 = x.astype(np.float64)
    half = hd // 2
    want = x64.copy()
    want[..., :half] = x64[..., :half] * c - x64[..., half:] * s
    want[..., half:] = x64[..., :half] * s + x64[..., half:] * c
    got = oracle.rope(x, start, 10000.0)
    assert np.max(np.abs(got - want)) < 2e-6
    want_i = x64.copy()
    want_i[..., 0::2] = x64[..., 0::2] * c - x64[..., 1::2] * s
    want_i[..., 1::2] = x64[..., 0::2] * s + x64[..., 1::2] * c
    got_i = oracle.rope(x, start, 10000.0, interleaved=True)
    assert np.max(np.abs(got_i - want_i)) < 2e-6
    # the two pairings really differ
    assert np.max(np.abs(got - got_i)) > 1e-2


def test_rope_batch_positions_restart():
    x = normal((2, 5, 2, 8), 4)
    got = oracle.rope(x, 3, 10000.0)
    assert (got[0] == oracle.rope(x[0], 3, 10000.0)).all()
    assert (got[1] == oracle.rope(x[1], 3, 10000.0)).all()


# --------------------------------------------------------------- pre-quant
def test_quant_code_ties_away_from_zero():
    # amax = 127 makes t = (xn*127)/127 == xn exactly for these xn
    for xn, want in [(2.5, 3), (-2.5, -3), (0.5, 1), (-0.5, -1), (1.5, 2), (126.5, 127),
                     (0.49999997, 0), (-0.49999997, 0), (127.0, 127), (-127.0, -127), (0.0, 0)]:
        assert oracle.quant_code(xn, 127.0) == want, xn


def test_quant_code_clamp_and_nan():
    assert oracle.quant_code(float("nan"), 1.0) == 0
    assert oracle.quant_code(10.0, 1.0) == 127
    assert oracle.quant_code(-10.0, 1.0) == -128
    assert oracle.quant_code(float("inf"), 1.0) == 127


def test_prequant_brute_force_small_rows():
    rng = np.random.default_rng(9)
    for cols in (1, 3, 8, 33):
        x = rng.standard_normal((5, cols)).astype(np.float32)
        x[1] = 0.0  # zero row -> amax guard
        g = (1 + 0.02 * rng.standard_normal(cols)).astype(np.float32)
        q, s = oracle.rms_norm_quant_i8(x, g, 1e-6)
        xn = oracle.rms_norm(x, g, 1e-6)  # the same normalisation, shared definition
        for r in range(5):
            amax = float(np.max(np.abs(xn[r])))
            a = 1.0 if amax < 1e-8 else amax
            assert s[r] == np.float32(np.float32(a) / np.float32(127.0))
            # every code reconstructs within half a step (f64 check)
            recon = q[r].astype(np.float64) * (a / 127.0)
            assert np.all(np.abs(recon - xn[r]) <= a / 127.0 * 0.5 * (1 + 1e-5) + 1e-12)
            if amax >= 1e-8:
                assert np.max(np.abs(q[r])) == 127  # the absmax element maps to +-127
        assert (q[1] == 0).all() and s[1] == np.float32(1.0 / 127.0)


def test_quant_math_identities_compiled(tmp_path):
    """The GPU kernel's fast quotient (Markstein) and ties-away rounding
    identities, checked in IEEE f32 on the CPU (tests/csrc/check_quant_math.c)."""
    import os
    import subprocess

    src = os.path.join(os.path.dirname(__file__), "csrc", "check_quant_math.c")
    exe = str(tmp_path / "cqm")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-mfma", "-o", exe, src, "-lm"], check=True)
    r = subprocess.run([exe, "3000000"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr


def test_segmented_exact_fold_compiled(tmp_path):
    """The row kernels' segmented exact fold (kore_amd/csrc/norm.hip),
    restated in scalar C with the kernel's segment sizes, estimates, run
    composition and checks, equals the plain left-to-right f32 fold on
    adversarial rows (ties, subnormals, overflow, NaN/Inf, zeros, outliers)."""
    import os
    import subprocess

    src = os.path.join(os.path.dirname(__file__), "csrc", "check_segmented_fold.c")
    exe = str(tmp_path / "csf")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe, src, "-lm"], check=True)
    r = subprocess.run([exe, "40000"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "MISMATCH" not in r.stdout


# ------------------------------------------------------- RMSNorm + SiLU gate
def test_rms_norm_silu_gate_reference_kat_and_f64():
    # crates/kore-kernels/src/cpu_fused.rs:451-483: x = 1..8 (2x4), gamma = 1,
    # z as below; all finite and SiLU(0) = 0 zeroes element 5.
    x = np.arange(1, 9, dtype=np.float32).reshape(2, 4)
    z = np.array([0.5, 1.0, -0.5, 2.0, -1.0, 0.0, 1.5, -2.0], np.float32).reshape(2, 4)
    y = oracle.rms_norm_silu_gate(x, np.ones(4, np.float32), z, 1e-6)
    assert np.isfinite(y).all() and y.ravel()[5] == 0.0
    # it is exactly RMSNorm (the pinned oracle) times the pinned silu
    assert (y == oracle.rms_norm(x, np.ones(4), 1e-6) * oracle.silu(z)).all()
    # cpu_fused.rs:660-697: extreme x and z; finite, silu(-50) and silu(0) gate to ~0
    xe = np.array([[100.0, -100.0, 0.0001, -0.0001]], np.float32)
    ze = np.array([[50.0, -50.0, 0.0, 100.0]], np.float32)
    ye = oracle.rms_norm_silu_gate(xe, np.ones(4, np.float32), ze, 1e-6)
    assert np.isfinite(ye).all() and abs(ye[0, 1]) < 1e-10 and abs(ye[0, 2]) < 1e-10
    assert abs(ye[0, 0] - 50.0 * 100.0 / np.sqrt(5000.000005)) < 1e-4
    xg, g = rmsnorm_inputs(8, 96, seed=2)
    zz = normal((8, 96), 3) * 3
    y = oracle.rms_norm_silu_gate(xg, g, zz, 1e-6)
    x64 = xg.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-6) * g * (zz / (1 + np.exp(-zz.astype(np.float64))))
    assert np.max(np.abs(y - ref) / np.maximum(np.abs(ref), 1e-6)) < 5e-6


# ----------------------------------------------------------------- softmax
def _softmax64(x):
    x = np.asarray(x, np.float64)
    e = np.exp(x - x.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def test_softmax_reference_kats():
    # cpu_fused.rs:278-304
    y = oracle.softmax(np.array([[1.0, 2.0, 3.0], [1.0, 2.0, 3.0]], np.float32))
    assert abs(y[0].sum() - 1) < 1e-6 and abs(y[1].sum() - 1) < 1e-6
    assert y[0, 2] > y[0, 1] > y[0, 0]
    y = oracle.softmax(np.array([[1000.0, 1001.0, 1002.0]], np.float32))
    assert np.isfinite(y).all() and abs(y.sum() - 1) < 1e-6


def test_softmax_f64_and_special_values():
    x = normal((16, 300), 4) * 8
    y = oracle.softmax(x)
    ref = _softmax64(x)
    assert np.allclose(y, ref, rtol=5e-6, atol=1e-9)
    # f32::max skips NaN, but exp(NaN - m) poisons the sum: the whole row is NaN
    r = oracle.softmax(np.array([[1.0, np.nan, 2.0]], np.float32))
    assert np.isnan(r).all()
    # -inf entries get 0; an all -inf row is NaN (exp(-inf - -inf))
    r = oracle.softmax(np.array([[0.0, -np.inf, 0.0]], np.float32))
    assert r[0, 1] == 0.0 and r[0, 0] == r[0, 2] == 0.5
    assert np.isnan(oracle.softmax(np.full((1, 3), -np.inf, np.float32))).all()
    # +inf: inf - inf = NaN at that entry -> NaN row
    assert np.isnan(oracle.softmax(np.array([[0.0, np.inf]], np.float32))).all()


def test_softmax_causal_prefix_closed_form():
    x = normal((6, 8), 5) * 3
    for off in (0, 2, 100):
        y = oracle.softmax_causal(x, off)
        for r in range(6):
            lim = min(off + r + 1, 8)
            # the kept prefix is the plain softmax of the prefix, bit for bit
            assert (y[r, :lim] == oracle.softmax(x[r:r + 1, :lim])[0]).all()
            assert (y[r, lim:] == 0.0).all()
    ones = oracle.softmax_causal(np.ones((3, 4), np.float32))
    assert np.allclose(ones, [[1, 0, 0, 0], [.5, .5, 0, 0], [1 / 3, 1 / 3, 1 / 3, 0]], atol=1e-7)


def test_softmax_backward_reference_kat_and_finite_differences():
    # cpu_fused_backward.rs:236-248: a uniform upstream gradient gives ~0
    dx = oracle.softmax_backward(np.ones((1, 3)), np.array([[0.2, 0.3, 0.5]]))
    assert np.abs(dx).max() < 1e-6
    # central differences of L(x) = sum(dy * softmax(x)) in f64
    x = normal((3, 7), 6).astype(np.float64)
    dy = normal((3, 7), 7).astype(np.float64)
    y = _softmax64(x)
    num = np.zeros_like(x)
    h = 1e-6
    for i in range(x.shape[0]):
        for j in range(x.shape[1]):
            xp, xm = x.copy(), x.copy()
            xp[i, j] += h
            xm[i, j] -= h
            num[i, j] = ((dy * _softmax64(xp)).sum() - (dy * _softmax64(xm)).sum()) / (2 * h)
    got = oracle.softmax_backward(dy.astype(np.float32), y.astype(np.float32))
    assert np.max(np.abs(got - num)) < 2e-6


# -------------------------------------------------------- RMSNorm backward
def test_rms_norm_backward_reference_kats():
    # cpu_fused_backward.rs:195-234
    dx, dg = oracle.rms_norm_backward(np.ones((2, 3)), np.arange(1, 7, dtype=np.float32).reshape(2, 3),
                                      np.ones(3), 1e-5)
    assert dx.shape == (2, 3) and dg.shape == (3,)
    dx, dg = oracle.rms_norm_backward(np.array([[0.1, -0.2, 0.3], [-0.1, 0.4, -0.5]]),
                                      np.array([[0.5, -0.3, 1.2], [-0.8, 0.1, 0.7]]), np.array([1.0, 0.5, 2.0]),
                                      1e-5)
    assert np.isfinite(dx).all() and np.isfinite(dg).all()
    dx, dg = oracle.rms_norm_backward(np.zeros((1, 3)), np.array([[1.0, 2.0, 3.0]]), np.ones(3), 1e-5)
    assert np.abs(dx).max() < 1e-6 and np.abs(dg).max() < 1e-6


def test_rms_norm_backward_matches_torch_autograd_f64():
    import torch

    rows, cols, eps = 9, 37, 1e-5
    x = normal((rows, cols), 8)
    g = normal((cols,), 9, 1.0, 0.3)
    dy = normal((rows, cols), 10)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    gt = torch.tensor(g, dtype=torch.float64, requires_grad=True)
    y = xt * torch.rsqrt((xt * xt).mean(dim=-1, keepdim=True) + eps) * gt
    y.backward(torch.tensor(dy, dtype=torch.float64))
    dx, dg = oracle.rms_norm_backward(dy, x, g, eps)
    assert np.allclose(dx, xt.grad.numpy(), rtol=1e-4, atol=2e-6)
    assert np.allclose(dg, gt.grad.numpy(), rtol=1e-4, atol=2e-6)


# -------------------------------------------------- cross-entropy backward
def test_cross_entropy_backward_reference_kats_and_f64():
    # cpu_fused_backward.rs:251-299
    g = oracle.cross_entropy_backward(np.array([[1, 2, 3], [1, 2, 3]], np.float32), np.array([2, 0], np.float32))
    assert g.shape == (2, 3)
    g = oracle.cross_entropy_backward(np.array([[1, 2, 3], [0.5, -0.5, 1]], np.float32), np.array([1, 2], np.float32))
    assert abs(g[0].sum()) < 1e-6 and abs(g[1].sum()) < 1e-6
    g = oracle.cross_entropy_backward(np.array([[0, 0, 10]], np.float32), np.array([2], np.float32))
    assert np.isfinite(g).all()
    g = oracle.cross_entropy_backward(np.array([[10, 0, 0]], np.float32), np.array([2], np.float32))
    assert g[0, 0] > 0 and g[0, 2] < 0
    # (softmax - one_hot) / batch in f64
    x = normal((5, 40), 12) * 3
    t = np.array([0, 39, 7, 7, 20], np.float32)
    e = np.exp(x.astype(np.float64) - x.max(axis=1, keepdims=True))
    ref = e / e.sum(axis=1, keepdims=True)
    ref[np.arange(5), t.astype(int)] -= 1.0
    ref /= 5
    assert np.allclose(oracle.cross_entropy_backward(x, t), ref, rtol=1e-5, atol=1e-7)


def test_cross_entropy_backward_target_cast():
    # `as usize`: truncation, NaN and negatives -> 0; out of range: no subtraction
    x = np.zeros((5, 4), np.float32)
    g = oracle.cross_entropy_backward(x, np.array([2.7, -3.0, np.nan, 0.5, 4.0], np.float32))
    base = np.float32(0.25) * (np.float32(1.0) * np.float32(1 / 5))
    for b, t in enumerate([2, 0, 0, 0, None]):
        for i in range(4):
            want = base - np.float32(0.2) if i == t else base
            assert abs(g[b, i] - want) < 1e-7, (b, i)


# ------------------------------------------------------------------ ternary
def _base3_digits(b: int) -> list:
    return [(b // 3 ** j) % 3 - 1 for j in range(5)]


def test_trit_codec_reference_kats():
    # encoder.rs tests: every byte 0..242 round-trips; five zeros encode to
    # 121 = 1+3+9+27+81; the (Pos, Neg, Zero, Pos, Neg) example round-trips.
    for b in range(243):
        t = oracle.decode_trits(b)
        assert list(t) == _base3_digits(b), b  # closed form: base-3 digits, lsd first
        assert oracle.encode_trits(t) == b
    assert oracle.encode_trits([0, 0, 0, 0, 0]) == 121
    assert list(oracle.decode_trits(121)) == [0] * 5
    assert oracle.decode_trits(oracle.encode_trits([1, -1, 0, 1, -1])).tolist() == [1, -1, 0, 1, -1]
    for b in range(243, 256):  # decode_trits: bytes past the table decode to zeros
        assert list(oracle.decode_trits(b)) == [0] * 5


def test_pack_weights_ternary_kats_and_brute_force():
    # cpu_ternary_matmul.rs test_pack_ternary: 2 rows x 4 -> one byte per row, scales > 0.
    p, s = oracle.pack_weights_ternary(np.array([1.0, -1.0, 0.0, 0.5, -0.5, 1.0, -1.0, 0.0], np.float32)
                                       .reshape(2, 4), 0.3)
    assert p.shape == (2, 1) and (s > 0).all()
    assert list(oracle.unpack_trits(p, 4)[0]) == [1, -1, 0, 1]
    # brute force: scale = row absmax (1.0 below 1e-8), trit = sign where |w/scale| > threshold,
    # padding trits are zeros
    w = np.random.default_rng(3).uniform(-1, 1, size=(7, 23)).astype(np.float32)
    w[2] = 0.0
    p, s = oracle.pack_weights_ternary(w, 0.3)
    amax = np.abs(w).max(axis=1)
    assert (s == np.where(amax < 1e-8, 1.0, amax).astype(np.float32)).all()
    nv = w / s[:, None]
    want = np.where(nv > 0.3, 1, np.where(nv < -0.3, -1, 0))
    assert (oracle.unpack_trits(p, 23) == want).all()
    assert (oracle.unpack_trits(p, 25)[:, 23:] == 0).all()


def test_ternary_matmul_reference_kats():
    # cpu_ternary_matmul.rs test_ternary_matmul_identity and
    # kore-edge ops/matmul.rs test_matmul_ternary_identity: C = I @ [[2,0],[0,3]]
    p, s = oracle.pack_weights_ternary(np.array([[1.0, 0.0], [0.0, 1.0]], np.float32), 0.3)
    c = oracle.ternary_matmul(p, s, np.array([[2.0, 0.0], [0.0, 3.0]], np.float32), 2, 2, 2)
    assert (c == np.array([[2.0, 0.0], [0.0, 3.0]], np.float32)).all()
    # kore-edge test_matmul_ternary_with_scale: [[+1, -1]] * 2 @ [[3], [1]] = 4
    row = oracle.encode_trits([1, -1, 0, 0, 0])
    c = oracle.ternary_matmul(np.array([[row]], np.uint8), np.array([2.0], np.float32),
                              np.array([[3.0], [1.0]], np.float32), 1, 1, 2)
    assert c[0, 0] == 4.0
    # test_ternary_matmul_larger: 8 x 20 x 4, weights (i % 3) - 1, b = (i % 5) * 0.2 -> finite
    w = (np.arange(160) % 3 - 1).astype(np.float32).reshape(8, 20)
    b = ((np.arange(80) % 5) * np.float32(0.2)).astype(np.float32).reshape(20, 4)
    p, s = oracle.pack_weights_ternary(w, 0.3)
    c = oracle.ternary_matmul(p, s, b, 8, 4, 20)
    assert c.shape == (8, 4) and np.isfinite(c).all()
    assert (oracle.unpack_trits(p, 20) == w).all()  # (i % 3) - 1 is already ternary, scale 1


def test_ternary_matmul_exact_and_f64():
    m, n, k = 9, 6, 47
    p = np.random.default_rng(5).integers(0, 256, size=(m, (k + 4) // 5)).astype(np.uint8)
    s = np.random.default_rng(6).uniform(0.5, 2.0, size=m).astype(np.float32)
    t = oracle.unpack_trits(p, k).astype(np.float64)
    # small-integer activations: every partial sum is exact, so c is the exact product times scale
    bi = np.random.default_rng(7).integers(-50, 50, size=(k, n)).astype(np.float32)
    c = oracle.ternary_matmul(p, s, bi, m, n, k)
    assert (c == ((t @ bi).astype(np.float32) * s[:, None])).all()
    # general activations: within the sequential-sum bound of the f64 product
    b = np.random.default_rng(8).standard_normal((k, n)).astype(np.float32)
    c = oracle.ternary_matmul(p, s, b, m, n, k).astype(np.float64)
    ref = (t @ b.astype(np.float64)) * s[:, None]
    bound = (k + 2) * 2.0 ** -24 * (np.abs(t) @ np.abs(b.astype(np.float64))) * s[:, None]
    assert (np.abs(c - ref) <= bound + 1e-30).all()


def test_ternary_matmul_sequential_order_and_zero_skip():
    # The fold runs in k order: (1e8 + 1) - 1e8 is 0 in f32 (ulp(1e8) = 8),
    # any other order or a wider accumulator gives 1.  Zero trits are skipped
    # (compute_row `if t == 0 { continue; }`): an Inf at a zero-trit position
    # leaves the output finite, at a nonzero trit it propagates.
    k = 10
    w = np.zeros((2, k), np.float32)
    w[0, :3] = 1.0
    w[1, 4] = -1.0
    p, s = oracle.pack_weights_ternary(w, 0.3)
    t = oracle.unpack_trits(p, k)
    assert list(t[0, :4]) == [1, 1, 1, 0] and t[1, 4] == -1 and t[1, 3] == 0
    b = np.zeros((k, 1), np.float32)
    b[:3, 0] = [1e8, 1.0, -1e8]
    b[3, 0] = np.inf
    c = oracle.ternary_matmul(p, s, b, 2, 1, k)
    assert c[0, 0] == 0.0 and c[1, 0] == 0.0
    b[4, 0] = np.inf
    c = oracle.ternary_matmul(p, s, b, 2, 1, k)
    assert c[0, 0] == 0.0 and c[1, 0] == -np.inf


def test_ternary_matmul_i8_exact():
    m, n, k = 11, 7, 93
    p = np.random.default_rng(9).integers(0, 256, size=(m, (k + 4) // 5)).astype(np.uint8)
    q = np.random.default_rng(10).integers(-128, 128, size=(n, k)).astype(np.int8)
    sa = np.random.default_rng(11).uniform(0.1, 2.0, size=m).astype(np.float32)
    sq = np.random.default_rng(12).uniform(0.001, 0.1, size=n).astype(np.float32)
    c = oracle.ternary_matmul_i8(p, sa, q, sq, m, n, k)
    acc = oracle.unpack_trits(p, k).astype(np.int64) @ q.astype(np.int64).T
    want = (acc.astype(np.float32) * sa[:, None]).astype(np.float32) * sq[None, :]
    assert c.tobytes() == want.astype(np.float32).tobytes()
    # equals ternary_matmul on the dequantised codes up to its sequential-sum rounding
    b = (q.astype(np.float32) * sq[:, None]).T.copy()
    ref = oracle.ternary_matmul(p, sa, b, m, n, k)
    bound = (k + 3) * 2.0 ** -24 * (np.abs(oracle.unpack_trits(p, k)) @ np.abs(b.astype(np.float64))) * sa[:, None]
    assert (np.abs(c.astype(np.float64) - ref) <= bound + 1e-30).all()


# ------------------------------------------------------ BitLinear::forward
def test_bit_linear_forward_reference_kats():
    """crates/kore-nn/src/bit_linear.rs tests: test_bit_linear_approximates_linear
    (ternary-friendly weights pack to themselves with scale 1, so y is the
    exact integer product [3, 4]) and test_bit_linear_bias (identity weights,
    bias [10, 20], x = [1, 1] -> [11, 21]); test_bit_linear_forward_shape's
    shapes ([4, 16] -> [4, 8])."""
    w = np.array([[1.0, -1.0, 0.0, 1.0], [-1.0, 1.0, 1.0, 0.0]], np.float32)
    p, s = oracle.pack_weights_ternary(w, 0.3)
    y = oracle.bit_linear_forward(p, s, np.array([[1.0, 2.0, 3.0, 4.0]], np.float32), None, 2, 1, 4)
    assert y.shape == (1, 2) and y.tolist() == [[3.0, 4.0]]
    p, s = oracle.pack_weights_ternary(np.array([[1.0, 0.0], [0.0, 1.0]], np.float32), 0.3)
    y = oracle.bit_linear_forward(p, s, np.ones((1, 2), np.float32), np.array([10.0, 20.0], np.float32), 2, 1, 2)
    assert y.tolist() == [[11.0, 21.0]]
    r = np.random.default_rng(5)
    p, s = oracle.pack_weights_ternary(r.standard_normal((8, 16)).astype(np.float32), 0.3)
    assert oracle.bit_linear_forward(p, s, np.ones((4, 16), np.float32), None, 8, 4, 16).shape == (4, 8)


def test_bit_linear_forward_composition():
    """The layer is out[b, o] = c[o, b] + bias[o] where c = ternary_matmul on
    the transposed input: against an f64 recomputation from the decoded trits
    (within the sequential-sum bound of c plus one rounding of the add), and
    column b of the output depends on row b of x only (the transposes put
    tokens on the output's rows)."""
    r = np.random.default_rng(6)
    m, n, k = 37, 5, 203
    p, s = oracle.pack_weights_ternary(r.standard_normal((m, k)).astype(np.float32), 0.5)
    x = r.standard_normal((n, k)).astype(np.float32)
    bias = r.standard_normal(m).astype(np.float32)
    y = oracle.bit_linear_forward(p, s, x, bias, m, n, k)
    t = oracle.unpack_trits(p, k).astype(np.float64)
    c64 = (x.astype(np.float64) @ t.T) * s.astype(np.float64)[None, :]
    bound = (k + 2) * 2.0 ** -24 * (np.abs(x).astype(np.float64) @ np.abs(t).T) * np.abs(s)[None, :]
    want = c64 + bias[None, :]
    assert np.all(np.abs(y - want) <= bound + 2.0 ** -23 * np.abs(want) + 1e-30)
    # token b's output row is the same when computed alone
    y1 = oracle.bit_linear_forward(p, s, x[2:3], bias, m, 1, k)
    assert y1.tobytes() == y[2:3].tobytes()
    # no bias: the matmul output itself, transposed
    y0 = oracle.bit_linear_forward(p, s, x, None, m, n, k)
    assert y0.tobytes() == np.ascontiguousarray(oracle.ternary_matmul(p, s, np.ascontiguousarray(x.T), m, n, k).T).tobytes()
    # the bias add is one f32 rounding of the finished output
    assert y.tobytes() == (y0 + bias[None, :]).astype(np.float32).tobytes()


def test_bit_linear_i8_composition():
    """The layer on pre-quant codes: exact integer products (int64 numpy) with
    the f32 epilogue, transposed, + bias."""
    r = np.random.default_rng(7)
    m, n, k = 29, 6, 160
    p, s = oracle.pack_weights_ternary(r.standard_normal((m, k)).astype(np.float32), 0.5)
    q = r.integers(-128, 128, size=(n, k)).astype(np.int8)
    qs = np.abs(r.standard_normal(n)).astype(np.float32) * 0.01
    bias = r.standard_normal(m).astype(np.float32)
    y = oracle.bit_linear_i8(p, s, q, qs, bias, m, n, k)
    acc = oracle.unpack_trits(p, k).astype(np.int64) @ q.astype(np.int64).T
    c = (acc.astype(np.float32) * s[:, None]) * qs[None, :]
    assert y.tobytes() == (np.ascontiguousarray(c.T) + bias[None, :]).astype(np.float32).tobytes()


def test_ternary_fold_crossing_statistics(tmp_path):
    """The f32-activation ternary fold (a signed random walk) leaves its start
    binade in most 40-term segments at K = 2560 (tests/csrc/
    ternary_fold_crossings.c), so a segmented exact fold would fold ~40 of 64
    segments one by one: more dependent adds than the plain fold."""
    import os
    import re
    import subprocess

    src = os.path.join(os.path.dirname(__file__), "csrc", "ternary_fold_crossings.c")
    exe = str(tmp_path / "xstat")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe, src, "-lm"], check=True)
    out = subprocess.run([exe, "2560", "4000"], capture_output=True, text=True, timeout=120).stdout
    folded = float(re.search(r"([0-9.]+) segments leave", out).group(1))
    changes = float(re.search(r"([0-9.]+) binade/sign changes", out).group(1))
    assert folded > 30 and changes > 200, out
