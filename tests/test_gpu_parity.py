"""GPU parity: every entry point of libkore_hip.so against the CPU oracle on
identical seeded inputs, through KORE's rocm_* op API (kore_amd.rocm).

Bar: embedding gather, RMSNorm and int8 codes/scales
bit-exact; GELU / SiLU / SwiGLU / RoPE within |d| <= 1e-6 or |d| <= 1e-5*|ref|
(inputs.assert_close).  Cases cover the reference's edge cases (empty work,
ragged rows, out-of-range ids, zero rows, NaN/Inf) plus every BASELINE config
at full size.
"""
import sys

import numpy as np
import pytest

import oracle
from inputs import (assert_bitexact, assert_close, assert_close_scaled, embedding_ids, max_err, normal,
                    prequant_inputs, rmsnorm_inputs)

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from kore_amd import rocm  # noqa: E402
from kore_amd.rocm import HipBuffer  # noqa: E402

DEV = 0


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def up(arr) -> HipBuffer:
    return HipBuffer.from_host(DEV, np.ascontiguousarray(arr))


def down(buf: HipBuffer, dtype, shape):
    return buf.to_host(dtype)[: int(np.prod(shape))].reshape(shape)


def unaligned(arr: np.ndarray) -> HipBuffer:
    """Device copy of arr starting 4 bytes past a 16-byte boundary."""
    t = torch.empty(arr.size + 1, dtype=torch.float32, device="cuda")
    t[1:].copy_(torch.from_numpy(np.ascontiguousarray(arr, np.float32).ravel()))
    return HipBuffer.from_tensor(t[1:])


def _offset_buffer(arr: np.ndarray, offset: int) -> HipBuffer:
    """Device copy of arr starting `offset` bytes past a 16-byte boundary."""
    t = torch.empty(arr.nbytes + offset, dtype=torch.uint8, device="cuda")
    t[offset:].copy_(torch.from_numpy(np.ascontiguousarray(arr).view(np.uint8).ravel()))
    return HipBuffer.from_tensor(t[offset:])


# ----------------------------------------------------------------- RMSNorm
RMS_SHAPES = [(1, 1), (3, 7), (2, 4), (5, 256), (17, 260), (6, 1000), (32, 2048), (9, 2560), (7, 4096),
              (3, 5000), (65, 512)]


@pytest.mark.parametrize("rows,cols", RMS_SHAPES)
def test_rms_norm_bit_exact(rows, cols):
    log(f"rms_norm rows={rows} cols={cols}")
    x, g = rmsnorm_inputs(rows, cols, seed=rows * 131 + cols)
    out = rocm.rocm_rms_norm_f32(DEV, up(x), up(g), rows, cols, 1e-6)
    got = down(out, np.float32, (rows, cols))
    want = oracle.rms_norm(x, g, 1e-6)
    assert_bitexact(got, want, "rms_norm")


def test_rms_norm_baseline_config0_and_sweep():
    # x[32,2048] ~ N(0,1), w ~ N(1,0.02), eps 1e-6, seed 0
    for rows, cols in [(32, 2048), (16384, 2048)]:
        log(f"rms_norm baseline rows={rows} cols={cols}")
        x, g = rmsnorm_inputs(rows, cols, seed=0)
        got = down(rocm.rocm_rms_norm_f32(DEV, up(x), up(g), rows, cols, 1e-6), np.float32, (rows, cols))
        assert_bitexact(got, oracle.rms_norm(x, g, 1e-6), "rms_norm baseline")


def test_rms_norm_in_place_and_unaligned():
    rows, cols = 10, 768
    x, g = rmsnorm_inputs(rows, cols, seed=3)
    want = oracle.rms_norm(x, g, 1e-6)
    buf = up(x)
    rocm.rocm_rms_norm_f32(DEV, buf, up(g), rows, cols, 1e-6, out=buf)
    assert_bitexact(down(buf, np.float32, (rows, cols)), want, "in place")
    xb = unaligned(x)
    out = rocm.rocm_rms_norm_f32(DEV, xb, up(g), rows, cols, 1e-6)
    assert_bitexact(down(out, np.float32, (rows, cols)), want, "unaligned")


def test_rms_norm_special_rows():
    cols = 300
    x = normal((6, cols), 8)
    x[1] = 0.0
    x[2, 5] = np.nan
    x[3, 7] = np.inf
    x[4] *= 1e20  # sum of squares overflows to inf -> inv 0
    x[5, :] = 1e-30  # underflowing squares
    g = np.ones(cols, np.float32)
    for eps in (1e-6, 0.0):
        got = down(rocm.rocm_rms_norm_f32(DEV, up(x), up(g), 6, cols, eps), np.float32, (6, cols))
        want = oracle.rms_norm(x, g, eps)
        assert_bitexact(got, want, f"special rows eps={eps}")


@pytest.mark.parametrize("seed", range(8))
def test_row_kernels_random_shapes(seed):
    """Seeded random shapes and input offsets for RMSNorm and the BitLinear
    pre-quant (every column-chunk count of the vector kernels, one or four
    waves per workgroup, the scalar path for odd widths or unaligned inputs),
    with random row scales spanning many binades: bit-exact against the
    oracle (normalised values, int8 codes and scales)."""
    r = np.random.default_rng(2000 + seed)
    for case in range(6):
        rows = int(r.choice([1, 2, 7, 31, 64, 100, 255, 256, 257, 700]))
        cols = int(r.choice([4, 8, 60, 256, 260, 512, 1000, 1024, 2048, 2560, 3000, 4096, 6144, 8192]))
        if r.random() < 0.2:
            cols += int(r.integers(1, 4))  # odd width: scalar path
        off = 4 * int(r.integers(0, 4)) if r.random() < 0.3 else 0
        x = normal((rows, cols), 100 * seed + case)
        x *= np.exp2(r.integers(-60, 60, size=(rows, 1))).astype(np.float32)
        g = normal((cols,), 7 * seed + case, 1.0, 0.02)
        log(f"row kernels random seed={seed} case={case} rows={rows} cols={cols} x+{off}")
        xb = _offset_buffer(x, off) if off else up(x)
        got = down(rocm.rocm_rms_norm_f32(DEV, xb, up(g), rows, cols, 1e-6), np.float32, (rows, cols))
        assert_bitexact(got, oracle.rms_norm(x, g, 1e-6), f"rms_norm {rows}x{cols}")
        q, sc = rocm.rocm_rms_norm_quant_i8(DEV, xb, up(g), rows, cols, 1e-6)
        wq, ws = oracle.rms_norm_quant_i8(x, g, 1e-6)
        assert down(sc, np.float32, (rows,)).tobytes() == ws.tobytes(), f"scales {rows}x{cols}"
        assert (down(q, np.int8, (rows, cols)) == wq).all(), f"codes {rows}x{cols}"


# ------------------------------------------------------- RMSNorm + SiLU gate
@pytest.mark.parametrize("rows,cols", [(1, 4), (3, 7), (2, 8), (32, 2048), (17, 260), (64, 2560), (4096, 2560),
                                       (5, 5000)])
def test_rms_norm_silu_gate(rows, cols):
    log(f"rms_norm_silu_gate rows={rows} cols={cols}")
    x, g = rmsnorm_inputs(rows, cols, seed=rows + cols)
    z = normal((rows, cols), rows * 7 + cols) * 3
    z.ravel()[: min(z.size, 24)] = special_values()[: min(z.size, 24)]
    out = rocm.rocm_fused_rms_norm_silu_gate_f32(DEV, up(x), up(g), up(z), rows, cols, 1e-6)
    got = down(out, np.float32, (rows, cols))
    want = oracle.rms_norm_silu_gate(x, g, z, 1e-6)
    assert_close(got, want, what="rms_norm_silu_gate")
    # the normalisation factor is the bit-exact RMSNorm one: where silu(z) == 1
    # the output is bit-identical to rms_norm
    ones = np.full_like(z, 1e30)
    got1 = down(rocm.rocm_fused_rms_norm_silu_gate_f32(DEV, up(x), up(g), up(ones), rows, cols, 1e-6),
                np.float32, (rows, cols))
    assert_bitexact(got1, oracle.rms_norm(x, g, 1e-6) * np.float32(1e30), "silu gate = identity")


@pytest.mark.parametrize("cols", [2560, 2562])  # vector path and scalar path
def test_rms_norm_silu_gate_wide_gate_range(cols):
    # The gate's error grows with |z| (exp argument rounding); sweep the
    # whole range where e^-z is finite, both signs, plus overflow territory.
    log(f"rms_norm_silu_gate wide z cols={cols}")
    rows = 64
    x, g = rmsnorm_inputs(rows, cols, seed=9)
    z = np.linspace(-100.0, 100.0, rows * cols, dtype=np.float32).reshape(rows, cols)
    out = rocm.rocm_fused_rms_norm_silu_gate_f32(DEV, up(x), up(g), up(z), rows, cols, 1e-6)
    got = down(out, np.float32, (rows, cols))
    assert_close(got, oracle.rms_norm_silu_gate(x, g, z, 1e-6), what="rms_norm_silu_gate wide z")


def test_rms_norm_silu_gate_reference_kat_on_device():
    # crates/kore-kernels/src/cpu_fused.rs:451-483
    x = np.arange(1, 9, dtype=np.float32).reshape(2, 4)
    z = np.array([0.5, 1.0, -0.5, 2.0, -1.0, 0.0, 1.5, -2.0], np.float32).reshape(2, 4)
    got = down(rocm.rocm_fused_rms_norm_silu_gate_f32(DEV, up(x), up(np.ones(4, np.float32)), up(z), 2, 4, 1e-6),
               np.float32, (2, 4))
    assert np.isfinite(got).all() and got.ravel()[5] == 0.0
    assert_close(got, oracle.rms_norm_silu_gate(x, np.ones(4), z, 1e-6), what="silu gate kat")
    # cpu_fused.rs:660-697
    xe = np.array([[100.0, -100.0, 0.0001, -0.0001]], np.float32)
    ze = np.array([[50.0, -50.0, 0.0, 100.0]], np.float32)
    ge = down(rocm.rocm_fused_rms_norm_silu_gate_f32(DEV, up(xe), up(np.ones(4, np.float32)), up(ze), 1, 4, 1e-6),
              np.float32, (1, 4))
    assert np.isfinite(ge).all() and abs(ge[0, 1]) < 1e-10 and abs(ge[0, 2]) < 1e-10
    assert_close(ge, oracle.rms_norm_silu_gate(xe, np.ones(4), ze, 1e-6), what="silu gate extreme kat")


# --------------------------------------------------------------- pre-quant
@pytest.mark.parametrize("rows,cols", [(1, 2560), (64, 2560), (4096, 2560), (5, 33), (9, 300), (3, 8),
                                       (20, 2048), (7, 4096), (2, 4100)])
def test_prequant_bit_exact(rows, cols):
    log(f"prequant rows={rows} cols={cols}")
    x, g = prequant_inputs(rows, cols, seed=rows + 17 * cols)
    q, s = rocm.rocm_rms_norm_quant_i8(DEV, up(x), up(g), rows, cols, 1e-6)
    gq = down(q, np.int8, (rows, cols))
    gs = down(s, np.float32, (rows,))
    wq, ws = oracle.rms_norm_quant_i8(x, g, 1e-6)
    assert gs.tobytes() == ws.tobytes()
    diff = np.argwhere(gq != wq)
    assert diff.size == 0, f"{len(diff)} codes differ, first {diff[:3].tolist()}"


def test_prequant_baseline_seed0():
    # BASELINE configs[4] at T = 4096, 64, 1 with seed 0
    for rows in (4096, 64, 1):
        log(f"prequant baseline T={rows}")
        x, g = prequant_inputs(rows, 2560, seed=0)
        q, s = rocm.rocm_rms_norm_quant_i8(DEV, up(x), up(g), rows, 2560, 1e-6)
        wq, ws = oracle.rms_norm_quant_i8(x, g, 1e-6)
        assert down(q, np.int8, (rows, 2560)).tobytes() == wq.tobytes()
        assert down(s, np.float32, (rows,)).tobytes() == ws.tobytes()


def test_prequant_special_rows_and_unaligned_q():
    cols = 512
    x = normal((7, cols), 4)
    x[0] = 0.0                        # amax guard -> codes 0, scale 1/127
    x[1, 3] = np.nan                  # NaN row -> all codes 0
    x[2, 9] = np.inf
    x[3] = 1e-12                      # tiny but non-zero
    x[4, ::2] = 0.0
    x[5] *= 1e20
    g = normal((cols,), 5, 1.0, 0.02)
    g[6] = np.nan                     # one NaN weight: its code is 0, the rest quantise
    wq, ws = oracle.rms_norm_quant_i8(x, g, 1e-6)
    q, s = rocm.rocm_rms_norm_quant_i8(DEV, up(x), up(g), 7, cols, 1e-6)
    assert down(q, np.int8, (7, cols)).tobytes() == wq.tobytes()
    assert down(s, np.float32, (7,)).tobytes() == ws.tobytes()
    # q buffer at an odd byte offset takes the scalar path
    qt = torch.empty(7 * cols + 1, dtype=torch.int8, device="cuda")
    qb = HipBuffer(qt[1:].view(torch.uint8), DEV)
    rocm.rocm_rms_norm_quant_i8(DEV, up(x), up(g), 7, cols, 1e-6, out_q=qb)
    assert qt[1:].cpu().numpy().tobytes() == wq.tobytes()


@pytest.mark.parametrize("cols", [2560, 2048, 512, 36])
def test_prequant_near_tie_codes(cols):
    """Integer-valued rows (|x| <= 254, unit weights): many quotients
    127 * xn / amax land within a few ulps of k + 0.5 (e.g. x = 1 against an
    absmax element 254), so the bracketed fast codes split and the exact
    per-lane recomputation decides them.  Bit-exact against the oracle."""
    rows = 512
    log(f"prequant near-tie rows cols={cols}")
    g = np.random.default_rng(cols)
    x = g.integers(-254, 255, size=(rows, cols)).astype(np.float32)
    x[:, 0] = 254.0
    x[::3, 1] = -254.0
    x[1::4] = np.round(x[1::4] / 127.0)  # rows of -2..2 with one 254
    w = np.ones(cols, np.float32)
    q, s = rocm.rocm_rms_norm_quant_i8(DEV, up(x), up(w), rows, cols, 1e-6)
    wq, ws = oracle.rms_norm_quant_i8(x, w, 1e-6)
    assert down(s, np.float32, (rows,)).tobytes() == ws.tobytes()
    gq = down(q, np.int8, (rows, cols))
    diff = np.argwhere(gq != wq)
    assert diff.size == 0, f"{len(diff)} codes differ, first {diff[:3].tolist()}"


@pytest.mark.parametrize("cols", [2560, 512])
def test_prequant_huge_weights_overflowing_numerator(cols):
    """|xn| * 127 above FLT_MAX: the reference's quotient is +-inf and the
    clamp gives 127 / -128; absmax at 2^120 and above, and just below it."""
    rows = 8
    log(f"prequant huge weights cols={cols}")
    x = normal((rows, cols), 31)
    w = np.full(cols, 1e37, np.float32)
    w[::7] = 1.0
    x[6, 5] = 30.0  # an outlier: a larger absmax for row 6
    x[7, :100] = 0.0
    wq, ws = oracle.rms_norm_quant_i8(x, w, 1e-6)
    assert (np.abs(wq) >= 127).any()  # overflowed numerators present
    q, s = rocm.rocm_rms_norm_quant_i8(DEV, up(x), up(w), rows, cols, 1e-6)
    assert down(s, np.float32, (rows,)).tobytes() == ws.tobytes()
    assert down(q, np.int8, (rows, cols)).tobytes() == wq.tobytes()
    for wv in (2e33, 3e33, 4e33):  # absmax either side of 2^120, the fast path's top end
        w2 = np.full(cols, wv, np.float32)
        wq2, ws2 = oracle.rms_norm_quant_i8(x, w2, 1e-6)
        q2, s2 = rocm.rocm_rms_norm_quant_i8(DEV, up(x), up(w2), rows, cols, 1e-6)
        assert down(s2, np.float32, (rows,)).tobytes() == ws2.tobytes()
        assert down(q2, np.int8, (rows, cols)).tobytes() == wq2.tobytes()


# ------------------------------------------------------------- activations
# (13 * 512 + 3 and 2049 * 512 - 5: block counts that do not divide over the
# 8 XCDs, for the binary kernels' per-XCD tile order)
ACT_SIZES = [1, 3, 4, 5, 255, 1024, 1027, 13 * 512 + 3, (1 << 20) + 3, 2049 * 512 - 5]


def special_values():
    return np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, 88.0, -88.0, 89.0, -89.0, 100.0, -100.0,
                     1e-38, -1e-38, 1e-45, 3.0e38, -3.0e38, 0.5, -0.5, 10.0, -10.0, 20.0, -20.0], np.float32)


@pytest.mark.parametrize("op", ["gelu", "silu"])
@pytest.mark.parametrize("n", ACT_SIZES)
def test_unary_activation(op, n):
    log(f"{op} n={n}")
    x = normal((n,), n) * 3
    x[: min(n, 24)] = special_values()[: min(n, 24)]
    got = down(getattr(rocm, f"rocm_{op}_f32")(DEV, up(x), n), np.float32, (n,))
    want = getattr(oracle, op)(x)
    assert_close(got, want, what=op)


@pytest.mark.parametrize("op", ["mul", "swiglu"])
@pytest.mark.parametrize("n", ACT_SIZES)
def test_binary_op(op, n):
    log(f"{op} n={n}")
    a = normal((n,), n) * 3
    b = normal((n,), n + 1)
    a[: min(n, 24)] = special_values()[: min(n, 24)]
    got = down(getattr(rocm, f"rocm_{op}_f32")(DEV, up(a), up(b), n), np.float32, (n,))
    if op == "mul":
        assert_bitexact(got, oracle.mul(a, b), "mul")
    else:
        assert_close(got, oracle.swiglu(a, b), what=op)


def test_activation_unaligned_and_in_place():
    n = 4099
    a, b = normal((n,), 1), normal((n,), 2)
    got = down(rocm.rocm_gelu_f32(DEV, unaligned(a), n), np.float32, (n,))
    assert_close(got, oracle.gelu(a), what="gelu unaligned")
    got = down(rocm.rocm_swiglu_f32(DEV, unaligned(a), up(b), n), np.float32, (n,))
    assert_close(got, oracle.swiglu(a, b), what="swiglu unaligned")
    buf = up(a)
    rocm.rocm_silu_f32(DEV, buf, n, out=buf)
    assert_close(down(buf, np.float32, (n,)), oracle.silu(a), what="silu in place")


@pytest.mark.slow
def test_swiglu_gelu_baseline_full():
    # gate, up [16384, 14336] ~ N(0,1); GELU on the same shape
    shape = (16384, 14336)
    n = shape[0] * shape[1]
    log("swiglu/gelu baseline full: generating inputs")
    gate = normal(shape, 0)
    upv = normal(shape, 1)
    out = rocm.rocm_swiglu_f32(DEV, up(gate), up(upv), n)
    got = down(out, np.float32, shape)
    del out
    log("swiglu: oracle")
    want = oracle.swiglu(gate, upv, threads=16)
    assert_close(got, want, what="swiglu full")
    log(f"swiglu max abs/rel err {max_err(got, want)}")
    del got, want, upv
    out = rocm.rocm_gelu_f32(DEV, up(gate), n)
    got = down(out, np.float32, shape)
    del out
    log("gelu: oracle")
    want = oracle.gelu(gate)
    assert_close(got, want, what="gelu full")
    log(f"gelu max abs/rel err {max_err(got, want)}")


def test_swiglu_against_serve_silu_specials():
    # The serving caller composes kore-serve's two-branch silu with mul
    # (crates/kore-serve/src/layered/engine.rs:640-643, :828-842); the kernel
    # follows kore-nn's form.  Both must sit within the f32 bar of that caller.
    gate = np.concatenate([np.linspace(-120, 40, 40001, dtype=np.float32),
                           np.array([-88.72, -88.73, -87.0, -103.0, -104.0, -0.0, 0.0, 1e-30, -1e-30,
                                     np.inf, -np.inf, np.nan, 3.4e38, -3.4e38], np.float32)])
    upv = normal(gate.shape, 16)
    got = down(rocm.rocm_swiglu_f32(DEV, up(gate), up(upv), gate.size), np.float32, gate.shape)
    assert_close(got, oracle.swiglu_serve(gate, upv), what="swiglu vs serve silu")


@pytest.mark.slow
def test_swiglu_against_serve_silu_full():
    # BASELINE configs[2] shape against the serve composition
    shape = (16384, 14336)
    log("swiglu vs serve silu full")
    gate = normal(shape, 0)
    upv = normal(shape, 1)
    got = down(rocm.rocm_swiglu_f32(DEV, up(gate), up(upv), gate.size), np.float32, shape)
    want = oracle.swiglu_serve(gate, upv)
    assert_close(got, want, what="swiglu vs serve silu full")
    log(f"swiglu vs serve max abs/rel err {max_err(got, want)}")


# -------------------------------------------------------------------- RoPE
@pytest.mark.parametrize("interleaved", [False, True])
@pytest.mark.parametrize("batch,seq,heads,hd,start", [(1, 1, 1, 4, 0), (2, 5, 3, 8, 7), (1, 3, 2, 6, 0),
                                                      (2, 9, 4, 128, 100000), (1, 17, 5, 64, 3),
                                                      (3, 4, 2, 2, 1), (1, 3, 3, 32, 5), (2, 3, 2, 256, 2047),
                                                      (1, 2, 9, 128, 0)])
def test_rope_small(interleaved, batch, seq, heads, hd, start):
    log(f"rope b={batch} s={seq} h={heads} d={hd} start={start} interleaved={interleaved}")
    x = normal((batch, seq, heads, hd), seq * hd + heads)
    buf = up(x)
    inv = rocm.rocm_rope_inv_freq_f32(DEV, hd, 10000.0)
    rocm.rocm_rope_f32(DEV, buf, inv, batch, seq, heads, hd, start, interleaved)
    got = down(buf, np.float32, x.shape)
    want = oracle.rope(x, start, 10000.0, interleaved)
    assert_close(got, want, what="rope")


@pytest.mark.parametrize("seed", range(4))
def test_rope_and_embedding_random_shapes(seed):
    """Seeded random shapes for RoPE (both layouts, every head width the
    per-lane kernel takes and some it does not, start positions, table and
    data offsets) and for the embedding gather (row widths on each side of
    the one-float4 kernel's limits, ids out of range): RoPE within the
    element-wise tolerance, the gather bit-exact."""
    r = np.random.default_rng(3000 + seed)
    for case in range(6):
        hd = int(r.choice([2, 4, 6, 8, 16, 32, 64, 128, 256, 96, 200]))
        batch, seq, heads = int(r.integers(1, 4)), int(r.integers(1, 300)), int(r.integers(1, 9))
        start, interleaved = int(r.integers(0, 5000)), bool(r.integers(0, 2))
        off = 4 * int(r.integers(0, 4)) if r.random() < 0.3 else 0
        log(f"rope random seed={seed} case={case} b={batch} s={seq} h={heads} d={hd} start={start} "
            f"interleaved={interleaved} x+{off}")
        x = normal((batch, seq, heads, hd), 500 * seed + case)
        buf = _offset_buffer(x, off) if off else up(x)
        inv = rocm.rocm_rope_inv_freq_f32(DEV, hd, 10000.0)
        rocm.rocm_rope_f32(DEV, buf, inv, batch, seq, heads, hd, start, interleaved)
        assert_close(down(buf, np.float32, x.shape), oracle.rope(x, start, 10000.0, interleaved), what="rope random")
        vocab = int(r.integers(1, 3000))
        dim = int(r.choice([1, 3, 4, 8, 100, 256, 1000, 4096, 4100, 8192, 12288]))
        n_ids = int(r.integers(1, 300))
        log(f"embedding random seed={seed} case={case} vocab={vocab} dim={dim} n={n_ids}")
        table = normal((vocab, dim), 600 * seed + case, 0.0, 0.02)
        ids = r.integers(0, vocab + 3, size=n_ids).astype(np.int32)  # some past the vocabulary
        out = rocm.rocm_embedding_f32(DEV, up(table), up(ids), n_ids, vocab, dim)
        assert down(out, np.float32, (n_ids, dim)).tobytes() == oracle.embedding(table, ids).tobytes()


def test_rope_unaligned_scalar_path():
    x = normal((2, 6, 3, 16), 5)
    buf = unaligned(x)
    inv = rocm.rocm_rope_inv_freq_f32(DEV, 16, 10000.0)
    rocm.rocm_rope_f32(DEV, buf, inv, 2, 6, 3, 16, 11, False)
    assert_close(buf.tensor(torch.float32).cpu().numpy().reshape(x.shape), oracle.rope(x, 11, 10000.0),
                 what="rope unaligned")



@pytest.mark.parametrize("interleaved", [False, True])
@pytest.mark.parametrize("hq,hk,hd", [(5, 3, 64), (9, 1, 128), (3, 2, 32), (2, 1, 256)])
def test_rope_qk_small(interleaved, hq, hk, hd):
    """The fused Q+K launch on head counts whose rows fill no whole
    workgroup, for every head_dim of the one-float4-per-thread path."""
    log(f"rope qk small hq={hq} hk={hk} d={hd} interleaved={interleaved}")
    q = normal((2, 7, hq, hd), 40 + hq)
    k = normal((2, 7, hk, hd), 50 + hk)
    qb, kb = up(q), up(k)
    inv = rocm.rocm_rope_inv_freq_f32(DEV, hd, 10000.0)
    rocm.rocm_rope_qk_f32(DEV, qb, kb, inv, 2, 7, hq, hk, hd, 3, interleaved)
    assert_close(down(qb, np.float32, q.shape), oracle.rope(q, 3, 10000.0, interleaved), what="rope q")
    assert_close(down(kb, np.float32, k.shape), oracle.rope(k, 3, 10000.0, interleaved), what="rope k")

@pytest.mark.slow
@pytest.mark.parametrize("interleaved", [False, True])
def test_rope_qk_baseline_full(interleaved):
    # Q[8,2048,32,128], K[8,2048,8,128] ~ N(0,1), theta 1e4, positions 0..2047
    log(f"rope qk baseline full interleaved={interleaved}")
    q = normal((8, 2048, 32, 128), 0)
    k = normal((8, 2048, 8, 128), 1)
    qb, kb = up(q), up(k)
    inv = rocm.rocm_rope_inv_freq_f32(DEV, 128, 10000.0)
    rocm.rocm_rope_qk_f32(DEV, qb, kb, inv, 8, 2048, 32, 8, 128, 0, interleaved)
    gq = down(qb, np.float32, q.shape)
    gk = down(kb, np.float32, k.shape)
    wq = oracle.rope(q, 0, 10000.0, interleaved)
    assert_close(gq, wq, what="rope q")
    log(f"rope q max abs/rel err {max_err(gq, wq)}")
    wk = oracle.rope(k, 0, 10000.0, interleaved)
    assert_close(gk, wk, what="rope k")
    # the fused launch equals two single-tensor launches
    qb2 = up(q)
    rocm.rocm_rope_f32(DEV, qb2, inv, 8, 2048, 32, 128, 0, interleaved)
    assert down(qb2, np.float32, q.shape).tobytes() == gq.tobytes()


# --------------------------------------------------------------- Embedding
@pytest.mark.parametrize("vocab,dim,n_ids", [(10, 4, 3), (50, 7, 20), (1000, 256, 513), (64, 4096, 100),
                                             (3, 2, 3), (100, 4100, 9)])
def test_embedding_bit_exact(vocab, dim, n_ids):
    log(f"embedding vocab={vocab} dim={dim} n={n_ids}")
    table = normal((vocab, dim), vocab, 0.0, 0.02)
    ids = embedding_ids(n_ids, vocab, seed=n_ids)
    ids[0] = vocab          # out of range -> zeros
    if n_ids > 2:
        ids[1] = -1         # negative int32 -> u32 max -> zeros
        ids[2] = vocab - 1
    out = rocm.rocm_embedding_f32(DEV, up(table), up(ids), n_ids, vocab, dim)
    got = down(out, np.float32, (n_ids, dim))
    assert got.tobytes() == oracle.embedding(table, ids).tobytes()


def test_embedding_reference_kat_on_device():
    # crates/kore-edge/src/ops/embedding.rs:33-41
    w = np.array([1, 2, 3, 4, 5, 6], np.float32)
    out = rocm.rocm_embedding_f32(DEV, up(w), up(np.array([0, 2, 1], np.uint32)), 3, 3, 2)
    assert down(out, np.float32, (6,)).tolist() == [1.0, 2.0, 5.0, 6.0, 3.0, 4.0]


def test_embedding_unaligned():
    table = normal((20, 8), 2)
    ids = np.array([3, 19, 0, 25], np.int32)
    out = rocm.rocm_embedding_f32(DEV, unaligned(table), up(ids), 4, 20, 8)
    assert down(out, np.float32, (4, 8)).tobytes() == oracle.embedding(table, ids).tobytes()


@pytest.mark.slow
def test_embedding_baseline_full():
    # table[128256,4096] ~ N(0,0.02), ids int32[8192], 5% repeats
    log("embedding baseline full")
    table = normal((128256, 4096), 0, 0.0, 0.02)
    ids = embedding_ids(8192, 128256, seed=0)
    assert len(np.unique(ids)) < 8192  # repeats present
    out = rocm.rocm_embedding_f32(DEV, up(table), up(ids), 8192, 128256, 4096)
    got = down(out, np.float32, (8192, 4096))
    assert got.tobytes() == oracle.embedding(table, ids).tobytes()


# Embedding::forward: f32 ids through Rust's `as usize` (embedding.rs:91-98)
F32_ID_SPECIALS = [float("nan"), -1.5, 0.9, 1e30, -0.0, float("inf"), -float("inf"), 2.0, 2.5]


@pytest.mark.parametrize("vocab,dim,n_ids", [(10, 4, 16), (1000, 256, 513), (64, 4096, 100), (100, 4100, 12),
                                             (30, 7, 20)])
def test_embedding_forward_f32_ids(vocab, dim, n_ids):
    log(f"embedding forward f32 ids vocab={vocab} dim={dim} n={n_ids}")
    table = normal((vocab, dim), vocab + 1, 0.0, 0.02)
    ids = embedding_ids(n_ids, vocab, seed=n_ids + 1).astype(np.float32)
    sp = F32_ID_SPECIALS + [float(vocab - 1), float(vocab), float(vocab + 1)]
    ids[:len(sp)] = np.array(sp[:n_ids], np.float32)
    out = rocm.rocm_embedding_forward_f32(DEV, up(table), up(ids), n_ids, vocab, dim)
    got = down(out, np.float32, (n_ids, dim))
    assert got.tobytes() == oracle.embedding_forward(table, ids).tobytes()


def test_embedding_forward_f32_ids_unaligned_table():
    table = normal((20, 8), 3)
    ids = np.array([3.7, float("nan"), 19.0, 20.0, -2.0], np.float32)
    out = rocm.rocm_embedding_forward_f32(DEV, unaligned(table), up(ids), 5, 20, 8)
    assert down(out, np.float32, (5, 8)).tobytes() == oracle.embedding_forward(table, ids).tobytes()


@pytest.mark.slow
def test_embedding_forward_baseline_shape():
    # BASELINE configs[3] shape with the ids handed over as f32, as Module::forward takes them
    log("embedding forward f32 ids baseline shape")
    table = normal((128256, 4096), 0, 0.0, 0.02)
    ids = embedding_ids(8192, 128256, seed=0).astype(np.float32)
    ids[:9] = np.array(F32_ID_SPECIALS, np.float32)
    out = rocm.rocm_embedding_forward_f32(DEV, up(table), up(ids), 8192, 128256, 4096)
    got = down(out, np.float32, (8192, 4096))
    assert got.tobytes() == oracle.embedding_forward(table, ids).tobytes()


# ----------------------------------------------------------------- softmax
# Tolerances.  The reference folds its sums left to right in f32, so its own
# result is only within the recursive-summation bound gamma_n = n * 2^-24
# (relative to the sum of |terms|) of the exact value; the kernel sums in a
# tree.  Each test therefore checks (a) accuracy: the kernel is within the
# plain f32 tolerance (1e-5 relative / 1e-6 absolute) of an f64 evaluation,
# and (b) parity with the oracle (semantics of NaN, inf, masks, padding) with
# rtol = 1e-5 + n * 2^-24, n = the number of terms the reference folds.
U32 = 2.0 ** -24


def _softmax64(x):
    x = np.asarray(x, np.float64)
    e = np.exp(x - x.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)

# one shape per kernel path: wave per row (<= 256/512/1024/2048/4096 cols),
# workgroup per row (<= 8192/16384), looped (longer rows, cols % 4 != 0)
SOFTMAX_SHAPES = [(1, 1), (3, 7), (5, 4), (4, 256), (7, 260), (9, 512), (6, 1000), (33, 2048), (5, 4096),
                  (5, 1028), (3, 1500),
                  (3, 8192), (2, 16384), (2, 20000), (3, 4099), (2, 128256)]


@pytest.mark.parametrize("rows,cols", SOFTMAX_SHAPES)
def test_softmax(rows, cols):
    log(f"softmax rows={rows} cols={cols}")
    x = normal((rows, cols), rows * 31 + cols) * 4
    got = down(rocm.rocm_softmax_f32(DEV, up(x), rows, cols), np.float32, (rows, cols))
    assert_close(got, _softmax64(x), what="softmax vs f64")
    assert_close(got, oracle.softmax(x), rtol=1e-5 + cols * U32, what="softmax vs oracle")


def test_softmax_special_rows_in_place_and_unaligned():
    log("softmax special rows")
    cols = 300
    x = normal((8, cols), 3) * 2
    x[0, 5] = np.nan
    x[1, :] = -np.inf
    x[2, 7] = np.inf
    x[3, ::3] = -np.inf
    x[4] = 1000.0 + x[4]
    x[5] = -3e38
    x[6, 0] = 3e38
    want = oracle.softmax(x)
    got = down(rocm.rocm_softmax_f32(DEV, up(x), 8, cols), np.float32, (8, cols))
    assert_close(got, want, rtol=1e-5 + cols * U32, what="softmax special")
    for c in (256, 1024, 4096):  # in place, register paths
        xx = normal((5, c), c) * 3
        b = up(xx)
        rocm.rocm_softmax_f32(DEV, b, 5, c, out=b)
        assert_close(down(b, np.float32, (5, c)), _softmax64(xx), what=f"softmax in place {c}")
    xu = normal((4, 512), 11)
    got = down(rocm.rocm_softmax_f32(DEV, unaligned(xu), 4, 512), np.float32, (4, 512))
    assert_close(got, _softmax64(xu), what="softmax unaligned")


@pytest.mark.parametrize("rows,cols,offset", [(6, 8, 0), (6, 8, 3), (40, 64, 0), (300, 256, 0), (17, 2048, 1000),
                                              (3, 8192, 4000), (2, 20000, 9999), (9, 4099, 10), (4, 33, 100),
                                              (7, 1028, 5), (5, 1500, 700)])
def test_softmax_causal(rows, cols, offset):
    log(f"softmax_causal rows={rows} cols={cols} offset={offset}")
    x = normal((rows, cols), rows + cols + offset) * 3
    got = down(rocm.rocm_softmax_causal_f32(DEV, up(x), rows, cols, offset), np.float32, (rows, cols))
    want = oracle.softmax_causal(x, offset)
    lim = np.minimum(offset + np.arange(rows) + 1, cols)
    assert_close(got, want, rtol=1e-5 + int(lim.max()) * U32, what="softmax_causal vs oracle")
    exact = np.zeros((rows, cols))
    for r in range(rows):
        exact[r, :lim[r]] = _softmax64(x[r, :lim[r]])
    assert_close(got, exact, what="softmax_causal vs f64")
    # masked entries are exact zeros
    mask = np.arange(cols)[None, :] >= lim[:, None]
    assert (got[mask] == 0.0).all()


def _softmax_bwd_scale(y, dy):
    y64, dy64 = y.astype(np.float64), dy.astype(np.float64)
    dot_abs = np.abs(y64 * dy64).sum(axis=-1, keepdims=True)
    return np.abs(y64) * (np.abs(dy64) + dot_abs)


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 7), (4, 256), (9, 512), (33, 2048), (5, 4096), (3, 8192),
                                       (2, 16384), (2, 20000), (3, 4099), (4, 1028), (6, 1500)])
def test_softmax_backward(rows, cols):
    log(f"softmax_backward rows={rows} cols={cols}")
    y = oracle.softmax(normal((rows, cols), cols) * 3)
    dy = normal((rows, cols), cols + 1)
    got = down(rocm.rocm_softmax_backward_f32(DEV, up(dy), up(y), rows, cols), np.float32, (rows, cols))
    want = oracle.softmax_backward(dy, y)
    assert_close_scaled(got, want, _softmax_bwd_scale(y, dy), rtol=1e-5 + cols * U32, what="softmax_backward")


def test_softmax_backward_reference_kat_on_device():
    # cpu_fused_backward.rs:236-248: uniform upstream gradient -> ~0
    y = np.array([[0.2, 0.3, 0.5]], np.float32)
    got = down(rocm.rocm_softmax_backward_f32(DEV, up(np.ones((1, 3), np.float32)), up(y), 1, 3), np.float32, (1, 3))
    assert np.abs(got).max() < 1e-6


# -------------------------------------------------------- RMSNorm backward
def _rms_bwd_scales(dy, x, g, eps):
    x64, dy64, g64 = x.astype(np.float64), dy.astype(np.float64), g.astype(np.float64)
    cols = x.shape[1]
    ss = (x64 * x64).sum(axis=1, keepdims=True)
    inv = 1.0 / np.sqrt(ss / cols + eps)
    coeff_abs = np.abs(x64 * dy64 * g64).sum(axis=1, keepdims=True) * inv / (ss + eps * cols)
    sdx = np.abs(g64) * inv * np.abs(dy64) + coeff_abs * np.abs(x64)
    sdg = (np.abs(dy64 * x64) * inv).sum(axis=0)
    return sdx, sdg


# vector path split over 1/2/4 waves, several row iterations, generic path
RMS_BWD_SHAPES = [(1, 4), (3, 7), (16, 64), (100, 256), (33, 1000), (64, 2048), (10, 4096), (5, 8192), (4099, 512),
                  (2000, 2050), (20000, 1024)]


@pytest.mark.parametrize("rows,cols", RMS_BWD_SHAPES)
def test_rms_norm_backward(rows, cols):
    log(f"rms_norm_backward rows={rows} cols={cols}")
    x, g = rmsnorm_inputs(rows, cols, seed=rows + cols)
    dy = normal((rows, cols), rows * 3 + cols)
    gx, gg = rocm.rocm_rms_norm_backward_f32(DEV, up(dy), up(x), up(g), rows, cols, 1e-5)
    dx_w, dg_w = oracle.rms_norm_backward(dy, x, g, 1e-5)
    sdx, sdg = _rms_bwd_scales(dy, x, g, 1e-5)
    assert_close_scaled(down(gx, np.float32, (rows, cols)), dx_w, sdx, rtol=1e-5 + cols * U32,
                        what="rms_norm_backward dx")
    assert_close_scaled(down(gg, np.float32, (cols,)), dg_w, sdg, rtol=1e-5 + rows * U32,
                        what="rms_norm_backward dgamma")


def test_rms_norm_backward_deterministic_and_edge_cases():
    log("rms_norm_backward determinism / edges")
    rows, cols = 3000, 2048
    x, g = rmsnorm_inputs(rows, cols, seed=1)
    dy = normal((rows, cols), 2)
    a = rocm.rocm_rms_norm_backward_f32(DEV, up(dy), up(x), up(g), rows, cols, 1e-5)
    b = rocm.rocm_rms_norm_backward_f32(DEV, up(dy), up(x), up(g), rows, cols, 1e-5)
    assert a[0].to_host(np.uint8).tobytes() == b[0].to_host(np.uint8).tobytes()
    assert a[1].to_host(np.uint8).tobytes() == b[1].to_host(np.uint8).tobytes()
    # zero upstream gradient -> zeros (cpu_fused_backward.rs:220-234)
    gx, gg = rocm.rocm_rms_norm_backward_f32(DEV, up(np.zeros((1, 3), np.float32)),
                                             up(np.array([[1.0, 2.0, 3.0]], np.float32)), up(np.ones(3, np.float32)),
                                             1, 3, 1e-5)
    assert np.abs(gx.to_host(np.float32)[:3]).max() < 1e-6 and np.abs(gg.to_host(np.float32)[:3]).max() < 1e-6
    # rows == 0 zeroes grad_gamma
    gg0 = up(np.full(64, 7.0, np.float32))
    rocm.rocm_rms_norm_backward_f32(DEV, up(np.zeros(4, np.float32)), up(np.zeros(4, np.float32)),
                                    up(np.ones(64, np.float32)), 0, 64, 1e-5, grad_gamma=gg0)
    assert (gg0.to_host(np.float32)[:64] == 0.0).all()
    # unaligned views take the generic path
    xu, dyu = normal((7, 256), 3), normal((7, 256), 4)
    gu = np.ones(256, np.float32)
    gx, gg = rocm.rocm_rms_norm_backward_f32(DEV, unaligned(dyu), unaligned(xu), up(gu), 7, 256, 1e-5)
    dx_w, dg_w = oracle.rms_norm_backward(dyu, xu, gu, 1e-5)
    sdx, sdg = _rms_bwd_scales(dyu, xu, gu, 1e-5)
    assert_close_scaled(down(gx, np.float32, (7, 256)), dx_w, sdx, rtol=1e-5 + 256 * U32, what="unaligned dx")
    assert_close_scaled(down(gg, np.float32, (256,)), dg_w, sdg, rtol=1e-5 + 7 * U32, what="unaligned dgamma")


# -------------------------------------------------- cross-entropy backward
@pytest.mark.parametrize("batch,classes", [(1, 1), (3, 7), (2, 3), (64, 256), (17, 1000), (8, 4096), (4, 8192),
                                           (3, 32000), (2, 128256), (5, 4099), (9, 2048), (5, 1500)])
def test_cross_entropy_backward(batch, classes):
    log(f"cross_entropy_backward batch={batch} classes={classes}")
    x = normal((batch, classes), batch + classes) * 3
    t = (np.arange(batch) * 7919 % classes).astype(np.float32)
    got = down(rocm.rocm_cross_entropy_backward_f32(DEV, up(x), up(t), batch, classes), np.float32, (batch, classes))
    want = oracle.cross_entropy_backward(x, t)
    assert_close(got, want, rtol=1e-5 + classes * U32, what="cross_entropy_backward vs oracle")
    e = np.exp(x.astype(np.float64) - x.max(axis=1, keepdims=True))
    ref = e / e.sum(axis=1, keepdims=True)
    ref[np.arange(batch), t.astype(int)] -= 1.0
    assert_close(got, ref / batch, what="cross_entropy_backward vs f64")


def test_cross_entropy_backward_target_cast_and_in_place():
    log("cross_entropy_backward targets / in place")
    for classes in (4, 256, 20000):  # register and looped paths
        x = normal((6, classes), classes) * 2
        t = np.array([2.7, -3.0, np.nan, 0.5, classes + 1.0, classes - 1], np.float32)
        b = up(x)
        rocm.rocm_cross_entropy_backward_f32(DEV, b, up(t), 6, classes, out=b)
        assert_close(down(b, np.float32, (6, classes)), oracle.cross_entropy_backward(x, t),
                     rtol=1e-5 + classes * U32, what=f"ce targets {classes}")


# ---------------------------------------------------- ternary (BitLinear i8)
TERN_SHAPES = [(1, 1, 16), (3, 5, 16), (128, 128, 160), (129, 130, 320), (200, 77, 2560), (64, 33, 6912),
               (5, 7, 13), (33, 65, 1000), (6912, 1, 2560), (300, 64, 2560), (17, 300, 2576)]


@pytest.mark.parametrize("m,n,k", TERN_SHAPES)
def test_ternary_matmul_i8(m, n, k):
    """Bit-exact against the oracle (integer dot product, the ternary_ternary
    epilogue), on arbitrary packed bytes: bytes >= 243 and nonzero padding
    trits past k included."""
    from inputs import int8_codes, raw_packed

    log(f"ternary_matmul_i8 m={m} n={n} k={k}")
    p = raw_packed(m, k, m + k)
    q = int8_codes(n, k, n + 1)
    sa = normal((m,), 3, 1.0, 0.1)
    sq = np.abs(normal((n,), 4, 0.02, 0.005))
    got = down(rocm.rocm_ternary_matmul_i8(DEV, up(p), up(sa), up(q), up(sq), m, n, k), np.float32, (m, n))
    assert_bitexact(got, oracle.ternary_matmul_i8(p, sa, q, sq, m, n, k), "ternary_matmul_i8")


@pytest.mark.parametrize("m,n,k", [(7, 1, 2560), (6912, 1, 2560), (130, 2, 1000), (257, 3, 6912), (64, 4, 8),
                                   (2560, 1, 6920), (300, 2, 5000), (61, 4, 4096), (9, 1, 12800), (3, 3, 2568),
                                   (2560, 8, 6920), (130, 6, 2560), (77, 5, 336),
                                   (2560, 64, 6912), (1000, 33, 2576), (7, 40, 6912), (300, 9, 160), (600, 100, 2560),
                                   (33, 8, 2568), (100, 9, 5128), (6912, 16, 2560), (5, 16, 40), (1, 12, 7688),
                                   (129, 17, 2560), (6912, 64, 2560), (70, 40, 6920)])
def test_ternary_matmul_i8_small_n(m, n, k):
    """The small-n path (n <= 8: 1, 2 or 4 waves per 4 weight rows, dot4 over
    40-column lane windows, K in 2560-column chunks shared by the waves;
    8-byte-aligned and unaligned packed rows), the skinny MFMA path (n <= 64:
    32 weight rows per workgroup, K split over 8 waves, aligned and unaligned
    packed rows) and the n past it
    (split-K MFMA tiles with integer atomics): bit-exact against the oracle on
    arbitrary packed bytes, ragged m, odd packed-row lengths and k % 16 != 0."""
    from inputs import int8_codes, raw_packed

    log(f"ternary_matmul_i8 small n m={m} n={n} k={k}")
    p = raw_packed(m, k, 3 * m + k)
    q = int8_codes(n, k, n + 7)
    sa = normal((m,), 8, 1.0, 0.1)
    sq = np.abs(normal((n,), 9, 0.02, 0.005))
    got = down(rocm.rocm_ternary_matmul_i8(DEV, up(p), up(sa), up(q), up(sq), m, n, k), np.float32, (m, n))
    assert_bitexact(got, oracle.ternary_matmul_i8(p, sa, q, sq, m, n, k), "ternary_matmul_i8 small n")


@pytest.mark.parametrize("m,n,k", [(4096, 3072, 640), (4100, 3000, 560), (6400, 2000, 320), (3333, 3900, 80),
                                   (4096, 3072, 160), (300, 49152, 160), (49200, 300, 160)])
def test_ternary_matmul_i8_wide_tiles(m, n, k):
    """The wide path (at least 144 output tiles of 256 x 256, 16-byte packed
    rows; at these few K steps 256 x 128 tiles, two workgroups per CU):
    whole and ragged tiles, a partial last K step (k % 160 != 0), a partial
    single step and a whole one; bit-exact against the oracle on arbitrary
    packed bytes (bytes >= 243 included)."""
    from inputs import int8_codes, raw_packed

    log(f"ternary_matmul_i8 wide m={m} n={n} k={k}")
    p = raw_packed(m, k, m + 3 * k)
    q = int8_codes(n, k, n + 11)
    sa = normal((m,), 12, 1.0, 0.1)
    sq = np.abs(normal((n,), 13, 0.02, 0.005))
    got = down(rocm.rocm_ternary_matmul_i8(DEV, up(p), up(sa), up(q), up(sq), m, n, k), np.float32, (m, n))
    assert_bitexact(got, oracle.ternary_matmul_i8(p, sa, q, sq, m, n, k), "ternary_matmul_i8 wide")


def test_ternary_matmul_i8_wide_tiles_unaligned_output():
    """The wide path with an output 4 bytes past a 16-byte boundary (n % 4 ==
    0): its epilogue stores element by element instead of 16-byte rows."""
    from inputs import int8_codes, raw_packed

    m, n, k = 4100, 3072, 560
    log(f"ternary_matmul_i8 wide unaligned c m={m} n={n} k={k}")
    lib = __import__("kore_amd._lib", fromlist=["load"]).load()
    p = raw_packed(m, k, 17)
    q = int8_codes(n, k, 18)
    sa = normal((m,), 19, 1.0, 0.1)
    sq = np.abs(normal((n,), 20, 0.02, 0.005))
    bp, bs, bq, bsq = up(p), up(sa), up(q), up(sq)
    t = torch.full((m * n + 1,), float("nan"), dtype=torch.float32, device="cuda")
    rc = lib.kore_hip_ternary_matmul_i8(bp.ptr, bs.ptr, bq.ptr, bsq.ptr, t[1:].data_ptr(), m, n, k, None)
    torch.cuda.synchronize()
    assert rc == 0
    got = t[1:].cpu().numpy().reshape(m, n)
    assert np.isnan(t[0].item())
    assert_bitexact(got, oracle.ternary_matmul_i8(p, sa, q, sq, m, n, k), "ternary_matmul_i8 wide unaligned c")


@pytest.mark.parametrize("m,n,k,c_off", [(2560, 3901, 1280, 0), (2560, 4096, 1280, 1), (2560, 3901, 1280, 3)])
def test_ternary_matmul_i8_wide_192_ragged_and_unaligned_output(m, n, k, c_off):
    """The 256 x 192 wide tiles (chosen here: 210 such tiles fit one round of
    256 CUs, K has 8 steps) with n % 4 != 0 and with the output 4 or 12
    bytes past a 16-byte boundary: the epilogue's element stores, including
    the skip of lanes past n, on 192-wide tiles.  Bit-exact against an f64
    GEMM of the decoded trits (exact for these integer sums) with the same
    f32 epilogue; the float before the output stays untouched."""
    from inputs import int8_codes, ternary_weights

    log(f"ternary_matmul_i8 wide 192 m={m} n={n} k={k} c_off={c_off}")
    lib = __import__("kore_amd._lib", fromlist=["load"]).load()
    p, sa = ternary_weights(m, k, 41)
    q = int8_codes(n, k, 42)
    sq = np.abs(normal((n,), 43, 0.02, 0.005))
    bp, bs, bq, bsq = up(p), up(sa), up(q), up(sq)
    t = torch.full((m * n + 4,), float("nan"), dtype=torch.float32, device="cuda")
    rc = lib.kore_hip_ternary_matmul_i8(bp.ptr, bs.ptr, bq.ptr, bsq.ptr, t[c_off:].data_ptr(), m, n, k, None)
    torch.cuda.synchronize()
    assert rc == 0
    got = t[c_off:c_off + m * n].reshape(m, n)
    if c_off:
        assert torch.isnan(t[:c_off]).all()
    assert torch.isnan(t[c_off + m * n:]).all()
    tr = torch.from_numpy(oracle.unpack_trits(p, k)).cuda().double()
    acc = (tr @ torch.from_numpy(q).cuda().double().T).float()
    want = (acc * torch.from_numpy(sa).cuda()[:, None]) * torch.from_numpy(sq).cuda()[None, :]
    assert torch.equal(got, want), f"ternary_matmul_i8 wide 192 {m}x{n}x{k} c_off={c_off}"


def test_ternary_matmul_i8_full_size_and_pipeline():
    """BitLinear 2560 -> 6912 on 4096 tokens (the pre-quant config's
    activations): bit-exact against an f64 GEMM of the decoded trits (exact
    for these integer sums) with the same f32 epilogue; then the end-to-end
    chain pre-quant codes -> ternary matmul against the oracle on a slice."""
    from inputs import ternary_weights

    m, n, k = 6912, 4096, 2560
    log(f"ternary_matmul_i8 full size m={m} n={n} k={k}")
    p, sa = ternary_weights(m, k, 21)
    x, g = prequant_inputs(n, k, 0)
    qb, sb = rocm.rocm_rms_norm_quant_i8(DEV, up(x), up(g), n, k, 1e-6)
    c = rocm.rocm_ternary_matmul_i8(DEV, up(p), up(sa), qb, sb, m, n, k)
    got = torch.from_numpy(down(c, np.float32, (m, n))).cuda()
    t = torch.from_numpy(oracle.unpack_trits(p, k)).cuda().double()
    qd = torch.from_numpy(down(qb, np.int8, (n, k))).cuda().double()
    acc = (t @ qd.T).float()
    want = (acc * torch.from_numpy(sa).cuda()[:, None]) * torch.from_numpy(down(sb, np.float32, (n,))).cuda()[None, :]
    assert torch.equal(got, want), "ternary_matmul_i8 full size vs f64 GEMM"
    # the chain on a slice of tokens, against the oracle end to end
    rows = 8
    wq, ws = oracle.rms_norm_quant_i8(x[:rows], g, 1e-6)
    ref = oracle.ternary_matmul_i8(p[:96], sa[:96], wq, ws, 96, rows, k)
    assert_bitexact(got[:96, :rows].cpu().numpy(), ref, "prequant -> ternary chain")


@pytest.mark.parametrize("m,n,k", [(2560, 4096, 6912), (6912, 1024, 2563), (2560, 3900, 1280), (3072, 3072, 1360),
                                   (2600, 4100, 1296), (4096, 4096, 2720), (4096, 4000, 2736)])
def test_ternary_matmul_i8_full_size_unaligned(m, n, k):
    """Full-size shapes: the FFN down-projection 6912 -> 2560 on 4096 tokens
    (1383-byte packed rows, 256 x 192 wide tiles), K = 2563 (code rows not
    16-byte aligned: the tile kernel's window code loads), and 256 x 192 tiles
    with a partial last column tile, aligned and unaligned packed rows; 256 x
    256 tiles with more than 16 K steps (the one-workgroup-per-CU kernel that
    two-workgroup 256 x 128 tiles replace at fewer steps); bit-exact against an f64 GEMM of the decoded trits (exact for these
    integer sums) with the same f32 epilogue."""
    from inputs import int8_codes, ternary_weights

    log(f"ternary_matmul_i8 full size unaligned m={m} n={n} k={k}")
    p, sa = ternary_weights(m, k, 23)
    q = int8_codes(n, k, 24)
    sq = np.abs(normal((n,), 25, 0.02, 0.005))
    c = rocm.rocm_ternary_matmul_i8(DEV, up(p), up(sa), up(q), up(sq), m, n, k)
    got = torch.from_numpy(down(c, np.float32, (m, n))).cuda()
    t = torch.from_numpy(oracle.unpack_trits(p, k)).cuda().double()
    acc = (t @ torch.from_numpy(q).cuda().double().T).float()
    want = (acc * torch.from_numpy(sa).cuda()[:, None]) * torch.from_numpy(sq).cuda()[None, :]
    assert torch.equal(got, want), f"ternary_matmul_i8 {m}x{n}x{k} vs f64 GEMM"


@pytest.mark.parametrize("m,n,k,offset", [(300, 49152, 176, 0), (49200, 300, 176, 0), (4100, 3000, 336, 0),
                                          (300, 49152, 160, 1), (4096, 3072, 640, 3), (2560, 4096, 336, 0),
                                          (3072, 3072, 336, 2)])
def test_ternary_matmul_i8_wide_tiles_unaligned_rows(m, n, k, offset):
    """The wide path on packed rows that are not 16-byte aligned: K = 176 and
    336 (rows of 36 and 68 bytes: a row's last window reaches into the next
    row, whose trits sit past k; the last row's last window reaches the end
    of the matrix), and aligned row lengths at a base 1 or 3 bytes past a
    16-byte boundary.  Bit-exact against the oracle."""
    from inputs import int8_codes, raw_packed

    log(f"ternary_matmul_i8 wide unaligned rows m={m} n={n} k={k} offset={offset}")
    p = raw_packed(m, k, m + 5 * k)
    q = int8_codes(n, k, n + 17)
    sa = normal((m,), 14, 1.0, 0.1)
    sq = np.abs(normal((n,), 15, 0.02, 0.005))
    t = torch.empty(p.size + offset, dtype=torch.uint8, device="cuda")
    t[offset:].copy_(torch.from_numpy(p.ravel()))
    got = down(rocm.rocm_ternary_matmul_i8(DEV, HipBuffer.from_tensor(t[offset:]), up(sa), up(q), up(sq), m, n, k),
               np.float32, (m, n))
    assert_bitexact(got, oracle.ternary_matmul_i8(p, sa, q, sq, m, n, k), "ternary_matmul_i8 wide unaligned rows")


@pytest.mark.parametrize("m,n,k", [(6912, 64, 2563), (1000, 300, 1001), (2560, 3, 6915), (130, 129, 1203),
                                   (7, 9, 3), (2000, 2000, 1001), (33, 17, 2570)])
def test_ternary_matmul_i8_unaligned_code_rows(m, n, k):
    """Code rows that are not 16-byte aligned (K % 16 != 0): the 128 x 128 tile
    kernel with dword-window code loads, zeros at columns >= k, the codes'
    last bytes read one by one; few tiles (split K, integer atomics) and many.
    Bit-exact against the oracle on arbitrary packed bytes."""
    from inputs import int8_codes, raw_packed

    log(f"ternary_matmul_i8 unaligned code rows m={m} n={n} k={k}")
    p = raw_packed(m, k, 7 * m + k)
    q = int8_codes(n, k, n + 19)
    sa = normal((m,), 16, 1.0, 0.1)
    sq = np.abs(normal((n,), 17, 0.02, 0.005))
    got = down(rocm.rocm_ternary_matmul_i8(DEV, up(p), up(sa), up(q), up(sq), m, n, k), np.float32, (m, n))
    assert_bitexact(got, oracle.ternary_matmul_i8(p, sa, q, sq, m, n, k), "ternary_matmul_i8 unaligned code rows")


def test_ternary_matmul_i8_edges():
    log("ternary_matmul_i8 edges")
    lib = __import__("kore_amd._lib", fromlist=["load"]).load()
    # empty work: nothing launched, status 0
    assert lib.kore_hip_ternary_matmul_i8(None, None, None, None, None, 0, 5, 16, None) == 0
    assert lib.kore_hip_ternary_matmul_i8(None, None, None, None, None, 5, 0, 16, None) == 0
    # k = 0: every dot product is 0
    sa, sq = np.ones(3, np.float32), np.ones(4, np.float32)
    c = rocm.rocm_ternary_matmul_i8(DEV, up(np.zeros(1, np.uint8)), up(sa), up(np.zeros(1, np.int8)), up(sq),
                                    3, 4, 0)
    assert (down(c, np.float32, (3, 4)) == 0).all()
    # argument errors
    assert lib.kore_hip_ternary_matmul_i8(None, None, None, None, None, 2, 2, 16, None) == -1
    assert lib.kore_hip_ternary_matmul_i8(1, 1, 1, 1, 1, 2, 2, (1 << 24) + 1, None) == -3
    # the output may not overlap an input
    cb = up(np.zeros(64 * 64 + 64 * 16, np.float32))
    assert lib.kore_hip_ternary_matmul_i8(1 << 40, 1 << 41, cb.ptr, 1 << 42, cb.ptr, 4, 4, 16, None) == -4
    # codes 1 byte past an aligned base (the tile kernel's window loads)
    m, n, k = 40, 9, 320
    from inputs import int8_codes, raw_packed

    p, q = raw_packed(m, k, 1), int8_codes(n, k, 2)
    sa, sq = normal((m,), 5), normal((n,), 6)
    t = torch.empty(n * k + 1, dtype=torch.int8, device="cuda")
    t[1:].copy_(torch.from_numpy(q.ravel()))
    got = down(rocm.rocm_ternary_matmul_i8(DEV, up(p), up(sa), HipBuffer.from_tensor(t[1:]), up(sq), m, n, k),
               np.float32, (m, n))
    assert_bitexact(got, oracle.ternary_matmul_i8(p, sa, q, sq, m, n, k), "ternary unaligned q")


TERN_F32_SHAPES = [(1, 1, 5), (7, 1, 2560), (6912, 1, 2560), (33, 3, 161), (64, 5, 1000), (130, 17, 320),
                   (65, 64, 2560), (9, 65, 2563), (257, 130, 799), (2, 200, 6920), (40, 33, 0), (6500, 64, 320),
                   (301, 24, 640),
                   # one column (the decode-step kernel): any packed-row alignment, partial
                   # last steps, more workgroups than CUs, and matrices whose last bytes
                   # sit at the end of the allocation (m * kp as small as 12)
                   (1, 1, 60), (3, 1, 21), (2, 1, 30), (37, 1, 333), (65, 1, 245), (300, 1, 1203),
                   (2560, 1, 6912), (20000, 1, 480), (129, 1, 241),
                   # two to four columns (the same kernel with one fold wave per column)
                   (6912, 2, 2560), (301, 4, 1203), (1, 2, 60), (129, 3, 241), (5, 4, 24), (2560, 3, 6912),
                   # fewer than 20 packed bytes with up to four columns (the per-lane kernel)
                   (3, 4, 25), (1, 3, 90),
                   # 5+ columns (the row-broadcast kernel): 16-column tiles (5-16 columns,
                   # four row slots a wave), 32-column tiles (17-32, two slots) and
                   # 64-column tiles; one, two and four rows per lane, masked columns,
                   # several column blocks, unaligned rows, a single whole chunk and
                   # partial last chunks
                   (300, 6, 1203), (2560, 8, 6912), (65, 5, 333), (6912, 16, 2560), (12300, 9, 160),
                   (1, 16, 80), (7, 12, 85), (130, 20, 1203), (6200, 20, 320), (2001, 32, 2563), (13, 17, 5),
                   (300, 64, 333), (100, 64, 80), (4000, 64, 165), (6501, 40, 250), (6200, 128, 400),
                   (1000, 100, 1000),
                   # 64-column tiles with five and seven rows per lane (many rows)
                   (10000, 64, 165), (13824, 64, 320), (6912, 128, 85)]


@pytest.mark.parametrize("m,n,k", TERN_F32_SHAPES)
def test_ternary_matmul_f32(m, n, k):
    """The f32-activation ternary_matmul (BitLinear::forward's matmul):
    bit-exact against the oracle's sequential fold, on arbitrary packed bytes
    (bytes >= 243, nonzero padding trits past k), every column-tile width and
    rows-per-lane choice, and K with a partial last chunk."""
    from inputs import raw_packed

    log(f"ternary_matmul_f32 m={m} n={n} k={k}")
    p = raw_packed(m, k, 5 * m + k) if k else np.zeros((m, 1), np.uint8)
    sa = normal((m,), 11, 1.0, 0.1)
    b = normal((k, n), 12) if k else np.zeros(1, np.float32)
    got = down(rocm.rocm_ternary_matmul_f32(DEV, up(p), up(sa), up(b), m, n, k), np.float32, (m, n))
    assert_bitexact(got, oracle.ternary_matmul(p, sa, b, m, n, k), "ternary_matmul_f32")


@pytest.mark.parametrize("n", [1, 2])
def test_ternary_matmul_f32_order_and_nonfinite(n):
    """Cancellation that only the reference's k order produces, and Inf/NaN
    activations at zero-trit positions (skipped by the reference) next to
    ones at nonzero trits (propagated); one column runs the decode-step
    kernel."""
    log(f"ternary_matmul_f32 order and non-finite n={n}")
    m, k = 3, 400
    w = np.zeros((m, k), np.float32)
    w[0, :3] = 1.0              # row 0: b0 + b1 + b2 in order
    w[1, 0] = 1.0; w[1, 5] = -1.0  # row 1: zero trits over the Inf/NaN positions
    w[2, 7] = 1.0               # row 2: picks up the Inf
    p, sa = oracle.pack_weights_ternary(w, 0.3)
    b = np.zeros((k, n), np.float32)
    b[0, :] = 1e8; b[1, :] = 1.0; b[2, :] = -1e8  # sequential: (1e8 + 1) - 1e8 = 0, not 1
    b[3, 0] = np.inf; b[5, :] = 2.0; b[7, 0] = np.inf
    if n > 1:
        b[4, 1] = np.nan
    want = oracle.ternary_matmul(p, sa, b, m, n, k)
    assert want[0, 0] == 0.0 and np.isfinite(want[1]).all() and np.isinf(want[2, 0])
    got = down(rocm.rocm_ternary_matmul_f32(DEV, up(p), up(sa), up(b), m, n, k), np.float32, (m, n))
    assert_bitexact(got, want, "ternary_matmul_f32 order/non-finite")



@pytest.mark.parametrize("m,n", [(130, 40), (4000, 64), (6500, 64), (300, 8), (12300, 16), (2000, 24), (6200, 32),
                                 (10000, 64), (13824, 64)])
def test_ternary_matmul_f32_rows_nonfinite(m, n):
    """5+ columns (the row-broadcast kernel: 16-, 32- and 64-column tiles,
    one, two, four, five and seven rows per lane): Inf/NaN activations in some chunks and columns only, and finite
    activations whose sum overflows; a chunk that meets them is redone with
    zero trits skipped and later chunks stay on that path.  Bit-exact against
    the oracle, non-finite outputs included."""
    from inputs import raw_packed

    k = 1203
    log(f"ternary_matmul_f32 rows non-finite m={m} n={n} k={k}")
    p, sa, b = raw_packed(m, k, 31), normal((m,), 32, 1.0, 0.1), normal((k, n), 33)
    b[5, 0] = np.inf; b[250, n - 1] = -np.inf; b[777, 0] = np.nan; b[1200, n // 2] = np.inf
    b[400:404, 3] = 3e38
    want = oracle.ternary_matmul(p, sa, b, m, n, k)
    assert np.isfinite(want).any() and not np.isfinite(want).all()
    got = down(rocm.rocm_ternary_matmul_f32(DEV, up(p), up(sa), up(b), m, n, k), np.float32, (m, n))
    assert_bitexact(got, want, f"ternary_matmul_f32 rows non-finite m={m} n={n}")


@pytest.mark.parametrize("n", [1, 3, 16, 64])
def test_ternary_matmul_f32_subnormal_activations(n):
    """Subnormal activations and signed zeros: every fold step is the
    reference's IEEE f32 add with gradual underflow (no flush to zero),
    bit-exact against the oracle (one and three columns: the decode-step
    kernel; 16 and 64: the row-broadcast kernel)."""
    from inputs import raw_packed

    m, k = 257, 803
    log(f"ternary_matmul_f32 subnormal m={m} n={n} k={k}")
    p, sa = raw_packed(m, k, 41), normal((m,), 42, 1.0, 0.1)
    b = (normal((k, n), 43) * np.float32(1e-39)).astype(np.float32)
    b[::7] = np.float32(-0.0)
    b[::11] = np.float32(0.0)
    b[5::13] = np.float32(1e-45)
    assert (np.abs(b[b != 0]) < np.finfo(np.float32).tiny).all()
    want = oracle.ternary_matmul(p, sa, b, m, n, k)
    got = down(rocm.rocm_ternary_matmul_f32(DEV, up(p), up(sa), up(b), m, n, k), np.float32, (m, n))
    assert_bitexact(got, want, f"ternary_matmul_f32 subnormal n={n}")

# Shapes that give the fp32 matrix-core kernel (64 rows x 16 columns per
# wave) at least 768 waves: whole and ragged row blocks, column groups and
# 80-column chunks, odd packed-row lengths (unaligned rows), K of one byte.
TERN_F32_MFMA_SHAPES = [(6912, 128, 2560), (3000, 300, 403), (2049, 500, 81), (6200, 130, 1), (5000, 200, 5),
                        (12288, 64, 161), (777, 1030, 333)]


@pytest.mark.parametrize("m,n,k", TERN_F32_MFMA_SHAPES)
def test_ternary_matmul_f32_matrix_cores(m, n, k):
    """The f32-activation ternary_matmul on the fp32 matrix cores (each
    v_mfma_f32_16x16x1_4b_f32 step one fused multiply-add per output, in k
    order): bit-exact against the oracle's sequential fold on arbitrary
    packed bytes."""
    from inputs import raw_packed

    log(f"ternary_matmul_f32 matrix cores m={m} n={n} k={k}")
    p = raw_packed(m, k, 7 * m + k)
    sa = normal((m,), 13, 1.0, 0.1)
    b = normal((k, n), 14)
    b *= np.exp2(np.random.default_rng(k).integers(-30, 30, size=(k, 1))).astype(np.float32)
    got = down(rocm.rocm_ternary_matmul_f32(DEV, up(p), up(sa), up(b), m, n, k), np.float32, (m, n))
    assert_bitexact(got, oracle.ternary_matmul(p, sa, b, m, n, k), "ternary_matmul_f32 matrix cores")


@pytest.mark.parametrize("oa,ob", [(1, 4), (3, 12)])
def test_ternary_matmul_f32_matrix_cores_unaligned(oa, ob):
    """Matrix-core path with the packed matrix and the activations at odd
    offsets (packed rows of any alignment, b 4-byte aligned only):
    bit-exact against the oracle."""
    from inputs import raw_packed

    m, n, k = 3100, 260, 419
    log(f"ternary_matmul_f32 matrix cores unaligned a+{oa} b+{ob} m={m} n={n} k={k}")
    p, sa, b = raw_packed(m, k, 81), normal((m,), 82, 1.0, 0.1), normal((k, n), 83)
    got = down(rocm.rocm_ternary_matmul_f32(DEV, _offset_buffer(p, oa), up(sa), _offset_buffer(b, ob), m, n, k),
               np.float32, (m, n))
    assert_bitexact(got, oracle.ternary_matmul(p, sa, b, m, n, k), "ternary_matmul_f32 matrix cores unaligned")


def test_ternary_matmul_f32_matrix_cores_nonfinite_and_subnormal():
    """Matrix-core path: Inf/NaN activations in some chunks and columns only
    (those chunks run element by element with zero trits skipped), finite
    activations whose sums overflow, subnormal activations and signed zeros
    (gradual underflow in every step): bit-exact against the oracle,
    non-finite outputs included."""
    from inputs import raw_packed

    m, n, k = 6500, 128, 803
    log(f"ternary_matmul_f32 matrix cores non-finite/subnormal m={m} n={n} k={k}")
    p, sa = raw_packed(m, k, 71), normal((m,), 72, 1.0, 0.1)
    b = normal((k, n), 73)
    b[100:180] *= np.float32(1e-39)            # a whole chunk of subnormals
    b[300:303, 5] = np.float32(-0.0)
    b[5, 0] = np.inf; b[250, n - 1] = -np.inf; b[777, 17] = np.nan; b[500, 64] = np.inf
    b[400:404, 3] = 3e38
    want = oracle.ternary_matmul(p, sa, b, m, n, k)
    assert np.isfinite(want).any() and not np.isfinite(want).all()
    got = down(rocm.rocm_ternary_matmul_f32(DEV, up(p), up(sa), up(b), m, n, k), np.float32, (m, n))
    assert_bitexact(got, want, "ternary_matmul_f32 matrix cores non-finite/subnormal")


@pytest.mark.parametrize("seed", range(20))
def test_ternary_matmuls_random_shapes(seed):
    """Seeded random shapes and base offsets for both ternary matmuls, so that
    every dispatch path (decode-step, row-broadcast at each tile width and
    rows-per-lane count, small-n, skinny, split-K and 128 x 128 tiles with
    aligned and unaligned weight and code rows) meets ragged sizes:
    bit-exact against the oracle on arbitrary packed bytes."""
    from inputs import int8_codes, raw_packed

    r = np.random.default_rng(1000 + seed)
    for case in range(8):
        m = int(r.integers(1, 3000))
        n = int(r.choice([1, 2, 3, 4, 5, 8, 9, 16, 17, 31, 33, 64, 65, 100, 200, 300]))
        k = int(r.integers(1, 3000))
        while m * n * k > 150_000_000:
            m = max(1, m // 2)
        oa, ob = int(r.integers(0, 4)), 4 * int(r.integers(0, 4))
        log(f"ternary random seed={seed} case={case} m={m} n={n} k={k} a+{oa} b+{ob}")
        p = raw_packed(m, k, 17 * seed + case)
        sa = normal((m,), 50 + case, 1.0, 0.1)
        bf = normal((k, n), 60 + case)
        got = down(rocm.rocm_ternary_matmul_f32(DEV, _offset_buffer(p, oa), up(sa),
                                                _offset_buffer(bf, ob), m, n, k), np.float32, (m, n))
        assert_bitexact(got, oracle.ternary_matmul(p, sa, bf, m, n, k), f"f32 {m}x{n}x{k}")
        q = int8_codes(n, k, 70 + case)
        sq = np.abs(normal((n,), 80 + case, 0.02, 0.005))
        oq = int(r.integers(0, 4))
        got = down(rocm.rocm_ternary_matmul_i8(DEV, _offset_buffer(p, oa), up(sa),
                                               _offset_buffer(q, oq), up(sq), m, n, k), np.float32, (m, n))
        assert_bitexact(got, oracle.ternary_matmul_i8(p, sa, q, sq, m, n, k), f"i8 {m}x{n}x{k}")


def test_ternary_matmul_f32_row_ranges():
    """A packed matrix of more than 2 GiB (32769 rows of 65536 packed bytes):
    the row-broadcast kernel runs over row ranges of less than 2 GiB each;
    the rows on both sides of the range boundary and the last rows are
    bit-exact against the oracle (rows are independent)."""
    m, n, kp = 32769, 5, 65536
    k = 5 * kp
    log(f"ternary_matmul_f32 row ranges m={m} n={n} k={k}")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(61)
    p = torch.randint(0, 256, (m, kp), dtype=torch.uint8, device="cuda", generator=gen)
    sa, b = normal((m,), 62, 1.0, 0.1), normal((k, n), 63)
    got = down(rocm.rocm_ternary_matmul_f32(DEV, HipBuffer.from_tensor(p), up(sa), up(b), m, n, k),
               np.float32, (m, n))
    span = 0x7FFFFFFF // kp
    rows = np.array([0, 1, span - 2, span - 1, span, m - 1])
    want = oracle.ternary_matmul(p[torch.from_numpy(rows).cuda()].cpu().numpy(), sa[rows], b, len(rows), n, k)
    del p
    torch.cuda.empty_cache()
    assert_bitexact(got[rows], want, "ternary_matmul_f32 row ranges")


@pytest.mark.parametrize("n", [1, 2, 3, 4])
def test_ternary_matmul_f32_decode_nonfinite_steps(n):
    """One to four columns over several K steps and workgroups, Inf/NaN
    activations in some steps and columns only (those take the explicit
    zero-trit skip, the others the fast path): bit-exact against the oracle,
    non-finite outputs included."""
    from inputs import raw_packed

    m, k = 130, 1203
    log(f"ternary_matmul_f32 decode non-finite m={m} n={n} k={k}")
    p, sa, b = raw_packed(m, k, 21), normal((m,), 22, 1.0, 0.1), normal((k, n), 23)
    b[5, 0] = np.inf; b[250, n - 1] = -np.inf; b[777, 0] = np.nan; b[1200, n // 2] = np.inf
    want = oracle.ternary_matmul(p, sa, b, m, n, k)
    assert np.isfinite(want).any() and not np.isfinite(want).all()
    got = down(rocm.rocm_ternary_matmul_f32(DEV, up(p), up(sa), up(b), m, n, k), np.float32, (m, n))
    assert_bitexact(got, want, f"ternary_matmul_f32 decode non-finite n={n}")


@pytest.mark.parametrize("m,k,threshold", [(2, 4, 0.3), (1, 1, 0.3), (7, 5, 0.0), (64, 2560, 0.3), (257, 6912, 0.5),
                                         (33, 333, 0.3), (6912, 2560, 0.3), (3, 64 * 5 + 3, 0.3),
                                         # K % 20 == 0 (the register-resident path, 1 to 8 chunks a lane)
                                         (9, 20, 0.3), (100, 1280, 0.3), (8, 2580, 0.3), (40, 6920, 0.5),
                                         (7, 10240, 0.3),
                                         # a negative and an infinite threshold (the per-weight fallback)
                                         (16, 100, -0.2), (8, 40, float("inf")),
                                         # k % 4 == 0, k % 20 != 0: a partial last chunk, byte stores
                                         (40, 6912, 0.3), (9, 2564, 0.3), (12, 8, 0.3),
                                         # a workgroup per long row (up to 8 slices a wave), and past it
                                         (3, 37120, 0.3), (2, 41000, 0.3), (2560, 6912, 0.3)])
def test_pack_weights_ternary(m, k, threshold):
    """pack_weights_ternary on the GPU: bytes and scales bit-exact against the
    oracle (the reference's KAT shape included), with a zero row (scale 1),
    a row below 1e-8, NaN and Inf weights, weights exactly at +-threshold *
    scale, and K not a multiple of 5; the packed result feeds the f32 matmul
    like the oracle's."""
    log(f"pack_weights_ternary m={m} k={k} threshold={threshold}")
    w = normal((m, k), 31 + m)
    if m >= 7:
        w[1] = 0.0
        w[2] *= 1e-9
        w[3, ::7] = np.nan
        w[4, 0] = np.inf
        w[5, :] = np.float32(1.0)
        w[5, ::3] = np.float32(threshold)   # w / scale == threshold: not > threshold
        w[6, ::2] = -w[6, ::2]
    if m >= 8:
        # quotients within a few ulps of +-threshold under a scale that is not
        # a power of two (where w * (1 / scale) and w / scale can differ)
        sc = np.float32(3.7)
        near = (np.float32(threshold) * sc) * (1 + np.arange(-6, 7, dtype=np.float32) * np.float32(2.0**-23))
        row = np.resize(np.concatenate([near, -near]), k).astype(np.float32)
        row[0] = sc
        w[7] = row
    if (m, k) == (2, 4):
        w = np.array([[1.0, -1.0, 0.0, 0.5], [-0.5, 1.0, -1.0, 0.0]], np.float32)  # cpu_ternary_matmul.rs:247-253
    want_p, want_s = oracle.pack_weights_ternary(w, threshold)
    gp, gs = rocm.rocm_pack_weights_ternary(DEV, up(w), m, k, threshold)
    assert_bitexact(down(gs, np.float32, (m,)), want_s, "pack scales")
    assert_bitexact(down(gp, np.uint8, want_p.shape), want_p, "pack bytes")
    if k >= 5 and m <= 300:
        b = normal((k, 2), 32)
        got = down(rocm.rocm_ternary_matmul_f32(DEV, gp, gs, up(b), m, 2, k), np.float32, (m, 2))
        assert_bitexact(got, oracle.ternary_matmul(want_p, want_s, b, m, 2, k), "pack -> ternary_matmul_f32")


def test_ternary_matmul_f32_edges():
    log("ternary_matmul_f32 edges")
    lib = __import__("kore_amd._lib", fromlist=["load"]).load()
    assert lib.kore_hip_ternary_matmul_f32(None, None, None, None, 0, 5, 16, None) == 0
    assert lib.kore_hip_ternary_matmul_f32(None, None, None, None, 5, 0, 16, None) == 0
    assert lib.kore_hip_ternary_matmul_f32(None, None, None, None, 2, 2, 16, None) == -1
    cb = up(np.zeros(64, np.float32))
    assert lib.kore_hip_ternary_matmul_f32(1 << 40, 1 << 41, cb.ptr, cb.ptr, 4, 4, 16, None) == -4
    # unaligned activations and an odd packed-row length: same results
    from inputs import raw_packed

    for m, n, k in ((50, 3, 333), (50, 1, 333)):
        p, sa, b = raw_packed(m, k, 3), normal((m,), 4), normal((k, n), 5)
        t = torch.empty(k * n + 1, dtype=torch.float32, device="cuda")
        t[1:].copy_(torch.from_numpy(b.ravel()))
        got = down(rocm.rocm_ternary_matmul_f32(DEV, up(p), up(sa), HipBuffer.from_tensor(t[1:]), m, n, k),
                   np.float32, (m, n))
        assert_bitexact(got, oracle.ternary_matmul(p, sa, b, m, n, k), f"ternary_matmul_f32 unaligned b n={n}")


@pytest.mark.parametrize("off", [1, 2, 3])
@pytest.mark.parametrize("m,n,k", [(4, 1, 25), (5, 2, 21), (37, 1, 333), (9, 4, 241), (300, 1, 1203)])
def test_ternary_matmul_f32_packed_at_byte_offsets(off, m, n, k):
    """The one-to-four-column kernel reads a step's packed bytes as three
    dwords around them; on a matrix that starts or ends inside a dword the
    steps touching those partial dwords read their bytes one by one, so
    nothing outside [a_packed, a_packed + m * kp) is read.  The matrix sits
    at byte offset off and ends at the end of its tensor."""
    from inputs import raw_packed

    log(f"ternary_matmul_f32 packed at +{off} m={m} n={n} k={k}")
    p = raw_packed(m, k, 7 * m + k + off)
    t = torch.empty(off + p.size, dtype=torch.uint8, device="cuda")
    t[off:].copy_(torch.from_numpy(p.ravel()))
    sa, b = normal((m,), 8), normal((k, n), 9)
    got = down(rocm.rocm_ternary_matmul_f32(DEV, HipBuffer.from_tensor(t[off:]), up(sa), up(b), m, n, k),
               np.float32, (m, n))
    assert_bitexact(got, oracle.ternary_matmul(p, sa, b, m, n, k), f"ternary_matmul_f32 packed at +{off}")


def test_decode_chain_graph_replays_match_eager():
    """A decode step's launches (pre-quant, the BitLinear matmul on its codes
    -- the split-K path's zero/finish kernels included at 64 tokens -- the
    RMSNorm+SiLU gate, RoPE, softmax, the f32 matmul and both BitLinear layer
    entry points with a bias) captured in one HIP
    graph on a side stream: no entry point allocates, synchronises or records
    a memset, so every replay, with eager work between replays, reproduces the
    eager outputs bit for bit."""
    from inputs import raw_packed

    lib = __import__("kore_amd._lib", fromlist=["load"]).load()
    dev = torch.device("cuda", DEV)
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    k, m, vocab = 2560, 6912, 4096
    out = {}

    def make(tokens):
        t = {"x": torch.randn(tokens, k, generator=g, device=dev),
             "w": torch.randn(k, generator=g, device=dev),
             "z": torch.randn(tokens, k, generator=g, device=dev),
             "a": torch.from_numpy(raw_packed(m, k, 3).ravel()).to(dev),
             "sa": torch.rand(m, generator=g, device=dev),
             "q": torch.randn(tokens, 4, 128, generator=g, device=dev),
             "kk": torch.randn(tokens, 2, 128, generator=g, device=dev),
             "inv": torch.from_numpy(oracle.rope_inv_freq(128, 10000.0)).to(dev),
             "logits": torch.randn(tokens, vocab, generator=g, device=dev)}
        t["codes"] = torch.empty(tokens, k, dtype=torch.int8, device=dev)
        t["scales"] = torch.empty(tokens, device=dev)
        t["c"] = torch.empty(m, tokens, device=dev)
        t["gate"] = torch.empty(tokens, k, device=dev)
        t["probs"] = torch.empty(tokens, vocab, device=dev)
        t["cf"] = torch.empty(m, tokens, device=dev)
        t["xt"] = t["x"].t().contiguous()
        t["bias"] = torch.randn(m, generator=g, device=dev)
        t["y8"] = torch.empty(tokens, m, device=dev)
        t["yf"] = torch.empty(tokens, m, device=dev)
        return t

    def step(t, tokens, s):
        P = lambda name: t[name].data_ptr()  # noqa: E731
        rc = [lib.kore_hip_rms_norm_quant_i8(P("x"), P("w"), P("codes"), P("scales"), tokens, k, 1e-6, s),
              lib.kore_hip_ternary_matmul_i8(P("a"), P("sa"), P("codes"), P("scales"), P("c"), m, tokens, k, s),
              lib.kore_hip_rms_norm_silu_gate_f32(P("x"), P("w"), P("z"), P("gate"), tokens, k, 1e-6, s),
              lib.kore_hip_rope_qk_f32(P("q"), P("kk"), P("inv"), 1, tokens, 4, 2, 128, 5, 0, s),
              lib.kore_hip_softmax_f32(P("logits"), P("probs"), tokens, vocab, s),
              lib.kore_hip_ternary_matmul_f32(P("a"), P("sa"), P("xt"), P("cf"), m, tokens, k, s),
              lib.kore_hip_bit_linear_i8(P("a"), P("sa"), P("codes"), P("scales"), P("bias"), P("y8"), m, tokens, k,
                                         s),
              lib.kore_hip_bit_linear_f32(P("a"), P("sa"), P("x"), P("bias"), P("yf"), m, tokens, k, s)]
        assert rc == [0] * len(rc), rc

    for tokens in (1, 64):
        log(f"decode chain graph tokens={tokens}")
        t = make(tokens)
        q0, k0 = t["q"].clone(), t["kk"].clone()
        step(t, tokens, torch.cuda.current_stream(dev).cuda_stream)
        torch.cuda.synchronize(dev)
        want = {n: t[n].clone() for n in ("codes", "scales", "c", "gate", "q", "kk", "probs", "cf", "y8", "yf")}
        side = torch.cuda.Stream(device=dev)
        graph = torch.cuda.CUDAGraph()
        t["q"].copy_(q0)
        t["kk"].copy_(k0)
        torch.cuda.synchronize(dev)
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                step(t, tokens, side.cuda_stream)
        torch.cuda.synchronize(dev)
        for rep in range(3):
            for n in ("codes", "scales", "c", "gate", "probs", "cf", "y8", "yf"):
                t[n].fill_(float("nan") if t[n].is_floating_point() else 0)
            t["q"].copy_(q0)
            t["kk"].copy_(k0)
            torch.cuda.synchronize(dev)
            graph.replay()
            torch.cuda.synchronize(dev)
            for n, v in want.items():
                assert torch.equal(t[n], v), (tokens, rep, n)
        out[tokens] = True
    assert out == {1: True, 64: True}


def _adversarial_rows(rows: int, cols: int, seed: int) -> np.ndarray:
    """Rows whose running sum of squares crosses many binades in awkward
    places: wide per-row scales, exponential ramps (every segment in a new
    binade), a few huge entries among tiny ones (late crossings), sums that
    sit just below powers of two, and subnormal-heavy rows."""
    g = np.random.default_rng(seed)
    x = g.standard_normal((rows, cols)).astype(np.float32)
    kind = np.arange(rows) % 6
    scale = (10.0 ** g.uniform(-18, 18, size=rows)).astype(np.float32)
    x[kind == 0] *= scale[kind == 0, None]
    ramp = (2.0 ** np.linspace(-20, 20, cols)).astype(np.float32)
    x[kind == 1] = (x[kind == 1] * ramp[None, :]).astype(np.float32)
    spikes = g.random((rows, cols)) < 0.002
    x[(kind == 2)[:, None] & spikes] *= np.float32(1e6)
    x[kind == 2] *= np.float32(1e-3)
    # constant rows whose sum of squares lands next to 2^k
    x[kind == 3] = np.float32(np.sqrt(2.0 ** 11 / cols)) * (1 + g.uniform(-1e-6, 1e-6, size=(int((kind == 3).sum()), cols))).astype(np.float32)
    x[kind == 4] *= np.float32(1e-22)
    x[kind == 5] = (x[kind == 5] * (g.random((int((kind == 5).sum()), cols)) < 0.5)).astype(np.float32)  # half zeros
    return x


@pytest.mark.parametrize("cols", [2048, 2560, 4096, 1000])
def test_norm_family_adversarial_rows_bit_exact(cols):
    """The exact segmented fold under stress: 6144 rows of the kinds above,
    RMSNorm and pre-quant bit-exact against the oracle's sequential fold."""
    rows = 6144
    log(f"adversarial rows cols={cols}")
    x = _adversarial_rows(rows, cols, cols)
    g = (1.0 + 0.02 * np.random.default_rng(cols + 1).standard_normal(cols)).astype(np.float32)
    got = down(rocm.rocm_rms_norm_f32(DEV, up(x), up(g), rows, cols, 1e-6), np.float32, (rows, cols))
    assert_bitexact(got, oracle.rms_norm(x, g, 1e-6), f"rms_norm adversarial {cols}")
    q, s = rocm.rocm_rms_norm_quant_i8(DEV, up(x), up(g), rows, cols, 1e-6)
    wq, ws = oracle.rms_norm_quant_i8(x, g, 1e-6)
    assert down(q, np.int8, (rows, cols)).tobytes() == wq.tobytes(), f"prequant codes adversarial {cols}"
    assert down(s, np.float32, (rows,)).tobytes() == ws.tobytes(), f"prequant scales adversarial {cols}"


@pytest.mark.parametrize("m,n,k", [(6912, 64, 2560), (4097, 48, 2563), (2600, 100, 2600), (4100, 64, 7680),
                                   (1500, 192, 6912)])
def test_ternary_matmul_f32_matrix_core_decode_batches(m, n, k):
    """ternary_matmul_f32 with [K, N] b on the 4 x 4 x 1 matrix-core kernel
    (41-192 columns, K >= 2560, at least 1024 waves of 4 rows x 64 columns): bit-exact against the oracle on every
    output, with Inf, NaN and subnormal activations in some columns (their
    chunks fold element by element, zero trits skipped), ragged row groups
    and K not a multiple of the 80-column chunk."""
    from inputs import raw_packed

    log(f"ternary_matmul_f32 4x4 matrix cores m={m} n={n} k={k}")
    p = raw_packed(m, k, m + 13 * k)
    sa = normal((m,), 90, 1.0, 0.1)
    b = normal((k, n), 91)
    r = np.random.default_rng(m + n)
    b[r.integers(0, k, 2), 1] = np.inf
    b[r.integers(0, k, 2), 2] = -np.inf
    b[r.integers(0, k, 1), 3] = np.nan
    b[:, 4] = (b[:, 4] * 1e-39).astype(np.float32)
    got = down(rocm.rocm_ternary_matmul_f32(DEV, up(p), up(sa), up(b), m, n, k), np.float32, (m, n))
    assert_bitexact(got, oracle.ternary_matmul(p, sa, b, m, n, k), "ternary_matmul_f32 4x4 matrix cores")
