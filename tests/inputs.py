"""Seeded synthetic inputs for the BASELINE configs and the parity tests.

One generator for tests and bench: numpy PCG64 (``default_rng(seed)``), f32
draws.  The distributions are BASELINE.json's:
  RMSNorm      x ~ N(0,1), weight ~ N(1, 0.02)
  RoPE         Q, K ~ N(0,1)
  SwiGLU/GELU  gate, up, x ~ N(0,1)
  Embedding    table ~ N(0, 0.02); ids uniform in [0, vocab) with 5% of the
               positions replaced by an earlier position's id
  Pre-quant    x ~ N(0,1) with 1% of entries scaled by 20; weight ~ N(1, 0.02)
"""
from __future__ import annotations

import numpy as np


def rng(seed: int = 0) -> np.random.Generator:
    return np.random.default_rng(seed)


def normal(shape, seed: int = 0, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    g = rng(seed)
    x = g.standard_normal(size=shape, dtype=np.float32)
    if std != 1.0:
        x *= np.float32(std)
    if mean != 0.0:
        x += np.float32(mean)
    return x


def rmsnorm_inputs(rows: int, cols: int, seed: int = 0):
    return normal((rows, cols), seed), normal((cols,), seed + 1, 1.0, 0.02)


def prequant_inputs(rows: int, cols: int, seed: int = 0):
    x = normal((rows, cols), seed)
    g = rng(seed + 7)
    mask = g.random(size=x.shape) < 0.01
    x[mask] *= np.float32(20.0)
    return x, normal((cols,), seed + 1, 1.0, 0.02)


def embedding_ids(n_ids: int, vocab: int, seed: int = 0, repeat_frac: float = 0.05) -> np.ndarray:
    g = rng(seed)
    ids = g.integers(0, vocab, size=n_ids, dtype=np.int64).astype(np.int32)
    n_rep = int(round(n_ids * repeat_frac))
    if n_ids > 1 and n_rep:
        pos = g.choice(np.arange(1, n_ids), size=min(n_rep, n_ids - 1), replace=False)
        for p in np.sort(pos):
            ids[p] = ids[g.integers(0, p)]
    return ids


def close_mask(got: np.ndarray, ref: np.ndarray, rtol: float = 1e-5, atol: float = 1e-6) -> np.ndarray:
    """BASELINE tolerance per element: |got-ref| <= atol or <= rtol*|ref|.
    NaN must meet NaN; infinities must match exactly."""
    got = np.asarray(got, dtype=np.float32)
    ref = np.asarray(ref, dtype=np.float32)
    nan_g, nan_r = np.isnan(got), np.isnan(ref)
    with np.errstate(invalid="ignore", over="ignore"):
        diff = np.abs(got.astype(np.float64) - ref.astype(np.float64))
        ok = (diff <= atol) | (diff <= rtol * np.abs(ref.astype(np.float64)))
    ok |= nan_g & nan_r
    ok &= nan_g == nan_r
    inf = np.isinf(ref) | np.isinf(got)
    ok[inf] = (got[inf] == ref[inf])
    return ok


def assert_close(got, ref, rtol: float = 1e-5, atol: float = 1e-6, what: str = "") -> None:
    ok = close_mask(got, ref, rtol, atol)
    if not ok.all():
        bad = np.argwhere(~ok.reshape(np.shape(ref)))
        i = tuple(bad[0])
        g = np.asarray(got)[i]
        r = np.asarray(ref)[i]
        raise AssertionError(f"{what}: {len(bad)} of {ok.size} elements outside tol "
                             f"(rtol={rtol}, atol={atol}); first at {i}: got {g!r} ref {r!r}")


def max_err(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    fin = np.isfinite(ref) & np.isfinite(got)
    d = np.abs(got - ref)[fin]
    if d.size == 0:
        return 0.0, 0.0
    rel = d / np.maximum(np.abs(ref[fin]), 1e-30)
    return float(d.max()), float(rel[np.abs(ref[fin]) > 1e-3].max() if (np.abs(ref[fin]) > 1e-3).any() else 0.0)


def assert_bitexact(got, ref, what: str = "") -> None:
    """Byte equality, except that any NaN matches any NaN (x86 and gfx950
    produce different default NaN payloads; the value class is what the
    reference defines)."""
    got = np.ascontiguousarray(got)
    ref = np.ascontiguousarray(ref)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    if got.dtype.kind == "f":
        nan = np.isnan(got) & np.isnan(ref)
        gb = got.view(np.uint32 if got.dtype == np.float32 else np.uint64).copy()
        rb = ref.view(gb.dtype).copy()
        gb[nan] = 0
        rb[nan] = 0
    else:
        gb, rb = got, ref
    bad = np.argwhere(gb != rb)
    if bad.size:
        i = tuple(bad[0])
        raise AssertionError(f"{what}: {len(bad)} of {gb.size} elements differ; first at {i}: "
                             f"got {got[i]!r} ref {ref[i]!r}")


def assert_close_scaled(got, ref, scale, rtol: float = 1e-5, atol: float = 1e-6, what: str = "") -> None:
    """|got - ref| <= atol + rtol * scale per element, for outputs that are a
    difference of rounded terms (backward passes): `scale` is the magnitude of
    the terms (e.g. |a| + |b| for a - b), so cancellation in the result does
    not turn the reference's own rounding into a relative error.  NaN must
    meet NaN."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    scale = np.broadcast_to(np.asarray(scale, dtype=np.float64), ref.shape)
    nan_g, nan_r = np.isnan(got), np.isnan(ref)
    with np.errstate(invalid="ignore"):
        ok = np.abs(got - ref) <= atol + rtol * scale
    ok |= nan_g & nan_r
    ok &= nan_g == nan_r
    if not ok.all():
        bad = np.argwhere(~ok)
        i = tuple(bad[0])
        raise AssertionError(f"{what}: {len(bad)} of {ok.size} elements outside tol (rtol={rtol} of scale, "
                             f"atol={atol}); first at {i}: got {got[i]!r} ref {ref[i]!r} scale {scale[i]!r}")


def ternary_weights(m: int, k: int, seed: int = 0, threshold: float = 0.3):
    """BitLinear weights: w ~ U(-1, 1) (the reference's BitLinear::random,
    crates/kore-nn/src/bit_linear.rs:93-108) packed by the oracle's
    pack_weights_ternary; returns (packed uint8[m, ceil(k/5)], scales f32[m])."""
    import oracle

    w = rng(seed).uniform(-1.0, 1.0, size=(m, k)).astype(np.float32)
    return oracle.pack_weights_ternary(w, threshold)


def raw_packed(m: int, k: int, seed: int = 0) -> np.ndarray:
    """Arbitrary packed bytes 0..255: includes bytes >= 243 (decode to zeros)
    and nonzero padding trits past column k (ignored by the reference's
    truncate(k))."""
    return rng(seed).integers(0, 256, size=(m, (k + 4) // 5), dtype=np.int64).astype(np.uint8)


def int8_codes(n: int, k: int, seed: int = 0) -> np.ndarray:
    return rng(seed).integers(-128, 128, size=(n, k), dtype=np.int64).astype(np.int8)
