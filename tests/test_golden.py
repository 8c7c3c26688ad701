"""The committed golden fixtures (tests/golden/golden.npz, manifest.json,
written by tests/golden/make_golden.py from the oracle): on the CPU the
arrays match their recorded checksums and the oracle still reproduces every
output bit for bit; on the GPU every entry point reproduces the fixture
outputs from the fixture inputs (bit-exact for norms, codes, gathers and
integer sums; the parity tests' tolerances where the reference calls libm)."""
import json
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import make_golden  # noqa: E402
from inputs import assert_bitexact, assert_close, assert_close_scaled  # noqa: E402

U32 = 2.0 ** -24


def load():
    with np.load(os.path.join(HERE, "golden", "golden.npz"), allow_pickle=False) as z:
        arrays = {k: z[k] for k in z.files}
    manifest = json.load(open(os.path.join(HERE, "golden", "manifest.json")))
    return arrays, manifest


def case(arrays, name, entry):
    ins = {k: arrays[f"{name}.{k}"] for k in entry["inputs"]}
    outs = {k: arrays[f"{name}.{k}"] for k in entry["outputs"]}
    return ins, outs


def test_golden_checksums():
    arrays, manifest = load()
    assert len(manifest) >= 20
    names = set()
    for name, entry in manifest.items():
        for kind in ("inputs", "outputs"):
            for k, meta in entry[kind].items():
                a = arrays[f"{name}.{k}"]
                assert str(a.dtype) == meta["dtype"] and list(a.shape) == meta["shape"], (name, k)
                assert make_golden.sha(a) == meta["sha256"], (name, k)
                names.add(f"{name}.{k}")
    assert names == set(arrays)


def test_oracle_reproduces_golden():
    arrays, manifest = load()
    cases = make_golden.cases()
    assert set(cases) == set(manifest)
    for name, entry in manifest.items():
        op, params, _, fn = cases[name]
        assert op == entry["op"] and params == entry["params"]
        ins, outs = case(arrays, name, entry)
        got = fn(ins, params)
        for k, v in outs.items():
            assert np.array_equal(np.asarray(got[k]).view(np.uint8), v.view(np.uint8)), (name, k)


def _rms_bwd_scales(dy, x, g, eps):
    x64, dy64, g64 = x.astype(np.float64), dy.astype(np.float64), g.astype(np.float64)
    cols = x.shape[1]
    ss = (x64 * x64).sum(axis=1, keepdims=True)
    inv = 1.0 / np.sqrt(ss / cols + eps)
    coeff_abs = np.abs(x64 * dy64 * g64).sum(axis=1, keepdims=True) * inv / (ss + eps * cols)
    return np.abs(g64) * inv * np.abs(dy64) + coeff_abs * np.abs(x64), (np.abs(dy64 * x64) * inv).sum(axis=0)


@pytest.mark.gpu
def test_hip_path_reproduces_golden():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from kore_amd import rocm
    from kore_amd.rocm import HipBuffer

    def up(a):
        return HipBuffer.from_host(0, np.ascontiguousarray(a))

    def down(b, dtype, shape):
        return b.to_host(dtype)[: int(np.prod(shape))].reshape(shape)

    arrays, manifest = load()
    seen = set()
    for name, entry in manifest.items():
        print(f"golden {name}", flush=True)
        op, p = entry["op"], entry["params"]
        i, o = case(arrays, name, entry)
        if op == "rms_norm":
            r, c = i["x"].shape
            assert_bitexact(down(rocm.rocm_rms_norm_f32(0, up(i["x"]), up(i["g"]), r, c, p["eps"]), np.float32,
                                 (r, c)), o["y"], name)
        elif op == "rms_norm_quant_i8":
            r, c = i["x"].shape
            q, s = rocm.rocm_rms_norm_quant_i8(0, up(i["x"]), up(i["g"]), r, c, p["eps"])
            assert_bitexact(down(q, np.int8, (r, c)), o["q"], name)
            assert_bitexact(down(s, np.float32, (r,)), o["scale"], name)
        elif op == "rms_norm_silu_gate":
            r, c = i["x"].shape
            y = rocm.rocm_fused_rms_norm_silu_gate_f32(0, up(i["x"]), up(i["g"]), up(i["z"]), r, c, p["eps"])
            assert_close(down(y, np.float32, (r, c)), o["y"], what=name)
        elif op in ("gelu", "silu"):
            n = i["x"].size
            f = rocm.rocm_gelu_f32 if op == "gelu" else rocm.rocm_silu_f32
            assert_close(down(f(0, up(i["x"]), n), np.float32, (n,)), o["y"], what=name)
        elif op == "swiglu":
            n = i["gate"].size
            assert_close(down(rocm.rocm_swiglu_f32(0, up(i["gate"]), up(i["up"]), n), np.float32, (n,)), o["y"],
                         what=name)
        elif op == "mul":
            n = i["a"].size
            assert_bitexact(down(rocm.rocm_mul_f32(0, up(i["a"]), up(i["b"]), n), np.float32, (n,)), o["y"], name)
        elif op == "rope_qk":
            b, s, hq, d = i["q"].shape
            hk = i["k"].shape[2]
            qb, kb = up(i["q"]), up(i["k"])
            inv = rocm.rocm_rope_inv_freq_f32(0, d, p["theta"])
            rocm.rocm_rope_qk_f32(0, qb, kb, inv, b, s, hq, hk, d, p["start"], bool(p["interleaved"]))
            assert_close(down(qb, np.float32, i["q"].shape), o["q_out"], what=name)
            assert_close(down(kb, np.float32, i["k"].shape), o["k_out"], what=name)
        elif op == "embedding":
            v, d = i["table"].shape
            n = i["ids"].size
            out = rocm.rocm_embedding_f32(0, up(i["table"]), up(i["ids"]), n, v, d)
            assert_bitexact(down(out, np.float32, (n, d)), o["out"], name)
        elif op == "embedding_forward":
            v, d = i["table"].shape
            n = i["ids"].size
            out = rocm.rocm_embedding_forward_f32(0, up(i["table"]), up(i["ids"]), n, v, d)
            assert_bitexact(down(out, np.float32, (n, d)), o["out"], name)
        elif op == "pack_weights_ternary":
            m, k = i["w"].shape
            pk, sc = rocm.rocm_pack_weights_ternary(0, up(i["w"]), m, k, p["threshold"])
            assert_bitexact(down(pk, np.uint8, o["packed"].shape), o["packed"], name)
            assert_bitexact(down(sc, np.float32, (m,)), o["scales"], name)
        elif op in ("softmax", "softmax_causal"):
            r, c = i["x"].shape
            y = (rocm.rocm_softmax_f32(0, up(i["x"]), r, c) if op == "softmax"
                 else rocm.rocm_softmax_causal_f32(0, up(i["x"]), r, c, p["offset"]))
            assert_close(down(y, np.float32, (r, c)), o["y"], rtol=1e-5 + c * U32, what=name)
        elif op == "softmax_backward":
            r, c = i["y"].shape
            dx = rocm.rocm_softmax_backward_f32(0, up(i["dy"]), up(i["y"]), r, c)
            y64, dy64 = i["y"].astype(np.float64), i["dy"].astype(np.float64)
            scale = np.abs(y64) * (np.abs(dy64) + np.abs(y64 * dy64).sum(axis=-1, keepdims=True))
            assert_close_scaled(down(dx, np.float32, (r, c)), o["dx"], scale, rtol=1e-5 + c * U32, what=name)
        elif op == "cross_entropy_backward":
            b, c = i["logits"].shape
            dx = rocm.rocm_cross_entropy_backward_f32(0, up(i["logits"]), up(i["targets"]), b, c)
            assert_close(down(dx, np.float32, (b, c)), o["dx"], rtol=1e-5 + c * U32, what=name)
        elif op == "rms_norm_backward":
            r, c = i["x"].shape
            gx, gg = rocm.rocm_rms_norm_backward_f32(0, up(i["dy"]), up(i["x"]), up(i["g"]), r, c, p["eps"])
            sdx, sdg = _rms_bwd_scales(i["dy"], i["x"], i["g"], p["eps"])
            assert_close_scaled(down(gx, np.float32, (r, c)), o["dx"], sdx, rtol=1e-5 + c * U32, what=name)
            assert_close_scaled(down(gg, np.float32, (c,)), o["dg"], sdg, rtol=1e-5 + r * U32, what=name)
        elif op == "ternary_matmul_i8":
            m, n, k = p["m"], p["n"], p["k"]
            cb = rocm.rocm_ternary_matmul_i8(0, up(i["a"]), up(i["sa"]), up(i["q"]), up(i["sq"]), m, n, k)
            assert_bitexact(down(cb, np.float32, (m, n)), o["c"], name)
        elif op == "ternary_matmul_f32":
            m, n, k = p["m"], p["n"], p["k"]
            cb = rocm.rocm_ternary_matmul_f32(0, up(i["a"]), up(i["sa"]), up(i["b"]), m, n, k)
            assert_bitexact(down(cb, np.float32, (m, n)), o["c"], name)
        else:
            raise AssertionError(f"no GPU check for {op}")
        seen.add(op)
    assert len(seen) == len({e["op"] for e in manifest.values()})
