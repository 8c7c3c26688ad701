"""Writes tests/golden/golden.npz and manifest.json: small seeded inputs for
every entry point of the path and the expected outputs, computed by the C
restatement of the reference's CPU functions (oracle/).  The reference ships
no fixtures for these functions (its own known-answer tests are restated in
tests/test_oracle.py), so these pin the oracle against regressions and give
the GPU path a fixed set of cases independent of the generators in
tests/inputs.py.

    python3 tests/golden/make_golden.py        # rewrite the fixtures
    python3 tests/golden/make_golden.py --check  # recompute and compare

Arrays are plain numeric .npy members (np.load(..., allow_pickle=False)).
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

import oracle  # noqa: E402
from inputs import (embedding_ids, int8_codes, normal, prequant_inputs, raw_packed,  # noqa: E402
                    rmsnorm_inputs)


def cases():
    """name -> (op, params, inputs dict, outputs function)."""
    c = {}
    x, g = rmsnorm_inputs(8, 2048, 0)
    x[5] = 0.0                     # zero row: ss = 0, inv = 1/sqrt(eps)
    x[6] *= np.float32(1e18)       # ss near f32 max
    x[7] *= np.float32(1e-20)      # ss in the subnormal range
    c["rms_norm"] = ("rms_norm", {"eps": 1e-6}, {"x": x, "g": g},
                     lambda i, p: {"y": oracle.rms_norm(i["x"], i["g"], p["eps"])})
    x, g = prequant_inputs(6, 2560, 0)
    x[4] = 0.0                     # all-zero row: absmax guard
    c["rms_norm_quant_i8"] = ("rms_norm_quant_i8", {"eps": 1e-6}, {"x": x, "g": g},
                              lambda i, p: dict(zip(("q", "scale"),
                                                    oracle.rms_norm_quant_i8(i["x"], i["g"], p["eps"]))))
    z = normal((4, 2560), 5) * np.float32(8.0)
    x, g = rmsnorm_inputs(4, 2560, 4)
    c["rms_norm_silu_gate"] = ("rms_norm_silu_gate", {"eps": 1e-6}, {"x": x, "g": g, "z": z},
                               lambda i, p: {"y": oracle.rms_norm_silu_gate(i["x"], i["g"], i["z"], p["eps"])})
    a, b = normal((4096,), 6) * np.float32(4.0), normal((4096,), 7) * np.float32(4.0)
    c["gelu"] = ("gelu", {}, {"x": a}, lambda i, p: {"y": oracle.gelu(i["x"])})
    c["silu"] = ("silu", {}, {"x": a}, lambda i, p: {"y": oracle.silu(i["x"])})
    c["swiglu"] = ("swiglu", {}, {"gate": a, "up": b}, lambda i, p: {"y": oracle.swiglu(i["gate"], i["up"])})
    c["mul"] = ("mul", {}, {"a": a, "b": b}, lambda i, p: {"y": oracle.mul(i["a"], i["b"])})
    q, k = normal((2, 16, 4, 128), 8), normal((2, 16, 2, 128), 9)
    for inter in (False, True):
        c[f"rope_qk_{'interleaved' if inter else 'half'}"] = (
            "rope_qk", {"start": 3, "theta": 10000.0, "interleaved": int(inter)}, {"q": q, "k": k},
            lambda i, p: {"q_out": oracle.rope(i["q"], p["start"], p["theta"], bool(p["interleaved"])),
                          "k_out": oracle.rope(i["k"], p["start"], p["theta"], bool(p["interleaved"]))})
    table = normal((50, 64), 10, 0.0, 0.02)
    ids = embedding_ids(20, 50, 11).astype(np.int64)
    ids[3], ids[7], ids[11] = 50, -1, 2**31  # out of range: zero rows
    c["embedding"] = ("embedding", {}, {"table": table, "ids": ids.astype(np.uint32)},
                      lambda i, p: {"out": oracle.embedding(i["table"], i["ids"])})
    fids = np.array([0.0, 2.0, 1.0, np.nan, -1.5, 0.9, 1e30, 49.0, 50.0, 51.0, 49.99, -0.0, np.inf, -np.inf,
                     7.7, 3.0], np.float32)  # Rust `as usize`: NaN and < 1 -> row 0, >= vocab -> zero row
    c["embedding_forward"] = ("embedding_forward", {}, {"table": table, "ids": fids},
                              lambda i, p: {"out": oracle.embedding_forward(i["table"], i["ids"])})
    # many rows: the four-waves-per-workgroup kernels (simple-segment runs)
    x, g = rmsnorm_inputs(264, 128, 24)
    c["rms_norm_264x128"] = ("rms_norm", {"eps": 1e-6}, {"x": x, "g": g},
                             lambda i, p: {"y": oracle.rms_norm(i["x"], i["g"], p["eps"])})
    x, g = prequant_inputs(264, 256, 25)
    c["rms_norm_quant_i8_264x256"] = ("rms_norm_quant_i8", {"eps": 1e-6}, {"x": x, "g": g},
                                      lambda i, p: dict(zip(("q", "scale"),
                                                            oracle.rms_norm_quant_i8(i["x"], i["g"], p["eps"]))))
    w = normal((7, 333), 26, 0.0, 0.05)
    w[2] = 0.0                    # all-zero row: the scale guard
    w[4, 5] = np.nan              # NaN dropped from the row max, a NaN quotient packs as zero
    w[5] *= np.float32(1e-9)      # absmax below 1e-8
    c["pack_weights_ternary"] = ("pack_weights_ternary", {"threshold": 0.5}, {"w": w},
                                 lambda i, p: dict(zip(("packed", "scales"),
                                                       oracle.pack_weights_ternary(i["w"], p["threshold"]))))
    lg = normal((4, 1000), 12) * np.float32(3.0)
    c["softmax"] = ("softmax", {}, {"x": lg}, lambda i, p: {"y": oracle.softmax(i["x"])})
    c["softmax_causal"] = ("softmax_causal", {"offset": 2}, {"x": normal((6, 16), 13)},
                           lambda i, p: {"y": oracle.softmax_causal(i["x"], p["offset"])})
    y = oracle.softmax(normal((4, 256), 14))
    c["softmax_backward"] = ("softmax_backward", {}, {"dy": normal((4, 256), 15), "y": y},
                             lambda i, p: {"dx": oracle.softmax_backward(i["dy"], i["y"])})
    t = np.array([3, 0, 99, 41, 7], np.float32)
    c["cross_entropy_backward"] = ("cross_entropy_backward", {}, {"logits": normal((5, 100), 16), "targets": t},
                                   lambda i, p: {"dx": oracle.cross_entropy_backward(i["logits"], i["targets"])})
    x, g = rmsnorm_inputs(8, 512, 17)
    c["rms_norm_backward"] = ("rms_norm_backward", {"eps": 1e-5}, {"dy": normal((8, 512), 18), "x": x, "g": g},
                              lambda i, p: dict(zip(("dx", "dg"),
                                                    oracle.rms_norm_backward(i["dy"], i["x"], i["g"], p["eps"]))))
    for (m, n, k, seed) in ((64, 8, 160, 19), (16, 3, 2560, 20), (9, 70, 333, 21)):
        c[f"ternary_i8_{m}x{n}x{k}"] = (
            "ternary_matmul_i8", {"m": m, "n": n, "k": k},
            {"a": raw_packed(m, k, seed), "sa": normal((m,), seed + 1, 1.0, 0.1), "q": int8_codes(n, k, seed + 2),
             "sq": np.abs(normal((n,), seed + 3, 0.02, 0.005))},
            lambda i, p: {"c": oracle.ternary_matmul_i8(i["a"], i["sa"], i["q"], i["sq"], p["m"], p["n"], p["k"])})
    for (m, n, k, seed) in ((40, 5, 333, 22), (70, 1, 2560, 23), (37, 48, 333, 26)):
        c[f"ternary_f32_{m}x{n}x{k}"] = (
            "ternary_matmul_f32", {"m": m, "n": n, "k": k},
            {"a": raw_packed(m, k, seed), "sa": normal((m,), seed + 1, 1.0, 0.1), "b": normal((k, n), seed + 2)},
            lambda i, p: {"c": oracle.ternary_matmul(i["a"], i["sa"], i["b"], p["m"], p["n"], p["k"])})
    return c


def sha(a: np.ndarray) -> str:
    a = np.ascontiguousarray(a)
    return hashlib.sha256(str(a.dtype).encode() + str(a.shape).encode() + a.tobytes()).hexdigest()


def build():
    arrays, manifest = {}, {}
    for name, (op, params, ins, fn) in cases().items():
        outs = fn(ins, params)
        entry = {"op": op, "params": params, "inputs": {}, "outputs": {}}
        for kind, d in (("inputs", ins), ("outputs", outs)):
            for k, v in d.items():
                v = np.ascontiguousarray(v)
                arrays[f"{name}.{k}"] = v
                entry[kind][k] = {"dtype": str(v.dtype), "shape": list(v.shape), "sha256": sha(v)}
        manifest[name] = entry
    return arrays, manifest


def main():
    arrays, manifest = build()
    if "--check" in sys.argv:
        want = json.load(open(os.path.join(HERE, "manifest.json")))
        bad = [n for n in manifest if manifest[n] != want.get(n)]
        print("golden fixtures reproduce" if not bad and set(want) == set(manifest) else f"differ: {bad}")
        return 1 if bad or set(want) != set(manifest) else 0
    np.savez_compressed(os.path.join(HERE, "golden.npz"), **arrays)
    with open(os.path.join(HERE, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
    print(f"wrote {len(arrays)} arrays for {len(manifest)} cases")
    return 0


if __name__ == "__main__":
    sys.exit(main())
