"""Writes tests/golden/reference_fixtures.json.

Inputs are the literal fixtures of the reference's own tests
(astorise/Magnetar-provider-CUDA src/tests_conformance.rs, cited per entry).
Expected outputs are computed here independently of the CPU oracle: float64
numpy for the f32 kernels (stored as the float32 rounding of the exact value,
with the tolerance each comparison uses), numpy float16 / an explicit bfloat16
rounding for the half path, exact arithmetic where the answer is exact.
The reference's oracle (magnetar_provider_cpu) itself is not available, so
these pin the restatement against the mathematics on the reference's inputs.

Run: python tests/golden/make_fixtures.py
"""
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def f32(x):
    return np.asarray(x, dtype=np.float32)


def bf16_rne(x):
    bits = f32(x).view(np.uint32).astype(np.uint64)
    rounded = (bits + 0x7FFF + ((bits >> 16) & 1)) >> 16
    return rounded.astype(np.uint16)


def rope_f64(x, base, dim, offset, heads, half_split=False):
    x = np.asarray(x, np.float64)
    rows, cols = x.shape
    hw = cols // heads
    out = x.copy()
    half = dim // 2
    for r in range(rows):
        pos = offset + r
        for h in range(heads):
            for p in range(half):
                theta = pos * base ** (-2.0 * p / dim)
                i1 = h * hw + (p if half_split else 2 * p)
                i2 = h * hw + (p + half if half_split else 2 * p + 1)
                a, b = x[r, i1], x[r, i2]
                out[r, i1] = a * np.cos(theta) - b * np.sin(theta)
                out[r, i2] = a * np.sin(theta) + b * np.cos(theta)
    return out


def main():
    fx = {}
    a23 = [[1, 2, 3], [4, 5, 6]]
    b23 = [[6, 5, 4], [3, 2, 1]]
    fx["add"] = {"source": "src/tests_conformance.rs:59-70", "a": a23, "b": b23,
                 "expected": (f32(a23) + f32(b23)).tolist(), "tolerance": 0}
    fx["mul"] = {"source": "src/tests_conformance.rs:106-117", "a": a23, "b": b23,
                 "expected": (f32(a23) * f32(b23)).tolist(), "tolerance": 0}
    a32 = [[1, 2], [3, 4], [5, 6]]
    fx["bias_add"] = {"source": "src/tests_conformance.rs:75-86", "a": a32, "bias": [100, 1000],
                      "expected": [[101, 1002], [103, 1004], [105, 1006]], "tolerance": 0}
    silu_in = [-2.0, -0.5, 0.0, 0.5, 1.0, 2.0]
    x = np.array(silu_in, np.float64)
    fx["silu"] = {"source": "src/tests_conformance.rs:119-125", "x": silu_in,
                  "expected": (x / (1 + np.exp(-x))).astype(np.float32).tolist(),
                  "tolerance": 3e-7}
    sm_in = [[1.0, 2.0, 3.0], [-1.0, 0.0, 1.0]]
    s = np.array(sm_in, np.float64)
    e = np.exp(s - s.max(axis=1, keepdims=True))
    fx["softmax"] = {"source": "src/tests_conformance.rs:127-136", "x": sm_in,
                     "expected": (e / e.sum(axis=1, keepdims=True)).astype(np.float32).tolist(),
                     "tolerance": 3e-7}
    table = [[0.0, 0.1, 0.2], [1.0, 1.1, 1.2], [2.0, 2.1, 2.2], [3.0, 3.1, 3.2]]
    fx["embedding"] = {"source": "src/tests_conformance.rs:138-161", "table": table,
                       "ids": [0.0, 2.0, 1.0],
                       "expected": f32(table)[[0, 2, 1]].tolist(), "tolerance": 0}
    fx["embedding_invalid"] = {"source": "src/tests_conformance.rs:163-175",
                               "table": [[0.0, 0.0], [0.0, 0.0]], "ids": [5.0],
                               "expected_status": 1}
    rx = np.array([[1.0, 2.0, 3.0], [-1.0, 0.5, 2.0]])
    rw = np.array([1.0, 0.5, 2.0])
    inv = 1.0 / np.sqrt((rx ** 2).mean(axis=1, keepdims=True) + 1e-5)
    fx["rmsnorm"] = {"source": "src/tests_conformance.rs:177-189", "x": rx.tolist(),
                     "weight": rw.tolist(), "eps": 1e-5,
                     "expected": (rx * inv * rw).astype(np.float32).tolist(), "tolerance": 3e-7}
    ropes = []
    ropes.append(dict(source="src/tests_conformance.rs:191-201",
                      x=[[1.0, 0.0, 0.0, 1.0], [0.5, 0.5, -0.5, -0.5]], base=10000.0,
                      dimension=4, offset=0, heads=1))
    ropes.append(dict(source="src/tests_conformance.rs:207-221",
                      x=(np.arange(16) * 0.25 - 2.0).reshape(2, 8).tolist(), base=10000.0,
                      dimension=2, offset=3, heads=4))
    ropes.append(dict(source="src/tests_conformance.rs:228-240",
                      x=(np.arange(16) * 0.1 - 0.8).reshape(2, 8).tolist(), base=10000.0,
                      dimension=2, offset=0, heads=2))
    ropes.append(dict(source="src/tests_conformance.rs:247-260",
                      x=(np.arange(16) * 0.05).reshape(2, 8).tolist(), base=10000.0,
                      dimension=4, offset=1, heads=2))
    for r in ropes:
        xin = f32(r["x"]).astype(np.float64)
        r["expected"] = rope_f64(xin, r["base"], r["dimension"], r["offset"], r["heads"]).astype(np.float32).tolist()
        r["tolerance"] = 1e-6
    fx["rope"] = ropes
    fx["matmul"] = {"source": "src/tests_conformance.rs:262-274", "a": a23,
                    "b": [[1, 0], [0, 1], [1, 1]], "expected": [[4, 5], [10, 11]], "tolerance": 0}
    fx["matmul_transposed_a"] = {"source": "src/tests_conformance.rs:276-288",
                                 "a": [[1, 4], [2, 5], [3, 6]], "b": [[1, 0], [0, 1], [1, 1]],
                                 "expected": [[4, 5], [10, 11]], "tolerance": 0}
    fx["attention_large_values"] = {"source": "src/tests_conformance.rs:2215-2245",
                                    "q": [[0.0, 0.0]], "k": [[0.0, 0.0]] * 4,
                                    "v": [[1e38, 1e38]] * 4, "heads": 1, "dimension": 2,
                                    "causal": False, "expected": [[1e38, 1e38]],
                                    "relative_tolerance": 1e-5}
    ha = [1.0, 2.5, 3.0, -4.25, 0.1, 100.0]
    hb = [6.0, 0.2, 4.0, 3.0, 0.2, -99.5]
    half = {"source": "src/tests_conformance.rs:2349-2423", "a": ha, "b": hb}
    for name, enc in (("f16", lambda v: f32(v).astype(np.float16).view(np.uint16)),
                      ("bf16", bf16_rne)):
        dec = (lambda h: h.view(np.float16).astype(np.float32)) if name == "f16" else \
            (lambda h: (h.astype(np.uint32) << 16).view(np.float32))
        ea, eb = enc(ha), enc(hb)
        half[f"{name}_a_bits"] = ea.tolist()
        half[f"{name}_b_bits"] = eb.tolist()
        half[f"{name}_add_bits"] = enc(dec(ea) + dec(eb)).tolist()
        half[f"{name}_mul_bits"] = enc(dec(ea) * dec(eb)).tolist()
    fx["half"] = half
    with open(os.path.join(HERE, "reference_fixtures.json"), "w") as f:
        json.dump(fx, f, indent=1)
    print("wrote", os.path.join(HERE, "reference_fixtures.json"))


if __name__ == "__main__":
    main()
