"""Writes the known-answer fixtures used by tests/test_oracle.py and the GPU
parity tests.

The inputs and expected values are the literal data of the reference's own
tests for this path, transcribed (not imported or run):

  q4dot_cases.json    internal/xblas/q4dot_test.go:11-86 (TestQ4DotBlock: six
                      nibble/scale/x cases; expected = sum over i of
                      float32(nib[i]-8)*scale*x[i] accumulated in fp32, the
                      test's own definition at :69-74) and :127-140 (zero
                      scale -> 0)
  ternary_cases.json  compute/ternary_gemv_test.go:25-45 (3x4 -> {3,1,-4}),
                      :76-90 (all zeros), :92-101 (1x1), :103-123 (identity
                      33x33), :125-141 (2x5 -> {-2,4});
                      tensor/ternary_storage_test.go:174-196 (byte counts)
  iq4nl_cases.json    tensor/iq4_storage_test.go:21-42 (nibbles i%16,
                      scale 2.0), :44-84 (two blocks, scales 1.5/0.75,
                      nibbles (7*bi+3*i)%16), :86-120 (48 elements, partial
                      block), :157-175 (table properties)

Run: python tests/golden/make_golden.py
"""
import json
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def f32(v):
    return float(np.float32(v))


def q4dot_cases():
    rnd = [3, 12, 7, 1, 14, 5, 9, 0, 15, 8, 2, 11, 6, 13, 4, 10]
    xr = [0.5, -0.3, 1.2, -0.7, 0.1, 0.9, -1.1, 0.4, -0.2, 0.8, 0.6, -0.5, 1.0, -0.8, 0.3, 0.7]
    alt = [15, 0] * 16
    cases = [
        ("zero block", [8] * 32, 1.0, [1, 2, 3, 4, 5, 6, 7, 8] * 4),
        ("all same nibble 15", [15] * 32, 0.5, [1.0] * 32),
        ("all same nibble 0", [0] * 32, 0.5, [1.0] * 32),
        ("max scale", alt, 100.0, [0.1] * 32),
        ("min scale", alt, 0.001, [1.0] * 32),
        ("random pattern", rnd + rnd, 0.25, xr + xr),
    ]
    out = []
    for name, nib, scale, x in cases:
        x32 = np.array(x, np.float32)
        s32 = np.float32(scale)
        want = np.float32(0)
        for i in range(32):
            want = np.float32(want + np.float32(np.float32(nib[i] - 8) * s32) * x32[i])
        out.append({"name": name, "nibbles": nib, "scale": f32(scale), "x": [f32(v) for v in x], "want": f32(want)})
    out.append({"name": "zero scale", "nibbles": [15] * 32, "scale": 0.0, "x": [1.0] * 32, "want": 0.0})
    return out


def ternary_cases():
    ident = np.zeros((33, 33), np.int8)
    np.fill_diagonal(ident, 1)
    xid = [f32(i * 0.5 - 8.0) for i in range(33)]
    return {
        "gemv": [
            {"name": "known_values", "rows": 3, "cols": 4, "w": [1, 0, -1, 1, -1, 1, 0, 0, 0, -1, 1, -1],
             "x": [2.0, 3.0, 4.0, 5.0], "want": [3.0, 1.0, -4.0]},
            {"name": "all_zeros", "rows": 16, "cols": 32, "w": [0] * 512, "x": [float(i + 1) for i in range(32)],
             "want": [0.0] * 16},
            {"name": "single_element_neg", "rows": 1, "cols": 1, "w": [-1], "x": [7.5], "want": [-7.5]},
            {"name": "single_element_zero", "rows": 1, "cols": 1, "w": [0], "x": [7.5], "want": [0.0]},
            {"name": "single_element_pos", "rows": 1, "cols": 1, "w": [1], "x": [7.5], "want": [7.5]},
            {"name": "identity_diagonal", "rows": 33, "cols": 33, "w": ident.reshape(-1).tolist(), "x": xid,
             "want": xid},
            {"name": "non_multiple_of_4_cols", "rows": 2, "cols": 5, "w": [1, -1, 0, 1, -1, 0, 1, -1, 0, 1],
             "x": [1.0, 2.0, 3.0, 4.0, 5.0], "want": [-2.0, 4.0]},
        ],
        "byte_counts": [[0, 0], [1, 1], [2, 1], [3, 1], [4, 1], [5, 2], [8, 2], [9, 3], [100, 25]],
    }


def iq4nl_cases():
    def block(scale, nib):
        return {"scale": scale, "nibbles": nib}

    return {
        "single_block": block(2.0, [i % 16 for i in range(32)]),
        "two_blocks": [block(1.5, [(bi * 7 + i * 3) % 16 for i in range(32)]) if bi == 0 else
                       block(0.75, [(bi * 7 + i * 3) % 16 for i in range(32)]) for bi in range(2)],
        "partial": {"num_elements": 48, "blocks": [block(1.0, [i % 16 for i in range(32)])] * 2},
        "table_zero_index": 7,
    }


if __name__ == "__main__":
    (HERE / "q4dot_cases.json").write_text(json.dumps(q4dot_cases(), indent=1))
    (HERE / "ternary_cases.json").write_text(json.dumps(ternary_cases()))
    (HERE / "iq4nl_cases.json").write_text(json.dumps(iq4nl_cases(), indent=1))
    print("wrote fixtures to", HERE)
