"""Writes the golden fixtures under tests/golden/ (numpy only, no product or
oracle code involved).

sym8_kat.json — the known-answer test of RwkvqFileTests.swift:237-256
(testSymOffSuperblockShapeUsesChain): OUT = 2, IN = 48, codes
Int8(truncatingIfNeeded: i·37 − 90), block scales qs = [3, -5, 7, 11, -2, 1],
super-block scales d = [0.0123, 0.25] stored as fp16.  Expected weights are
computed as the test states them: scale = Float(Float16(Float(qs)·d16)),
w = Float(code)·scale, with numpy's IEEE float16 as the half type.

Run:  python tests/golden/make_golden.py
"""
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def sym8_kat():
    OUT, IN = 2, 48
    codes = np.array([((i * 37 - 90) + 128) % 256 - 128 for i in range(OUT * IN)], dtype=np.int8)
    qs = np.array([3, -5, 7, 11, -2, 1], dtype=np.int8)
    d16 = np.array([0.0123, 0.25], dtype=np.float32).astype(np.float16)
    dh = d16.astype(np.float32)
    want = []
    for r in range(OUT):
        for c in range(IN):
            scale = np.float32(np.float16(np.float32(qs[r * 3 + c // 16]) * dh[r]))
            want.append(float(np.float32(codes[r * IN + c]) * scale))
    return {
        "source": "Tests/RWKVGenTests/RwkvqFileTests.swift:237-256",
        "OUT": OUT, "IN": IN, "bits": 8,
        "codes_u8": [int(x) for x in codes.view(np.uint8)],
        "qs_u8": [int(x) for x in qs.view(np.uint8)],
        "d_f16_bits": [int(x) for x in d16.view(np.uint16)],
        "expected_f32": want,
    }


if __name__ == "__main__":
    with open(os.path.join(HERE, "sym8_kat.json"), "w") as f:
        json.dump(sym8_kat(), f, indent=1)
    print("wrote sym8_kat.json")
