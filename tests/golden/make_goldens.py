"""Writes tests/golden/reference_goldens.json: the known-answer vectors that
the reference's own tests hold for this path, as input/expected data.

Each entry names the reference test it comes from.  Inputs are rebuilt from
the recipes those tests state (deterministic formulas), the expected values
are the numbers those tests assert.  Run: python tests/golden/make_goldens.py
"""
import json
import os

import numpy as np

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_goldens.json")


def q4k_golden_block():
    # crates/sosomodel/tests/dequant_golden.rs:18-34 (same recipe in
    # tools/gsp-hostcheck/main.c:2629-2700): d = 0.5 (0x3800), dmin = 0.25
    # (0x3400), fixed scales, qs[i] = (i*7+3) % 256.
    b = np.zeros(144, dtype=np.uint8)
    b[0], b[1], b[2], b[3] = 0x00, 0x38, 0x00, 0x34
    b[4:16] = [0x41, 0x82, 0xC3, 0x04, 0x45, 0x86, 0xC7, 0x08, 0x9A, 0xBC, 0xDE, 0xF0]
    b[16:] = [(i * 7 + 3) % 256 for i in range(128)]
    return b


def x256():
    # dequant_golden.rs:36-42: x[i] = ((i % 13) - 6) * 0.125
    return [((i % 13) - 6) * 0.125 for i in range(256)]


def q80_golden_block():
    # dequant_golden.rs:95-105: scale 0.25 (f32 LE) + q[i] = (i*9 - 100) as i8
    b = np.zeros(36, dtype=np.uint8)
    b[:4] = np.frombuffer(np.float32(0.25).tobytes(), dtype=np.uint8)
    b[4:] = [((i * 9 - 100) + 256) % 256 for i in range(32)]
    return b


def q6k_known_block():
    # crates/gguf2som/src/lib.rs:1868-1876: ql = qh = 0, scales = 1, d = f16(1/32)
    b = np.zeros(210, dtype=np.uint8)
    b[192:208] = 1
    b[208], b[209] = 0x00, 0x28  # 1/32 = 2^-5 in f16
    return b


def main():
    g = {
        "q4k_golden": {
            "source": "crates/sosomodel/tests/dequant_golden.rs:44-93",
            "block_hex": q4k_golden_block().tobytes().hex(),
            "x": x256(),
            "scale_min": [[1, 5], [2, 6], [3, 7], [4, 8], [26, 25], [44, 43], [62, 61], [0, 15]],
            "dot": -15.875, "dot_tol": 1e-2,
        },
        "q80_golden": {
            "source": "crates/sosomodel/tests/dequant_golden.rs:95-114",
            "block_hex": q80_golden_block().tobytes().hex(),
            "x": x256()[:32],
            "dot": 172.59375, "dot_tol": 1e-3,
        },
        "q6k_known": {
            "source": "crates/gguf2som/src/lib.rs:1868-1889",
            "block_hex": q6k_known_block().tobytes().hex(),
            "value": -1.0,
        },
        "f16_cases": {
            "source": "crates/soso-llm-core/src/f16.rs:43-52",
            "cases": [[0x3C00, 1.0], [0xBC00, -1.0], [0x3800, 0.5], [0x0000, 0.0], [0x0001, 2.0 ** -24]],
            "inf": [0x7C00], "nan": [0x7E00],
        },
        "row_bytes": {
            "source": "crates/soso-llm-core/src/quant.rs:409-420",
            "cases": [[3, 256, 144], [3, 5632, 22 * 144], [3, 255, None], [3, 0, None],
                      [2, 32, 36], [2, 33, None], [1, 256, None]],
        },
        "q4k_known_positions": {
            "source": "crates/soso-llm-core/src/quant.rs:433-449 (block of quant.rs:221-237)",
            "sc": [1, 2, 3, 4, 33, 34, 35, 63], "m": [0, 1, 2, 3, 48, 49, 50, 62],
            "d": 0.5, "dmin": 0.25,
            "positions": [[0, 0, 0, 0], [5, 0, 5, 0], [32, 1, 0, 1], [64, 2, 0, 2], [65, 2, 1, 2], [255, 7, 9, 7]],
            "note": "positions: [element, scale index, q, min index]; qs byte i = (i%16) | ((i*7)%16)<<4",
        },
        "topk": {
            "source": "crates/soso-llm-core/tests/moe.rs:146-153",
            "logits": [1.0, 2.0, 3.0, 0.5], "k": 2, "first": 2,
        },
    }
    with open(OUT, "w") as f:
        json.dump(g, f, indent=1)
    print(OUT)


if __name__ == "__main__":
    main()
