"""Writes tests/golden/bfp16_kat.json: hand-derived known answers of the bfp16ebs8 encoder.

Every case below is derived by hand from the format definition (redline/npu_layouts.py:62-73: E = the largest
float32 exponent field of the block, q = clip(rint(x * 2^(133 - E)), -128, 127), round half to even), not computed
by the oracle, so that the oracle and the GPU kernel are both checked against an independent statement. The reasoning
for each case is in its "why" field. Run: python tests/golden/make_vectors.py
"""

import json
import os
import struct


def f32_hex(x):
    return struct.pack("<f", x).hex()


CASES = [
    # x values, E, q, why
    ([1.0, 0, 0, 0, 0, 0, 0, 0], 127, [64, 0, 0, 0, 0, 0, 0, 0],
     "1.0 has exponent field 127; 1.0 * 2^(133-127) = 64; the kernels' identity row (kernels/glue/ln_mod.cc:41-43)"),
    ([0.0] * 8, 0, [0] * 8, "all zeros: E = 0, every q = 0"),
    ([1.0, 2**-7, 3 * 2**-7, -2**-7, 255 / 128, -255 / 128, 5 * 2**-7, 0.0], 127,
     [64, 0, 2, 0, 127, -128, 2, 0],
     "scale 64: 2^-7 -> 0.5 ties to 0; 3*2^-7 -> 1.5 ties to 2; -0.5 -> -0; 255/128 -> 127.5 -> 128 saturates to "
     "127; -127.5 -> -128 is kept; 2.5 ties to 2"),
    ([3.0, 0, 0, 0, 0, 0, 0, 0], 128, [96, 0, 0, 0, 0, 0, 0, 0], "3.0 = 1.5 * 2^1, E = 128, 3 * 2^5 = 96"),
    ([1024.0, 1.0, 0, 0, 0, 0, 0, 0], 137, [64, 0, 0, 0, 0, 0, 0, 0],
     "E = 137 (2^10), scale 2^-4: 1.0 -> 0.0625 rounds to 0"),
    ([2**-127, 0, 0, 0, 0, 0, 0, 0], 0, [64, 0, 0, 0, 0, 0, 0, 0],
     "a subnormal block: E = 0, scale 2^133, 2^-127 * 2^133 = 64; decodes back to exactly 2^-127"),
    ([-1.0, 0.75, -0.5, 0.25, 1.9921875, -1.9921875, 0.0078125, -0.0078125], 127,
     [-64, 48, -32, 16, 127, -128, 0, 0],
     "scale 64: 1.9921875 * 64 = 127.5 rounds to 128 and saturates to 127; -127.5 is a tie and rounds to the even "
     "-128, which is in range; +-0.5 tie to 0"),
    ([2.0**100, -(2.0**100) * 1.5, 1.0, 0, 0, 0, 0, 0], 227, [64, -96, 0, 0, 0, 0, 0, 0],
     "E = 227 (2^100): 1.5 * 64 = 96; 1.0 underflows to 0"),
    ([6.0, 5.0, 4.0, 3.0, 2.0, 1.0, 0.5, 0.25], 129, [96, 80, 64, 48, 32, 16, 8, 4],
     "E = 129 (max |x| in [4, 8)), scale 2^4: exact integers"),
    ([1.0 + 2**-7, 1.0 + 3 * 2**-7, 1.0 + 2**-6, 0, 0, 0, 0, 0], 127, [64, 66, 65, 0, 0, 0, 0, 0],
     "scale 64: 64.5 ties to the even 64; 65.5 ties to the even 66; 65 is exact"),
]


def main():
    rows = []
    for x, E, q, why in CASES:
        b = bytes([E]) + bytes((v & 0xFF) for v in q)
        rows.append({"x_f32_hex": [f32_hex(float(v)) for v in x], "E": E, "q": q, "bytes_hex": b.hex(), "why": why})
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "bfp16_kat.json")
    with open(path, "w") as f:
        json.dump({"format": "bfp16ebs8 [E][q0..q7], redline/npu_layouts.py:62-73", "cases": rows}, f, indent=1)
    print(f"wrote {len(rows)} cases to {path}")


if __name__ == "__main__":
    main()
