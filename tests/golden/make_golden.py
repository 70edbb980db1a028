"""Regenerates tests/golden/fills.json with implementations independent of the C
oracle: Python integers for the LCG and splitmix64 state, numpy's float32
arithmetic and float16 casts for the value and its rounding.

    python tests/golden/make_golden.py

The reference fill (check-gemm.cu:139-145) and the splitmix64 mixer (Steele, Lea,
Flood 2014) are restated here from their published definitions.
"""
import json
import os

import numpy as np

M32 = (1 << 32) - 1
M64 = (1 << 64) - 1


def lcg_states(seed, n):
    s, out = seed & M32, []
    for _ in range(n):
        s = (s * 1664525 + 1013904223) & M32
        out.append(s)
    return out


def lcg_value_bits(state):
    v = np.float32((state >> 16) & 0x7FFF) / np.float32(32767.0) - np.float32(0.5)
    return int(np.array([v], dtype=np.float32).astype(np.float16).view(np.uint16)[0])


def splitmix64(seed, n):
    s, out = seed & M64, []
    for _ in range(n):
        s = (s + 0x9E3779B97F4A7C15) & M64
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
        out.append(z ^ (z >> 31))
    return out


def uniform_bits(seed, n):
    bits = []
    for z in splitmix64(seed, n):
        v = np.float32(z >> 40) * np.float32(1.0 / 8388608.0) - np.float32(1.0)
        bits.append(int(np.array([v], dtype=np.float32).astype(np.float16).view(np.uint16)[0]))
    return bits


def main():
    seeds = [0x1234 + 256, 0x9ABC + 512, 0x55AA, 0xC0FFEE]
    fix = {
        "lcg": {str(s): {"states": lcg_states(s, 16), "half_bits": [lcg_value_bits(x) for x in lcg_states(s, 16)]}
                for s in seeds},
        "splitmix64": {"1234567": [str(x) for x in splitmix64(1234567, 5)]},
        "uniform": {str(s): uniform_bits(s, 16) for s in (1, 2, 0x5EED)},
    }
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "fills.json")
    with open(path, "w") as f:
        json.dump(fix, f, indent=1)
    print("wrote", path)


if __name__ == "__main__":
    main()
