"""Writes config C1's committed fixture (tests/golden/gemm_256.npz) as the raw arrays
TestGPUMatMulC1Golden reads from $GONNGPU_C1_FIXTURE: A (256x256 float32), B (256x256
float32), then the float64 reference product C64, row-major, back to back."""
import os
import sys

import numpy as np

GOLD = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "golden", "gemm_256.npz")


def write(path):
    z = np.load(GOLD)
    with open(path, "wb") as f:
        f.write(np.ascontiguousarray(z["A"], dtype=np.float32).tobytes())
        f.write(np.ascontiguousarray(z["B"], dtype=np.float32).tobytes())
        f.write(np.ascontiguousarray(z["C64"], dtype=np.float64).tobytes())


if __name__ == "__main__":
    write(sys.argv[1])
