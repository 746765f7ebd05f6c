"""Writes tests/golden/q4_k_q6_k.npz: Q4_K and Q6_K blocks and their values for a
fixed row of 1024 weights (a closed-form sequence, no RNG), as the oracle's
quantizers produce them.  The hand-built known-answer tests in test_oracle.py pin
the block layouts; this fixture freezes the quantizers' exact bits so that the
product's own quantizers (and any later change to either) are held to them."""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import oracle as O  # noqa: E402


def row():
    i = np.arange(1024, dtype=np.float64)
    x = 0.03 * np.sin(i * 0.37) + 0.011 * np.cos(i * 1.91) - 0.004 * ((i % 29) / 29.0)
    x[256:288] = np.abs(x[256:288])          # a sub-block with no negative weight
    x[512:528] = 0.0                           # a Q6_K group of zeros
    x[700] = -0.2                              # an outlier
    return x.astype(np.float32)


def main():
    x = row()
    q4k = O.quantize_q4_k_row(x)
    q6k = O.quantize_q6_k_row(x)
    np.savez(os.path.join(os.path.dirname(os.path.abspath(__file__)), "q4_k_q6_k.npz"),
             x=x, q4_k=q4k, q4_k_values=O.dequantize_q4_k_row(q4k, x.size),
             q6_k=q6k, q6_k_values=O.dequantize_q6_k_row(q6k, x.size))


if __name__ == "__main__":
    main()
