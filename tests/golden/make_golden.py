"""Writes tests/golden/rbf_ref_small.npz from the reference's own CPU loops.

The expected outputs come from cpu_forward / cpu_backward of the reference's
cases/rbf/delivery/rbf_test.cu:24-52, compiled in place into
oracle/_ref/librbf_ref.so (`make -C oracle ref`).  Inputs are drawn from a
fixed NumPy generator.  Run in the container that holds /root/reference:

    python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import native  # noqa: E402

CASES = [  # (name, N, M, D, gamma, input scale)
    ("tiny", 5, 7, 3, 1.0 / 64.0, 1.0),
    ("small", 8, 6, 64, 0.5, 0.125),
    ("ragged", 33, 17, 64, 0.5, 0.125),
    ("refdefault", 24, 40, 64, 1.0 / 64.0, 1.0),
]


def main():
    native.build(with_reference=True)
    assert native.ref_lib() is not None, "oracle/_ref/librbf_ref.so was not built"
    rng = np.random.default_rng(20240601)
    out = {}
    for name, N, M, D, gamma, scale in CASES:
        X = (rng.standard_normal((N, D)) * scale).astype(np.float32)
        Y = (rng.standard_normal((M, D)) * scale).astype(np.float32)
        G = rng.standard_normal((N, M)).astype(np.float32)
        K = native.ref_rbf_forward(X, Y, gamma)
        dX, dY = native.ref_rbf_backward(X, Y, G, K, gamma)
        for k, v in (("X", X), ("Y", Y), ("G", G), ("K", K), ("dX", dX), ("dY", dY)):
            out[f"{name}_{k}"] = v
        out[f"{name}_gamma"] = np.float32(gamma)
    path = os.path.join(HERE, "rbf_ref_small.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
