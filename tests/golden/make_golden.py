"""Writes tests/golden/golden.npz: small input/output vectors of the oracle.

    python -m tests.golden.make_golden

The reference is Rust and cannot run in this image, so these vectors come
from the CPU oracle (oracle/nrq_oracle.c), whose pins are in
tests/test_oracle.py. They freeze the oracle's outputs (a regression check on
it) and give the GPU tests a fixed, seeded set of inputs with known answers:
ragged row counts, several blocks per row, both f32 orders, a batch of 5
(one 4-wide tile plus a remainder), and adversarial activations.
"""
from __future__ import annotations

import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "golden.npz")

SHAPES = {1: (37, 160), 2: (37, 768), 3: (37, 768)}  # dtype -> (rows, cols)
NAMES = {1: "q8_0", 2: "q4k", 3: "q6k"}


def build(O) -> dict:
    g = {}
    for dtype, (rows, cols) in SHAPES.items():
        n = NAMES[dtype]
        qk = O.QK[dtype]
        rng = O.Rng(0x5EED0000 + dtype)
        w = O.quantize_weights_ref(dtype, rng.adversarial(rows * cols))
        xf = rng.normal(cols)
        xsf = rng.adversarial(5 * cols)
        x = O.quantize_act(dtype, xf)
        xs = O.quantize_act(dtype, xsf)
        g[f"{n}_w"] = w
        g[f"{n}_xf"] = xf
        g[f"{n}_x"] = x
        g[f"{n}_xsf"] = xsf
        g[f"{n}_xs"] = xs
        for order, on in ((O.ORDER_SCALAR, "scalar"), (O.ORDER_AVX2, "avx2")):
            g[f"{n}_y_{on}"] = O.matvec(dtype, order, w, x, rows, cols)
            g[f"{n}_ym_{on}"] = O.matmul(dtype, order, w, xs, rows, cols, 5)
        bpr = cols // qk
        g[f"{n}_sums"] = np.concatenate([O.block_sums(dtype, w[r * bpr:(r + 1) * bpr], x) for r in range(rows)])
    return g


def main() -> None:
    import oracle as O

    O.build()
    np.savez_compressed(OUT, **build(O))
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
