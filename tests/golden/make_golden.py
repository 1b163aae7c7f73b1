#!/usr/bin/env python3
"""Writes the golden fixtures under tests/golden/ from the reference's own CPU
IntLSE (intlse/cpu/lse_kernel_simd.c compiled by oracle/Makefile into
oracle/_ref/liblse_kernel_simd.so).  Run in the container that has the
reference tree mounted:

    make -C oracle && python tests/golden/make_golden.py

Fixtures are data only: seeded inputs and the reference's outputs.
  intlse_cpu_ref.npz : rows x (fp32) and outputs of lse_q16_2d_simd and
                       lse_q16_2d_simd_neg_inf for shapes covering the scalar
                       path (N < 64), whole 64-blocks, odd block counts,
                       scalar tails, saturation and -inf entries.
  q16_pair_ref.npz   : N=2 rows (scalar quantiser + one scalar pair) over a
                       dense sweep of operand gaps, and the reference outputs.
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402

SHAPES = [(4, 2), (4, 3), (6, 17), (6, 63), (6, 64), (6, 65), (5, 127), (5, 128), (5, 129), (4, 200),
          (3, 1000), (3, 4097), (2, 9000), (1, 33000)]


def rows_for(shape, seed):
    rng = np.random.default_rng(seed)
    B, N = shape
    lo, hi = [(-1, 0), (-100, 0), (-500, 0), (-10, 10)][seed % 4]
    x = (rng.random((B, N)) * (hi - lo) + lo).astype(np.float32)
    if B >= 4 and N >= 3:
        x[-1, ::7] = -np.inf          # sparse -inf
        x[-2, 1] = 3.0e9               # saturates the quantiser, wraps the pair difference
        x[-3, 0] = -3.0e9
    return x


def main():
    if not O.ref_available():
        raise SystemExit("oracle/_ref not built: run `make -C oracle` with the reference tree mounted")
    xs, outs, outs_ni, shapes = [], [], [], []
    for k, shp in enumerate(SHAPES):
        x = rows_for(shp, k)
        xs.append(x.ravel())
        outs.append(O.ref_intlse_cpu_rows(x, False))
        outs_ni.append(O.ref_intlse_cpu_rows(x, True))
        shapes.append(shp)
    np.savez_compressed(os.path.join(HERE, "intlse_cpu_ref.npz"),
                        shapes=np.array(shapes, np.int64),
                        x=np.concatenate(xs), out=np.concatenate(outs), out_neg_inf=np.concatenate(outs_ni))

    # N=2 rows: a = 0, b = -d / CONV for a dense set of gaps d (in Q16 LSBs),
    # plus random pairs over a wide range.
    d = np.concatenate([np.arange(0, 70000, 1), np.arange(70000, 1_200_000, 97)]).astype(np.float64)
    b = (-d / float(O.Q16_CONV)).astype(np.float32)
    a = np.zeros_like(b)
    rng = np.random.default_rng(99)
    ra = (rng.standard_normal(20000) * 40).astype(np.float32)
    rb = (rng.standard_normal(20000) * 40).astype(np.float32)
    pairs = np.stack([np.concatenate([a, ra]), np.concatenate([b, rb])], axis=1)
    out = O.ref_intlse_cpu_rows(pairs, False)
    np.savez_compressed(os.path.join(HERE, "q16_pair_ref.npz"), x=pairs, out=out)
    print("wrote", os.listdir(HERE))


if __name__ == "__main__":
    main()
