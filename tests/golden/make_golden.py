#!/usr/bin/env python3
"""Writes the golden fixtures under tests/golden/ from the reference's own CPU
paths compiled by oracle/Makefile into oracle/_ref: IntLSE
(intlse/cpu/lse_kernel_simd.c -> liblse_kernel_simd.so) and FuseLSE-CPU
(fuselse/cpu/fused_fp32_cpu.cpp -> fused_fp32_cpu.so).  Run in the container
that has the reference tree mounted:

    make -C oracle && python tests/golden/make_golden.py [intlse] [fuselse_cpu]

Fixtures are data only: seeded inputs and the reference's outputs.
  intlse_cpu_ref.npz : rows x (fp32) and outputs of lse_q16_2d_simd and
                       lse_q16_2d_simd_neg_inf for shapes covering the scalar
                       path (N < 64), whole 64-blocks, odd block counts,
                       scalar tails, saturation and -inf entries.
  q16_pair_ref.npz   : N=2 rows (scalar quantiser + one scalar pair) over a
                       dense sweep of operand gaps, and the reference outputs.
  fuselse_cpu_ref.npz: rows x (fp32) and outputs of cpu_lse_float for the C1
                       shapes (32, 256) and (200, 1000) with x ~ N(0, 1), a C2
                       style sample (N(0, 3^2) with +15 spikes), N = 1, 2, 3,
                       and rows with ties, -inf, +inf, NaN, -1e30 and huge
                       values.
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


def fuselse_cpu_rows_for_fixture():
    """(name, rows) sets of the FuseLSE-CPU fixture."""
    sets = [("c1_32x256", np.random.default_rng(0).standard_normal((32, 256), dtype=np.float32)),
            ("c1_200x1000", np.random.default_rng(0).standard_normal((200, 1000), dtype=np.float32)),
            ("c2_sample_4x20000", O.make_c2_input(4, 20000, seed=3)),
            ("n1", np.array([[1.5], [-np.inf], [np.nan]], np.float32)),
            ("n2", np.array([[0.0, 0.0], [1.0, -1.0], [-30.0, 30.0], [3e38, 3e38], [-np.inf, 2.0],
                             [2.0, -np.inf], [-np.inf, -np.inf]], np.float32)),
            ("n3", np.array([[0.0, 0.0, 0.0], [1e-30, -1e-30, 0.0], [-1e30, -1e30, -1e30]], np.float32))]
    sp = np.random.default_rng(5).standard_normal((8, 513)).astype(np.float32)
    sp[0, :] = 7.25                  # ties throughout
    sp[1, 10] = np.inf
    sp[2, 100] = np.nan
    sp[3, ::3] = -np.inf
    sp[4, 0] = -np.inf               # -inf seed: -inf - -inf never arises, x > y picks the finite
    sp[5, :] = -1e30
    sp[6, 7] = 1e30
    sp[7, :] = -np.inf
    sets.append(("special_8x513", sp))
    return sets


def write_fuselse_cpu():
    if not O.ref_fuselse_available():
        raise SystemExit("oracle/_ref/fused_fp32_cpu.so not built: run `make -C oracle` with the reference tree")
    names, shapes, xs, outs = [], [], [], []
    for name, x in fuselse_cpu_rows_for_fixture():
        names.append(name)
        shapes.append(x.shape)
        xs.append(x.ravel())
        outs.append(O.ref_fuselse_cpu(x))
    np.savez_compressed(os.path.join(HERE, "fuselse_cpu_ref.npz"), names=np.array(names),
                        shapes=np.array(shapes, np.int64), x=np.concatenate(xs), out=np.concatenate(outs))


def main():
    which = set(sys.argv[1:]) or {"intlse", "fuselse_cpu"}
    if "fuselse_cpu" in which:
        write_fuselse_cpu()
    if "intlse" in which:
        write_intlse()
    print("wrote", sorted(os.listdir(HERE)))


def write_intlse():
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


if __name__ == "__main__":
    main()
