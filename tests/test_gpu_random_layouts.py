"""GPU parity over seeded random layouts, at the same bars as tests/test_gpu_parity.py.

The hand-written cases use small shapes; the kernels pick their path by size and layout, so these
cases are drawn (from a fixed seed, so every run sees the same ones) to land on each path: whole
and partial 64x64 tiles of a transposed operand, broadcasts on any axis, ranks 1-4, long rows that
the row reduction splits into ordered segments, tall columns that the leading-axis reduction splits
into chunks, middle-axis reductions (the generic kernel), and their backwards. Values are normal,
special (signed zeros, infinities, NaN, denormals, extremes) or small integers (ties)."""
from __future__ import annotations

import numpy as np
import pytest

from cases import BINARY, REDUCE, UNARY, Arr, Case, _bshape, _red_shape
from plast_amd.abi import DIM_ALL
from test_gpu_parity import check_case

pytestmark = pytest.mark.gpu

DIMS = [1, 2, 3, 5, 7, 16, 31, 64, 65, 130]


def _dist(rng, op):
    if op in ("log", "div"):
        return "pos"
    return str(rng.choice(["normal", "normal", "special", "ties"]))


def _shape(rng, rank, cap=1 << 20):
    while True:
        sh = tuple(int(rng.choice(DIMS)) for _ in range(rank))
        if np.prod(sh) <= cap:
            return sh


def random_cases(n: int, seed: int) -> list[Case]:
    rng = np.random.RandomState(seed)
    cases = []
    for i in range(n):
        kind = ["binary", "tile", "unary", "rows", "cols", "middle", "binary_bwd", "reduce_bwd"][i % 8]
        s = seed * 10000 + i * 10
        if kind in ("binary", "binary_bwd"):
            op = str(rng.choice(BINARY))
            rank = rng.randint(1, 5)
            sa = _shape(rng, rank)
            tr = None
            if rank >= 2 and rng.rand() < 0.5:
                d0, d1 = sorted(rng.choice(rank, 2, replace=False))
                tr = (int(d0), int(d1))
            bwd = kind == "binary_bwd"
            a = Arr(sa, _dist(rng, "x"), s, transpose=tr, requires_grad=bwd)
            # b: a trailing part of a's view shape with some axes broadcast
            vs = a.view_shape
            sb = tuple(d if rng.rand() < 0.6 else 1 for d in vs[rng.randint(0, rank):])
            b = Arr(sb, _dist(rng, op), s + 1, requires_grad=bwd)
            cases.append(Case(f"s{seed}r{i}_{op}_{'bwd' if bwd else 'fwd'}_{sa}_{sb}_{tr}", op,
                              "bwd" if bwd else "fwd", [a, b], _bshape(a.view_shape, sb),
                              exact=not (bwd and sb != a.view_shape)))
        elif kind == "tile":
            # a transposed operand over whole or partial 64x64 tiles, plus a broadcast operand
            op = str(rng.choice(BINARY))
            p, q = (int(rng.choice([64, 65, 128, 130, 200, 256])) for _ in range(2))
            bat = int(rng.choice([1, 2, 3]))
            a = Arr((bat, p, q), _dist(rng, "x"), s, transpose=(1, 2))
            vs = a.view_shape
            sb = [(1, vs[1], 1), (bat, 1, vs[2]), (vs[2],), vs][rng.randint(0, 4)]
            cases.append(Case(f"s{seed}r{i}_{op}_tile_{a.shape}_{sb}", op, "fwd",
                              [a, Arr(tuple(sb), _dist(rng, op), s + 1)], _bshape(vs, tuple(sb))))
        elif kind == "unary":
            op = str(rng.choice(UNARY))
            rank = rng.randint(1, 4)
            sh = _shape(rng, rank)
            tr = (0, rank - 1) if rank >= 2 and rng.rand() < 0.5 else None
            a = Arr(sh, _dist(rng, op), s, transpose=tr)
            al = float(rng.choice([0.0, 0.01])) if op == "leaky_relu" else 0.0
            cases.append(Case(f"s{seed}r{i}_{op}_{sh}_{tr}", op, "fwd", [a], a.view_shape, (0, 0, al)))
        else:
            op = str(rng.choice(REDUCE + ["argmax"]))
            if kind == "rows":      # few long rows: ordered segments
                sh = (int(rng.choice([1, 2, 3, 7])), int(rng.choice([8192, 10001, 40000])))
                dim = int(rng.choice([1, DIM_ALL]))
            elif kind == "cols":    # tall columns: chunks of the leading axis
                sh = (int(rng.choice([128, 300, 5000])), int(rng.choice([3, 64, 256, 1000])))
                dim = 0
            elif kind == "middle":  # a middle axis, with or without a transposed view
                sh = _shape(rng, 3, 1 << 18)
                dim = 1
            else:                   # reduce_bwd
                op = str(rng.choice(REDUCE))
                sh = _shape(rng, rng.randint(1, 4), 1 << 18)
                dim = int(rng.choice(list(range(len(sh))) + [DIM_ALL]))
            keep = 0 if dim == DIM_ALL else int(rng.randint(0, 2))
            tr = (0, 1) if kind == "middle" and rng.rand() < 0.5 else None
            bwd = kind == "reduce_bwd"
            a = Arr(sh, _dist(rng, "x"), s, transpose=tr, requires_grad=bwd)
            cases.append(Case(f"s{seed}r{i}_{op}_{'bwd' if bwd else 'fwd'}_{sh}_d{dim}_k{keep}_{tr}", op,
                              "bwd" if bwd else "fwd", [a], _red_shape(a.view_shape, dim, keep),
                              (dim, keep, 0.0), "i64" if op == "argmax" else "f32"))
    return cases


# seed 102's 400 include broadcast gradients of thousands of cancelling terms (r150, r326)
CASES = random_cases(160, 7) + random_cases(400, 102)


@pytest.mark.parametrize("c", CASES, ids=[c.id for c in CASES])
def test_random_layout(c):
    check_case(c)
