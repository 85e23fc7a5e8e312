"""Sums whose fp32 value overflows, or meets inf - inf, have an outcome that depends on the order of
the additions: the reference adds in index order from 0.0f (reduce_ops.c:57-61), so
[3e38, 3e38, -inf] sums to NaN there (+inf first) while [-inf, 3e38, 3e38] stays -inf. A GPU sum
that comes out non-finite is summed again in that order, so it equals the oracle's bit for bit
(NaN against NaN). A GPU sum that stays finite where the serial one overflowed is closer to the
exact value and passes the usual bar (within 1e-5 * sum|x| of the oracle, or at least as close to
the float64 sum). Cases cover each reduction path: one wave per row, rows split into segments, the
whole tensor, the leading axis in one chunk and in several, and the mean."""
from __future__ import annotations

import numpy as np
import pytest

from cases import assert_sum_parity
from hostlib import HostTensor, oracle_forward

pytestmark = pytest.mark.gpu

BIG = np.float32(3e38)
INF = np.float32(np.inf)


def _lines(n, count, rng):
    """`count` lines of n values: each an order-sensitive overflow pattern or a finite control."""
    out = []
    for i in range(count):
        x = rng.randn(n).astype(np.float32)
        k = i % 6
        if k == 0:                      # overflow to +inf, then -inf: NaN in index order
            x[:4] = BIG
            x[-1] = -INF
        elif k == 1:                    # -inf first: stays -inf in index order
            x[0] = -INF
            x[1:5] = BIG
        elif k == 2:                    # overflow to +inf then back down with -3e38s: stays +inf
            x[:2] = BIG
            x[n // 2:n // 2 + 3] = -BIG
        elif k == 3:                    # the negatives first: -inf, then +3e38s cannot undo it
            x[:3] = -BIG
            x[n // 2:n // 2 + 4] = BIG
        elif k == 4:                    # a NaN anywhere: NaN in every order
            x[n // 3] = np.nan
            x[:2] = BIG
        out.append(x)                   # k == 5: finite
    return np.stack(out)


def _check(x, op, dim, keep=0):
    from plast_amd import ops, runtime as rt
    from plast_amd.abi import KernelParams
    dx = rt.DeviceTensor.from_numpy(x)
    got = ops.reduce(op, dx, None if dim == 9 else dim, bool(keep)).numpy()
    shape = got.shape
    want = HostTensor(np.zeros(shape, np.float32))
    oracle_forward(op, [HostTensor(x)], want, KernelParams(dim, keep, 0.0))
    x64 = x.astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        if dim == 9:
            truth, scale = np.array([x64.sum()]), np.array([np.abs(x64).sum()])
        else:
            truth, scale = x64.sum(axis=dim, keepdims=bool(keep)), np.abs(x64).sum(axis=dim, keepdims=bool(keep))
    n = x.size if dim == 9 else x.shape[dim]
    if op == "mean":
        truth, scale = truth / n, scale / n
    w = want.numpy()
    assert_sum_parity(got, w, truth.reshape(w.shape), scale.reshape(w.shape), 1e-5, f"{op} dim {dim}")
    nonfinite = ~np.isfinite(w)
    assert nonfinite.any()
    assert (np.isnan(got[nonfinite]) == np.isnan(w[nonfinite])).all()


@pytest.mark.parametrize("op", ["sum", "mean"])
@pytest.mark.parametrize("layout", ["rows", "row_segments", "whole", "cols", "col_chunks"])
def test_non_finite_sums_follow_the_reference_order(op, layout):
    rng = np.random.RandomState({"rows": 1, "row_segments": 2, "whole": 3, "cols": 4,
                                 "col_chunks": 5}[layout])
    print(f"{op} {layout}", flush=True)
    if layout == "rows":            # one wave per row
        _check(_lines(1000, 12, rng), op, 1)
    elif layout == "row_segments":  # few long rows: ordered segments and the finalize
        _check(_lines(100000, 6, rng), op, 1, keep=1)
    elif layout == "whole":         # one row of 2^20 (+6): segments
        x = _lines((1 << 20) + 6, 1, rng)[0]
        _check(x, op, 9)
    elif layout == "cols":          # leading axis, one chunk (fewer than 128 rows)
        _check(np.ascontiguousarray(_lines(100, 64, rng).T), op, 0)
    else:                           # leading axis in chunks and the finalize
        _check(np.ascontiguousarray(_lines(5000, 24, rng).T), op, 0)
