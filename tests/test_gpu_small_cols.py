"""GPU parity of small leading-axis sums, which run in one launch (red_cols_small_kernel: narrow
column slices that walk every row, no finalize): sum and mean over axis 0 and a middle axis, with
partial column slices (inner 20), several outer indices, exactly 128 rows (the shortest axis that
is split), and columns whose sum overflows, meets -inf after overflowing, or holds a NaN (those are
summed again in the reference's index order, so they match the oracle bit for bit). Finite sums are
held to 1e-5 of sum |x| per output against the oracle's serial sum (src/kernels/cpu/
reduce_ops.c:44-64). Config 1's bias gradient through ADD's backward ([1024, 256] into [256],
kernel_macros.h:283-299) and the same sum repeated are deterministic."""
from __future__ import annotations

import numpy as np
import pytest

from cases import assert_bits, assert_sum_parity
from hostlib import HostTensor, oracle_backward, oracle_forward
from plast_amd.abi import KernelParams

pytestmark = pytest.mark.gpu

SHAPES = [((1024, 256), 0), ((300, 20), 0), ((128, 64), 0), ((3, 200, 64), 1), ((2, 4096, 16), 1),
          ((1000, 1000), 0)]


def _x(shape, axis, seed):
    rng = np.random.RandomState(seed)
    x = rng.randn(*shape).astype(np.float32)

    def at(rows, col):  # rows of the reduced axis, one column of the last axis, other axes 0
        return tuple(rows if d == axis else (col if d == len(shape) - 1 else 0)
                     for d in range(len(shape)))

    if shape[-1] >= 4:
        x[at(slice(0, 3), 1)] = 3e38          # overflows to +inf in index order
        x[at(slice(0, 2), 2)] = 3e38          # overflows, then meets -inf: NaN in index order
        x[at(5, 2)] = -np.inf
        x[at(7, 3)] = np.nan
    return x


@pytest.mark.parametrize("op", ["sum", "mean"])
@pytest.mark.parametrize("shape, axis", SHAPES, ids=[f"{s}-ax{a}" for s, a in SHAPES])
def test_small_leading_axis_sum(shape, axis, op):
    from plast_amd import ops, runtime as rt
    print(f"small {op} over axis {axis} of {shape}", flush=True)
    x = _x(shape, axis, sum(shape) + axis)
    dx = rt.DeviceTensor.from_numpy(x)
    got = ops.reduce(op, dx, dim=axis).numpy()
    out_shape = tuple(s for d, s in enumerate(shape) if d != axis)
    want = HostTensor(np.zeros(out_shape, np.float32))
    oracle_forward(op, [HostTensor(x)], want, KernelParams(axis, 0, 0.0))
    w = want.numpy()
    with np.errstate(invalid="ignore", over="ignore"):
        fin = np.where(np.isfinite(x), x, 0.0).astype(np.float64)
        scale = np.abs(fin).sum(axis=axis)
        exact = x.astype(np.float64).sum(axis=axis)
    if op == "mean":
        scale, exact = scale / shape[axis], exact / shape[axis]
    special = ~np.isfinite(w)
    assert_bits(got[special], w[special], f"{op} {shape} non-finite outputs")
    assert_sum_parity(got[~special], w[~special], exact[~special], scale[~special], 1e-5,
                      f"{op} {shape}")
    again = ops.reduce(op, dx, dim=axis).numpy()
    assert_bits(again, got, f"{op} {shape} repeated")


def test_config1_bias_gradient_through_add_backward():
    from plast_amd import runtime as rt
    print("config 1 bias gradient through ADD backward", flush=True)
    rng = np.random.RandomState(3)
    x = rng.uniform(-1, 1, (1024, 256)).astype(np.float32)
    b = rng.uniform(-1, 1, 256).astype(np.float32)
    gy = rng.uniform(-1, 1, (1024, 256)).astype(np.float32)
    X, B = rt.DeviceTensor.from_numpy(x, True), rt.DeviceTensor.from_numpy(b, True)
    Y = rt.DeviceTensor((1024, 256), requires_grad=True, zero=False)
    rt.forward("add", [X, B], Y)
    rt.lib().arena_memcpy_h2d_hip(Y.grad.ptr, gy.ctypes.data, gy.nbytes)
    rt.backward("add", [X, B], Y)
    db = B.grad.numpy()
    hx, hb = HostTensor(x, requires_grad=True), HostTensor(b, requires_grad=True)
    hy = HostTensor(np.zeros_like(x), requires_grad=True)
    oracle_forward("add", [hx, hb], hy)
    hy.grad.buf[:] = gy.reshape(-1)
    oracle_backward("add", [hx, hb], hy)
    assert_sum_parity(db, hb.grad.numpy(), gy.astype(np.float64).sum(0),
                      np.abs(gy).astype(np.float64).sum(0), 1e-5, "db")
    assert_bits(X.grad.numpy(), hx.grad.numpy(), "dX")
