"""GPU parity of leading-axis sums over long contiguous rows of 2048 to 16384 columns (the chunked
column kernel with its ordered finalize): sum and mean over axis 0 at ragged column counts (a lane
past the row's end) and rows from 512 up, with columns whose sum overflows, meets -inf after
overflowing, or holds a NaN (summed again in the reference's index order, so they match the oracle
bit for bit). Finite sums are held to 1e-5 of sum |x| per output against the oracle's serial sum
(src/kernels/cpu/reduce_ops.c:44-64). The one-pass relu-gradient modulation and bias sum
(src/kernels/cuda/matmul_relu.cu:138-151) equals the two calls bit for bit on the same shapes, also
written over its input with a refolded column."""
from __future__ import annotations

import numpy as np
import pytest

from cases import assert_bits, assert_sum_parity
from hostlib import HostTensor, oracle_forward
from plast_amd.abi import KernelParams
from test_epilogue import epilogue_inputs, oracle_bias, oracle_modulate

pytestmark = pytest.mark.gpu

# (rows, cols): column counts that are and are not multiples of the 256-column slices of a
# workgroup (2052, 4100, 12292), rows from 512 up
SHAPES = [(512, 2048), (2000, 2052), (1024, 4096), (777, 4100), (600, 8192), (513, 16384),
          (520, 12292)]


def _x(shape, seed):
    rng = np.random.RandomState(seed)
    x = rng.randn(*shape).astype(np.float32)
    x[0:3, 1] = 3e38           # overflows to +inf in index order
    x[0:2, 2] = 3e38           # overflows, then meets -inf: NaN in index order
    x[5, 2] = -np.inf
    x[7, 3] = np.nan
    x[100:103, shape[1] - 1] = -3e38  # the last column (the ragged lane's), to -inf
    return x


@pytest.mark.parametrize("op", ["sum", "mean"])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{r}x{c}" for r, c in SHAPES])
def test_long_row_leading_axis_sum(shape, op):
    from plast_amd import ops, runtime as rt
    print(f"long-row {op} over axis 0 of {shape}", flush=True)
    x = _x(shape, sum(shape))
    dx = rt.DeviceTensor.from_numpy(x)
    got = ops.reduce(op, dx, dim=0).numpy()
    want = HostTensor(np.zeros(shape[1], np.float32))
    oracle_forward(op, [HostTensor(x)], want, KernelParams(0, 0, 0.0))
    w = want.numpy()
    with np.errstate(invalid="ignore", over="ignore"):
        fin = np.where(np.isfinite(x), x, 0.0).astype(np.float64)
        scale = np.abs(fin).sum(axis=0)
        exact = x.astype(np.float64).sum(axis=0)
    if op == "mean":
        scale, exact = scale / shape[0], exact / shape[0]
    special = ~np.isfinite(w)
    assert special[[1, 2, 3, shape[1] - 1]].all()
    assert_bits(got[special], w[special], f"{op} {shape} non-finite outputs")
    assert_sum_parity(got[~special], w[~special], exact[~special], scale[~special], 1e-5,
                      f"{op} {shape}")
    again = ops.reduce(op, dx, dim=0).numpy()
    assert_bits(again, got, f"{op} {shape} repeated")


@pytest.mark.parametrize("shape", SHAPES[:4] + SHAPES[5:6], ids=lambda s: f"{s[0]}x{s[1]}")
def test_long_row_one_pass_epilogue(shape):
    from plast_amd import runtime as rt
    M, N = shape
    alpha = 0.5
    print(f"long-row one-pass epilogue {shape}", flush=True)
    L = rt.lib()
    dout, out = epilogue_inputs(M, N, M + 7 * N)
    dout[:3, 1] = 3e38         # three 3e38 * 0.5 terms, then -inf: NaN in index order
    out[:3, 1] = -1.0
    dout[5, 1] = -np.inf
    out[5, 1] = 1.0
    D, O = rt.DeviceTensor.from_numpy(dout), rt.DeviceTensor.from_numpy(out)
    DC = rt.DeviceTensor((M, N), zero=False)
    DB = rt.DeviceTensor((N,), zero=False)
    L.launch_relu_grad_modulate_hip(D.ptr, O.ptr, DC.ptr, M * N, alpha, 0, 0)
    L.bias_grad_reduce_hip(DC.ptr, DB.ptr, M * N, N)
    L.check("two calls")
    wdc, wdb = DC.numpy(), DB.numpy()
    assert np.isnan(wdb[1])
    dc = oracle_modulate(dout, out, alpha)
    assert_bits(wdc, dc, "dc vs oracle")
    ob = oracle_bias(dc, N)
    special = ~np.isfinite(ob)
    assert_bits(wdb[special], ob[special], "dbias non-finite vs oracle")
    assert_sum_parity(wdb[~special], ob[~special], dc.astype(np.float64).sum(0)[~special],
                      np.abs(np.where(np.isfinite(dc), dc, 0)).astype(np.float64).sum(0)[~special],
                      1e-5, "dbias vs oracle")
    for in_place in (False, True):
        D2 = rt.DeviceTensor.from_numpy(dout)
        DC2 = D2 if in_place else rt.DeviceTensor((M, N), zero=False)
        DB2 = rt.DeviceTensor((N,), zero=False)
        L.relu_grad_modulate_bias_grad_hip(D2.ptr, O.ptr, DC2.ptr, DB2.ptr, M * N, N, alpha)
        L.check("one pass")
        assert_bits(DC2.numpy(), wdc, f"dc, one pass (in place: {in_place})")
        assert_bits(DB2.numpy(), wdb, f"dbias, one pass vs two calls (in place: {in_place})")
