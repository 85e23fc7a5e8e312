"""GPU parity of softmax / log-softmax over the last axis (softmax_hip_* / log_softmax_hip_*).

Forward: against the reference's own op chain run through the oracle (plast/nn/functional.py:75-97:
MAX(dim, keepdim) -> SUB -> EXP -> SUM(dim, keepdim) -> DIV, or -> LOG -> SUB). The max is
bit-exact; the only other difference is the row sum's order. The GPU's sum is held to 1e-5
relative of the exact (float64) sum and the oracle's serial fp32 sum over a long row carries an
error e_row of its own, so softmax must be within (2e-5 + 2 e_row) * |y| (plus expf's 2 ulp) and
log-softmax within 1e-5 + 2 e_row + 4e-7 * |y| (log s moves by the sum's relative error); NaN
against NaN.
Backward: against the closed form in float64 from the same y, x.grad += y * (dy - sum(dy * y)) or
dy - exp(y) * sum(dy), within 1e-5 of the terms' magnitude per element, accumulated into an
existing gradient."""
from __future__ import annotations

import numpy as np
import pytest

from hostlib import HostTensor, oracle_forward
from plast_amd.abi import KernelParams

pytestmark = pytest.mark.gpu

# (600, 2052), (600, 2048) and (300, 8192) give the persistent forward more rows than workgroups
# (with special rows in later iterations), the first with a partial last float4 unit per lane
SHAPES = [(4, 10), (33, 1000), (8, 32000), (2, 3, 257), (1, 1), (5, 4096), (6, 9), (600, 2052),
          (600, 2048), (300, 8192),
          # from a wider seeded sweep: 1200 rows of 32000 (four or five per workgroup, the late
          # special rows in both register sets), rows of 5000 over three leading axes, and rows
          # that are not whole float4 (1023) or one workgroup's width (1024)
          (2, 600, 32000), (3, 100, 5000), (300, 1023), (2, 300, 1024)]


def _put_specials(rows, r0):
    rows[r0 + 0, 1] = np.nan                      # NaN row
    rows[r0 + 1, :] = -np.inf                     # max is -FLT_MAX: every term 0, y NaN
    rows[r0 + 2, 2] = np.inf                      # inf - inf
    rows[r0 + 3, :2] = [3e38, -3e38]              # extreme spread: terms underflow
    rows[r0 + 4, :] = 0.0                         # ties at zero, both signs
    rows[r0 + 4, ::2] = -0.0
    rows[r0 + 5, 0] = 1e-40                       # subnormal


# The persistent forward runs one workgroup per CU (256 on MI355X) and holds two rows in turn
# (iteration k of workgroup b is row k*256 + b, in the first register set when k is even): special
# rows also sit in the second and third iterations, where the next row's loads are in flight.
LATE_SPECIALS = (256 + 6, 512 + 8)


def _x(shape, seed):
    rng = np.random.RandomState(seed)
    x = (rng.randn(*shape) * 3).astype(np.float32)
    rows = x.reshape(-1, shape[-1])
    if rows.shape[0] >= 6 and rows.shape[1] >= 4:
        _put_specials(rows, 0)
        for r0 in LATE_SPECIALS:
            if r0 + 6 <= rows.shape[0]:
                _put_specials(rows, r0)
    return x


def _oracle(x, log):
    C = x.shape[-1]
    rows = x.reshape(-1, C)
    R = rows.shape[0]

    def t(a):
        return HostTensor(np.ascontiguousarray(a, np.float32))

    m = t(np.zeros((R, 1)))
    oracle_forward("max", [t(rows)], m, KernelParams(1, 1, 0.0))
    sh = t(np.zeros((R, C)))
    oracle_forward("sub", [t(rows), m], sh)
    e = t(np.zeros((R, C)))
    oracle_forward("exp", [sh], e)
    s = t(np.zeros((R, 1)))
    oracle_forward("sum", [e], s, KernelParams(1, 1, 0.0))
    y = t(np.zeros((R, C)))
    if log:
        ls = t(np.zeros((R, 1)))
        oracle_forward("log", [s], ls)
        oracle_forward("sub", [sh, ls], y)
    else:
        oracle_forward("div", [e, s], y)
    # the oracle's serial sum against the exact sum of its own terms, per row
    with np.errstate(invalid="ignore", divide="ignore"):
        exact = e.numpy().astype(np.float64).sum(1, keepdims=True)
        err = np.abs(s.numpy().astype(np.float64) - exact) / exact
    err = np.where(np.isfinite(err), err, 0.0)
    lead = x.shape[:-1] + (1,)
    return y.numpy().reshape(x.shape), err.reshape(lead)


def _close(got, want, tol, what):
    both_nan = np.isnan(got) & np.isnan(want)
    same = (got == want) | both_nan
    with np.errstate(invalid="ignore"):
        ok = same | (np.abs(got.astype(np.float64) - want) <= tol)
    if not ok.all():
        i = tuple(np.argwhere(~ok)[0])
        raise AssertionError(f"{what}: {int((~ok).sum())} of {ok.size} off; first at {i}: "
                             f"gpu {got[i]!r} want {want[i]!r} tol {np.broadcast_to(tol, got.shape)[i]!r}")


@pytest.mark.parametrize("log", [False, True], ids=["softmax", "log_softmax"])
@pytest.mark.parametrize("shape", SHAPES, ids=[str(s) for s in SHAPES])
def test_softmax_forward_and_backward(shape, log):
    from plast_amd import runtime as rt
    name = "log_softmax" if log else "softmax"
    print(f"{name} {shape}", flush=True)
    x = _x(shape, len(shape) * 100 + shape[-1])
    dx = rt.DeviceTensor.from_numpy(x, requires_grad=True)
    y = rt.DeviceTensor(shape, requires_grad=True, zero=False)
    p = KernelParams(len(shape) - 1, 0, 0.0)
    rt.forward(name, [dx], y, p)
    got = y.numpy()
    want, e_row = _oracle(x, log)
    with np.errstate(invalid="ignore", over="ignore"):
        tol = ((1e-5 + 2 * e_row + 4e-7 * np.abs(want)) if log else
               ((2e-5 + 2 * e_row) * np.abs(want) + 1e-37))
    _close(got, want, tol, f"{name} forward")

    rng = np.random.RandomState(5)
    dy = rng.randn(*shape).astype(np.float32)
    prev = rng.randn(*shape).astype(np.float32)
    L = rt.lib()
    L.arena_memcpy_h2d_hip(y.grad.ptr, dy.ctypes.data, dy.nbytes)
    L.arena_memcpy_h2d_hip(dx.grad.ptr, prev.ctypes.data, prev.nbytes)
    rt.backward(name, [dx], y, p)
    g = dx.grad.numpy()
    y64, dy64 = got.astype(np.float64), dy.astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        if log:
            ey = np.exp(y64)
            term = dy64 - ey * dy64.sum(-1, keepdims=True)
            scale = np.abs(dy64) + ey * np.abs(dy64).sum(-1, keepdims=True)
        else:
            term = y64 * (dy64 - (dy64 * y64).sum(-1, keepdims=True))
            scale = np.abs(y64) * (np.abs(dy64) + np.abs(dy64 * y64).sum(-1, keepdims=True))
        want_g = prev.astype(np.float64) + term
        tol_g = 1e-5 * scale + 2.4e-7 * np.abs(want_g) + 1e-30
    _close(g, want_g, tol_g, f"{name} backward")


def test_softmax_rejects_other_axes():
    from plast_amd import runtime as rt
    x = rt.DeviceTensor.from_numpy(np.ones((3, 4), np.float32))
    y = rt.DeviceTensor((3, 4), zero=False)
    with pytest.raises(rt.PlastHipError, match="last axis"):
        rt.forward("softmax", [x], y, KernelParams(0, 0, 0.0))


def test_softmax_full_size_properties():
    """The persistent forward at the benchmarked [32768, 32000], through size-independent
    properties checked on the device with the library's own pinned reductions: every softmax row
    sums to 1, every exp(log-softmax) row sums to 1 (within 32000 terms' fp32 rounding plus the
    exponential's error), and each row's argmax is the argmax of its logits (softmax is monotonic;
    ties are vanishingly unlikely for N(0, 2) logits)."""
    from plast_amd import ops, runtime as rt
    print("softmax at [32768, 32000]", flush=True)
    N, Cn = 32768, 32000
    x = rt.DeviceTensor((N, Cn), zero=False).fill_("normal", 21, 0.0, 2.0)
    y = rt.DeviceTensor((N, Cn), zero=False)
    try:
        rt.forward("softmax", [x], y, KernelParams(1, 0, 0.0))
        s = ops.reduce("sum", y, dim=1).numpy()
        assert np.all(np.abs(s.astype(np.float64) - 1.0) <= 2e-4), f"row sums {s.min()}..{s.max()}"
        ax, ay = ops.reduce("argmax", x, dim=1).numpy(), ops.reduce("argmax", y, dim=1).numpy()
        assert np.array_equal(ax, ay), f"{int((ax != ay).sum())} rows change their argmax"
        rt.forward("log_softmax", [x], y, KernelParams(1, 0, 0.0))
        e = rt.DeviceTensor((N, Cn), zero=False)
        rt.forward("exp", [y], e)
        s = ops.reduce("sum", e, dim=1).numpy()
        e.free()
        assert np.all(np.abs(s.astype(np.float64) - 1.0) <= 2e-4), f"exp row sums {s.min()}..{s.max()}"
    finally:
        x.free()
        y.free()
