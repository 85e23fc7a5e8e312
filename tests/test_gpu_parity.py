"""GPU parity: every case of tests/cases.py through the HIP library versus the oracle on the same
seeded inputs.

Bars (the path's stated tolerances):
  add/sub/mul/div/neg/abs/relu/max/min/argmax, index math, every backward without a reduction:
      bit-exact (NaN matches NaN);
  exp/log (and sin/cos/tan): within 2 ulp of glibc;
  sum/mean reductions: |gpu - oracle| <= 1e-5 * sum|x| over the reduced set;
  broadcast-gradient reductions: |gpu - oracle| <= 1e-5 * (sum of |dout * d out / d input| over the
      positions summed into the element + |value|); where the oracle's serial order overflowed and
      the exact (fp64) sum is a float, within that bar of the exact sum; other non-finite values
      exactly.
"""
from __future__ import annotations

import numpy as np
import pytest

from cases import (CASES, assert_bits, assert_close_sum, assert_sum_parity, grad_init_values,
                   materialize, run_case)
from hostlib import HostBackend

pytestmark = pytest.mark.gpu

FLT_MAX = float(np.finfo(np.float32).max)
TRANSCENDENTAL = {"exp", "log", "sin", "cos", "tan"}


def _reduced_abs(c, x):
    dim, keep, _ = c.params
    ax = np.abs(x.astype(np.float64))
    if dim == 9:
        return np.array([ax.sum()])
    r = ax.sum(axis=dim, keepdims=bool(keep))
    return r if r.ndim else r.reshape(1)


def _reduced_sum(c, x):
    dim, keep, _ = c.params
    x64 = x.astype(np.float64)
    if dim == 9:
        return np.array([x64.sum()])
    r = x64.sum(axis=dim, keepdims=bool(keep))
    return r if r.ndim else r.reshape(1)


# each input's gradient term dout * d out / d input of the binary ops, in fp32 and in the oracle's
# operation order (binary_ops.c:18-57), from the operands broadcast to the output's shape
_TERMS = {
    "add": (lambda g, x, y: g, lambda g, x, y: g),
    "sub": (lambda g, x, y: g, lambda g, x, y: -g),
    "mul": (lambda g, x, y: g * y, lambda g, x, y: g * x),
    "div": (lambda g, x, y: g / y, lambda g, x, y: (-g * x) / (y * y)),
}


def _sum_to(x, shape):
    """x summed over the axes that broadcasting added or stretched to reach it from `shape`."""
    while x.ndim > len(shape):
        x = x.sum(axis=0)
    for ax, n in enumerate(shape):
        if n == 1 and x.shape[ax] != 1:
            x = x.sum(axis=ax, keepdims=True)
    return x


def _grad_layout(v, a, shape):
    """v, in the view's element order, as the gradient buffer read back holds it: a transposed view
    with a gradient of its own is written through the view's data strides (the reference's
    indexing, kernel_macros.h:314-317) into a buffer that reads back contiguously."""
    if not (a.transpose and a.own_grad):
        return v.reshape(shape)
    base = a.base_array()
    st = list(np.array(base.strides) // base.itemsize)
    d0, d1 = a.transpose
    st[d0], st[d1] = st[d1], st[d0]
    idx = np.zeros(a.view_shape, np.int64)
    for ax, stride in enumerate(st):
        sh = [1] * len(st)
        sh[ax] = a.view_shape[ax]
        idx = idx + (np.arange(a.view_shape[ax]) * stride).reshape(sh)
    out = np.zeros(int(np.prod(shape)), v.dtype)
    out[idx.reshape(-1)] = v.reshape(-1)
    return out.reshape(shape)


def _grad_terms(c, k, w):
    """A broadcast gradient's exact value and the scale of its 1e-5 bar, per element, in fp64: the
    sum of the fp32 terms dout * d out / d input k over every output position that broadcasts onto
    it (both
    operands' terms when one tensor is both) plus the gradient the buffer held before, and the sum
    of those terms' magnitudes plus |value|. A bar relative to the value alone asks a cancelling
    sum of thousands of terms for more than any summation order gives (the oracle's serial sum
    included). The exact value is None where the buffer held values in a view's layout."""
    host = HostBackend("oracle")
    vals = [materialize(host, a)[0].numpy() for a in c.inputs]
    d = np.random.RandomState(c.dout_seed).randn(*c.out_shape).astype(np.float32)
    a, b = (np.broadcast_to(v, c.out_shape) for v in vals)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore", under="ignore"):
        parts = [f(d, a, b).astype(np.float64) for f in _TERMS[c.op]]
        own = parts[0] + parts[1] if c.same_input else parts[k]
        mag = np.abs(parts[0]) + np.abs(parts[1]) if c.same_input else np.abs(parts[k])
        exact = _grad_layout(_sum_to(own, vals[k].shape), c.inputs[k], w.shape)
        scale = _grad_layout(_sum_to(mag, vals[k].shape), c.inputs[k], w.shape) + \
            np.abs(w).astype(np.float64)
    if c.grad_init is not None:
        if c.inputs[k].transpose:
            return None, scale
        exact = exact + grad_init_values(c, k, w.size).astype(np.float64).reshape(w.shape)
    return exact, scale


@pytest.mark.parametrize("c", CASES, ids=[c.id for c in CASES])
def test_case(c):
    check_case(c)


def check_case(c):
    """One case through the HIP library and the oracle, compared at the bars above."""
    from gpu_backend import DeviceBackend, ulp_distance

    print(f"case {c.id}", flush=True)
    got = run_case(DeviceBackend(), c)
    want = run_case(HostBackend("oracle"), c)
    assert set(got) == set(want)
    for k in want:
        g, w = got[k], want[k]
        assert g.shape == w.shape, f"{c.id}:{k} shape {g.shape} vs {w.shape}"
        what = f"{c.id}:{k}"
        if c.op in ("sum", "mean") and k == "out":
            x = materialize(HostBackend("oracle"), c.inputs[0])[0].numpy()
            scale = _reduced_abs(c, x)
            truth = _reduced_sum(c, x)
            if c.op == "mean":
                n = x.size if c.params[0] == 9 else x.shape[c.params[0]]
                scale = scale / max(n, 1)
                truth = truth / max(n, 1)
            assert_sum_parity(g, w, truth.reshape(w.shape), scale.reshape(w.shape), 1e-5, what)
        elif c.op in TRANSCENDENTAL and k == "out":
            d = ulp_distance(g, w)
            assert d.max() <= 2, f"{what}: max ulp {d.max()} at {np.unravel_index(d.argmax(), d.shape)}"
        elif c.op in TRANSCENDENTAL:
            # gradient = da + dout * f'(a): f' within 2 ulp, then one product and one sum
            assert_close_sum(g, w, np.abs(w).astype(np.float64) + 1e-30, 2e-6, what)
        elif not c.exact and k.startswith("grad"):
            exact, scale = _grad_terms(c, int(k[4:]), w)
            # a value the oracle's serial order overflowed where the exact sum did not is held to
            # that sum (the reference adds these terms with omp atomics, in no fixed order)
            rescue = np.zeros(w.shape, bool)
            if exact is not None:
                rescue = ~np.isfinite(w) & np.isfinite(exact) & (np.abs(exact) <= FLT_MAX)
                assert_close_sum(g[rescue], exact[rescue], scale[rescue], 1e-5,
                                 what + " (the oracle's order overflowed)")
            # other non-finite values match exactly (an infinite scale would accept anything)
            nf = (~np.isfinite(w) | ~np.isfinite(g)) & ~rescue
            assert_bits(g[nf], w[nf], what + " non-finite")
            fin = ~nf & ~rescue
            assert_close_sum(g[fin], w[fin], scale[fin], 1e-5, what)
        else:
            assert_bits(g, w, what)
