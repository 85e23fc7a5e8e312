"""GPU parity: every case of tests/cases.py through the HIP library versus the oracle on the same
seeded inputs.

Bars (the path's stated tolerances):
  add/sub/mul/div/neg/abs/relu/max/min/argmax, index math, every backward without a reduction:
      bit-exact (NaN matches NaN);
  exp/log (and sin/cos/tan): within 2 ulp of glibc;
  sum/mean and broadcast-gradient reductions: |gpu - oracle| <= 1e-5 * sum|x| over the reduced set.
"""
from __future__ import annotations

import numpy as np
import pytest

from cases import CASES, assert_bits, assert_close_sum, assert_sum_parity, materialize, run_case
from hostlib import HostBackend

pytestmark = pytest.mark.gpu

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
        elif not c.exact:
            assert_close_sum(g, w, np.abs(w).astype(np.float64) + 1.0, 1e-5, what)
        else:
            assert_bits(g, w, what)
