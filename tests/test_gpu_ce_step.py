"""GPU parity of the one-pass cross-entropy step (softmax_cross_entropy_step_hip): the forward's row
statistics and loss, the backward's dlogits = dloss * (softmax - onehot) and the bias gradient
sum_rows dlogits, from one read of the logits. Checked against the oracle (the reference chain of
src/api/loss.c:97-169 and its backward, bit-exact against the compiled reference on the CPU) at the
stated tolerances:
  row max: bit-exact; log-sum-exp and loss: 1e-5 relative (the exp-sum's order differs);
  dlogits: 1e-5 of |value| + 1e-2 / N; dbias: 1e-5 of sum_rows |dlogits|.
Rows hold NaN, -inf, zero maxima, signed zeros and huge spreads (the exact-refold path), labels
sit in the SIMD tail of the loss's NEG rule, and shapes cover every register layout, rows that are
not whole float4 (the three-pass path) and config 5's full [32768, 32000] (size-independent
properties there: rows of dlogits sum to 0, the bias gradient's total mass is 0, the max matches)."""
from __future__ import annotations

import numpy as np
import pytest

from cases import assert_bits, assert_close_sum
from hostlib import HostTensor, oracle_backward, oracle_forward
from plast_amd.abi import KernelParams

pytestmark = pytest.mark.gpu


def _step(rt, X, lab, g, with_bias=True):
    N, Cn = X.shape
    st = rt.DeviceTensor((N, 2), zero=False)
    loss = rt.DeviceTensor((N,), zero=False)
    dx = rt.DeviceTensor((N, Cn), zero=False).fill_("uniform", 3, 5.0, 6.0)  # overwritten
    db = rt.DeviceTensor((Cn,), zero=False).fill_("uniform", 4, 5.0, 6.0) if with_bias else None
    G = rt.DeviceTensor.from_numpy(g)
    L = rt.lib()
    L.softmax_cross_entropy_step_hip(X.ptr, lab.ptr, G.ptr, st.ptr, loss.ptr, dx.ptr,
                                     db.ptr if db is not None else None, N, Cn)
    L.check("ce step")
    return st.numpy(), loss.numpy(), dx.numpy(), db.numpy() if db is not None else None


def _oracle(x, lab, g):
    N, Cn = x.shape
    hx = HostTensor(x, requires_grad=True)
    hl = HostTensor(lab)
    hs = HostTensor(np.zeros((N, 2), np.float32))
    ho = HostTensor(np.zeros(N, np.float32), requires_grad=True)
    oracle_forward("softmax_cross_entropy", [hx, hl, hs], ho)
    ho.grad.buf[:] = g
    oracle_backward("softmax_cross_entropy", [hx, hl, hs], ho)
    return hs.numpy(), ho.numpy(), hx.grad.numpy()


def _special_rows(x):
    N = x.shape[0]
    if N >= 8:
        x[1, 3] = np.nan           # NaN row: loss NaN (reference chain)
        x[2, :] = 0.0              # zero maximum
        x[2, 1] = -0.0
        x[3, 0] = -np.inf          # 0 * -inf in the one-hot product gives NaN
        x[4, :] = -3.0e38          # huge negative row
        x[4, 0] = 3.0e38           # x - max overflows to -inf
        x[5, :] = -np.inf          # every logit -inf


@pytest.mark.parametrize("special", [False, True], ids=["clean", "special_rows"])
@pytest.mark.parametrize("N, Cn", [(13, 4), (64, 2048), (37, 8192), (40, 12000), (33, 32000),
                                   (9, 65536), (17, 1001), (8, 6)])
def test_step_matches_oracle(N, Cn, special):
    """With special rows every column of the bias gradient is NaN (a NaN row reaches all of them),
    so its values are compared on the clean inputs."""
    from plast_amd import runtime as rt
    print(f"ce step {N}x{Cn} {'special' if special else 'clean'}", flush=True)
    rng = np.random.RandomState(N * 7 + Cn)
    x = (rng.randn(N, Cn) * 2).astype(np.float32)
    lab = rng.randint(0, Cn, N).astype(np.int32)
    if special:
        _special_rows(x)
    g = np.full(N, np.float32(1.0) / np.float32(N), np.float32)
    g[-1] = 0.5                    # the upstream gradient is per row
    X, Lb = rt.DeviceTensor.from_numpy(x), rt.DeviceTensor.from_numpy(lab)
    st, loss, dx, db = _step(rt, X, Lb, g)
    wst, wloss, wdx = _oracle(x, lab, g)
    assert_bits(st[:, 0], wst[:, 0], "row max")
    assert_close_sum(st[:, 1], wst[:, 1], np.abs(wst[:, 1]) + 1e-6, 1e-5, "row log-sum-exp")
    assert_close_sum(loss, wloss, np.abs(wloss) + np.abs(wst[:, 1]) + 1e-6, 1e-5, "row loss")
    finite = np.isfinite(wdx).all(1)
    assert_close_sum(dx[finite], wdx[finite], np.abs(wdx[finite]) + 1e-2 / N, 1e-5, "dlogits")
    assert_bits(np.isnan(dx), np.isnan(wdx), "NaN positions of dlogits")
    # the bias gradient against the column sums of the oracle's dlogits (float64)
    want = wdx.astype(np.float64).sum(0)
    ok = np.isfinite(want)
    assert_close_sum(db[ok], want[ok], np.abs(wdx.astype(np.float64)).sum(0)[ok] + 1e-12, 1e-5,
                     "dbias")
    assert_bits(np.isnan(db), np.isnan(want), "NaN columns of dbias")
    # without a bias gradient the other outputs are the same bits
    st2, loss2, dx2, _ = _step(rt, X, Lb, g, with_bias=False)
    assert_bits(loss2, loss, "loss without bias")
    assert_bits(dx2, dx, "dlogits without bias")


def test_step_is_deterministic_and_matches_the_op_path():
    """Two steps give identical bits; against the op path (forward op, overwriting backward op,
    then the column sum) the row max is bit-equal and the rest within the bars above."""
    from plast_amd import ops, runtime as rt
    N, Cn = 512, 32000
    print(f"ce step vs op path {N}x{Cn}", flush=True)
    X = rt.DeviceTensor((N, Cn), requires_grad=True, zero=False).fill_("normal", 42, 0.0, 2.0)
    from plast_amd.abi import INT32
    Lb = rt.DeviceTensor((N,), INT32, zero=False).fill_("randint", 45, 0, Cn)
    g = np.full(N, np.float32(1.0) / np.float32(N), np.float32)
    a = _step(rt, X, Lb, g)
    b = _step(rt, X, Lb, g)
    for u, v, what in zip(a, b, ("stats", "loss", "dlogits", "dbias")):
        assert_bits(u, v, f"repeat: {what}")
    loss, stats = ops.softmax_cross_entropy(X, Lb, requires_grad=True)
    rt.lib().arena_memcpy_h2d_hip(loss.grad.ptr, g.ctypes.data, g.nbytes)
    rt.backward("softmax_cross_entropy", [X, Lb, stats], loss, KernelParams(0, 1, 0.0))
    bias = ops.reduce("sum", X.grad, dim=0).numpy()
    st, lo, dx, db = a
    assert_bits(st[:, 0], stats.numpy()[:, 0], "row max vs op path")
    assert_close_sum(lo, loss.numpy(), np.abs(loss.numpy()) + 1e-6, 1e-5, "loss vs op path")
    gx = X.grad.numpy()
    assert_close_sum(dx, gx, np.abs(gx) + 1e-2 / N, 1e-5, "dlogits vs op path")
    assert_close_sum(db, bias, np.abs(gx).sum(0) + 1e-12, 1e-5, "dbias vs op path")


def test_step_full_size_properties():
    """Config 5 at [32768, 32000]: logits ~ N(0, 2), labels uniform. Sampled rows against a float64
    log-sum-exp; every dlogits row sums to 0 (to 1e-5 / N per row); the bias gradient's total is 0;
    the row max equals numpy's max."""
    from plast_amd import runtime as rt
    from plast_amd.abi import INT32
    N, Cn = 32768, 32000
    print("ce step full size", flush=True)
    X = rt.DeviceTensor((N, Cn), zero=False).fill_("normal", 42, 0.0, 2.0)
    Lb = rt.DeviceTensor((N,), INT32, zero=False).fill_("randint", 45, 0, Cn)
    g = np.full(N, np.float32(1.0) / np.float32(N), np.float32)
    st, loss, dx, db = _step(rt, X, Lb, g)
    xh, yl = X.numpy(), Lb.numpy()
    for r in np.random.RandomState(3).choice(N, 16, replace=False):
        row = xh[r].astype(np.float64)
        lse = np.log(np.exp(row - row.max()).sum()) + row.max()
        assert abs(loss[r] - (lse - row[yl[r]])) <= 1e-5 * (abs(lse) + abs(row[yl[r]]))
        assert st[r, 0] == xh[r].max()
    assert np.abs(dx.astype(np.float64).sum(1)).max() <= 1e-5 / N * 10
    assert abs(db.astype(np.float64).sum()) <= 1e-4
    assert_close_sum(db, dx.astype(np.float64).sum(0), np.abs(dx).astype(np.float64).sum(0) + 1e-12,
                     1e-5, "dbias = column sums of dlogits")
