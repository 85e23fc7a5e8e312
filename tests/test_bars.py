"""The parity bars themselves, on the CPU: the cross-entropy row check (`cases.check_ce_rows`) and
the broadcast-gradient bar of `test_gpu_parity` accept the oracle's own outputs and reject planted
mistakes of the sizes they are meant to catch."""
from __future__ import annotations

import numpy as np
import pytest

from cases import CASES, check_ce_rows, run_case
from hostlib import HostBackend, HostTensor, oracle_backward, oracle_forward


def _ce_oracle(x, lab, g):
    N, Cn = x.shape
    hx = HostTensor(x, requires_grad=True)
    hl = HostTensor(lab)
    hs = HostTensor(np.zeros((N, 2), np.float32))
    ho = HostTensor(np.zeros(N, np.float32), requires_grad=True)
    oracle_forward("softmax_cross_entropy", [hx, hl, hs], ho)
    ho.grad.buf[:] = g
    oracle_backward("softmax_cross_entropy", [hx, hl, hs], ho)
    return hs.numpy(), ho.numpy(), hx.grad.numpy()


@pytest.fixture(scope="module")
def ce_case():
    rng = np.random.RandomState(3)
    N, Cn = 300, 2000
    x = (rng.randn(N, Cn) * 2).astype(np.float32)
    lab = rng.randint(0, Cn, N).astype(np.int32)
    x[5, :] = -3.0e38                     # an overflowing row
    x[5, 0] = 3.0e38
    g = np.full(N, np.float32(1.0 / N), np.float32)
    return x, lab, g, _ce_oracle(x, lab, g)


def test_ce_rows_accept_the_oracle(ce_case):
    x, lab, g, (st, loss, dx) = ce_case
    check_ce_rows(x, lab, g, st, loss, dx, st, loss, dx, 1e-2 / x.shape[0])


@pytest.mark.parametrize("what", ["lse", "loss", "dlogit", "label_dlogit", "max"])
def test_ce_rows_reject_a_planted_mistake(ce_case, what):
    x, lab, g, (st, loss, dx) = ce_case
    st2, loss2, dx2 = st.copy(), loss.copy(), dx.copy()
    r = 17
    if what == "lse":
        st2[r, 1] += np.float32(3e-5)               # the exp-sum off by 3e-5 relative
    elif what == "loss":
        loss2[r] += np.float32(3e-5) * (abs(loss2[r]) + 1)
    elif what == "dlogit":
        c = int(np.argmax(np.where(np.arange(x.shape[1]) == lab[r], 0, np.abs(dx2[r]))))
        dx2[r, c] *= np.float32(1 + 5e-5)         # the row's largest non-label gradient
    elif what == "label_dlogit":
        dx2[r, lab[r]] = np.float32(dx2[r, lab[r]] + g[r])   # the one-hot term dropped
    else:
        st2[r, 0] = np.nextafter(st2[r, 0], np.float32(np.inf))
    with pytest.raises(AssertionError):
        check_ce_rows(x, lab, g, st2, loss2, dx2, st, loss, dx, 1e-2 / x.shape[0])


def test_ce_rows_accept_the_exact_value_where_the_oracle_drifts(ce_case):
    """A row statistic equal to the fp64 value passes even where the oracle's serial fp32 sum is
    further than the bar from it (here the oracle's value is moved off by 2e-5 to stand for that
    drift)."""
    x, lab, g, (st, loss, dx) = ce_case
    r = 40
    m = st[r, 0].astype(np.float64)
    l64 = np.log(np.exp(x[r].astype(np.float64) - m).sum())
    ref = st.copy()
    ref[r, 1] = np.float32(l64 + 2e-5)
    gpu = st.copy()
    gpu[r, 1] = np.float32(l64)
    xy = np.float64(x[r, lab[r]])
    ref_loss, gpu_loss = loss.copy(), loss.copy()
    ref_loss[r] = np.float32(l64 + 2e-5 - (xy - m))
    gpu_loss[r] = np.float32(l64 - (xy - m))
    check_ce_rows(x, lab, g, gpu, gpu_loss, dx, ref, ref_loss, dx, 1e-2 / x.shape[0])


def _bcast_grad_cases():
    return [c for c in CASES if not c.exact and c.kind == "bwd"][:12]


def _max_to(x, shape):
    """x's maximum over the axes that broadcasting added or stretched to reach it from `shape`."""
    while x.ndim > len(shape):
        x = x.max(axis=0)
    for ax, n in enumerate(shape):
        if n == 1 and x.shape[ax] != 1:
            x = x.max(axis=ax, keepdims=True)
    return x


@pytest.mark.parametrize("c", _bcast_grad_cases(), ids=lambda c: c.id)
def test_broadcast_gradient_bar(c):
    """The oracle's broadcast gradients sit within the bar of the fp64 sum of their fp32 terms, and
    the bar is tighter than the largest term behind each element: a gradient that drops that term
    (or flips its sign) falls outside it."""
    import test_gpu_parity as P
    from cases import materialize
    want = run_case(HostBackend("oracle"), c)
    host = HostBackend("oracle")
    vals = [materialize(host, a)[0].numpy() for a in c.inputs]
    d = np.random.RandomState(c.dout_seed).randn(*c.out_shape).astype(np.float32)
    a, b = (np.broadcast_to(v, c.out_shape) for v in vals)
    for k in [k for k in want if k.startswith("grad")]:
        kk = int(k[4:])
        w = want[k]
        exact, scale = P._grad_terms(c, kk, w)
        fin = np.isfinite(w) & np.isfinite(scale)
        if exact is not None:
            assert np.all(np.abs(w[fin] - exact[fin]) <= 1e-5 * scale[fin])
        with np.errstate(all="ignore"):
            terms = [np.abs(f(d, a, b).astype(np.float64)) for f in P._TERMS[c.op]]
            big = np.maximum(terms[0], terms[1]) if c.same_input else terms[kk]
            tmax = P._grad_layout(_max_to(big, vals[kk].shape), c.inputs[kk], w.shape)
        sel = fin & np.isfinite(tmax) & (tmax > 0)
        assert np.all(tmax[sel] > 1e-5 * scale[sel]), f"{c.id}:{k}: a dropped term would pass"
