"""GPU parity of the one-pass cross-entropy step (softmax_cross_entropy_step_hip): the forward's row
statistics and loss, the backward's dlogits = dloss * (softmax - onehot) and the bias gradient
sum_rows dlogits, from one read of the logits. Checked against the oracle (the reference chain of
src/api/loss.c:97-169 and its backward, bit-exact against the compiled reference on the CPU) at the
stated tolerances:
  row max: bit-exact; log-sum-exp l = log(S): 1e-5 absolute, the exp-sum S to 1e-5 relative (its
  order differs; a relative error of S is an absolute one of l); loss: 1e-5 of |loss| + 1;
  dlogits: 1e-5 of |value| + 1e-2 / N; dbias: 1e-5 of sum_rows |dlogits|.
Rows hold NaN, -inf, zero maxima, signed zeros and huge spreads (the exact-refold path), labels
sit in the SIMD tail of the loss's NEG rule, and shapes cover every register layout, rows that are
not whole float4 (the three-pass path), row counts several times the persistent grid (each
workgroup loops over many rows, with special rows met in later iterations on both register sets)
and config 5's full [32768, 32000] (sampled dlogits rows and every bias-gradient entry against a
float64 closed form there)."""
from __future__ import annotations

import contextlib

import numpy as np
import pytest

from cases import LSE_SCALE, assert_bits, assert_close_sum, check_ce_rows
from hostlib import HostTensor, oracle_backward, oracle_forward
from plast_amd import abi
from plast_amd.abi import KernelParams

pytestmark = pytest.mark.gpu


@contextlib.contextmanager
def deterministic(on=True):
    """plast_hip_set_deterministic for the duration (the step's bias gradient is then the same
    bits on every call; by default its split over workgroups follows the run's timing)."""
    from plast_amd import runtime as rt
    L = rt.lib()
    old = L.plast_hip_deterministic()
    L.plast_hip_set_deterministic(int(on))
    try:
        yield
    finally:
        L.plast_hip_set_deterministic(old)


def _step(rt, X, lab, g, with_bias=True, want_mean=False):
    N, Cn = X.shape
    st = rt.DeviceTensor((N, 2), zero=False)
    loss = rt.DeviceTensor((N,), zero=False)
    dx = rt.DeviceTensor((N, Cn), zero=False).fill_("uniform", 3, 5.0, 6.0)  # overwritten
    db = rt.DeviceTensor((Cn,), zero=False).fill_("uniform", 4, 5.0, 6.0) if with_bias else None
    mean = rt.DeviceTensor((1,), zero=False).fill_("uniform", 5, 5.0, 6.0) if want_mean else None
    G = rt.DeviceTensor.from_numpy(g)
    L = rt.lib()
    L.softmax_cross_entropy_step_hip(X.ptr, lab.ptr, G.ptr, st.ptr, loss.ptr, dx.ptr,
                                     db.ptr if db is not None else None,
                                     mean.ptr if mean is not None else None, N, Cn)
    L.check("ce step")
    out = (st.numpy(), loss.numpy(), dx.numpy(), db.numpy() if db is not None else None)
    return out + (float(mean.numpy()[0]),) if want_mean else out


def _check_mean(mean, loss, wloss):
    """The step's MEAN output against the oracle's mean (the reference's serial float sum, then
    / N) of the step's own per-row losses at 1e-5 of sum |loss| / N, and of the oracle's losses
    with the per-row loss bar added."""
    N = loss.shape[0]
    out = HostTensor(np.zeros(1, np.float32))
    oracle_forward("mean", [HostTensor(loss.copy())], out, KernelParams(abi.DIM_ALL, 0, 0.0))
    own = float(out.numpy()[0])
    oracle_forward("mean", [HostTensor(wloss.copy())], out, KernelParams(abi.DIM_ALL, 0, 0.0))
    ref = float(out.numpy()[0])
    if np.isnan(ref):
        assert np.isnan(mean) and np.isnan(own), f"mean {mean}, want NaN"
        return
    if np.isinf(own) or np.isinf(ref):
        assert mean == own == ref, f"mean {mean}, its losses' mean {own}, the oracle's {ref}"
        return
    a = np.abs(loss.astype(np.float64)).sum() / N
    assert abs(mean - own) <= 1e-5 * a + 1e-30, f"mean {mean} vs its losses' mean {own}"
    b = (np.abs(wloss.astype(np.float64)) + LSE_SCALE).sum() / N
    assert abs(mean - ref) <= 1e-5 * (a + b), f"mean {mean} vs the oracle's {ref}"


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
    st, loss, dx, db, mean = _step(rt, X, Lb, g, want_mean=True)
    wst, wloss, wdx = _oracle(x, lab, g)
    check_ce_rows(x, lab, g, st, loss, dx, wst, wloss, wdx, 1e-2 / N)
    _check_mean(mean, loss, wloss)
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
    """In deterministic mode two steps give identical bits; by default stats, loss and dlogits
    still do and the bias gradient is within the sum bar of the deterministic one. Against the op
    path (forward op, overwriting backward op, then the column sum) the row max is bit-equal and
    the rest within the bars above."""
    from plast_amd import ops, runtime as rt
    N, Cn = 512, 32000
    print(f"ce step vs op path {N}x{Cn}", flush=True)
    X = rt.DeviceTensor((N, Cn), requires_grad=True, zero=False).fill_("normal", 42, 0.0, 2.0)
    from plast_amd.abi import INT32
    Lb = rt.DeviceTensor((N,), INT32, zero=False).fill_("randint", 45, 0, Cn)
    g = np.full(N, np.float32(1.0) / np.float32(N), np.float32)
    with deterministic():
        a = _step(rt, X, Lb, g)
        b = _step(rt, X, Lb, g)
    for u, v, what in zip(a, b, ("stats", "loss", "dlogits", "dbias")):
        assert_bits(u, v, f"deterministic repeat: {what}")
    c = _step(rt, X, Lb, g)
    for u, v, what in zip(a[:3], c[:3], ("stats", "loss", "dlogits")):
        assert_bits(u, v, f"dynamic order: {what}")
    assert_close_sum(c[3], a[3], np.abs(a[2]).astype(np.float64).sum(0) + 1e-12, 1e-5,
                     "dynamic order: dbias")
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
    """Config 5 at [32768, 32000]: logits ~ N(0, 2), labels uniform, a per-row upstream gradient.
    Against float64: the loss of sampled rows, 256 sampled rows of dlogits element by element
    (g * (softmax - onehot) at 1e-5 of |value| + 1e-2 |g|), and every one of the 32000 bias-gradient
    entries against the float64 column sums of that closed form over all 32768 rows (1e-5 of the
    sum of the terms' magnitudes). Each workgroup walks 128 rows here. Size-independent properties
    too: every dlogits row sums to 0, the row max equals numpy's."""
    from plast_amd import runtime as rt
    from plast_amd.abi import INT32
    N, Cn = 32768, 32000
    print("ce step full size", flush=True)
    X = rt.DeviceTensor((N, Cn), zero=False).fill_("normal", 42, 0.0, 2.0)
    Lb = rt.DeviceTensor((N,), INT32, zero=False).fill_("randint", 45, 0, Cn)
    g = (np.random.RandomState(7).uniform(0.5, 1.5, N) / N).astype(np.float32)
    st, loss, dx, db = _step(rt, X, Lb, g)
    xh, yl = X.numpy(), Lb.numpy()
    X.free()
    rows = np.random.RandomState(3).choice(N, 256, replace=False)
    for r in rows[:16]:
        row = xh[r].astype(np.float64)
        lse = np.log(np.exp(row - row.max()).sum()) + row.max()
        assert abs(loss[r] - (lse - row[yl[r]])) <= 1e-5 * (abs(lse) + abs(row[yl[r]]))
    assert_bits(st[:, 0], xh.max(1), "row max")
    print("ce step full size: float64 closed form", flush=True)
    picked, col, acol = _closed_form_fp64(xh, yl, g, rows)
    for r in rows:
        assert_close_sum(dx[r], picked[r], np.abs(picked[r]) + 1e-2 * abs(float(g[r])), 1e-5,
                         f"dlogits row {r}")
    assert_close_sum(db, col, acol + 1e-12, 1e-5, "dbias against the float64 column sums")
    assert np.abs(dx.astype(np.float64).sum(1)).max() <= 1e-5 * float(g.max()) * 10
    assert abs(db.astype(np.float64).sum()) <= 1e-4


def test_step_full_size_repeats():
    """Config 5 at [32768, 32000], called repeatedly: in deterministic mode every output repeats
    bit for bit; in the default order the per-row outputs (statistics, loss, each dlogits row's sum
    and max taken by the library's fixed-order reductions) and the mean repeat bit for bit and equal
    the deterministic ones, and the bias gradient stays within 1e-5 of the sum of its terms'
    magnitudes of the deterministic one."""
    from plast_amd import ops, runtime as rt
    from plast_amd.abi import INT32
    N, Cn = 32768, 32000
    print("ce step full size, repeated calls", flush=True)
    L = rt.lib()
    X = rt.DeviceTensor((N, Cn), zero=False).fill_("normal", 42, 0.0, 2.0)
    Lb = rt.DeviceTensor((N,), INT32, zero=False).fill_("randint", 45, 0, Cn)
    G = rt.DeviceTensor((N,), zero=False).fill_("uniform", 7, 1.0 / N, 1.0 / N)
    st, lo = rt.DeviceTensor((N, 2), zero=False), rt.DeviceTensor((N,), zero=False)
    dx, db, mn = (rt.DeviceTensor((N, Cn), zero=False), rt.DeviceTensor((Cn,), zero=False),
                  rt.DeviceTensor((1,), zero=False))

    def call():
        L.softmax_cross_entropy_step_hip(X.ptr, Lb.ptr, G.ptr, st.ptr, lo.ptr, dx.ptr, db.ptr,
                                         mn.ptr, N, Cn)
        L.check("softmax_cross_entropy_step_hip")
        out = dict(st=st.numpy(), loss=lo.numpy(), mean=mn.numpy(),
                   rsum=ops.reduce("sum", dx, dim=1).numpy(),
                   rmax=ops.reduce("max", dx, dim=1).numpy(), db=db.numpy())
        return {k: v.copy() for k, v in out.items()}

    rows = ("st", "loss", "mean", "rsum", "rmax")
    try:
        with deterministic():
            ref = call()
            for i in range(8):
                got = call()
                for k in rows + ("db",):
                    assert_bits(got[k], ref[k], f"deterministic call {i + 2}: {k}")
        first = call()
        for k in rows:
            assert_bits(first[k], ref[k], f"default order: {k} against deterministic mode")
        dxh = dx.numpy()
        acol = np.zeros(Cn)
        for r0 in range(0, N, 2048):
            acol += np.abs(dxh[r0:r0 + 2048].astype(np.float64)).sum(0)
        del dxh
        for i in range(8):
            got = call()
            for k in rows:
                assert_bits(got[k], first[k], f"default order, call {i + 2}: {k}")
            assert_close_sum(got["db"], ref["db"], acol + 1e-12, 1e-5, f"default order, call {i + 2}: dbias")
    finally:
        for t in (X, Lb, G, st, lo, dx, db, mn):
            t.free()


# Rows outnumber the one-pass step's workgroups (one per CU, 256 on MI355X) several times over, and
# the row count is not a multiple of the grid: each workgroup's loop runs many iterations,
# alternates its two register sets, ends on either set (odd and even row counts per workgroup) and
# clamps its last prefetch to the final row. (771, 12000) gives each lane a ragged unit count.
# (1036, 8) and (2974, 100): rows whose exp-sum is barely above 1 (one dominant logit), where
# log(S) is small and the bar on it is absolute
MANY_ROWS = [(805, 32000), (2085, 8192), (1281, 4096), (771, 12000), (1036, 8), (2974, 100)]
GRID = 256


def _late_special_rows(x, finite):
    """Special rows placed where workgroup b meets them in its second, third and later iterations,
    on both register sets (with a grid of G, row r is workgroup r % G's iteration r // G, held in
    the first register set when that is even), and in the last two rows. `finite` keeps every
    gradient finite (no NaN or all -inf row), so the bias gradient stays comparable."""
    N, Cn = x.shape
    G = GRID
    at = [r for r in (G + 44, G + 45, 2 * G + 5, 2 * G + 6, 3 * G + 12, 3 * G + 13, 4 * G + 30,
                      7 * G + 7, N - 2, N - 1) if 0 <= r < N]
    kinds = ["zero_max", "overflow", "neg_inf_entry", "all_equal_huge"]
    if not finite:
        kinds += ["nan", "all_neg_inf"]
    for i, r in enumerate(at):
        k = kinds[i % len(kinds)]
        if k == "zero_max":
            x[r, :] = 0.0
            x[r, 1::3] = -0.0
        elif k == "overflow":
            x[r, :] = -3.0e38
            x[r, Cn // 3] = 3.0e38
        elif k == "neg_inf_entry":
            x[r, 7 % Cn] = -np.inf
        elif k == "all_equal_huge":
            x[r, :] = 1.0e30
        elif k == "nan":
            x[r, Cn - 1] = np.nan
        elif k == "all_neg_inf":
            x[r, :] = -np.inf
    return at


@pytest.mark.parametrize("specials", ["clean", "finite_specials", "nan_specials"])
@pytest.mark.parametrize("N, Cn", MANY_ROWS, ids=[f"{n}x{c}" for n, c in MANY_ROWS])
def test_step_many_rows_per_workgroup_matches_oracle(N, Cn, specials):
    """Every row against the oracle with a per-row upstream gradient (zero and negative ones
    included), at the bars of test_step_matches_oracle; the bias gradient against the float64
    column sums of the oracle's dlogits wherever those are finite."""
    from plast_amd import runtime as rt
    print(f"ce step many rows {N}x{Cn} {specials}", flush=True)
    rng = np.random.RandomState(N + 3 * Cn)
    x = (rng.randn(N, Cn) * 2).astype(np.float32)
    lab = rng.randint(0, Cn, N).astype(np.int32)
    lab[N - 1] = Cn - 1                         # the label in the row's last float4
    lab[N - 2] = 0
    at = _late_special_rows(x, specials == "finite_specials") if specials != "clean" else []
    if len(at) > 1:
        lab[at[1]] = Cn // 3                    # the label on the overflowing row's maximum
    g = (rng.uniform(0.2, 2.0, N) / N).astype(np.float32)
    g[GRID + 44 if GRID + 44 < N else 0] = 0.0
    g[2 * GRID + 5 if 2 * GRID + 5 < N else 1] = np.float32(-1.0 / N)
    X, Lb = rt.DeviceTensor.from_numpy(x), rt.DeviceTensor.from_numpy(lab)
    st, loss, dx, db, mean = _step(rt, X, Lb, g, want_mean=True)
    wst, wloss, wdx = _oracle(x, lab, g)
    check_ce_rows(x, lab, g, st, loss, dx, wst, wloss, wdx, np.abs(g) * 1e-2)
    assert_bits(np.isnan(loss), np.isnan(wloss), "NaN rows of the loss")
    _check_mean(mean, loss, wloss)
    assert_bits(np.isnan(dx), np.isnan(wdx), "NaN positions of dlogits")
    want = wdx.astype(np.float64).sum(0)
    ok = np.isfinite(want)
    if specials != "nan_specials":
        assert ok.all(), "these inputs keep every column of the bias gradient finite"
    assert_close_sum(db[ok], want[ok], np.abs(wdx.astype(np.float64)).sum(0)[ok] + 1e-12, 1e-5,
                     "dbias")
    assert_bits(np.isnan(db), np.isnan(want), "NaN columns of dbias")
    # the same inputs again: identical per-row bits (the column sums start from zero on every
    # call); then in deterministic mode, the static row split: the same bars, and its repeat is
    # the same bits in every output
    st2, loss2, dx2, db2 = _step(rt, X, Lb, g)
    for u, v, what in ((st2, st, "stats"), (loss2, loss, "loss"), (dx2, dx, "dlogits")):
        assert_bits(u, v, f"repeat: {what}")
    assert_close_sum(db2[ok], want[ok], np.abs(wdx.astype(np.float64)).sum(0)[ok] + 1e-12, 1e-5,
                     "dbias, second call")
    with deterministic():
        d1 = _step(rt, X, Lb, g)
        d2 = _step(rt, X, Lb, g)
    for u, v, what in zip(d1, d2, ("stats", "loss", "dlogits", "dbias")):
        assert_bits(u, v, f"deterministic repeat: {what}")
    for u, v, what in ((d1[0], st, "stats"), (d1[1], loss, "loss"), (d1[2], dx, "dlogits")):
        assert_bits(u, v, f"deterministic against dynamic: {what}")
    assert_close_sum(d1[3][ok], want[ok], np.abs(wdx.astype(np.float64)).sum(0)[ok] + 1e-12, 1e-5,
                     "deterministic dbias")
    assert_bits(np.isnan(d1[3]), np.isnan(want), "deterministic NaN columns of dbias")


def _closed_form_fp64(xh, yl, g, rows=None, chunk=1024):
    """g_r * (softmax(x_r) - onehot(y_r)) in float64, for the listed rows, and its column sums
    (and the sums of its magnitudes) over every row."""
    N, Cn = xh.shape
    col = np.zeros(Cn, np.float64)
    acol = np.zeros(Cn, np.float64)
    picked = {}
    want_rows = set() if rows is None else set(int(r) for r in rows)
    for r0 in range(0, N, chunk):
        x64 = xh[r0:r0 + chunk].astype(np.float64)
        x64 -= x64.max(1, keepdims=True)
        np.exp(x64, out=x64)
        x64 /= x64.sum(1, keepdims=True)
        x64[np.arange(x64.shape[0]), yl[r0:r0 + chunk]] -= 1.0
        x64 *= g[r0:r0 + chunk, None].astype(np.float64)
        for r in want_rows.intersection(range(r0, r0 + x64.shape[0])):
            picked[r] = x64[r - r0].copy()
        col += x64.sum(0)
        np.abs(x64, out=x64)
        acol += x64.sum(0)
    return picked, col, acol
