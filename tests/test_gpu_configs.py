"""GPU parity for the five BASELINE.json configs, at their full shapes where the oracle finishes in
seconds, otherwise at a reduced leading extent with the same row/column geometry, plus
size-independent properties at full size.

Tolerances (written here): add/mul/relu/max/argmax bit-exact; exp within 2 ulp
of glibc; sum/mean/log-sum-exp |gpu - oracle| <= 1e-5 * (sum of |terms|)."""
from __future__ import annotations

import numpy as np
import pytest

from cases import assert_bits, assert_close_sum, assert_sum_parity, check_ce_rows
from hostlib import HostTensor, fused_chain2, oracle_backward, oracle_forward

pytestmark = pytest.mark.gpu


def _dev():
    from plast_amd import ops, runtime
    return ops, runtime


def _ulp(x, y):
    from gpu_backend import ulp_distance
    return ulp_distance(x, y)


def _host(arr, grad=False):
    return HostTensor(arr, requires_grad=grad)


# ----------------------------------------------------------------------------- config 1
def test_config1_bias_relu_and_grad_b():
    ops, rt = _dev()
    from plast_amd.abi import KernelParams
    rng = np.random.RandomState(42)
    X = rng.uniform(-1, 1, (1024, 256)).astype(np.float32)
    b = rng.uniform(-1, 1, 256).astype(np.float32)
    gY = rng.uniform(-1, 1, (1024, 256)).astype(np.float32)
    dX, db = rt.DeviceTensor.from_numpy(X), rt.DeviceTensor.from_numpy(b, requires_grad=True)
    s = ops.binary("add", dX, db)
    y = ops.unary("leaky_relu", s, 0.0)
    hs = _host(np.zeros_like(X))
    hy = _host(np.zeros_like(X))
    oracle_forward("add", [_host(X), _host(b)], hs)
    oracle_forward("leaky_relu", [hs], hy, KernelParams(0, 0, 0.0))
    assert_bits(y.numpy(), hy.numpy(), "relu(X+b) unfused")
    # fused single launch
    tape = ops.make_tape([("LOAD", 0, 0, 0, 0.0), ("ADD", 1, 1, 0, 0.0), ("LEAKY_RELU", 0, 0, 0, 0.0)], 2)
    yf = ops.fused(tape, [dX, db], (1024, 256))
    assert_bits(yf.numpy(), hy.numpy(), "relu(X+b) fused")
    # grad_b = sum over axis 0 of grad_Y
    gb = ops.reduce("sum", rt.DeviceTensor.from_numpy(gY), dim=0)
    ho = _host(np.zeros(256, np.float32))
    oracle_forward("sum", [_host(gY)], ho, KernelParams(0, 0, 0.0))
    assert_close_sum(gb.numpy(), ho.numpy(), np.abs(gY).sum(0), 1e-5, "grad_b")
    # the same through the ADD node's backward (broadcast reduction into b.grad)
    out = rt.DeviceTensor((1024, 256), requires_grad=True)
    rt.lib().arena_memcpy_h2d_hip(out.grad.ptr, gY.ctypes.data, gY.nbytes)
    rt.backward("add", [dX, db], out)
    assert_close_sum(db.grad.numpy(), ho.numpy(), np.abs(gY).sum(0), 1e-5, "add backward grad_b")


# ----------------------------------------------------------------------------- config 2
@pytest.mark.parametrize("n", [1 << 20, (1 << 20) + 12, 1 << 26])
def test_config2_fused_chain_matches_oracle(n):
    ops, rt = _dev()
    from plast_amd.abi import KernelParams
    from plast_amd.graph import Graph
    print(f"config2 n={n}", flush=True)
    rng = np.random.default_rng(42)
    a, b, c = (rng.standard_normal(n, dtype=np.float32) for _ in range(3))
    A, B, Cc = (rt.DeviceTensor.from_numpy(v) for v in (a, b, c))
    ys = []
    for fuse in (True, False):
        T = [rt.DeviceTensor((n,), zero=False) for _ in range(4)]
        Y = rt.DeviceTensor((n,), zero=False)
        g = Graph()
        m = g.node("mul", [A, B], T[0])
        s = g.node("add", [m, Cc], T[1])
        r = g.node("leaky_relu", [s], T[2], KernelParams(0, 0, 0.0))
        ng = g.node("neg", [r], T[3])
        g.node("exp", [ng], Y)
        k = g.build(Y, fuse=fuse)
        assert k == (1 if fuse else 0)
        g.forward()
        ys.append(Y.numpy())
    want = fused_chain2(a, b, c)
    d = _ulp(ys[0], want)
    assert d.max() <= 2, f"fused: max ulp {d.max()}"
    assert_bits(ys[0], ys[1], "fused == unfused launches")


# ----------------------------------------------------------------------------- config 3
@pytest.mark.parametrize("shape", [(16, 512, 512), (3, 68, 72), (2, 8, 12)])
def test_config3_permuted_broadcast(shape):
    ops, rt = _dev()
    print(f"config3 {shape}", flush=True)
    I, J, K = shape
    rng = np.random.RandomState(42)
    base = rng.randn(I, K, J).astype(np.float32)      # A_base; the view is permute(0,2,1)
    Bv = rng.uniform(0.5, 1.5, (1, J, 1)).astype(np.float32)
    Cv = rng.uniform(0.5, 1.5, (I, 1, K)).astype(np.float32)
    dA = rt.DeviceTensor.from_numpy(base)
    Av = ops.permute(dA, (0, 2, 1))
    dB, dC = rt.DeviceTensor.from_numpy(Bv), rt.DeviceTensor.from_numpy(Cv)
    t = ops.binary("add", Av, dB)
    o = ops.binary("mul", t, dC)
    # oracle: the same strided view
    hb = _host(base)
    hv = HostTensor(base=hb, shape=(I, J, K), strides=(J * K, 1, J))
    ht, ho = _host(np.zeros((I, J, K), np.float32)), _host(np.zeros((I, J, K), np.float32))
    oracle_forward("add", [hv, _host(Bv)], ht)
    oracle_forward("mul", [ht, _host(Cv)], ho)
    assert_bits(t.numpy(), ht.numpy(), "add(permuted, B)")
    assert_bits(o.numpy(), ho.numpy(), "mul(., C)")
    tape = ops.make_tape([("LOAD", 0, 0, 0, 0.0), ("ADD", 1, 1, 0, 0.0), ("MUL", 1, 2, 0, 0.0)], 3)
    of = ops.fused(tape, [Av, dB, dC], (I, J, K))
    assert_bits(of.numpy(), ho.numpy(), "fused (A_v + B) * C")


# ----------------------------------------------------------------------------- config 4
@pytest.mark.parametrize("rows,cols", [(4096, 4096), (300, 1000), (7, 65536)])
def test_config4_row_reductions(rows, cols):
    ops, rt = _dev()
    from plast_amd.abi import KernelParams, INT64
    print(f"config4 rows {rows}x{cols}", flush=True)
    x = np.random.RandomState(rows + cols).randn(rows, cols).astype(np.float32)
    # special rows: NaN positions, signed-zero maxima, ties, all -inf
    x[0, 5] = np.nan
    x[1, -1] = np.nan
    x[2, :] = -1.0
    x[2, 3], x[2, 9] = 0.0, -0.0
    x[3, :] = -np.inf
    x[4, ::7] = x[4].max() + 1.0
    dx = rt.DeviceTensor.from_numpy(x)
    hx = _host(x)
    for op in ("sum", "mean", "max", "min", "argmax"):
        g = ops.reduce(op, dx, dim=1).numpy()
        ho = _host(np.zeros(rows, np.int64 if op == "argmax" else np.float32))
        oracle_forward(op, [hx], ho, KernelParams(1, 0, 0.0))
        if op in ("sum", "mean"):
            div = cols if op == "mean" else 1
            scale = np.abs(x.astype(np.float64)).sum(1) / div
            truth = x.astype(np.float64).sum(1) / div
            assert_sum_parity(g, ho.numpy(), truth, scale, 1e-5, f"{op} rows")
        else:
            assert_bits(g, ho.numpy(), f"{op} rows")


@pytest.mark.parametrize("rows,cols", [(4096, 4096), (1000, 300), (65536, 8)])
def test_config4_axis0_reductions(rows, cols):
    ops, rt = _dev()
    from plast_amd.abi import KernelParams
    print(f"config4 axis0 {rows}x{cols}", flush=True)
    x = np.random.RandomState(rows * 3 + cols).randn(rows, cols).astype(np.float32)
    x[7, 0] = np.nan
    x[:, 1] = -1.0
    x[10, 1], x[20, 1] = -0.0, 0.0
    x[:, 2] = -np.inf
    dx, hx = rt.DeviceTensor.from_numpy(x), _host(x)
    for op in ("sum", "mean", "max", "min", "argmax"):
        g = ops.reduce(op, dx, dim=0).numpy()
        ho = _host(np.zeros(cols, np.int64 if op == "argmax" else np.float32))
        oracle_forward(op, [hx], ho, KernelParams(0, 0, 0.0))
        if op in ("sum", "mean"):
            div = rows if op == "mean" else 1
            scale = np.abs(x.astype(np.float64)).sum(0) / div
            truth = x.astype(np.float64).sum(0) / div
            assert_sum_parity(g, ho.numpy(), truth, scale, 1e-5, f"{op} axis0")
        else:
            assert_bits(g, ho.numpy(), f"{op} axis0")


def test_config4_full_size_properties():
    ops, rt = _dev()
    print("config4 full size", flush=True)
    X = rt.DeviceTensor((65536, 4096), zero=False).fill_("normal", 42, 0.0, 1.0)
    mx = ops.reduce("max", X, dim=1).numpy()
    am = ops.reduce("argmax", X, dim=1).numpy()
    sm = ops.reduce("sum", X, dim=1).numpy()
    rows = np.random.RandomState(0).choice(65536, 64, replace=False)
    xh = X.numpy()
    for r in rows:
        row = xh[r]
        assert row[am[r]] == mx[r] == row.max() and am[r] == int(np.argmax(row))
        assert abs(float(sm[r]) - row.astype(np.float64).sum()) <= 1e-5 * np.abs(row).sum()
    XT = rt.DeviceTensor((4096, 65536), zero=False).fill_("normal", 43, 0.0, 1.0)
    cs = ops.reduce("sum", XT, dim=0).numpy()
    cm = ops.reduce("max", XT, dim=0).numpy()
    xt = XT.numpy()
    cols = np.random.RandomState(1).choice(65536, 64, replace=False)
    for c in cols:
        col = xt[:, c]
        assert cm[c] == col.max()
        assert abs(float(cs[c]) - col.astype(np.float64).sum()) <= 1e-5 * np.abs(col).sum()


# ----------------------------------------------------------------------------- config 5
@pytest.mark.parametrize("N,Cn", [(512, 32000), (64, 1000), (33, 4), (8, 7)])
def test_config5_softmax_ce(N, Cn):
    ops, rt = _dev()
    from plast_amd.abi import INT32, KernelParams
    print(f"config5 {N}x{Cn}", flush=True)
    rng = np.random.RandomState(N + Cn)
    x = (rng.randn(N, Cn) * 2).astype(np.float32)
    lab = rng.randint(0, Cn, N).astype(np.int32)
    if N >= 8:
        x[1, 3] = np.nan           # NaN row: loss NaN (reference chain)
        x[2, :] = 0.0              # zero maximum
        x[2, 1] = -0.0
        x[3, 0] = -np.inf          # 0 * -inf in the one-hot product gives NaN
        x[4, :] = -3.0e38          # huge negative row
        x[4, 0] = 3.0e38           # x - max overflows to -inf
    dx = rt.DeviceTensor.from_numpy(x, requires_grad=True)
    dl = rt.DeviceTensor.from_numpy(lab)
    loss, stats = ops.softmax_cross_entropy(dx, dl, requires_grad=True)
    hx, hl = _host(x, grad=True), _host(lab)
    hs, ho = _host(np.zeros((N, 2), np.float32)), _host(np.zeros(N, np.float32), grad=True)
    oracle_forward("softmax_cross_entropy", [hx, hl, hs], ho)
    st, wst = stats.numpy(), hs.numpy()
    # backward with dloss = 1/N (the MEAN node's backward)
    g = np.full(N, np.float32(1.0) / np.float32(N), np.float32)
    rt.lib().arena_memcpy_h2d_hip(loss.grad.ptr, g.ctypes.data, g.nbytes)
    ho.grad.buf[:] = g
    rt.backward("softmax_cross_entropy", [dx, dl, stats], loss)
    oracle_backward("softmax_cross_entropy", [hx, hl, hs], ho)
    gx, wx = dx.grad.numpy(), hx.grad.numpy()
    # statistics, loss and dlogits against the oracle, or the fp64 value where its serial
    # exp-sum drifts
    check_ce_rows(x, lab, g, st, loss.numpy(), gx, wst, ho.numpy(), wx, 1e-2 / N)
    # overwrite mode gives the same values into a fresh buffer
    dx2 = rt.DeviceTensor.from_numpy(x, requires_grad=True)
    rt.backward("softmax_cross_entropy", [dx2, dl, stats], loss, KernelParams(0, 1, 0.0))
    assert_bits(dx2.grad.numpy(), gx, "overwrite == accumulate into zeros")
    # bias grad = sum over rows of the logits gradient (ADD backward into a broadcast [C] bias)
    bg = ops.reduce("sum", dx.grad, dim=0).numpy()
    wb = _host(np.zeros(Cn, np.float32))
    oracle_forward("sum", [_host(gx)], wb, KernelParams(0, 0, 0.0))
    assert_close_sum(bg[np.isfinite(bg)], wb.numpy()[np.isfinite(bg)],
                     np.abs(gx).sum(0)[np.isfinite(bg)] + 1e-12, 1e-5, "bias grad")


def test_config5_full_size_properties():
    ops, rt = _dev()
    from plast_amd.abi import INT32
    print("config5 full size", flush=True)
    N, Cn = 32768, 32000
    X = rt.DeviceTensor((N, Cn), requires_grad=True, zero=True)
    X.fill_("normal", 42, 0.0, 2.0)
    lab = rt.DeviceTensor((N,), INT32, zero=False).fill_("randint", 45, 0, Cn)
    loss, stats = ops.softmax_cross_entropy(X, lab, requires_grad=True)
    g = np.full(N, np.float32(1.0) / np.float32(N), np.float32)
    rt.lib().arena_memcpy_h2d_hip(loss.grad.ptr, g.ctypes.data, g.nbytes)
    rt.backward("softmax_cross_entropy", [X, lab, stats], loss)
    rows = np.random.RandomState(3).choice(N, 16, replace=False)
    xh = X.numpy()
    gh = X.grad.numpy()
    lh, st, yl = loss.numpy(), stats.numpy(), lab.numpy()
    for r in rows:
        row = xh[r].astype(np.float64)
        lse = np.log(np.exp(row - row.max()).sum()) + row.max()
        assert abs(lh[r] - (lse - row[yl[r]])) <= 1e-5 * (abs(lse) + abs(row[yl[r]]))
        assert st[r, 0] == xh[r].max()
        assert abs(gh[r].astype(np.float64).sum()) <= 1e-5 / N * 10     # rows of (p - onehot) sum to 0
    bias = ops.reduce("sum", X.grad, dim=0).numpy()
    assert abs(bias.astype(np.float64).sum()) <= 1e-4                  # total gradient mass is 0
