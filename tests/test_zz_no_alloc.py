"""The allocation-free cross-entropy step (softmax_cross_entropy_step_noalloc_hip) against the
allocating one (softmax_cross_entropy_step_hip) through the C-ABI: stats, loss, dlogits, the mean
loss and the bias gradient bit for bit in deterministic mode (both run the same kernels over the same grid, one
rule shared by the two entry points; by default the bias gradient's split over workgroups follows
the run's timing, so there it is held to the sum bar), on calls in a row whose second input is smaller than the first (the device array
keeps the previous call's contents), with no workspace growth, recorded into a graph and replayed,
and the rejection of rows the one-pass kernel cannot take."""
from __future__ import annotations

import contextlib

import numpy as np
import pytest

from cases import assert_bits, assert_close_sum

pytestmark = pytest.mark.gpu


@contextlib.contextmanager
def deterministic(L, on=True):
    old = L.plast_hip_deterministic()
    L.plast_hip_set_deterministic(int(on))
    try:
        yield
    finally:
        L.plast_hip_set_deterministic(old)


def _inputs(rt, N, Cn, seed, special=False):
    rng = np.random.RandomState(seed)
    x = (rng.randn(N, Cn) * 2).astype(np.float32)
    if special and N >= 4:
        x[1, 3] = np.nan
        x[2, :] = -np.inf
        x[3, :] = -3.0e38
        x[3, 0] = 3.0e38
    lab = rng.randint(0, Cn, N).astype(np.int32)
    g = np.full(N, np.float32(1.0) / np.float32(N), np.float32)
    return (rt.DeviceTensor.from_numpy(x), rt.DeviceTensor.from_numpy(lab),
            rt.DeviceTensor.from_numpy(g))


NAMES = ("stats", "loss", "dlogits", "mean loss", "dbias")


def _run(rt, entry, X, Lb, G, with_bias=True):
    N, Cn = X.shape
    st = rt.DeviceTensor((N, 2), zero=False).fill_("uniform", 1, 5.0, 6.0)
    loss = rt.DeviceTensor((N,), zero=False).fill_("uniform", 2, 5.0, 6.0)
    dx = rt.DeviceTensor((N, Cn), zero=False).fill_("uniform", 3, 5.0, 6.0)
    mean = rt.DeviceTensor((1,), zero=False).fill_("uniform", 5, 5.0, 6.0)
    db = rt.DeviceTensor((Cn,), zero=False).fill_("uniform", 4, 5.0, 6.0) if with_bias else None
    L = rt.lib()
    getattr(L, entry)(X.ptr, Lb.ptr, G.ptr, st.ptr, loss.ptr, dx.ptr,
                      db.ptr if db is not None else None, mean.ptr, N, Cn)
    L.check(entry)
    return ([st.numpy(), loss.numpy(), dx.numpy(), mean.numpy()] +
            ([db.numpy()] if with_bias else []))


def _same(rt, N, Cn, seed, special=False, with_bias=True):
    print(f"no-alloc step {N}x{Cn} special={special} bias={with_bias}", flush=True)
    L = rt.lib()
    X, Lb, G = _inputs(rt, N, Cn, seed, special)
    with deterministic(L):
        got = _run(rt, "softmax_cross_entropy_step_noalloc_hip", X, Lb, G, with_bias)
        want = _run(rt, "softmax_cross_entropy_step_hip", X, Lb, G, with_bias)
    for name, a, b in zip(NAMES, got, want):
        assert_bits(a, b, f"{N}x{Cn} {name}")
    # the default (dynamic) order: per-row outputs (and their mean, summed in a fixed order) the
    # same bits, the bias gradient to the sum bar
    dyn = _run(rt, "softmax_cross_entropy_step_noalloc_hip", X, Lb, G, with_bias)
    for name, a, b in zip(NAMES[:4], dyn, want):
        assert_bits(a, b, f"{N}x{Cn} {name}, dynamic order")
    if with_bias:
        assert_close_sum(dyn[4], want[4], np.abs(want[2]).astype(np.float64).sum(0) + 1e-12,
                         1e-5, f"{N}x{Cn} dbias, dynamic order")


def test_no_workspace_is_touched():
    """The no-alloc calls leave every workspace slot's size as it was. In a fresh process every
    slot is empty, so a call that went through the library's workspace for these column sums
    (256 x 32768 floats) would grow slot 0; after other tests it would unless an earlier call had
    already made the slot that large."""
    from plast_amd import runtime as rt
    L = rt.lib()
    print("no-alloc step: workspace sizes", flush=True)
    X, Lb, G = _inputs(rt, 300, 32768, 11)
    before = [L.plast_hip_workspace_bytes(s) for s in range(3)]
    with deterministic(L):
        a = _run(rt, "softmax_cross_entropy_step_noalloc_hip", X, Lb, G)
        b = _run(rt, "softmax_cross_entropy_step_noalloc_hip", X, Lb, G)
    assert [L.plast_hip_workspace_bytes(s) for s in range(3)] == before
    for name, u, v in zip(NAMES, a, b):
        assert_bits(u, v, f"repeat {name}")


def test_captured_no_alloc_step_replays():
    """One no-alloc call recorded into a graph (after an eager call has looked up the device
    array) and replayed with fresh logits between replays: each replay equals the eager call on the
    same inputs, bit for bit."""
    from plast_amd import runtime as rt
    L = rt.lib()
    print("no-alloc step: captured", flush=True)
    N, Cn = 600, 4096
    X, Lb, G = _inputs(rt, N, Cn, 12)
    st, loss = rt.DeviceTensor((N, 2), zero=False), rt.DeviceTensor((N,), zero=False)
    dx, db = rt.DeviceTensor((N, Cn), zero=False), rt.DeviceTensor((Cn,), zero=False)
    mean = rt.DeviceTensor((1,), zero=False)
    args = (X.ptr, Lb.ptr, G.ptr, st.ptr, loss.ptr, dx.ptr, db.ptr, mean.ptr, N, Cn)
    outs = (st, loss, dx, mean, db)
    with deterministic(L):
        _captured_replays(L, args, X, outs, exact=True)
    # the default order: the counter its workgroups take rows from is returned to zero by every
    # launch, so replays of a captured launch cover every row too
    _captured_replays(L, args, X, outs, exact=False)


def _captured_replays(L, args, X, outs, exact):
    L.softmax_cross_entropy_step_noalloc_hip(*args)
    L.check("eager no-alloc")
    assert L.plast_hip_capture_begin() == 0
    try:
        L.softmax_cross_entropy_step_noalloc_hip(*args)
    finally:
        graph = L.plast_hip_capture_end()
    L.check("capture of the no-alloc step")
    assert graph
    try:
        for rep in range(3):
            X.fill_("normal", 100 + rep, 0.0, 2.0)
            assert L.plast_hip_graph_launch(graph) == 0
            got = [t.numpy() for t in outs]
            L.softmax_cross_entropy_step_noalloc_hip(*args)
            L.check("eager no-alloc")
            now = [t.numpy() for t in outs]
            for name, u, v in zip(NAMES, got, now):
                if exact or name != "dbias":
                    assert_bits(u, v, f"replay {rep} {name}")
                else:
                    assert_close_sum(u, v, np.abs(now[2]).astype(np.float64).sum(0) + 1e-12,
                                     1e-5, f"replay {rep} dbias")
    finally:
        L.plast_hip_graph_destroy(graph)


def test_two_calls_second_smaller():
    from plast_amd import runtime as rt
    _same(rt, 3000, 8192, 1)          # 256 workgroups of column sums in the device array
    _same(rt, 37, 2048, 2)            # fewer workgroups and shorter rows: stale sums unread


@pytest.mark.parametrize("N, Cn, special, with_bias", [
    (13, 4, False, True), (64, 32000, True, True), (300, 32768, False, True),
    (9, 32768, True, True), (40, 12000, False, False), (1, 1024, True, True)])
def test_matches_allocating_step(N, Cn, special, with_bias):
    from plast_amd import runtime as rt
    _same(rt, N, Cn, N + Cn, special, with_bias)


def test_rows_beyond_the_one_pass_kernel_are_rejected():
    from plast_amd import runtime as rt
    L = rt.lib()
    for N, Cn in ((8, 6), (4, 32772), (3, 65536)):
        X, Lb, G = _inputs(rt, N, Cn, 5)
        st, loss = rt.DeviceTensor((N, 2)), rt.DeviceTensor((N,))
        dx = rt.DeviceTensor((N, Cn))
        L.softmax_cross_entropy_step_noalloc_hip(X.ptr, Lb.ptr, G.ptr, st.ptr, loss.ptr, dx.ptr,
                                                 None, None, N, Cn)
        with pytest.raises(rt.PlastHipError, match="not one-pass rows"):
            L.check("noalloc")
