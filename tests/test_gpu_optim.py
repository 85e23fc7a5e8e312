"""GPU parity of the optimizer row: sgd/adam/adamw_step_hip and zero_grad_hip through the C-ABI,
bit for bit against the oracle (itself pinned to the compiled reference and golden vectors) after
three steps; parameters without gradients, NULL entries, misaligned tensors, more tensors than one
launch group (their table in device memory: two parameter lists in turn, so the table is replaced
on every call, and a misaligned tensor inside it; under graph capture, launches of one group each,
replayed against eager steps), and the moment allocation / release life cycle."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from cases import assert_bits
from optim_cases import MANY, OVER, SIZES, SPECIAL, SPECIAL_SEED, grads, initial, make_opt
from plast_amd import abi
from test_optim import run_host

pytestmark = pytest.mark.gpu


def _rt():
    from plast_amd import runtime
    return runtime


def _h2d(ptr, arr):
    L = _rt().lib()
    a = np.ascontiguousarray(arr, dtype=np.float32)
    L.arena_memcpy_h2d_hip(ptr, a.ctypes.data, a.nbytes)
    L.check("h2d")


def _d2h(t: abi.Tensor) -> np.ndarray:
    L = _rt().lib()
    shape = abi.shape_of(t)
    out = np.empty(shape, np.float32)
    if out.nbytes:
        L.arena_memcpy_d2h_hip(out.ctypes.data, t.data, out.nbytes)
        L.check("d2h")
    return out


def _run_device(kind, sizes, seed, steps, with_grad, nulls=()):
    """Same protocol as run_host, through the HIP entry points; `nulls` are positions of NULL
    entries inserted into the parameter array."""
    rt = _rt()
    L = rt.lib()
    p0 = initial(sizes, seed)
    dev = [rt.DeviceTensor.from_numpy(x, requires_grad=w) for x, w in zip(p0, with_grad)]
    slots = []
    it = iter(dev)
    for i in range(len(dev) + len(nulls)):
        slots.append(None if i in nulls else next(it))
    arr = (abi.TensorP * len(slots))(*[C.pointer(d.t) if d is not None else None for d in slots])
    ptrs = C.cast(arr, abi.TensorPP)
    opt = make_opt(kind)
    step = getattr(L, f"{kind}_step_hip")
    for s in range(steps):
        for d, g, w in zip(dev, grads(sizes, seed, s), with_grad):
            if w:
                _h2d(d.grad.ptr, g)
        step(C.byref(opt), ptrs, len(slots))
        L.check(f"{kind}_step_hip")
    ps = [d.numpy() for d in dev]
    mv = None
    if kind != "sgd":
        mv = [(_d2h(opt.m[i].contents), _d2h(opt.v[i].contents))
              for i, d in enumerate(slots) if d is not None]
        getattr(L, f"plast_hip_{kind}_release")(C.byref(opt), len(slots))
        L.check("release")
        assert not opt.m and not opt.v
    return ps, mv


@pytest.mark.parametrize("kind", ["sgd", "adam", "adamw"])
@pytest.mark.parametrize("set_name", ["shapes", "many", "over", "special_grads"])
def test_gpu_optimizer_matches_oracle(kind, set_name):
    sizes = {"shapes": SIZES, "many": MANY, "over": OVER, "special_grads": SPECIAL}[set_name]
    seed = SPECIAL_SEED if set_name == "special_grads" else 11
    print(f"optimizer {kind} {set_name}", flush=True)
    with_grad = [i % 5 != 3 for i in range(len(sizes))]
    po, mvo, _ = run_host("oracle", kind, sizes, seed, 3, with_grad)
    pd, mvd = _run_device(kind, sizes, seed, 3, with_grad)
    for i in range(len(sizes)):
        assert_bits(pd[i], po[i], f"{kind} p{i} {sizes[i]}")
        if mvo is not None:
            assert_bits(mvd[i][0], mvo[i][0], f"{kind} m{i}")
            assert_bits(mvd[i][1], mvo[i][1], f"{kind} v{i}")


@pytest.mark.parametrize("kind", ["sgd", "adamw"])
def test_gpu_optimizer_skips_null_entries(kind):
    sizes = [(33,), (1024,)]
    a, _ = _run_device(kind, sizes, 3, 2, [True, True])
    b, _ = _run_device(kind, sizes, 3, 2, [True, True], nulls=(0, 2))
    for i in range(2):
        assert_bits(b[i], a[i], f"{kind} with NULL entries, p{i}")


def test_gpu_optimizer_misaligned_parameter():
    """A parameter whose data starts 4 bytes into an allocation takes the scalar path."""
    rt = _rt()
    L = rt.lib()
    n = 1027
    base = rt.DeviceTensor((n + 1,), zero=True)
    gbase = rt.DeviceTensor((n + 1,), zero=True)
    p = rt.DeviceTensor((n,), base=base, offset=1, zero=False)
    g = rt.DeviceTensor((n,), base=gbase, offset=1, zero=False)
    p.t.grad = C.pointer(g.t)
    p0 = initial([(n,)], 21)[0]
    _h2d(p.ptr, p0)
    gs = [grads([(n,)], 21, s)[0] for s in range(2)]
    opt = make_opt("adam")
    ptrs, keep = abi.tensor_array(p.t)
    for s in range(2):
        _h2d(g.ptr, gs[s])
        L.adam_step_hip(C.byref(opt), ptrs, 1)
        L.check("adam_step_hip")
    got = p.numpy()
    L.plast_hip_adam_release(C.byref(opt), 1)
    want, _, _ = run_host("oracle", "adam", [(n,)], 21, 2)
    assert_bits(got, want[0], "misaligned adam")


def test_gpu_zero_grad():
    rt = _rt()
    L = rt.lib()
    x = rt.DeviceTensor.from_numpy(np.ones((7, 13), np.float32), requires_grad=True)
    _h2d(x.grad.ptr, np.arange(91, dtype=np.float32) - 45)
    L.zero_grad_hip(C.byref(x.t))
    L.check("zero_grad_hip")
    assert_bits(x.grad.numpy(), np.zeros((7, 13), np.float32), "zero_grad")
    assert_bits(x.numpy(), np.ones((7, 13), np.float32), "data untouched")
    L.zero_grad_hip(None)              # NULL tensor: no-op, as in the reference
    y = rt.DeviceTensor((5,))
    L.zero_grad_hip(C.byref(y.t))      # no grad: no-op
    L.check("zero_grad_hip no-op")


def test_gpu_adam_caller_provided_moments_are_kept():
    """Moments set by the caller are used as given and never freed by the release call."""
    rt = _rt()
    L = rt.lib()
    p0 = initial([(300,)], 8)[0]
    p = rt.DeviceTensor.from_numpy(p0, requires_grad=True)
    m, v = rt.DeviceTensor((300,)), rt.DeviceTensor((300,))
    marr = (abi.TensorP * 1)(C.pointer(m.t))
    varr = (abi.TensorP * 1)(C.pointer(v.t))
    opt = make_opt("adam")
    opt.m = C.cast(marr, abi.TensorPP)
    opt.v = C.cast(varr, abi.TensorPP)
    ptrs, keep = abi.tensor_array(p.t)
    _h2d(p.grad.ptr, grads([(300,)], 8, 0)[0])
    L.adam_step_hip(C.byref(opt), ptrs, 1)
    L.check("adam_step_hip")
    L.plast_hip_adam_release(C.byref(opt), 1)
    assert opt.m and opt.v                      # not owned by the library: left alone
    want, mv, _ = run_host("oracle", "adam", [(300,)], 8, 1)
    assert_bits(p.numpy(), want[0], "adam with caller moments")
    assert_bits(m.numpy(), mv[0][0], "caller m")


def _device_params(sizes, seed, misaligned=()):
    """Device parameters with gradient buffers; positions in `misaligned` start 4 bytes into
    their allocations. Returns (tensors kept alive, pointer array)."""
    rt = _rt()
    keep, ts = [], []
    for i, x in enumerate(initial(sizes, seed)):
        if i in misaligned:
            n = x.size
            base, gbase = rt.DeviceTensor((n + 1,)), rt.DeviceTensor((n + 1,))
            p = rt.DeviceTensor(x.shape, base=base, offset=1, zero=False)
            g = rt.DeviceTensor(x.shape, base=gbase, offset=1, zero=False)
            p.t.grad = C.pointer(g.t)
            _h2d(p.ptr, x)
            keep += [base, gbase, p, g]
            ts.append((p, g))
        else:
            d = rt.DeviceTensor.from_numpy(x, requires_grad=True)
            keep.append(d)
            ts.append((d, d.grad))
    arr = (abi.TensorP * len(ts))(*[C.pointer(p.t) for p, _ in ts])
    return ts, keep, arr


@pytest.mark.parametrize("kind", ["sgd", "adamw"])
def test_gpu_optimizer_tables_in_turn(kind):
    """Two lists of more than one launch group (83 and 70 tensors, the second with a misaligned
    tensor) stepped in turn: each call replaces the device table the other left."""
    print(f"optimizer {kind}: two tables in turn", flush=True)
    L = _rt().lib()
    sizes_b = [(33,)] * 30 + [(1029,)] * 39 + [(7, 5)]
    lists = [(OVER, 11, ()), (sizes_b, 12, (31,))]
    state = []
    for sizes, seed, mis in lists:
        ts, keep, arr = _device_params(sizes, seed, mis)
        state.append((sizes, seed, ts, keep, arr, make_opt(kind)))
    step = getattr(L, f"{kind}_step_hip")
    for s in range(3):
        for sizes, seed, ts, keep, arr, opt in state:
            for (p, g), gr in zip(ts, grads(sizes, seed, s)):
                _h2d(g.ptr, gr)
            step(C.byref(opt), C.cast(arr, abi.TensorPP), len(ts))
            L.check(f"{kind}_step_hip")
    for sizes, seed, ts, keep, arr, opt in state:
        want, _, _ = run_host("oracle", kind, sizes, seed, 3, [True] * len(sizes))
        for i, (p, _) in enumerate(ts):
            assert_bits(p.numpy(), want[i], f"{kind} list of {len(sizes)}, p{i}")
        if kind != "sgd":
            getattr(L, f"plast_hip_{kind}_release")(C.byref(opt), len(ts))


def test_gpu_optimizer_many_tensors_captured():
    """An SGD step over 83 tensors captured as a graph (launches of one group each, no table
    upload recorded) and replayed three times, eager work and synchronisations in between, equals
    three eager steps bit for bit."""
    print("optimizer: SGD over 83 tensors captured", flush=True)
    L = _rt().lib()
    results = []
    for captured in (False, True):
        ts, keep, arr = _device_params(OVER, 5)
        for (p, g), gr in zip(ts, grads(OVER, 5, 0)):
            _h2d(g.ptr, gr)
        opt = make_opt("sgd")
        ptrs = C.cast(arr, abi.TensorPP)
        if not captured:
            for _ in range(3):
                L.sgd_step_hip(C.byref(opt), ptrs, len(ts))
                L.check("sgd eager")
        else:
            assert L.plast_hip_capture_begin() == 0
            try:
                L.sgd_step_hip(C.byref(opt), ptrs, len(ts))
            finally:
                graph = L.plast_hip_capture_end()
            L.check("capture")
            assert graph
            try:
                for _ in range(3):
                    assert L.plast_hip_graph_launch(graph) == 0
                    L.plast_hip_synchronize()
                    _rt().DeviceTensor((1000,)).fill_("uniform", 1, 0.0, 1.0)  # eager work
            finally:
                L.plast_hip_graph_destroy(graph)
            L.check("replays")
        results.append([p.numpy() for p, _ in ts])
    for i, (e, c) in enumerate(zip(*results)):
        assert_bits(c, e, f"captured SGD p{i}")
