"""GPU checks of graph capture (plast_hip_capture_begin / capture_end / graph_launch): config 1's
training step (the fused relu(X + b) chain, then grad_b = Σ_rows grad_Y through the split
leading-axis reduction and its finalize) captured once and replayed several times, with fresh
inputs uploaded eagerly between replays, each replay checked bit for bit against the same step
run eagerly; the same step as the DAG runs it with the fused leaky_relu(x + bias) node and its
backward; plus a flat fused chain (2^20 elements, the tape interpreter), softmax with its backward
and the one-pass epilogue captured and replayed, and the error paths (nested capture, a launch
inside a capture, ending a capture that is not open)."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from cases import assert_bits

pytestmark = pytest.mark.gpu


def _rt():
    from plast_amd import runtime
    return runtime


def _h2d(dev, arr):
    L = _rt().lib()
    a = np.ascontiguousarray(arr, np.float32)
    L.arena_memcpy_h2d_hip(dev.ptr, a.ctypes.data, a.nbytes)
    L.check("h2d")


def test_config1_step_replays_match_eager():
    from plast_amd import abi, ops
    from plast_amd.abi import KernelParams
    rt = _rt()
    L = rt.lib()
    print("graph: config 1 step", flush=True)
    X, b, gy = (rt.DeviceTensor(s, zero=False) for s in ((1024, 256), (256,), (1024, 256)))
    Y, gb = rt.DeviceTensor((1024, 256), zero=False), rt.DeviceTensor((256,), zero=False)
    tape = ops.make_tape([("LOAD", 0, 0, 0, 0.0), ("ADD", abi.SRC_INPUT, 1, 0, 0.0),
                          ("LEAKY_RELU", 0, 0, 0, 0.0)], 2)

    def step():
        rt.forward("fused_elementwise", [X, b], Y, KernelParams(C.addressof(tape), 0, 0.0))
        rt.forward("sum", [gy], gb, KernelParams(0, 0, 0.0))

    rng = np.random.RandomState(1)
    for t, shape in ((X, (1024, 256)), (b, (256,)), (gy, (1024, 256))):
        _h2d(t, rng.uniform(-1, 1, shape))
    step()                                   # sizes the workspaces outside the capture
    assert L.plast_hip_capture_begin() == 0
    step()
    graph = L.plast_hip_capture_end()
    L.check("capture")
    assert graph
    try:
        for rep in range(5):
            for t, shape in ((X, (1024, 256)), (b, (256,)), (gy, (1024, 256))):
                _h2d(t, rng.uniform(-1, 1, shape))
            assert L.plast_hip_graph_launch(graph) == 0
            y_g, gb_g = Y.numpy(), gb.numpy()
            step()                           # the same step, eagerly, on the same inputs
            assert_bits(y_g, Y.numpy(), f"replay {rep}: relu(X + b)")
            assert_bits(gb_g, gb.numpy(), f"replay {rep}: grad_b")
    finally:
        L.plast_hip_graph_destroy(graph)


@pytest.mark.parametrize("shape", [(1024, 256), (4096, 1024)], ids=["config1", "4096x1024"])
def test_fused_dag_step_replays(shape):
    """Config 1's training step as the DAG runs it, the ADD -> LEAKY_RELU pair fused with
    gradients (forward writing Y; backward writing dX and adding grad_b's column sums, in the
    one-launch small form at config 1's size and the chunked pass with its finalize at the
    larger one), captured once and replayed with fresh inputs and cleared gradients, each replay
    bit for bit the same step run eagerly."""
    from plast_amd.abi import KernelParams
    from plast_amd.graph import Graph
    rt = _rt()
    L = rt.lib()
    print(f"graph: fused dag step {shape}", flush=True)
    R, Cn = shape
    X = rt.DeviceTensor(shape, requires_grad=True, zero=False)
    B = rt.DeviceTensor((Cn,), requires_grad=True, zero=False)
    S = rt.DeviceTensor(shape, requires_grad=True, zero=False)
    Y = rt.DeviceTensor(shape, requires_grad=True, zero=False)
    g = Graph()
    g.node("add", [X, B], S)
    g.node("leaky_relu", [S], Y, KernelParams(0, 0, 0.0))
    assert g.build(Y, fuse=True) == 1 and g.op_types() == ["FUSED_ELEMENTWISE"]

    def fresh(seed):
        X.fill_("uniform", seed, -1.0, 1.0)
        B.fill_("uniform", seed + 1, -1.0, 1.0)
        Y.grad.fill_("uniform", seed + 2, -1.0, 1.0)
        X.grad.fill_("uniform", seed + 3, 0.0, 0.0)
        B.grad.fill_("uniform", seed + 4, 0.0, 0.0)

    def step():
        g.forward()
        g.backward()

    fresh(10)
    step()                                   # sizes the workspaces outside the capture
    assert L.plast_hip_capture_begin() == 0
    step()
    graph = L.plast_hip_capture_end()
    L.check("capture")
    assert graph
    try:
        for rep in range(3):
            fresh(20 + 10 * rep)
            assert L.plast_hip_graph_launch(graph) == 0
            got = [t.numpy() for t in (Y, X.grad, B.grad)]
            fresh(20 + 10 * rep)
            step()
            for name, a, t in zip(("Y", "dX", "grad_b"), got, (Y, X.grad, B.grad)):
                assert_bits(a, t.numpy(), f"replay {rep}: {name}")
    finally:
        L.plast_hip_graph_destroy(graph)


def test_softmax_and_one_pass_epilogue_replay():
    """Softmax (rows in registers), its backward, and the one-pass relu-gradient modulation +
    bias-gradient sum (the column kernel, its 16 chunks and the 8-lane finalize) captured as one
    graph; each replay against the same calls run eagerly, bit for bit."""
    from plast_amd.abi import KernelParams
    rt = _rt()
    L = rt.lib()
    print("graph: softmax + one-pass epilogue", flush=True)
    R, Cn = 1024, 1000
    x = rt.DeviceTensor((R, Cn), requires_grad=True, zero=False)
    y = rt.DeviceTensor((R, Cn), requires_grad=True, zero=False)
    dout, z, dc = (rt.DeviceTensor((R, Cn), zero=False) for _ in range(3))
    db = rt.DeviceTensor((Cn,), zero=False)
    p = KernelParams(1, 0, 0.0)

    def step():
        rt.forward("softmax", [x], y, p)
        rt.backward("softmax", [x], y, p)
        L.relu_grad_modulate_bias_grad_hip(dout.ptr, z.ptr, dc.ptr, db.ptr, R * Cn, Cn, 0.01)
        L.check("one-pass epilogue")

    rng = np.random.RandomState(2)

    def fresh():
        for t in (x, y.grad, dout, z):
            _h2d(t, rng.randn(R, Cn))
        _h2d(x.grad, np.zeros((R, Cn)))

    fresh()
    step()                                   # sizes the workspaces outside the capture
    assert L.plast_hip_capture_begin() == 0
    step()
    graph = L.plast_hip_capture_end()
    L.check("capture")
    assert graph
    try:
        for rep in range(4):
            fresh()
            assert L.plast_hip_graph_launch(graph) == 0
            got = [t.numpy() for t in (y, x.grad, dc, db)]
            _h2d(x.grad, np.zeros((R, Cn)))
            step()                           # the same calls, eagerly, on the same inputs
            for g, t, what in zip(got, (y, x.grad, dc, db), ("y", "dx", "dc", "dbias")):
                assert_bits(g, t.numpy(), f"replay {rep}: {what}")
    finally:
        L.plast_hip_graph_destroy(graph)


def test_fused_chain_replays():
    from plast_amd import ops
    rt = _rt()
    L = rt.lib()
    print("graph: fused chain (tape interpreter)", flush=True)
    n = 1 << 20
    tape = ops.make_tape([("LOAD", 0, 0, 0, 0.0), ("MUL", 1, 1, 0, 0.0), ("ADD", 1, 2, 0, 0.0),
                          ("LEAKY_RELU", 0, 0, 0, 0.0), ("NEG", 0, 0, 0, 0.0),
                          ("EXP", 0, 0, 0, 0.0)], 3)
    ins = [rt.DeviceTensor((n,), zero=False) for _ in range(3)]
    out = rt.DeviceTensor((n,), zero=False)
    from plast_amd.abi import KernelParams

    def run():
        rt.forward("fused_elementwise", ins, out, KernelParams(C.addressof(tape), 0, 0.0))

    rng = np.random.RandomState(2)
    for t in ins:
        _h2d(t, rng.randn(n))
    run()
    assert L.plast_hip_capture_begin() == 0
    run()
    graph = L.plast_hip_capture_end()
    assert graph
    try:
        for rep in range(3):
            for t in ins:
                _h2d(t, rng.randn(n))
            assert L.plast_hip_graph_launch(graph) == 0
            got = out.numpy()
            run()
            assert_bits(got, out.numpy(), f"replay {rep}")
    finally:
        L.plast_hip_graph_destroy(graph)


def test_capture_errors():
    rt = _rt()
    L = rt.lib()
    x = rt.DeviceTensor((1024,), zero=False)
    y = rt.DeviceTensor((1024,), zero=False)
    L.plast_hip_clear_error()
    assert L.plast_hip_capture_begin() == 0
    graph = None
    try:
        assert L.plast_hip_capture_begin() == -1               # nested
        assert L.plast_hip_graph_launch(C.c_void_p(1)) == -1   # refused before the handle is used
        assert L.plast_hip_error_count() == 2
        L.plast_hip_clear_error()
        rt.forward("neg", [x], y)                              # recorded, not run
    finally:
        graph = L.plast_hip_capture_end()
    assert graph
    L.plast_hip_graph_destroy(graph)
    assert L.plast_hip_capture_end() is None                   # nothing open
    assert L.plast_hip_error_count() == 1
    L.plast_hip_clear_error()


def test_workspace_outgrown_while_a_graph_lives():
    """A captured step whose leading-axis sum keeps its chunk partials in workspace slot 0 (a
    [4096, 1024] sum, large enough for the chunked path), beside config 1's fused forward; then
    eager work grows slot 0 (a reserve past its size, then a cross-entropy step whose partial sums
    need more): the outgrown buffers are retired, not freed, so every replay still reads and writes
    the buffer it was recorded with and matches the eager step bit for bit; destroying the graph
    frees them."""
    from plast_amd import abi, ops
    from plast_amd.abi import KernelParams
    rt = _rt()
    L = rt.lib()
    print("graph: workspace outgrown while the graph lives", flush=True)
    X, b = (rt.DeviceTensor(s, zero=False) for s in ((1024, 256), (256,)))
    Y = rt.DeviceTensor((1024, 256), zero=False)
    gy, gb = rt.DeviceTensor((4096, 1024), zero=False), rt.DeviceTensor((1024,), zero=False)
    tape = ops.make_tape([("LOAD", 0, 0, 0, 0.0), ("ADD", abi.SRC_INPUT, 1, 0, 0.0),
                          ("LEAKY_RELU", 0, 0, 0, 0.0)], 2)

    def step():
        rt.forward("fused_elementwise", [X, b], Y, KernelParams(C.addressof(tape), 0, 0.0))
        rt.forward("sum", [gy], gb, KernelParams(0, 0, 0.0))

    rng = np.random.RandomState(3)

    def fresh():
        for t, shape in ((X, (1024, 256)), (b, (256,)), (gy, (4096, 1024))):
            _h2d(t, rng.uniform(-1, 1, shape))

    fresh()
    step()                                   # the sum sizes slot 0 outside the capture
    assert L.plast_hip_workspace_bytes(0) > 0
    alive0, retired0 = L.plast_hip_graphs_alive(), L.plast_hip_workspace_retired()
    assert L.plast_hip_capture_begin() == 0
    try:
        step()
    finally:
        graph = L.plast_hip_capture_end()
    L.check("capture")
    assert graph and L.plast_hip_graphs_alive() == alive0 + 1
    try:
        size0 = L.plast_hip_workspace_bytes(0)
        assert L.plast_hip_workspace_reserve(0, size0 + (1 << 20)) == 0
        L.check("reserve")
        assert L.plast_hip_workspace_bytes(0) >= size0 + (1 << 20)
        assert L.plast_hip_workspace_retired() == retired0 + 1
        # a cross-entropy step whose 256 workgroups' column sums outgrow slot 0 again
        N, Cn = 512, 4 * (L.plast_hip_workspace_bytes(0) // (256 * 4 * 4) + 1)
        if Cn <= 32768:
            logits = rt.DeviceTensor((N, Cn), zero=False).fill_("uniform", 7, -2.0, 2.0)
            labels = rt.DeviceTensor.from_numpy(rng.randint(0, Cn, N).astype(np.int32))
            dloss = rt.DeviceTensor.from_numpy(np.full(N, 1.0 / N, np.float32))
            st, loss = rt.DeviceTensor((N, 2), zero=False), rt.DeviceTensor((N,), zero=False)
            dx, db = rt.DeviceTensor((N, Cn), zero=False), rt.DeviceTensor((Cn,), zero=False)
            L.softmax_cross_entropy_step_hip(logits.ptr, labels.ptr, dloss.ptr, st.ptr, loss.ptr,
                                             dx.ptr, db.ptr, None, N, Cn)
            L.check("ce step")
            assert L.plast_hip_workspace_retired() == retired0 + 2
        for rep in range(3):
            fresh()
            assert L.plast_hip_graph_launch(graph) == 0
            y_g, gb_g = Y.numpy(), gb.numpy()
            step()                           # eagerly, through the grown slot
            assert_bits(y_g, Y.numpy(), f"replay {rep}: relu(X + b)")
            assert_bits(gb_g, gb.numpy(), f"replay {rep}: column sum")
    finally:
        L.plast_hip_graph_destroy(graph)
    assert L.plast_hip_graphs_alive() == alive0
    if alive0 == 0:
        assert L.plast_hip_workspace_retired() == 0


def test_free_during_capture_is_deferred():
    """A tensor freed while a graph is being recorded (Python may collect one at any time): the
    free is deferred instead of waiting on the recording stream, so the capture stays valid. The
    freed tensor here is the captured op's own input: its buffer is held until the graph is
    destroyed, so every replay still reads it (the values it held, which the eager op gave), and
    only the graph's destruction frees it."""
    rt = _rt()
    L = rt.lib()
    print("graph: free of a captured input during capture", flush=True)
    x = rt.DeviceTensor((4096,), zero=False)
    y = rt.DeviceTensor((4096,), zero=False)
    unused = rt.DeviceTensor((1 << 20,), zero=False)
    rng = np.random.RandomState(5)
    _h2d(x, rng.randn(4096))
    rt.forward("neg", [x], y)
    want = y.numpy()
    retired0, alive0 = L.plast_hip_workspace_retired(), L.plast_hip_graphs_alive()
    L.plast_hip_clear_error()
    assert L.plast_hip_capture_begin() == 0
    try:
        rt.forward("neg", [x], y)
        x.free()                                        # the captured input: deferred
        unused.free()                                   # a buffer the graph never touches
        assert L.plast_hip_error_count() == 0
    finally:
        graph = L.plast_hip_capture_end()
    L.check("capture with frees inside")
    assert graph
    try:
        # both buffers are held with the graph's lifetime, not freed at the capture's end
        assert L.plast_hip_workspace_retired() == retired0 + 2
        scratch = rt.DeviceTensor((1 << 20,), zero=False).fill_("uniform", 9, -1.0, 1.0)
        for rep in range(3):
            _h2d(y, rng.randn(4096))
            assert L.plast_hip_graph_launch(graph) == 0
            assert_bits(y.numpy(), want, f"replay {rep} over the freed input")
        scratch.free()
    finally:
        L.plast_hip_graph_destroy(graph)
    assert L.plast_hip_graphs_alive() == alive0
    if alive0 == 0:
        assert L.plast_hip_workspace_retired() == 0
