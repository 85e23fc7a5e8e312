"""The drop-in through the reference's own executor. Nodes are made by the compiled reference's
arena_node_alloc (src/core/node.c:3-20) with the GPU slots of plast_hip_get_op_impl, ordered by its
build_dag (src/core/graph.c:30-55), passed through its fusion_optimize (src/scheduler/fusion.c:
209-224; no matmul/conv pattern here) and then the elementwise-chain pass the integration adds
there, and run by its dag_forward / dag_backward (graph.c:57-65). Those call execute_forward /
execute_backward (node.c:22-32), whose dispatchers (src/core/op.c) pick the `cuda` slots for
tensors on device 1: the HIP kernels.

Checked against the oracle:
  config 2's five-node chain, fused by the pass into one FUSED_ELEMENTWISE node (exp within 2 ulp,
  the rest bit for bit);
  config 1's training step relu(X + b) (not fused: it requires grad), its backward with an upstream
  gradient, dX bit for bit and the bias gradient within 1e-5 of sum_rows |terms| (the reference's
  broadcast accumulation order is unspecified);
  config 2's chain as a training graph (five unfused nodes forward and backward), every leaf
  gradient within 4 ulp (each passes through exp's backward, which multiplies by exp's output,
  itself within 2 ulp).

Needs oracle/_ref/libplast_ref.so, built in a container that holds the reference's sources; skipped
where it is absent."""
from __future__ import annotations

import numpy as np
import pytest

from cases import assert_bits, assert_close_sum
from hostlib import REF_PATH, HostTensor, oracle_backward, oracle_forward
from plast_amd.abi import KernelParams
from ref_executor import CHAIN, RefGraph

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not REF_PATH.exists(), reason="oracle/_ref/libplast_ref.so absent")]


def _ulp(x, y):
    xi = np.asarray(x, np.float32).view(np.int32).astype(np.int64)
    yi = np.asarray(y, np.float32).view(np.int32).astype(np.int64)
    return np.abs(np.where(xi < 0, -(xi & 0x7FFFFFFF), xi) - np.where(yi < 0, -(yi & 0x7FFFFFFF), yi))


def _chain(g, leaves, n, requires_grad, dev):
    """Config 2's chain exp(-leaky_relu(a * b + c, 0)) as five nodes; returns the tensors."""
    ts = {}
    for i, (op, srcs) in enumerate(CHAIN):
        ins = [leaves[s] if isinstance(s, int) else ts[s] for s in srcs]
        out = dev.DeviceTensor((n,), requires_grad=requires_grad, zero=False)
        g.node(op, ins, out, KernelParams(0, 0, 0.0))
        ts[f"t{i}"] = out
    return ts


def test_config2_chain_fused_by_the_pass_runs_in_the_reference_dag_forward():
    from plast_amd import runtime as rt
    print("reference executor: config 2 chain, fused", flush=True)
    n = (1 << 20) + 3
    rng = np.random.RandomState(11)
    a, b, c = (rng.randn(n).astype(np.float32) for _ in range(3))
    leaves = [rt.DeviceTensor.from_numpy(v) for v in (a, b, c)]
    g = RefGraph()
    try:
        ts = _chain(g, leaves, n, False, rt)
        assert g.build(fuse=True) == 1
        assert g.op_types() == ["FUSED_ELEMENTWISE"], g.op_types()
        g.forward()
        got = ts["t4"].numpy()
    finally:
        g.close()
    h = [HostTensor(v) for v in (a, b, c)]
    hts = {}
    for i, (op, srcs) in enumerate(CHAIN):
        ins = [h[s] if isinstance(s, int) else hts[s] for s in srcs]
        out = HostTensor(np.zeros(n, np.float32))
        oracle_forward(op, ins, out, KernelParams(0, 0, 0.0))
        hts[f"t{i}"] = out
    assert _ulp(got, hts["t4"].numpy()).max() <= 2


def test_config1_training_step_through_the_reference_executor():
    from plast_amd import runtime as rt
    print("reference executor: config 1 training step", flush=True)
    rng = np.random.RandomState(12)
    x = rng.uniform(-1, 1, (1024, 256)).astype(np.float32)
    bias = rng.uniform(-1, 1, 256).astype(np.float32)
    gy = rng.uniform(-1, 1, (1024, 256)).astype(np.float32)
    X, B = rt.DeviceTensor.from_numpy(x, True), rt.DeviceTensor.from_numpy(bias, True)
    S = rt.DeviceTensor((1024, 256), requires_grad=True, zero=False)
    Y = rt.DeviceTensor((1024, 256), requires_grad=True, zero=False)
    g = RefGraph()
    try:
        g.node("add", [X, B], S)
        g.node("leaky_relu", [S], Y, KernelParams(0, 0, 0.0))
        assert g.build(fuse=True) == 0          # requires grad: left for the backward
        assert g.op_types() == ["ADD", "LEAKY_RELU"]
        g.forward()
        rt.lib().arena_memcpy_h2d_hip(Y.grad.ptr, gy.ctypes.data, gy.nbytes)
        g.backward()
        y, dx, db = Y.numpy(), X.grad.numpy(), B.grad.numpy()
    finally:
        g.close()
    hx, hb = HostTensor(x, requires_grad=True), HostTensor(bias, requires_grad=True)
    hs = HostTensor(np.zeros_like(x), requires_grad=True)
    hy = HostTensor(np.zeros_like(x), requires_grad=True)
    oracle_forward("add", [hx, hb], hs)
    oracle_forward("leaky_relu", [hs], hy, KernelParams(0, 0, 0.0))
    hy.grad.buf[:] = gy.reshape(-1)
    oracle_backward("leaky_relu", [hs], hy, KernelParams(0, 0, 0.0))
    oracle_backward("add", [hx, hb], hs)
    assert_bits(y, hy.numpy(), "relu(X + b)")
    assert_bits(dx, hx.grad.numpy(), "dX")
    scale = np.abs(hs.grad.numpy()).sum(axis=0)
    assert_close_sum(db, hb.grad.numpy(), scale, 1e-5, "db")


def test_config2_chain_as_a_training_graph():
    from plast_amd import runtime as rt
    print("reference executor: config 2 chain, forward and backward", flush=True)
    n = 4099
    rng = np.random.RandomState(13)
    a, b, c = (rng.randn(n).astype(np.float32) for _ in range(3))
    gy = rng.uniform(-1, 1, n).astype(np.float32)
    leaves = [rt.DeviceTensor.from_numpy(v, True) for v in (a, b, c)]
    g = RefGraph()
    try:
        ts = _chain(g, leaves, n, True, rt)
        assert g.build(fuse=True) == 0
        assert g.op_types() == ["MUL", "ADD", "LEAKY_RELU", "NEG", "EXP"]
        g.forward()
        rt.lib().arena_memcpy_h2d_hip(ts["t4"].grad.ptr, gy.ctypes.data, gy.nbytes)
        g.backward()
        got = [t.grad.numpy() for t in leaves]
    finally:
        g.close()
    h = [HostTensor(v, requires_grad=True) for v in (a, b, c)]
    hts, order = {}, []
    for i, (op, srcs) in enumerate(CHAIN):
        ins = [h[s] if isinstance(s, int) else hts[s] for s in srcs]
        out = HostTensor(np.zeros(n, np.float32), requires_grad=True)
        oracle_forward(op, ins, out, KernelParams(0, 0, 0.0))
        hts[f"t{i}"] = out
        order.append((op, ins, out))
    hts["t4"].grad.buf[:] = gy
    for op, ins, out in reversed(order):
        oracle_backward(op, ins, out, KernelParams(0, 0, 0.0))
    for name, gv, ht in zip("abc", got, h):
        # every gradient passes through exp's backward (exp within 2 ulp, then products)
        d = _ulp(gv, ht.grad.numpy())
        assert d.max() <= 4, f"d{name}: {int(d.max())} ulp"
