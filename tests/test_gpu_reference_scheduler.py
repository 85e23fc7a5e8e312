"""The reference's own scheduler over the HIP slots: oracle/_ref/libplast_ref_hip.so is the
reference's C sources built with the drop-in's scheduler edit applied (-DPLAST_HIP: its
fusion_optimize, src/scheduler/fusion.c:209-224, calls plast_hip_fuse_elementwise_chains after its
own patterns; oracle/hip_fusion_hook.py makes that edit on a temporary copy of fusion.c). Nodes are
made by its arena_node_alloc with the GPU slots of plast_hip_get_op_impl, and `schedule`
(src/scheduler/scheduler.c:16-52) runs them in JIT mode: a first call misses the cache
(jit.c:54-66), builds the DAG, lets fusion_optimize fuse it, inserts it (jit.c:84-104) and runs
it; a second call over the same graph finds it (jit_lookup) and replays the cached, fused DAG.

Checked against the oracle:
  config 2's chain exp(-leaky_relu(a * b + c, 0)): one FUSED_ELEMENTWISE node in the cached DAG,
  output within 2 ulp (exp) and bit for bit otherwise on the miss and again on the hit, with new
  inputs written between the calls (the replay reads the buffers as they are then);
  config 1's training step relu(X + b): schedule(FORWARD) then schedule(BACKWARD) on the same root
  (the backward is a cache hit), Y and dX bit for bit, the bias gradient within 1e-5 of
  sum_rows |terms| (the reference accumulates it with omp atomics, in no fixed order).

Needs oracle/_ref/libplast_ref_hip.so, built (with libplast_hip.so) in a container that holds the
reference's sources."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from cases import assert_bits, assert_close_sum
from hostlib import REF_HIP_PATH, HostTensor, oracle_backward, oracle_forward
from plast_amd import abi
from plast_amd.abi import KernelParams
from ref_executor import BACKWARD, CHAIN, FORWARD, RefGraph

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not REF_HIP_PATH.exists(),
                                 reason="oracle/_ref/libplast_ref_hip.so absent")]


def _ulp(x, y):
    xi = np.asarray(x, np.float32).view(np.int32).astype(np.int64)
    yi = np.asarray(y, np.float32).view(np.int32).astype(np.int64)
    return np.abs(np.where(xi < 0, -(xi & 0x7FFFFFFF), xi) - np.where(yi < 0, -(yi & 0x7FFFFFFF), yi))


def _cached_ops(sched):
    """(number of cached DAGs, op names of each)."""
    jit = sched.contents.jit.contents
    dags = [jit.entries[i].dag.contents for i in range(jit.cap) if jit.entries[i].occupied]
    return jit.count, [[abi.OP_NAMES[d.nodes[k].contents.op_type] for k in range(d.count)]
                       for d in dags]


def _oracle_chain(a, b, c):
    h = [HostTensor(v) for v in (a, b, c)]
    hts = {}
    for i, (op, srcs) in enumerate(CHAIN):
        ins = [h[s] if isinstance(s, int) else hts[s] for s in srcs]
        out = HostTensor(np.zeros(a.size, np.float32))
        oracle_forward(op, ins, out, KernelParams(0, 0, 0.0))
        hts[f"t{i}"] = out
    return hts["t4"].numpy()


def test_jit_schedule_fuses_on_a_miss_and_replays_on_a_hit():
    from plast_amd import runtime as rt
    print("reference scheduler: config 2 chain, JIT miss then hit", flush=True)
    n = (1 << 20) + 3
    rng = np.random.RandomState(21)
    a, b, c = (rng.randn(n).astype(np.float32) for _ in range(3))
    leaves = [rt.DeviceTensor.from_numpy(v) for v in (a, b, c)]
    g = RefGraph(ref_path=REF_HIP_PATH)
    R = g.R
    sched = R.init_scheduler(R.jit_create(16))
    R.set_jit_mode(sched, True)
    try:
        ts = {}
        for i, (op, srcs) in enumerate(CHAIN):
            ins = [leaves[s] if isinstance(s, int) else ts[s] for s in srcs]
            out = rt.DeviceTensor((n,), zero=False)
            g.node(op, ins, out, KernelParams(0, 0, 0.0))
            ts[f"t{i}"] = out
        fp = R.jit_fingerprint(g.root)
        R.schedule(sched, g.root, FORWARD, C.byref(g.arena))
        rt.lib().check("schedule (miss)")
        count, ops = _cached_ops(sched)
        assert count == 1 and ops == [["FUSED_ELEMENTWISE"]], ops
        assert R.jit_fingerprint(g.root) == fp, "the pass changed the graph's fingerprint"
        assert _ulp(ts["t4"].numpy(), _oracle_chain(a, b, c)).max() <= 2, "miss"
        # new inputs in the same buffers; the hit replays the cached DAG over them
        a2, b2, c2 = (rng.randn(n).astype(np.float32) for _ in range(3))
        for t, v in zip(leaves, (a2, b2, c2)):
            rt.lib().arena_memcpy_h2d_hip(t.ptr, v.ctypes.data, v.nbytes)
        R.schedule(sched, g.root, FORWARD, C.byref(g.arena))
        rt.lib().check("schedule (hit)")
        count, ops = _cached_ops(sched)
        assert count == 1 and ops == [["FUSED_ELEMENTWISE"]], "the second call was not a hit"
        assert _ulp(ts["t4"].numpy(), _oracle_chain(a2, b2, c2)).max() <= 2, "hit"
    finally:
        R.scheduler_release(sched)
        g.R.arena_release(C.byref(g.arena))


def test_jit_schedule_config1_forward_then_backward():
    from plast_amd import runtime as rt
    print("reference scheduler: config 1 training step, forward then backward", flush=True)
    rng = np.random.RandomState(22)
    x = rng.uniform(-1, 1, (1024, 256)).astype(np.float32)
    bias = rng.uniform(-1, 1, 256).astype(np.float32)
    gy = rng.uniform(-1, 1, (1024, 256)).astype(np.float32)
    X, B = rt.DeviceTensor.from_numpy(x, True), rt.DeviceTensor.from_numpy(bias, True)
    S = rt.DeviceTensor((1024, 256), requires_grad=True, zero=False)
    Y = rt.DeviceTensor((1024, 256), requires_grad=True, zero=False)
    g = RefGraph(ref_path=REF_HIP_PATH)
    R = g.R
    sched = R.init_scheduler(R.jit_create(16))
    R.set_jit_mode(sched, True)
    try:
        g.node("add", [X, B], S)
        g.node("leaky_relu", [S], Y, KernelParams(0, 0, 0.0))
        R.schedule(sched, g.root, FORWARD, C.byref(g.arena))
        rt.lib().check("schedule forward")
        count, ops = _cached_ops(sched)
        assert count == 1, ops
        fused_ops = ops[0]
        rt.lib().arena_memcpy_h2d_hip(Y.grad.ptr, gy.ctypes.data, gy.nbytes)
        R.schedule(sched, g.root, BACKWARD, C.byref(g.arena))
        rt.lib().check("schedule backward")
        count, ops = _cached_ops(sched)
        assert count == 1 and ops == [fused_ops], "the backward was not a cache hit"
        y, dx, db = Y.numpy(), X.grad.numpy(), B.grad.numpy()
    finally:
        R.scheduler_release(sched)
        g.R.arena_release(C.byref(g.arena))
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
    assert_close_sum(db, hb.grad.numpy(), np.abs(hs.grad.numpy()).sum(axis=0), 1e-5, "db")
