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
  config 1's training step leaky_relu(X + b) with gradients, fused by the pass into one node whose
  backward writes dX and adds the bias's column sum in one pass: Y and dX bit for bit, the bias
  gradient within 1e-5 of sum_rows |terms| (the reference's broadcast accumulation order is
  unspecified), over both operand orders, either gradient alone, slopes 0 and > 0, a rank-3 X,
  odd column counts, one row, and values where IEEE rules decide the mask and the sums;
  config 2's chain as a training graph (its ADD -> LEAKY_RELU pair fused with gradients, the other
  three nodes unfused, forward and backward), every leaf gradient within 4 ulp (each passes
  through exp's backward, which multiplies by exp's output, itself within 2 ulp).

Needs oracle/_ref/libplast_ref.so, built in a container that holds the reference's sources; skipped
where it is absent."""
from __future__ import annotations

import zlib

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


def _plant_specials(x, bias, gy):
    """Values where the mask or the sums are decided by IEEE rules: x + b overflowing to +-inf
    (with slope 0, -inf * 0 is NaN in y), NaN inputs, exact zeros of both signs, infinite and NaN
    upstream gradients."""
    x2, g2 = x.reshape(-1, x.shape[-1]), gy.reshape(-1, gy.shape[-1])
    C = x2.shape[1]
    if C < 8 or x2.shape[0] < 3:
        return
    bias[0], bias[1] = 3.0e38, -3.0e38
    x2[0, 0], x2[1, 1] = 3.0e38, -3.0e38
    x2[2, 2] = np.nan
    x2[0, 3], bias[3] = np.float32(-0.5), np.float32(0.5)     # x + b == +0
    x2[1, 4], bias[4] = np.float32(-0.0), np.float32(-0.0)    # x + b == -0
    g2[2, 5], g2[1, 6], g2[0, 7] = np.inf, np.nan, -0.0


CONFIG1_CASES = [
    # (name, x shape, slope, x grad, bias grad, bias first, bias 1-D, prefilled grads, specials)
    ("config1", (1024, 256), 0.0, True, True, False, True, False, False),
    ("leaky_bias_first", (1000, 260), 0.01, True, True, True, True, True, True),
    ("x_grad_only", (333, 132), 0.2, True, False, False, True, True, True),
    ("bias_grad_only", (333, 132), 0.0, False, True, True, False, True, True),
    ("rank3_odd_columns", (4, 37, 130), 0.0, True, True, False, True, True, True),
    ("one_row", (1, 4096), 0.1, True, True, False, False, True, False),
    ("many_rows", (16384, 64), 0.0, True, True, False, True, True, True),
]


@pytest.mark.parametrize("name, shape, alpha, gx, gb, bias_first, bias_1d, prefill, specials",
                         CONFIG1_CASES, ids=[c[0] for c in CONFIG1_CASES])
def test_config1_training_step_fused_through_the_reference_executor(
        name, shape, alpha, gx, gb, bias_first, bias_1d, prefill, specials):
    """leaky_relu(X + b) with gradients: the pass fuses the pair into one FUSED_ELEMENTWISE node
    (forward one launch writing Y only; backward one pass writing dX and adding the bias's column
    sum), run by the reference's dag_forward / dag_backward and checked against the unfused
    oracle: Y and dX bit for bit, the bias gradient within 1e-5 of sum_rows |terms| (the
    reference's broadcast accumulation order is unspecified). Gradients already holding values
    are added to, as the reference's backwards add."""
    from plast_amd import runtime as rt
    print(f"reference executor: fused leaky_relu(X + b) {name} {shape}", flush=True)
    rng = np.random.RandomState(zlib.crc32(name.encode()) % 1000)
    C = shape[-1]
    x = rng.uniform(-1, 1, shape).astype(np.float32)
    bias = rng.uniform(-1, 1, C if bias_1d else (1, C)).astype(np.float32)
    gy = rng.uniform(-1, 1, shape).astype(np.float32)
    if specials:
        _plant_specials(x, bias.reshape(-1), gy)
    gx0 = rng.uniform(-1, 1, shape).astype(np.float32) if prefill else np.zeros(shape, np.float32)
    gb0 = (rng.uniform(-1, 1, bias.shape).astype(np.float32) if prefill
           else np.zeros(bias.shape, np.float32))
    X, B = rt.DeviceTensor.from_numpy(x, gx), rt.DeviceTensor.from_numpy(bias, gb)
    if gx:
        rt.lib().arena_memcpy_h2d_hip(X.grad.ptr, gx0.ctypes.data, gx0.nbytes)
    if gb:
        rt.lib().arena_memcpy_h2d_hip(B.grad.ptr, gb0.ctypes.data, gb0.nbytes)
    S = rt.DeviceTensor(shape, requires_grad=True, zero=False)
    Y = rt.DeviceTensor(shape, requires_grad=True, zero=False)
    g = RefGraph()
    try:
        g.node("add", [B, X] if bias_first else [X, B], S)
        g.node("leaky_relu", [S], Y, KernelParams(0, 0, alpha))
        assert g.build(fuse=True) == 1
        assert g.op_types() == ["FUSED_ELEMENTWISE"], g.op_types()
        g.forward()
        rt.lib().arena_memcpy_h2d_hip(Y.grad.ptr, gy.ctypes.data, gy.nbytes)
        g.backward()
        y = Y.numpy()
        dx = X.grad.numpy() if gx else None
        db = B.grad.numpy() if gb else None
    finally:
        g.close()
    hx, hb = HostTensor(x, requires_grad=True), HostTensor(bias, requires_grad=True)
    hx.grad.buf[:] = gx0.reshape(-1)
    hb.grad.buf[:] = gb0.reshape(-1)
    hs = HostTensor(np.zeros_like(x), requires_grad=True)
    hy = HostTensor(np.zeros_like(x), requires_grad=True)
    ins = [hb, hx] if bias_first else [hx, hb]
    oracle_forward("add", ins, hs)
    oracle_forward("leaky_relu", [hs], hy, KernelParams(0, 0, alpha))
    hy.grad.buf[:] = gy.reshape(-1)
    oracle_backward("leaky_relu", [hs], hy, KernelParams(0, 0, alpha))
    oracle_backward("add", ins, hs)
    assert_bits(y, hy.numpy(), "leaky_relu(X + b)")
    if gx:
        assert_bits(dx, hx.grad.numpy(), "dX")
    if gb:
        scale = np.abs(hs.grad.numpy().astype(np.float64)).reshape(-1, C).sum(axis=0)
        scale = scale + np.abs(gb0.astype(np.float64)).reshape(-1)
        assert_close_sum(db.reshape(-1), hb.grad.numpy().reshape(-1), scale, 1e-5, "db")


def _random_case(seed):
    rng = np.random.RandomState(seed)
    C = int(rng.choice([1, 3, 4, 7, 64, 129, 256, 700]))
    if rng.rand() < 0.3:
        shape = (int(rng.randint(1, 9)), int(rng.randint(1, 200)), C)
    else:
        shape = (int(rng.choice([1, 2, 5, 31, 257, 1024, 3001])), C)
    gx, gb = [(True, True), (True, False), (False, True)][rng.randint(3)]
    return (f"random{seed}", shape, float(rng.choice([0.0, 0.01, 0.3])), gx, gb,
            bool(rng.rand() < 0.5), bool(rng.rand() < 0.5), bool(rng.rand() < 0.5),
            bool(rng.rand() < 0.5))


@pytest.mark.parametrize("seed", range(64))
def test_fused_step_random_shapes(seed):
    """Seeded random shapes (ranks 2 and 3, one row to 3001, one column to 700, float4 and
    scalar forms), slopes, operand orders, bias forms and gradients wanted, through the same
    check as the listed cases."""
    test_config1_training_step_fused_through_the_reference_executor(*_random_case(seed))


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
        # ADD(a*b, c) -> LEAKY_RELU is the pair the pass fuses with gradients (c, of the output's
        # extent, is a one-row bias); the other nodes stay, as they require grad
        assert g.build(fuse=True) == 1
        assert g.op_types() == ["MUL", "FUSED_ELEMENTWISE", "NEG", "EXP"], g.op_types()
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
