"""The reference's own pytest cases for this path, restated against the HIP backend.

Each case keeps the reference test's inputs (np.random.RandomState(42) per test, as its `rng`
fixture: tests/conftest.py:56-58), its op sequence and its numpy closed form, and its tolerance
(rtol 1e-3 / atol 1e-4: conftest.py:5-6; exp at atol 1e-3). Sources:
tests/test_ops.py:18-189, 205-287, 407-433 (elementwise, reductions, shape ops, leaky relu, ops with
gradients) and tests/test_gradients.py:20-188 (autograd basics and per-op gradients). Matmul and
conv cases are out of this path. The expressions run through reference_api, which builds the DAG
of `<op>_hip_forward/backward` nodes."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SHAPES = [(4,), (2, 3), (3, 2, 4)]
BROADCAST_PAIRS = [((4,), (1,)), ((2, 3), (1, 3)), ((3, 1, 4), (1, 2, 1))]
TOL = dict(rtol=1e-3, atol=1e-4)


@pytest.fixture
def rng():
    return np.random.RandomState(42)


@pytest.fixture
def P():
    import reference_api
    reference_api.reset()
    return reference_api


def close(got, want, **kw):
    np.testing.assert_allclose(got, want, **(kw or TOL))


# ------------------------------------------------------------------ test_ops.py: elementwise
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("op", ["add", "sub", "mul", "div"])
def test_binary_forward(P, rng, shape, op):
    a = rng.randn(*shape).astype(np.float32)
    if op == "div":
        b = np.abs(rng.randn(*shape)).astype(np.float32) + 0.1
    else:
        b = rng.randn(*shape).astype(np.float32)
    ta, tb = P.tensor(a), P.tensor(b)
    tc = {"add": ta + tb, "sub": ta - tb, "mul": ta * tb, "div": ta / tb}[op]
    P.forward(tc)
    close(tc.numpy(), {"add": a + b, "sub": a - b, "mul": a * b, "div": a / b}[op])


@pytest.mark.parametrize("shape_a, shape_b", BROADCAST_PAIRS)
def test_add_broadcast(P, rng, shape_a, shape_b):
    a = rng.randn(*shape_a).astype(np.float32)
    b = rng.randn(*shape_b).astype(np.float32)
    tc = P.tensor(a) + P.tensor(b)
    P.forward(tc)
    close(tc.numpy(), a + b)


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("op", ["neg", "abs", "exp", "log", "sin", "cos", "tan"])
def test_unary_forward(P, rng, shape, op):
    a = rng.randn(*shape).astype(np.float32)
    if op == "log":
        a = np.abs(a).astype(np.float32) + 0.1
    ta = P.tensor(a)
    tc = {"neg": lambda: -ta, "abs": lambda: abs(ta)}.get(op, lambda: getattr(ta, op)())()
    P.forward(tc)
    want = {"neg": np.negative, "abs": np.abs, "exp": np.exp, "log": np.log, "sin": np.sin,
            "cos": np.cos, "tan": np.tan}[op](a)
    if op == "exp":
        close(tc.numpy(), want, atol=1e-3)
    else:
        close(tc.numpy(), want)


# ------------------------------------------------------------------ test_ops.py: reductions
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("op", ["sum", "mean", "max", "min"])
def test_full_reduction(P, rng, shape, op):
    a = rng.randn(*shape).astype(np.float32)
    tc = getattr(P.tensor(a), op)()
    P.forward(tc)
    close(tc.numpy(), np.array([getattr(np, op)(a)]))


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("op", ["sum", "mean"])
def test_dim_reduction(P, rng, shape, op):
    a = rng.randn(*shape).astype(np.float32)
    ta = P.tensor(a)
    for dim in range(len(shape)):
        tc = getattr(ta, op)(dim=dim)
        P.forward(tc)
        close(tc.numpy().reshape(-1), getattr(np, op)(a, axis=dim).reshape(-1))


@pytest.mark.parametrize("shape", [(2, 3), (3, 4)])
def test_max_dim_keepdim(P, rng, shape):
    a = rng.randn(*shape).astype(np.float32)
    ta = P.tensor(a)
    for dim in range(len(shape)):
        tc = ta.max(dim=dim, keepdim=True)
        P.forward(tc)
        close(tc.numpy(), np.max(a, axis=dim, keepdims=True))


# ------------------------------------------------------------------ test_ops.py: shape ops
@pytest.mark.parametrize("shape", [(2, 3, 4), (4, 6)])
def test_view(P, rng, shape):
    a = rng.randn(*shape).astype(np.float32)
    tc = P.tensor(a).view(shape[0], -1)
    P.forward(tc)
    close(tc.numpy(), a.reshape(shape[0], -1))


def test_reshape(P, rng):
    a = rng.randn(2, 6).astype(np.float32)
    tc = P.tensor(a).reshape(3, 4)
    P.forward(tc)
    close(tc.numpy(), a.reshape(3, 4))


@pytest.mark.parametrize("shape", [(2, 3, 4), (4, 5)])
def test_transpose(P, rng, shape):
    a = rng.randn(*shape).astype(np.float32)
    tc = P.tensor(a).transpose(0, 1)
    P.forward(tc)
    close(tc.numpy(), np.transpose(a, (1, 0, 2)) if len(shape) == 3 else a.T)


def test_squeeze_unsqueeze_flatten_expand(P, rng):
    a = rng.randn(1, 3, 1, 4).astype(np.float32)
    tc = P.tensor(a).squeeze()
    P.forward(tc)
    assert tc.shape == [3, 4]
    close(tc.numpy(), a.reshape(3, 4))
    b = rng.randn(3, 4).astype(np.float32)
    tu = P.tensor(b).unsqueeze(0)
    P.forward(tu)
    assert tu.shape == [1, 3, 4]
    close(tu.numpy(), b[np.newaxis, ...])
    c = rng.randn(2, 3, 4).astype(np.float32)
    tf = P.tensor(c).flatten(1, 2)
    P.forward(tf)
    close(tf.numpy(), c.reshape(2, -1))
    d = rng.randn(1, 3, 1).astype(np.float32)
    te = P.tensor(d).expand(4, 3, 5)
    P.forward(te)
    close(te.numpy(), np.broadcast_to(d, (4, 3, 5)))


@pytest.mark.parametrize("shape", SHAPES)
def test_leaky_relu_forward(P, rng, shape):
    a = rng.randn(*shape).astype(np.float32)
    tc = P.tensor(a).leaky_relu(0.01)
    P.forward(tc)
    close(tc.numpy(), np.where(a > 0, a, 0.01 * a))


# ------------------------------------------------------------------ test_ops.py: with gradients
def test_add_mul_backward(P, rng):
    a = rng.randn(2, 3).astype(np.float32)
    b = rng.randn(2, 3).astype(np.float32)
    ta, tb = P.tensor(a, True), P.tensor(b, True)
    loss = (ta + tb).sum()
    P.forward(loss)
    loss.backward()
    np.testing.assert_allclose(ta.grad.numpy(), np.ones((2, 3)))
    P.reset()
    ta, tb = P.tensor(a, True), P.tensor(b, True)
    loss = (ta * tb).sum()
    P.forward(loss)
    loss.backward()
    close(ta.grad.numpy(), b)
    close(tb.grad.numpy(), a)


# ------------------------------------------------------------------ test_gradients.py
def test_gradient_accumulation_with_zero_grad(P, rng):
    import ctypes as C
    from plast_amd.runtime import lib
    x = P.tensor(rng.randn(3).astype(np.float32), True)
    y = P.tensor(rng.randn(3).astype(np.float32), True)
    z = (x * y).sum()
    P.forward(z)
    z.backward()
    first = x.grad.numpy().copy()
    P.reset()
    for p in (x, y):
        lib().zero_grad_hip(C.byref(p.dev.t))
    z2 = (x * y).sum()
    P.forward(z2)
    z2.backward()
    close(x.grad.numpy(), first)


def test_requires_grad_false(P, rng):
    x = P.tensor(rng.randn(3).astype(np.float32), True)
    y = P.tensor(rng.randn(3).astype(np.float32), False)
    z = (x * y).sum()
    P.forward(z)
    z.backward()
    assert x.grad is not None and y.grad is None


def test_multi_input_graph(P, rng):
    a = P.tensor(rng.randn(2, 3).astype(np.float32), True)
    b = P.tensor(rng.randn(2, 3).astype(np.float32), True)
    c = P.tensor(rng.randn(2, 3).astype(np.float32), False)
    loss = ((a + b) * c).sum()
    P.forward(loss)
    loss.backward()
    close(a.grad.numpy(), c.numpy())
    close(b.grad.numpy(), c.numpy())


def test_add_sub_grad_of_mean(P, rng):
    a = P.tensor(rng.randn(2, 3).astype(np.float32), True)
    b = P.tensor(rng.randn(2, 3).astype(np.float32), True)
    loss = (a + b).mean()
    P.forward(loss)
    loss.backward()
    close(a.grad.numpy(), np.ones((2, 3)) / 6)
    close(b.grad.numpy(), np.ones((2, 3)) / 6)
    P.reset()
    a = P.tensor(rng.randn(2, 3).astype(np.float32), True)
    b = P.tensor(rng.randn(2, 3).astype(np.float32), True)
    loss = (a - b).sum()
    P.forward(loss)
    loss.backward()
    close(a.grad.numpy(), np.ones((2, 3)))
    close(b.grad.numpy(), -np.ones((2, 3)))


def test_div_grad(P, rng):
    a_data = rng.randn(2, 3).astype(np.float32)
    b_data = np.abs(rng.randn(2, 3)).astype(np.float32) + 0.1
    a, b = P.tensor(a_data, True), P.tensor(b_data, True)
    loss = (a / b).sum()
    P.forward(loss)
    loss.backward()
    close(a.grad.numpy(), 1.0 / b_data)
    close(b.grad.numpy(), -a_data / (b_data ** 2))


@pytest.mark.parametrize("op", ["sin", "cos", "exp", "log", "neg", "abs", "tan", "leaky_relu"])
def test_unary_grad(P, rng, op):
    x_data = rng.randn(3).astype(np.float32)
    if op == "log":
        x_data = (np.abs(x_data) + 0.1).astype(np.float32)
    x = P.tensor(x_data, True)
    y = {"neg": lambda: -x, "abs": lambda: abs(x),
         "leaky_relu": lambda: x.leaky_relu(0.01)}.get(op, lambda: getattr(x, op)())()
    loss = y.sum()
    P.forward(loss)
    loss.backward()
    want = {"sin": np.cos(x_data), "cos": -np.sin(x_data), "exp": np.exp(x_data),
            "log": 1.0 / x_data, "neg": -np.ones(3),
            "abs": np.where(x_data > 0, 1.0, np.where(x_data < 0, -1.0, 0.0)),
            "tan": 1.0 / (np.cos(x_data) ** 2), "leaky_relu": np.where(x_data > 0, 1.0, 0.01)}[op]
    if op == "abs":
        close(x.grad.numpy(), want, atol=1e-4)
    else:
        close(x.grad.numpy(), want)
