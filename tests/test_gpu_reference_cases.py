"""The reference's own pytest cases for this path, restated against the HIP backend.

Each case keeps the reference test's inputs (np.random.RandomState(42) per test, as its `rng`
fixture: tests/conftest.py:56-58), its op sequence and its numpy closed form, and its tolerance
(rtol 1e-3 / atol 1e-4: conftest.py:5-6; exp at atol 1e-3). Sources:
tests/test_ops.py:18-189, 205-287, 407-433 (elementwise, reductions, shape ops, leaky relu, ops with
gradients) and tests/test_gradients.py:20-188 (autograd basics and per-op gradients), tests/test_edge_cases.py:6-147
(small shapes, broadcasts, op chains, view ops) and tests/test_nn.py:35-110 (activations and losses
composed of these ops: plast/nn/functional.py) and tests/test_optim.py:22-112 (the optimizer steps
whose gradients come from these ops). Matmul, conv and Linear cases are out of this path. The expressions run through reference_api, which builds the DAG
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


# ------------------------------------------------------------------ test_edge_cases.py
def test_single_element_tensor(P):
    a = P.tensor(np.array([42.0], dtype=np.float32))
    assert a.item() == 42.0 and a.shape == [1] and a.numel() == 1


def test_scalar_arithmetic(P):
    c = P.tensor(np.array([3.0], np.float32)) + P.tensor(np.array([2.0], np.float32))
    P.forward(c)
    close(c.numpy(), [5.0])


def test_large_tensor_creation_and_high_dim(P, rng):
    a = P.tensor(np.zeros((100, 100), np.float32))
    assert a.shape == [100, 100] and a.numel() == 10000
    b = P.tensor(rng.randn(2, 3, 4, 5).astype(np.float32))
    assert b.ndim == 4 and b.shape == [2, 3, 4, 5]


@pytest.mark.parametrize("sa, sb", [((3, 1), (1, 4)), ((4, 1), (1, 4))])
def test_broadcast_add_outer(P, rng, sa, sb):
    a, b = rng.randn(*sa).astype(np.float32), rng.randn(*sb).astype(np.float32)
    c = P.tensor(a) + P.tensor(b)
    P.forward(c)
    close(c.numpy(), a + b)


def test_multiple_ops_chain(P, rng):
    """(a + b) * c -> sin -> sum, backward; the reference checks the grads exist, the closed forms
    pin them: d/da = d/db = cos((a+b)c) c, d/dc = cos((a+b)c) (a+b)."""
    a, b, c = (rng.randn(2, 3).astype(np.float32) for _ in range(3))
    ta, tb, tc = (P.tensor(x, True) for x in (a, b, c))
    loss = ((ta + tb) * tc).sin().sum()
    P.forward(loss)
    loss.backward()
    s = (a + b).astype(np.float32)
    g = np.cos(s * c)
    close(ta.grad.numpy(), g * c)
    close(tb.grad.numpy(), g * c)
    close(tc.grad.numpy(), g * s)


def test_grad_non_requires_grad_input(P, rng):
    a = P.tensor(rng.randn(3).astype(np.float32), True)
    b = P.tensor(rng.randn(3).astype(np.float32), False)
    loss = (a + b).sum()
    P.forward(loss)
    loss.backward()
    assert a.grad is not None and b.grad is None
    close(a.grad.numpy(), np.ones(3))


def test_tensor_arithmetic_chain(P, rng):
    a, b, c = (rng.randn(2, 3).astype(np.float32) for _ in range(3))
    one = np.ones((2, 3), np.float32)
    ta, tb, tc, to = (P.tensor(x) for x in (a, b, c, one))
    d = (ta + tb) * tc - ta / (tb + to)
    P.forward(d)
    close(d.numpy(), (a + b) * c - a / (b + 1.0))


def test_unsqueeze_chain(P, rng):
    a = rng.randn(3).astype(np.float32)
    tb = P.tensor(a).unsqueeze(0).unsqueeze(2)
    P.forward(tb)
    assert tb.shape == [1, 3, 1]
    close(tb.numpy(), a[np.newaxis, :, np.newaxis])


def test_squeeze_all_and_dim(P, rng):
    a = rng.randn(1, 3, 1, 4, 1).astype(np.float32)
    tb = P.tensor(a).squeeze()
    P.forward(tb)
    close(tb.numpy(), a.reshape(3, 4))
    a2 = rng.randn(1, 3, 1, 4).astype(np.float32)
    tc = P.tensor(a2).squeeze(dim=0)
    P.forward(tc)
    assert tc.shape == [3, 1, 4]
    close(tc.numpy(), a2.reshape(3, 1, 4))


@pytest.mark.parametrize("dims", [(-2, -1), (1, 2)])
def test_transpose_last_two(P, rng, dims):
    a = rng.randn(2, 3, 4).astype(np.float32)
    tb = P.tensor(a).transpose(*dims)
    P.forward(tb)
    close(tb.numpy(), np.transpose(a, (0, 2, 1)))


def test_view_then_op(P, rng):
    a = rng.randn(2, 6).astype(np.float32)
    b = rng.randn(4).astype(np.float32)
    tc = P.tensor(a).view(3, 4) + P.tensor(b)
    P.forward(tc)
    close(tc.numpy(), a.reshape(3, 4) + b)


# ------------------------------------------------------------------ test_nn.py: activations, losses
def test_relu_forward(P, rng):
    x = rng.randn(2, 3).astype(np.float32)
    out = P.relu(P.tensor(x))
    P.forward(out)
    close(out.numpy(), np.maximum(x, 0))


def test_tanh_forward(P, rng):
    x = rng.randn(2, 3).astype(np.float32)
    out = P.tanh(P.tensor(x))
    P.forward(out)
    close(out.numpy(), np.tanh(x), atol=1e-3)


def test_leaky_relu_module(P, rng):
    x = rng.randn(2, 3).astype(np.float32)
    out = P.tensor(x).leaky_relu(0.02)
    P.forward(out)
    close(out.numpy(), np.where(x > 0, x, 0.02 * x))


def test_softmax(P, rng):
    x = rng.randn(2, 4).astype(np.float32)
    out = P.softmax(P.tensor(x), dim=1)
    P.forward(out)
    close(out.numpy(), np.exp(x) / np.sum(np.exp(x), axis=1, keepdims=True))


@pytest.mark.parametrize("reduction", ["mean", "sum"])
def test_mse_loss(P, rng, reduction):
    pred, target = rng.randn(4, 1).astype(np.float32), rng.randn(4, 1).astype(np.float32)
    loss = P.mse_loss(P.tensor(pred), P.tensor(target), reduction)
    P.forward(loss)
    d = pred - target
    close(loss.numpy(), np.array([np.mean(d ** 2) if reduction == "mean" else np.sum(d ** 2)]))


def test_l1_loss(P, rng):
    pred, target = rng.randn(4, 1).astype(np.float32), rng.randn(4, 1).astype(np.float32)
    loss = P.l1_loss(P.tensor(pred), P.tensor(target))
    P.forward(loss)
    close(loss.numpy(), np.array([np.mean(np.abs(pred - target))]))


def test_cross_entropy_loss(P, rng):
    """The composed chain (functional.py:312-333) at the reference's atol 1e-2, and the fused
    softmax_cross_entropy op's mean row loss on the same logits."""
    from plast_amd import ops, runtime as rt
    logits = rng.randn(3, 5).astype(np.float32)
    labels = np.array([0, 2, 4], dtype=np.int32)
    loss = P.cross_entropy(P.tensor(logits), labels)
    P.forward(loss)
    e = np.exp(logits - logits.max(1, keepdims=True))
    sm = e / e.sum(1, keepdims=True)
    want = -np.mean(np.log(sm[np.arange(3), labels] + 1e-8))
    close(loss.numpy(), np.array([want]), atol=1e-2)
    rows, _ = ops.softmax_cross_entropy(rt.DeviceTensor.from_numpy(logits),
                                        rt.DeviceTensor.from_numpy(labels))
    close(np.array([rows.numpy().mean()]), loss.numpy(), rtol=1e-5, atol=1e-6)


# ------------------------------------------------------------------ test_optim.py: in-path cases
# The reference's optimizer tests whose gradients come from this path's ops (its matmul-based
# ones and the host-only learning-rate schedulers are off the path), stepped through
# sgd/adam/adamw_step_hip and zero_grad_hip, each also checked against the update's closed form
# (src/optimizers/cpu/sgd.c:25, adam.c:48-49, 63-65, adamw.c:130).
def _step(kind, opt, params):
    import ctypes as C
    from plast_amd import abi
    from plast_amd.runtime import lib
    L = lib()
    ptrs, keep = abi.tensor_array(*[p.dev.t for p in params])
    getattr(L, f"{kind}_step_hip")(C.byref(opt), ptrs, len(params))
    L.check(f"{kind}_step_hip")


def _release(kind, opt, n):
    import ctypes as C
    from plast_amd.runtime import lib
    getattr(lib(), f"plast_hip_{kind}_release")(C.byref(opt), n)


def _adam_closed_form(p, grads, lr, b1, b2, eps, wd=0.0):
    """The reference's update in float64, one gradient per step."""
    p = p.astype(np.float64)
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    for t, g in enumerate(grads, start=1):
        g = g.astype(np.float64)
        p = p - lr * wd * p
        m = b1 * m + (1 - b1) * g
        v = b2 * v + (1 - b2) * g * g
        lr_t = lr * np.sqrt(1 - b2 ** t) / (1 - b1 ** t)
        p = p - lr_t * m / (np.sqrt(v) + eps)
    return p


def test_sgd_multiple_params(P, rng):
    """test_optim.py:36-54: (w1 * x * w2).sum(), one SGD step over both parameters."""
    from plast_amd import abi
    w1n, w2n, xn = (rng.randn(3).astype(np.float32) for _ in range(3))
    w1, w2, x = P.tensor(w1n, True), P.tensor(w2n, True), P.tensor(xn)
    y = (w1 * x * w2).sum()
    P.forward(y)
    y.backward()
    g1, g2 = w1.grad.numpy().copy(), w2.grad.numpy().copy()
    close(g1, xn * w2n)
    close(g2, w1n * xn)
    lr = 0.05
    _step("sgd", abi.SGD(lr), [w1, w2])
    close(w1.numpy(), w1n - lr * g1)
    close(w2.numpy(), w2n - lr * g2)


def test_sgd_zero_grad(P, rng):
    """test_optim.py:22-34: gradients are zero after zero_grad (the reference's matmul loss
    replaced by (w * x).sum())."""
    import ctypes as C
    from plast_amd.runtime import lib
    w = P.tensor(rng.randn(2, 3).astype(np.float32), True)
    x = P.tensor(rng.randn(2, 3).astype(np.float32))
    y = (w * x).sum()
    P.forward(y)
    y.backward()
    assert np.abs(w.grad.numpy()).max() > 0
    lib().zero_grad_hip(C.byref(w.dev.t))
    lib().check("zero_grad_hip")
    assert np.all(w.grad.numpy() == 0)


def test_adam_multiple_steps(P, rng):
    """test_optim.py:70-84: five steps of zero_grad, (w * x).sum() with x = 1, backward, step;
    every gradient is 1, so w follows the closed-form update."""
    import ctypes as C
    from plast_amd import abi
    from plast_amd.runtime import lib
    w0 = rng.randn(3).astype(np.float32)
    w = P.tensor(w0, True)
    x = P.tensor(np.ones(3, dtype=np.float32))
    lr, b1, b2, eps = 0.01, 0.9, 0.999, 1e-8
    opt = abi.Adam(lr, b1, b2, eps, 0, None, None, None, None)
    try:
        for _ in range(5):
            lib().zero_grad_hip(C.byref(w.dev.t))
            y = (w * x).sum()
            P.forward(y)
            y.backward()
            close(w.grad.numpy(), np.ones(3, np.float32))
            _step("adam", opt, [w])
            P.reset()
        assert w.grad is not None
        close(w.numpy(), _adam_closed_form(w0, [np.ones(3)] * 5, lr, b1, b2, eps),
              rtol=1e-5, atol=1e-6)
    finally:
        _release("adam", opt, 1)


def test_adamw_weight_decay(P):
    """test_optim.py:101-112: w = [2, 2], (w * w).sum() (the tensor used twice: gradient 2w),
    one AdamW step with lr 0.1 and weight decay 0.1."""
    from plast_amd import abi
    w0 = np.array([2.0, 2.0], dtype=np.float32)
    w = P.tensor(w0, True)
    y = (w * w).sum()
    P.forward(y)
    y.backward()
    close(w.grad.numpy(), 2 * w0)
    lr, b1, b2, eps, wd = 0.1, 0.9, 0.999, 1e-8, 0.1
    opt = abi.AdamW(lr, b1, b2, eps, wd, 0, None, None, None, None)
    try:
        _step("adamw", opt, [w])
        got = w.numpy()
        assert not np.allclose(got, w0)
        close(got, _adam_closed_form(w0, [2 * w0], lr, b1, b2, eps, wd), rtol=1e-5, atol=1e-6)
    finally:
        _release("adamw", opt, 1)
