"""A lazy tensor API over the HIP C-ABI, shaped like the reference's Python `plast.tensor`
(plast/tensor.py: operators build nodes, `plast.forward(t)` runs the DAG, `loss.backward()` seeds a
ones gradient and runs it backwards), so the reference's own test cases can be restated here
against this backend. Output shapes follow plast/tensor.py (broadcast_shape 74-93, reductions
597-659); every value is computed by the library's `<op>_hip_forward/backward` slots through the
graph harness (plast_amd/graph.py)."""
from __future__ import annotations

import numpy as np

from plast_amd import abi
from plast_amd.abi import DIM_ALL, KernelParams
from plast_amd.graph import Graph
from plast_amd.ops import broadcast_shape
from plast_amd.runtime import DeviceTensor, lib

_GRAPH: list[Graph] = []


def _graph() -> Graph:
    if not _GRAPH:
        _GRAPH.append(Graph())
    return _GRAPH[0]


def reset() -> None:
    """A fresh graph (the reference's reset_transient_arenas)."""
    _GRAPH.clear()


class T:
    def __init__(self, dev: DeviceTensor, requires_grad: bool):
        self.dev = dev
        self.requires_grad = requires_grad

    @property
    def shape(self):
        return list(abi.shape_of(self.dev.t))

    @property
    def ndim(self):
        return len(self.shape)

    def numel(self):
        return int(np.prod(self.shape))

    def item(self):
        """tensor.py:299-310: the one element as a Python float."""
        assert self.numel() == 1
        return float(self.numpy().reshape(-1)[0])

    # ---------------------------------------------------------------- construction helpers
    def _op(self, op, inputs, shape, p=None):
        rg = any(x.requires_grad for x in inputs)
        out = DeviceTensor(shape, requires_grad=rg, zero=True)
        _graph().node(op, [x.dev for x in inputs], out, p)
        return T(out, rg)

    def _view_op(self, op, shape, p=None):
        rg = self.requires_grad
        out = DeviceTensor(shape, base=self.dev, zero=False)
        if rg:
            g = DeviceTensor(shape, zero=True)
            out.grad = g
            import ctypes as C
            out.t.grad = C.pointer(g.t)
            out.t.requires_grad = True
        _graph().node(op, [self.dev], out, p)
        return T(out, rg)

    def _bin(self, op, other):
        other = other if isinstance(other, T) else tensor(np.full(1, other, np.float32))
        return self._op(op, [self, other], broadcast_shape(self.shape, other.shape))

    # ---------------------------------------------------------------- arithmetic
    def __add__(self, o): return self._bin("add", o)
    def __sub__(self, o): return self._bin("sub", o)
    def __mul__(self, o): return self._bin("mul", o)
    def __truediv__(self, o): return self._bin("div", o)
    def __neg__(self): return self._op("neg", [self], self.shape)
    def __abs__(self): return self._op("abs", [self], self.shape)
    def exp(self): return self._op("exp", [self], self.shape)
    def log(self): return self._op("log", [self], self.shape)
    def sin(self): return self._op("sin", [self], self.shape)
    def cos(self): return self._op("cos", [self], self.shape)
    def tan(self): return self._op("tan", [self], self.shape)

    def leaky_relu(self, alpha):
        return self._op("leaky_relu", [self], self.shape, KernelParams(0, 0, alpha))

    # ---------------------------------------------------------------- reductions
    def _red(self, op, dim=None, keepdim=False):
        if dim is None:
            return self._op(op, [self], [1], KernelParams(DIM_ALL, 0, 0.0))
        if dim < 0:
            dim += self.ndim
        shape = list(self.shape)
        if keepdim:
            shape[dim] = 1
        else:
            shape.pop(dim)
            shape = shape or [1]
        return self._op(op, [self], shape, KernelParams(dim, int(keepdim), 0.0))

    def sum(self, dim=None, keepdim=False): return self._red("sum", dim, keepdim)
    def mean(self, dim=None, keepdim=False): return self._red("mean", dim, keepdim)
    def max(self, dim=None, keepdim=False): return self._red("max", dim, keepdim)
    def min(self, dim=None, keepdim=False): return self._red("min", dim, keepdim)

    # ---------------------------------------------------------------- shape ops
    def view(self, *shape):
        shape = list(shape)
        if -1 in shape:
            k = shape.index(-1)
            rest = int(np.prod([s for s in shape if s != -1]))
            shape[k] = int(np.prod(self.shape)) // rest
        return self._view_op("view", shape)

    reshape = view

    def transpose(self, d0, d1):
        d0, d1 = d0 % self.ndim, d1 % self.ndim   # tensor.py:716-725
        shape = list(self.shape)
        shape[d0], shape[d1] = shape[d1], shape[d0]
        return self._view_op("transpose", shape, KernelParams(d0, d1, 0.0))

    def squeeze(self, dim=None):
        """tensor.py:758-771: every size-1 axis, or axis `dim` when it has size 1."""
        if dim is None:
            return self._view_op("squeeze", [s for s in self.shape if s != 1] or [1])
        dim = dim % self.ndim
        if self.shape[dim] != 1:
            return self
        shape = list(self.shape)
        shape.pop(dim)
        return self._view_op("squeeze", shape)

    def unsqueeze(self, dim):
        shape = list(self.shape)
        shape.insert(dim, 1)
        return self._view_op("unsqueeze", shape)

    def flatten(self, start, end):
        shape = self.shape
        return self._view_op("flatten", shape[:start] + [int(np.prod(shape[start:end + 1]))]
                             + shape[end + 1:])

    def expand(self, *shape):
        return self._view_op("expand", list(shape))

    # ---------------------------------------------------------------- execution
    def numpy(self) -> np.ndarray:
        return self.dev.numpy()

    @property
    def grad(self):
        return None if self.dev.grad is None else _GradView(self.dev.grad)

    def backward(self):
        """set_ones_grad (src/core/tensor.c:143-152) then the DAG in reverse."""
        L = lib()
        import ctypes as C
        L.set_ones_grad_hip(C.byref(self.dev.t))
        L.check("set_ones_grad_hip")
        _graph().backward()


class _GradView:
    def __init__(self, dev):
        self.dev = dev

    def numpy(self):
        return self.dev.numpy()


def tensor(a, requires_grad=False) -> T:
    return T(DeviceTensor.from_numpy(np.ascontiguousarray(a, np.float32), requires_grad), requires_grad)


# ------------------------------------------------------------- compositions of plast/nn/functional.py
def relu(x: T) -> T:
    """functional.py:24-26."""
    return x.leaky_relu(0.0)


def tanh(x: T) -> T:
    """functional.py:48-54: (e^x - e^-x) / (e^x + e^-x), op by op."""
    ex = x.exp()
    enx = (-x).exp()
    return (ex - enx) / (ex + enx)


def softmax(x: T, dim: int = -1) -> T:
    """functional.py:77-86."""
    shifted = x - x.max(dim=dim, keepdim=True)
    e = shifted.exp()
    return e / e.sum(dim=dim, keepdim=True)


def log_softmax(x: T, dim: int = -1) -> T:
    """functional.py:89-97."""
    shifted = x - x.max(dim=dim, keepdim=True)
    return shifted - shifted.exp().sum(dim=dim, keepdim=True).log()


def _reduce(loss: T, reduction: str) -> T:
    """functional.py:391-396."""
    return loss.mean() if reduction == "mean" else loss.sum() if reduction == "sum" else loss


def mse_loss(pred: T, target: T, reduction: str = "mean") -> T:
    """functional.py:279-284."""
    d = pred - target
    return _reduce(d * d, reduction)


def l1_loss(pred: T, target: T, reduction: str = "mean") -> T:
    """functional.py:287-291."""
    return _reduce(abs(pred - target), reduction)


def cross_entropy(logits: T, labels: np.ndarray, reduction: str = "mean") -> T:
    """functional.py:312-333 with class indices: a dense one-hot built on the host, then
    -(onehot * log_softmax(x, 1)).sum(1), reduced."""
    n, c = logits.shape
    onehot = np.zeros((n, c), np.float32)
    onehot[np.arange(n), labels] = 1.0
    loss = -(tensor(onehot) * log_softmax(logits, dim=1)).sum(dim=1)
    return _reduce(loss, reduction)


def forward(t: T) -> None:
    g = _graph()
    g.build(t.dev)
    g.forward()
