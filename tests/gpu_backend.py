"""Runs tests/cases.py cases through the HIP library (device tensors, C-ABI entry points)."""
from __future__ import annotations

import ctypes as C

import numpy as np

from cases import Backend
from plast_amd import abi
from plast_amd.abi import FLOAT32, INT64
from plast_amd.runtime import DeviceTensor, backward, forward, lib


class DeviceBackend(Backend):
    def __init__(self):
        self.keep = []

    def tensor(self, arr, requires_grad):
        t = DeviceTensor.from_numpy(np.ascontiguousarray(arr), requires_grad)
        self.keep.append(t)
        return t

    def view(self, base, shape, strides, own_grad=False):
        v = DeviceTensor(shape, base.dtype, base=base, strides=strides, zero=False)
        v.t.requires_grad = base.t.requires_grad
        if base.grad is not None:
            if own_grad:
                # a zero-filled gradient of its own, contiguous in the view's shape
                g = DeviceTensor(shape, base.dtype, zero=True)
            else:
                g = DeviceTensor(shape, base.dtype, base=base.grad, strides=strides, zero=False)
            self.keep.append(g)
            v.grad = g
            v.t.grad = C.pointer(g.t)
        self.keep.append(v)
        return v

    def empty(self, shape, dtype, requires_grad=False):
        t = DeviceTensor(shape, INT64 if dtype == "i64" else FLOAT32, requires_grad)
        self.keep.append(t)
        return t

    def fwd(self, op, ins, out, p):
        forward(op, ins, out, p)

    def bwd(self, op, ins, out, p):
        backward(op, ins, out, p)

    def read(self, t):
        return t.numpy()

    def read_grad(self, t):
        return t.grad.numpy()

    def set_grad(self, t, arr):
        a = np.ascontiguousarray(arr, dtype=np.float32)
        assert a.size == self.grad_size(t), "set_grad writes the whole gradient buffer"
        lib().arena_memcpy_h2d_hip(t.grad.ptr, a.ctypes.data, a.nbytes)
        lib().check("set_grad")

    def grad_size(self, t):
        return int(np.prod(t.grad.shape))


def ulp_distance(x: np.ndarray, y: np.ndarray) -> np.ndarray:
    """|ordinal(x) - ordinal(y)| for float32 (0 where both NaN or both equal, inf where one NaN)."""
    x = np.asarray(x, np.float32)
    y = np.asarray(y, np.float32)

    def ordinal(v):
        i = v.view(np.int32).astype(np.int64)
        return np.where(i < 0, -(i & 0x7FFFFFFF), i)

    d = np.abs(ordinal(x) - ordinal(y)).astype(np.float64)
    xn, yn = np.isnan(x), np.isnan(y)
    d[xn & yn] = 0
    d[xn ^ yn] = np.inf
    return d
