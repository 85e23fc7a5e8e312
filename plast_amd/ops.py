"""Functional layer over the HIP entry points, shaped like the reference's Python `Tensor` methods
(plast/tensor.py): it computes output shapes the same way, allocates the output and calls the op.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import abi
from .abi import DIM_ALL, FLOAT32, INT32, INT64, KernelParams
from .runtime import DeviceTensor, backward, forward, lib


def broadcast_shape(s1, s2) -> tuple[int, ...]:
    """numpy broadcasting, raising on incompatible shapes (plast/tensor.py:74-93)."""
    n = max(len(s1), len(s2))
    out = []
    for i in range(n):
        a = s1[len(s1) - 1 - i] if i < len(s1) else 1
        b = s2[len(s2) - 1 - i] if i < len(s2) else 1
        if a != b and a != 1 and b != 1:
            raise ValueError(f"shapes {tuple(s1)} and {tuple(s2)} are not broadcastable")
        out.append(max(a, b))
    return tuple(reversed(out))


def binary(name: str, a: DeviceTensor, b: DeviceTensor, requires_grad: bool = False) -> DeviceTensor:
    out = DeviceTensor(broadcast_shape(abi.shape_of(a.t), abi.shape_of(b.t)), FLOAT32,
                       requires_grad, zero=False)
    forward(name, [a, b], out)
    return out


def unary(name: str, a: DeviceTensor, alpha: float = 0.0, requires_grad: bool = False) -> DeviceTensor:
    out = DeviceTensor(abi.shape_of(a.t), FLOAT32, requires_grad, zero=False)
    forward(name, [a], out, KernelParams(0, 0, alpha))
    return out


def reduced_shape(shape, dim, keepdim) -> tuple[int, ...]:
    """Output shape of a reduction (plast/tensor.py:597-659)."""
    if dim is None:
        return (1,)
    out = list(shape)
    if keepdim:
        out[dim] = 1
    else:
        out.pop(dim)
        if not out:
            out = [1]
    return tuple(out)


def reduce(name: str, a: DeviceTensor, dim=None, keepdim: bool = False,
           requires_grad: bool = False) -> DeviceTensor:
    shape = abi.shape_of(a.t)
    if dim is not None and dim < 0:
        dim += len(shape)
    dt = INT64 if name == "argmax" else FLOAT32
    out = DeviceTensor(reduced_shape(shape, dim, keepdim), dt, requires_grad, zero=False)
    forward(name, [a], out, KernelParams(DIM_ALL if dim is None else dim, int(keepdim), 0.0))
    return out


def transpose(a: DeviceTensor, d0: int, d1: int) -> DeviceTensor:
    """A view with two axes swapped (shape_ops.c:59-80), sharing a's buffer."""
    v = DeviceTensor(abi.shape_of(a.t), a.dtype, base=a.base or a, zero=False)
    v.t.data = a.t.data
    forward("transpose", [a], v, KernelParams(d0, d1, 0.0))
    v.shape = abi.shape_of(v.t)
    return v


def permute(a: DeviceTensor, dims) -> DeviceTensor:
    """As a sequence of transposes, the way plast/tensor.py:730-756 builds it."""
    cur = list(range(len(dims)))
    res = a
    for target, orig in enumerate(dims):
        pos = cur.index(orig)
        if pos != target:
            res = transpose(res, pos, target)
            cur[pos], cur[target] = cur[target], cur[pos]
    return res


def expand(a: DeviceTensor, shape) -> DeviceTensor:
    v = DeviceTensor(tuple(shape), a.dtype, base=a.base or a, zero=False)
    forward("expand", [a], v)
    return v


def softmax_cross_entropy(logits: DeviceTensor, labels: DeviceTensor, requires_grad: bool = False):
    """Per-row loss [N] and stats [N, 2] (row max, log exp-sum)."""
    n = abi.shape_of(logits.t)[0]
    stats = DeviceTensor((n, 2), FLOAT32, zero=False)
    loss = DeviceTensor((n,), FLOAT32, requires_grad, zero=False)
    forward("softmax_cross_entropy", [logits, labels, stats], loss)
    return loss, stats


def make_tape(instructions, num_inputs: int) -> abi.FusedTape:
    """instructions: list of (op_name, src, idx, acc_rhs, imm)."""
    tape = abi.FusedTape()
    tape.num_inputs = num_inputs
    tape.num_ins = len(instructions)
    for i, (op, src, idx, rhs, imm) in enumerate(instructions):
        tape.ins[i] = abi.TapeIns(abi.TAPE[op], src, idx, rhs, imm)
    return tape


def fused(tape: abi.FusedTape, inputs, shape) -> DeviceTensor:
    out = DeviceTensor(tuple(shape), FLOAT32, zero=False)
    forward("fused_elementwise", inputs, out,
            KernelParams(C.addressof(tape), 0, 0.0))
    return out


__all__ = ["binary", "unary", "reduce", "transpose", "permute", "expand", "softmax_cross_entropy",
           "make_tape", "fused", "broadcast_shape", "reduced_shape", "backward", "forward", "lib",
           "DeviceTensor", "np", "INT32"]
