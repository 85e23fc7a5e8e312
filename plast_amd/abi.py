"""ctypes mirror of the boundary structs declared in include/plast_abi.h.

The same `Tensor` structure is handed to the HIP library, the oracle and the compiled reference,
so one calling convention serves all three (the reference's ForwardKernel / BackwardKernel,
include/core/op.h:5-6).
"""
from __future__ import annotations

import ctypes as C

MAX_NDIM = 8
DIM_ALL = MAX_NDIM + 1  # reduce over every element (src/kernels/cpu/reduce_ops.c:69)

# DTYPE (include/core/tensor.h:8, INT64 appended)
INT32, FLOAT32, INT64 = 0, 1, 2
# DEVICE (include/core/arena.h:16)
CPU, GPU = 0, 1

# OP_TYPE (include/core/op.h:8-37, extensions appended)
OP_NAMES = [
    "ADD", "SUB", "MUL", "DIV", "MATMUL", "LEAKY_RELU", "LOG", "EXP", "ABS", "NEG", "SIN", "COS",
    "TAN", "VIEW", "TRANSPOSE", "UNSQUEEZE", "SQUEEZE", "EXPAND", "FLATTEN", "BROADCAST", "MEAN",
    "MIN", "MAX", "SUM", "CONV2D", "MATMUL_RELU", "MATMUL_BIAS_RELU", "CONV_RELU",
    "ARGMAX", "FUSED_ELEMENTWISE", "SOFTMAX_CROSS_ENTROPY", "SOFTMAX", "LOG_SOFTMAX",
]
OP = {name: i for i, name in enumerate(OP_NAMES)}

# PlastTapeOp / PlastTapeSrc (include/plast_hip.h)
TAPE_OPS = ["LOAD", "ADD", "SUB", "MUL", "DIV", "LEAKY_RELU", "EXP", "LOG", "NEG", "ABS", "SIN",
            "COS", "TAN"]
TAPE = {name: i for i, name in enumerate(TAPE_OPS)}
SRC_NONE, SRC_INPUT, SRC_ACC, SRC_IMM = 0, 1, 2, 3
TAPE_MAX_INS = 16
TAPE_MAX_INPUTS = 4


class Tensor(C.Structure):
    pass


Tensor._fields_ = [
    ("grad", C.POINTER(Tensor)),
    ("creator", C.c_void_p),
    ("data", C.c_void_p),
    ("shape", C.c_uint64 * MAX_NDIM),
    ("strides", C.c_uint64 * MAX_NDIM),
    ("ndim", C.c_uint64),
    ("dtype", C.c_int),
    ("device", C.c_int),
    ("requires_grad", C.c_bool),
]


class KernelParams(C.Structure):
    _fields_ = [("dim", C.c_uint64), ("keepdim", C.c_uint64), ("fval", C.c_float)]


TensorP = C.POINTER(Tensor)
TensorPP = C.POINTER(TensorP)
ForwardKernel = C.CFUNCTYPE(None, TensorPP, TensorP, KernelParams)
BackwardKernel = C.CFUNCTYPE(None, TensorPP, TensorP, KernelParams)


class Op(C.Structure):
    _fields_ = [
        ("cpu_forward", C.c_void_p),
        ("gpu_forward", C.c_void_p),
        ("cpu_backward", C.c_void_p),
        ("gpu_backward", C.c_void_p),
    ]


class ArenaBlock(C.Structure):
    pass


ArenaBlock._fields_ = [
    ("prev", C.POINTER(ArenaBlock)),
    ("capacity", C.c_uint64),
    ("offset", C.c_uint64),
    ("buffer", C.c_void_p),
]


class Arena(C.Structure):
    _fields_ = [("current", C.POINTER(ArenaBlock)), ("device", C.c_int)]


class Node(C.Structure):
    _fields_ = [
        ("inputs", TensorPP),
        ("output", TensorP),
        ("op", Op),
        ("op_type", C.c_int),
        ("num_inputs", C.c_int),
        ("visited", C.c_bool),
        ("on_stack", C.c_bool),
        ("params", KernelParams),
    ]


class DAG(C.Structure):
    _fields_ = [
        ("nodes", C.POINTER(C.POINTER(Node))),
        ("count", C.c_uint32),
        ("capacity", C.c_uint32),
        ("changed", C.c_bool),
        ("arena", C.POINTER(Arena)),
    ]


class TapeIns(C.Structure):
    _fields_ = [("op", C.c_uint8), ("src", C.c_uint8), ("idx", C.c_uint8), ("acc_rhs", C.c_uint8),
                ("imm", C.c_float)]


class FusedTape(C.Structure):
    _fields_ = [("num_inputs", C.c_uint32), ("num_ins", C.c_uint32),
                ("ins", TapeIns * TAPE_MAX_INS)]


ArenaAllocFn = C.CFUNCTYPE(C.c_void_p, C.POINTER(Arena), C.c_uint64, C.c_uint64)


# Contiguous image of a possibly strided tensor (include/kernels/pack.h:17-20 CudaTensorPack)
class HipTensorPack(C.Structure):
    _fields_ = [("data", C.c_void_p), ("_d_buf", C.c_void_p)]


# Optimizer state (include/optimizers/sgd.h:5-7, adam.h:5-15, adamw.h:5-16)
class SGD(C.Structure):
    _fields_ = [("lr", C.c_float)]


class Adam(C.Structure):
    _fields_ = [("lr", C.c_float), ("beta1", C.c_float), ("beta2", C.c_float),
                ("epsilon", C.c_float), ("t", C.c_int), ("m", TensorPP), ("v", TensorPP),
                ("data_arena", C.POINTER(Arena)), ("optimizer_arena", C.POINTER(Arena))]


class AdamW(C.Structure):
    _fields_ = [("lr", C.c_float), ("beta1", C.c_float), ("beta2", C.c_float),
                ("epsilon", C.c_float), ("weight_decay", C.c_float), ("t", C.c_int),
                ("m", TensorPP), ("v", TensorPP), ("data_arena", C.POINTER(Arena)),
                ("optimizer_arena", C.POINTER(Arena))]


def params(dim: int = 0, keepdim: int = 0, fval: float = 0.0) -> KernelParams:
    return KernelParams(dim, keepdim, fval)


def row_major(shape) -> list[int]:
    st, s = [0] * len(shape), 1
    for d in range(len(shape) - 1, -1, -1):
        st[d] = s
        s *= shape[d]
    return st


def make_tensor(data_ptr: int, shape, strides=None, dtype: int = FLOAT32, device: int = GPU,
                requires_grad: bool = False, grad: Tensor | None = None) -> Tensor:
    t = Tensor()
    shape = list(shape)
    strides = row_major(shape) if strides is None else list(strides)
    if len(shape) > MAX_NDIM:
        raise ValueError(f"rank {len(shape)} exceeds MAX_NDIM={MAX_NDIM}")
    t.data = data_ptr
    t.ndim = len(shape)
    for d, (n, s) in enumerate(zip(shape, strides)):
        t.shape[d] = n
        t.strides[d] = s
    t.dtype = dtype
    t.device = device
    t.requires_grad = requires_grad
    if grad is not None:
        t.grad = C.pointer(grad)
    return t


def shape_of(t: Tensor) -> tuple[int, ...]:
    return tuple(t.shape[d] for d in range(t.ndim))


def strides_of(t: Tensor) -> tuple[int, ...]:
    return tuple(t.strides[d] for d in range(t.ndim))


def tensor_array(*ts: Tensor):
    """A `Tensor **` holding pointers to the given structs (kept alive by the caller)."""
    arr = (TensorP * len(ts))(*[C.pointer(t) for t in ts])
    return C.cast(arr, TensorPP), arr
