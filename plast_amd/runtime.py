"""Loader for libplast_hip.so and a small device-tensor wrapper over its C-ABI.

This is host plumbing (the role the reference's pybind11 bindings play for its CUDA slots,
src/python/bindings.cpp:43-374): it allocates device buffers through the library's arena hooks,
builds `Tensor` structs and calls the `<op>_hip_forward/backward` entry points. All arithmetic runs
in the HIP kernels; there is no CPU fallback: if the library is not built, `lib()` raises.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

from . import abi
from .abi import FLOAT32, GPU, INT32, INT64, KernelParams, Tensor, TensorP, TensorPP

LIB_PATH = Path(__file__).resolve().parent / "libplast_hip.so"

_NP_DTYPE = {FLOAT32: np.float32, INT32: np.int32, INT64: np.int64}
_DT_OF_NP = {np.dtype(np.float32): FLOAT32, np.dtype(np.int32): INT32, np.dtype(np.int64): INT64}

OP_NAMES = ["add", "sub", "mul", "div", "exp", "log", "neg", "abs", "sin", "cos", "tan",
            "leaky_relu", "sum", "mean", "max", "min", "argmax", "view", "flatten", "squeeze",
            "unsqueeze", "expand", "broadcast", "transpose", "fused_elementwise",
            "softmax_cross_entropy", "softmax", "log_softmax"]


class PlastHipError(RuntimeError):
    pass


class Library:
    def __init__(self, path: Path = LIB_PATH):
        if not Path(path).exists():
            raise PlastHipError(
                f"{path} is not built; run `python -m plast_amd.build` (no CPU fallback exists)")
        self.path = str(path)
        L = C.CDLL(self.path)
        self._L = L
        # (kind, op name) -> bound entry point, looked up once: the per-call path does no
        # attribute lookups or string formatting
        self.entry = {}
        for name in OP_NAMES:
            for kind in ("forward", "backward"):
                f = getattr(L, f"{name}_hip_{kind}")
                f.argtypes, f.restype = [TensorPP, TensorP, KernelParams], None
                self.entry[kind, name] = f
        sig = {
            "plast_hip_init": ([C.c_int], C.c_int),
            "plast_hip_set_sync": ([C.c_int], None),
            "plast_hip_set_deterministic": ([C.c_int], None),
            "plast_hip_deterministic": ([], C.c_int),
            "plast_hip_synchronize": ([], C.c_int),
            "plast_hip_capture_begin": ([], C.c_int),
            "plast_hip_capture_end": ([], C.c_void_p),
            "plast_hip_graph_launch": ([C.c_void_p], C.c_int),
            "plast_hip_graph_destroy": ([C.c_void_p], None),
            "plast_hip_workspace_reserve": ([C.c_int, C.c_uint64], C.c_int),
            "plast_hip_workspace_bytes": ([C.c_int], C.c_uint64),
            "plast_hip_graphs_alive": ([], C.c_int),
            "plast_hip_workspace_retired": ([], C.c_int),
            "plast_hip_stream": ([], C.c_void_p),
            "plast_hip_error_count": ([], C.c_int),
            "plast_hip_last_error": ([], C.c_char_p),
            "plast_hip_clear_error": ([], None),
            "plast_hip_timer_begin": ([], C.c_int),
            "plast_hip_timer_end": ([], C.c_float),
            "plast_hip_fill_uniform": ([C.c_void_p, C.c_uint64, C.c_uint64, C.c_float, C.c_float], None),
            "plast_hip_fill_normal": ([C.c_void_p, C.c_uint64, C.c_uint64, C.c_float, C.c_float], None),
            "plast_hip_fill_randint": ([C.c_void_p, C.c_uint64, C.c_uint64, C.c_int32, C.c_int32], None),
            "plast_hip_copy": ([C.c_void_p, C.c_void_p, C.c_uint64], None),
            "plast_hip_get_op_impl": ([C.c_int], abi.Op),
            "plast_hip_fuse_elementwise_chains": ([C.POINTER(abi.DAG), abi.ArenaAllocFn], C.c_uint32),
            "sgd_step_hip": ([C.POINTER(abi.SGD), TensorPP, C.c_int], None),
            "adam_step_hip": ([C.POINTER(abi.Adam), TensorPP, C.c_int], None),
            "adamw_step_hip": ([C.POINTER(abi.AdamW), TensorPP, C.c_int], None),
            "zero_grad_hip": ([TensorP], None),
            "plast_hip_adam_release": ([C.POINTER(abi.Adam), C.c_int], None),
            "plast_hip_adamw_release": ([C.POINTER(abi.AdamW), C.c_int], None),
            "hip_tensor_pack_init": ([C.POINTER(abi.HipTensorPack), TensorP], None),
            "hip_tensor_pack_release": ([C.POINTER(abi.HipTensorPack)], None),
            "plast_hip_tensor_to_host": ([TensorP, C.c_void_p], C.c_int),
            "plast_hip_tensor_from_host": ([TensorP, C.c_void_p], C.c_int),
            "plast_hip_pack_trim": ([], None),
            "launch_relu_grad_modulate_hip": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64,
                                               C.c_float, C.c_int, C.c_int], None),
            "bias_grad_reduce_hip": ([C.c_void_p, C.c_void_p, C.c_uint64, C.c_uint64], None),
            "softmax_cross_entropy_step_hip": ([C.c_void_p] * 8 + [C.c_uint64, C.c_uint64], None),
            "softmax_cross_entropy_step_noalloc_hip": ([C.c_void_p] * 8 + [C.c_uint64, C.c_uint64],
                                                       None),
            "relu_grad_modulate_bias_grad_hip": ([C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                                  C.c_uint64, C.c_uint64, C.c_float], None),
            "plast_hip_host_alloc": ([C.c_uint64], C.c_void_p),
            "plast_hip_host_free": ([C.c_void_p], None),
            "arena_alloc_hip": ([C.c_uint64], C.c_void_p),
            "arena_free_hip": ([C.c_void_p], None),
            "arena_memset_hip": ([C.c_void_p, C.c_int, C.c_uint64], None),
            "arena_memcpy_h2d_hip": ([C.c_void_p, C.c_void_p, C.c_uint64], None),
            "arena_memcpy_d2h_hip": ([C.c_void_p, C.c_void_p, C.c_uint64], None),
            "arena_memcpy_d2d_hip": ([C.c_void_p, C.c_void_p, C.c_uint64], None),
            "zeros_hip": ([TensorP, C.c_uint64], None),
            "ones_hip": ([TensorP, C.c_uint64], None),
            "set_ones_grad_hip": ([TensorP], None),
            "reshape_backward_hip": ([C.c_void_p, C.c_void_p, C.c_uint64], None),
            "transpose_backward_hip": ([C.c_void_p, C.c_void_p, C.POINTER(C.c_uint64),
                                        C.POINTER(C.c_uint64), C.POINTER(C.c_uint64), C.c_uint64,
                                        C.c_uint64, C.c_uint64, C.c_uint64], None),
        }
        for name, (args, res) in sig.items():
            f = getattr(L, name)
            f.argtypes, f.restype = args, res
        self.error_count = L.plast_hip_error_count

    def __getattr__(self, name):
        return getattr(self._L, name)

    def check(self, what: str = "") -> None:
        """Raise if the library reported an error since the last check."""
        if self.error_count():
            self.raise_error(what)

    def raise_error(self, what: str = "") -> None:
        msg = self._L.plast_hip_last_error().decode()
        self._L.plast_hip_clear_error()
        raise PlastHipError(f"{what}: {msg}" if what else msg)


_LIB: Library | None = None


def lib() -> Library:
    global _LIB
    if _LIB is None:
        _LIB = Library(Path(os.environ.get("PLAST_HIP_LIB", LIB_PATH)))
        if _LIB.plast_hip_init(int(os.environ.get("PLAST_HIP_DEVICE", "0"))) != 0:
            _LIB.check("plast_hip_init")
    return _LIB


def load_library(path: Path) -> Library:
    """Another build of the library (a variant built with `plast_amd.build --out`), loaded beside
    the current one and initialised on the same device. Each build keeps its own state (stream,
    workspaces, errors); device memory is the process's, so tensors allocated through one build
    can be passed to another's entry points."""
    L = Library(Path(path))
    if L.plast_hip_init(int(os.environ.get("PLAST_HIP_DEVICE", "0"))) != 0:
        L.check("plast_hip_init")
    return L


def use_library(L: Library) -> Library:
    """Make lib() return L from now on (for timing builds against each other in one process);
    returns the build it replaces."""
    global _LIB
    prev = lib()
    _LIB = L
    return prev


def _row_major(shape) -> tuple[int, ...]:
    st, acc = [], 1
    for e in reversed(shape):
        st.append(acc)
        acc *= e
    return tuple(reversed(st))


class DeviceTensor:
    """A device allocation plus the `Tensor` struct that describes it (host metadata)."""

    def __init__(self, shape, dtype: int = FLOAT32, requires_grad: bool = False, *,
                 strides=None, base: "DeviceTensor | None" = None, offset: int = 0,
                 zero: bool = True):
        L = lib()
        self.shape = tuple(int(s) for s in shape)
        self.dtype = dtype
        self.itemsize = np.dtype(_NP_DTYPE[dtype]).itemsize
        n = int(np.prod(self.shape)) if self.shape else 1
        self.base = base
        if base is None:
            self.nbytes = n * self.itemsize
            self.ptr = L.arena_alloc_hip(max(self.nbytes, 1))
            self._own = True
        else:
            self.nbytes = base.nbytes
            self.ptr = base.ptr + offset * self.itemsize
            self._own = False
        self.grad: DeviceTensor | None = None
        if requires_grad:
            self.grad = DeviceTensor(self.shape, dtype, strides=strides)
        self.t = abi.make_tensor(self.ptr, self.shape, strides, dtype, GPU, requires_grad,
                                 self.grad.t if self.grad is not None else None)
        self.p = C.pointer(self.t)  # what the entry points take; built once
        if zero and self._own:
            L.zeros_hip(C.byref(self.t), n)
            L.check("zeros_hip")

    # --- transfer
    @classmethod
    def from_numpy(cls, arr: np.ndarray, requires_grad: bool = False) -> "DeviceTensor":
        arr = np.ascontiguousarray(arr)
        dt = _DT_OF_NP[arr.dtype]
        t = cls(arr.shape, dt, requires_grad, zero=False)
        if arr.nbytes:
            lib().arena_memcpy_h2d_hip(t.ptr, arr.ctypes.data, arr.nbytes)
            lib().check("h2d")
        return t

    def numpy(self) -> np.ndarray:
        """Copy the whole underlying buffer back and apply this tensor's strides on the host."""
        base = self if self.base is None else self.base
        buf = np.empty(base.nbytes // self.itemsize, dtype=_NP_DTYPE[self.dtype])
        if buf.nbytes:
            lib().arena_memcpy_d2h_hip(buf.ctypes.data, base.ptr, buf.nbytes)
            lib().check("d2h")
        off = (self.t.data - base.ptr) // self.itemsize
        shape = abi.shape_of(self.t)
        strides = abi.strides_of(self.t)
        return np.lib.stride_tricks.as_strided(
            buf[off:], shape=shape, strides=[s * self.itemsize for s in strides]).copy()

    def rows_numpy(self, r0: int, rows: int) -> np.ndarray:
        """Rows [r0, r0 + rows) of a contiguous tensor, copied back without the rest."""
        if self.base is not None or abi.strides_of(self.t) != _row_major(self.shape):
            raise ValueError("rows_numpy needs a contiguous tensor of its own")
        row = int(np.prod(self.shape[1:])) if len(self.shape) > 1 else 1
        out = np.empty((rows,) + self.shape[1:], dtype=_NP_DTYPE[self.dtype])
        if out.nbytes:
            lib().arena_memcpy_d2h_hip(out.ctypes.data, self.ptr + r0 * row * self.itemsize,
                                       out.nbytes)
            lib().check("d2h")
        return out

    def fill_(self, kind: str, seed: int, a: float, b: float) -> "DeviceTensor":
        L = lib()
        n = int(np.prod(self.shape))
        if kind == "uniform":
            L.plast_hip_fill_uniform(self.ptr, n, seed, a, b)
        elif kind == "normal":
            L.plast_hip_fill_normal(self.ptr, n, seed, a, b)
        elif kind == "randint":
            L.plast_hip_fill_randint(self.ptr, n, seed, int(a), int(b))
        else:
            raise ValueError(kind)
        L.check("fill")
        return self

    def free(self) -> None:
        if getattr(self, "_own", False) and self.ptr:
            lib().arena_free_hip(self.ptr)
            self.ptr = 0
            self._own = False
        if self.grad is not None:
            self.grad.free()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


_PTR_ARRAY = [TensorP * n for n in range(17)]


def _ptr(x) -> TensorP:
    return x.p if isinstance(x, DeviceTensor) else C.pointer(x)


def _call(kind: str, name: str, inputs, output, p: KernelParams):
    L = lib()
    n = len(inputs)
    arr = (_PTR_ARRAY[n] if n < len(_PTR_ARRAY) else TensorP * n)(*map(_ptr, inputs))
    fn = L.entry.get((kind, name))
    if fn is None:
        raise PlastHipError(f"no entry point {name}_hip_{kind}")
    fn(arr, _ptr(output), p)
    if L.error_count():
        L.raise_error(f"{name}_hip_{kind}")


def forward(name: str, inputs, output, p: KernelParams | None = None) -> None:
    """Call `<name>_hip_forward(inputs, output, params)`."""
    _call("forward", name, inputs, output, p or KernelParams(0, 0, 0.0))


def backward(name: str, inputs, output, p: KernelParams | None = None) -> None:
    """Call `<name>_hip_backward(inputs, output, params)`."""
    _call("backward", name, inputs, output, p or KernelParams(0, 0, 0.0))


def synchronize() -> None:
    L = lib()
    L.plast_hip_synchronize()
    L.check("synchronize")
