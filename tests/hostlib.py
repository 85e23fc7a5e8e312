"""Host-side wrappers for the CPU libraries used as checkers: the oracle (oracle/liboracle.so, this
repository's C restatement), the compiled reference (oracle/_ref/libplast_ref.so, built from
/root/reference's own C sources with FMA contraction off) and, where it was built, the same sources
under the reference's own flags (oracle/_ref/libplast_ref_native.so, contraction on). All take the
same `Tensor` structs as the HIP library."""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

from plast_amd import abi
from plast_amd.abi import CPU, FLOAT32, INT32, INT64, KernelParams, TensorP, TensorPP

ROOT = Path(__file__).resolve().parent.parent
ORACLE_PATH = ROOT / "oracle" / "liboracle.so"
REF_PATH = ROOT / "oracle" / "_ref" / "libplast_ref.so"
NATIVE_PATH = ROOT / "oracle" / "_ref" / "libplast_ref_native.so"
# the reference with the drop-in's scheduler edit applied, linked against the HIP library
REF_HIP_PATH = ROOT / "oracle" / "_ref" / "libplast_ref_hip.so"

_DT = {np.dtype(np.float32): FLOAT32, np.dtype(np.int32): INT32, np.dtype(np.int64): INT64}

_oracle = None
_ref = None
_native = None


def oracle():
    global _oracle
    if _oracle is None:
        if not ORACLE_PATH.exists():
            raise RuntimeError(f"{ORACLE_PATH} missing: run `make -C oracle`")
        _oracle = C.CDLL(str(ORACLE_PATH))
    return _oracle


def ref_available() -> bool:
    return REF_PATH.exists()


def ref():
    global _ref
    if _ref is None:
        _ref = C.CDLL(str(REF_PATH))
    return _ref


def native_available() -> bool:
    return NATIVE_PATH.exists()


def native():
    global _native
    if _native is None:
        _native = C.CDLL(str(NATIVE_PATH))
    return _native


class HostTensor:
    """A numpy buffer described by a reference `Tensor` struct (device CPU)."""

    def __init__(self, arr=None, *, shape=None, dtype=np.float32, requires_grad=False,
                 strides=None, base: "HostTensor | None" = None, offset: int = 0):
        if base is not None:
            self.buf = base.buf
            ptr = base.buf.ctypes.data + offset * base.buf.itemsize
            self.shape = tuple(shape)
            dt = _DT[base.buf.dtype]
        else:
            if arr is None:
                arr = np.zeros(shape, dtype=dtype)
            self.buf = np.ascontiguousarray(arr).reshape(-1).copy()
            self.shape = tuple(np.shape(arr))
            ptr = self.buf.ctypes.data
            dt = _DT[self.buf.dtype]
        self.grad = None
        if requires_grad:
            self.grad = HostTensor(np.zeros(self.shape, dtype=self.buf.dtype))
            if strides is not None:
                self.grad.t.ndim = len(self.shape)
                for d, s in enumerate(strides):
                    self.grad.t.strides[d] = s
        self.t = abi.make_tensor(ptr, self.shape, strides, dt, CPU, requires_grad,
                                 self.grad.t if self.grad else None)
        self.base = base

    def numpy(self) -> np.ndarray:
        """Apply this struct's (possibly rewritten) shape/strides to the buffer."""
        isz = self.buf.itemsize
        off = (self.t.data - self.buf.ctypes.data) // isz
        shape = abi.shape_of(self.t)
        st = abi.strides_of(self.t)
        return np.lib.stride_tricks.as_strided(self.buf[off:], shape=shape,
                                               strides=[s * isz for s in st]).copy()


def _call(libh, fname, inputs, output, p):
    arr = (TensorP * len(inputs))(*[C.pointer(x.t if isinstance(x, HostTensor) else x)
                                    for x in inputs])
    f = getattr(libh, fname)
    f.argtypes = [TensorPP, TensorP, KernelParams]
    f.restype = None
    out = output.t if isinstance(output, HostTensor) else output
    f(C.cast(arr, TensorPP), C.byref(out), p)


def oracle_forward(name, inputs, output, p=None):
    _call(oracle(), f"oracle_{name}_forward", inputs, output, p or KernelParams(0, 0, 0.0))


def oracle_backward(name, inputs, output, p=None):
    _call(oracle(), f"oracle_{name}_backward", inputs, output, p or KernelParams(0, 0, 0.0))


def ref_forward(name, inputs, output, p=None):
    _call(ref(), f"{name}_cpu_forward", inputs, output, p or KernelParams(0, 0, 0.0))


def ref_backward(name, inputs, output, p=None):
    _call(ref(), f"{name}_cpu_backward", inputs, output, p or KernelParams(0, 0, 0.0))


def fused_chain2(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    o = oracle()
    f = o.oracle_fused_chain2
    f.argtypes = [C.c_void_p] * 4 + [C.c_uint64]
    f.restype = None
    out = np.empty_like(a)
    f(a.ctypes.data, b.ctypes.data, c.ctypes.data, out.ctypes.data, a.size)
    return out


def libm_expf(x: np.ndarray) -> np.ndarray:
    """glibc expf elementwise (the routine the reference calls: unary_ops.c:158)."""
    libm = C.CDLL("libm.so.6")
    f = libm.expf
    f.argtypes = [C.c_float]
    f.restype = C.c_float
    return np.array([f(float(v)) for v in np.asarray(x, np.float32).ravel()],
                    dtype=np.float32).reshape(np.shape(x))


# ------------------------------------------------------------------------------- case backends
from cases import Backend  # noqa: E402


class HostBackend(Backend):
    """Runs cases through the oracle ("oracle"), the compiled reference ("ref") or the reference
    built with its own flags ("native")."""

    def __init__(self, which: str):
        self.which = which
        self.keep = []

    def tensor(self, arr, requires_grad):
        t = HostTensor(arr, requires_grad=requires_grad)
        self.keep.append(t)
        return t

    def view(self, base, shape, strides, own_grad=False):
        v = HostTensor(base=base, shape=shape, strides=strides)
        v.t.requires_grad = base.t.requires_grad
        if base.grad is not None:
            if own_grad:
                # a zero-filled gradient of its own, contiguous in the view's shape
                g = HostTensor(np.zeros(shape, np.float32))
            else:
                # the view's gradient aliases the base gradient with the view's strides
                g = HostTensor(base=base.grad, shape=shape, strides=strides)
            v.grad = g
            v.t.grad = C.pointer(g.t)
        self.keep.append(v)
        return v

    def empty(self, shape, dtype, requires_grad=False):
        npdt = np.int64 if dtype == "i64" else np.float32
        t = HostTensor(np.zeros(shape, npdt), requires_grad=requires_grad)
        self.keep.append(t)
        return t

    def fwd(self, op, ins, out, p):
        if self.which == "oracle":
            oracle_forward(op, ins, out, p)
        else:
            _call(ref() if self.which == "ref" else native(), f"{op}_cpu_forward", ins, out,
                  p or KernelParams(0, 0, 0.0))

    def bwd(self, op, ins, out, p):
        if self.which == "oracle":
            oracle_backward(op, ins, out, p)
        else:
            _call(ref() if self.which == "ref" else native(), f"{op}_cpu_backward", ins, out,
                  p or KernelParams(0, 0, 0.0))

    def read(self, t):
        return t.numpy()

    def read_grad(self, t):
        g = t.grad
        return g.numpy()

    def set_grad(self, t, arr):
        t.grad.buf[:] = np.ascontiguousarray(arr, dtype=t.grad.buf.dtype).reshape(-1)

    def grad_size(self, t):
        return int(t.grad.buf.size)


def ref_ce_chain(logits: np.ndarray, labels: np.ndarray, which: str = "ref", backward: bool = True):
    """The reference's cross-entropy op chain (src/api/loss.c:97-169) node by node through a CPU
    library, then its backward in reverse node order. Returns (row_loss, row_max, row_logsum,
    mean_loss, dlogits)."""
    fwd = ref_forward if which == "ref" else oracle_forward
    bwd = ref_backward if which == "ref" else oracle_backward
    N, Cn = logits.shape
    onehot = np.zeros((N, Cn), np.float32)
    onehot[np.arange(N), labels] = 1.0
    x = HostTensor(logits, requires_grad=backward)
    tgt = HostTensor(onehot)
    keep = []

    def node(op, ins, shape, p=(0, 0, 0.0)):
        out = HostTensor(np.zeros(shape, np.float32), requires_grad=backward)
        fwd(op, ins, out, KernelParams(*p))
        keep.append((op, ins, out, p))
        return out

    mx = node("max", [x], (N, 1), (1, 1, 0.0))
    sh = node("sub", [x, mx], (N, Cn))
    ex = node("exp", [sh], (N, Cn))
    se = node("sum", [ex], (N, 1), (1, 1, 0.0))
    ls = node("log", [se], (N, 1))
    lsm = node("sub", [sh, ls], (N, Cn))
    tl = node("mul", [tgt, lsm], (N, Cn))
    sm = node("sum", [tl], (N, 1), (1, 1, 0.0))
    ng = node("neg", [sm], (N, 1))
    mean = node("mean", [ng], (1,), (abi.DIM_ALL, 0, 0.0))
    dx = None
    if backward:
        mean.grad.buf[:] = 1.0
        for op, ins, out, p in reversed(keep):
            bwd(op, ins, out, KernelParams(*p))
        dx = x.grad.numpy()
    return (ng.numpy().reshape(N), mx.numpy().reshape(N), ls.numpy().reshape(N),
            mean.numpy().reshape(()), dx)
