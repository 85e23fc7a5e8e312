"""CPU checks of the matmul-epilogue row: the oracle's relu-gradient modulation and bias-gradient
column sum against the reference's own matmul_bias_relu_cpu_backward (src/kernels/cpu/
fused_ops.c:245-307, compiled into oracle/_ref). With an identity weight its da equals its
internal dc_mod exactly (each da element is one product by 1 plus exact zeros), and its dbias is
the column sum itself."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from cases import assert_bits
from hostlib import HostTensor, oracle, ref, ref_available
from plast_amd import abi
from plast_amd.abi import KernelParams

CASES = [(7, 5, 0.0), (64, 33, 0.01), (300, 128, 0.2)]


def epilogue_inputs(M, N, seed):
    rng = np.random.RandomState(seed)
    dout = rng.randn(M, N).astype(np.float32)
    dout[dout == 0] = 1.0                          # keep every product nonzero (no signed zeros)
    out = rng.randn(M, N).astype(np.float32)
    out.flat[: min(4, out.size)] = [0.0, -0.0, np.float32(1e-38), -np.float32(1e-38)][: min(4, out.size)]
    return dout, out


def oracle_modulate(dout, out, alpha):
    o = oracle()
    f = o.oracle_relu_grad_modulate
    f.argtypes = [C.c_void_p] * 3 + [C.c_uint64, C.c_float]
    dc = np.empty_like(dout)
    f(dout.ctypes.data, out.ctypes.data, dc.ctypes.data, dout.size, alpha)
    return dc


def oracle_bias(dc, cols):
    o = oracle()
    f = o.oracle_bias_grad_reduce
    f.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64, C.c_uint64]
    db = np.empty(cols, np.float32)
    f(dc.ctypes.data, db.ctypes.data, dc.size, cols)
    return db


def reference_epilogue(dout, out, alpha):
    """(dc_mod, dbias) as the compiled reference computes them."""
    M, N = dout.shape
    a = HostTensor(np.zeros((M, N), np.float32), requires_grad=True)
    b = HostTensor(np.eye(N, dtype=np.float32))
    bias = HostTensor(np.zeros(N, np.float32), requires_grad=True)
    y = HostTensor(out, requires_grad=True)
    y.grad.buf[:] = dout.ravel()
    f = ref().matmul_bias_relu_cpu_backward
    f.argtypes = [abi.TensorPP, abi.TensorP, KernelParams]
    ptrs, keep = abi.tensor_array(a.t, b.t, bias.t)
    f(ptrs, C.byref(y.t), KernelParams(0, 0, alpha))
    return a.grad.numpy(), bias.grad.numpy()


@pytest.mark.skipif(not ref_available(), reason="oracle/_ref not built (needs /root/reference)")
@pytest.mark.parametrize("M,N,alpha", CASES)
def test_oracle_epilogue_matches_compiled_reference(M, N, alpha):
    dout, out = epilogue_inputs(M, N, M + N)
    dc_ref, db_ref = reference_epilogue(dout, out, alpha)
    dc = oracle_modulate(dout, out, alpha)
    # da = 0.0f + dc_mod (the GEMM's sum starts at +0), so a -0 (alpha = 0) arrives as +0; the
    # sign itself is pinned by the closed-form test below
    assert_bits(dc + np.float32(0.0), dc_ref, "dc_mod")
    assert_bits(oracle_bias(dc, N), db_ref, "dbias")


@pytest.mark.parametrize("M,N,alpha", CASES)
def test_oracle_epilogue_closed_forms(M, N, alpha):
    dout, out = epilogue_inputs(M, N, 3 * M + N)
    dc = oracle_modulate(dout, out, alpha)
    want = np.where(out > 0, dout, dout * np.float32(alpha)).astype(np.float32)
    assert_bits(dc, want, "modulate: one rounding per element")
    db = oracle_bias(dc, N)
    exact = dc.astype(np.float64).sum(0)
    assert np.all(np.abs(db - exact) <= 1e-5 * np.abs(dc).astype(np.float64).sum(0) + 1e-30)
