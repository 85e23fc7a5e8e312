"""The fused chain's backward contract on the host (fused_elementwise_hip_backward, epilogue.hip):
which tapes carry a gradient is decided before any GPU work, so these run on the CPU with tensor
structs whose data pointers are never dereferenced. A chain formed without gradients has a no-op
backward; only leaky_relu(x + bias) with a slope >= 0 over (x, bias row) may carry one, and
anything else with a gradient is reported as an error (the pass never forms it: fusion_fuzz.cpp)."""
from __future__ import annotations

import ctypes as C

import pytest

from plast_amd import abi
from plast_amd.abi import KernelParams
from plast_amd.ops import make_tape
from plast_amd.runtime import LIB_PATH, Library

pytestmark = pytest.mark.skipif(not LIB_PATH.exists(), reason="libplast_hip.so not built")

FAKE = 0x10000  # a device address the checks never reach


def _backward(tape, shapes, grads, out_shape):
    L = Library(LIB_PATH)  # not initialised: no GPU is touched on these paths
    keep = []
    ins = []
    for shape, g in zip(shapes, grads):
        gt = abi.make_tensor(FAKE, shape) if g else None
        keep.append(gt)
        ins.append(abi.make_tensor(FAKE, shape, requires_grad=g, grad=gt))
    gy = abi.make_tensor(FAKE, out_shape)
    y = abi.make_tensor(FAKE, out_shape, requires_grad=True, grad=gy)
    arr, _keep = abi.tensor_array(*ins)
    before = L.plast_hip_error_count()
    L.entry["backward", "fused_elementwise"](arr, C.byref(y), KernelParams(C.addressof(tape), 0, 0.0))
    msg = L.plast_hip_last_error().decode() if L.plast_hip_error_count() != before else None
    L.plast_hip_clear_error()
    return msg


def _pair(alpha):
    return make_tape([("LOAD", 0, 0, 0, 0.0), ("ADD", abi.SRC_INPUT, 1, 0, 0.0),
                      ("LEAKY_RELU", 0, 0, 0, alpha)], 2)


def test_chain_without_gradients_is_a_no_op():
    tape = make_tape([("LOAD", 0, 0, 0, 0.0), ("EXP", 0, 0, 0, 0.0)], 1)
    assert _backward(tape, [(4, 8)], [False], (4, 8)) is None


def test_other_chains_with_a_gradient_are_errors():
    tape = make_tape([("LOAD", 0, 0, 0, 0.0), ("EXP", 0, 0, 0, 0.0)], 1)
    msg = _backward(tape, [(4, 8)], [True], (4, 8))
    assert msg and "only a fused leaky_relu(x + bias) chain" in msg


def test_negative_slope_is_an_error():
    msg = _backward(_pair(-0.1), [(4, 8), (8,)], [True, True], (4, 8))
    assert msg and "alpha >= 0" in msg


def test_nan_slope_is_an_error():
    msg = _backward(_pair(float("nan")), [(4, 8), (8,)], [True, False], (4, 8))
    assert msg and "alpha >= 0" in msg


def test_operands_that_are_not_x_and_a_bias_row_are_errors():
    # a column broadcast, not a row of the last extent
    msg = _backward(_pair(0.0), [(4, 8), (4, 1)], [True, True], (4, 8))
    assert msg and "not (x, bias)" in msg
    # two full tensors
    msg = _backward(_pair(0.0), [(4, 8), (4, 8)], [True, True], (4, 8))
    assert msg and "not (x, bias)" in msg


def test_missing_gradient_buffer_is_an_error():
    """A tensor that requires grad but has no gradient buffer (the checks run before any launch)."""
    L = Library(LIB_PATH)
    tape = _pair(0.0)
    x = abi.make_tensor(FAKE, (4, 8), requires_grad=True)       # no grad buffer
    b = abi.make_tensor(FAKE, (8,))
    gy = abi.make_tensor(FAKE, (4, 8))
    y = abi.make_tensor(FAKE, (4, 8), requires_grad=True, grad=gy)
    before = L.plast_hip_error_count()
    # ensure_init comes first on this path; on a host without a GPU it reports instead
    arr, _keep = abi.tensor_array(x, b)
    L.entry["backward", "fused_elementwise"](arr, C.byref(y), KernelParams(C.addressof(tape), 0, 0.0))
    assert L.plast_hip_error_count() > before
    L.plast_hip_clear_error()
