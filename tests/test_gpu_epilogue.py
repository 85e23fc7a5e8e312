"""GPU parity of the matmul-epilogue row through the C-ABI: launch_relu_grad_modulate_hip bit for
bit against the oracle, bias_grad_reduce_hip within the reduction tolerance (sum order differs:
|gpu - oracle| <= 1e-5 * sum|x| per column, or at least as close to the float64 sum)."""
from __future__ import annotations

import numpy as np
import pytest

from cases import assert_bits, assert_sum_parity
from test_epilogue import epilogue_inputs, oracle_bias, oracle_modulate

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,N,alpha", [(7, 5, 0.0), (64, 33, 0.01), (300, 128, 0.2),
                                       (4096, 1000, 0.01), (16384, 4096, 0.0)])
def test_gpu_epilogue_matches_oracle(M, N, alpha):
    from plast_amd import runtime as rt
    print(f"epilogue {M}x{N} alpha={alpha}", flush=True)
    L = rt.lib()
    dout, out = epilogue_inputs(M, N, M + N)
    D, O = rt.DeviceTensor.from_numpy(dout), rt.DeviceTensor.from_numpy(out)
    DC = rt.DeviceTensor((M, N), zero=False)
    L.launch_relu_grad_modulate_hip(D.ptr, O.ptr, DC.ptr, M * N, alpha, 0, 0)
    L.check("modulate")
    dc = oracle_modulate(dout, out, alpha)
    assert_bits(DC.numpy(), dc, "modulate")
    DB = rt.DeviceTensor((N,), zero=False)
    L.bias_grad_reduce_hip(DC.ptr, DB.ptr, M * N, N)
    L.check("bias_grad_reduce")
    assert_sum_parity(DB.numpy(), oracle_bias(dc, N), dc.astype(np.float64).sum(0),
                      np.abs(dc).astype(np.float64).sum(0), 1e-5, "bias grad")


def test_gpu_bias_grad_rejects_ragged_rows():
    from plast_amd import runtime as rt
    L = rt.lib()
    X = rt.DeviceTensor((10,))
    B = rt.DeviceTensor((3,))
    L.bias_grad_reduce_hip(X.ptr, B.ptr, 10, 3)
    assert L.plast_hip_error_count() > 0
    L.plast_hip_clear_error()
