"""GPU parity of the matmul-epilogue row through the C-ABI: launch_relu_grad_modulate_hip bit for
bit against the oracle, bias_grad_reduce_hip within the reduction tolerance (sum order differs:
|gpu - oracle| <= 1e-5 * sum|x| per column, or at least as close to the float64 sum), and the
one-pass relu_grad_modulate_bias_grad_hip bit for bit against those two calls in sequence."""
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


def _two_step(L, D, O, M, N, alpha):
    from plast_amd import runtime as rt
    DC = rt.DeviceTensor((M, N), zero=False)
    DB = rt.DeviceTensor((N,), zero=False)
    L.launch_relu_grad_modulate_hip(D, O, DC.ptr, M * N, alpha, 0, 0)
    L.bias_grad_reduce_hip(DC.ptr, DB.ptr, M * N, N)
    L.check("two steps")
    dc, db = DC.numpy(), DB.numpy()
    DC.free()
    DB.free()
    return dc, db


# float4 shapes (cols % 4 == 0), scalar shapes, one row (no reduced axis), one column (a row
# reduction: both of these take the two-step form), and the bench's [16384, 4096]
@pytest.mark.parametrize("M,N,alpha", [(1024, 256, 0.0), (300, 128, 0.2), (333, 37, 0.01),
                                       (1, 64, 0.0), (77, 1, 0.1), (2, 3, 0.5),
                                       (16384, 4096, 0.0)])
def test_gpu_fused_modulate_bias_grad_matches_two_steps(M, N, alpha):
    from plast_amd import runtime as rt
    print(f"fused epilogue {M}x{N} alpha={alpha}", flush=True)
    L = rt.lib()
    dout, out = epilogue_inputs(M, N, 3 * M + N)
    out[0, :min(N, 3)] = [0.0, -0.0, np.float32(1e-45)][:min(N, 3)]  # the z > 0 boundary
    D, O = rt.DeviceTensor.from_numpy(dout), rt.DeviceTensor.from_numpy(out)
    wdc, wdb = _two_step(L, D.ptr, O.ptr, M, N, alpha)
    DC = rt.DeviceTensor((M, N), zero=False)
    DB = rt.DeviceTensor((N,), zero=False)
    L.relu_grad_modulate_bias_grad_hip(D.ptr, O.ptr, DC.ptr, DB.ptr, M * N, N, alpha)
    L.check("fused")
    assert_bits(DC.numpy(), wdc, "dc, one pass vs two steps")
    assert_bits(DB.numpy(), wdb, "dbias, one pass vs two steps")
    dc = oracle_modulate(dout, out, alpha)
    assert_bits(DC.numpy(), dc, "dc vs oracle")
    assert_sum_parity(DB.numpy(), oracle_bias(dc, N), dc.astype(np.float64).sum(0),
                      np.abs(dc).astype(np.float64).sum(0), 1e-5, "dbias vs oracle")


def test_gpu_fused_modulate_bias_grad_unaligned_and_in_place():
    """Operands one float off 16-byte alignment (the scalar form), a dc whose alignment differs
    from the inputs' (the two-step form), dc written over dout (each element is read before it
    is written by the same lane), and an empty gradient (dbias all zeros)."""
    from plast_amd import runtime as rt
    L = rt.lib()
    M, N, alpha = 96, 64, 0.05
    dout, out = epilogue_inputs(M, N, 5)
    n = M * N
    base_d = rt.DeviceTensor.from_numpy(np.concatenate([[7.0], dout.ravel()]).astype(np.float32))
    base_o = rt.DeviceTensor.from_numpy(np.concatenate([[7.0], out.ravel()]).astype(np.float32))
    D, O = base_d.ptr + 4, base_o.ptr + 4
    wdc, wdb = _two_step(L, D, O, M, N, alpha)
    for dc_off in (4, 0):
        base_c = rt.DeviceTensor((n + 1,), zero=False)
        DB = rt.DeviceTensor((N,), zero=False)
        L.relu_grad_modulate_bias_grad_hip(D, O, base_c.ptr + dc_off, DB.ptr, n, N, alpha)
        L.check("fused, unaligned")
        got = base_c.numpy()[dc_off // 4:dc_off // 4 + n].reshape(M, N)
        assert_bits(got, wdc, f"dc (dc offset {dc_off} B)")
        assert_bits(DB.numpy(), wdb, f"dbias (dc offset {dc_off} B)")
    D2 = rt.DeviceTensor.from_numpy(dout)
    O2 = rt.DeviceTensor.from_numpy(out)
    DB = rt.DeviceTensor((N,), zero=False)
    L.relu_grad_modulate_bias_grad_hip(D2.ptr, O2.ptr, D2.ptr, DB.ptr, n, N, alpha)
    L.check("fused, in place")
    assert_bits(D2.numpy(), wdc, "dc over dout")
    assert_bits(DB.numpy(), wdb, "dbias, in place")
    E = rt.DeviceTensor.from_numpy(np.full(N, 3.0, np.float32))
    L.relu_grad_modulate_bias_grad_hip(D2.ptr, O2.ptr, D2.ptr, E.ptr, 0, N, alpha)
    L.check("fused, empty")
    assert (E.numpy() == 0.0).all() and not np.signbit(E.numpy()).any()


@pytest.mark.parametrize("M,N", [(96, 64), (4096, 1024)], ids=["one-launch", "chunked"])
def test_gpu_fused_in_place_refold_reads_the_stored_terms(M, N):
    """A column whose sum is not finite is summed again in index order. With dc written over dout,
    the terms must be read back as stored: re-modulating the overwritten inputs would scale the
    out <= 0 terms by alpha twice. Column 1 holds three 1.5e38 terms (3e38 with out < 0, alpha 0.5)
    and then -inf: index order gives inf + -inf = NaN, the doubly scaled terms -inf. Checked
    against the two calls (modulation into a separate buffer, then the column sum), bit for bit,
    for the one-launch small sum and the chunked sum with its finalize."""
    from plast_amd import runtime as rt
    L = rt.lib()
    alpha = 0.5
    dout, out = epilogue_inputs(M, N, 11)
    dout[:3, 1] = 3e38
    out[:3, 1] = -1.0
    dout[5, 1] = -np.inf
    out[5, 1] = 1.0
    D, O = rt.DeviceTensor.from_numpy(dout), rt.DeviceTensor.from_numpy(out)
    wdc, wdb = _two_step(L, D.ptr, O.ptr, M, N, alpha)
    assert np.isnan(wdb[1])
    DB = rt.DeviceTensor((N,), zero=False)
    L.relu_grad_modulate_bias_grad_hip(D.ptr, O.ptr, D.ptr, DB.ptr, M * N, N, alpha)
    L.check("fused, in place")
    assert_bits(D.numpy(), wdc, "dc over dout")
    assert_bits(DB.numpy(), wdb, "dbias, in place")


def test_gpu_bias_grad_rejects_ragged_rows():
    from plast_amd import runtime as rt
    L = rt.lib()
    X = rt.DeviceTensor((10,))
    B = rt.DeviceTensor((3,))
    L.bias_grad_reduce_hip(X.ptr, B.ptr, 10, 3)
    assert L.plast_hip_error_count() > 0
    L.plast_hip_clear_error()
    L.relu_grad_modulate_bias_grad_hip(X.ptr, X.ptr, X.ptr, B.ptr, 10, 3, 0.0)
    assert L.plast_hip_error_count() > 0
    L.plast_hip_clear_error()
