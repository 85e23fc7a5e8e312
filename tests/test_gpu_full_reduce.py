"""GPU parity of whole-tensor reductions (dim == 9, reduce_ops.c:69-79) large enough that the row
kernel splits the one row into thousands of ordered segments and the finalize merges them with a
wave (runs per lane, then an ordered tree). Sum and mean: within 1e-5·Σ|x| of the oracle's serial
fp32 sum, or at least as close to the fp64 sum as that serial sum is (over 2^24 terms the serial
sum drifts by percent). Max and min: bit-exact against the reference's fold, with NaN, signed
zeros and ties placed in different segments. Argmax: numpy's first index."""
from __future__ import annotations

import numpy as np
import pytest

from cases import assert_bits, assert_sum_parity
from hostlib import HostTensor, oracle_forward

pytestmark = pytest.mark.gpu
N = (1 << 24) + 12      # 1986 segments of 8448, the last one ragged


def _x(seed, specials):
    rng = np.random.RandomState(seed)
    x = rng.randn(N).astype(np.float32)
    if specials == "zeros":          # the maximum is a zero, with both signs in many segments
        x = -np.abs(x)
        x[::5000] = -0.0
        x[7::9001] = 0.0
    elif specials == "nan":          # a NaN resets the fold mid-tensor
        x[N // 3] = np.nan
        x[N // 3 + 4096 * 7 + 5] = 50.0
    elif specials == "ties":         # the maximum value appears in several segments
        x[[123, 4096 * 900 + 1, N - 1]] = 9.0
    return x


@pytest.mark.parametrize("specials", ["plain", "zeros", "nan", "ties"])
def test_whole_tensor_reductions(specials):
    from plast_amd import ops, runtime as rt
    from plast_amd.abi import DIM_ALL, KernelParams
    print(f"whole-tensor reductions over {N} ({specials})", flush=True)
    x = _x(5, specials)
    dx = rt.DeviceTensor.from_numpy(x)
    scale = float(np.abs(x[np.isfinite(x)]).astype(np.float64).sum())
    for op in ("sum", "mean", "max", "min"):
        got = ops.reduce(op, dx).numpy()
        want = HostTensor(np.zeros(1, np.float32))
        oracle_forward(op, [HostTensor(x)], want, KernelParams(DIM_ALL, 0, 0.0))
        w = want.numpy()
        if op in ("max", "min"):
            assert_bits(got, w, f"{op} ({specials})")
        else:
            exact = np.nansum(x.astype(np.float64)) if specials != "nan" else np.nan
            if op == "mean":
                exact = exact / N
            assert_sum_parity(got, w, np.array([exact]), scale / (N if op == "mean" else 1),
                              1e-5, f"{op} ({specials})")
    am = ops.reduce("argmax", dx).numpy()
    assert int(am[0]) == int(np.argmax(x)), f"argmax ({specials})"
