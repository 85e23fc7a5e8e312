"""GPU checks of launches larger than one dispatch allows. A dispatch packet's grid size is 32-bit
(fewer than 2^32 work-items per dimension), so the library splits such work over several launches
or moves it to a grid-stride kernel: cross-entropy over more than 2^24 rows (row-range launches,
with the NEG rule's boundary carried into each range), fills past 2^34 words, an elementwise
space of 2^34 elements, and an optimizer tensor split into several launch entries. Each case
checks against the oracle (cross-entropy) or values fixed by construction, at the range
boundaries. The multi-GiB cases skip when the device lacks the memory."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from cases import LSE_SCALE, assert_bits, assert_close_sum
from hostlib import HostTensor, oracle_backward, oracle_forward

pytestmark = pytest.mark.gpu

GiB = 1 << 30
ROWS_PER_LAUNCH = (1 << 32) // 256 - 1      # rows per cross-entropy launch (2^24 - 1)
FILL_WORDS_PER_LAUNCH = ROWS_PER_LAUNCH * 256 * 4


def _rt():
    from plast_amd import runtime
    return runtime


def _need(nbytes):
    _rt().lib()  # the library has initialised the HIP runtime and selected its device
    hip = C.CDLL("libamdhip64.so.7")  # the runtime the library is linked against
    free, total = C.c_size_t(0), C.c_size_t(0)
    assert hip.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    free = free.value
    if free < nbytes + 8 * GiB:
        pytest.skip(f"needs {nbytes / GiB:.0f} GiB of device memory, {free / GiB:.0f} GiB free")


def _read(ptr, index, dtype=np.float32):
    """Elements `index` of the device array at ptr (one small copy each)."""
    L = _rt().lib()
    out = np.empty(len(index), dtype)
    size = out.itemsize
    for j, i in enumerate(index):
        L.arena_memcpy_d2h_hip(out[j:].ctypes.data, ptr + int(i) * size, size)
    L.check("d2h")
    return out


@pytest.mark.parametrize("C_", [4, 3], ids=["wave-per-row", "workgroup-per-row"])
def test_ce_rows_beyond_one_launch(C_):
    from plast_amd import ops
    rt = _rt()
    N = ROWS_PER_LAUNCH + 37
    print(f"cross-entropy {N}x{C_}", flush=True)
    rng = np.random.RandomState(C_)
    x = rng.randn(N, C_).astype(np.float32)
    lab = rng.randint(0, C_, N).astype(np.int32)
    # rows whose loss is exactly zero, so the sign of that zero shows which side of the NEG
    # rule's boundary (the last multiple of 8 rows) each was computed on: around the launch
    # boundary and around the rule's boundary
    se = N // 8 * 8
    for r in (ROWS_PER_LAUNCH - 2, ROWS_PER_LAUNCH - 1, ROWS_PER_LAUNCH, ROWS_PER_LAUNCH + 1,
              se - 2, se - 1, se, N - 1):
        x[r, :] = -200.0          # exp underflows to 0: log-sum-exp exactly 0
        x[r, lab[r]] = 0.0
    dx = rt.DeviceTensor.from_numpy(x, requires_grad=True)
    dl = rt.DeviceTensor.from_numpy(lab)
    loss, stats = ops.softmax_cross_entropy(dx, dl, requires_grad=True)
    hx, hl = HostTensor(x, requires_grad=True), HostTensor(lab)
    hs = HostTensor(np.zeros((N, 2), np.float32))
    ho = HostTensor(np.zeros(N, np.float32), requires_grad=True)
    oracle_forward("softmax_cross_entropy", [hx, hl, hs], ho)
    st, wst = stats.numpy(), hs.numpy()
    assert_bits(st[:, 0], wst[:, 0], "row max")
    # l = log(s) with s the row's sum of exp terms (s >= 1): the sum tolerance |ds| <= 1e-5 * s
    # bounds |dl| by 1e-5 absolute (with three classes s is often near 1 and l tiny, so a
    # tolerance relative to l itself would ask for more than the sum's)
    assert_close_sum(st[:, 1], wst[:, 1], LSE_SCALE, 1e-5, "row log-sum-exp")
    got, want = loss.numpy(), ho.numpy()
    assert_close_sum(got, want, np.abs(want) + LSE_SCALE, 1e-5, "row loss")
    zero_rows = [ROWS_PER_LAUNCH - 1, ROWS_PER_LAUNCH, se - 1, se, N - 1]
    assert_bits(got[zero_rows], want[zero_rows], "signed zero losses at the boundaries")
    assert np.signbit(got[se]) and not np.signbit(got[se - 1])
    g = np.full(N, np.float32(1.0) / np.float32(N), np.float32)
    rt.lib().arena_memcpy_h2d_hip(loss.grad.ptr, g.ctypes.data, g.nbytes)
    ho.grad.buf[:] = g
    print("cross-entropy backward", flush=True)
    rt.backward("softmax_cross_entropy", [dx, dl, stats], loss)
    oracle_backward("softmax_cross_entropy", [hx, hl, hs], ho)
    gx, wx = dx.grad.numpy(), hx.grad.numpy()
    finite = np.isfinite(wx).all(1)
    assert_close_sum(gx[finite], wx[finite], np.abs(wx[finite]) + 1.0 / N * 1e-2, 1e-5, "dlogits")


def test_fill_beyond_one_launch_and_generic_elementwise():
    """ones_hip over 2^34 + 6 words (two fill launches, the second ending in a partial uint4), then
    NEG over that 2^34 + 6 element space: one float4 per lane would need more than 2^32 lanes, so
    the launch goes to the 64-bit grid-stride kernel."""
    rt = _rt()
    L = rt.lib()
    n = (1 << 34) + 6
    _need(2 * 4 * n)
    print(f"fill {n} words", flush=True)
    a = rt.DeviceTensor((n,), zero=False)
    L.ones_hip(C.byref(a.t), n)
    L.check("ones_hip")
    idx = [0, 1, FILL_WORDS_PER_LAUNCH - 1, FILL_WORDS_PER_LAUNCH, FILL_WORDS_PER_LAUNCH + 1,
           (1 << 32) - 1, 1 << 32, n - 5, n - 2, n - 1]
    assert (_read(a.ptr, idx) == 1.0).all()
    print("neg over 2^34 + 6 elements", flush=True)
    o = rt.DeviceTensor((n,), zero=False)
    rt.forward("neg", [a], o)
    got = _read(o.ptr, idx)
    assert (got == -1.0).all(), got
    o.free()
    a.free()


def test_sgd_tensor_split_over_launch_entries():
    """One SGD parameter of 2^34 + 1000 elements: more workgroups than one launch holds, so it is
    updated as three entries; p = 1, g = 1, lr = 0.5 gives 0.5 everywhere."""
    from plast_amd import abi
    rt = _rt()
    L = rt.lib()
    n = (1 << 34) + 1000
    _need(2 * 4 * n)
    print(f"sgd over {n} parameters", flush=True)
    p = rt.DeviceTensor((n,), requires_grad=True, zero=False)
    L.ones_hip(C.byref(p.t), n)
    L.ones_hip(C.byref(p.grad.t), n)
    L.check("ones_hip")
    arr = (abi.TensorP * 1)(C.pointer(p.t))
    L.sgd_step_hip(C.byref(abi.SGD(0.5)), C.cast(arr, abi.TensorPP), 1)
    L.check("sgd_step_hip")
    piece = ((1 << 32) // 256 - 1) // 2 * 1024
    idx = [0, piece - 1, piece, 2 * piece - 1, 2 * piece, n - 1]
    assert (_read(p.ptr, idx) == 0.5).all()
    p.free()
