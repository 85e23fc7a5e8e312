"""GPU parity of the pack row: hip_tensor_pack_init / hip_tensor_pack_release and the strided host
transfers through the C-ABI, bit for bit against the row-major gather (the closed form the
reference's own pack is checked against in test_pack.py), for float32, int32 and int64 views."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from cases import assert_bits
from plast_amd import abi
from plast_amd.abi import FLOAT32, INT32, INT64
from test_pack import VIEWS, gather

pytestmark = pytest.mark.gpu
NP = {FLOAT32: np.float32, INT32: np.int32, INT64: np.int64}


def _rt():
    from plast_amd import runtime
    return runtime


def _base(bshape, dtype, seed):
    rng = np.random.RandomState(seed)
    if dtype == FLOAT32:
        return rng.randn(*bshape).astype(np.float32)
    if dtype == INT32:
        return rng.randint(-2**31, 2**31 - 1, size=bshape, dtype=np.int64).astype(np.int32)
    return rng.randint(-2**62, 2**62, size=bshape, dtype=np.int64)


def _view(rt, base_dev, shape, strides, offset, dtype):
    return rt.DeviceTensor(shape, dtype, base=base_dev, strides=strides, offset=offset, zero=False)


def _read(ptr, shape, dtype):
    out = np.empty(shape, NP[dtype])
    if out.nbytes:
        _rt().lib().arena_memcpy_d2h_hip(out.ctypes.data, ptr, out.nbytes)
        _rt().lib().check("d2h")
    return out


@pytest.mark.parametrize("dtype", [FLOAT32, INT32, INT64], ids=["f32", "i32", "i64"])
@pytest.mark.parametrize("view", VIEWS, ids=[str(v[1:3]) for v in VIEWS])
def test_gpu_pack_matches_gather(view, dtype):
    rt = _rt()
    L = rt.lib()
    bshape, shape, strides, off = view
    base = _base(bshape, dtype, 3)
    bdev = rt.DeviceTensor.from_numpy(base)
    v = _view(rt, bdev, shape, strides, off, dtype)
    p = abi.HipTensorPack()
    L.hip_tensor_pack_init(C.byref(p), C.byref(v.t))
    L.check("hip_tensor_pack_init")
    assert p.data and p._d_buf and p.data == p._d_buf
    assert_bits(_read(p.data, shape, dtype), gather(base, shape, strides, off), "pack")
    L.hip_tensor_pack_release(C.byref(p))
    assert not p.data and not p._d_buf
    # the same through the host transfer
    host = np.empty(shape, NP[dtype])
    assert L.plast_hip_tensor_to_host(C.byref(v.t), host.ctypes.data) == 0
    assert_bits(host, gather(base, shape, strides, off), "to_host")


def test_gpu_pack_aliases_contiguous():
    rt = _rt()
    L = rt.lib()
    x = rt.DeviceTensor.from_numpy(np.arange(24, dtype=np.float32).reshape(2, 3, 4))
    p = abi.HipTensorPack()
    L.hip_tensor_pack_init(C.byref(p), C.byref(x.t))
    assert p.data == x.ptr and not p._d_buf
    L.hip_tensor_pack_release(C.byref(p))
    # a padded leading stride is not contiguous here (the reference would alias it)
    base = rt.DeviceTensor.from_numpy(np.arange(40, dtype=np.float32).reshape(8, 5))
    v = rt.DeviceTensor((3, 5), base=base, strides=(10, 1), zero=False)
    L.hip_tensor_pack_init(C.byref(p), C.byref(v.t))
    L.check("pack")
    assert p._d_buf
    assert_bits(_read(p.data, (3, 5), FLOAT32), np.arange(40, dtype=np.float32).reshape(8, 5)[0:6:2],
                "padded rows packed")
    L.hip_tensor_pack_release(C.byref(p))


@pytest.mark.parametrize("dtype", [FLOAT32, INT64], ids=["f32", "i64"])
def test_gpu_from_host_scatters_into_views(dtype):
    rt = _rt()
    L = rt.lib()
    base = _base((3, 5, 7), dtype, 5)
    bdev = rt.DeviceTensor.from_numpy(base)
    v = _view(rt, bdev, (3, 7, 5), (35, 1, 7), 0, dtype)      # permute (0, 2, 1)
    src = _base((3, 7, 5), dtype, 6)
    assert L.plast_hip_tensor_from_host(C.byref(v.t), src.ctypes.data) == 0
    assert_bits(_read(bdev.ptr, (3, 5, 7), dtype), src.transpose(0, 2, 1), "scatter")
    # contiguous destination: plain copy
    c = rt.DeviceTensor((4, 4), dtype, zero=True)
    s2 = _base((4, 4), dtype, 7)
    assert L.plast_hip_tensor_from_host(C.byref(c.t), s2.ctypes.data) == 0
    assert_bits(_read(c.ptr, (4, 4), dtype), s2, "contiguous from_host")


def test_gpu_from_host_rejects_broadcast_destination():
    rt = _rt()
    L = rt.lib()
    base = rt.DeviceTensor((5,), zero=True)
    v = rt.DeviceTensor((4, 5), base=base, strides=(0, 1), zero=False)
    src = np.ones((4, 5), np.float32)
    assert L.plast_hip_tensor_from_host(C.byref(v.t), src.ctypes.data) == -1
    assert L.plast_hip_error_count() > 0
    L.plast_hip_clear_error()


def test_gpu_pack_config3_size():
    """Config 3's permuted operand: pack [256,512,512] viewed as permute (0,2,1) of its base."""
    rt = _rt()
    L = rt.lib()
    print("pack [256,512,512] permuted", flush=True)
    shape = (256, 512, 512)
    bdev = rt.DeviceTensor(shape, zero=False).fill_("normal", 42, 0.0, 1.0)
    v = rt.DeviceTensor(shape, base=bdev, strides=(262144, 1, 512), zero=False)
    p = abi.HipTensorPack()
    L.hip_tensor_pack_init(C.byref(p), C.byref(v.t))
    L.check("pack")
    got = _read(p.data, shape, FLOAT32)
    L.hip_tensor_pack_release(C.byref(p))
    want = bdev.numpy().transpose(0, 2, 1)
    assert_bits(got, want, "config-3 pack")


def _random_views(n, seed):
    """Seeded random views of a contiguous base: a slice with steps on each axis, then a
    permutation of the axes, sometimes with a broadcast (stride 0) axis inserted; sizes reach the
    whole-tile transposed path (both tile axes of 64 or more)."""
    rng = np.random.RandomState(seed)
    out = []
    for _ in range(n):
        rank = rng.randint(1, 5)
        big = rng.rand() < 0.4 and rank >= 2
        bshape = tuple(int(rng.choice([130, 200, 256])) if big and d >= rank - 2 else
                       int(rng.randint(1, 12)) for d in range(rank))
        base = np.arange(int(np.prod(bshape)), dtype=np.int64).reshape(bshape)
        sl = []
        for d in bshape:
            start = int(rng.randint(0, max(1, d // 3)))
            step = int(rng.choice([1, 1, 1, 2, 3]))
            sl.append(slice(start, None, step))
        v = base[tuple(sl)].transpose(rng.permutation(rank))
        if rng.rand() < 0.3:
            ax = int(rng.randint(0, v.ndim + 1))
            v = np.expand_dims(v, ax)
            shp = list(v.shape)
            shp[ax] = int(rng.choice([2, 3, 5]))
            v = np.broadcast_to(v, shp)
        shape = tuple(int(s) for s in v.shape)
        strides = tuple(int(s) // 8 for s in v.strides)
        offset = int((v.__array_interface__["data"][0] - base.__array_interface__["data"][0]) // 8)
        out.append((bshape, shape, strides, offset))
    return out


RANDOM_VIEWS = _random_views(40, 5)


@pytest.mark.parametrize("view", RANDOM_VIEWS, ids=[f"v{i}" for i in range(len(RANDOM_VIEWS))])
def test_gpu_pack_random_views(view):
    rt = _rt()
    L = rt.lib()
    bshape, shape, strides, off = view
    print(f"pack {bshape} -> {shape} strides {strides} offset {off}", flush=True)
    base = _base(bshape, FLOAT32, 9)
    bdev = rt.DeviceTensor.from_numpy(base)
    v = _view(rt, bdev, shape, strides, off, FLOAT32)
    p = abi.HipTensorPack()
    L.hip_tensor_pack_init(C.byref(p), C.byref(v.t))
    L.check("hip_tensor_pack_init")
    assert_bits(_read(p.data, shape, FLOAT32), gather(base, shape, strides, off), "pack")
    L.hip_tensor_pack_release(C.byref(p))
    L.check("hip_tensor_pack_release")
