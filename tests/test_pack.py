"""CPU checks of the pack row: HipTensorPack's layout equals the reference's pack struct, and the
closed form the GPU pack is compared with (a row-major gather, numpy's as_strided) is what the
reference's own tensor_pack_init (src/kernels/cpu/pack.c:30-48, compiled into oracle/_ref)
produces, including its one deliberate deviation (the strides[0] quirk)."""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np
import pytest

from cases import assert_bits
from hostlib import HostTensor, ref, ref_available
from plast_amd import abi

ROOT = Path(__file__).resolve().parent.parent
REF_INC = Path("/root/reference/include")

# (base shape, view shape, view strides, element offset): permutes, slices, broadcasts
VIEWS = [
    ((4, 6), (6, 4), (1, 6), 0),                       # transpose
    ((3, 5, 7), (3, 7, 5), (35, 1, 7), 0),             # permute (0, 2, 1)
    ((3, 5, 7), (7, 3, 5), (1, 35, 7), 0),             # permute (2, 0, 1)
    ((6, 10), (6, 4), (10, 1), 3),                     # column slice
    ((5,), (4, 5), (0, 1), 0),                         # expand along a new leading axis
    ((2, 3, 4, 5), (5, 4, 3, 2), (1, 5, 20, 60), 0),   # full reversal of axes
    ((9, 8), (3, 8), (24, 1), 0),                      # every third row
]


def gather(base: np.ndarray, shape, strides, offset) -> np.ndarray:
    """The closed form: element i of the pack is the view's element at coordinates(i)."""
    flat = base.reshape(-1)
    return np.lib.stride_tricks.as_strided(
        flat[offset:], shape=shape, strides=[s * flat.itemsize for s in strides]).copy()


def test_pack_struct_layout(tmp_path):
    src = tmp_path / "probe.c"
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "plast_hip.h"\n'
                   'int main(void){printf("%zu %zu %zu\\n", sizeof(HipTensorPack), '
                   'offsetof(HipTensorPack, data), offsetof(HipTensorPack, _d_buf));return 0;}\n')
    subprocess.run(["gcc", "-o", str(tmp_path / "p"), str(src), f"-I{ROOT / 'include'}"], check=True)
    out = subprocess.run([str(tmp_path / "p")], capture_output=True, text=True, check=True).stdout
    assert out.split() == ["16", "0", "8"]
    assert C.sizeof(abi.HipTensorPack) == 16


@pytest.mark.skipif(not REF_INC.exists(), reason="reference headers absent")
def test_pack_struct_matches_reference(tmp_path):
    """The reference's CudaTensorPack is {void *data; void *_d_buf;} like its TensorPack; the C
    view of pack.h holds TensorPack only (CudaTensorPack needs the CUDA headers)."""
    src = tmp_path / "probe.c"
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "kernels/pack.h"\n'
                   'int main(void){printf("%zu %zu %zu\\n", sizeof(TensorPack), '
                   'offsetof(TensorPack, data), offsetof(TensorPack, _buf));return 0;}\n')
    subprocess.run(["gcc", "-o", str(tmp_path / "p"), str(src), f"-I{REF_INC}"], check=True)
    out = subprocess.run([str(tmp_path / "p")], capture_output=True, text=True, check=True).stdout
    assert out.split() == ["16", "0", "8"]


def _ref_pack(base: np.ndarray, shape, strides, offset):
    L = ref()
    f, rel = L.tensor_pack_init, L.tensor_pack_release
    f.argtypes = [C.POINTER(abi.HipTensorPack), abi.TensorP]
    rel.argtypes = [C.POINTER(abi.HipTensorPack)]
    hb = HostTensor(base)
    view = HostTensor(shape=shape, strides=strides, base=hb, offset=offset)
    p = abi.HipTensorPack()
    f(C.byref(p), C.byref(view.t))
    n = int(np.prod(shape))
    out = np.ctypeslib.as_array((C.c_float * n).from_address(p.data)).copy().reshape(shape)
    rel(C.byref(p))
    return out


def ref_calls_contiguous(shape, strides) -> bool:
    """The reference's is_contiguous (src/core/tensor.c:32-42): row-major strides on every axis
    but the first."""
    want = 1
    for d in range(len(shape) - 1, 0, -1):
        if strides[d] != want:
            return False
        want *= shape[d]
    return True


def truly_contiguous(shape, strides) -> bool:
    want = 1
    for d in range(len(shape) - 1, -1, -1):
        if shape[d] != 1 and strides[d] != want:
            return False
        want *= shape[d]
    return True


@pytest.mark.skipif(not ref_available(), reason="oracle/_ref not built (needs /root/reference)")
@pytest.mark.parametrize("view", VIEWS, ids=[str(v[1:3]) for v in VIEWS])
def test_reference_pack_is_the_row_major_gather(view):
    """Where the reference's contiguity test is right, its pack is the row-major gather; where
    its strides[0] quirk calls a strided view contiguous, it aliases the view's first numel
    elements of storage instead (the HIP pack gathers in both cases)."""
    bshape, shape, strides, off = view
    base = np.random.RandomState(1).randn(*bshape).astype(np.float32)
    n = int(np.prod(shape))
    quirk = ref_calls_contiguous(shape, strides) and not truly_contiguous(shape, strides)
    if quirk and off + n > base.size:
        pytest.skip("the reference would alias more elements than the storage holds "
                    "(its pack then reads past the buffer); the HIP pack gathers this view")
    got = _ref_pack(base, shape, strides, off)
    if quirk:
        assert_bits(got, base.reshape(-1)[off:off + n].reshape(shape), "reference aliases")
    else:
        assert_bits(got, gather(base, shape, strides, off), "pack")


@pytest.mark.skipif(not ref_available(), reason="oracle/_ref not built (needs /root/reference)")
def test_reference_pack_strides0_quirk_is_the_documented_deviation():
    """The reference's is_contiguous ignores strides[0] (src/core/tensor.c:32-42), so a view that
    skips rows is aliased instead of packed; the HIP pack honours every stride. Here the reference
    returns the base's first rows, the gather the rows the view names."""
    base = np.arange(40, dtype=np.float32).reshape(8, 5)
    got = _ref_pack(base, (3, 5), (10, 1), 0)
    assert_bits(got, base[:3], "reference aliases")
    assert not np.array_equal(got, gather(base, (3, 5), (10, 1), 0))
