"""CPU checks of the chain compiler: the source it writes for each case of chain_cases.TAPES
compiles with hiprtc for gfx950 under the library's own flags (no device needed), and spells out
each tape instruction as the interpreter's statement for it (TapeBody::eval_units in ew.hpp)."""
from __future__ import annotations

import ctypes as C

import pytest

from chain_cases import TAPES
from plast_amd import abi
from plast_amd.ops import make_tape

try:
    RTC = C.CDLL("libhiprtc.so.7")
except OSError:
    RTC = None


_L = []


def _lib():
    """The library without device initialisation (the source writer needs no device)."""
    if not _L:
        from plast_amd.runtime import Library
        _L.append(Library())
    return _L[0]


def source(ins, nin, pattern, tile=False, rows=False) -> str:
    """The flat form's source (pattern: broadcast mask), the rows form's (pattern: per-row scalar
    mask | re-read mask << 8) or the tile form's (pattern: roles)."""
    tape = make_tape(ins, nin)
    L = _lib()
    f = (L.plast_hip_chain_jit_tile_source if tile else
         L.plast_hip_chain_jit_rows_source if rows else L.plast_hip_chain_jit_source)
    n = f(C.addressof(tape), pattern, None, 0)
    assert n > 0
    buf = C.create_string_buffer(int(n) + 1)
    assert f(C.addressof(tape), pattern, buf, n + 1) == n
    return buf.value.decode()


def roles(*r):
    return sum(v << (2 * k) for k, v in enumerate(r))


# (tape case, roles): config 3's pattern and the others the fixed-role interpreter instantiates,
# plus one that only the compiled form covers
TILE_CASES = [(TAPES[0], roles(0, 1, 2)), (TAPES[0], roles(0, 3, 3)), (TAPES[0], roles(0, 0, 0)),
              (TAPES[1], roles(0, 0)), (TAPES[1], roles(3, 0)), (TAPES[2], roles(0)),
              (TAPES[3], roles(2, 0)), (TAPES[4], roles(0, 1, 3, 2))]


def test_malformed_tape_gives_no_source():
    tape = abi.FusedTape()
    assert _lib().plast_hip_chain_jit_source(C.addressof(tape), 0, None, 0) == 0


def test_config2_statements():
    name, nin, bcast, ins = TAPES[0]
    s = source(ins, nin, bcast)
    body = [l.strip() for l in s.splitlines() if l.strip().startswith("a = ")]
    assert body == ["a = a * x1[c];", "a = a + x2[c];", "a = a > 0.0f ? a : a * A.imm[3];",
                    "a = simd ? 0.0f - a : -a;", "a = expf(a);"]
    assert "float a = x0[c];" in s
    assert s.count("__builtin_nontemporal_load") == 3


def test_operand_orders_and_broadcast_scalars():
    s = source(TAPES[1][3], 2, 0)
    body = [l.strip() for l in s.splitlines() if l.strip().startswith("a = ")]
    assert body == ["a = x0[c] - a;", "a = a / x1[c];", "a = a - A.imm[3];", "a = A.imm[4] / a;",
                    "a = a + a;"]
    s = source(TAPES[4][3], 4, 0b1010)
    assert "const f4 x1 = f4(A.in[1][0]);" in s and "const f4 x3 = f4(A.in[3][0]);" in s
    assert s.count("__builtin_nontemporal_load") == 2


def test_tile_source_follows_roles():
    (name, nin, _, ins), r = TILE_CASES[0]
    s = source(ins, nin, r, tile=True)
    assert s.count("__builtin_nontemporal_load") == 1          # operand 0 staged
    assert "v1[r] = src[r * step]" in s                         # operand 1: scalar per row
    assert "const f4 v2 = *(const f4 *)" in s                   # operand 2: one float4 along p
    assert "__syncthreads();" in s
    assert "a = a * x1[c];" in s and "a = expf(a);" in s


def _compile(src: bytes):
    prog = C.c_void_p()
    assert RTC.hiprtcCreateProgram(C.byref(prog), src, b"plast_chain.hip", 0, None, None) == 0
    opts = [b"--offload-arch=gfx950", b"-O3", b"-std=c++17", b"-ffp-contract=off",
            b"-Xclang", b"-target-feature", b"-Xclang", b"-packed-fp32-ops"]
    arr = (C.c_char_p * len(opts))(*opts)
    rc = RTC.hiprtcCompileProgram(prog, len(opts), arr)
    size = C.c_size_t(0)
    RTC.hiprtcGetProgramLogSize(prog, C.byref(size))
    log = C.create_string_buffer(size.value + 1)
    RTC.hiprtcGetProgramLog(prog, log)
    code = C.c_size_t(0)
    RTC.hiprtcGetCodeSize(prog, C.byref(code))
    RTC.hiprtcDestroyProgram(C.byref(prog))
    assert rc == 0, log.value.decode(errors="replace")
    assert code.value > 1000


@pytest.mark.skipif(RTC is None, reason="libhiprtc not present")
@pytest.mark.parametrize("case, r", TILE_CASES, ids=[f"{c[0]}-{r:x}" for c, r in TILE_CASES])
def test_generated_tile_source_compiles_for_gfx950(case, r):
    name, nin, _, ins = case
    _compile(source(ins, nin, r, tile=True).encode())


@pytest.mark.skipif(RTC is None, reason="libhiprtc not present")
@pytest.mark.parametrize("case", TAPES, ids=[t[0] for t in TAPES])
def test_generated_source_compiles_for_gfx950(case):
    name, nin, bcast, ins = case
    _compile(source(ins, nin, bcast).encode())


# (tape case, per-row scalar mask, re-read mask): a bias row, a per-row scalar, both
ROWS_CASES = [(TAPES[0], 0b000, 0b010), (TAPES[0], 0b100, 0b010), (TAPES[1], 0b00, 0b01),
              (TAPES[4], 0b0010, 0b1000)]


def test_rows_source_follows_pattern():
    (name, nin, _, ins), sc, rr = ROWS_CASES[1]
    s = source(ins, nin, sc | rr << 8, rows=True)
    assert "x2_0 = f4(*(A.in[2] + (long long)row0 * A.ist[2]));" in s   # per-row scalar
    assert "x1_0 = *(const f4 *)(A.in[1]" in s                          # re-read row
    assert "x0_0 = __builtin_nontemporal_load(" in s                    # x0 streams
    assert "*dst = r;" in s                                             # ordinary stores
    assert "gridDim.x / 8" not in s                                               # dispatch order


@pytest.mark.skipif(RTC is None, reason="libhiprtc not present")
@pytest.mark.parametrize("case, sc, rr", ROWS_CASES, ids=[f"{c[0]}-{s:x}-{r:x}" for c, s, r in ROWS_CASES])
def test_generated_rows_source_compiles_for_gfx950(case, sc, rr):
    name, nin, _, ins = case
    _compile(source(ins, nin, sc | rr << 8, rows=True).encode())
