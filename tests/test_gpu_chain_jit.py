"""GPU parity of the chain compiler: every chain_cases.TAPES case over a flat space past the
compiler's threshold (2^20 elements, plus 4 so the last float4 falls in the NEG rule's tail), run
once compiled and once on the tape interpreter; the two outputs must be bit-identical, the compiled
run must have been a compiled launch, and, where the chain's error is bounded per element, both
match the oracle's unfused chain (bit-exact arithmetic, 2 ulp for a final exp). Inputs hold ±0,
±inf, NaN and subnormals, and the last float4 lies in the NEG rule's tail."""
from __future__ import annotations

import numpy as np
import pytest

from cases import assert_bits
from chain_cases import TAPES

pytestmark = pytest.mark.gpu
N = (1 << 20) + 4


def _inputs(nin, bcast, seed):
    rng = np.random.RandomState(seed)
    xs = []
    for k in range(nin):
        if bcast >> k & 1:
            xs.append(np.array([rng.uniform(0.5, 2.0)], np.float32))
            continue
        x = rng.randn(N).astype(np.float32) * 3
        x[:8] = [0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -1e-40, 88.0]
        x[-4:] = [-0.0, 0.0, 1e-39, -2.0]
        xs.append(x)
    return xs


def _run(rt, ops, tape, devs, jit):
    L = rt.lib()
    prev = L.plast_hip_set_chain_jit(1 if jit else 0)
    before = L.plast_hip_chain_jit_launches()
    try:
        out = ops.fused(tape, devs, (N,))
        L.check("fused")
    finally:
        L.plast_hip_set_chain_jit(prev)
    return out.numpy(), L.plast_hip_chain_jit_launches() - before


def _oracle(ins, xs, n=N):
    """The unfused chain, node by node, through the oracle's ops (ones the reference runs), over n
    elements (inputs of one element are broadcast scalars)."""
    from hostlib import HostTensor, oracle_forward
    from plast_amd.abi import KernelParams
    n1 = {"NEG": "neg", "EXP": "exp", "LOG": "log", "ABS": "abs", "SIN": "sin", "COS": "cos",
          "TAN": "tan"}
    n2 = {"ADD": "add", "SUB": "sub", "MUL": "mul", "DIV": "div"}
    full = [np.broadcast_to(x, (n,)).astype(np.float32) for x in xs]
    acc = full[ins[0][2]].copy()
    for op, src, idx, rhs, imm in ins[1:]:
        out = HostTensor(np.zeros(n, np.float32))
        if op in n1:
            oracle_forward(n1[op], [HostTensor(acc)], out)
        elif op == "LEAKY_RELU":
            oracle_forward("leaky_relu", [HostTensor(acc)], out, KernelParams(0, 0, imm))
        else:
            o = full[idx] if src == 1 else np.full(n, imm, np.float32) if src == 3 else acc
            a, b = (o, acc) if rhs else (acc, o)
            oracle_forward(n2[op], [HostTensor(np.ascontiguousarray(a)), HostTensor(np.ascontiguousarray(b))], out)
        acc = out.numpy().copy()
    return acc


@pytest.mark.parametrize("case", TAPES, ids=[t[0] for t in TAPES])
def test_compiled_chain_matches_interpreter_and_oracle(case):
    from gpu_backend import ulp_distance
    from plast_amd import ops, runtime as rt
    name, nin, bcast, ins = case
    print(f"chain {name} over {N}", flush=True)
    xs = _inputs(nin, bcast, 7)
    devs = [rt.DeviceTensor.from_numpy(x) for x in xs]
    tape = ops.make_tape(ins, nin)
    got, launched = _run(rt, ops, tape, devs, jit=True)
    assert launched == 1, "the chain did not run compiled"
    interp, launched = _run(rt, ops, tape, devs, jit=False)
    assert launched == 0
    assert_bits(got, interp, f"{name}: compiled vs interpreter")
    # against the oracle where the chain's error is bounded per element: exact chains bit for bit,
    # chains whose only inexact op comes last within 2 ulp (elsewhere an inexact op's last-place
    # difference is amplified by what follows; the interpreter's equality above is the check)
    inexact = [i for i, (op, *_) in enumerate(ins) if op in ("EXP", "LOG", "SIN", "COS", "TAN")]
    if inexact and inexact != [len(ins) - 1]:
        return
    want = _oracle(ins, xs)
    if inexact:
        d = ulp_distance(got, want)
        assert int(np.max(d)) <= 2, f"{name}: {int(np.max(d))} ulp"
    else:
        assert_bits(got, want, f"{name}: compiled vs oracle")


def test_below_threshold_and_strided_chains_stay_on_the_interpreter():
    from plast_amd import ops, runtime as rt
    L = rt.lib()
    tape = ops.make_tape(TAPES[0][3], 3)
    small = [rt.DeviceTensor.from_numpy(np.ones(4096, np.float32)) for _ in range(3)]
    before = L.plast_hip_chain_jit_launches()
    ops.fused(tape, small, (4096,))
    assert L.plast_hip_chain_jit_launches() == before


# ------------------------------------------------------------------ tile form
B_, P_, Q_ = 16, 256, 256        # 2^20 outputs of [16, 256, 256], whole 64x64 tiles


def _operand(rt, kind, seed):
    """(device tensor over the output space, host array of the same values as [16, 256, 256])."""
    rng = np.random.RandomState(seed)
    if kind == "permuted":           # permute (0, 2, 1) of a contiguous base: staged through LDS
        base = rng.randn(B_, P_, Q_).astype(np.float32)
        base[0, 0, :8] = [0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -1e-40, 5.0]
        d = rt.DeviceTensor.from_numpy(base)
        v = rt.DeviceTensor((B_, P_, Q_), base=d, strides=(P_ * Q_, 1, Q_), zero=False)
        return (d, v), base.transpose(0, 2, 1)
    if kind == "contiguous":         # read directly
        a = rng.randn(B_, P_, Q_).astype(np.float32)
        return (rt.DeviceTensor.from_numpy(a),), a
    if kind == "row":                # [1, P, 1]: one scalar per output row
        a = rng.uniform(0.5, 1.5, (1, P_, 1)).astype(np.float32)
        return (rt.DeviceTensor.from_numpy(a),), np.broadcast_to(a, (B_, P_, Q_))
    a = rng.uniform(0.5, 1.5, (B_, 1, Q_)).astype(np.float32)   # "col": one float4 along p
    return (rt.DeviceTensor.from_numpy(a),), np.broadcast_to(a, (B_, P_, Q_))


TILE_CASES = [
    (TAPES[0], ["permuted", "row", "col"]),                    # config 3's roles (0, 1, 2)
    (TAPES[0], ["permuted", "contiguous", "contiguous"]),      # (0, 3, 3)
    (TAPES[1], ["permuted", "permuted"]),                      # (0, 0): two LDS slots
    (TAPES[1], ["contiguous", "permuted"]),                    # (3, 0)
    (TAPES[2], ["permuted"]),                                  # (0)
    (TAPES[3], ["col", "permuted"]),                           # (2, 0)
    (TAPES[4], ["permuted", "row", "contiguous", "col"]),      # (0, 1, 3, 2): runtime-role interpreter
]


@pytest.mark.parametrize("case, kinds", TILE_CASES, ids=[f"{c[0]}-{'-'.join(k)}" for c, k in TILE_CASES])
def test_compiled_tile_matches_interpreter_and_oracle(case, kinds):
    from gpu_backend import ulp_distance
    from plast_amd import ops, runtime as rt
    name, nin, _, ins = case
    print(f"tile chain {name} {kinds}", flush=True)
    keep, devs, hosts = [], [], []
    for k, kind in enumerate(kinds):
        d, h = _operand(rt, kind, 11 + k)
        keep.append(d)
        devs.append(d[-1])
        hosts.append(np.ascontiguousarray(h).reshape(-1))
    tape = ops.make_tape(ins, nin)
    L = rt.lib()

    def run(jit):
        prev = L.plast_hip_set_chain_jit(1 if jit else 0)
        before = L.plast_hip_chain_jit_launches()
        try:
            out = ops.fused(tape, devs, (B_, P_, Q_))
            L.check("fused")
        finally:
            L.plast_hip_set_chain_jit(prev)
        return out.numpy().reshape(-1), L.plast_hip_chain_jit_launches() - before

    got, n = run(True)
    assert n == 1, "the chain did not run compiled"
    interp, n = run(False)
    assert n == 0
    assert_bits(got, interp, f"{name}: compiled tile vs interpreter")
    inexact = [i for i, (op, *_) in enumerate(ins) if op in ("EXP", "LOG", "SIN", "COS", "TAN")]
    if inexact and inexact != [len(ins) - 1]:
        return
    want = _oracle(ins, hosts, B_ * P_ * Q_)
    if inexact:
        assert int(np.max(ulp_distance(got, want))) <= 2
    else:
        assert_bits(got, want, f"{name}: compiled tile vs oracle")


# ------------------------------------------------------------------ rows form
ROWS_CASES = [
    (TAPES[0], (2048, 1024), ["full", "row", "full"]),          # a bias row re-read for every row
    (TAPES[0], (2047, 1028), ["full", "row", "col"]),           # plus a per-row scalar; NEG tail
    (TAPES[1], (2048, 1024), ["row", "full"]),
    (TAPES[4], (2048, 1024), ["full", "col", "full", "row"]),
]


@pytest.mark.parametrize("case, shape, kinds", ROWS_CASES,
                         ids=[f"{c[0]}-{s[0]}x{s[1]}-{'-'.join(k)}" for c, s, k in ROWS_CASES])
def test_compiled_rows_match_interpreter_and_oracle(case, shape, kinds):
    from gpu_backend import ulp_distance
    from plast_amd import ops, runtime as rt
    name, nin, _, ins = case
    R, Cn = shape
    print(f"rows chain {name} {shape} {kinds}", flush=True)
    rng = np.random.RandomState(17)
    hosts, devs = [], []
    for kind in kinds:
        if kind == "full":
            a = (rng.randn(R, Cn) * 2).astype(np.float32)
            a[0, :6] = [0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40]
        elif kind == "row":
            a = rng.uniform(0.5, 1.5, (1, Cn)).astype(np.float32)
        else:
            a = rng.uniform(0.5, 1.5, (R, 1)).astype(np.float32)
        devs.append(rt.DeviceTensor.from_numpy(a))
        hosts.append(np.ascontiguousarray(np.broadcast_to(a, (R, Cn))).reshape(-1))
    tape = ops.make_tape(ins, nin)
    L = rt.lib()

    def run(jit):
        prev = L.plast_hip_set_chain_jit(1 if jit else 0)
        before = L.plast_hip_chain_jit_launches()
        try:
            out = ops.fused(tape, devs, (R, Cn))
            L.check("fused")
        finally:
            L.plast_hip_set_chain_jit(prev)
        return out.numpy().reshape(-1), L.plast_hip_chain_jit_launches() - before

    got, n = run(True)
    assert n == 1, "the chain did not run compiled"
    interp, n = run(False)
    assert n == 0
    assert_bits(got, interp, f"{name}: compiled rows vs interpreter")
    inexact = [i for i, (op, *_) in enumerate(ins) if op in ("EXP", "LOG", "SIN", "COS", "TAN")]
    if inexact and inexact != [len(ins) - 1]:
        return
    want = _oracle(ins, hosts, R * Cn)
    if inexact:
        assert int(np.max(ulp_distance(got, want))) <= 2
    else:
        assert_bits(got, want, f"{name}: compiled rows vs oracle")


def test_compiled_rows_into_a_strided_output_view():
    """The output is a column slice of a wider tensor (rows padded to 1280 floats): the rows form
    writes through the output's row stride and leaves the padding alone, and since the output is
    not contiguous the NEG rule takes its tail form (-x) everywhere, as the interpreter does."""
    from plast_amd import ops, runtime as rt
    L = rt.lib()
    R, Cn, W, off = 2048, 1024, 1280, 128
    print("rows chain into a strided view", flush=True)
    rng = np.random.RandomState(23)
    x = rng.randn(R, Cn).astype(np.float32)
    x[0, :4] = [0.0, -0.0, 1.0, -1.0]
    b = rng.uniform(-1, 1, (1, Cn)).astype(np.float32)
    tape = ops.make_tape([("LOAD", 0, 0, 0, 0.0), ("ADD", 1, 1, 0, 0.0), ("NEG", 0, 0, 0, 0.0),
                          ("LEAKY_RELU", 0, 0, 0, 0.0)], 2)
    dx, db = rt.DeviceTensor.from_numpy(x), rt.DeviceTensor.from_numpy(b)
    results = []
    for jit in (1, 0):
        base = rt.DeviceTensor.from_numpy(np.full((R, W), 7.0, np.float32))
        view = rt.DeviceTensor((R, Cn), base=base, strides=(W, 1), offset=off, zero=False)
        prev = L.plast_hip_set_chain_jit(jit)
        before = L.plast_hip_chain_jit_launches()
        try:
            from plast_amd.abi import KernelParams
            import ctypes as C
            rt.forward("fused_elementwise", [dx, db], view, KernelParams(C.addressof(tape), 0, 0.0))
        finally:
            L.plast_hip_set_chain_jit(prev)
        assert L.plast_hip_chain_jit_launches() - before == jit
        results.append(base.numpy())
    got, interp = results
    assert_bits(got, interp, "compiled rows into a view vs interpreter")
    assert (got[:, :off] == 7.0).all() and (got[:, off + Cn:] == 7.0).all(), "padding overwritten"
    s = (x + b).astype(np.float32)
    want = -s                                     # the tail form of NEG: -x, so -(+0) = -0
    want = np.where(want > 0, want, want * np.float32(0.0))
    assert_bits(got[:, off:off + Cn], want, "compiled rows into a view vs closed form")
