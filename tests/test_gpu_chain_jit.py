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


def _oracle(ins, xs):
    """The unfused chain, node by node, through the oracle's ops (ones the reference runs)."""
    from hostlib import HostTensor, oracle_forward
    from plast_amd.abi import KernelParams
    n1 = {"NEG": "neg", "EXP": "exp", "LOG": "log", "ABS": "abs", "SIN": "sin", "COS": "cos",
          "TAN": "tan"}
    n2 = {"ADD": "add", "SUB": "sub", "MUL": "mul", "DIV": "div"}
    full = [np.broadcast_to(x, (N,)).astype(np.float32) for x in xs]
    acc = full[ins[0][2]].copy()
    for op, src, idx, rhs, imm in ins[1:]:
        out = HostTensor(np.zeros(N, np.float32))
        if op in n1:
            oracle_forward(n1[op], [HostTensor(acc)], out)
        elif op == "LEAKY_RELU":
            oracle_forward("leaky_relu", [HostTensor(acc)], out, KernelParams(0, 0, imm))
        else:
            o = full[idx] if src == 1 else np.full(N, imm, np.float32) if src == 3 else acc
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
