"""GPU parity of fused elementwise chains (the tape interpreter, the only fused path): every
chain_cases.TAPES case over a flat space (2^20 + 4 elements, so the last float4 falls in the NEG
rule's tail; this runs the one-shot vector kernel), over whole and partial transposed-operand tiles and over
[rows, inner] layouts with a re-read bias row and per-row scalars. Each fused result must equal the
unfused chain of library ops bit for bit, and, where the chain's error is bounded per element, the
oracle's unfused chain (bit-exact arithmetic, 2 ulp for a final exp). Inputs hold ±0, ±inf, NaN and
subnormals. The config chains also run at their full BASELINE.json sizes: config 2's 64M chain and
config 3's [256, 512, 512] fused broadcast over a permuted view."""
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


def _run(rt, ops, tape, devs, shape=(N,)):
    out = ops.fused(tape, devs, shape)
    rt.lib().check("fused")
    return out.numpy()


def _broadcast_view(rt, dev, shape):
    """dev itself when it has the output's shape, else a stride-0 view of it over that shape (so
    a unary op applied to a broadcast input yields the output's shape; no value changes)."""
    if tuple(dev.shape) == tuple(shape):
        return dev
    from plast_amd import abi
    src_shape = abi.shape_of(dev.t)
    src_st = [int(dev.t.strides[d]) for d in range(len(src_shape))]
    lead = len(shape) - len(src_shape)
    st = [0 if d < lead or src_shape[d - lead] == 1 else src_st[d - lead] for d in range(len(shape))]
    return rt.DeviceTensor(shape, base=dev, strides=st, zero=False)


def _unfused(rt, ins, devs, shape):
    """The chain as one library op per instruction (each op pinned to the oracle elsewhere)."""
    from plast_amd.abi import KernelParams
    n1 = {"NEG": "neg", "EXP": "exp", "LOG": "log", "ABS": "abs", "SIN": "sin", "COS": "cos",
          "TAN": "tan", "LEAKY_RELU": "leaky_relu"}
    n2 = {"ADD": "add", "SUB": "sub", "MUL": "mul", "DIV": "div"}
    acc = _broadcast_view(rt, devs[ins[0][2]], shape)
    keep = []
    for op, src, idx, rhs, imm in ins[1:]:
        out = rt.DeviceTensor(shape, zero=False)
        if op in n1:
            rt.forward(n1[op], [acc], out, KernelParams(0, 0, imm))
        else:
            if src == 1:
                o = devs[idx]
            elif src == 3:
                o = rt.DeviceTensor.from_numpy(np.array([imm], np.float32))
                keep.append(o)
            else:
                o = acc
            a, b = (o, acc) if rhs else (acc, o)
            rt.forward(n2[op], [a, b], out)
        acc = out
    return acc.numpy()


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


def _inexact_positions(ins):
    return [i for i, (op, *_) in enumerate(ins) if op in ("EXP", "LOG", "SIN", "COS", "TAN")]


def _check_against_oracle(name, got, ins, hosts, n):
    """Exact chains bit for bit; chains whose only inexact op comes last within 2 ulp (elsewhere an
    inexact op's last-place difference is amplified by what follows; the unfused-op equality is the
    check there)."""
    from gpu_backend import ulp_distance
    inexact = _inexact_positions(ins)
    if inexact and inexact != [len(ins) - 1]:
        return
    want = _oracle(ins, hosts, n)
    if inexact:
        d = ulp_distance(got, want)
        assert int(np.max(d)) <= 2, f"{name}: {int(np.max(d))} ulp"
    else:
        assert_bits(got, want, f"{name}: fused vs oracle")


@pytest.mark.parametrize("case", TAPES, ids=[t[0] for t in TAPES])
def test_flat_chain_matches_unfused_ops_and_oracle(case):
    from plast_amd import ops, runtime as rt
    name, nin, bcast, ins = case
    print(f"chain {name} over {N}", flush=True)
    xs = _inputs(nin, bcast, 7)
    devs = [rt.DeviceTensor.from_numpy(x) for x in xs]
    tape = ops.make_tape(ins, nin)
    got = _run(rt, ops, tape, devs)
    assert_bits(got, _unfused(rt, ins, devs, (N,)), f"{name}: fused vs unfused ops")
    _check_against_oracle(name, got, ins, xs, N)


@pytest.mark.parametrize("n", [1, 3, 4, 5, 8, 255, 1024, 1027, 65536 * 4 + 12, 3 * (1 << 18) + 20])
def test_flat_chain_sizes(n):
    """Sizes around the vector kernel's float4 units and two-unit lanes, and around the NEG rule's
    8-element SIMD blocks, on config 2's chain."""
    from plast_amd import ops, runtime as rt
    name, nin, _, ins = TAPES[0]
    print(f"config-2 chain over {n}", flush=True)
    rng = np.random.RandomState(n)
    xs = [rng.randn(n).astype(np.float32) for _ in range(nin)]
    xs[0][: min(n, 4)] = [0.0, -0.0, 1.0, -1.0][: min(n, 4)]
    devs = [rt.DeviceTensor.from_numpy(x) for x in xs]
    got = _run(rt, ops, ops.make_tape(ins, nin), devs, (n,))
    assert_bits(got, _unfused(rt, ins, devs, (n,)), f"n={n}: fused vs unfused ops")
    _check_against_oracle(f"n={n}", got, ins, xs, n)


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
def test_tile_chain_matches_unfused_ops_and_oracle(case, kinds):
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
    got = _run(rt, ops, tape, devs, (B_, P_, Q_)).reshape(-1)
    assert_bits(got, _unfused(rt, ins, devs, (B_, P_, Q_)).reshape(-1),
                f"{name}: fused tile vs unfused ops")
    _check_against_oracle(name, got, ins, hosts, B_ * P_ * Q_)


# ------------------------------------------------------------------ rows form
ROWS_CASES = [
    (TAPES[0], (2048, 1024), ["full", "row", "full"]),          # a bias row re-read for every row
    (TAPES[0], (2047, 1028), ["full", "row", "col"]),           # plus a per-row scalar; NEG tail
    (TAPES[1], (2048, 1024), ["row", "full"]),
    (TAPES[4], (2048, 1024), ["full", "col", "full", "row"]),
]


@pytest.mark.parametrize("case, shape, kinds", ROWS_CASES,
                         ids=[f"{c[0]}-{s[0]}x{s[1]}-{'-'.join(k)}" for c, s, k in ROWS_CASES])
def test_rows_chain_matches_unfused_ops_and_oracle(case, shape, kinds):
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
    got = _run(rt, ops, tape, devs, (R, Cn)).reshape(-1)
    assert_bits(got, _unfused(rt, ins, devs, (R, Cn)).reshape(-1), f"{name}: fused rows vs unfused")
    _check_against_oracle(name, got, ins, hosts, R * Cn)


def test_rows_chain_into_a_strided_output_view():
    """The output is a column slice of a wider tensor (rows padded to 1280 floats): the chain writes
    through the output's row stride and leaves the padding alone. The NEG in the middle of the chain
    reads and writes contiguous intermediates in the unfused chain, so it takes the reference's
    contiguous form (0 - x, every index below the SIMD end) even though the final output is
    strided."""
    import ctypes as C
    from plast_amd import ops, runtime as rt
    from plast_amd.abi import KernelParams
    R, Cn, W, off = 2048, 1024, 1280, 128
    print("rows chain into a strided view", flush=True)
    rng = np.random.RandomState(23)
    x = rng.randn(R, Cn).astype(np.float32)
    x[0, :4] = [0.0, -0.0, 1.0, -1.0]
    b = rng.uniform(-1, 1, (1, Cn)).astype(np.float32)
    tape = ops.make_tape([("LOAD", 0, 0, 0, 0.0), ("ADD", 1, 1, 0, 0.0), ("NEG", 0, 0, 0, 0.0),
                          ("LEAKY_RELU", 0, 0, 0, 0.0)], 2)
    dx, db = rt.DeviceTensor.from_numpy(x), rt.DeviceTensor.from_numpy(b)
    base = rt.DeviceTensor.from_numpy(np.full((R, W), 7.0, np.float32))
    view = rt.DeviceTensor((R, Cn), base=base, strides=(W, 1), offset=off, zero=False)
    rt.forward("fused_elementwise", [dx, db], view, KernelParams(C.addressof(tape), 0, 0.0))
    got = base.numpy()
    assert (got[:, :off] == 7.0).all() and (got[:, off + Cn:] == 7.0).all(), "padding overwritten"
    s = (x + b).astype(np.float32)
    want = np.float32(0.0) - s                    # the contiguous form of NEG: 0 - x, so 0 - (+0) = +0
    want = np.where(want > 0, want, want * np.float32(0.0))
    assert_bits(got[:, off:off + Cn], want, "fused rows into a view vs closed form")


@pytest.mark.parametrize("where", ["first_on_permuted_input", "last_into_strided_output",
                                   "first_on_contiguous_input"])
def test_neg_rule_follows_each_negs_own_operands(where):
    """The reference's neg computes 0 - x inside its 8-wide SIMD blocks only when its input and its
    output are both contiguous (kernel_macros.h:19-31), and -x otherwise; the two differ on signed
    zeros. In a chain only a NEG reading the loaded input or writing the chain's output can meet a
    strided tensor. Each case must equal the unfused ops (which apply the rule per op) bit for bit."""
    import ctypes as C
    from plast_amd import ops, runtime as rt
    from plast_amd.abi import KernelParams
    print(f"neg rule: {where}", flush=True)
    I, J, K = 4, 64, 128
    rng = np.random.RandomState(5)
    base = rng.randn(I, K, J).astype(np.float32)
    base.reshape(-1)[::3] = 0.0
    base.reshape(-1)[1::7] = -0.0
    bias = rng.uniform(-1, 1, (1, J, 1)).astype(np.float32)
    bias.reshape(-1)[::2] = 0.0
    dbase, dbias = rt.DeviceTensor.from_numpy(base), rt.DeviceTensor.from_numpy(bias)
    if where == "first_on_permuted_input":
        x = rt.DeviceTensor((I, J, K), base=dbase, strides=(J * K, 1, J), zero=False)
        ins = [("LOAD", 0, 0, 0, 0.0), ("NEG", 0, 0, 0, 0.0), ("ADD", 1, 1, 0, 0.0)]
    elif where == "first_on_contiguous_input":
        x = rt.DeviceTensor.from_numpy(base.transpose(0, 2, 1).copy())
        ins = [("LOAD", 0, 0, 0, 0.0), ("NEG", 0, 0, 0, 0.0), ("ADD", 1, 1, 0, 0.0)]
    else:
        x = rt.DeviceTensor.from_numpy(base.transpose(0, 2, 1).copy())
        ins = [("LOAD", 0, 0, 0, 0.0), ("ADD", 1, 1, 0, 0.0), ("NEG", 0, 0, 0, 0.0)]
    tape = ops.make_tape(ins, 2)
    if where == "last_into_strided_output":
        # the output is the permuted view of a contiguous buffer
        obuf = rt.DeviceTensor((I, K, J), zero=False)
        out = rt.DeviceTensor((I, J, K), base=obuf, strides=(J * K, 1, J), zero=False)
        rt.forward("fused_elementwise", [x, dbias], out, KernelParams(C.addressof(tape), 0, 0.0))
        got = obuf.numpy().reshape(I, K, J).transpose(0, 2, 1)
        t = rt.DeviceTensor((I, J, K), zero=False)
        rt.forward("add", [x, dbias], t)
        obuf2 = rt.DeviceTensor((I, K, J), zero=False)
        out2 = rt.DeviceTensor((I, J, K), base=obuf2, strides=(J * K, 1, J), zero=False)
        rt.forward("neg", [t], out2)
        want = obuf2.numpy().reshape(I, K, J).transpose(0, 2, 1)
    else:
        got = ops.fused(tape, [x, dbias], (I, J, K)).numpy()
        want = _unfused(rt, ins, [x, dbias], (I, J, K))
    assert_bits(np.ascontiguousarray(got), np.ascontiguousarray(want), f"{where}: fused vs unfused")


# ------------------------------------------------------------------ config sizes
def test_config2_chain_at_full_size():
    """Config 2 at its BASELINE.json size: exp(-relu(a*b + c)) over 2^26 elements (a, b, c ~ N(0,1),
    the bench's device-generated inputs) through the scheduler-fused node, against the oracle's
    unfused chain over every element: add/mul/relu/neg bit-exact, so the whole chain is within the
    2 ulp of its final exp."""
    from gpu_backend import ulp_distance
    from hostlib import fused_chain2
    from plast_amd import ops, runtime as rt
    n = 1 << 26
    print("config 2 at 2^26", flush=True)
    a, b, c = (rt.DeviceTensor((n,), zero=False).fill_("normal", s, 0.0, 1.0) for s in (42, 43, 44))
    tape = ops.make_tape(TAPES[0][3], 3)
    got = _run(rt, ops, tape, [a, b, c], (n,))
    want = fused_chain2(a.numpy(), b.numpy(), c.numpy())
    d = ulp_distance(got, want)
    assert int(d.max()) <= 2, f"config 2: {int(d.max())} ulp at {int(np.argmax(d))}"


def test_config3_at_full_size():
    """Config 3 at its BASELINE.json size: A [256, 512, 512] ~ N(0,1) as the permuted (0, 2, 1) view,
    B [1, 512, 1] and C [256, 1, 512] ~ U(0.5, 1.5). The add, the multiply and the fused chain, each
    bit-exact against the oracle's broadcast ops over all 2^26 outputs."""
    from hostlib import HostTensor, oracle_forward
    from plast_amd import ops, runtime as rt
    print("config 3 at [256, 512, 512]", flush=True)
    shp = (256, 512, 512)
    Ab = rt.DeviceTensor(shp, zero=False).fill_("normal", 42, 0.0, 1.0)
    Av = rt.DeviceTensor(shp, base=Ab, strides=(262144, 1, 512), zero=False)
    B = rt.DeviceTensor((1, 512, 1), zero=False).fill_("uniform", 43, 0.5, 1.5)
    Cm = rt.DeviceTensor((256, 1, 512), zero=False).fill_("uniform", 44, 0.5, 1.5)
    T = rt.DeviceTensor(shp, zero=False)
    O = rt.DeviceTensor(shp, zero=False)
    rt.forward("add", [Av, B], T)
    rt.forward("mul", [T, Cm], O)
    tape = ops.make_tape([("LOAD", 0, 0, 0, 0.0), ("ADD", 1, 1, 0, 0.0), ("MUL", 1, 2, 0, 0.0)], 3)
    F = ops.fused(tape, [Av, B, Cm], shp)
    hA = HostTensor(Ab.numpy().reshape(shp))
    hv = HostTensor(base=hA, shape=shp, strides=(262144, 1, 512))
    hB, hC = HostTensor(B.numpy().reshape(1, 512, 1)), HostTensor(Cm.numpy().reshape(256, 1, 512))
    hT, hO = HostTensor(np.zeros(shp, np.float32)), HostTensor(np.zeros(shp, np.float32))
    oracle_forward("add", [hv, hB], hT)
    oracle_forward("mul", [hT, hC], hO)
    assert_bits(T.numpy().reshape(shp), hT.numpy(), "config 3 add vs oracle")
    assert_bits(O.numpy().reshape(shp), hO.numpy(), "config 3 mul vs oracle")
    assert_bits(F.numpy().reshape(shp), hO.numpy(), "config 3 fused vs oracle")
