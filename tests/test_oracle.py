"""CPU tests that pin the oracle (oracle/oracle.c) before it is trusted as the GPU parity checker:
against the compiled reference, the committed golden vectors made from it, and closed forms."""
from __future__ import annotations

import re
from pathlib import Path

import numpy as np
import pytest

from cases import CASES, assert_bits, assert_close_sum, materialize, run_case
from hostlib import (HostBackend, HostTensor, fused_chain2, libm_expf, native_available, oracle_backward,
                     oracle_forward, ref_available, ref_ce_chain, ref_forward)
from plast_amd.abi import DIM_ALL, KernelParams

GOLDEN = Path(__file__).resolve().parent / "golden" / "reference_cases.npz"
REF_CASES = [c for c in CASES if c.op != "argmax"]


def _key(case_id):
    return re.sub(r"[^A-Za-z0-9_.-]+", "_", case_id)


def _compare(c, got: dict, want: dict, what: str):
    assert set(got) == set(want), f"{c.id}: outputs {sorted(got)} vs {sorted(want)}"
    for k in want:
        if c.exact:
            assert_bits(got[k], want[k], f"{c.id}:{k} ({what})")
        else:
            scale = np.abs(want[k]).astype(np.float64) + 1.0
            assert_close_sum(got[k], want[k], scale, 1e-5, f"{c.id}:{k} ({what})")


@pytest.mark.skipif(not ref_available(), reason="oracle/_ref not built (needs /root/reference)")
@pytest.mark.parametrize("c", REF_CASES, ids=[c.id for c in REF_CASES])
def test_oracle_matches_compiled_reference(c):
    _compare(c, run_case(HostBackend("oracle"), c), run_case(HostBackend("ref"), c), "vs reference")


def test_oracle_matches_golden_vectors():
    assert GOLDEN.exists(), "tests/golden/reference_cases.npz missing"
    g = np.load(GOLDEN, allow_pickle=False)
    checked = 0
    for c in REF_CASES:
        k = _key(c.id)
        for i, a in enumerate(c.inputs):
            np.testing.assert_array_equal(a.base_array(), g[f"{k}@in{i}"], err_msg=f"{c.id} input {i}")
        want = {n.split("@", 1)[1]: g[n] for n in g.files
                if n.startswith(k + "@") and not n[len(k) + 1:].startswith("in")}
        _compare(c, run_case(HostBackend("oracle"), c), want, "vs golden")
        checked += 1
    assert checked == len(REF_CASES)


@pytest.mark.parametrize("c", [c for c in CASES if c.op == "argmax"], ids=lambda c: c.id)
def test_argmax_is_numpy_argmax(c):
    """argmax has no reference op: it is pinned to numpy.argmax (first max, first NaN)."""
    out = run_case(HostBackend("oracle"), c)["out"]
    x = materialize(HostBackend("oracle"), c.inputs[0])[0].numpy()
    dim, keep, _ = c.params
    if dim == DIM_ALL:
        want = np.array([np.argmax(x)])
    else:
        want = np.argmax(x, axis=dim)
        if keep:
            want = np.expand_dims(want, dim)
        if want.ndim == 0:
            want = want.reshape(1)
    np.testing.assert_array_equal(out, want.astype(np.int64))


@pytest.mark.parametrize("n", [1, 7, 1000, 100_003])
def test_sum_and_mean_within_serial_bound(n):
    """Serial fp32 summation error is at most (n-1)*u*sum|x| (u = 2^-24): check against fp64."""
    x = np.random.RandomState(n).randn(n).astype(np.float32)
    a = HostTensor(x)
    o = HostTensor(np.zeros(1, np.float32))
    oracle_forward("sum", [a], o, KernelParams(DIM_ALL, 0, 0.0))
    s64 = x.astype(np.float64).sum()
    bound = max(n - 1, 1) * 2.0 ** -24 * np.abs(x).astype(np.float64).sum()
    assert abs(float(o.numpy()[0]) - s64) <= bound
    oracle_forward("mean", [a], o, KernelParams(DIM_ALL, 0, 0.0))
    assert abs(float(o.numpy()[0]) - s64 / n) <= bound / n + 2.0 ** -24 * abs(s64 / n)


def test_max_fold_rules():
    """The literal fold `acc > x ? acc : x` from -FLT_MAX: a NaN resets it, ties keep the later
    element, all -inf gives -FLT_MAX (reduce_ops.c:9, 26-30)."""
    def mx(v):
        a = HostTensor(np.array(v, np.float32))
        o = HostTensor(np.zeros(1, np.float32))
        oracle_forward("max", [a], o, KernelParams(DIM_ALL, 0, 0.0))
        return o.numpy()[0]
    nan = np.float32("nan")
    assert np.isnan(mx([1.0, 5.0, nan]))
    assert mx([1.0, nan, 0.5, -2.0]) == np.float32(0.5)
    assert mx([-np.inf, -np.inf]) == np.float32(-3.4028235e38)
    assert np.signbit(mx([0.0, -0.0])) and not np.signbit(mx([-0.0, 0.0]))


def test_exp_log_call_glibc():
    x = np.concatenate([np.random.RandomState(3).uniform(-90, 90, 2000),
                        [0.0, -0.0, 88.72, -103.97, 1e-40, np.inf, -np.inf, np.nan]]).astype(np.float32)
    a = HostTensor(x)
    o = HostTensor(np.zeros_like(x))
    oracle_forward("exp", [a], o)
    assert_bits(o.numpy(), libm_expf(x), "exp vs glibc expf")


@pytest.mark.skipif(not ref_available(), reason="oracle/_ref not built")
@pytest.mark.parametrize("N,Cn", [(1, 1), (9, 5), (37, 50), (16, 1003)])
def test_softmax_ce_matches_reference_chain(N, Cn):
    rng = np.random.RandomState(N * 131 + Cn)
    x = (rng.randn(N, Cn) * 2).astype(np.float32)
    lab = rng.randint(0, Cn, N).astype(np.int32)
    loss_r, mx_r, ls_r, _, dx_r = ref_ce_chain(x, lab)
    X = HostTensor(x, requires_grad=True)
    L = HostTensor(lab)
    S = HostTensor(np.zeros((N, 2), np.float32))
    O = HostTensor(np.zeros(N, np.float32), requires_grad=True)
    oracle_forward("softmax_cross_entropy", [X, L, S], O)
    assert_bits(O.numpy(), loss_r, "row loss")
    assert_bits(S.numpy()[:, 0], mx_r, "row max")
    assert_bits(S.numpy()[:, 1], ls_r, "row log-sum")
    O.grad.buf[:] = np.float32(1.0) / np.float32(N)   # the MEAN node's backward
    oracle_backward("softmax_cross_entropy", [X, L, S], O)
    d = X.grad.numpy()
    # the chain's max path adds only rounding residue; elementwise error ~ a few ulp of 1/N
    assert np.abs(d - dx_r).max() <= 1e-5 * max(np.abs(dx_r).max(), 1.0 / N)


def test_softmax_ce_invariants():
    rng = np.random.RandomState(11)
    N, Cn = 64, 300
    x = (rng.randn(N, Cn) * 2).astype(np.float32)
    lab = rng.randint(0, Cn, N).astype(np.int32)
    X = HostTensor(x, requires_grad=True)
    L = HostTensor(lab)
    S = HostTensor(np.zeros((N, 2), np.float32))
    O = HostTensor(np.zeros(N, np.float32), requires_grad=True)
    oracle_forward("softmax_cross_entropy", [X, L, S], O)
    st = S.numpy()
    p = np.exp((x.astype(np.float64) - st[:, :1]) - st[:, 1:])
    np.testing.assert_allclose(p.sum(1), 1.0, rtol=1e-5)
    lse = np.log(np.exp(x.astype(np.float64)).sum(1))
    np.testing.assert_allclose(O.numpy(), lse - x[np.arange(N), lab], rtol=1e-5, atol=1e-5)
    O.grad.buf[:] = 1.0
    oracle_backward("softmax_cross_entropy", [X, L, S], O)
    np.testing.assert_allclose(X.grad.numpy().sum(1), 0.0, atol=1e-5)


def _chain2_by_ops(fwd, a, b, c):
    """Config 2's chain as the reference runs it unfused: MUL, ADD, LEAKY_RELU(0), NEG, EXP, each a
    separate op over contiguous [n] tensors (five nodes of the reference DAG)."""
    n = a.size
    A, B, Cc = HostTensor(a), HostTensor(b), HostTensor(c)
    T = [HostTensor(np.zeros(n, np.float32)) for _ in range(5)]
    fwd("mul", [A, B], T[0])
    fwd("add", [T[0], Cc], T[1])
    fwd("leaky_relu", [T[1]], T[2], KernelParams(0, 0, 0.0))
    fwd("neg", [T[2]], T[3])
    fwd("exp", [T[3]], T[4])
    return T[4].numpy()


def _chain2_inputs(n, seed):
    rng = np.random.RandomState(seed)
    a, b, c = (rng.randn(n).astype(np.float32) for _ in range(3))
    # specials: signed zeros into relu (-> -0.0, then neg -> +0/-0 by the SIMD rule), infinities,
    # NaN and values whose exp under/overflows
    sp = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 100.0, -100.0, 1e-30], np.float32)
    k = min(n, sp.size)
    a[:k] = sp[:k]
    c[:k] = -sp[:k]
    return a, b, c


@pytest.mark.parametrize("n", [1, 7, 8, 13, 4096, 100_003])
def test_chain2_oracle_equals_its_pinned_ops(n):
    """oracle_fused_chain2 is bit-identical to the oracle's own MUL/ADD/LEAKY_RELU/NEG/EXP kernels,
    each of which is pinned to the golden vectors; n covers the NEG rule's SIMD block and tail."""
    a, b, c = _chain2_inputs(n, n)
    assert_bits(fused_chain2(a, b, c), _chain2_by_ops(oracle_forward, a, b, c), "chain vs ops")


@pytest.mark.skipif(not ref_available(), reason="oracle/_ref not built (needs /root/reference)")
@pytest.mark.parametrize("n", [1, 13, 100_003])
def test_chain2_oracle_equals_reference_chain(n):
    a, b, c = _chain2_inputs(n, 7 * n + 1)
    assert_bits(fused_chain2(a, b, c), _chain2_by_ops(ref_forward, a, b, c), "chain vs reference")


def test_planted_mistake_is_caught():
    """The comparison machinery must flag a wrong oracle: plant `add` where `sub` is expected."""
    c = next(c for c in CASES if c.id.startswith("sub_fwd_(2, 3)"))
    good = run_case(HostBackend("oracle"), c)

    class Planted(HostBackend):
        def fwd(self, op, ins, out, p):
            super().fwd("add" if op == "sub" else op, ins, out, p)

    bad = run_case(Planted("oracle"), c)
    with pytest.raises(AssertionError):
        assert_bits(bad["out"], good["out"], "planted")


EXPAND_CASES = [((3,), (2, 3)), ((1, 3), (4, 3)), ((2, 1, 4), (2, 5, 4)), ((1,), (7,)),
                ((2, 3), (2, 3)), ((1, 1), (3, 2)), ((4, 1), (2, 4, 6)), ("T", (5, 3, 2))]


@pytest.mark.parametrize("a_shape, out_shape", EXPAND_CASES, ids=[str(c) for c in EXPAND_CASES])
def test_expand_metadata(a_shape, out_shape):
    """oracle_expand_forward (shape_ops.c:54-57 with cpu_utils.c:59-76) against the compiled
    reference's expand_cpu_forward and broadcast_cpu_forward, the HIP library's expand and
    broadcast forwards (host-side metadata, no device needed) and numpy's broadcast_to strides:
    the output aliases the input's data and gradient, new leading axes and expanded size-1 axes
    get stride 0, every other axis keeps the input's stride. "T" is a transposed [3, 1] input."""
    import ctypes as C
    from plast_amd import abi
    if a_shape == "T":
        base = HostTensor(np.arange(3, dtype=np.float32).reshape(1, 3), requires_grad=True)
        a = HostTensor(base=base, shape=(3, 1), strides=(1, 3))
        a.grad = base.grad
        a.t.grad = C.pointer(base.grad.t)
        a.t.requires_grad = True
        a_strides = (1, 3)
    else:
        a = HostTensor(np.zeros(a_shape, np.float32), requires_grad=True)
        a_strides = abi.strides_of(a.t)
    view = np.lib.stride_tricks.as_strided(np.zeros(1, np.float32), shape=a.t.shape[:a.t.ndim],
                                           strides=[4 * s for s in a_strides])
    want = tuple(s // 4 for s in np.broadcast_to(view, out_shape).strides)
    runs = [("oracle", lambda o: oracle_forward("expand", [a], o))]
    if ref_available():
        runs += [("ref expand", lambda o: ref_forward("expand", [a], o)),
                 ("ref broadcast", lambda o: ref_forward("broadcast", [a], o))]
    from plast_amd.runtime import LIB_PATH
    hip = C.CDLL(str(LIB_PATH))   # loaded without initialising a device: these calls need none
    for f in (hip.expand_hip_forward, hip.broadcast_hip_forward):
        f.argtypes, f.restype = [abi.TensorPP, abi.TensorP, KernelParams], None
    ins = (abi.TensorP * 1)(C.pointer(a.t))
    runs += [("hip expand", lambda o: hip.expand_hip_forward(ins, C.byref(o.t), KernelParams(0, 0, 0.0))),
             ("hip broadcast", lambda o: hip.broadcast_hip_forward(ins, C.byref(o.t),
                                                                   KernelParams(0, 0, 0.0)))]
    for name, run in runs:
        o = HostTensor(np.zeros(out_shape, np.float32))
        run(o)
        assert o.t.data == a.t.data, f"{name}: data not aliased"
        assert C.cast(o.t.grad, C.c_void_p).value == C.cast(a.t.grad, C.c_void_p).value, \
            f"{name}: grad not shared"
        assert abi.strides_of(o.t) == want, f"{name}: strides {abi.strides_of(o.t)} != {want}"


@pytest.mark.skipif(not native_available(),
                    reason="oracle/_ref/libplast_ref_native.so not built (needs /root/reference)")
def test_separate_rounding_against_the_natively_built_reference():
    """The reference's Makefile:7 flags (-O3 -march=native) leave GCC's FMA contraction on, so that
    build computes a backward's `da += g * x` as fma(g, x, da): one rounding where the C source reads
    two. The oracle (and so the HIP path, bit-equal to it) keeps the source's two roundings. Here:
    every forward output is bit-identical to the native build; every exactly-ordered backward is
    within 2^-21 * (|increment| + |result|) of it, where increment is what the same backward adds to
    a zero gradient (one rounding of the product, one of the sum, doubled for two terms into one
    buffer). From a zero gradient fma(g, x, 0) rounds as g * x, so only a gradient formula with a
    product inside (tan's 1 + t*t) can differ there. The counts of differing elements are
    printed."""
    from cases import Case
    import dataclasses
    fwd_same = 0
    acc_diff, acc_total, worst = {}, {}, 0.0
    for c in REF_CASES:
        got = run_case(HostBackend("oracle"), c)
        nat = run_case(HostBackend("native"), c)
        if c.kind == "fwd":
            for k in got:
                assert_bits(got[k], nat[k], f"{c.id}:{k} forward vs native")
            fwd_same += 1
            continue
        if not c.exact:   # the reference's omp atomics: order unspecified
            continue
        start = "zero" if c.grad_init is None and not c.same_input else "acc"
        zero = run_case(HostBackend("oracle"), dataclasses.replace(c, grad_init=None))
        for k in got:
            if not k.startswith("grad"):
                assert_bits(got[k], nat[k], f"{c.id}:{k}")
                continue
            g64, n64 = got[k].astype(np.float64), nat[k].astype(np.float64)
            bound = 2.0 ** -21 * (np.abs(zero[k].astype(np.float64)) + np.abs(g64)) + 2.0 ** -149
            d = np.abs(g64 - n64)
            both_nan = np.isnan(g64) & np.isnan(n64)
            ok = both_nan | (d <= bound)
            assert ok.all(), f"{c.id}:{k}: {int((~ok).sum())} beyond the contraction bound"
            worst = max(worst, float(np.max(np.where(both_nan, 0.0, d / bound))))
            diff = int(((got[k].view(np.uint32) != nat[k].view(np.uint32)) & ~both_nan).sum())
            key = (start, c.op)
            acc_diff[key] = acc_diff.get(key, 0) + diff
            acc_total[key] = acc_total.get(key, 0) + got[k].size
    print(f"forward cases bit-identical to the native build: {fwd_same}")
    for start in ("zero", "acc"):
        print(f"backward from a {start} gradient, elements differing from the native build: " +
              ", ".join(f"{op} {acc_diff[(st, op)]}/{acc_total[(st, op)]}"
                        for st, op in sorted(acc_diff) if st == start))
    print(f"largest difference as a fraction of the bound: {worst:.3f}")
