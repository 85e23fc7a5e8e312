"""CPU checks of the optimizer row: struct layouts against the reference headers, the oracle's
SGD / Adam / AdamW / zero_grad against the reference's own src/optimizers/cpu sources (compiled
into oracle/_ref) bit for bit over several steps, and against a float64 restatement."""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np
import pytest

from cases import assert_bits
from hostlib import HostTensor, native, native_available, oracle, ref, ref_available
from optim_cases import (HYPER, MANY, OVER, SIZES, SPECIAL, SPECIAL_SEED, f64_reference, grads, host_array, initial, make_opt,
                         read_moments)
from plast_amd import abi

ROOT = Path(__file__).resolve().parent.parent
REF_INC = Path("/root/reference/include")

OPT_PROBE = r"""
#include <stdio.h>
#include <stddef.h>
#define F(T, m) printf(#T "." #m " %zu\n", offsetof(T, m))
#define S(T) printf(#T " %zu\n", sizeof(T))
int main(void) {
  S(SGD); F(SGD, lr);
  S(Adam); F(Adam, lr); F(Adam, beta1); F(Adam, beta2); F(Adam, epsilon); F(Adam, t); F(Adam, m);
  F(Adam, v); F(Adam, data_arena); F(Adam, optimizer_arena);
  S(AdamW); F(AdamW, lr); F(AdamW, beta1); F(AdamW, beta2); F(AdamW, epsilon);
  F(AdamW, weight_decay); F(AdamW, t); F(AdamW, m); F(AdamW, v); F(AdamW, data_arena);
  F(AdamW, optimizer_arena);
  return 0;
}
"""


def _probe(tmp_path, includes, flags):
    src = tmp_path / "probe.c"
    src.write_text(includes + OPT_PROBE)
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-o", str(exe), str(src), *flags], check=True)
    return subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout


@pytest.mark.skipif(not REF_INC.exists(), reason="reference headers absent")
def test_optimizer_layouts_match_reference(tmp_path):
    ours = _probe(tmp_path, '#include "plast_abi.h"\n', [f"-I{ROOT / 'include'}"])
    theirs = _probe(tmp_path, '#include "sgd.h"\n#include "adam.h"\n#include "adamw.h"\n',
                    [f"-I{REF_INC}", f"-I{REF_INC / 'optimizers'}"])
    assert ours == theirs


def test_ctypes_optimizer_mirror(tmp_path):
    out = _probe(tmp_path, '#include "plast_abi.h"\n', [f"-I{ROOT / 'include'}"])
    vals = dict(line.rsplit(" ", 1) for line in out.splitlines())
    assert int(vals["Adam"]) == C.sizeof(abi.Adam)
    assert int(vals["AdamW"]) == C.sizeof(abi.AdamW)
    assert int(vals["AdamW.optimizer_arena"]) == abi.AdamW.optimizer_arena.offset
    assert int(vals["Adam.m"]) == abi.Adam.m.offset


# ----------------------------------------------------------------------------- host steppers
def _host_params(p0, with_grad):
    return [HostTensor(x, requires_grad=w) for x, w in zip(p0, with_grad)]


def _step_fn(lib, kind, prefix):
    f = getattr(lib, f"{prefix}{kind}_step{'' if prefix == 'oracle_' else '_cpu'}")
    typ = {"sgd": abi.SGD, "adam": abi.Adam, "adamw": abi.AdamW}[kind]
    f.argtypes = [C.POINTER(typ), abi.TensorPP, C.c_int]
    f.restype = None
    return f


_ARENAS = []


def _ref_opt(kind, which="ref"):
    """The reference's own optimizer struct with CPU arenas (its first step allocates m and v in
    them through init(..., zeros): adam.c:29-46)."""
    L = ref() if which == "ref" else native()
    L.arena_create.restype = abi.Arena
    L.arena_create.argtypes = [C.c_uint64, C.c_int]
    opt = make_opt(kind)
    if kind != "sgd":
        a1, a2 = L.arena_create(1 << 20, abi.CPU), L.arena_create(1 << 22, abi.CPU)
        _ARENAS.append((a1, a2))
        opt.optimizer_arena = C.pointer(_ARENAS[-1][0])
        opt.data_arena = C.pointer(_ARENAS[-1][1])
    return opt


def run_host(which, kind, sizes, seed, steps, with_grad=None):
    """Run `steps` updates through the oracle ("oracle"), the compiled reference ("ref") or the
    reference built with its own flags ("native"); returns the parameters and, for Adam/AdamW, the
    moments after the last step."""
    with_grad = with_grad or [True] * len(sizes)
    p0 = initial(sizes, seed)
    params = _host_params(p0, with_grad)
    ptrs, keep = abi.tensor_array(*[t.t for t in params])
    opt = make_opt(kind) if which == "oracle" else _ref_opt(kind, which)
    lib = {"oracle": oracle, "ref": ref, "native": native}[which]()
    f = _step_fn(lib, kind, "oracle_" if which == "oracle" else "")
    for s in range(steps):
        for t, g, w in zip(params, grads(sizes, seed, s), with_grad):
            if w:
                t.grad.buf[:] = g.ravel()
        f(C.byref(opt), ptrs, len(params))
    ps = [t.numpy() for t in params]
    mv = read_moments(opt, len(params), host_array) if kind != "sgd" else None
    return ps, mv, opt


@pytest.mark.skipif(not ref_available(), reason="oracle/_ref not built (needs /root/reference)")
@pytest.mark.parametrize("kind", ["sgd", "adam", "adamw"])
@pytest.mark.parametrize("sizes,seed", [(SIZES, 11), (MANY, 11), (OVER, 11), (SPECIAL, SPECIAL_SEED)],
                         ids=["shapes", "many", "over", "special_grads"])
def test_oracle_optimizer_matches_compiled_reference(kind, sizes, seed):
    with_grad = [i % 5 != 3 for i in range(len(sizes))]   # some parameters carry no grad
    po, mvo, _ = run_host("oracle", kind, sizes, seed, 3, with_grad)
    pr, mvr, _ = run_host("ref", kind, sizes, seed, 3, with_grad)
    for i, (a, b) in enumerate(zip(po, pr)):
        assert_bits(a, b, f"{kind} param {i}")
    if mvo is not None:
        for i, ((mo, vo), (mr, vr)) in enumerate(zip(mvo, mvr)):
            assert_bits(mo, mr, f"{kind} m {i}")
            assert_bits(vo, vr, f"{kind} v {i}")


@pytest.mark.parametrize("kind", ["sgd", "adam", "adamw"])
def test_oracle_optimizer_matches_float64_update(kind):
    steps = 4
    po, mvo, _ = run_host("oracle", kind, SIZES, 5, steps)
    p0 = initial(SIZES, 5)
    pf, mf, vf = f64_reference(kind, p0, [grads(SIZES, 5, s) for s in range(steps)])
    for i in range(len(SIZES)):
        # a few fp32 roundings per step on O(1) values; moments are O(grad)
        np.testing.assert_allclose(po[i], pf[i], rtol=1e-5, atol=1e-6, err_msg=f"{kind} p{i}")
        if mvo is not None:
            np.testing.assert_allclose(mvo[i][0], mf[i], rtol=1e-5, atol=1e-7)
            np.testing.assert_allclose(mvo[i][1], vf[i], rtol=1e-5, atol=1e-9)


def test_oracle_optimizer_catches_a_wrong_bias_correction():
    """A planted mistake (beta1 and beta2 swapped in the bias correction) must be visible to the
    float64 check above, so that check pins the step size and not only the moment recursions."""
    h = dict(HYPER["adam"])
    p0 = initial(SIZES, 5)
    gs = [grads(SIZES, 5, 0)]
    good, _, _ = f64_reference("adam", p0, gs)
    HYPER["adam"] = dict(h, beta1=h["beta2"], beta2=h["beta1"])
    try:
        bad, _, _ = f64_reference("adam", p0, gs)
    finally:
        HYPER["adam"] = h
    po, _, _ = run_host("oracle", "adam", SIZES, 5, 1)
    assert any(not np.allclose(po[i], bad[i], rtol=1e-5, atol=1e-6) for i in range(len(SIZES)))
    assert all(np.allclose(po[i], good[i], rtol=1e-5, atol=1e-6) for i in range(len(SIZES)))


@pytest.mark.skipif(not ref_available(), reason="oracle/_ref not built (needs /root/reference)")
def test_oracle_zero_grad_matches_reference():
    for which, fname in (("oracle", "oracle_zero_grad"), ("ref", "zero_grad_cpu")):
        t = HostTensor(np.ones((3, 5), np.float32), requires_grad=True)
        t.grad.buf[:] = np.arange(15, dtype=np.float32) - 7
        lib = oracle() if which == "oracle" else ref()
        f = getattr(lib, fname)
        f.argtypes, f.restype = [abi.TensorP], None
        f(C.byref(t.t))
        assert_bits(t.grad.numpy(), np.zeros((3, 5), np.float32), f"{which} zero_grad")
        assert_bits(t.numpy(), np.ones((3, 5), np.float32), f"{which} data untouched")


@pytest.mark.parametrize("kind", ["sgd", "adam", "adamw"])
@pytest.mark.parametrize("set_name", ["shapes", "many"])
def test_oracle_optimizer_matches_golden_vectors(kind, set_name):
    """The same three steps as above against the committed outputs of the compiled reference
    (tests/golden/make_golden_optim.py), so the pin holds where /root/reference is absent."""
    g = np.load(Path(__file__).resolve().parent / "golden" / "optimizer_cases.npz",
                allow_pickle=False)
    sizes = SIZES if set_name == "shapes" else MANY
    with_grad = [i % 5 != 3 for i in range(len(sizes))]
    ps, mv, _ = run_host("oracle", kind, sizes, 11, 3, with_grad)
    for i, p in enumerate(ps):
        assert_bits(p, g[f"{set_name}@{kind}@p{i}"], f"{kind} p{i}")
        if mv is not None:
            assert_bits(mv[i][0], g[f"{set_name}@{kind}@m{i}"], f"{kind} m{i}")
            assert_bits(mv[i][1], g[f"{set_name}@{kind}@v{i}"], f"{kind} v{i}")


@pytest.mark.skipif(not native_available(),
                    reason="oracle/_ref/libplast_ref_native.so not built (needs /root/reference)")
@pytest.mark.parametrize("kind", ["sgd", "adam", "adamw"])
def test_oracle_optimizer_against_the_natively_built_reference(kind):
    """Under the reference's own flags GCC contracts the moment updates (b1 * m + (1 - b1) * g, ...)
    into FMAs, one rounding where the source reads two; the oracle and the HIP path keep the
    source's roundings. After three steps every value is within 2^-18 (a few ulps per step) of the
    native build's, measured against the value's magnitude plus the magnitudes it was summed from
    (values can cancel towards 0): for a parameter its total update, for m the sum of |g| over the
    steps, for v the sum of g^2. NaN matches NaN; the differing counts are printed. SGD
    (p -= lr * g) contracts too."""
    sizes, seed, steps = SIZES, 11, 3
    p0 = initial(sizes, seed)
    gs = [grads(sizes, seed, st) for st in range(steps)]
    po, mvo, _ = run_host("oracle", kind, sizes, seed, steps)
    pn, mvn, _ = run_host("native", kind, sizes, seed, steps)
    pairs = [("param", a, b, np.abs(a.astype(np.float64) - x0)) for a, b, x0 in zip(po, pn, p0)]
    if mvo is not None:
        for i, ((mo, vo), (mn, vn)) in enumerate(zip(mvo, mvn)):
            g64 = [g[i].astype(np.float64).reshape(mo.shape) for g in gs]
            pairs += [("m", mo, mn, sum(np.abs(g) for g in g64)),
                      ("v", vo, vn, sum(g * g for g in g64))]
    diff, total = {}, {}
    for name, a, b, moved in pairs:
        a64, b64 = a.astype(np.float64), b.astype(np.float64)
        nan = np.isnan(a64) & np.isnan(b64)
        tol = 2.0 ** -18 * (np.maximum(np.abs(a64), np.abs(b64)) + moved) + 2.0 ** -149
        ok = nan | (np.abs(a64 - b64) <= tol)
        assert ok.all(), f"{kind} {name}: {int((~ok).sum())} beyond the bound"
        diff[name] = diff.get(name, 0) + int(((a.view(np.uint32) != b.view(np.uint32)) & ~nan).sum())
        total[name] = total.get(name, 0) + a.size
    print(f"{kind}: elements differing from the native build after 3 steps: " +
          ", ".join(f"{k} {diff[k]}/{total[k]}" for k in diff))
