"""Shared parameter sets and steppers for the optimizer tests (oracle, compiled reference, HIP).

A case is a list of parameter shapes plus a seed; every step draws fresh gradients from the seed,
so all backends see identical bytes. Shapes cover the float4 body, scalar tails (numel % 4 != 0),
tiny tensors, a 40-tensor set (the golden vectors' "many") and more tensors than one launch
groups (64).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from plast_amd import abi

SIZES = [(1,), (3,), (4,), (5,), (7, 5), (1000,), (4099,), (64, 33), (2, 3, 4)]
MANY = [(17,)] * 20 + [(260,)] * 20  # 40 tensors
OVER = [(17,)] * 40 + [(260,)] * 40 + [(4099,)] * 3  # 83 tensors: two launch groups

HYPER = {
    "sgd": dict(lr=0.05),
    "adam": dict(lr=1e-2, beta1=0.9, beta2=0.999, epsilon=1e-8),
    "adamw": dict(lr=1e-2, beta1=0.9, beta2=0.999, epsilon=1e-8, weight_decay=0.01),
}


def initial(sizes, seed):
    rng = np.random.RandomState(seed)
    return [rng.randn(*s).astype(np.float32) for s in sizes]


SPECIAL_SEED = 66  # grads() for this seed also hold infinities, NaN, subnormals and extremes
SPECIAL = [(4099,), (260,), (33,)]
_POOL = np.array([np.inf, -np.inf, np.nan, 1e-40, -1e-40, 3e38, -3e38, 1e-20], np.float32)


def grads(sizes, seed, step):
    rng = np.random.RandomState(seed * 1000 + step)
    out = []
    for s in sizes:
        g = (rng.randn(*s) * 0.3).astype(np.float32)
        if g.size > 2:
            g.flat[0] = 0.0          # zero gradient: v stays at its decay, sqrt(v) path near 0
            g.flat[1] = -0.0
        if seed == SPECIAL_SEED:
            flat = g.reshape(-1)
            flat[2:2 + min(len(_POOL), flat.size - 2)] = _POOL[:max(0, min(len(_POOL), flat.size - 2))]
            pick = rng.rand(flat.size) < 0.01
            flat[pick] = _POOL[rng.randint(0, len(_POOL), int(pick.sum()))]
        out.append(g)
    return out


def make_opt(kind):
    h = HYPER[kind]
    if kind == "sgd":
        return abi.SGD(h["lr"])
    if kind == "adam":
        return abi.Adam(h["lr"], h["beta1"], h["beta2"], h["epsilon"], 0, None, None, None, None)
    return abi.AdamW(h["lr"], h["beta1"], h["beta2"], h["epsilon"], h["weight_decay"], 0, None,
                     None, None, None)


def f64_reference(kind, p0, gs_per_step):
    """The update restated in float64 (what the mathematics fixes, up to fp32 rounding). The
    hyperparameters are the fp32 values the optimizer structs hold (0.999f is not 0.999)."""
    h = {k: float(np.float32(x)) for k, x in HYPER[kind].items()}
    p = [x.astype(np.float64) for x in p0]
    m = [np.zeros_like(x) for x in p]
    v = [np.zeros_like(x) for x in p]
    for t, gs in enumerate(gs_per_step, start=1):
        for i, g in enumerate(gs):
            g = g.astype(np.float64)
            if kind == "sgd":
                p[i] = p[i] - h["lr"] * g
                continue
            lr_t = h["lr"] * np.sqrt(1 - h["beta2"] ** t) / (1 - h["beta1"] ** t)
            if kind == "adamw":
                p[i] = p[i] - h["lr"] * h["weight_decay"] * p[i]
            m[i] = h["beta1"] * m[i] + (1 - h["beta1"]) * g
            v[i] = h["beta2"] * v[i] + (1 - h["beta2"]) * g * g
            p[i] = p[i] - lr_t * m[i] / (np.sqrt(v[i]) + h["epsilon"])
    return p, m, v


def read_moments(opt, n, reader):
    """[(m_i, v_i)] through `reader(Tensor) -> ndarray` (host or device memory)."""
    out = []
    for i in range(n):
        mp, vp = opt.m[i], opt.v[i]
        out.append((reader(mp.contents) if mp else None, reader(vp.contents) if vp else None))
    return out


def host_array(t: abi.Tensor) -> np.ndarray:
    n = int(np.prod(abi.shape_of(t))) if t.ndim else 1
    buf = (C.c_float * n).from_address(t.data)
    return np.ctypeslib.as_array(buf).copy().reshape(abi.shape_of(t))
