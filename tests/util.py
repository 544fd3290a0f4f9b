"""Shared helpers for the parity tests."""
import importlib

import numpy as np

b2 = importlib.import_module("getting-over-it-rl_amd.box2d")
wd = b2.world


def leaf_mismatches(ref, got):
    """[(leaf name, worlds that differ)] comparing two batched numpy States bit for bit."""
    out = []
    for (g, name, _, _), a, b in zip(wd.LEAVES, wd.leaves(ref), wd.leaves(got)):
        a, b = np.asarray(a), np.asarray(b)
        if a.shape != b.shape:
            out.append((f"{g}.{name}", "shape"))
            continue
        if a.tobytes() != b.tobytes():
            diff = (a != b).reshape(a.shape[0], -1).any(1) if a.ndim > 1 else (a != b)
            out.append((f"{g}.{name}", np.nonzero(diff)[0][:8].tolist()))
    return out


def perturbed(state, n, seed=1, sigma=0.2):
    """n copies of a single-world State with the dynamic bodies' velocities perturbed per world."""
    st = wd.batch(state, n)
    rng = np.random.default_rng(seed)
    dyn = (np.asarray(st.bodies.type) == wd.DYNAMIC)[..., None]
    awake = np.asarray(st.bodies.awake)[..., None]
    dv = np.where(dyn & awake, rng.normal(0.0, sigma, st.bodies.v.shape), 0.0).astype(np.float32)
    dv[0] = 0.0
    st.bodies.v[...] = st.bodies.v + dv
    return st
