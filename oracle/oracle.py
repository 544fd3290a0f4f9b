"""ctypes wrapper of the CPU restatement (liboracle_b2.so). TEST INFRASTRUCTURE ONLY: tests/, smoke() and bench.py's
cpu_baseline leg use it, to check the device step and to time the CPU baseline; the product path never imports
it.

States are batched numpy States (leading world axis, contiguous), in either fixture layout; the oracle steps them in
place. `step` copies first and returns the stepped copy.
"""
import ctypes
import importlib
import os
import subprocess
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
LIB = HERE / "liboracle_b2.so"
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))
box2d = importlib.import_module("getting-over-it-rl_amd.box2d")
_abi = importlib.import_module("getting-over-it-rl_amd.box2d._abi")
wd = box2d.world

_L = None


def build():
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib():
    """The oracle library; GOI_ORACLE_LIB names another build of the restatement (a copy with a planted mistake, when
    checking that the pins catch it)."""
    global _L
    if _L is None:
        other = os.environ.get("GOI_ORACLE_LIB")
        if other:
            _L = load(Path(other))
            return _L
        if not LIB.exists():
            build()
        _L = load(LIB)
    return _L


def load(path):
    """A ctypes handle on an oracle library at `path` with the argument types set (the tests also load variants of
    the restatement built with a planted mistake, to show that the pins catch it)."""
    L = ctypes.CDLL(str(path))
    P = ctypes.c_void_p
    L.oracle_step.argtypes = [ctypes.POINTER(_abi.GoiModelDesc), P] + [ctypes.c_int32] * 5 + [
        ctypes.POINTER(_abi.GoiSettings), ctypes.c_float, ctypes.c_int32, ctypes.POINTER(_abi.GoiDebug)]
    L.oracle_collide.argtypes = [ctypes.POINTER(_abi.GoiModelDesc), P] + [ctypes.c_int32] * 5 + [
        ctypes.POINTER(_abi.GoiSettings), ctypes.c_int32]
    L.oracle_evaluate.argtypes = [ctypes.POINTER(_abi.GoiModelDesc), ctypes.c_int, ctypes.c_int, P, P,
                                  ctypes.POINTER(_abi.GoiSettings), P, P, P]
    L.oracle_distance.argtypes = [ctypes.POINTER(_abi.GoiModelDesc), ctypes.c_int, ctypes.c_int, P, P]
    L.oracle_distance.restype = ctypes.c_float
    L.oracle_toi.argtypes = [ctypes.POINTER(_abi.GoiModelDesc), ctypes.c_int, ctypes.c_int, P, P,
                             ctypes.c_float, P]
    L.oracle_sincos.argtypes = [P, P, P, ctypes.c_int32]
    return L


def model_desc(model):
    """GoiModelDesc over a Model in either layout (the oracle also takes the full layout)."""
    keep = []

    def arr(a, dt):
        if a is None:
            return None
        x = np.ascontiguousarray(np.asarray(a), dtype=dt)
        keep.append(x)
        return x.ctypes.data_as(ctypes.c_void_p)
    I, F, U = np.int32, np.float32, np.uint8
    d = _abi.GoiModelDesc()
    d.F, d.J, d.P = model.fixture_body.shape[0], model.joint_type.shape[0], model.pair_a.shape[0]
    d.B = 0 if model.body_type is None else model.body_type.shape[0]
    for name, dt in dict(fixture_body=I, shape_type=I, radius=F, count=I, verts=F, normals=F, joint_type=I,
                         joint_a=I, joint_b=I, local_anchor_a=F, local_anchor_b=F, local_axis_a=F, local_yaxis_a=F,
                         reference_angle=F, pair_a=I, pair_b=I, fixture_slot=I, static_fat=F, static_friction=F,
                         static_restitution=F, body_type=I, centroid=F, edge_flags=I).items():
        setattr(d, name, arr(getattr(model, name), dt))
    d.toi_bodies = arr(model.toi_bodies, U)
    return d, keep


def _leaves(state):
    vals = [np.ascontiguousarray(np.asarray(x)) for x in wd.leaves(state)]
    ptrs = (ctypes.c_void_p * len(vals))(*[v.ctypes.data for v in vals])
    return vals, ptrs


def step_(model, state, settings, dt, n_threads=0, debug=None):
    """One step in place on a batched contiguous numpy State; returns it. debug: dict of int32 arrays
    body_island [B, N], contact_island [C, N], contact_order [C, N], n_islands [N] to fill (optional)."""
    vals, ptrs = _leaves(state)
    for a, b in zip(vals, wd.leaves(state)):
        if a is not b and not np.shares_memory(a, b):
            raise ValueError("oracle.step_ needs contiguous numpy leaves")
    n = vals[0].shape[0]
    B, R, J, C = wd.dims(state)
    desc, keep = model_desc(model)
    cs = settings.to_c()
    dbg = None
    if debug is not None:
        dbg = _abi.GoiDebug()
        for k, v in debug.items():
            setattr(dbg, k, v.ctypes.data_as(ctypes.c_void_p))
        dbg = ctypes.byref(dbg)
    lib().oracle_step(ctypes.byref(desc), ptrs, n, B, C, R, J, ctypes.byref(cs), ctypes.c_float(np.float32(dt)),
                      n_threads, dbg)
    return state


def copy(state):
    return wd.from_leaves([np.array(x, copy=True) for x in wd.leaves(state)])


def step(model, state, settings, dt, n_threads=0):
    return step_(model, copy(state), settings, dt, n_threads)


def collide_(model, state, settings, n_threads=0):
    vals, ptrs = _leaves(state)
    n = vals[0].shape[0]
    B, R, J, C = wd.dims(state)
    desc, keep = model_desc(model)
    cs = settings.to_c()
    lib().oracle_collide(ctypes.byref(desc), ptrs, n, B, C, R, J, ctypes.byref(cs), n_threads)
    return state


def evaluate(model, fa, fb, xfa, xfb, settings):
    """The narrowphase manifold of fixtures (fa, fb) at transforms (px, py, c, s). `settings` is a Settings or the
    linear slop of stock Settings."""
    if not isinstance(settings, box2d.Settings):
        settings = box2d.Settings(linear_slop=np.float32(settings))
    desc, keep = model_desc(model)
    cs = settings.to_c()
    xa, xb = np.asarray(xfa, np.float32), np.asarray(xfb, np.float32)
    mc, geo, ids = np.zeros(2, np.int32), np.zeros(8, np.float32), np.zeros(2, np.int32)
    lib().oracle_evaluate(ctypes.byref(desc), fa, fb, xa.ctypes.data, xb.ctypes.data, ctypes.byref(cs),
                          mc.ctypes.data, geo.ctypes.data, ids.ctypes.data)
    return dict(mtype=int(mc[0]), count=int(mc[1]), local_normal=geo[0:2], local_point=geo[2:4],
                point_local=geo[4:8].reshape(2, 2), point_id=ids)


def distance(model, fa, fb, xfa, xfb):
    desc, keep = model_desc(model)
    xa, xb = np.asarray(xfa, np.float32), np.asarray(xfb, np.float32)
    return float(lib().oracle_distance(ctypes.byref(desc), fa, fb, xa.ctypes.data, xb.ctypes.data))


def time_of_impact(model, fa, fb, sweep_a, sweep_b, linear_slop):
    """b2TimeOfImpact (state, t); sweeps are (lcx, lcy, c0x, c0y, cx, cy, a0, a)."""
    desc, keep = model_desc(model)
    sa, sb = np.asarray(sweep_a, np.float32), np.asarray(sweep_b, np.float32)
    t = np.zeros(1, np.float32)
    st = lib().oracle_toi(ctypes.byref(desc), fa, fb, sa.ctypes.data, sb.ctypes.data, np.float32(linear_slop),
                          t.ctypes.data)
    return int(st), float(t[0])


def sincos(x):
    x = np.ascontiguousarray(x, np.float32)
    s, c = np.empty_like(x), np.empty_like(x)
    lib().oracle_sincos(x.ctypes.data, s.ctypes.data, c.ctypes.data, x.size)
    return s, c
