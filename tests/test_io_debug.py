"""State and Model files (.npz, no pickling) and the host getters (body records, contact records with the world
manifold), CPU only. The world manifold is pinned by a float64 restatement of b2WorldManifold::Initialize and by
closed forms (a resting box's points and separations, a circle pair's normal)."""
import numpy as np
import pytest

from util import b2
import scene_defs

F32 = np.float32
wd = b2.world
io = b2.io
dbg = b2.debug


def _scene_state(name, steps, oracle):
    s, m, st = scene_defs.build_test_scene(name, iterations=(8, 3))
    st = wd.batch(st, 2)
    for _ in range(steps):
        oracle.step_(m, st, s, 1.0 / 60.0)
    return s, m, st


def test_state_file_round_trip(tmp_path, oracle):
    s, m, st = _scene_state("pile", 30, oracle)
    io.save_state(tmp_path / "st.npz", st)
    back = io.load_state(tmp_path / "st.npz")
    for a, b in zip(wd.leaves(st), wd.leaves(back)):
        a, b = np.asarray(a), np.asarray(b)
        assert a.dtype == b.dtype and a.shape == b.shape and a.tobytes() == b.tobytes()
    # the restored State steps exactly like the original
    oracle.step_(m, st, s, 1.0 / 60.0)
    oracle.step_(m, back, s, 1.0 / 60.0)
    assert all(np.asarray(a).tobytes() == np.asarray(b).tobytes() for a, b in zip(wd.leaves(st), wd.leaves(back)))


def test_state_file_is_checked(tmp_path, oracle):
    s, m, st = _scene_state("box_stack", 2, oracle)
    io.save_state(tmp_path / "st.npz", st)
    with np.load(tmp_path / "st.npz") as f:
        arrays = {k: f[k] for k in f.files}
    bad = dict(arrays)
    del bad["contacts.key"]
    np.savez(tmp_path / "missing.npz", **bad)
    with pytest.raises(ValueError, match="missing"):
        io.load_state(tmp_path / "missing.npz")
    bad = dict(arrays)
    bad["bodies.c"] = bad["bodies.c"].astype(np.float64)
    np.savez(tmp_path / "dtype.npz", **bad)
    with pytest.raises(TypeError):
        io.load_state(tmp_path / "dtype.npz")
    bad = dict(arrays)
    bad["bodies.v"] = bad["bodies.v"][:, :-1]
    np.savez(tmp_path / "shape.npz", **bad)
    with pytest.raises(ValueError):
        io.load_state(tmp_path / "shape.npz")


def test_model_file_round_trip(tmp_path):
    s, m, st, cfg = b2.scenes.make_config(1, edges="native")
    io.save_model(tmp_path / "m.npz", m)
    back = io.load_model(tmp_path / "m.npz")
    for f in wd.Model._fields:
        a, b = getattr(m, f), getattr(back, f)
        assert (a is None) == (b is None), f
        if a is not None:
            assert np.asarray(a).tobytes() == np.asarray(b).tobytes() and np.asarray(a).dtype == np.asarray(b).dtype, f


def test_body_record():
    s, m, st = scene_defs.build_test_scene("free_fall")
    st = wd.batch(st, 1)
    r = dbg.body_record(st, 0, 1)
    bd = st.bodies
    assert r.dtype == F32 and r.shape == (24,)
    assert tuple(r[:3]) == (bd.xf_p[0, 1, 0], bd.xf_p[0, 1, 1], bd.a[0, 1])
    assert tuple(r[5:8]) == (bd.v[0, 1, 0], bd.v[0, 1, 1], bd.w[0, 1])
    assert r[10] == wd.DYNAMIC and r[12] == bd.mass[0, 1] and tuple(r[16:18]) == tuple(bd.local_center[0, 1])
    assert int(r[22]) & dbg.AWAKE_FLAG and int(r[22]) & dbg.ACTIVE_FLAG


def _world_manifold_f64(c, xa, qa, xb, qb, ra, rb):
    """b2WorldManifold::Initialize in float64 from the definition."""
    def mul(q, p, v):
        return np.array([q[0] * v[0] - q[1] * v[1] + p[0], q[1] * v[0] + q[0] * v[1] + p[1]])

    def rot(q, v):
        return np.array([q[0] * v[0] - q[1] * v[1], q[1] * v[0] + q[0] * v[1]])
    n, mt = c["pointCount"], c["manifoldType"]
    if mt == 0:
        pa, pb = mul(qa, xa, c["localPoint"]), mul(qb, xb, c["pointLocal"][0])
        nrm = (pb - pa) / np.linalg.norm(pb - pa)
        ca, cb = pa + ra * nrm, pb - rb * nrm
        return nrm, [0.5 * (ca + cb)], [np.dot(cb - ca, nrm)]
    if mt == 1:
        nrm, plane = rot(qa, c["localNormal"]), mul(qa, xa, c["localPoint"])
        pts, seps = [], []
        for i in range(n):
            clip = mul(qb, xb, c["pointLocal"][i])
            ca, cb = clip + (ra - np.dot(clip - plane, nrm)) * nrm, clip - rb * nrm
            pts.append(0.5 * (ca + cb)); seps.append(np.dot(cb - ca, nrm))
        return nrm, pts, seps
    nrm, plane = rot(qb, c["localNormal"]), mul(qb, xb, c["localPoint"])
    pts, seps = [], []
    for i in range(n):
        clip = mul(qa, xa, c["pointLocal"][i])
        cb, ca = clip + (rb - np.dot(clip - plane, nrm)) * nrm, clip - ra * nrm
        pts.append(0.5 * (ca + cb)); seps.append(np.dot(ca - cb, nrm))
    return -nrm, pts, seps


@pytest.mark.parametrize("name", ["pile", "polygons", "circles", "edges"])
def test_contact_records_world_manifold(oracle, name):
    """Live contacts newest first; the float32 world manifold agrees with a float64 one to 1e-5; the normal is a
    unit vector from A to B (the separations it measures shrink as B moves along it)."""
    s, m, st = _scene_state(name, 40, oracle)
    bd = st.bodies
    seen = 0
    for w in range(2):
        recs = dbg.contacts(m, st, w)
        keys = [r["key"] for r in recs]
        assert keys == sorted(keys, reverse=True) and len(recs) == int((np.asarray(st.contacts.pair[w]) >= 0).sum())
        for r in recs:
            if r["pointCount"] == 0:
                assert "worldNormal" not in r
                continue
            seen += 1
            ba, bb = r["bodyA"], r["bodyB"]
            ra, rb = float(m.radius[r["fixtureA"]]), float(m.radius[r["fixtureB"]])
            n64, p64, s64 = _world_manifold_f64(r, bd.xf_p[w, ba].astype(float), bd.xf_q[w, ba].astype(float),
                                                bd.xf_p[w, bb].astype(float), bd.xf_q[w, bb].astype(float), ra, rb)
            assert abs(np.linalg.norm(r["worldNormal"]) - 1) < 1e-5
            assert np.allclose(r["worldNormal"], n64, atol=1e-5)
            assert np.allclose(r["worldPoints"], np.array(p64), atol=1e-5)
            assert np.allclose(r["separations"], np.array(s64), atol=1e-5)
    assert seen > 3


def test_resting_box_world_manifold(oracle):
    """A box resting on the ground: normal (0, 1) from the ground (A) to the box (B), two points at the box's bottom
    corners, separations at the solver's rest depth (about -linear_slop)."""
    d = wd.WorldDef(b2.Settings.stock(gravity=(0.0, -10.0)))
    g = d.add_body(wd.STATIC)
    d.add_box(g, (5.0, 0.5))
    b = d.add_body(wd.DYNAMIC, (0.0, 1.0), mass=1.0, inertia=F32(1) / F32(6))
    d.add_box(b, (0.5, 0.5))
    model, state = d.build(4)
    st = wd.batch(state, 1)
    for _ in range(120):
        oracle.step_(model, st, d.settings, 1.0 / 60.0)
    (r,) = dbg.contacts(model, st, 0)
    assert (r["bodyA"], r["bodyB"], r["pointCount"]) == (g, b, 2)
    assert np.allclose(r["worldNormal"], (0, 1), atol=1e-6)
    assert np.allclose(sorted(r["worldPoints"][:, 0]), (-0.5, 0.5), atol=2e-3)
    assert np.allclose(r["separations"], -0.005, atol=1.5e-3)


# ---------------------------------------------------------------------------------------------------------------
# the per-world status word (GoiDebug.status): the step's failure counters, each forced from the host

def _status_run(oracle, st, m, s, dt, steps, acts=None):
    """OR of the oracle's status words over `steps` steps, per world."""
    n = st.bodies.type.shape[0]
    seen = np.zeros(n, np.int32)
    for k in range(steps):
        if acts is not None:
            b2.scenes.apply_actions(st.joints.motor_speed, st.joints.max_motor, acts[k])
        d = {key: np.full(shape, -7, np.int32) for key, shape in b2.debug_shapes(n, wd.dims(st)).items()}
        before = np.asarray(st.overflow).copy()
        oracle.step_(m, st, s, dt, debug=d)
        assert np.array_equal((d["status"] & b2._abi.STATUS_OVERFLOW) != 0, np.asarray(st.overflow) != before)
        seen |= d["status"]
    return seen


def test_status_word(oracle):
    """Each bit from the condition that sets it: a small contact table (overflow), non-finite bodies, max_events 1
    (SolveTOI capped with an event pending), dt 0 with continuous physics (SolveTOI skipped); none on a healthy run."""
    from dataclasses import replace
    from test_host_sanitized import nonfinite_case
    A = b2._abi
    rng = np.random.default_rng(3)
    s, m, st, cfg = b2.scenes.make_config(4, 64)
    acts = [b2.scenes.actions(rng, 64) for _ in range(10)]
    healthy = _status_run(oracle, oracle.copy(st), m, s, cfg.dt, 10, acts)
    assert (healthy == 0).all()
    s6, m6, st6, _ = b2.scenes.make_config(4, 64, capacity=6)
    assert (_status_run(oracle, st6, m6, s6, cfg.dt, 10, acts) & A.STATUS_OVERFLOW).any()
    mn, stn, sn, dtn, actsn = nonfinite_case()
    bad = _status_run(oracle, stn, mn, sn, dtn, 3, list(actsn))
    # world 9's 1e30 m/s stays finite: h v squared overflows, so the max-translation clamp scales v by 2 / inf = 0
    assert np.array_equal(np.nonzero(bad & A.STATUS_NONFINITE)[0], [3, 5, 7, 11])
    assert np.isfinite(stn.bodies.c[9]).all() and np.isfinite(stn.bodies.v[9]).all()
    capped = _status_run(oracle, oracle.copy(st), m, replace(s, max_events=1), cfg.dt, 10, acts)
    assert (capped & A.STATUS_TOI_CAPPED).any() and not (healthy & A.STATUS_TOI_CAPPED).any()
    skipped = _status_run(oracle, oracle.copy(st), m, s, np.float32(0.0), 1, acts)
    assert (skipped == A.STATUS_TOI_SKIPPED).all()
