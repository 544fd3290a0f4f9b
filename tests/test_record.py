"""The recording loader (box2d/record.py) on synthetic records: no recordings of the game exist, so parity of the
decoder is unpinned. A test-side encoder writes step records and geometry blobs in the plugin's layout
(plugin/GameRecord.cs:20-28, plugin/NativeRecord.cs:92-182, offsets of plugin/NativeBox2D.cs:32-60 and the JSON
dump's field list at NativeBox2D.cs:400-468) from States the oracle stepped; the decoder must give those States back
(every field a record carries) and a decoded State must step like the original."""
import importlib
import struct

import numpy as np
import pytest

from util import b2, wd

R = importlib.import_module("getting-over-it-rl_amd.box2d.record")
scenes = b2.scenes
F32 = np.float32

ADDR0 = 0x7F1200000000  # synthetic native addresses: body k at ADDR0 + 0x1000 k


def _put(buf, off, fmt, *vals):
    struct.pack_into("<" + fmt, buf, off, *vals)


def _fv(x):
    """The float32 values of x (an array, or a list of arrays and scalars), flattened in order."""
    parts = x if isinstance(x, list) else [x]
    return [float(v) for p in parts for v in np.ravel(np.asarray(p, F32))]


def encode_geometry(model, state, ground_rb=-1):
    """GOG1 of a full-layout single-world Model/State: bodies newest first (the ground, created first, last), each
    body's fixtures newest first; fixture f is (collider f, piece 0); dynamic body k has Rigidbody2D index k."""
    out = bytearray(struct.pack("<Ii", R.GEOMETRY_MAGIC, 3))
    B = state.bodies.type.shape[0]
    out += struct.pack("<i", B)
    for b in reversed(range(B)):
        t = int(state.bodies.type[b])
        fx = [f for f in range(model.fixture_body.shape[0]) if model.fixture_body[f] == b]
        out += struct.pack("<iii", b if t != wd.STATIC else ground_rb, t, len(fx))
        for f in reversed(fx):
            fixture = bytearray(R.FIXTURE_BYTES)
            _put(fixture, 0x14, "f", 1.0)  # density
            _put(fixture, 0x30, "ff", *_fv([state.fixtures.friction[f], state.fixtures.restitution[f]]))
            _put(fixture, 0x44, "HHh", 1, 0xFFFF, 0)
            shape = bytearray(R.SHAPE_BYTES)
            st = int(model.shape_type[f])
            _put(shape, 0x08, "i", st)
            _put(shape, 0x0C, "f", *_fv([model.radius[f]]))
            if st == 0:
                _put(shape, 0x10, "ff", *_fv(model.verts[f, 0]))
            else:
                n = int(model.count[f])
                _put(shape, 0x10, "ff", *_fv(model.centroid[f]))
                _put(shape, 0x18, f"{2 * n}f", *_fv(model.verts[f, :n]))
                _put(shape, 0x58, f"{2 * n}f", *_fv(model.normals[f, :n]))
                _put(shape, 0x98, "i", n)
            out += struct.pack("<ii", f, 0) + bytes(fixture) + bytes(shape)
    names = "\n".join(f"collider{f}#0" for f in range(model.fixture_body.shape[0])) + "\n\n\n"
    out += struct.pack("<i", len(names.encode())) + names.encode()
    return bytes(out)


def encode_native(model, state, settings):
    """A NAT payload of a single-world State: world block, non-static bodies newest first with list links, joints
    newest first, live contacts in list order (key descending)."""
    bd, jn, ct, toi = state.bodies, state.joints, state.contacts, state.toi
    B = bd.type.shape[0]
    addr = [ADDR0 + 0x1000 * k for k in range(B)]
    order = list(reversed(range(B)))  # list order
    out = bytearray(struct.pack("<i", R.WORLD_BYTES))
    w = bytearray(R.WORLD_BYTES)
    _put(w, 0x10, "ii", B, jn.motor_speed.shape[0])
    _put(w, 0x58, "ff", *_fv(state.gravity))
    w[0x60] = int(settings.allow_sleep)
    _put(w, 0x78, "f", *_fv([state.inv_dt0]))
    w[0x7C], w[0x7D] = int(settings.warm_starting), int(settings.continuous_physics)
    _put(w, 0x80, "i", (1 if bool(state.new_fixture) else 0) | (4 if settings.auto_clear_forces else 0))
    out += w
    dyn = [b for b in order if int(bd.type[b]) != wd.STATIC]
    out += struct.pack("<i", len(dyn))
    for b in dyn:
        raw = bytearray(R.BODY_BYTES)
        li = order.index(b)
        fl = (0x02 * bool(bd.awake[b]) | 0x04 * bool(bd.allow_sleep[b]) | 0x08 * bool(bd.bullet[b])
              | 0x20 * bool(bd.active[b]) | 0x80 * bool(bd.continuous[b]))
        _put(raw, 0x00, "iIi", int(bd.type[b]), fl, -1)
        _put(raw, 0x0C, "ffff", *_fv([bd.xf_p[b, 0], bd.xf_p[b, 1], bd.xf_q[b, 1], bd.xf_q[b, 0]]))
        _put(raw, 0x1C, "9f", *_fv([bd.local_center[b], bd.c0[b], bd.c[b], bd.a0[b], bd.a[b], toi.alpha0[b]]))
        _put(raw, 0x40, "ff", *_fv(bd.v[b]))
        _put(raw, 0x48, "f", *_fv([bd.w[b]]))
        _put(raw, 0x4C, "fff", *_fv([bd.force[b], bd.torque[b]]))
        _put(raw, 0x60, "qq", addr[order[li - 1]] if li > 0 else 0, addr[order[li + 1]] if li + 1 < B else 0)
        _put(raw, 0x90, "ff", *_fv([bd.mass[b], bd.inv_mass[b]]))
        _put(raw, 0xA0, "6f", *_fv([bd.inertia[b], bd.inv_inertia[b], bd.linear_damping[b], bd.angular_damping[b],
                                    bd.gravity_scale[b], bd.sleep_time[b]]))
        out += struct.pack("<i", b) + bytes(raw)
    J = jn.motor_speed.shape[0]
    out += struct.pack("<i", J)
    x = R.Layout.JOINT_BASE
    for j in reversed(range(J)):
        raw = bytearray(R.JOINT_BYTES)
        t = int(model.joint_type[j])
        _put(raw, 0x08, "i", t)
        _put(raw, 0x60, "qq", addr[int(model.joint_a[j])], addr[int(model.joint_b[j])])
        if t == wd.REVOLUTE:
            _put(raw, x, "4f", *_fv([model.local_anchor_a[j], model.local_anchor_b[j]]))
            _put(raw, x + 0x10, "6f", *_fv([jn.impulse[j], jn.motor_impulse[j], jn.lower_impulse[j],
                                             jn.upper_impulse[j]]))
            raw[x + 0x28] = int(jn.enable_motor[j])
            _put(raw, x + 0x2C, "ff", *_fv([jn.max_motor[j], jn.motor_speed[j]]))
            raw[x + 0x34] = int(jn.enable_limit[j])
            _put(raw, x + 0x38, "fff", *_fv([model.reference_angle[j], jn.lower[j], jn.upper[j]]))
        else:
            raise AssertionError("the encoder writes revolute joints only")
        out += struct.pack("<i", j) + bytes(raw)
    live = [s for s in range(ct.pair.shape[0]) if int(ct.pair[s]) >= 0]
    live.sort(key=lambda s: -int(ct.key[s]))
    out += struct.pack("<i", len(live))
    m = R.Layout.CONTACT_MANIFOLD
    for s in live:
        img = bytearray(R.CONTACT_BYTES)
        fl = 0x02 * bool(ct.touching[s]) | 0x04 * bool(toi.enabled[s]) | 0x20 * bool(toi.flag[s])
        _put(img, 0x08, "I", fl)
        cnt = int(ct.count[s])
        for k in range(cnt):
            _put(img, m + 0x14 * k, "ffffi", *_fv([ct.point_local[s, k], ct.normal_impulse[s, k],
                                                   ct.tangent_impulse[s, k]]), int(ct.point_id[s, k]))
        _put(img, m + 0x28, "4fii", *_fv([ct.local_normal[s], ct.local_point[s]]), int(ct.mtype[s]), cnt)
        _put(img, 0x110, "if", int(toi.count[s]), *_fv([toi.toi[s]]))
        _put(img, 0x118, "fff", *_fv([ct.friction[s], ct.restitution[s], ct.tangent_speed[s]]))
        out += struct.pack("<iiii", int(ct.fa[s]), 0, int(ct.fb[s]), 0)
        for off, n in R.CONTACT_SLICES:
            out += img[off:off + n]
    return bytes(out)


def encode_record(sections, version=3):
    out = bytearray(struct.pack("<Ii", R.RECORD_MAGIC, version))
    for tag, payload in sections:
        out += struct.pack("<Ii", tag, len(payload)) + payload
    return bytes(out)


def _world(state, w):
    return wd.from_leaves([np.array(x[w], copy=True) for x in wd.leaves(state)])


@pytest.fixture(scope="module")
def stepped():
    """Config 4's terrain and rig, 6 worlds placed with the benchmark's velocities, stepped 14 times by the oracle
    with random actions: live contacts with manifolds, impulses and TOI bookkeeping."""
    from oracle import oracle as O
    cfg = scenes.CONFIGS[4]
    s = scenes.settings_for(cfg)
    model, state, pts = scenes.build_world(cfg, s)
    st = scenes.place_worlds(cfg, model, state, pts, 6)
    rng = np.random.default_rng(3)
    for _ in range(14):
        scenes.apply_actions(st.joints.motor_speed, st.joints.max_motor, scenes.actions(rng, 6))
        O.step_(model, st, s, cfg.dt)
    return O, s, model, st, cfg


def _canonical_contacts(state):
    """Live slots in list order (key descending), every contact and contact-TOI field but the key's value. A manifold
    without points keeps its type, normal and point from whatever last wrote the slot (b2Contact's memory comes from
    the block allocator unset), which nothing reads: those three count only when the manifold has points."""
    ct, toi = state.contacts, state.toi
    live = sorted((s for s in range(ct.pair.shape[0]) if ct.pair[s] >= 0), key=lambda s: -int(ct.key[s]))
    rows = []
    for s in live:
        cnt = int(ct.count[s])
        geo = (int(ct.mtype[s]), ct.local_normal[s].tobytes(), ct.local_point[s].tobytes()) if cnt else None
        rows.append((int(ct.pair[s]), int(ct.fa[s]), int(ct.fb[s]), bool(ct.touching[s]), cnt, geo,
                     ct.point_local[s, :cnt].tobytes(),
                     ct.point_id[s, :cnt].tobytes(), ct.normal_impulse[s, :cnt].tobytes(),
                     ct.tangent_impulse[s, :cnt].tobytes(), ct.friction[s].tobytes(), ct.restitution[s].tobytes(),
                     ct.tangent_speed[s].tobytes(), int(toi.count[s]), toi.toi[s].tobytes(), bool(toi.flag[s]),
                     bool(toi.enabled[s])))
    return rows


BODY_FIELDS = [f for f in wd.Bodies._fields]
JOINT_FIELDS = [f for f in wd.Joints._fields]


def test_framing_sections_and_errors():
    scr = struct.pack("<i", 3) + np.array([1.5, -2.0, 0.25], "<f4").tobytes() + struct.pack("<i", 2) + \
        struct.pack("<ii", 7, 9) + struct.pack("<i", 0)
    tm = np.array([3.5, 1.25], "<f4").tobytes() + struct.pack("<i", 42) + np.array([0.5, -0.75], "<f4").tobytes()
    rec = encode_record([(R.TAG_SCRIPT + (1 << 24), scr), (R.TAG_NATIVE, struct.pack("<i", -1)), (R.TAG_TIME, tm)])
    r = R.read_record(rec)
    assert r.version == 3 and len(r.sections) == 3
    floats, lists = r.script(1)
    assert floats.tolist() == [1.5, -2.0, 0.25] and [x.tolist() for x in lists] == [[7, 9], []]
    assert r.script(0) is None
    assert r.native(0) is None  # the -1 of an unmapped world
    assert r.native(1) is None  # absent
    assert r.time() == {"record_ms": 3.5, "native_ms": 1.25, "generation": 42, "action": (0.5, -0.75)}
    # a 'W' reply: count, then length-prefixed records
    reply = struct.pack("<i", 2) + b"".join(struct.pack("<i", len(x)) + x for x in (rec, rec))
    assert [len(x.sections) for x in R.read_action(reply)] == [3, 3]
    with pytest.raises(R.RecordError, match="magic"):
        R.read_record(b"XXXX" + rec[4:])
    with pytest.raises(R.RecordError, match="truncated"):
        R.read_record(rec[:-3])
    with pytest.raises(R.RecordError, match="magic"):
        R.read_geometry(rec)
    with pytest.raises(R.RecordError, match="world block"):
        R.decode_native(struct.pack("<i", 0x40) + bytes(0x40))


@pytest.mark.parametrize("w", [0, 3, 5])
def test_snapshot_round_trip(stepped, w):
    """Geometry and NAT payload of a stepped world decode to its Model and State: every body and joint leaf, every
    live contact's fields in list order, the world's gravity and inv_dt0, and the Settings flags."""
    O, s, model, st, cfg = stepped
    one = _world(st, w)
    assert int(np.sum(one.contacts.pair >= 0)) > 0
    geo = R.read_geometry(encode_geometry(model, one))
    rec = R.read_record(encode_record([(R.TAG_NATIVE, encode_native(model, one, s)),
                                       (R.TAG_NATIVE + (1 << 24), encode_native(model, one, s))]))
    snap = rec.native(0)
    assert len(snap.bodies) == 4 and len(snap.joints) == 3
    m2, s2, set2, maps = R.to_world(geo, snap, s, contact_capacity=one.contacts.pair.shape[0])
    for f in ("fixture_body", "shape_type", "radius", "count", "verts", "normals", "joint_type", "joint_a", "joint_b",
              "local_anchor_a", "local_anchor_b", "reference_angle", "pair_a", "pair_b", "centroid"):
        assert np.asarray(getattr(m2, f)).tobytes() == np.asarray(getattr(model, f)).tobytes(), f
    for f in BODY_FIELDS:
        assert getattr(s2.bodies, f).tobytes() == getattr(one.bodies, f).tobytes(), f
    for f in JOINT_FIELDS:
        if f == "limit_state":  # the v2.4.1 revolute keeps no limit state
            continue
        assert getattr(s2.joints, f).tobytes() == getattr(one.joints, f).tobytes(), f
    assert s2.fixtures.friction.tobytes() == one.fixtures.friction.tobytes()
    assert s2.toi.alpha0.tobytes() == one.toi.alpha0.tobytes()
    assert _canonical_contacts(s2) == _canonical_contacts(one)
    assert s2.gravity.tobytes() == one.gravity.tobytes() and s2.inv_dt0.tobytes() == one.inv_dt0.tobytes()
    assert (set2.allow_sleep, set2.warm_starting, set2.continuous_physics) == (
        s.allow_sleep, s.warm_starting, s.continuous_physics)
    assert maps.body_of_rb == {1: 1, 2: 2, 3: 3, 4: 4} and maps.ground == [0]
    assert maps.joint_of == {0: 0, 1: 1, 2: 2}
    assert maps.fixture_of[(5, 0)] == 5


def test_decoded_state_steps_like_the_original(stepped):
    """The 6 worlds decoded and stepped 12 times by the oracle equal the originals stepped alike: bodies and joints bit
    for bit, contacts in list order, with TOI events on the way. The fat AABBs are not in a record (recomputed from
    the pose), so the test hands the originals' over before stepping."""
    O, s, model, st, cfg = stepped
    n = st.bodies.type.shape[0]
    geo = R.read_geometry(encode_geometry(model, _world(st, 0)))
    dec = []
    for w in range(n):
        one = _world(st, w)
        m2, s2, set2, _ = R.to_world(geo, R.decode_native(encode_native(model, one, s)), s,
                                     contact_capacity=one.contacts.pair.shape[0])
        dec.append(s2._replace(fixtures=s2.fixtures._replace(fat=one.fixtures.fat.copy())))
    a = wd.from_leaves([np.array(x, copy=True) for x in wd.leaves(st)])
    b = wd.from_leaves([np.stack(v) for v in zip(*[wd.leaves(x) for x in dec])])
    rng = np.random.default_rng(11)
    events = 0
    for k in range(12):
        act = scenes.actions(rng, n)
        for x, mm in ((a, model), (b, m2)):
            scenes.apply_actions(x.joints.motor_speed, x.joints.max_motor, act)
            O.step_(mm, x, set2, cfg.dt)
        events += int(a.toi.events.sum())
        for f in BODY_FIELDS:
            assert getattr(a.bodies, f).tobytes() == getattr(b.bodies, f).tobytes(), (k, f)
        for f in JOINT_FIELDS:
            assert getattr(a.joints, f).tobytes() == getattr(b.joints, f).tobytes(), (k, f)
        for w in range(n):
            assert _canonical_contacts(_world(a, w)) == _canonical_contacts(_world(b, w)), (k, w)
    assert events > 0  # the TOI path ran on the decoded States


def test_body_addresses_from_list_links():
    """List [D0, S1, D2, D3, S4] (D recorded with Rigidbody2D indices 0, 2, 3; S static, unrecorded): each recorded
    body names its neighbours' addresses; D0's own address is known to no recorded neighbour."""
    A = [0x1000 * (k + 1) for k in range(5)]

    def body(rb, k):
        raw = bytearray(R.BODY_BYTES)
        struct.pack_into("<iIi", raw, 0, wd.DYNAMIC, 0x22, -1)
        struct.pack_into("<qq", raw, 0x60, A[k - 1] if k > 0 else 0, A[k + 1] if k + 1 < 5 else 0)
        return R.NativeBody(rb, bytes(raw))
    geo = [R.GeoBody(0, wd.DYNAMIC, []), R.GeoBody(-1, wd.STATIC, []), R.GeoBody(2, wd.DYNAMIC, []),
           R.GeoBody(3, wd.DYNAMIC, []), R.GeoBody(-1, wd.STATIC, [])]
    snap = R.NativeSnapshot(None, [body(0, 0), body(2, 2), body(3, 3)], [], [])
    assert R._body_addresses(snap, geo) == {A[1]: 1, A[2]: 2, A[3]: 3, A[4]: 4}


def test_unmapped_objects_are_refused(stepped):
    O, s, model, st, cfg = stepped
    one = _world(st, 2)
    geo = R.read_geometry(encode_geometry(model, one))
    snap = R.decode_native(encode_native(model, one, s))
    snap.contacts[0].fixture_a = (99999, 0)
    with pytest.raises(R.RecordError, match="not in the geometry"):
        R.to_world(geo, snap, s, contact_capacity=one.contacts.pair.shape[0])
    snap = R.decode_native(encode_native(model, one, s))
    snap.joints[0].raw = snap.joints[0].raw[:0x60] + struct.pack("<q", 0x1234560) + snap.joints[0].raw[0x68:]
    with pytest.raises(R.RecordError, match="body address"):
        R.to_world(geo, snap, s, contact_capacity=one.contacts.pair.shape[0])
    snap = R.decode_native(encode_native(model, one, s))
    with pytest.raises(R.RecordError, match="exceed"):
        R.to_world(geo, snap, s, contact_capacity=1)
    # a moving body at the head of the snapshot's list with no geometry (created after the maps: the gift,
    # NativeRecord.cs:98), unmapped (-1) or with a Rigidbody2D index the geometry does not know
    for rb in (-1, 77):
        snap = R.decode_native(encode_native(model, one, s))
        snap.bodies.insert(0, R.NativeBody(rb, snap.bodies[0].raw))
        with pytest.raises(R.RecordError, match="no entry in the geometry"):
            R.to_world(geo, snap, s, contact_capacity=one.contacts.pair.shape[0])
