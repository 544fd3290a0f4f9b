"""The game plugin's step records decoded into this package's Model and State.

A step record (plugin/GameRecord.cs:20-28) is little-endian: int32 magic "GOR1", int32 version, then sections
{int32 tag, int32 length, payload}. The sections this module reads:
  - NAT0 / NAT1 (tag "NAT0" + which << 24): the native b2World just before and just after Simulate, written by
    NativeBox2D.Snapshot (plugin/NativeRecord.cs:92-152): the world's fields after m_bodyList, every non-static body
    (its Rigidbody2D index and the raw b2Body), every joint (its Joint2D index and raw bytes), every contact (the
    (collider, piece) ids of both fixtures and three raw slices of the b2Contact);
  - SCR0..SCR2: the controller's script-state floats (GameRecord.cs:33-47), then the tracked collider lists;
  - TIME: record and native-read milliseconds, generation, and the action the controller read (GameRecord.cs:172-179).
A geometry blob (GameRecord.cs:337-360, "GOG1") holds every body's fixtures with the raw b2Fixture and shape bytes
(NativeRecord.cs:156-182) and the collider / body / joint name tables.

The raw blocks are read at the offsets of the game's Box2D build (plugin/NativeBox2D.cs:32-60, the JSON dump's field
list at NativeBox2D.cs:400-468). to_world() lays a geometry and one snapshot out as (Model, State) the way
WorldDef.build would: bodies, fixtures and joints in creation order (the native lists reversed: Box2D prepends), the
contacts in slots with keys that keep the native list order (newest first = largest key).

What a record does not carry, and what stands in for it:
  - the static bodies' transforms (only non-static bodies are snapshotted): identity, as for the game's ground body,
    whose colliders are baked in world coordinates;
  - the broad-phase fat AABBs: recomputed from the recorded pose as b2BroadPhase::CreateProxy makes them (the game's
    tree is history-dependent; this only moves when a new contact begins);
  - a joint's collideConnected flag: false (the game's joints);
  - a body's own address: each recorded body's list links give its neighbours' addresses, so a joint can be
    attached to every body next to a recorded one; a body whose neighbours are both unrecorded (static) cannot be
    found, and a joint on it is refused;
  - Unity's Continuous mode per body: bit 0x0080 of b2Body::m_flags, the bit the reference's Box2D patch gives it
    (scripts/patches/box2d-2.3.1-goi.patch: e_continuousFlag).
No recordings exist to check this against: parity of the decoder is unpinned. The tests pin it against an encoder
written from the same layout (round trips of every field) and by stepping a decoded State against the original.
"""
import struct
from dataclasses import dataclass, field, replace

import numpy as np

from . import shapes
from . import world as wd

F32, I32 = np.float32, np.int32

RECORD_MAGIC = 0x31524F47    # "GOR1" (GameRecord.cs:164)
GEOMETRY_MAGIC = 0x31474F47  # "GOG1" (GameRecord.cs:343)
TAG_SCRIPT, TAG_NATIVE, TAG_EVENTS, TAG_TIME = 0x30524353, 0x3054414E, 0x53545645, 0x454D4954  # GameRecord.cs:49
TAG_POINTS, TAG_TRANSFORMS = 0x53545043, 0x304D4654

# Raw block sizes kept per object (NativeRecord.cs:13-17 over NativeBox2D.cs:32-60).
WORLD_BYTES = 0x88
BODY_BYTES = 0xC8
JOINT_BYTES = 0x150
CONTACT_SLICES = ((0x08, 0x04), (0x70, 0x58), (0x110, 0x14))  # (offset in b2Contact, length)
CONTACT_BYTES = 0x130
FIXTURE_BYTES = 0x58
SHAPE_BYTES = 0xA0


class Layout:
    """Field offsets of the game's Box2D build (NativeBox2D.cs:32-60)."""
    BODY_TYPE, BODY_FLAGS, BODY_ISLAND, BODY_XF, BODY_SWEEP = 0x00, 0x04, 0x08, 0x0C, 0x1C
    BODY_V, BODY_W, BODY_FORCE, BODY_TORQUE, BODY_PREV, BODY_NEXT = 0x40, 0x48, 0x4C, 0x54, 0x60, 0x68
    BODY_MASS, BODY_INV_MASS, BODY_I, BODY_INV_I = 0x90, 0x94, 0xA0, 0xA4
    BODY_LINEAR_DAMPING, BODY_ANGULAR_DAMPING, BODY_GRAVITY_SCALE, BODY_SLEEP_TIME = 0xA8, 0xAC, 0xB0, 0xB4
    FIX_DENSITY, FIX_FRICTION, FIX_RESTITUTION, FIX_FILTER, FIX_SENSOR = 0x14, 0x30, 0x34, 0x44, 0x4A
    SHAPE_TYPE, SHAPE_RADIUS, CIRCLE_P, POLY_CENTROID, POLY_VERTS, POLY_NORMALS, POLY_COUNT = (
        0x08, 0x0C, 0x10, 0x10, 0x18, 0x58, 0x98)
    CONTACT_FLAGS, CONTACT_INDEX_A, CONTACT_INDEX_B, CONTACT_MANIFOLD, CONTACT_RADII = 0x08, 0x70, 0x74, 0x80, 0xC0
    CONTACT_TOI_COUNT, CONTACT_TOI, CONTACT_FRICTION, CONTACT_RESTITUTION, CONTACT_TANGENT_SPEED = (
        0x110, 0x114, 0x118, 0x11C, 0x120)
    JOINT_TYPE, JOINT_BODY_A, JOINT_BODY_B, JOINT_BASE = 0x08, 0x60, 0x68, 0x98
    WORLD_BODY_COUNT, WORLD_JOINT_COUNT, WORLD_GRAVITY, WORLD_ALLOW_SLEEP = 0x10, 0x14, 0x58, 0x60
    WORLD_INV_DT0, WORLD_WARM_STARTING, WORLD_CONTINUOUS, WORLD_SUB_STEPPING, WORLD_STEP_COMPLETE = (
        0x78, 0x7C, 0x7D, 0x7E, 0x7F)
    WORLD_FLAGS = 0x80


# b2Body::m_flags and b2Contact::m_flags (Box2D 2.3.1 b2Body.h, b2Contact.h; continuous: the reference's patch)
BODY_AWAKE, BODY_AUTO_SLEEP, BODY_BULLET, BODY_FIXED_ROTATION, BODY_ACTIVE, BODY_CONTINUOUS = (
    0x02, 0x04, 0x08, 0x10, 0x20, 0x80)
CONTACT_TOUCHING, CONTACT_ENABLED, CONTACT_TOI = 0x02, 0x04, 0x20
WORLD_NEW_FIXTURE, WORLD_CLEAR_FORCES = 0x01, 0x04  # b2World::m_flags


class RecordError(ValueError):
    """A record or geometry blob that does not parse."""


class _Cursor:
    def __init__(self, buf, what):
        self.b = memoryview(bytes(buf))
        self.o = 0
        self.what = what

    def take(self, n):
        if n < 0 or self.o + n > len(self.b):
            raise RecordError(f"{self.what}: truncated at byte {self.o} (needs {n} more)")
        v = self.b[self.o:self.o + n]
        self.o += n
        return bytes(v)

    def i32(self):
        return struct.unpack("<i", self.take(4))[0]

    def u32(self):
        return struct.unpack("<I", self.take(4))[0]

    def f32(self):
        return np.frombuffer(self.take(4), "<f4")[0]

    def left(self):
        return len(self.b) - self.o


def _f(raw, o, n=None):
    """float32 at byte o of raw (n of them as an array)."""
    if n is None:
        return np.frombuffer(raw, "<f4", 1, o)[0]
    return np.frombuffer(raw, "<f4", n, o).copy()


def _i(raw, o):
    return struct.unpack_from("<i", raw, o)[0]


def _u(raw, o):
    return struct.unpack_from("<I", raw, o)[0]


def _p(raw, o):
    return struct.unpack_from("<q", raw, o)[0]


# ---------------------------------------------------------------- framing

@dataclass
class Record:
    """One step record: its version and sections in file order."""
    version: int
    sections: list  # [(tag, payload bytes)]

    def payload(self, tag):
        for t, p in self.sections:
            if t == tag:
                return p
        return None

    def native(self, which):
        """The NAT<which> snapshot (0: before Simulate, 1: after), None if absent or unreadable at record time."""
        p = self.payload(TAG_NATIVE + (which << 24))
        return None if p is None else decode_native(p)

    def script(self, which):
        """SCR<which>: (floats, hammer's tracked colliders, pot's tracked colliders) (GameRecord.cs:255-290)."""
        p = self.payload(TAG_SCRIPT + (which << 24))
        if p is None:
            return None
        c = _Cursor(p, "SCR section")
        n = c.i32()
        floats = np.frombuffer(c.take(4 * n), "<f4").copy()
        lists = []
        while c.left() >= 4:
            k = c.i32()
            lists.append(np.frombuffer(c.take(4 * k), "<i4").copy())
        return floats, lists

    def time(self):
        """TIME: dict of record_ms, native_ms, generation and the action the controller read."""
        p = self.payload(TAG_TIME)
        if p is None:
            return None
        c = _Cursor(p, "TIME section")
        out = {"record_ms": float(c.f32()), "native_ms": float(c.f32()), "generation": c.i32()}
        out["action"] = (float(c.f32()), float(c.f32()))
        return out


def read_record(buf):
    """A Record from the bytes of one step record."""
    c = _Cursor(buf, "record")
    magic = c.u32()
    if magic != RECORD_MAGIC:
        raise RecordError(f"not a step record (magic {magic:#x})")
    version = c.i32()
    sections = []
    while c.left():
        tag = c.u32()
        n = c.i32()
        sections.append((tag, c.take(n)))
    return Record(version, sections)


def read_action(buf):
    """The records of one 'W' reply (GameRecord.cs:104-120): int32 count, then {int32 length, record} each."""
    c = _Cursor(buf, "action reply")
    return [read_record(c.take(c.i32())) for _ in range(c.i32())]


# ---------------------------------------------------------------- native snapshot

@dataclass
class NativeBody:
    rb: int        # Rigidbody2D index (-1: unmapped)
    raw: bytes     # the b2Body's first BODY_BYTES bytes

    type = property(lambda s: _i(s.raw, Layout.BODY_TYPE))
    flags = property(lambda s: _u(s.raw, Layout.BODY_FLAGS))
    prev = property(lambda s: _p(s.raw, Layout.BODY_PREV))
    next = property(lambda s: _p(s.raw, Layout.BODY_NEXT))


@dataclass
class NativeJoint:
    index: int     # Joint2D index (-1: unmapped)
    raw: bytes     # JOINT_BYTES bytes: the base b2Joint, then the derived class's fields from Layout.JOINT_BASE

    type = property(lambda s: _i(s.raw, Layout.JOINT_TYPE))
    body_a = property(lambda s: _p(s.raw, Layout.JOINT_BODY_A))
    body_b = property(lambda s: _p(s.raw, Layout.JOINT_BODY_B))


@dataclass
class NativeContact:
    fixture_a: tuple  # (collider, piece); (-1, -1) unmapped
    fixture_b: tuple
    raw: bytes        # a CONTACT_BYTES image with the recorded slices in place, zeros elsewhere

    flags = property(lambda s: _u(s.raw, Layout.CONTACT_FLAGS))


@dataclass
class NativeSnapshot:
    world: bytes      # WORLD_BYTES from m_bodyList, or None
    bodies: list      # NativeBody, non-static, in body-list order (newest first)
    joints: list      # NativeJoint in joint-list order
    contacts: list    # NativeContact in contact-list order (newest first)

    def world_fields(self):
        """gravity, inv_dt0 and the world's flags, None without the world block."""
        w = self.world
        if w is None:
            return None
        L = Layout
        return {"gravity": _f(w, L.WORLD_GRAVITY, 2), "inv_dt0": _f(w, L.WORLD_INV_DT0),
                "allow_sleep": bool(w[L.WORLD_ALLOW_SLEEP]), "warm_starting": bool(w[L.WORLD_WARM_STARTING]),
                "continuous_physics": bool(w[L.WORLD_CONTINUOUS]), "sub_stepping": bool(w[L.WORLD_SUB_STEPPING]),
                "step_complete": bool(w[L.WORLD_STEP_COMPLETE]), "body_count": _i(w, L.WORLD_BODY_COUNT),
                "joint_count": _i(w, L.WORLD_JOINT_COUNT),
                "new_fixture": bool(_i(w, L.WORLD_FLAGS) & WORLD_NEW_FIXTURE),
                "auto_clear_forces": bool(_i(w, L.WORLD_FLAGS) & WORLD_CLEAR_FORCES)}


def decode_native(payload):
    """A NativeSnapshot from a NAT section's payload (NativeRecord.cs:92-152); None for the -1 written when the
    world could not be mapped (GameRecord.cs:248)."""
    c = _Cursor(payload, "NAT section")
    nw = c.i32()
    if nw == -1:
        return None
    if nw not in (0, WORLD_BYTES):
        raise RecordError(f"NAT section: world block of {nw} bytes")
    world = c.take(nw) if nw else None
    bodies = []
    for _ in range(c.i32()):
        rb = c.i32()
        bodies.append(NativeBody(rb, c.take(BODY_BYTES)))
    joints = []
    for _ in range(c.i32()):
        ji = c.i32()
        joints.append(NativeJoint(ji, c.take(JOINT_BYTES)))
    contacts = []
    for _ in range(c.i32()):
        ca, pa, cb, pb = c.i32(), c.i32(), c.i32(), c.i32()
        img = bytearray(CONTACT_BYTES)
        for off, n in CONTACT_SLICES:
            img[off:off + n] = c.take(n)
        contacts.append(NativeContact((ca, pa), (cb, pb), bytes(img)))
    if c.left():
        raise RecordError(f"NAT section: {c.left()} bytes past the last contact")
    return NativeSnapshot(world, bodies, joints, contacts)


# ---------------------------------------------------------------- geometry

@dataclass
class GeoFixture:
    collider: int
    piece: int
    fixture: bytes  # FIXTURE_BYTES of the b2Fixture
    shape: bytes    # SHAPE_BYTES of its shape (zeros past a circle's fields)

    shape_type = property(lambda s: _i(s.shape, Layout.SHAPE_TYPE))
    radius = property(lambda s: _f(s.shape, Layout.SHAPE_RADIUS))
    friction = property(lambda s: _f(s.fixture, Layout.FIX_FRICTION))
    restitution = property(lambda s: _f(s.fixture, Layout.FIX_RESTITUTION))
    density = property(lambda s: _f(s.fixture, Layout.FIX_DENSITY))
    sensor = property(lambda s: bool(s.fixture[Layout.FIX_SENSOR]))

    def filter(self):
        """(categoryBits, maskBits, groupIndex) of b2Filter."""
        return struct.unpack_from("<HHh", self.fixture, Layout.FIX_FILTER)


@dataclass
class GeoBody:
    rb: int        # Rigidbody2D index (-1: the static ground, or unmapped)
    type: int      # b2BodyType (-1: unreadable at record time)
    fixtures: list  # GeoFixture in the body's fixture-list order (newest first)


@dataclass
class Geometry:
    version: int
    bodies: list              # GeoBody in body-list order (newest first, the ground last)
    colliders: list = field(default_factory=list)  # names, by collider index
    rigidbodies: list = field(default_factory=list)
    joints: list = field(default_factory=list)


def read_geometry(buf):
    """A Geometry from the bytes of a 'g' reply (GameRecord.cs:337-360, NativeRecord.cs:156-182)."""
    c = _Cursor(buf, "geometry")
    magic = c.u32()
    if magic != GEOMETRY_MAGIC:
        raise RecordError(f"not a geometry blob (magic {magic:#x})")
    version = c.i32()
    nb = c.i32()
    bodies = []
    for _ in range(max(nb, 0)):
        rb, btype, nf = c.i32(), c.i32(), c.i32()
        fixtures = []
        for _ in range(nf):
            col, piece = c.i32(), c.i32()
            fixtures.append(GeoFixture(col, piece, c.take(FIXTURE_BYTES), c.take(SHAPE_BYTES)))
        bodies.append(GeoBody(rb, btype, fixtures))
    names = [[], [], []]
    if c.left():
        text = c.take(c.i32()).decode("utf-8")
        parts = text.split("\n\n")
        for k in range(min(3, len(parts))):
            names[k] = [ln for ln in parts[k].split("\n") if ln]
    return Geometry(version, bodies, *names)


# ---------------------------------------------------------------- into a Model and State

@dataclass
class Maps:
    """How the record's objects map onto the built Model: body / fixture / joint index of each."""
    body_of_rb: dict      # Rigidbody2D index -> body
    ground: list          # bodies without a Rigidbody2D (static), in creation order
    fixture_of: dict      # (collider, piece) -> fixture
    joint_of: dict        # Joint2D index -> joint (in the snapshot's joint list, creation order)


def _body_addresses(snap, geo_order):
    """Native addresses of the bodies, recovered from the recorded list links. geo_order is the full body list
    (GeoBody) in list order; the recorded (non-static) bodies sit in it at their Rigidbody2D's positions, and the
    bodies between two recorded ones are static. For consecutive recorded bodies a, b: if they are neighbours in the
    list, a.next is b's address and b.prev is a's; otherwise a.next is the address of the body right after a and
    b.prev that of the body right before b. The last recorded body's next and the first one's prev name their
    neighbours the same way. Returns {address: position in geo_order}."""
    rb_pos = {g.rb: k for k, g in enumerate(geo_order) if g.rb >= 0}
    addr = {}
    R = [b for b in snap.bodies if b.rb in rb_pos]
    for k, b in enumerate(R):
        pk = rb_pos[b.rb]
        if b.next and pk + 1 < len(geo_order):
            addr[b.next] = pk + 1
        if b.prev and pk > 0:
            addr[b.prev] = pk - 1
    return addr


def to_world(geometry, snap, settings=None, contact_capacity=None):
    """(Model, State, Settings, Maps) of one snapshot over its geometry, laid out as WorldDef.build does (full fixture
    layout; compact_model / prepare make the compact one). Settings: `settings` (Settings.game() by default) with
    the world's recorded gravity, allow_sleep, warm_starting, continuous_physics and clear-forces flag.
    contact_capacity defaults to the recorded contact count (at least 1)."""
    from .settings import Settings
    settings = settings or Settings.game()
    wf = snap.world_fields()
    if wf is not None:
        settings = replace(settings, gravity=(F32(wf["gravity"][0]), F32(wf["gravity"][1])),
                           allow_sleep=wf["allow_sleep"], warm_starting=wf["warm_starting"],
                           continuous_physics=wf["continuous_physics"], auto_clear_forces=wf["auto_clear_forces"])
    geo_list = geometry.bodies  # list order
    order = list(range(len(geo_list)))[::-1]  # creation order
    snap_of_rb = {b.rb: b for b in snap.bodies if b.rb >= 0}
    # every moving body of the snapshot must have its geometry (a body created after the maps were built, such as
    # the gift at the list's head, NativeRecord.cs:98, has none and would otherwise vanish from the world)
    geo_rbs = {g.rb for g in geo_list if g.rb >= 0}
    for nb in snap.bodies:
        if nb.type != wd.STATIC and (nb.rb < 0 or nb.rb not in geo_rbs):
            raise RecordError(f"non-static snapshot body (rigidbody {nb.rb}) has no entry in the geometry")
    d = wd.WorldDef(settings)
    body_of_pos, body_of_rb, ground, fixture_of = {}, {}, [], {}
    for pos in order:
        g = geo_list[pos]
        if g.type < 0:
            raise RecordError(f"geometry body {pos} was unreadable at record time")
        nb = snap_of_rb.get(g.rb)
        if g.type != wd.STATIC and nb is None:
            raise RecordError(f"non-static body (rigidbody {g.rb}) missing from the snapshot")
        bid = d.add_body(g.type)
        body_of_pos[pos] = bid
        if g.rb >= 0:
            body_of_rb[g.rb] = bid
        else:
            ground.append(bid)
        if nb is not None:
            _body_from_raw(d.bodies[bid], nb.raw)
        for fx in reversed(g.fixtures):
            fid = _fixture_from_raw(d, bid, fx)
            if fx.collider >= 0:
                fixture_of[(fx.collider, fx.piece)] = fid
    addr = _body_addresses(snap, geo_list)
    joint_of = {}
    for nj in reversed(snap.joints):
        a, b = addr.get(nj.body_a), addr.get(nj.body_b)
        if a is None or b is None:
            raise RecordError(f"joint {nj.index}: body address not in the recorded body list")
        jid = _joint_from_raw(d, body_of_pos[a], body_of_pos[b], nj.raw)
        if nj.index >= 0:
            joint_of[nj.index] = jid
    cap = max(1, len(snap.contacts)) if contact_capacity is None else contact_capacity
    if len(snap.contacts) > cap:
        raise RecordError(f"{len(snap.contacts)} contacts exceed the contact capacity {cap}")
    model, state = d.build(contact_capacity=cap)
    state = _joint_state(state, d, snap, addr, body_of_pos)
    state = _contact_state(model, state, snap, fixture_of)
    # the prismatic axes as stored (the builder would normalise the recorded unit axis again)
    x = Layout.JOINT_BASE
    for j, nj in enumerate(reversed(snap.joints)):
        if nj.type == wd.PRISMATIC:
            model.local_axis_a[j] = _f(nj.raw, x + 0x10, 2)
            model.local_yaxis_a[j] = _f(nj.raw, x + 0x18, 2)
    bd = state.bodies
    c0, a0, alpha0 = bd.c0.copy(), bd.a0.copy(), state.toi.alpha0.copy()
    sleep, force, torque = bd.sleep_time.copy(), bd.force.copy(), bd.torque.copy()
    for rb, nb in snap_of_rb.items():
        k, raw = body_of_rb[rb], nb.raw
        c0[k] = _f(raw, Layout.BODY_SWEEP + 8, 2)
        a0[k] = _f(raw, Layout.BODY_SWEEP + 24)
        alpha0[k] = _f(raw, Layout.BODY_SWEEP + 32)
        sleep[k] = _f(raw, Layout.BODY_SLEEP_TIME)
        force[k] = _f(raw, Layout.BODY_FORCE, 2)
        torque[k] = _f(raw, Layout.BODY_TORQUE)
    bodies = bd._replace(c0=c0, a0=a0, sleep_time=sleep, force=force, torque=torque)
    inv_dt0 = np.asarray(F32(wf["inv_dt0"])) if wf is not None else state.inv_dt0
    new_fixture = np.asarray(bool(wf["new_fixture"])) if wf is not None else state.new_fixture
    state = state._replace(bodies=bodies, toi=state.toi._replace(alpha0=alpha0), inv_dt0=inv_dt0,
                           gravity=np.array(settings.gravity, F32), new_fixture=new_fixture)
    return model, state, settings, Maps(body_of_rb, ground, fixture_of, joint_of)


def _body_from_raw(rec, raw):
    """A BodyRecord's fields from a raw b2Body: b2Transform {p, q = (s, c)}, b2Sweep {localCenter, c0, c, a0, a,
    alpha0}, velocities, mass data, damping, flags. c0, a0 and alpha0 go into the State after build (the builder
    starts c0 = c, a0 = a)."""
    L = Layout
    rec.type = _i(raw, L.BODY_TYPE)
    rec.origin = _f(raw, L.BODY_XF, 2)
    s, c = _f(raw, L.BODY_XF + 8), _f(raw, L.BODY_XF + 12)
    rec.rot = (c, s)
    rec.local_center = _f(raw, L.BODY_SWEEP, 2)
    rec.center = _f(raw, L.BODY_SWEEP + 16, 2)
    rec.angle = _f(raw, L.BODY_SWEEP + 28)
    rec.v = _f(raw, L.BODY_V, 2)
    rec.w = _f(raw, L.BODY_W)
    rec.mass, rec.inv_mass = _f(raw, L.BODY_MASS), _f(raw, L.BODY_INV_MASS)
    rec.inertia, rec.inv_inertia = _f(raw, L.BODY_I), _f(raw, L.BODY_INV_I)
    rec.linear_damping, rec.angular_damping = _f(raw, L.BODY_LINEAR_DAMPING), _f(raw, L.BODY_ANGULAR_DAMPING)
    rec.gravity_scale = _f(raw, L.BODY_GRAVITY_SCALE)
    fl = _u(raw, L.BODY_FLAGS)
    rec.awake, rec.allow_sleep = bool(fl & BODY_AWAKE), bool(fl & BODY_AUTO_SLEEP)
    rec.bullet, rec.fixed_rotation = bool(fl & BODY_BULLET), bool(fl & BODY_FIXED_ROTATION)
    rec.active, rec.continuous = bool(fl & BODY_ACTIVE), bool(fl & BODY_CONTINUOUS)


def _fixture_from_raw(d, body, fx):
    """A fixture with the recorded shape's bits (vertices, normals, centroid, radius as stored)."""
    cat, mask, group = fx.filter()
    st = fx.shape_type
    if st == shapes.CIRCLE:
        return d._add_fixture(body, shapes.CIRCLE, _f(fx.shape, Layout.CIRCLE_P, 2)[None], np.zeros((1, 2), F32),
                              fx.radius, fx.friction, fx.restitution, fx.sensor, 0, cat, mask, group)
    if st != shapes.POLYGON:
        raise RecordError(f"fixture ({fx.collider}, {fx.piece}): shape type {st} (the game uses circles and polygons)")
    n = _i(fx.shape, Layout.POLY_COUNT)
    if not 3 <= n <= wd.MAX_POLYGON_VERTICES:
        raise RecordError(f"fixture ({fx.collider}, {fx.piece}): polygon of {n} vertices")
    v = _f(fx.shape, Layout.POLY_VERTS, 2 * n).reshape(n, 2)
    nr = _f(fx.shape, Layout.POLY_NORMALS, 2 * n).reshape(n, 2)
    return d._add_fixture(body, shapes.POLYGON, v, nr, fx.radius, fx.friction, fx.restitution, fx.sensor, 0, cat,
                          mask, group, centroid=_f(fx.shape, Layout.POLY_CENTROID, 2))


def _joint_from_raw(d, a, b, raw):
    """A joint record from the derived class's fields (NativeBox2D.cs:448-468): revolute (v2.4.1 fields), prismatic
    and weld (v2.3.1)."""
    x, t = Layout.JOINT_BASE, _i(raw, Layout.JOINT_TYPE)
    if t == wd.REVOLUTE:
        lim = (float(_f(raw, x + 0x3C)), float(_f(raw, x + 0x40))) if raw[x + 0x34] else None
        j = d.add_revolute(a, b, tuple(_f(raw, x, 2)), tuple(_f(raw, x + 8, 2)), float(_f(raw, x + 0x38)),
                           limits=lim, motor_speed=float(_f(raw, x + 0x30)), max_motor_torque=float(_f(raw, x + 0x2C)),
                           enable_motor=bool(raw[x + 0x28]))
        if lim is None:  # the limits are State leaves even when disabled
            d.joints[j].lower, d.joints[j].upper = float(_f(raw, x + 0x3C)), float(_f(raw, x + 0x40))
        return j
    if t == wd.PRISMATIC:
        lim = (float(_f(raw, x + 0x34)), float(_f(raw, x + 0x38))) if raw[x + 0x44] else None
        j = d.add_prismatic(a, b, tuple(_f(raw, x, 2)), tuple(_f(raw, x + 8, 2)), tuple(_f(raw, x + 0x10, 2)),
                            float(_f(raw, x + 0x20)), limits=lim, motor_speed=float(_f(raw, x + 0x40)),
                            max_motor_force=float(_f(raw, x + 0x3C)), enable_motor=bool(raw[x + 0x45]))
        if lim is None:
            d.joints[j].lower, d.joints[j].upper = float(_f(raw, x + 0x34)), float(_f(raw, x + 0x38))
        return j
    if t == wd.WELD:
        return d.add_weld(a, b, tuple(_f(raw, x + 0xC, 2)), tuple(_f(raw, x + 0x14, 2)), float(_f(raw, x + 0x1C)),
                          frequency=float(_f(raw, x)), damping=float(_f(raw, x + 4)))
    raise RecordError(f"joint type {t} (the step takes revolute, prismatic and weld)")


def _joint_state(state, d, snap, addr, body_of_pos):
    """The joints' impulses (and limit state) from the raw joints; joint j of the State is the snapshot's joint
    len - 1 - j (creation order)."""
    jn = state.joints
    imp, mimp, lst = jn.impulse.copy(), jn.motor_impulse.copy(), jn.limit_state.copy()
    lo_i, up_i = jn.lower_impulse.copy(), jn.upper_impulse.copy()
    x = Layout.JOINT_BASE
    for j, nj in enumerate(reversed(snap.joints)):
        raw, t = nj.raw, nj.type
        if t == wd.REVOLUTE:
            imp[j] = _f(raw, x + 0x10, 3)
            mimp[j] = _f(raw, x + 0x1C)
            lo_i[j], up_i[j] = _f(raw, x + 0x20), _f(raw, x + 0x24)
        elif t == wd.PRISMATIC:
            imp[j] = _f(raw, x + 0x24, 3)
            mimp[j] = _f(raw, x + 0x30)
            lst[j] = _i(raw, x + 0x48)
        elif t == wd.WELD:
            imp[j] = _f(raw, x + 0x24, 3)
    return state._replace(joints=jn._replace(impulse=imp, motor_impulse=mimp, limit_state=lst, lower_impulse=lo_i,
                                             upper_impulse=up_i))


def _contact_state(model, state, snap, fixture_of):
    """The contact table: the recorded contacts in slots 0.. (newest first) with keys n - 1 .. 0, next_key n."""
    ct, toi = state.contacts, state.toi
    C = ct.pair.shape[0]
    pair_of = {(int(a), int(b)): k for k, (a, b) in enumerate(zip(model.pair_a, model.pair_b))}
    out = {k: np.array(v, copy=True) for k, v in ct._asdict().items()}
    tc, tt, tf, ten = toi.count.copy(), toi.toi.copy(), toi.flag.copy(), toi.enabled.copy()
    n = len(snap.contacts)
    m = Layout.CONTACT_MANIFOLD
    for s, nc in enumerate(snap.contacts):
        fa, fb = fixture_of.get(nc.fixture_a), fixture_of.get(nc.fixture_b)
        if fa is None or fb is None:
            raise RecordError(f"contact {s}: fixture {nc.fixture_a if fa is None else nc.fixture_b} not in the geometry")
        p = pair_of.get((fa, fb))
        if p is None:
            raise RecordError(f"contact {s}: fixtures ({fa}, {fb}) are not a candidate pair in that order")
        raw = nc.raw
        out["pair"][s], out["fa"][s], out["fb"][s], out["key"][s] = p, fa, fb, n - 1 - s
        fl = nc.flags
        out["touching"][s] = bool(fl & CONTACT_TOUCHING)
        out["mtype"][s] = _i(raw, m + 0x38)
        cnt = _i(raw, m + 0x3C)
        if not 0 <= cnt <= 2:
            raise RecordError(f"contact {s}: manifold of {cnt} points")
        out["count"][s] = cnt
        out["local_normal"][s] = _f(raw, m + 0x28, 2)
        out["local_point"][s] = _f(raw, m + 0x30, 2)
        for k in range(cnt):
            q = m + 0x14 * k
            out["point_local"][s, k] = _f(raw, q, 2)
            out["normal_impulse"][s, k] = _f(raw, q + 8)
            out["tangent_impulse"][s, k] = _f(raw, q + 12)
            out["point_id"][s, k] = _i(raw, q + 16)
        out["friction"][s] = _f(raw, Layout.CONTACT_FRICTION)
        out["restitution"][s] = _f(raw, Layout.CONTACT_RESTITUTION)
        out["tangent_speed"][s] = _f(raw, Layout.CONTACT_TANGENT_SPEED)
        tc[s] = _i(raw, Layout.CONTACT_TOI_COUNT)
        tt[s] = _f(raw, Layout.CONTACT_TOI)
        tf[s] = bool(fl & CONTACT_TOI)
        ten[s] = bool(fl & CONTACT_ENABLED)
    if n > C:
        raise RecordError(f"{n} contacts exceed {C} slots")
    return state._replace(contacts=wd.Contacts(**out), next_key=np.asarray(I32(n)), new_fixture=np.asarray(False),
                          toi=toi._replace(count=tc, toi=tt, flag=tf, enabled=ten))

