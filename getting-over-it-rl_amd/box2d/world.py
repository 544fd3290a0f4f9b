"""World layout: the shared Model and the per-world State pytrees, the host builder WorldDef, and the compact fixture
layout (mirror of goi_jax/box2d/world.py:30-563; same field names, shapes, dtypes and creation-order rules).

Host values are numpy arrays (a State built here has no batch axis). `layout.py` moves a batch of States to the GPU
as torch tensors in the kernels' worlds-minor layout and back.

Indices follow creation order, which Box2D uses for its orderings (world.py:7-11): body i is the i-th created (the
body list is newest first, so islands are seeded from the highest index); fixture i gets broad-phase proxy id order i;
joint i is the i-th created (each body's joint list is newest first).
"""
from dataclasses import dataclass
from typing import NamedTuple

import numpy as np

from . import shapes
from .settings import MAX_POLYGON_VERTICES, Settings

F32, I32 = np.float32, np.int32
STATIC, KINEMATIC, DYNAMIC = 0, 1, 2  # b2BodyType
REVOLUTE, PRISMATIC, WELD = 1, 2, 8  # b2JointType
INACTIVE_LIMIT, AT_LOWER, AT_UPPER, EQUAL_LIMITS = 0, 1, 2, 3  # b2LimitState
CIRCLES, FACE_A, FACE_B = 0, 1, 2  # b2Manifold::Type


class Model(NamedTuple):
    """Scene constants shared by every world (world.py:30-67)."""
    fixture_body: np.ndarray  # i32[F]
    shape_type: np.ndarray  # i32[F]
    radius: np.ndarray  # f32[F]
    count: np.ndarray  # i32[F]
    verts: np.ndarray  # f32[F, 8, 2]
    normals: np.ndarray  # f32[F, 8, 2]
    joint_type: np.ndarray  # i32[J]
    joint_a: np.ndarray  # i32[J]
    joint_b: np.ndarray  # i32[J]
    local_anchor_a: np.ndarray  # f32[J, 2]
    local_anchor_b: np.ndarray  # f32[J, 2]
    local_axis_a: np.ndarray  # f32[J, 2]
    local_yaxis_a: np.ndarray  # f32[J, 2]
    reference_angle: np.ndarray  # f32[J]
    pair_a: np.ndarray  # i32[P]
    pair_b: np.ndarray  # i32[P]
    toi_bodies: np.ndarray = None  # bool[B]
    fixture_slot: np.ndarray = None  # i32[F] (compact layout)
    slot_fixture: np.ndarray = None  # i32[Fd]
    static_fat: np.ndarray = None  # f32[F, 4]
    static_friction: np.ndarray = None  # f32[F]
    static_restitution: np.ndarray = None  # f32[F]
    # The reference's culled-scan tables for its FindNewContacts kernel (world.py:57-65, scan_tables). Accepted so
    # that a reference Model keeps its fields and their order; unused here: goi_model_create builds a BVH over the
    # static fat AABBs instead.
    scan_cand: np.ndarray = None
    scan_row: np.ndarray = None
    scan_box: np.ndarray = None
    body_type: np.ndarray = None  # i32[B] the body types every world shares (the compact layout requires it)
    centroid: np.ndarray = None  # f32[F, 2] b2PolygonShape::m_centroid (read by edge contacts only)
    edge_flags: np.ndarray = None  # i32[F] edge fixtures' ghost flags (shapes.EDGE_HAS_V0 | EDGE_HAS_V3 | EDGE_CHAIN)


class Bodies(NamedTuple):
    type: np.ndarray
    active: np.ndarray
    awake: np.ndarray
    allow_sleep: np.ndarray
    bullet: np.ndarray
    continuous: np.ndarray
    sleep_time: np.ndarray
    xf_p: np.ndarray
    xf_q: np.ndarray
    local_center: np.ndarray
    c0: np.ndarray
    c: np.ndarray
    a0: np.ndarray
    a: np.ndarray
    v: np.ndarray
    w: np.ndarray
    force: np.ndarray
    torque: np.ndarray
    mass: np.ndarray
    inv_mass: np.ndarray
    inertia: np.ndarray
    inv_inertia: np.ndarray
    linear_damping: np.ndarray
    angular_damping: np.ndarray
    gravity_scale: np.ndarray


class Fixtures(NamedTuple):
    friction: np.ndarray
    restitution: np.ndarray
    fat: np.ndarray


class Joints(NamedTuple):
    enable_motor: np.ndarray
    motor_speed: np.ndarray
    max_motor: np.ndarray
    enable_limit: np.ndarray
    lower: np.ndarray
    upper: np.ndarray
    frequency: np.ndarray
    damping: np.ndarray
    impulse: np.ndarray
    motor_impulse: np.ndarray
    limit_state: np.ndarray
    lower_impulse: np.ndarray
    upper_impulse: np.ndarray


class Contacts(NamedTuple):
    pair: np.ndarray
    fa: np.ndarray
    fb: np.ndarray
    key: np.ndarray
    touching: np.ndarray
    mtype: np.ndarray
    count: np.ndarray
    local_normal: np.ndarray
    local_point: np.ndarray
    point_local: np.ndarray
    point_id: np.ndarray
    normal_impulse: np.ndarray
    tangent_impulse: np.ndarray
    friction: np.ndarray
    restitution: np.ndarray
    tangent_speed: np.ndarray


class ContactTOI(NamedTuple):
    alpha0: np.ndarray
    count: np.ndarray
    toi: np.ndarray
    flag: np.ndarray
    enabled: np.ndarray
    solved: np.ndarray
    normal_impulse: np.ndarray
    tangent_impulse: np.ndarray
    events: np.ndarray


class State(NamedTuple):
    bodies: Bodies
    fixtures: Fixtures
    joints: Joints
    contacts: Contacts
    gravity: np.ndarray
    inv_dt0: np.ndarray
    next_key: np.ndarray
    new_fixture: np.ndarray
    overflow: np.ndarray
    toi: ContactTOI = None


# The State leaves in pytree order with dtype and per-world inner shape (B bodies, R fixture rows, J joints, C slots).
# The order is the C ABI's enum GoiLeaf (include/goi_b2.h).
_B, _R, _J, _C = "B", "R", "J", "C"
LEAVES = [
    ("bodies", "type", I32, (_B,)), ("bodies", "active", bool, (_B,)), ("bodies", "awake", bool, (_B,)),
    ("bodies", "allow_sleep", bool, (_B,)), ("bodies", "bullet", bool, (_B,)), ("bodies", "continuous", bool, (_B,)),
    ("bodies", "sleep_time", F32, (_B,)), ("bodies", "xf_p", F32, (_B, 2)), ("bodies", "xf_q", F32, (_B, 2)),
    ("bodies", "local_center", F32, (_B, 2)), ("bodies", "c0", F32, (_B, 2)), ("bodies", "c", F32, (_B, 2)),
    ("bodies", "a0", F32, (_B,)), ("bodies", "a", F32, (_B,)), ("bodies", "v", F32, (_B, 2)),
    ("bodies", "w", F32, (_B,)), ("bodies", "force", F32, (_B, 2)), ("bodies", "torque", F32, (_B,)),
    ("bodies", "mass", F32, (_B,)), ("bodies", "inv_mass", F32, (_B,)), ("bodies", "inertia", F32, (_B,)),
    ("bodies", "inv_inertia", F32, (_B,)), ("bodies", "linear_damping", F32, (_B,)),
    ("bodies", "angular_damping", F32, (_B,)), ("bodies", "gravity_scale", F32, (_B,)),
    ("fixtures", "friction", F32, (_R,)), ("fixtures", "restitution", F32, (_R,)), ("fixtures", "fat", F32, (_R, 4)),
    ("joints", "enable_motor", bool, (_J,)), ("joints", "motor_speed", F32, (_J,)),
    ("joints", "max_motor", F32, (_J,)), ("joints", "enable_limit", bool, (_J,)), ("joints", "lower", F32, (_J,)),
    ("joints", "upper", F32, (_J,)), ("joints", "frequency", F32, (_J,)), ("joints", "damping", F32, (_J,)),
    ("joints", "impulse", F32, (_J, 3)), ("joints", "motor_impulse", F32, (_J,)),
    ("joints", "limit_state", I32, (_J,)), ("joints", "lower_impulse", F32, (_J,)),
    ("joints", "upper_impulse", F32, (_J,)),
    ("contacts", "pair", I32, (_C,)), ("contacts", "fa", I32, (_C,)), ("contacts", "fb", I32, (_C,)),
    ("contacts", "key", I32, (_C,)), ("contacts", "touching", bool, (_C,)), ("contacts", "mtype", I32, (_C,)),
    ("contacts", "count", I32, (_C,)), ("contacts", "local_normal", F32, (_C, 2)),
    ("contacts", "local_point", F32, (_C, 2)), ("contacts", "point_local", F32, (_C, 2, 2)),
    ("contacts", "point_id", I32, (_C, 2)), ("contacts", "normal_impulse", F32, (_C, 2)),
    ("contacts", "tangent_impulse", F32, (_C, 2)), ("contacts", "friction", F32, (_C,)),
    ("contacts", "restitution", F32, (_C,)), ("contacts", "tangent_speed", F32, (_C,)),
    (None, "gravity", F32, (2,)), (None, "inv_dt0", F32, ()), (None, "next_key", I32, ()),
    (None, "new_fixture", bool, ()), (None, "overflow", I32, ()),
    ("toi", "alpha0", F32, (_B,)), ("toi", "count", I32, (_C,)), ("toi", "toi", F32, (_C,)),
    ("toi", "flag", bool, (_C,)), ("toi", "enabled", bool, (_C,)), ("toi", "solved", bool, (_C,)),
    ("toi", "normal_impulse", F32, (_C, 2)), ("toi", "tangent_impulse", F32, (_C, 2)), ("toi", "events", I32, ()),
]
assert len(LEAVES) == 71


def dims(state):
    """(B, R, J, C) of a State (batched or not)."""
    return (state.bodies.type.shape[-1], state.fixtures.friction.shape[-1], state.joints.motor_speed.shape[-1],
            state.contacts.pair.shape[-1])


def leaf_shape(inner, d):
    B, R, J, C = d
    sub = {"B": B, "R": R, "J": J, "C": C}
    return tuple(sub.get(s, s) for s in inner)


def leaves(state):
    """The 71 leaves of a State in ABI order."""
    out = []
    for group, name, _, _ in LEAVES:
        holder = state if group is None else getattr(state, group)
        out.append(getattr(holder, name))
    return out


def from_leaves(vals):
    """A State from 71 leaves in ABI order."""
    groups = {"bodies": [], "fixtures": [], "joints": [], "contacts": [], "toi": []}
    scal = {}
    for (group, name, _, _), v in zip(LEAVES, vals):
        if group is None:
            scal[name] = v
        else:
            groups[group].append(v)
    return State(bodies=Bodies(*groups["bodies"]), fixtures=Fixtures(*groups["fixtures"]),
                 joints=Joints(*groups["joints"]), contacts=Contacts(*groups["contacts"]), toi=ContactTOI(*groups["toi"]),
                 **scal)


# ---------------------------------------------------------------- the host builder

@dataclass
class BodyRecord:
    """One body as the builder holds it before build(): the b2Body fields the State starts from (float32)."""
    type: int
    origin: np.ndarray          # b2Transform.p
    rot: tuple                  # b2Rot (cos, sin) of `angle`, correctly rounded
    angle: np.float32
    center: np.ndarray          # world centre of mass (b2Sweep.c)
    local_center: np.ndarray
    v: np.ndarray
    w: np.float32
    mass: np.float32
    inv_mass: np.float32
    inertia: np.float32
    inv_inertia: np.float32
    linear_damping: np.float32
    angular_damping: np.float32
    gravity_scale: np.float32
    fixed_rotation: bool
    bullet: bool
    continuous: bool
    awake: bool
    allow_sleep: bool
    active: bool


@dataclass
class FixtureRecord:
    body: int
    shape_type: int
    verts: np.ndarray           # (8, 2) slots
    normals: np.ndarray         # (8, 2) slots
    count: int
    radius: np.float32
    friction: np.float32
    restitution: np.float32
    sensor: bool
    layer: int
    category: int
    mask: int
    group: int
    centroid: np.ndarray
    edge_flags: int


@dataclass
class JointRecord:
    type: int
    body_a: int
    body_b: int
    anchor_a: tuple
    anchor_b: tuple
    reference_angle: float
    axis: tuple
    enable_limit: bool
    lower: float
    upper: float
    motor_speed: float
    max_motor: float
    enable_motor: bool
    frequency: float
    damping: float
    collide_connected: bool


def mass_update(body, mass, center, inertia, exact=True):
    """The reference oracle's goi_b2_body_set_mass on a dynamic BodyRecord (world.py:220-244, capi.cpp:234-252):
    b2MassData {mass, center, I = inertia + mass |center|^2} through b2Body::SetMassData (a non-positive mass counts
    as 1; the rotational inertia about the centre I - m |c|^2 only when positive and the rotation is free), then, with
    `exact`, the given centroidal inertia verbatim; the centre of mass moves with the new local centre and the
    velocity picks up b2Cross(w, centre shift). float32, one rounding per operation in that order."""
    if body.type != DYNAMIC:
        return
    m_in, i_com = F32(mass), F32(inertia)
    lc = np.array([center[0], center[1]], F32)
    c2 = lc[0] * lc[0] + lc[1] * lc[1]
    i_total = i_com + m_in * c2
    m = m_in if m_in > 0 else F32(1)
    body.mass, body.inv_mass = m, F32(1) / m
    body.inertia = body.inv_inertia = F32(0)
    if i_total > 0 and not body.fixed_rotation:
        body.inertia = i_total - m * c2
        body.inv_inertia = F32(1) / body.inertia
    if exact and body.inertia > 0:
        body.inertia, body.inv_inertia = i_com, F32(1) / i_com
    cos, sin = body.rot
    moved = np.array([(cos * lc[0] - sin * lc[1]) + body.origin[0], (sin * lc[0] + cos * lc[1]) + body.origin[1]],
                     F32)
    shift = moved - body.center
    body.local_center, body.center = lc, moved
    body.v = np.array([body.v[0] - body.w * shift[1], body.v[1] + body.w * shift[0]], F32)


def _collide_filter(fx, layer_masks, rows):
    """Filter::ShouldCollide of fixtures `rows` (a slice) against every fixture (the reference oracle's contact
    filter, world.py:177-183), as a (len(rows), F) boolean matrix: with a layer matrix, bit layer(b) of
    layer_masks[layer(a)]; otherwise b2ContactFilter: a shared non-zero group decides by its sign, else category and
    mask must match both ways."""
    layer = np.array([f.layer for f in fx], np.int64)
    if layer_masks is not None:
        mine = np.array([int(layer_masks[x]) & 0xFFFFFFFF for x in layer[rows]], np.int64)
        return ((mine[:, None] >> layer[None, :]) & 1) == 1
    group = np.array([f.group for f in fx], np.int64)
    cat = np.array([f.category for f in fx], np.int64)
    msk = np.array([f.mask for f in fx], np.int64)
    g = group[rows][:, None]
    same_group = (g == group[None, :]) & (g != 0)
    by_bits = ((msk[rows][:, None] & cat[None, :]) != 0) & ((cat[rows][:, None] & msk[None, :]) != 0)
    return np.where(same_group, g > 0, by_bits)


class WorldDef:
    """Host-side builder with the reference's methods and defaults (world.py:186-387): bodies, fixtures and joints are
    recorded in creation order (which Box2D's orderings follow) and laid out as the Model and State by build()."""

    def __init__(self, settings=None, layer_masks=None):
        self.settings = settings or Settings()
        self.layer_masks = layer_masks
        self.bodies: list = []    # BodyRecord
        self.fixtures: list = []  # FixtureRecord
        self.joints: list = []    # JointRecord

    # ---- bodies

    def add_body(self, type=DYNAMIC, position=(0, 0), angle=0.0, velocity=(0, 0), angular_velocity=0.0, *,
                 mass=None, center=(0, 0), inertia=0.0, exact_inertia=True, linear_damping=0.0,
                 angular_damping=0.0, gravity_scale=1.0, fixed_rotation=False, bullet=False, continuous=False,
                 awake=True, allow_sleep=True, active=True):
        """A body at `position` and `angle`; a dynamic body starts with unit mass until set_mass (or `mass`) gives
        its mass data. A non-static body given a velocity is woken to take it, unless awake=False asks it to sleep,
        which zeroes the velocity again (b2Body::SetAwake(false)). Returns the body id."""
        ang = F32(angle)
        sin, cos = shapes.host_sin_cos(ang)
        unit = F32(1 if type == DYNAMIC else 0)
        here = np.array(position, F32)
        rec = BodyRecord(type=type, origin=here, rot=(cos, sin), angle=ang, center=here.copy(),
                         local_center=np.zeros(2, F32), v=np.zeros(2, F32), w=F32(0), mass=unit, inv_mass=unit,
                         inertia=F32(0), inv_inertia=F32(0), linear_damping=F32(linear_damping),
                         angular_damping=F32(angular_damping), gravity_scale=F32(gravity_scale),
                         fixed_rotation=bool(fixed_rotation), bullet=bool(bullet), continuous=bool(continuous),
                         awake=bool(awake), allow_sleep=bool(allow_sleep), active=bool(active))
        self.bodies.append(rec)
        if mass is not None:
            mass_update(rec, mass, center, inertia, exact_inertia)
        moving = velocity[0] or velocity[1] or angular_velocity
        if type != STATIC and moving:
            rec.awake = bool(awake)
            if awake:
                rec.v, rec.w = np.array(velocity, F32), F32(angular_velocity)
            else:
                rec.v, rec.w = np.zeros(2, F32), F32(0)
        return len(self.bodies) - 1

    def set_mass(self, body, mass, center=(0, 0), inertia=0.0, exact=True):
        """Mass data of a dynamic body (goi_b2_body_set_mass; see mass_update). No effect on other bodies."""
        mass_update(self.bodies[body], mass, center, inertia, exact)

    # ---- fixtures

    def _add_fixture(self, body, shape_type, verts, normals, radius, friction, restitution, sensor, layer,
                     category, mask, group, centroid=(0.0, 0.0), edge_flags=0, count=None):
        slots_v, slots_n = shapes.pad(verts, normals)
        self.fixtures.append(FixtureRecord(
            body=body, shape_type=shape_type, verts=slots_v, normals=slots_n,
            count=len(verts) if count is None else count, radius=F32(radius), friction=F32(friction),
            restitution=F32(restitution), sensor=bool(sensor), layer=int(layer) & 31, category=category, mask=mask,
            group=group, centroid=np.asarray(centroid, F32), edge_flags=int(edge_flags)))
        return len(self.fixtures) - 1

    def add_polygon(self, body, vertices, radius=None, raw=False, *, friction=0.2, restitution=0.0, density=0.0,
                    sensor=False, layer=0, category=1, mask=0xFFFF, group=0):
        """A polygon: vertices as given (raw; strictly convex CCW) or through b2PolygonShape::Set's hull."""
        if raw:
            v, n = shapes.polygon_raw(vertices)
            centroid = shapes.centroid_raw(v)
        else:
            v, n = shapes.polygon_set(vertices, self.settings.linear_slop)
            centroid = shapes.centroid_set(v)
        skin = self.settings.polygon_radius if radius is None else radius
        return self._add_fixture(body, shapes.POLYGON, v, n, skin, friction, restitution, sensor, layer, category,
                                 mask, group, centroid=centroid)

    def add_box(self, body, half_extents, center=(0, 0), angle=0.0, radius=None, *, friction=0.2, restitution=0.0,
                density=0.0, sensor=False, layer=0, category=1, mask=0xFFFF, group=0):
        """b2PolygonShape::SetAsBox(hx, hy, center, angle)."""
        v, n = shapes.box(half_extents[0], half_extents[1], center, angle)
        skin = self.settings.polygon_radius if radius is None else radius
        return self._add_fixture(body, shapes.POLYGON, v, n, skin, friction, restitution, sensor, layer, category,
                                 mask, group, centroid=center)

    def add_circle(self, body, radius, center=(0, 0), *, friction=0.2, restitution=0.0, density=0.0, sensor=False,
                   layer=0, category=1, mask=0xFFFF, group=0):
        """A circle of `radius` centred at `center` in body coordinates."""
        return self._add_fixture(body, shapes.CIRCLE, np.array([center], F32), np.zeros((1, 2), F32), radius,
                                 friction, restitution, sensor, layer, category, mask, group)

    def add_edge(self, body, p0, p1, thickness=0.1, *, friction=0.2, restitution=0.0, layer=0, category=1,
                 mask=0xFFFF, group=0):
        """A terrain segment as a thin polygon quad (shapes.edge_quad)."""
        v, n = shapes.edge_quad(p0, p1, thickness)
        return self._add_fixture(body, shapes.POLYGON, v, n, self.settings.polygon_radius, friction, restitution,
                                 False, layer, category, mask, group, centroid=shapes.centroid_raw(v))

    def _add_edge_shape(self, body, v, flags, friction, restitution, layer, category, mask, group):
        if self.bodies[body].type != STATIC:
            raise ValueError("edge and chain shapes go on static bodies only (they are terrain)")
        return self._add_fixture(body, shapes.EDGE, v, np.zeros((4, 2), F32), self.settings.polygon_radius,
                                 friction, restitution, False, layer, category, mask, group, edge_flags=flags,
                                 count=2)

    def add_segment(self, body, v1, v2, v0=None, v3=None, *, friction=0.2, restitution=0.0, layer=0, category=1,
                    mask=0xFFFF, group=0):
        """A native b2EdgeShape from v1 to v2 with optional ghost vertices v0 (before v1) and v3 (after v2)."""
        v, flags = shapes.edge_shape(v1, v2, v0, v3)
        return self._add_edge_shape(body, v, flags, friction, restitution, layer, category, mask, group)

    def add_chain(self, body, points, loop=False, prev_vertex=None, next_vertex=None, *, friction=0.2,
                  restitution=0.0, layer=0, category=1, mask=0xFFFF, group=0):
        """A native b2ChainShape as its child edges, one fixture each in child order (shapes.chain_edges).
        Returns the fixture ids."""
        return [self._add_edge_shape(body, v, flags, friction, restitution, layer, category, mask, group)
                for v, flags in shapes.chain_edges(points, loop, prev_vertex, next_vertex)]

    # ---- joints (anchors in each body's frame, angles in radians)

    def _joint(self, kind, body_a, body_b, anchor_a, anchor_b, reference_angle, collide, axis=(1, 0),
               limits=None, motor_speed=0.0, max_motor=0.0, enable_motor=False, frequency=0.0, damping=0.0):
        lo, hi = (0.0, 0.0) if limits is None else limits
        self.joints.append(JointRecord(
            type=kind, body_a=body_a, body_b=body_b, anchor_a=anchor_a, anchor_b=anchor_b,
            reference_angle=reference_angle, axis=axis, enable_limit=limits is not None, lower=lo, upper=hi,
            motor_speed=motor_speed, max_motor=max_motor, enable_motor=enable_motor, frequency=frequency,
            damping=damping, collide_connected=collide))
        return len(self.joints) - 1

    def add_revolute(self, body_a, body_b, anchor_a=(0, 0), anchor_b=(0, 0), reference_angle=0.0, *,
                     limits=None, motor_speed=0.0, max_motor_torque=0.0, enable_motor=False, collide=False):
        return self._joint(REVOLUTE, body_a, body_b, anchor_a, anchor_b, reference_angle, collide, limits=limits,
                           motor_speed=motor_speed, max_motor=max_motor_torque, enable_motor=enable_motor)

    def add_prismatic(self, body_a, body_b, anchor_a=(0, 0), anchor_b=(0, 0), axis=(1, 0), reference_angle=0.0, *,
                      limits=None, motor_speed=0.0, max_motor_force=0.0, enable_motor=False, collide=False):
        return self._joint(PRISMATIC, body_a, body_b, anchor_a, anchor_b, reference_angle, collide, axis=axis,
                           limits=limits, motor_speed=motor_speed, max_motor=max_motor_force,
                           enable_motor=enable_motor)

    def add_weld(self, body_a, body_b, anchor_a=(0, 0), anchor_b=(0, 0), reference_angle=0.0, *, frequency=0.0,
                 damping=0.0, collide=False):
        return self._joint(WELD, body_a, body_b, anchor_a, anchor_b, reference_angle, collide, frequency=frequency,
                           damping=damping)

    # ---- build

    def candidate_pairs(self):
        """Every fixture pair that can ever make a contact, in b2BroadPhase::UpdatePairs order (ascending lower
        fixture, then higher), as an (P, 2) int32 array of (fixture A, fixture B) in b2Contact::Create's order: an
        edge before any other shape, a polygon before a circle, else the lower index first (world.py:308-329 and
        b2Contact's registry for edges). Left out for good: two fixtures of one body, a sensor, two static bodies,
        bodies joined with collideConnected false, the contact filter, and two edges."""
        fx = self.fixtures
        F = len(fx)
        if F == 0:
            return np.zeros((0, 2), I32)
        body = np.array([f.body for f in fx], np.int64)
        kind = np.array([f.shape_type for f in fx], np.int64)
        sensor = np.array([f.sensor for f in fx], bool)
        static = np.array([self.bodies[b].type == STATIC for b in body], bool)
        joined = np.zeros((len(self.bodies),) * 2, bool)
        for j in self.joints:
            if not j.collide_connected:
                joined[j.body_a, j.body_b] = joined[j.body_b, j.body_a] = True
        out = []
        for r0 in range(0, F, 512):  # row blocks bound the (rows, F) temporaries
            rows = slice(r0, min(r0 + 512, F))
            ok = _collide_filter(fx, self.layer_masks, rows)
            ok &= body[rows, None] != body[None, :]
            ok &= ~(sensor[rows, None] | sensor[None, :])
            ok &= ~(static[rows, None] & static[None, :])
            ok &= ~joined[body[rows, None], body[None, :]]
            ok &= ~((kind[rows, None] == shapes.EDGE) & (kind[None, :] == shapes.EDGE))
            ok &= np.arange(r0, rows.stop)[:, None] < np.arange(F)[None, :]  # each pair once, lower index first
            lo, hi = np.nonzero(ok)  # row-major: ascending lower index, then higher
            lo = lo + r0
            swap = ((kind[lo] == shapes.CIRCLE) & (kind[hi] == shapes.POLYGON)) | \
                   ((kind[hi] == shapes.EDGE) & (kind[lo] != shapes.EDGE))
            out.append(np.stack([np.where(swap, hi, lo), np.where(swap, lo, hi)], axis=1))
        return np.concatenate(out).astype(I32)

    def build(self, contact_capacity=16):
        """(Model, State) as numpy arrays without a batch axis: fat AABBs as b2BroadPhase::CreateProxy gives them,
        an empty contact table of `contact_capacity` slots and new_fixture set, as after CreateFixture
        (world.py:331-386)."""
        bodies, fixtures, joints = self.bodies, self.fixtures, self.joints
        B, F, J = len(bodies), len(fixtures), len(joints)

        def col(records, pick, dtype, tail=()):
            return np.array([pick(r) for r in records], dtype).reshape((len(records),) + tail)

        pairs = self.candidate_pairs()
        centers = col(bodies, lambda b: b.center, F32, (2,))
        bd = Bodies(
            type=col(bodies, lambda b: b.type, I32), active=col(bodies, lambda b: b.active, bool),
            awake=col(bodies, lambda b: b.awake, bool), allow_sleep=col(bodies, lambda b: b.allow_sleep, bool),
            bullet=col(bodies, lambda b: b.bullet, bool), continuous=col(bodies, lambda b: b.continuous, bool),
            sleep_time=np.zeros(B, F32), xf_p=col(bodies, lambda b: b.origin, F32, (2,)),
            xf_q=col(bodies, lambda b: b.rot, F32, (2,)), local_center=col(bodies, lambda b: b.local_center, F32, (2,)),
            c0=centers.copy(), c=centers, a0=col(bodies, lambda b: b.angle, F32), a=col(bodies, lambda b: b.angle, F32),
            v=col(bodies, lambda b: b.v, F32, (2,)), w=col(bodies, lambda b: b.w, F32), force=np.zeros((B, 2), F32),
            torque=np.zeros(B, F32), mass=col(bodies, lambda b: b.mass, F32),
            inv_mass=col(bodies, lambda b: b.inv_mass, F32), inertia=col(bodies, lambda b: b.inertia, F32),
            inv_inertia=col(bodies, lambda b: b.inv_inertia, F32),
            linear_damping=col(bodies, lambda b: b.linear_damping, F32),
            angular_damping=col(bodies, lambda b: b.angular_damping, F32),
            gravity_scale=col(bodies, lambda b: b.gravity_scale, F32))
        # prismatic axis: normalized twice, as the reference oracle does (its builder, then the b2PrismaticJoint
        # constructor; world.py:352-356); the y axis is b2Cross(1, x axis) = (-x.y, x.x)
        ax = np.array([shapes.normalize_host(*shapes.normalize_host(j.axis[0], j.axis[1])) for j in joints],
                      F32).reshape(J, 2)
        model = Model(
            fixture_body=col(fixtures, lambda f: f.body, I32), shape_type=col(fixtures, lambda f: f.shape_type, I32),
            radius=col(fixtures, lambda f: f.radius, F32), count=col(fixtures, lambda f: f.count, I32),
            verts=col(fixtures, lambda f: f.verts, F32, (MAX_POLYGON_VERTICES, 2)),
            normals=col(fixtures, lambda f: f.normals, F32, (MAX_POLYGON_VERTICES, 2)),
            joint_type=col(joints, lambda j: j.type, I32), joint_a=col(joints, lambda j: j.body_a, I32),
            joint_b=col(joints, lambda j: j.body_b, I32), local_anchor_a=col(joints, lambda j: j.anchor_a, F32, (2,)),
            local_anchor_b=col(joints, lambda j: j.anchor_b, F32, (2,)), local_axis_a=ax,
            local_yaxis_a=np.stack([-ax[:, 1], ax[:, 0]], axis=1).reshape(J, 2),
            reference_angle=col(joints, lambda j: j.reference_angle, F32),
            pair_a=np.ascontiguousarray(pairs[:, 0]), pair_b=np.ascontiguousarray(pairs[:, 1]),
            toi_bodies=bd.bullet | bd.continuous, body_type=bd.type.copy(),
            centroid=col(fixtures, lambda f: f.centroid, F32, (2,)), edge_flags=col(fixtures, lambda f: f.edge_flags, I32))
        owner = model.fixture_body
        fat = fixture_fat_host(model, bd.xf_p[owner, 0], bd.xf_p[owner, 1], bd.xf_q[owner, 0], bd.xf_q[owner, 1])
        fxs = Fixtures(friction=col(fixtures, lambda f: f.friction, F32),
                       restitution=col(fixtures, lambda f: f.restitution, F32), fat=fat)
        jn = Joints(
            enable_motor=col(joints, lambda j: j.enable_motor, bool), motor_speed=col(joints, lambda j: j.motor_speed, F32),
            max_motor=col(joints, lambda j: j.max_motor, F32), enable_limit=col(joints, lambda j: j.enable_limit, bool),
            lower=col(joints, lambda j: j.lower, F32), upper=col(joints, lambda j: j.upper, F32),
            frequency=col(joints, lambda j: j.frequency, F32), damping=col(joints, lambda j: j.damping, F32),
            impulse=np.zeros((J, 3), F32), motor_impulse=np.zeros(J, F32), limit_state=np.zeros(J, I32),
            lower_impulse=np.zeros(J, F32), upper_impulse=np.zeros(J, F32))
        state = State(bodies=bd, fixtures=fxs, joints=jn, contacts=empty_contacts(contact_capacity),
                      gravity=np.array(self.settings.gravity, F32), inv_dt0=np.asarray(F32(0)),
                      next_key=np.asarray(I32(0)), new_fixture=np.asarray(F > 0), overflow=np.asarray(I32(0)),
                      toi=empty_toi(B, contact_capacity))
        return model, state


def fixture_fat_host(model, px, py, c, s):
    """b2Shape::ComputeAABB at the given transforms, then the b2_aabbExtension margin (shapes.py:118-146), in
    float32 with C's operation order. A chain child's box has no skin radius (b2ChainShape::ComputeAABB)."""
    F = model.fixture_body.shape[0]
    out = np.zeros((F, 4), F32)
    e = F32(0.1)
    for f in range(F):
        r = model.radius[f]
        if model.shape_type[f] == shapes.CIRCLE:
            vx, vy = model.verts[f, 0]
            rx = F32(F32(c[f] * vx) - F32(s[f] * vy))
            ry = F32(F32(s[f] * vx) + F32(c[f] * vy))
            x, y = F32(px[f] + rx), F32(py[f] + ry)
            lx, ly, ux, uy = F32(x - r), F32(y - r), F32(x + r), F32(y + r)
        else:
            n = int(model.count[f])
            if model.edge_flags is not None and model.edge_flags[f] & shapes.EDGE_CHAIN:
                r = F32(0)
            vx, vy = model.verts[f, :n, 0], model.verts[f, :n, 1]
            wx = ((c[f] * vx).astype(F32) - (s[f] * vy).astype(F32)).astype(F32) + F32(px[f])
            wy = ((s[f] * vx).astype(F32) + (c[f] * vy).astype(F32)).astype(F32) + F32(py[f])
            lx, ly = F32(F32(wx.min()) - r), F32(F32(wy.min()) - r)
            ux, uy = F32(F32(wx.max()) + r), F32(F32(wy.max()) + r)
        out[f] = (F32(lx - e), F32(ly - e), F32(ux + e), F32(uy + e))
    return out


def _blank(group, dims, fill):
    """The leaves of one State group (in LEAVES order) for capacities dims = (B, R, J, C), zero except the given fill
    values by leaf name."""
    return [np.full(leaf_shape(inner, dims), fill.get(name, 0), dt)
            for g, name, dt, inner in LEAVES if g == group]


def empty_contacts(C):
    """An empty contact table of C slots: every slot free (pair -1), everything else zero."""
    return Contacts(*_blank("contacts", (0, 0, 0, C), {"pair": -1}))


def empty_toi(B, C):
    """ContactTOI as SolveTOI resets it (world.py:157-161): toi 1 and enabled, everything else zero or false."""
    return ContactTOI(*_blank("toi", (B, 0, 0, C), {"toi": 1, "enabled": True}))


# ---------------------------------------------------------------- compact fixture layout (world.py:400-563)

def is_compact(model, state):
    return model.fixture_slot is not None and state.fixtures.fat.shape[-2] != model.fixture_body.shape[-1]


def compact_model(model, state):
    """The Model with the compact fixture tables (world.py:437-472), from a full-layout State with any leading batch
    axes: static bodies' fixtures keep their fat AABB, friction and restitution once in the Model (fixture_slot -1),
    the others get State rows in fixture order. Requires body types and the static fixtures' rows to be the same in
    every world (a step never changes them). A Model that already has the tables is returned as it is."""
    if model.fixture_slot is not None:
        return model
    types = np.asarray(state.bodies.type)
    types = types.reshape(-1, types.shape[-1])
    shared = types[0]
    if (types != shared).any():
        raise ValueError("compact_model: the worlds' body types differ, so static fixtures cannot be shared")
    owner = np.asarray(model.fixture_body)
    F = owner.shape[0]
    on_static = shared[owner] == STATIC
    n = len(types)
    per_world = {"fat": np.asarray(state.fixtures.fat).reshape(n, F, 4),
                 "friction": np.asarray(state.fixtures.friction).reshape(n, F),
                 "restitution": np.asarray(state.fixtures.restitution).reshape(n, F)}
    tables = {}
    for name, rows in per_world.items():
        if (rows[:, on_static] != rows[:1, on_static]).any():
            raise ValueError(f"compact_model: a static fixture's {name} differs between worlds")
        table = np.zeros_like(rows[0])
        table[on_static] = rows[0][on_static]
        tables[name] = table
    moving = np.flatnonzero(~on_static).astype(I32)
    slot = np.full(F, -1, I32)
    slot[moving] = np.arange(moving.size, dtype=I32)
    return model._replace(fixture_slot=slot, slot_fixture=moving, static_fat=tables["fat"],
                          static_friction=tables["friction"], static_restitution=tables["restitution"],
                          body_type=shared.copy())


def compact_state(model, state):
    """A full-layout State (any leading batch axes) in the compact layout of `model` (world.py:524-549)."""
    if model.fixture_slot is None or is_compact(model, state):
        return state
    rows = np.asarray(model.slot_fixture)
    fx = state.fixtures
    return state._replace(fixtures=Fixtures(friction=np.take(fx.friction, rows, axis=-1),
                                            restitution=np.take(fx.restitution, rows, axis=-1),
                                            fat=np.take(fx.fat, rows, axis=-2)))


def expand_state(model, state):
    """The full-layout State of a compact one (static rows from the Model), numpy (world.py:551-563)."""
    if not is_compact(model, state):
        return state
    fx = state.fixtures
    rows = np.asarray(model.slot_fixture)
    lead = fx.fat.shape[:-2]
    fat = np.broadcast_to(model.static_fat, lead + model.static_fat.shape).copy()
    fr = np.broadcast_to(model.static_friction, lead + model.static_friction.shape).copy()
    rs = np.broadcast_to(model.static_restitution, lead + model.static_restitution.shape).copy()
    fat[..., rows, :] = fx.fat
    fr[..., rows] = fx.friction
    rs[..., rows] = fx.restitution
    return state._replace(fixtures=Fixtures(friction=fr, restitution=rs, fat=fat))


def batch(state, n):
    """n copies of a single-world State stacked on a leading axis (numpy)."""
    return from_leaves([np.repeat(np.asarray(x)[None], n, axis=0) for x in leaves(state)])
