"""World layout: the shared Model and the per-world State pytrees, the host builder WorldDef, and the compact fixture
layout (mirror of goi_jax/box2d/world.py:30-563; same field names, shapes, dtypes and creation-order rules).

Host values are numpy arrays (a State built here has no batch axis). `layout.py` moves a batch of States to the GPU
as torch tensors in the kernels' worlds-minor layout and back.

Indices follow creation order, which Box2D uses for its orderings (world.py:7-11): body i is the i-th created (the
body list is newest first, so islands are seeded from the highest index); fixture i gets broad-phase proxy id order i;
joint i is the i-th created (each body's joint list is newest first).
"""
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


def _filter_ok(fa, fb, masks):
    """Filter::ShouldCollide (world.py:177-183): the layer matrix when given, else b2ContactFilter's groups."""
    if masks is not None:
        return bool((int(masks[fa["layer"]]) & 0xFFFFFFFF) >> fb["layer"] & 1)
    if fa["group"] == fb["group"] and fa["group"] != 0:
        return fa["group"] > 0
    return (fa["mask"] & fb["category"]) != 0 and (fa["category"] & fb["mask"]) != 0


class WorldDef:
    """Host-side builder (world.py:186-387): same methods, defaults and float32 arithmetic."""

    def __init__(self, settings=None, layer_masks=None):
        self.settings = settings or Settings()
        self.layer_masks = layer_masks
        self.bodies, self.fixtures, self.joints = [], [], []

    def add_body(self, type=DYNAMIC, position=(0, 0), angle=0.0, velocity=(0, 0), angular_velocity=0.0, *,
                 mass=None, center=(0, 0), inertia=0.0, exact_inertia=True, linear_damping=0.0,
                 angular_damping=0.0, gravity_scale=1.0, fixed_rotation=False, bullet=False, continuous=False,
                 awake=True, allow_sleep=True, active=True):
        a = F32(angle)
        s, c = shapes.host_sin_cos(a)
        b = dict(type=type, active=active, awake=awake, allow_sleep=allow_sleep, bullet=bullet,
                 continuous=continuous, fixed_rotation=fixed_rotation, p=np.array(position, F32), q=(c, s),
                 local_center=np.zeros(2, F32), c=np.array(position, F32), a=a, v=np.zeros(2, F32), w=F32(0),
                 mass=F32(1 if type == DYNAMIC else 0), inv_mass=F32(1 if type == DYNAMIC else 0),
                 inertia=F32(0), inv_inertia=F32(0), linear_damping=F32(linear_damping),
                 angular_damping=F32(angular_damping), gravity_scale=F32(gravity_scale), sleep_time=F32(0))
        self.bodies.append(b)
        bid = len(self.bodies) - 1
        if mass is not None:
            self.set_mass(bid, mass, center, inertia, exact_inertia)
        if type != STATIC and (velocity[0] or velocity[1] or angular_velocity):
            b["v"], b["w"] = np.array(velocity, F32), F32(angular_velocity)
            b["awake"] = True
            if not awake:  # the reference builder re-sleeps it: SetAwake(false) zeroes the velocity
                b["awake"], b["v"], b["w"] = False, np.zeros(2, F32), F32(0)
        return bid

    def set_mass(self, body, mass, center=(0, 0), inertia=0.0, exact=True):
        """goi_b2_body_set_mass (world.py:220-244): b2MassData.I = I_com + m |c|^2, b2Body::SetMassData, then
        (exact) the given I_com verbatim."""
        b = self.bodies[body]
        if b["type"] != DYNAMIC:
            return
        mass, cx, cy, icom = F32(mass), F32(center[0]), F32(center[1]), F32(inertia)
        cc = F32(F32(cx * cx) + F32(cy * cy))
        md_i = F32(icom + F32(mass * cc))
        m = mass if mass > 0 else F32(1)
        b["mass"], b["inv_mass"] = m, F32(F32(1) / m)
        b["inertia"], b["inv_inertia"] = F32(0), F32(0)
        if md_i > 0 and not b["fixed_rotation"]:
            b["inertia"] = F32(md_i - F32(m * cc))
            b["inv_inertia"] = F32(F32(1) / b["inertia"])
        if exact and b["inertia"] > 0:
            b["inertia"], b["inv_inertia"] = icom, F32(F32(1) / icom)
        old = b["c"].copy()
        c, s = b["q"]
        px, py = b["p"]
        b["local_center"] = np.array([cx, cy], F32)
        b["c"] = np.array([F32(F32(F32(c * cx) - F32(s * cy)) + px), F32(F32(F32(s * cx) + F32(c * cy)) + py)], F32)
        dx, dy = F32(b["c"][0] - old[0]), F32(b["c"][1] - old[1])
        w = b["w"]
        b["v"] = np.array([F32(b["v"][0] + F32(-w * dy)), F32(b["v"][1] + F32(w * dx))], F32)

    def _add_fixture(self, body, shape_type, verts, normals, radius, friction, restitution, sensor, layer,
                     category, mask, group, centroid=(0.0, 0.0), edge_flags=0, count=None):
        vv, nn = shapes.pad(verts, normals)
        self.fixtures.append(dict(body=body, shape_type=shape_type, verts=vv, normals=nn,
                                  count=len(verts) if count is None else count, radius=F32(radius),
                                  friction=F32(friction), restitution=F32(restitution), sensor=bool(sensor),
                                  layer=int(layer) & 31, category=category, mask=mask, group=group,
                                  centroid=np.asarray(centroid, F32), edge_flags=int(edge_flags)))
        return len(self.fixtures) - 1

    def add_polygon(self, body, vertices, radius=None, raw=False, *, friction=0.2, restitution=0.0, density=0.0,
                    sensor=False, layer=0, category=1, mask=0xFFFF, group=0):
        v, n = shapes.polygon_raw(vertices) if raw else shapes.polygon_set(vertices, self.settings.linear_slop)
        r = self.settings.polygon_radius if radius is None else radius
        c = shapes.centroid_raw(v) if raw else shapes.centroid_set(v)
        return self._add_fixture(body, shapes.POLYGON, v, n, r, friction, restitution, sensor, layer, category,
                                 mask, group, centroid=c)

    def add_box(self, body, half_extents, center=(0, 0), angle=0.0, radius=None, *, friction=0.2, restitution=0.0,
                density=0.0, sensor=False, layer=0, category=1, mask=0xFFFF, group=0):
        v, n = shapes.box(half_extents[0], half_extents[1], center, angle)
        r = self.settings.polygon_radius if radius is None else radius
        return self._add_fixture(body, shapes.POLYGON, v, n, r, friction, restitution, sensor, layer, category,
                                 mask, group, centroid=center)

    def add_circle(self, body, radius, center=(0, 0), *, friction=0.2, restitution=0.0, density=0.0, sensor=False,
                   layer=0, category=1, mask=0xFFFF, group=0):
        v = np.array([center], F32)
        return self._add_fixture(body, shapes.CIRCLE, v, np.zeros((1, 2), F32), radius, friction, restitution,
                                 sensor, layer, category, mask, group)

    def add_edge(self, body, p0, p1, thickness=0.1, *, friction=0.2, restitution=0.0, layer=0, category=1,
                 mask=0xFFFF, group=0):
        """A terrain edge segment as a thin polygon quad (shapes.edge_quad)."""
        v, n = shapes.edge_quad(p0, p1, thickness)
        return self._add_fixture(body, shapes.POLYGON, v, n, self.settings.polygon_radius, friction, restitution,
                                 False, layer, category, mask, group, centroid=shapes.centroid_raw(v))

    def _add_edge_shape(self, body, v, flags, friction, restitution, layer, category, mask, group):
        if self.bodies[body]["type"] != STATIC:
            raise ValueError("edge shapes belong to static bodies (the terrain)")
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

    def _add_joint(self, **j):
        self.joints.append(j)
        return len(self.joints) - 1

    def add_revolute(self, body_a, body_b, anchor_a=(0, 0), anchor_b=(0, 0), reference_angle=0.0, *,
                     limits=None, motor_speed=0.0, max_motor_torque=0.0, enable_motor=False, collide=False):
        lo, hi = limits if limits is not None else (0.0, 0.0)
        return self._add_joint(type=REVOLUTE, a=body_a, b=body_b, la=anchor_a, lb=anchor_b, ref=reference_angle,
                               axis=(1, 0), enable_limit=limits is not None, lower=lo, upper=hi,
                               motor_speed=motor_speed, max_motor=max_motor_torque, enable_motor=enable_motor,
                               frequency=0.0, damping=0.0, collide=collide)

    def add_prismatic(self, body_a, body_b, anchor_a=(0, 0), anchor_b=(0, 0), axis=(1, 0), reference_angle=0.0, *,
                      limits=None, motor_speed=0.0, max_motor_force=0.0, enable_motor=False, collide=False):
        lo, hi = limits if limits is not None else (0.0, 0.0)
        return self._add_joint(type=PRISMATIC, a=body_a, b=body_b, la=anchor_a, lb=anchor_b, ref=reference_angle,
                               axis=axis, enable_limit=limits is not None, lower=lo, upper=hi,
                               motor_speed=motor_speed, max_motor=max_motor_force, enable_motor=enable_motor,
                               frequency=0.0, damping=0.0, collide=collide)

    def add_weld(self, body_a, body_b, anchor_a=(0, 0), anchor_b=(0, 0), reference_angle=0.0, *, frequency=0.0,
                 damping=0.0, collide=False):
        return self._add_joint(type=WELD, a=body_a, b=body_b, la=anchor_a, lb=anchor_b, ref=reference_angle,
                               axis=(1, 0), enable_limit=False, lower=0.0, upper=0.0, motor_speed=0.0,
                               max_motor=0.0, enable_motor=False, frequency=frequency, damping=damping,
                               collide=collide)

    def candidate_pairs(self):
        """b2BroadPhase::UpdatePairs order with b2Contact::Create's swap (world.py:308-329): a polygon before a
        circle, an edge before either (b2Contact's registry); no contact between two edges."""
        no_collide = {frozenset((j["a"], j["b"])) for j in self.joints if not j["collide"]}
        out = []
        fs, bs = self.fixtures, self.bodies
        static_body = [b["type"] == STATIC for b in bs]
        for i, fi in enumerate(fs):
            for k in range(i + 1, len(fs)):
                fk = fs[k]
                if fi["body"] == fk["body"] or fi["sensor"] or fk["sensor"]:
                    continue
                if static_body[fi["body"]] and static_body[fk["body"]]:
                    continue
                if frozenset((fi["body"], fk["body"])) in no_collide or not _filter_ok(fi, fk, self.layer_masks):
                    continue
                ti, tk = fi["shape_type"], fk["shape_type"]
                if ti == shapes.EDGE and tk == shapes.EDGE:
                    continue
                if (ti == shapes.CIRCLE and tk == shapes.POLYGON) or (tk == shapes.EDGE and ti != shapes.EDGE):
                    out.append((k, i))
                else:
                    out.append((i, k))
        return out

    def build(self, contact_capacity=16):
        """(Model, State) as numpy (no batch axis); fat AABBs as b2BroadPhase::CreateProxy gives them; contacts start
        empty with new_fixture set (world.py:331-386)."""
        B, F, J, C = len(self.bodies), len(self.fixtures), len(self.joints), contact_capacity
        bs, fs, js = self.bodies, self.fixtures, self.joints
        pairs = self.candidate_pairs()
        arr = lambda key, dt=F32: np.array([x[key] for x in bs], dt)  # noqa: E731
        q = np.array([b["q"] for b in bs], F32).reshape(B, 2)
        bodies = Bodies(
            type=arr("type", I32), active=arr("active", bool), awake=arr("awake", bool),
            allow_sleep=arr("allow_sleep", bool), bullet=arr("bullet", bool), continuous=arr("continuous", bool),
            sleep_time=arr("sleep_time"), xf_p=np.array([b["p"] for b in bs], F32).reshape(B, 2), xf_q=q,
            local_center=np.array([b["local_center"] for b in bs], F32).reshape(B, 2),
            c0=np.array([b["c"] for b in bs], F32).reshape(B, 2), c=np.array([b["c"] for b in bs], F32).reshape(B, 2),
            a0=arr("a"), a=arr("a"), v=np.array([b["v"] for b in bs], F32).reshape(B, 2), w=arr("w"),
            force=np.zeros((B, 2), F32), torque=np.zeros(B, F32), mass=arr("mass"), inv_mass=arr("inv_mass"),
            inertia=arr("inertia"), inv_inertia=arr("inv_inertia"), linear_damping=arr("linear_damping"),
            angular_damping=arr("angular_damping"), gravity_scale=arr("gravity_scale"))
        farr = lambda key, dt=F32, shape=(): np.array([f[key] for f in fs], dt).reshape((F,) + shape)  # noqa: E731
        jarr = lambda key, dt=F32, shape=(): np.array([j[key] for j in js], dt).reshape((J,) + shape)  # noqa: E731
        axes = []
        for j in js:  # prismatic axis normalized twice, as the reference oracle does (world.py:352-356)
            x, y = shapes.normalize_host(*shapes.normalize_host(F32(j["axis"][0]), F32(j["axis"][1])))
            axes.append(((x, y), (F32(-F32(1) * y), F32(F32(1) * x))))
        model = Model(
            fixture_body=farr("body", I32), shape_type=farr("shape_type", I32), radius=farr("radius"),
            count=farr("count", I32), verts=farr("verts", F32, (MAX_POLYGON_VERTICES, 2)),
            normals=farr("normals", F32, (MAX_POLYGON_VERTICES, 2)),
            joint_type=jarr("type", I32), joint_a=jarr("a", I32), joint_b=jarr("b", I32),
            local_anchor_a=jarr("la", F32, (2,)), local_anchor_b=jarr("lb", F32, (2,)),
            local_axis_a=np.array([a[0] for a in axes], F32).reshape(J, 2),
            local_yaxis_a=np.array([a[1] for a in axes], F32).reshape(J, 2),
            reference_angle=jarr("ref"),
            pair_a=np.array([p[0] for p in pairs], I32).reshape(-1),
            pair_b=np.array([p[1] for p in pairs], I32).reshape(-1),
            toi_bodies=bodies.bullet | bodies.continuous, body_type=bodies.type.copy(),
            centroid=farr("centroid", F32, (2,)), edge_flags=farr("edge_flags", I32))
        fb = model.fixture_body
        fat = fixture_fat_host(model, bodies.xf_p[fb, 0], bodies.xf_p[fb, 1], q[fb, 0], q[fb, 1])
        fixtures = Fixtures(friction=farr("friction"), restitution=farr("restitution"), fat=fat)
        joints = Joints(
            enable_motor=jarr("enable_motor", bool), motor_speed=jarr("motor_speed"), max_motor=jarr("max_motor"),
            enable_limit=jarr("enable_limit", bool), lower=jarr("lower"), upper=jarr("upper"),
            frequency=jarr("frequency"), damping=jarr("damping"), impulse=np.zeros((J, 3), F32),
            motor_impulse=np.zeros(J, F32), limit_state=np.zeros(J, I32), lower_impulse=np.zeros(J, F32),
            upper_impulse=np.zeros(J, F32))
        state = State(bodies=bodies, fixtures=fixtures, joints=joints, contacts=empty_contacts(C),
                      gravity=np.array(self.settings.gravity, F32), inv_dt0=np.asarray(F32(0)),
                      next_key=np.asarray(I32(0)), new_fixture=np.asarray(len(fs) > 0),
                      overflow=np.asarray(I32(0)), toi=empty_toi(B, C))
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


def empty_contacts(C):
    z = lambda *s: np.zeros((C,) + s, F32)  # noqa: E731
    zi = lambda *s: np.zeros((C,) + s, I32)  # noqa: E731
    return Contacts(pair=np.full((C,), -1, I32), fa=zi(), fb=zi(), key=zi(), touching=np.zeros((C,), bool),
                    mtype=zi(), count=zi(), local_normal=z(2), local_point=z(2), point_local=z(2, 2),
                    point_id=zi(2), normal_impulse=z(2), tangent_impulse=z(2), friction=z(), restitution=z(),
                    tangent_speed=z())


def empty_toi(B, C):
    """ContactTOI as SolveTOI resets it (world.py:157-161)."""
    return ContactTOI(alpha0=np.zeros((B,), F32), count=np.zeros((C,), I32), toi=np.ones((C,), F32),
                      flag=np.zeros((C,), bool), enabled=np.ones((C,), bool), solved=np.zeros((C,), bool),
                      normal_impulse=np.zeros((C, 2), F32), tangent_impulse=np.zeros((C, 2), F32),
                      events=np.asarray(I32(0)))


# ---------------------------------------------------------------- compact fixture layout (world.py:400-563)

def is_compact(model, state):
    return model.fixture_slot is not None and state.fixtures.fat.shape[-2] != model.fixture_body.shape[-1]


def compact_model(model, state):
    """The Model with the compact fixture tables (world.py:437-472) from a full-layout State (any leading batch
    axes) whose static-body fixture rows agree in every world. Idempotent."""
    if model.fixture_slot is not None:
        return model
    btype = np.asarray(state.bodies.type).reshape(-1, np.asarray(state.bodies.type).shape[-1])
    if not (btype == btype[0]).all():
        raise ValueError("compact_model: body types differ between worlds")
    fb = np.asarray(model.fixture_body)
    static = btype[0][fb] == STATIC
    F = fb.shape[0]
    fat = np.asarray(state.fixtures.fat).reshape(-1, F, 4)
    fr = np.asarray(state.fixtures.friction).reshape(-1, F)
    rs = np.asarray(state.fixtures.restitution).reshape(-1, F)
    for name, a in (("fat", fat), ("friction", fr), ("restitution", rs)):
        if not (a[:, static] == a[:1, static]).all():
            raise ValueError(f"compact_model: static fixtures' {name} differs between worlds")
    rows = np.nonzero(~static)[0].astype(I32)
    slot = np.full(F, -1, I32)
    slot[rows] = np.arange(len(rows), dtype=I32)
    keep = lambda a: np.where(static.reshape((F,) + (1,) * (a.ndim - 1)), a, 0).astype(a.dtype)  # noqa: E731
    return model._replace(fixture_slot=slot, slot_fixture=rows, static_fat=keep(fat[0]),
                          static_friction=keep(fr[0]), static_restitution=keep(rs[0]), body_type=btype[0].copy())


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
