"""Seeded synthetic worlds: the static terrain (edge chain + convex rocks), the 4-body character rig with its
action-driven motor, the five benchmark configurations, and small deterministic test scenes.

Terrain edges are thin polygon quads (shapes.edge_quad) by default: the reference has no edge or chain shapes
(goi_jax/box2d/shapes.py:13), so every contact stays on reference-defined polygon code. `edges="native"` builds the
same chain as a b2ChainShape (native edges with ghost vertices) instead.

Fixture order (= broad-phase proxy order): the terrain body's fixtures first (edges, then rocks), then the rig bodies'
(pot, torso, handle, head), then any extra boxes. Candidate index of (terrain fixture t, rig fixture d) is therefore
t * n_dyn + d, followed by the non-jointed dynamic pairs.
"""
import math
from dataclasses import dataclass

import numpy as np

from . import shapes
from . import world as wd
from .settings import Settings

F32, I32 = np.float32, np.int32

# rig geometry (half extents, metres) and layout in the rig frame (pot centre at the origin)
POT_R = 0.5
TORSO = (0.2, 0.3)
HANDLE = (0.8, 0.03)
HEAD = (0.15, 0.075)
RIG_LOCAL = {  # body origin in the rig frame
    "pot": (0.0, 0.0),
    "torso": (0.0, 0.5),
    "handle": (0.8, 0.5),
    "head": (1.75, 0.5),
}
MOTOR_JOINT = 1  # torso-handle revolute: the action-driven motor
MOTOR_GAIN = F32(10.0)  # motor_speed = gain * action_x (rad/s)
MOTOR_TORQUE = F32(40.0)  # maxMotorTorque = torque * |action| (N m)
BOX_STACKS = 3  # the extra boxes of the large-island configuration stand in this many stacks
STACK_LIFT = 2.6  # height of the stacks' base above the pot centre (m)
RIG_BODIES = 4


@dataclass(frozen=True)
class Config:
    name: str
    worlds: int
    n_edges: int
    n_rocks: int
    seed: int
    steps: int
    capacity: int = 40
    v_sigma: float = 0.0
    head_w: float = 0.0
    boxes: int = 0
    dt: float = 0.02
    collide_only: bool = False


CONFIGS = {
    1: Config("rig-1world-cpu", 1, 256, 64, 0, 500),
    2: Config("collide-4096", 4096, 256, 64, 1, 1, collide_only=True),
    3: Config("fullstep-4096", 4096, 1024, 256, 2, 200, v_sigma=1.0),
    4: Config("toi-16384", 16384, 1024, 256, 2, 100, v_sigma=25.0, head_w=60.0),
    5: Config("island-65536", 65536, 2048, 512, 4, 300, capacity=128, boxes=12),
}


def settings_for(cfg=None):
    """Stock Box2D settings with g = -9.81, 8 / 3 iterations, continuous physics on (stock TOI pair rule)."""
    return Settings.stock(gravity=(0.0, -9.81), continuous_physics=True)


# ---------------------------------------------------------------- terrain

def _convex_polygon(rng, radius, centre):
    """A strictly convex CCW polygon at `centre`, convex after the float32 translation too (far from the origin the
    rounding can merge close vertices; such draws are redrawn)."""
    while True:
        n = int(rng.integers(3, 9))
        ang = np.sort(rng.uniform(0.0, 2.0 * np.pi, n))
        v = np.stack([radius * np.cos(ang), radius * np.sin(ang)], 1).astype(F32)
        try:
            shapes.polygon_raw(v)
            return shapes.polygon_raw((v + np.asarray(centre, F32)).astype(F32))
        except ValueError:
            continue


def terrain(seed, n_edges, n_rocks):
    """(chain points (n_edges + 1, 2) float64, rock list [(verts, normals)]) from a seeded generator: segment lengths
    U[0.5, 3] m, heading random walk N(0, 0.25) rad clamped to +-1.2 rad from (0, 0); rocks of 3-8 vertices at sorted
    random angles on a circle of radius U[0.3, 2] m, centred on the chain at a random x."""
    rng = np.random.default_rng(seed)
    pts = [np.zeros(2)]
    heading = 0.0
    for _ in range(n_edges):
        heading = float(np.clip(heading + rng.normal(0.0, 0.25), -1.2, 1.2))
        length = rng.uniform(0.5, 3.0)
        pts.append(pts[-1] + length * np.array([math.cos(heading), math.sin(heading)]))
    pts = np.array(pts)
    rocks = []
    for _ in range(n_rocks):
        radius = rng.uniform(0.3, 2.0)
        x = rng.uniform(pts[0, 0], pts[-1, 0])
        y = float(np.interp(x, pts[:, 0], pts[:, 1]))
        rocks.append(_convex_polygon(rng, radius, (x, y)))
    return pts, rocks


def height_at(pts, x):
    return np.interp(x, pts[:, 0], pts[:, 1])


# ---------------------------------------------------------------- rig

def _mass_props():
    """Density-1 mass and centroidal inertia of the rig bodies, float32."""
    pot_m = F32(math.pi * POT_R * POT_R)
    out = {"pot": (pot_m, F32(F32(0.5) * pot_m * F32(POT_R * POT_R)))}
    for name, (hx, hy) in (("torso", TORSO), ("handle", HANDLE), ("head", HEAD)):
        w, h = 2 * hx, 2 * hy
        m = F32(w * h)
        out[name] = (m, F32(m * F32((w * w + h * h) / 12.0)))
    return out


def add_rig(d, origin=(0.0, 10.0), friction=0.5):
    """The 4-body rig (pot circle, torso, handle, hammer head) with 3 revolute joints (pot-torso free, torso-handle
    the action-driven motor, handle-head limited to +-0.5 rad), collideConnected false. Returns the body ids."""
    mp = _mass_props()
    ox, oy = origin
    ids = {}
    for name in ("pot", "torso", "handle", "head"):
        lx, ly = RIG_LOCAL[name]
        m, inertia = mp[name]
        ids[name] = d.add_body(wd.DYNAMIC, (ox + lx, oy + ly), 0.0, mass=m, inertia=inertia)
    d.add_circle(ids["pot"], POT_R, friction=friction)
    d.add_box(ids["torso"], TORSO, friction=friction)
    d.add_box(ids["handle"], HANDLE, friction=friction)
    d.add_box(ids["head"], HEAD, friction=friction)
    d.add_revolute(ids["pot"], ids["torso"], (0.0, 0.0), (0.0, -0.5))
    d.add_revolute(ids["torso"], ids["handle"], (0.0, 0.0), (-0.8, 0.0), motor_speed=0.0,
                   max_motor_torque=float(MOTOR_TORQUE), enable_motor=True)
    d.add_revolute(ids["handle"], ids["head"], (0.8, 0.0), (-0.15, 0.0), limits=(-0.5, 0.5))
    return ids


def build_world(cfg, settings=None, edges="quad"):
    """(Model, single-world State, chain points) of a configuration: terrain body 0, rig bodies 1-4, boxes after.
    edges: "quad" (thin polygon quads) or "native" (one b2ChainShape)."""
    settings = settings or settings_for(cfg)
    pts, rocks = terrain(cfg.seed, cfg.n_edges, cfg.n_rocks)
    d = wd.WorldDef(settings)
    g = d.add_body(wd.STATIC)
    if edges == "native":
        d.add_chain(g, pts, friction=0.8)
    elif edges == "quad":
        for i in range(cfg.n_edges):
            d.add_edge(g, pts[i], pts[i + 1], friction=0.8)
    else:
        raise ValueError(f"edges must be 'quad' or 'native', not {edges!r}")
    for v, _ in rocks:
        d.add_polygon(g, v, raw=True, friction=0.8)
    x0 = 20.0
    y0 = float(height_at(pts, x0)) + 2.0
    add_rig(d, (x0, y0))
    # the boxes (sides U[0.2, 0.6] m, density U[0.5, 2]) in BOX_STACKS unrotated stacks, column j's boxes on top of
    # each other, the stacks side by side with no gap, the lowest boxes STACK_LIFT m above the pot centre (clear of
    # the rig at any angle); place_worlds keeps this layout relative to the pot without rotating it
    rng = np.random.default_rng(1000 + cfg.seed)
    sizes = [(rng.uniform(0.1, 0.3, 2), rng.uniform(0.5, 2.0)) for _ in range(cfg.boxes)]
    pitch = 2.0 * max([float(h[0]) for h, _ in sizes], default=0.0)
    top = [STACK_LIFT] * BOX_STACKS
    for i, ((hx, hy), dens) in enumerate(sizes):
        col = i % BOX_STACKS
        m = F32(dens * 4 * hx * hy)
        inertia = F32(m * F32((4 * hx * hx + 4 * hy * hy) / 12.0))
        b = d.add_body(wd.DYNAMIC, (x0 + (col - (BOX_STACKS - 1) / 2.0) * pitch, y0 + top[col] + hy),
                       mass=m, inertia=inertia)
        top[col] += 2.0 * hy
        d.add_box(b, (hx, hy), friction=0.6)
    model, state = d.build(contact_capacity=cfg.capacity)
    return model, state, pts


def _rot(a):
    s = np.array([math.sin(float(x)) for x in a.astype(np.float64)], F32)
    c = np.array([math.cos(float(x)) for x in a.astype(np.float64)], F32)
    return c, s


def fat_rows(model, state_b, rows):
    """Fat AABBs (shape AABB + b2_aabbExtension) of fixture `rows` at every world's body transforms, float32 in C
    operation order; state_b is batched. Returns (N, len(rows), 4)."""
    out = []
    e = F32(0.1)
    for f in rows:
        b = int(model.fixture_body[f])
        px, py = state_b.bodies.xf_p[:, b, 0], state_b.bodies.xf_p[:, b, 1]
        c, s = state_b.bodies.xf_q[:, b, 0], state_b.bodies.xf_q[:, b, 1]
        r = model.radius[f]
        if model.shape_type[f] == shapes.CIRCLE:
            vx, vy = model.verts[f, 0]
            x = px + ((c * vx).astype(F32) - (s * vy).astype(F32)).astype(F32)
            y = py + ((s * vx).astype(F32) + (c * vy).astype(F32)).astype(F32)
            lx, ly, ux, uy = x - r, y - r, x + r, y + r
        else:
            n = int(model.count[f])
            vx, vy = model.verts[f, :n, 0][None, :], model.verts[f, :n, 1][None, :]
            wx = ((c[:, None] * vx).astype(F32) - (s[:, None] * vy).astype(F32)).astype(F32) + px[:, None]
            wy = ((s[:, None] * vx).astype(F32) + (c[:, None] * vy).astype(F32)).astype(F32) + py[:, None]
            lx, ly = wx.min(1) - r, wy.min(1) - r
            ux, uy = wx.max(1) + r, wy.max(1) + r
        out.append(np.stack([lx - e, ly - e, ux + e, uy + e], 1).astype(F32))
    return np.stack(out, 1)


def place_worlds(cfg, model, state, pts, n=None, seed=None):
    """A batched State of n worlds: the rig moved rigidly to a random pose per world (x U[0, 200] m, pot centre at
    terrain height + 0.5 + U[0.5, 2] m, rig angle U[-pi, pi]) and the boxes' stacks moved with the pot, unrotated;
    linear velocities N(0, v_sigma) m/s, head angular velocity U[-head_w, head_w] rad/s. Fat AABBs of the moved
    fixtures recomputed."""
    n = cfg.worlds if n is None else n
    rng = np.random.default_rng(7919 * (cfg.seed + 1) if seed is None else seed)
    st = wd.batch(state, n)
    bd = st.bodies
    dyn = np.nonzero(bd.type[0] == wd.DYNAMIC)[0]
    x = rng.uniform(0.0, 200.0, n)
    y = height_at(pts, x) + 0.5 + rng.uniform(0.5, 2.0, n)
    ang = rng.uniform(-np.pi, np.pi, n).astype(F32)
    c, s = _rot(ang)
    pot = int(dyn[0])
    base = bd.xf_p[0, pot].astype(np.float64)
    for i, b in enumerate(dyn):
        lx, ly = bd.xf_p[0, b].astype(np.float64) - base
        rigid = i < RIG_BODIES
        cb, sb = (c, s) if rigid else (np.ones(n, F32), np.zeros(n, F32))
        px = (x + (cb.astype(np.float64) * lx - sb.astype(np.float64) * ly)).astype(F32)
        py = (y + (sb.astype(np.float64) * lx + cb.astype(np.float64) * ly)).astype(F32)
        bd.xf_p[:, b, 0], bd.xf_p[:, b, 1] = px, py
        bd.xf_q[:, b, 0], bd.xf_q[:, b, 1] = cb, sb
        bd.a[:, b] = ang if rigid else 0.0
        bd.a0[:, b] = ang if rigid else 0.0
        lc = bd.local_center[:, b]
        cx = (px + ((cb * lc[:, 0]).astype(F32) - (sb * lc[:, 1]).astype(F32))).astype(F32)
        cy = (py + ((sb * lc[:, 0]).astype(F32) + (cb * lc[:, 1]).astype(F32))).astype(F32)
        bd.c[:, b, 0], bd.c[:, b, 1] = cx, cy
        bd.c0[:, b, 0], bd.c0[:, b, 1] = cx, cy
        if cfg.v_sigma > 0:
            bd.v[:, b] = rng.normal(0.0, cfg.v_sigma, (n, 2)).astype(F32)
    if cfg.head_w > 0:
        head = int(dyn[3])
        bd.w[:, head] = rng.uniform(-cfg.head_w, cfg.head_w, n).astype(F32)
    rows = [f for f in range(model.fixture_body.shape[0]) if bd.type[0, model.fixture_body[f]] != wd.STATIC]
    st.fixtures.fat[:, rows] = fat_rows(model, st, rows)
    return st


def actions(rng, n):
    """Actions uniform in the unit disk (sqrt(U) radius, U angle), float32 (n, 2)."""
    r = np.sqrt(rng.uniform(0.0, 1.0, n))
    t = rng.uniform(0.0, 2.0 * np.pi, n)
    return np.stack([r * np.cos(t), r * np.sin(t)], 1).astype(F32)


def apply_actions(joint_speed, joint_torque, a):
    """Write actions into the motor joint's leaves (numpy or torch (N, J) views, in place):
    motor_speed = gain * a_x, max_motor = torque * |a| on the torso-handle joint.

    Device State leaves (worlds-minor, as layout.empty_device_state makes them) take one launch of the library's
    goi_apply_motor_actions on torch's current stream; numpy arrays (the oracle's side) take the same float32
    operations on the host."""
    if _native_actions(joint_speed, joint_torque, a):
        return
    ax = a[:, 0]
    mag = (a[:, 0] * a[:, 0] + a[:, 1] * a[:, 1]) ** 0.5
    joint_speed[:, MOTOR_JOINT] = MOTOR_GAIN * ax
    joint_torque[:, MOTOR_JOINT] = MOTOR_TORQUE * mag


def _native_actions(speed, torque, a):
    """goi_apply_motor_actions for CUDA float32 (N, J) leaves with the State's worlds-minor strides (1, pitch) and a
    contiguous (N, 2) float32 action tensor on the same device; False for anything else."""
    if not getattr(speed, "is_cuda", False):
        return False
    import torch
    n, J = speed.shape
    if not (getattr(torque, "is_cuda", False) and getattr(a, "is_cuda", False) and speed.dtype == torch.float32
            and torque.dtype == torch.float32 and a.dtype == torch.float32 and a.shape == (n, 2)
            and a.is_contiguous() and torque.shape == speed.shape and speed.stride() == torque.stride()
            and speed.stride(0) == 1 and J > MOTOR_JOINT and a.device == speed.device == torque.device):
        return False
    from . import _abi
    L = _abi.lib()
    stream = torch.cuda.current_stream(speed.device).cuda_stream
    _abi.check(L.goi_apply_motor_actions(a.data_ptr(), speed.data_ptr(), torque.data_ptr(), int(n),
                                         int(speed.stride(1)) if J > 1 else int(n), MOTOR_JOINT,
                                         float(MOTOR_GAIN), float(MOTOR_TORQUE), stream), L)
    return True


def make_config(k, n=None, edges="quad"):
    """(settings, compact Model, batched compact numpy State, Config) of benchmark configuration k (1-5)."""
    cfg = CONFIGS[k]
    settings = settings_for(cfg)
    model, state, pts = build_world(cfg, settings, edges)
    st = place_worlds(cfg, model, state, pts, n)
    cm = wd.compact_model(model, st)
    return settings, cm, wd.compact_state(cm, st), cfg


# ---------------------------------------------------------------- small deterministic test scenes
# Scene inputs follow the reference's parity scenes (tests/box2d/box2d_scenes.py:21-355, tests/box2d/test_toi.py:20-121).

def _ngon(n, r, phase=0.0):
    a = phase + 2 * np.pi * np.arange(n) / n
    return np.stack([r * np.cos(a), r * np.sin(a)], 1).astype(F32)


def scene_free_fall(s):
    d = wd.WorldDef(s)
    a = d.add_body(wd.DYNAMIC, (1.25, 7.5), 0.0, (3, 2), 0.0, mass=4, inertia=1, linear_damping=0.2)
    d.add_box(a, (0.3, 0.2))
    b = d.add_body(wd.DYNAMIC, (-2, 3), 0.7, (-1, 4), 5.0, mass=1.5, center=(0.1, -0.05), inertia=0.3,
                   linear_damping=0.05, angular_damping=0.5)
    d.add_polygon(b, _ngon(5, 0.4))
    k = d.add_body(wd.KINEMATIC, (5, 0), 0.1, (0.5, -0.25), 1.0)
    d.add_box(k, (0.5, 0.1))
    return d


def scene_box_stack(s):
    d = wd.WorldDef(s)
    g = d.add_body(wd.STATIC)
    d.add_box(g, (10, 0.5), friction=0.6)
    for i in range(4):
        b = d.add_body(wd.DYNAMIC, (0.03 * i, 1.0 + 0.995 * i + 0.01), 0.002 * i, mass=1, inertia=F32(1) / F32(6))
        d.add_box(b, (0.5, 0.49), friction=0.6)
    return d


def scene_polygons(s):
    d = wd.WorldDef(s)
    g = d.add_body(wd.STATIC)
    d.add_box(g, (12, 0.5), friction=0.8)
    d.add_polygon(g, [(4, 0.5), (9, 0.5), (9, 2.3)], friction=0.8)
    for i, ang in enumerate((0.0, 0.3, np.pi / 4, 1.4, -0.7)):
        b = d.add_body(wd.DYNAMIC, (-8 + 2.2 * i, 1.6 + 0.1 * i), ang, (0, -1), 0.5 * (i - 2), mass=1 + 0.3 * i,
                       inertia=0.2 + 0.05 * i)
        d.add_box(b, (0.45, 0.3 + 0.05 * i), friction=0.5)
    h = d.add_body(wd.DYNAMIC, (6.5, 2.2), 0.1, mass=2, inertia=0.4)
    d.add_polygon(h, _ngon(6, 0.45, 0.2), friction=0.4)
    tri = d.add_body(wd.DYNAMIC, (3.0, 1.2), 2.0, mass=1, inertia=0.1)
    d.add_polygon(tri, [(0.4, 0.0), (-0.3, 0.35), (-0.25, -0.3)], friction=0.9)
    p = d.add_body(wd.DYNAMIC, (0.0, 4.0), 0.2, (2, 0), 0, mass=1, inertia=0.15)
    d.add_box(p, (0.3, 0.3))
    q = d.add_body(wd.DYNAMIC, (1.2, 4.1), -0.3, (-2, 0), 1, mass=1.5, inertia=0.2)
    d.add_box(q, (0.35, 0.25))
    return d


def scene_circles(s):
    d = wd.WorldDef(s)
    g = d.add_body(wd.STATIC)
    d.add_box(g, (12, 0.5), friction=0.7)
    d.add_polygon(g, [(-9, 0.5), (-4, 0.5), (-9, 2.0)], friction=0.7)
    c1 = d.add_body(wd.DYNAMIC, (0, 0.82), mass=1, inertia=0.05)
    d.add_circle(c1, 0.3, friction=0.5)
    c2 = d.add_body(wd.DYNAMIC, (-6.5, 2.0), 0.0, (0, 0), -2.0, mass=1, inertia=0.04)
    d.add_circle(c2, 0.25, (0.02, 0.0), friction=0.9)
    bx = d.add_body(wd.STATIC, (4, 1.5), 0.3)
    d.add_box(bx, (0.5, 0.2))
    c3 = d.add_body(wd.DYNAMIC, (4.6, 2.4), 0.0, (-0.5, -1), 0, mass=0.5, inertia=0.01)
    d.add_circle(c3, 0.2)
    c4 = d.add_body(wd.DYNAMIC, (1.5, 3.0), 0.0, (1.5, 0), 0, mass=0.8, inertia=0.02)
    d.add_circle(c4, 0.25)
    c5 = d.add_body(wd.DYNAMIC, (2.6, 3.05), 0.0, (-1.5, 0), 0, mass=1.0, inertia=0.03)
    d.add_circle(c5, 0.3)
    s1 = d.add_body(wd.DYNAMIC, (-2, 0.81), mass=1, inertia=0.05)
    d.add_circle(s1, 0.3)
    s2 = d.add_body(wd.DYNAMIC, (-1.98, 1.4), mass=0.5, inertia=0.02)
    d.add_circle(s2, 0.28)
    hb = d.add_body(wd.DYNAMIC, (7, 1.4), 0.6, (0, -0.5), 0, mass=1, inertia=0.1)
    d.add_box(hb, (0.4, 0.3))
    hc = d.add_body(wd.DYNAMIC, (7.1, 2.3), 0.0, (0, -1), 0, mass=0.3, inertia=0.005)
    d.add_circle(hc, 0.15)
    return d


def scene_joints(s):
    """Revolute (motor + limits, free, chain), prismatic (motor into a limit, limited pair, equal limits) and weld
    (rigid, soft, pair) joints together."""
    d = wd.WorldDef(s)
    g = d.add_body(wd.STATIC)
    d.add_box(g, (0.2, 0.2), (0, 5))
    a = d.add_body(wd.DYNAMIC, (1.0, 5.0), 0.0, mass=1, inertia=0.1)
    d.add_box(a, (0.5, 0.1))
    d.add_revolute(g, a, (0, 5), (-0.5, 0), 0.0, limits=(-0.6, 0.4), motor_speed=2.0, max_motor_torque=30.0,
                   enable_motor=True)
    b = d.add_body(wd.DYNAMIC, (-1.0, 5.0), 0.0, mass=2, inertia=0.3)
    d.add_box(b, (0.6, 0.1))
    d.add_revolute(g, b, (0, 5), (0.6, 0), 0.0, limits=(-0.5, 0.5))
    c = d.add_body(wd.DYNAMIC, (-2.2, 5.0), 0.0, (0, 1), 0, mass=1, inertia=0.1)
    d.add_box(c, (0.6, 0.08))
    d.add_revolute(b, c, (-0.6, 0), (0.6, 0), 0.0, motor_speed=-1.0, max_motor_torque=5.0, enable_motor=True)
    g2 = d.add_body(wd.STATIC, (10, 0))
    d.add_box(g2, (0.2, 0.2))
    sl = d.add_body(wd.DYNAMIC, (10.5, 0.5), 0.3, mass=2, inertia=0.2)
    d.add_box(sl, (0.3, 0.1))
    d.add_prismatic(g2, sl, (0, 0), (0, 0), (np.cos(0.7), np.sin(0.7)), 0.3, limits=(-0.2, 1.0), motor_speed=1.5,
                    max_motor_force=200.0, enable_motor=True)
    u = d.add_body(wd.DYNAMIC, (13, 2), 0.1, (0.5, 0), 0.2, mass=1, inertia=0.1)
    d.add_box(u, (0.3, 0.3))
    v = d.add_body(wd.DYNAMIC, (13.6, 2.05), 0.1, mass=0.5, inertia=0.05)
    d.add_box(v, (0.2, 0.2))
    d.add_prismatic(u, v, (0.3, 0), (-0.2, 0), (1, 0), 0.0, limits=(-0.05, 0.25), motor_speed=-0.5,
                    max_motor_force=10.0, enable_motor=True)
    e = d.add_body(wd.DYNAMIC, (8, 1), 0.0, mass=1, inertia=0.1)
    d.add_box(e, (0.2, 0.2))
    d.add_prismatic(g2, e, (-2, 1), (0, 0), (0, 1), 0.0, limits=(0.0, 0.0))
    g3 = d.add_body(wd.STATIC, (0, -10))
    d.add_box(g3, (0.2, 0.5), (0, 3))
    wa = d.add_body(wd.DYNAMIC, (0.7, -7.0), 0.0, mass=1, inertia=0.1)
    d.add_box(wa, (0.5, 0.1))
    d.add_weld(g3, wa, (0.2, 3.0), (-0.5, 0.0), 0.0)
    wb = d.add_body(wd.DYNAMIC, (-0.7, -7.0), 0.0, mass=1, inertia=0.1)
    d.add_box(wb, (0.5, 0.1))
    d.add_weld(g3, wb, (-0.2, 3.0), (0.5, 0.0), 0.0, frequency=5.0, damping=0.7)
    wc = d.add_body(wd.DYNAMIC, (3, -7), 0.2, (1, 0), 1.0, mass=1, inertia=0.1)
    d.add_box(wc, (0.3, 0.1))
    wdd = d.add_body(wd.DYNAMIC, (3.6, -6.88), 0.2, mass=2, inertia=0.2)
    d.add_box(wdd, (0.3, 0.1))
    d.add_weld(wc, wdd, (0.3, 0), (-0.3, 0), 0.0, frequency=70.0, damping=1.0)
    return d


def scene_pile(s):
    d = wd.WorldDef(s)
    g = d.add_body(wd.STATIC)
    d.add_box(g, (6, 0.3), friction=0.6)
    d.add_polygon(g, [(-6, 0.3), (-5.5, 0.3), (-6, 3.0)], friction=0.6)
    d.add_polygon(g, [(5.5, 0.3), (6, 0.3), (6, 3.0)], friction=0.6)
    rng = np.random.default_rng(7)
    for i in range(12):
        x, y = F32(rng.uniform(-3, 3)), F32(1.2 + 0.9 * i)
        ang, w = F32(rng.uniform(-1.5, 1.5)), F32(rng.uniform(-2, 2))
        b = d.add_body(wd.DYNAMIC, (x, y), ang, (F32(rng.uniform(-1, 1)), 0), w, mass=F32(0.5 + 0.1 * i),
                       inertia=F32(0.05 + 0.01 * i))
        kind = i % 3
        if kind == 0:
            d.add_box(b, (F32(0.25 + 0.02 * i), F32(0.2)), friction=0.5)
        elif kind == 1:
            d.add_polygon(b, _ngon(3 + i % 5, 0.3), friction=0.4)
        else:
            d.add_circle(b, F32(0.2 + 0.01 * i), friction=0.6)
    return d


def scene_misc(s):
    d = wd.WorldDef(s)
    g = d.add_body(wd.STATIC)
    d.add_box(g, (12, 0.5), friction=0.6)
    k = d.add_body(wd.KINEMATIC, (-4.0, 0.9), 0.0, (1.5, 0.0), 0.3)
    d.add_box(k, (0.2, 0.3))
    pushed = d.add_body(wd.DYNAMIC, (-3.2, 0.81), mass=1, inertia=0.05)
    d.add_box(pushed, (0.3, 0.3), friction=0.4)
    sleeper = d.add_body(wd.DYNAMIC, (2.0, 0.995), mass=1, inertia=0.1, awake=False)
    d.add_box(sleeper, (0.5, 0.49))
    faller = d.add_body(wd.DYNAMIC, (2.1, 2.6), 0.2, mass=0.5, inertia=0.03)
    d.add_box(faller, (0.25, 0.25))
    ball = d.add_body(wd.DYNAMIC, (5.0, 2.5), 0.0, (0.3, 0.0), 0.0, mass=0.4, inertia=0.004, gravity_scale=0.5)
    d.add_circle(ball, 0.2, restitution=0.6)
    awake_box = d.add_body(wd.DYNAMIC, (-7.0, 1.2), 0.1, mass=1, inertia=0.1, allow_sleep=False)
    d.add_box(awake_box, (0.3, 0.3))
    ghost = d.add_body(wd.DYNAMIC, (8.0, 0.6), 0.0, mass=1, inertia=0.1, active=False)
    d.add_box(ghost, (0.3, 0.3))
    return d


def scene_ball_wall(s):
    d = wd.WorldDef(s)
    w = d.add_body(wd.STATIC, (5.0, 0.0))
    d.add_box(w, (0.05, 2.0))
    b = d.add_body(wd.DYNAMIC, (0.0, 0.1), 0.0, (900.0, 3.0), 0.0, mass=1.0, inertia=0.005, continuous=True)
    d.add_circle(b, 0.1)
    dd = d.add_body(wd.DYNAMIC, (0.0, -1.0), 0.0, (900.0, 0.0), 0.0, mass=1.0, inertia=0.005)
    d.add_circle(dd, 0.1)
    return d


def scene_poly_angles(s):
    d = wd.WorldDef(s)
    g = d.add_body(wd.STATIC)
    d.add_box(g, (30.0, 0.5), friction=0.8)
    d.add_polygon(g, [(10, 0.5), (16, 0.5), (16, 3.0)], friction=0.6)
    for i, (ang, vel, w) in enumerate([(0.0, (0, -400), 0.0), (0.4, (60, -350), 3.0), (1.1, (-80, -500), -8.0),
                                        (2.5, (200, -300), 20.0)]):
        b = d.add_body(wd.DYNAMIC, (-12.0 + 6 * i, 4.0 + 0.3 * i), ang, vel, w, mass=1.0 + 0.2 * i,
                       inertia=0.1 + 0.02 * i, continuous=True)
        d.add_box(b, (0.3, 0.12 + 0.03 * i), friction=0.5)
    tri = d.add_body(wd.DYNAMIC, (13.0, 6.0), 0.3, (20, -420), 5.0, mass=0.8, inertia=0.05, continuous=True)
    d.add_polygon(tri, [(0.3, 0.0), (-0.2, 0.25), (-0.2, -0.2)], friction=0.9)
    return d


def scene_hammer_chain(s):
    d = wd.WorldDef(s)
    g = d.add_body(wd.STATIC)
    d.add_box(g, (10.0, 0.5), friction=0.7)
    d.add_polygon(g, [(-1.0, 0.5), (1.5, 0.5), (0.2, 1.4)], friction=0.7)
    hub = d.add_body(wd.KINEMATIC, (0.0, 2.6))
    d.add_circle(hub, 0.05, group=-1)
    arm = d.add_body(wd.DYNAMIC, (0.9, 2.6), 0.0, mass=2.0, center=(0.0, 0.0), inertia=0.3)
    d.add_box(arm, (0.9, 0.04), group=-1)
    head = d.add_body(wd.DYNAMIC, (1.9, 2.6), 0.0, mass=0.5, inertia=0.004, continuous=True)
    d.add_box(head, (0.1, 0.06), friction=0.7, group=-1)
    d.add_revolute(hub, arm, (0.0, 0.0), (-0.9, 0.0), motor_speed=-40.0, max_motor_torque=5000.0, enable_motor=True)
    d.add_revolute(arm, head, (0.9, 0.0), (-0.1, 0.0), limits=(-0.3, 0.3))
    return d


def scene_multi_event(s):
    d = wd.WorldDef(s)
    w = d.add_body(wd.STATIC)
    d.add_box(w, (0.05, 3.0), (3.0, 0.0), restitution=1.0)
    d.add_box(w, (0.05, 3.0), (3.6, 0.0), restitution=1.0)
    d.add_box(w, (0.05, 3.0), (-3.0, 5.0))
    a = d.add_body(wd.DYNAMIC, (3.3, 0.0), 0.0, (300.0, 40.0), 1.0, mass=1.0, inertia=0.01, continuous=True)
    d.add_circle(a, 0.08, restitution=1.0, friction=0.0)
    b = d.add_body(wd.DYNAMIC, (0.0, 5.0), 0.3, (-700.0, -20.0), 4.0, mass=1.0, inertia=0.02, continuous=True)
    d.add_box(b, (0.1, 0.1))
    return d


def scene_stock_bullets(s):
    d = wd.WorldDef(s)
    g = d.add_body(wd.STATIC)
    d.add_box(g, (10.0, 0.5))
    box = d.add_body(wd.DYNAMIC, (3.0, 1.1), mass=4.0, inertia=0.6)
    d.add_box(box, (0.5, 0.5))
    bul = d.add_body(wd.DYNAMIC, (-3.0, 1.2), 0.0, (800.0, 0.0), 0.0, mass=0.2, inertia=0.001, bullet=True)
    d.add_circle(bul, 0.05)
    fall = d.add_body(wd.DYNAMIC, (-6.0, 6.0), 0.2, (0.0, -600.0), 0.0, mass=1.0, inertia=0.1)
    d.add_box(fall, (0.2, 0.2))
    return d


def scene_island_walk(s):
    d = wd.WorldDef(s)
    g = d.add_body(wd.STATIC)
    d.add_box(g, (20.0, 0.5), friction=0.6)
    d.add_box(g, (0.05, 2.0), (6.0, 2.5))
    d.add_box(g, (0.05, 2.0), (6.3, 2.5))
    k = d.add_body(wd.KINEMATIC, (-6.0, 1.5), 0.0, (0.0, 0.0), 0.0)
    d.add_box(k, (0.05, 1.0))
    b = d.add_body(wd.DYNAMIC, (0.0, 0.6), 0.0, (500.0, 0.0), 0.0, mass=1.0, inertia=0.05, continuous=True)
    d.add_box(b, (0.2, 0.1), friction=0.5)
    c = d.add_body(wd.DYNAMIC, (-1.0, 0.75), 0.0, (-450.0, 0.0), 0.0, mass=1.0, inertia=0.05, continuous=True)
    d.add_box(c, (0.2, 0.25), friction=0.5)
    sp = d.add_body(wd.DYNAMIC, (3.0, 0.62), 0.0, (0.0, 0.0), 0.0, mass=1.0, inertia=0.05)
    d.add_box(sp, (0.1, 0.1))
    return d


def scene_toi_tie(s):
    """A ball falling at 60 m/s between two equal static circles set symmetrically about its path (fixture 0 at
    x = -0.2, fixture 1 at x = +0.2). While the ball moves along x = 0, every float operation of the two contacts'
    TOIs is the mirror image of the other's, so their TOIs are equal to the bit and the event order is the tie
    rule's (toi.py:552-556)."""
    d = wd.WorldDef(s)
    g = d.add_body(wd.STATIC)
    d.add_circle(g, 0.2, center=(-0.2, 0.0))
    d.add_circle(g, 0.2, center=(0.2, 0.0))
    b = d.add_body(wd.DYNAMIC, (0.0, 2.5), 0.0, (0.0, -60.0), 0.0, mass=1.0, inertia=0.01)
    d.add_circle(b, 0.1)
    return d


def scene_wake_cascade(s, xy_newer=True):
    """Zero-gravity Collide wake cascade (pairs.py:90-117): box X (0.2 x 0.2) drifts at 0.075 m/s toward box Y
    (0.8 x 0.2, body 1) from 0.08 m away; box Z (0.2 x 0.2) rests 0.05 m beyond Y. All three are made in one
    FindNewContacts pass, keyed in fixture order: the fixtures are made Z, Y, X when xy_newer (X is body 2, Z body 0,
    and the X-Y contact is the newer) and X, Y, Z otherwise (X body 0, Z body 2)."""
    d = wd.WorldDef(s)
    for name in ("ZYX" if xy_newer else "XYZ"):
        if name == "X":
            b = d.add_body(wd.DYNAMIC, (-0.58, 0.0), 0.0, (0.075, 0.0), mass=1.0, inertia=0.1)
            d.add_box(b, (0.1, 0.1))
        elif name == "Y":
            b = d.add_body(wd.DYNAMIC, (0.0, 0.0), mass=1.0, inertia=0.1)
            d.add_box(b, (0.4, 0.1))
        else:
            b = d.add_body(wd.DYNAMIC, (0.55, 0.0), mass=1.0, inertia=0.1)
            d.add_box(b, (0.1, 0.1))
    return d


def scene_toi_plank(s, ball_bullet=False, plank_bullet=False):
    """Zero-gravity TOI island membership (toi.py:604-716): a ball touching the top of a floating plank (body 1)
    slides at 150 m/s into a static face that leans over the plank (normal left-down), so the TOI velocity solve
    presses the ball into the plank. The plank joins the TOI island only if the ball or the plank is a bullet."""
    d = wd.WorldDef(s)
    g = d.add_body(wd.STATIC)
    d.add_polygon(g, [(2.3, 0.75), (2.6, 0.75), (2.6, 1.5), (1.9, 1.5)])
    plank = d.add_body(wd.DYNAMIC, (0.0, 0.6), mass=4.0, inertia=6.0, bullet=plank_bullet)
    d.add_box(plank, (2.25, 0.1))
    ball = d.add_body(wd.DYNAMIC, (-1.5, 0.81), 0.0, (150.0, 0.0), 0.0, mass=0.5, inertia=0.0025,
                      bullet=ball_bullet)
    d.add_circle(ball, 0.1)
    return d


def scene_edges(s):
    """Native edge shapes: an open chain with convex and concave corners and a collinear run, a closed loop, an
    isolated two-sided segment and a segment with ghost vertices but no neighbours; boxes slide across the chain's
    junctions, polygons and circles land on corners, a fast circle reaches the loop by TOI."""
    d = wd.WorldDef(s)
    g = d.add_body(wd.STATIC)
    d.add_chain(g, [(-12, 4), (-8, 0.5), (-4, 0), (-2, 0), (0, 0), (2, 0), (4, 0.8), (6, 0.2), (9, 2.5), (12, 6)],
                friction=0.6)
    d.add_chain(g, [(-1, 3), (1, 3), (1, 3.5), (-1, 3.5)], loop=True, friction=0.6)
    d.add_segment(g, (5, 4), (8, 4.5), friction=0.4)
    d.add_segment(g, (-7, 5), (-5, 5), v0=(-8, 5.5), v3=(-4, 4.5), friction=0.4)
    a = d.add_body(wd.DYNAMIC, (-3.5, 0.26), 0.0, (6.0, 0.0), 0.0, mass=1.0, inertia=F32(1) / F32(24))
    d.add_box(a, (0.5, 0.25), friction=0.1)
    b = d.add_body(wd.DYNAMIC, (-1.0, 0.4), 0.3, (-3.0, 0.0), 0.0, mass=0.8, inertia=0.02)
    d.add_polygon(b, _ngon(5, 0.3), friction=0.3)
    c = d.add_body(wd.DYNAMIC, (-9.0, 2.5), 0.0, (1.0, 0.0), 0.0, mass=0.5, inertia=0.01)
    d.add_circle(c, 0.25, friction=0.5)
    e = d.add_body(wd.DYNAMIC, (4.2, 2.0), 0.8, (0.0, -2.0), 1.0, mass=1.2, inertia=0.05)
    d.add_polygon(e, [(-0.3, -0.2), (0.4, -0.1), (0.1, 0.35)], friction=0.5)
    f = d.add_body(wd.DYNAMIC, (6.5, 5.0), 0.0, (0.0, 0.0), 0.0, mass=0.3, inertia=0.005)
    d.add_circle(f, 0.15, friction=0.2)
    h = d.add_body(wd.DYNAMIC, (-6.0, 6.0), 0.2, (0.0, 0.0), 0.0, mass=0.6, inertia=0.02)
    d.add_box(h, (0.3, 0.2), friction=0.4)
    k = d.add_body(wd.DYNAMIC, (0.0, 9.0), 0.0, (0.5, -120.0), 0.0, mass=0.2, inertia=0.002, bullet=True)
    d.add_circle(k, 0.1, friction=0.3)
    return d


# (builder, settings, contact capacity); game settings as the reference scenes use them
def _game(**kw):
    return Settings.game(**kw)


def _toi(unity=True, gravity=(0.0, -30.0)):
    return Settings.game(unity_toi=unity, gravity=gravity)


TEST_SCENES = {
    "free_fall": (scene_free_fall, _game, 16),
    "box_stack": (scene_box_stack, _game, 16),
    "polygons": (scene_polygons, _game, 24),
    "circles": (scene_circles, _game, 24),
    "joints": (scene_joints, _game, 16),
    "joints_v23": (scene_joints, lambda: Settings.game(revolute_v24=False), 16),
    "pile": (scene_pile, _game, 64),
    "misc": (scene_misc, _game, 24),
    "ball_wall": (scene_ball_wall, lambda: _toi(gravity=(0.0, 0.0)), 16),
    "poly_angles": (scene_poly_angles, _toi, 24),
    "hammer_chain": (scene_hammer_chain, _toi, 16),
    "multi_event": (scene_multi_event, lambda: _toi(gravity=(0.0, 0.0)), 16),
    "stock_bullets": (scene_stock_bullets, lambda: _toi(unity=False), 16),
    "island_walk": (scene_island_walk, _toi, 32),
    "edges": (scene_edges, _toi, 32),
    "toi_tie": (scene_toi_tie, lambda: Settings.stock(gravity=(0.0, 0.0), continuous_physics=True), 8),
    "toi_tie_oldest": (scene_toi_tie, lambda: Settings.stock(gravity=(0.0, 0.0), continuous_physics=True,
                                                             toi_tie_oldest=True), 8),
    "toi_plank": (scene_toi_plank, lambda: Settings.stock(gravity=(0.0, 0.0), continuous_physics=True), 8),
    "toi_plank_bullet": (lambda s: scene_toi_plank(s, ball_bullet=True),
                         lambda: Settings.stock(gravity=(0.0, 0.0), continuous_physics=True), 8),
}


def build_test_scene(name, iterations=None):
    """(settings, compact Model, single-world compact State) of a test scene; iterations=(v, p) overrides the
    game's 300 / 30 to keep CPU checks fast."""
    from dataclasses import replace
    fn, sfn, cap = TEST_SCENES[name]
    s = sfn()
    if iterations is not None:
        s = replace(s, velocity_iterations=iterations[0], position_iterations=iterations[1])
    d = fn(s)
    model, state = d.build(contact_capacity=cap)
    cm = wd.compact_model(model, state)
    return s, cm, wd.compact_state(cm, state)
