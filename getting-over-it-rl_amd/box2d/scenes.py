"""Seeded synthetic worlds of the benchmark workloads: the static terrain (edge chain + convex rocks), the 4-body
character rig with its action-driven motor, the large-island configuration's stacked boxes, and the five benchmark
configurations.

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


def make_config(k, n=None, edges="quad", capacity=None):
    """(settings, compact Model, batched compact numpy State, Config) of benchmark configuration k (1-5); `capacity`
    replaces the configuration's contact slots per world (a small table makes FindNewContacts drop pairs)."""
    cfg = CONFIGS[k]
    if capacity is not None:
        from dataclasses import replace
        cfg = replace(cfg, capacity=int(capacity))
    settings = settings_for(cfg)
    model, state, pts = build_world(cfg, settings, edges)
    st = place_worlds(cfg, model, state, pts, n)
    cm = wd.compact_model(model, st)
    return settings, cm, wd.compact_state(cm, st), cfg
