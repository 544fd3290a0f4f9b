"""Pins of the CPU oracle (oracle/b2_oracle.c) that need no reference import: closed forms, known answers, brute
force and physical invariants, each chosen so that a plausible slip (a dropped term, a swapped operand, a wrong
index, a wrong tie rule) fails it. The checks follow the reference's own oracle tests where it has them
(tests/reference/test_box2d_reference.py:23-155, tests/box2d/test_toi.py:23-35, test_box2d_parity.py:44-50) and
the b2Distance / b2TimeOfImpact / b2Collide contracts otherwise. CPU only.
"""
import numpy as np
import pytest

from util import b2
import scene_defs

F32 = np.float32
H = b2.GAME_DT
wd = b2.world
S = b2.Settings
CIRCLE, POLYGON = b2.shapes.CIRCLE, b2.shapes.POLYGON


def run(d, steps, capacity=16, settings=None, dt=H, n=1, oracle=None, each=None):
    model, state = d.build(capacity)
    st = wd.batch(state, n)
    for k in range(steps):
        oracle.step_(model, st, settings or d.settings, dt)
        if each is not None:
            each(k, st)
    return model, st


# ---------------------------------------------------------------------------------------------------------------
# sin / cos: correctly rounded float32, (float)sin((double)x)   (math2d.py:291-310, test_box2d_parity.py:44-50)

def test_sincos_known_answers(oracle):
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.uniform(-8, 8, 20000), rng.uniform(-300, 300, 5000), [0.0, -0.0, np.pi],
                        rng.uniform(-1e4, 1e4, 20000)]).astype(F32)
    s, c = oracle.sincos(x)
    xs = x.astype(np.float64)
    assert np.array_equal(s, np.sin(xs).astype(F32)) and np.array_equal(c, np.cos(xs).astype(F32))
    assert np.signbit(s[25001]) and not np.signbit(s[25000])  # sin(-0) = -0
    assert s[25002] == F32(np.sin(np.float64(F32(np.pi))))


# ---------------------------------------------------------------------------------------------------------------
# integration: semi-implicit Euler with 2.3.1 damping, bit exact   (test_box2d_reference.py:23-35, step.py:86-93)

@pytest.mark.parametrize("drag", [0.0, 0.2])
def test_free_fall_is_semi_implicit_euler_bit_exact(oracle, drag):
    d = wd.WorldDef(S.game())
    d.add_body(wd.DYNAMIC, (1.25, 7.5), velocity=(3, 2), mass=4, inertia=1, linear_damping=drag)
    g = F32(-30)
    x, y, vx, vy = F32(1.25), F32(7.5), F32(3), F32(2)
    damp = F32(1) / (F32(1) + H * F32(drag))
    model, st = d.build(4)
    st = wd.batch(st, 1)
    for _ in range(300):
        oracle.step_(model, st, d.settings, H)
        vx = (vx + H * (F32(1) * F32(0) + F32(0))) * damp
        vy = (vy + H * (F32(1) * g + F32(0))) * damp
        x, y = x + H * vx, y + H * vy
        got = (st.bodies.c[0, 0, 0], st.bodies.c[0, 0, 1], st.bodies.v[0, 0, 0], st.bodies.v[0, 0, 1])
        assert got == (x, y, vx, vy)
        assert tuple(st.bodies.xf_p[0, 0]) == (x, y)  # local centre 0: xf.p = c


def test_max_translation_clamp(oracle):
    """b2Island::Solve: a step that would move further than max_translation is scaled to exactly that length."""
    d = wd.WorldDef(S.stock(gravity=(0, 0)))
    d.add_body(wd.DYNAMIC, (0, 0), velocity=(300, 400), mass=1, inertia=1)
    model, st = run(d, 1, dt=F32(1 / 60), oracle=oracle, settings=d.settings)
    moved = float(np.hypot(*st.bodies.c[0, 0]))
    assert moved == pytest.approx(2.0, rel=1e-6)  # stock max_translation 2 m
    assert float(np.hypot(*st.bodies.v[0, 0])) == pytest.approx(120.0, rel=1e-6)


# ---------------------------------------------------------------------------------------------------------------
# resting contact   (test_box2d_reference.py:14-63)

def resting_box(settings=None, y=1.015):
    d = wd.WorldDef(settings or S.game())
    ground = d.add_body(wd.STATIC)
    d.add_box(ground, (10, 0.5), friction=1.0)
    box = d.add_body(wd.DYNAMIC, (0, y), mass=2, inertia=F32(2) / F32(6))
    d.add_box(box, (0.5, 0.5), friction=0.5)
    return d, box


def world_points(model, st, w, slot, bodies=None, normal=False):
    """b2WorldManifold::Initialize for one slot: (points [count, 2], separations [count]) in float64, at the body
    transforms of `bodies` (default st.bodies); with normal=True also the world normal."""
    ct, bd = st.contacts, (st.bodies if bodies is None else bodies)
    fa, fb = int(ct.fa[w, slot]), int(ct.fb[w, slot])
    ba, bb = int(model.fixture_body[fa]), int(model.fixture_body[fb])
    ra, rb = float(model.radius[fa]), float(model.radius[fb])

    def xf(b):
        return np.array(bd.xf_p[w, b], np.float64), np.array(bd.xf_q[w, b], np.float64)

    def mul(t, v):
        (p, (c, s)) = t
        return np.array([c * v[0] - s * v[1] + p[0], s * v[0] + c * v[1] + p[1]])

    def rot(t, v):
        c, s = t[1]
        return np.array([c * v[0] - s * v[1], s * v[0] + c * v[1]])
    xa, xb = xf(ba), xf(bb)
    mt, n = int(ct.mtype[w, slot]), int(ct.count[w, slot])
    pts, seps = [], []
    for i in range(n):
        lp = ct.point_local[w, slot, i].astype(np.float64)
        if mt == 0:
            pa, pb = mul(xa, ct.local_point[w, slot]), mul(xb, lp)
            nrm = pb - pa
            nrm = nrm / np.linalg.norm(nrm) if np.linalg.norm(nrm) > 1e-12 else np.array([1.0, 0.0])
            ca, cb = pa + ra * nrm, pb - rb * nrm
        elif mt == 1:
            nrm = rot(xa, ct.local_normal[w, slot])
            plane = mul(xa, ct.local_point[w, slot])
            clip = mul(xb, lp)
            ca = clip + (ra - np.dot(clip - plane, nrm)) * nrm
            cb = clip - rb * nrm
        else:
            nrm = rot(xb, ct.local_normal[w, slot])
            plane = mul(xb, ct.local_point[w, slot])
            clip = mul(xa, lp)
            cb = clip + (rb - np.dot(clip - plane, nrm)) * nrm
            ca = clip - ra * nrm
            nrm = -nrm
        pts.append(0.5 * (ca + cb))
        seps.append(float(np.dot(cb - ca, nrm)))
    if normal:
        return np.array(pts).reshape(-1, 2), np.array(seps), nrm
    return np.array(pts).reshape(-1, 2), np.array(seps)


def test_box_rests_and_sleeps(oracle):
    d, box = resting_box()
    model, state = d.build(8)
    x0, y0 = state.bodies.c[box]
    _, st = run(d, 240, capacity=8, oracle=oracle)
    assert abs(st.bodies.c[0, box, 0] - x0) < 1e-5 and abs(st.bodies.a[0, box]) < 1e-5
    assert abs(st.bodies.c[0, box, 1] - y0) < 1e-3  # settles only into the linear-slop skin
    assert not st.bodies.awake[0, box]  # time_to_sleep 0.5 s at rest
    assert np.all(st.bodies.v[0, box] == 0) and st.bodies.w[0, box] == 0  # sleeping zeroes velocity


def test_contact_impulses_carry_the_weight(oracle):
    d, box = resting_box()
    model, st = run(d, 30, capacity=8, oracle=oracle)
    ct = st.contacts
    live = np.nonzero((ct.pair[0] >= 0) & ct.touching[0])[0]
    assert len(live) == 1
    k = int(live[0])
    assert int(ct.mtype[0, k]) in (1, 2) and int(ct.count[0, k]) == 2
    assert len(set(ct.point_id[0, k].tolist())) == 2  # distinct feature ids
    total = float(ct.normal_impulse[0, k].sum())
    assert total == pytest.approx(2 * 30 * float(H), rel=1e-3)  # m g dt per step at rest
    assert ct.friction[0, k] == pytest.approx(np.sqrt(F32(0.5) * F32(1.0)), rel=1e-6)
    assert ct.friction[0, k] == F32(np.sqrt(np.float64(F32(F32(0.5) * F32(1.0)))))  # b2MixFriction in float32
    _, seps = world_points(model, st, 0, k)
    assert -0.02 < seps.min() < 0  # rests inside the 2 x 0.01 skin


@pytest.mark.parametrize("iterations", [8, 1])
def test_block_solver_solves_the_two_point_lcp(oracle, iterations):
    """The block solver (contact_solver.py:236-279) solves the two-point normal LCP exactly in each velocity
    iteration: with x the accumulated normal impulses and vn the normal velocities at the two points, x >= 0,
    vn >= 0 and x_i vn_i = 0. K is positive definite, so that solution is unique whichever of the four cases finds
    it. A spinning box falls onto flat ground; after every step whose contact has two points, with the box awake and
    no TOI event, the step's final velocities (those of the last normal solve) meet the conditions at the manifold
    points and the transforms the solver used (the step's start). The run covers case 1 (both points push) and
    cases 2 and 3 (one point lifts)."""
    d = wd.WorldDef(S.stock(gravity=(0, -9.81), continuous_physics=True, velocity_iterations=iterations))
    g = d.add_body(wd.STATIC)
    d.add_box(g, (10, 0.5), friction=0.6)
    box = d.add_body(wd.DYNAMIC, (0, 1.4), 0.3, (1.0, 0.0), 4.0, mass=2, inertia=F32(2) / F32(6))
    d.add_box(box, (0.5, 0.5), friction=0.6)
    model, st = d.build(4)
    n = 16
    st = wd.batch(st, n)
    rng = np.random.default_rng(2)
    st.bodies.w[:, box] = rng.uniform(-8, 8, n).astype(F32)
    st.bodies.v[:, box, 0] = rng.uniform(-2, 2, n).astype(F32)
    dt = F32(1 / 60)
    both = one = 0
    for _ in range(120):
        before = oracle.copy(st).bodies  # the transforms the step's solver works at
        oracle.step_(model, st, d.settings, dt)
        ct = st.contacts
        for i in range(n):
            live = np.nonzero(ct.pair[i] >= 0)[0]
            if len(live) != 1 or int(ct.count[i, live[0]]) != 2 or not st.bodies.awake[i, box] or st.toi.events[i]:
                continue
            k = int(live[0])
            pts, _, nrm = world_points(model, st, i, k, bodies=before, normal=True)
            c = np.asarray(before.c[i, box], np.float64)
            v, w = st.bodies.v[i, box].astype(np.float64), float(st.bodies.w[i, box])
            x = ct.normal_impulse[i, k].astype(np.float64)
            vn = np.array([np.dot(v + w * np.array([-(p - c)[1], (p - c)[0]]), nrm) for p in pts])
            tol = 2e-5 * (1 + np.abs(v).sum() + abs(w))
            assert (x >= 0).all() and (vn >= -tol).all(), (i, x, vn)
            assert (np.abs(vn[x > 0]) <= tol).all(), (i, x, vn)
            both += int((x > 0).all())
            one += int((x > 0).sum() == 1)
    assert both >= 100 and one >= 10, (both, one)


def test_restitution_mix_is_max(oracle):
    """b2MixRestitution = max(a, b); friction mix = sqrt(a * b) (pairs.py:134-178)."""
    d = wd.WorldDef(S.stock())
    g = d.add_body(wd.STATIC)
    d.add_box(g, (10, 0.5), friction=0.9, restitution=0.1)
    b = d.add_body(wd.DYNAMIC, (0, 1.0), mass=1, inertia=0.1)
    d.add_box(b, (0.5, 0.5), friction=0.4, restitution=0.6)
    _, st = run(d, 2, capacity=4, oracle=oracle, dt=F32(1 / 60))
    k = int(np.nonzero(st.contacts.pair[0] >= 0)[0][0])
    assert st.contacts.restitution[0, k] == F32(0.6)
    assert st.contacts.friction[0, k] == F32(np.sqrt(np.float64(F32(F32(0.9) * F32(0.4)))))


def test_bounce_with_restitution_one(oracle):
    """A ball dropped on a restitutive floor comes back up: restitution bias applies when the approach speed exceeds
    velocity_threshold (contact_solver.py:32-147)."""
    d = wd.WorldDef(S.stock(gravity=(0, -10)))
    g = d.add_body(wd.STATIC)
    d.add_box(g, (10, 0.5), restitution=1.0)
    ball = d.add_body(wd.DYNAMIC, (0, 3.0), mass=1, inertia=0.01)
    d.add_circle(ball, 0.25, restitution=1.0)
    vmax = []
    _, st = run(d, 120, capacity=4, oracle=oracle, dt=F32(1 / 60),
                each=lambda k, s: vmax.append(float(s.bodies.v[0, ball, 1])))
    v = np.array(vmax)
    hit = int(np.argmax(v > 0))
    assert hit > 0 and v[hit] == pytest.approx(-v[hit - 1], rel=0.05)


# ---------------------------------------------------------------------------------------------------------------
# solver invariants

def test_normal_impulses_non_negative(oracle):
    """Accumulated normal impulses are clamped at 0 (contact_solver.py:194-290), over a pile of boxes."""
    s, m, st = scene_defs.build_test_scene("pile", iterations=(8, 3))
    st = wd.batch(st, 4)
    for _ in range(60):
        oracle.step_(m, st, s, F32(1 / 60))
        ct = st.contacts
        npts = (np.arange(2)[None, None, :] < ct.count[..., None]) & (ct.pair >= 0)[..., None]
        assert (ct.normal_impulse[npts] >= 0).all()


@pytest.mark.parametrize("mu,slides", [(0.5, False), (0.1, True)])
def test_box_on_incline(oracle, mu, slides):
    """Coulomb friction: on a slope of angle th a box sticks when tan th < mu, else slides with acceleration
    g (sin th - mu cos th); both fixtures carry mu so the mixed friction sqrt(mu mu) is mu."""
    th, g = 0.3, 10.0
    d = wd.WorldDef(S.stock(gravity=(0, -g)))
    ground = d.add_body(wd.STATIC, (0, 0), th)
    d.add_box(ground, (20, 0.5), friction=mu)
    n = np.array([-np.sin(th), np.cos(th)])
    box = d.add_body(wd.DYNAMIC, tuple(n * (0.5 + 0.25)), th, mass=1, inertia=1 / 24)
    d.add_box(box, (0.25, 0.25), friction=mu)
    t_hat = np.array([np.cos(th), np.sin(th)])
    pos = []
    run(d, 120, capacity=4, oracle=oracle, dt=F32(1 / 60),
        each=lambda k, s: pos.append(float(np.dot(s.bodies.c[0, box].astype(np.float64), t_hat))))
    x = np.array(pos[30:])
    if not slides:
        assert abs(x[-1] - x[0]) < 1e-3
    else:
        acc = np.polyfit(np.arange(len(x)) / 60.0, x, 2)[0] * 2
        assert acc == pytest.approx(-g * (np.sin(th) - mu * np.cos(th)), rel=0.03)


def test_momentum_conserved_in_free_collision(oracle):
    """Two free boxes collide in zero gravity: total linear momentum is unchanged by the contact impulses (equal and
    opposite, applied to both bodies) to float32 accuracy; so is angular momentum about the origin, since both
    impulses act at the same world point. Position iterations are off: their projection moves the centres (not the
    centre of mass) without a matching velocity change, which is Box2D's behaviour but not a conserved quantity."""
    d = wd.WorldDef(S.stock(gravity=(0, 0), position_iterations=0))
    a = d.add_body(wd.DYNAMIC, (-1.0, 0.05), velocity=(4, 0), angular_velocity=0.5, mass=2, inertia=0.3)
    d.add_box(a, (0.3, 0.2), friction=0.6)
    b = d.add_body(wd.DYNAMIC, (1.0, -0.05), velocity=(-3, 0.5), angular_velocity=-1.0, mass=1, inertia=0.1)
    d.add_box(b, (0.25, 0.25), friction=0.6)
    m = np.array([2.0, 1.0])
    inertia = np.array([0.3, 0.1])

    def momenta(st):
        v = st.bodies.v[0].astype(np.float64)
        c = st.bodies.c[0].astype(np.float64)
        w = st.bodies.w[0].astype(np.float64)
        p = (m[:, None] * v).sum(0)
        L = float((inertia * w + m * (c[:, 0] * v[:, 1] - c[:, 1] * v[:, 0])).sum())
        return p, L
    model, state = d.build(4)
    p0, L0 = momenta(wd.batch(state, 1))
    touched = []
    _, st = run(d, 60, capacity=4, oracle=oracle, dt=F32(1 / 60),
                each=lambda k, s: touched.append(bool(s.contacts.touching[0].any())))
    p1, L1 = momenta(st)
    assert any(touched)
    assert np.allclose(p1, p0, atol=1e-4 * np.abs(p0).sum())
    assert L1 == pytest.approx(L0, abs=1e-5)


# ---------------------------------------------------------------------------------------------------------------
# joints   (test_box2d_reference.py:90-127)

def test_pendulum_conserves_energy_and_joint(oracle):
    d = wd.WorldDef(S.game())
    pivot = d.add_body(wd.STATIC)
    L, m, inertia = 2.0, 1.0, 0.01
    bob = d.add_body(wd.DYNAMIC, (L, 0), mass=m, inertia=inertia)
    d.add_revolute(pivot, bob, (0, 0), (-L, 0))
    trace = []
    run(d, 240, capacity=2, oracle=oracle,
        each=lambda k, s: trace.append((s.bodies.c[0, bob].astype(np.float64), s.bodies.v[0, bob].astype(np.float64))))
    lowest = None
    for c, v in trace:
        assert abs(np.hypot(*c) - L) < 1e-3
        if lowest is None and c[0] <= 0:
            lowest = v
    assert lowest is not None
    assert np.hypot(*lowest) == pytest.approx(np.sqrt(2 * 30 * L / (1 + inertia / (m * L * L))), rel=0.03)


@pytest.mark.parametrize("v24", [True, False])
def test_revolute_limit_and_motor(oracle, v24):
    d = wd.WorldDef(S.game(gravity=(0, 0), revolute_v24=v24))
    pivot = d.add_body(wd.STATIC)
    arm = d.add_body(wd.DYNAMIC, (1, 0), mass=1, inertia=0.1)
    d.add_revolute(pivot, arm, (0, 0), (-1, 0), limits=(-0.5, 0.5), motor_speed=2.0, max_motor_torque=1000,
                   enable_motor=True)
    model, st = run(d, 12, capacity=2, oracle=oracle)
    assert st.bodies.w[0, arm] == pytest.approx(2.0, rel=1e-4)
    for _ in range(120):
        oracle.step_(model, st, d.settings, H)
    assert st.joints.limit_state[0, 0] == 2  # AT_UPPER
    assert st.bodies.a[0, arm] == pytest.approx(0.5, abs=float(b2.settings.deg2rad(2)))


def test_prismatic_limit_holds(oracle):
    """A prismatic joint along x with limits keeps the body on the axis and within [lower, upper] (+ slop)."""
    d = wd.WorldDef(S.stock(gravity=(0, -10)))
    g = d.add_body(wd.STATIC)
    box = d.add_body(wd.DYNAMIC, (0, 0), velocity=(5, 0), mass=1, inertia=0.1)
    d.add_prismatic(g, box, (0, 0), (0, 0), axis=(1, 0), limits=(-1.0, 1.0))
    ys, xs = [], []
    run(d, 120, capacity=2, oracle=oracle, dt=F32(1 / 60),
        each=lambda k, s: (ys.append(float(s.bodies.c[0, box, 1])), xs.append(float(s.bodies.c[0, box, 0]))))
    assert max(abs(y) for y in ys) < 0.01
    assert max(xs) < 1.0 + 0.05 and max(xs) > 0.9


def test_weld_keeps_relative_pose(oracle):
    """A rigid weld joint holds two boxes' relative pose while the pair falls and spins."""
    d = wd.WorldDef(S.stock(gravity=(0, -10)))
    a = d.add_body(wd.DYNAMIC, (0, 0), angular_velocity=2.0, mass=1, inertia=0.1)
    b = d.add_body(wd.DYNAMIC, (1, 0), mass=1, inertia=0.1)
    d.add_weld(a, b, (0.5, 0), (-0.5, 0))
    _, st = run(d, 90, capacity=2, oracle=oracle, dt=F32(1 / 60))
    c = st.bodies.c[0].astype(np.float64)
    ang = st.bodies.a[0].astype(np.float64)
    assert np.hypot(*(c[1] - c[0])) == pytest.approx(1.0, abs=5e-3)
    assert ang[1] - ang[0] == pytest.approx(0.0, abs=1e-2)


@pytest.mark.parametrize("kind,v24", [("revolute", True), ("revolute", False), ("prismatic", True),
                                      ("prismatic", False), ("weld", True)])
def test_joint_velocity_rows_solve_the_constraint(oracle, kind, v24):
    """A joint that is its island's only constraint is solved exactly by each velocity iteration's rows
    (joints.py:61-622; no motor, no limit): after every step, the relative velocity the joint forbids vanishes at the
    anchors and transforms the solver used (the step's start). Revolute (v2.4.1 and 2.3.1): the anchor points move
    together, vB + wB x rB - vA - wA x rA = 0. Prismatic: no velocity across the axis and no relative spin,
    perp . (vB - vA) + s2 wB - s1 wA = 0 and wB - wA = 0 with s1 = (d + rA) x perp, s2 = rB x perp. Weld: both. Two
    spinning dynamic bodies fall under gravity, so every mass and inertia term of the rows' effective mass enters."""
    d = wd.WorldDef(S.stock(gravity=(0, -9.81), revolute_v24=v24))
    a = d.add_body(wd.DYNAMIC, (0, 0), 0.2, (0.3, 0.0), 2.0, mass=1, inertia=0.1)
    b = d.add_body(wd.DYNAMIC, (1, -0.5), 0.2, (0.5, 1.0), -1.5, mass=2, inertia=0.3)
    la, lb = np.array([0.5, -0.25]), np.array([-0.5, 0.25])
    getattr(d, "add_" + kind)(a, b, tuple(la), tuple(lb))
    model, st = d.build(2)
    st = wd.batch(st, 1)

    def cross_sv(w, r):
        return np.array([-w * r[1], w * r[0]])

    def rot(ang, v):
        c, s = np.cos(ang), np.sin(ang)
        return np.array([c * v[0] - s * v[1], s * v[0] + c * v[1]])
    for _ in range(60):
        before = oracle.copy(st).bodies
        oracle.step_(model, st, d.settings, F32(1 / 60))
        bd = st.bodies
        aA, aB = float(before.a[0, a]), float(before.a[0, b])
        rA, rB = rot(aA, la), rot(aB, lb)
        vA, vB = bd.v[0, a].astype(np.float64), bd.v[0, b].astype(np.float64)
        wA, wB = float(bd.w[0, a]), float(bd.w[0, b])
        tol = 2e-5 * (1 + np.abs(vA).sum() + np.abs(vB).sum() + abs(wA) + abs(wB))
        if kind in ("revolute", "weld"):
            assert np.abs(vB + cross_sv(wB, rB) - vA - cross_sv(wA, rA)).max() <= tol
        if kind in ("prismatic", "weld"):
            assert abs(wB - wA) <= tol
        if kind == "prismatic":
            perp = rot(aA, np.array([0.0, 1.0]))
            dd = before.c[0, b].astype(np.float64) + rB - before.c[0, a].astype(np.float64) - rA
            s1 = (dd + rA)[0] * perp[1] - (dd + rA)[1] * perp[0]
            s2 = rB[0] * perp[1] - rB[1] * perp[0]
            assert abs(np.dot(perp, vB - vA) + s2 * wB - s1 * wA) <= tol


# ---------------------------------------------------------------------------------------------------------------
# continuous collision   (test_box2d_reference.py:130-155, test_toi.py:23-35)

def _bullet_through_wall(oracle, continuous=False, unity=True):
    d = wd.WorldDef(S.game(gravity=(0, 0), unity_toi=unity))
    wall = d.add_body(wd.STATIC, (0, 0))
    d.add_box(wall, (0.05, 2))
    ball = d.add_body(wd.DYNAMIC, (-1, 0), velocity=(240, 0), mass=1, inertia=0.01, continuous=continuous)
    d.add_circle(ball, 0.05)
    _, st = run(d, 3, capacity=4, oracle=oracle)
    return float(st.bodies.c[0, ball, 0])


def test_toi_pair_rules(oracle):
    assert _bullet_through_wall(oracle) > 0  # Unity rule: a discrete body tunnels
    assert _bullet_through_wall(oracle, continuous=True) < 0  # a Continuous body is stopped
    assert _bullet_through_wall(oracle, unity=False) < 0  # stock rule: every dynamic-vs-static pair gets TOI


def test_toi_tie_rule(oracle):
    """b2World::SolveTOI's minimum over the contact list (toi.py:552-556): of equal TOIs the stock rule takes the
    first contact in list order (the newest, the larger key) and toi_tie_oldest the last. In scene_toi_tie the two
    contacts' TOIs are equal to the bit (mirror images), and with one event allowed per step the event's contact
    (toi.count) is the one the rule names. Swapping which fixture the rule favours mirrors the whole outcome, so the
    two runs are mirror images of each other to the bit: the tie, not a difference of TOIs, decided."""
    out = {}
    for oldest in (False, True):
        s = S.stock(gravity=(0, 0), continuous_physics=True, toi_tie_oldest=oldest, max_events=1)
        model, st = scene_defs.scene_toi_tie(s).build(4)
        st = wd.batch(st, 1)
        dt = F32(1.0 / 60.0)
        for k in range(3):
            oracle.step_(model, st, s, dt)
            assert int(st.toi.events[0]) == (1 if k == 2 else 0)
        keys, counts = st.contacts.key[0, :2], st.toi.count[0, :2]
        assert sorted(st.contacts.fa[0, :2].tolist()) == [0, 1] and keys[0] != keys[1]
        named = int(np.argmin(keys) if oldest else np.argmax(keys))
        assert counts[named] == 1 and counts[1 - named] == 0
        out[oldest] = st
    a, b = out[False], out[True]
    assert a.bodies.c[0, 1, 0] != 0
    assert np.array_equal(a.bodies.c[0, 1] * F32([-1, 1]), b.bodies.c[0, 1])
    assert np.array_equal(a.bodies.v[0, 1] * F32([-1, 1]), b.bodies.v[0, 1])


def test_toi_island_membership(oracle):
    """b2World::SolveTOI's island walk (toi.py:604-716) skips a dynamic neighbour unless the walked body or the
    neighbour is a bullet. In scene_toi_plank the ball's TOI event (the second step) presses it into the plank it
    touches: with no bullet the plank stays out of the TOI island, so it ends the event step exactly as with
    continuous physics off (at rest: it never moves in Solve); with either body a bullet it joins, takes an impulse,
    and the two bullet choices give the same step to the bit (the rule is symmetric in the two bodies)."""
    def plank_after(cont, **bullets):
        s = S.stock(gravity=(0, 0), continuous_physics=cont)
        model, st = scene_defs.scene_toi_plank(s, **bullets).build(8)
        st = wd.batch(st, 1)
        for k in range(2):
            oracle.step_(model, st, s, F32(1 / 60))
            assert int(st.toi.events[0]) == (1 if (cont and k == 1) else 0)
        return st.bodies.c[0, 1].copy(), st.bodies.v[0, 1].copy(), st.bodies.c[0, 2].copy()
    c_off, v_off, _ = plank_after(False)
    c, v, ball = plank_after(True)
    assert ball[0] < 2.3  # the ball was stopped at the face, not tunnelled
    assert np.array_equal(c, c_off) and np.array_equal(v, v_off) and not v.any()
    c_b, v_b, _ = plank_after(True, ball_bullet=True)
    c_p, v_p, _ = plank_after(True, plank_bullet=True)
    assert v_b[1] < -1.0  # pressed down by the ball in the TOI velocity solve
    assert np.array_equal(c_b, c_p) and np.array_equal(v_b, v_p)


def wake_cascade_run(step, st, xy_newer):
    """Drive scene_wake_cascade (one world, numpy State `st`, `step(st)` advances it in place): step until Y and Z
    sleep, move the sleeping Z 0.04 m toward Y (inside its fat box, so that the Y-Z contact would touch if updated),
    then step until X first touches Y and once more. Returns [(Z awake, Y-Z touching)] for those last two steps."""
    X, Z = (2, 0) if xy_newer else (0, 2)
    bd = st.bodies
    for k in range(60):
        if not bd.awake[0, 1] and not bd.awake[0, Z]:
            break
        step(st)
    assert bd.awake[0, X] and not bd.awake[0, 1] and not bd.awake[0, Z]
    for leaf in (bd.c, bd.c0, bd.xf_p):
        leaf[0, Z, 0] -= F32(0.04)  # Z lies right of Y

    def touching(b1, b2):
        ct = st.contacts
        for i in range(ct.pair.shape[1]):
            bs = {int(ct.fa[0, i]), int(ct.fb[0, i])}  # one fixture per body here: fixture i is body i
            if ct.pair[0, i] >= 0 and bs == {b1, b2}:
                return bool(ct.touching[0, i])
        raise AssertionError("contact missing")
    out = []
    for k in range(60):
        step(st)
        if touching(X, 1):
            out.append((bool(bd.awake[0, Z]), touching(1, Z)))
            step(st)
            out.append((bool(bd.awake[0, Z]), touching(1, Z)))
            return out
    raise AssertionError("X never reached Y")


@pytest.mark.parametrize("xy_newer", [True, False])
def test_collide_wake_cascade_in_list_order(oracle, xy_newer):
    """b2ContactManager::Collide (pairs.py:38-117) walks the contact list newest first and skips a contact whose
    bodies are both asleep; an update whose touching flips wakes both bodies, which later contacts of the same walk
    see and earlier ones do not. In scene_wake_cascade, in the step where X first touches the sleeping Y: when the
    X-Y contact is the newer, the walk wakes Y before it reaches Y-Z, which then touches and wakes Z in that same
    step; when it is the older, Y-Z was passed over asleep, so Z sleeps through that step and wakes in the next."""
    s = S.stock(gravity=(0, 0))
    model, st = scene_defs.scene_wake_cascade(s, xy_newer).build(8)
    st = wd.batch(st, 1)
    got = wake_cascade_run(lambda x: oracle.step_(model, x, s, F32(1 / 60)), st, xy_newer)
    assert got == ([(True, True), (True, True)] if xy_newer else [(False, False), (True, True)])


def test_toi_off_tunnels(oracle):
    d = wd.WorldDef(S.game(gravity=(0, 0), continuous_physics=False))
    wall = d.add_body(wd.STATIC)
    d.add_box(wall, (0.05, 2))
    ball = d.add_body(wd.DYNAMIC, (-1, 0), velocity=(240, 0), mass=1, inertia=0.01, continuous=True)
    d.add_circle(ball, 0.05)
    _, st = run(d, 3, capacity=4, oracle=oracle)
    assert st.bodies.c[0, ball, 0] > 0 and int(st.toi.events[0]) == 0


def _sweep_xf(sw, t):
    lc, c0, c, a0, a = sw[0:2], sw[2:4], sw[4:6], sw[6], sw[7]
    cc = (1 - t) * c0 + t * c
    aa = (1 - t) * a0 + t * a
    q = np.array([np.cos(aa), np.sin(aa)])
    p = cc - np.array([q[0] * lc[0] - q[1] * lc[1], q[1] * lc[0] + q[0] * lc[1]])
    return np.array([p[0], p[1], q[0], q[1]], np.float32)


def test_time_of_impact_head_on_circles_root_steps(oracle):
    """b2TimeOfImpact's root finder (toi.py:420-446) alternates bisection and secant steps, bisection first, and stops
    once |s(t) - target| < tol = slop / 4. Two circles closing head-on without rotation have a separation linear in
    t, s(t) = s0 - t travel, so the outcome is fixed in closed form: t = 1/2 when s(1/2) is already within tol of the
    target, else the secant step that follows lands on the root, t = (s0 - target) / travel, to float rounding
    (where the contract alone would allow any t within tol of distance). Random speeds, directions and radii, plus
    roots placed just beside 1/2 on either side of the tolerance."""
    d = wd.WorldDef(S.stock())
    g = d.add_body(wd.STATIC)
    for r in (0.05, 0.1, 0.3):
        d.add_circle(g, r)
    model, _ = d.build(2)
    slop = float(S.stock().linear_slop)
    tol = 0.25 * slop
    rng = np.random.default_rng(21)
    halves = roots = 0
    for trial in range(240):
        fa, fb = (int(x) for x in rng.integers(0, 3, 2))
        ra, rb = float(model.radius[fa]), float(model.radius[fb])
        target = max(slop, ra + rb - 3 * slop)
        u = rng.normal(size=2)
        u /= np.linalg.norm(u)
        travel = rng.uniform(2.5, 6.0)
        if trial % 4 == 0:  # the root beside 1/2: inside the tolerance, or just outside it
            gap = target + travel * 0.5 + rng.choice([-0.6, 0.6, -1.6, 1.6]) * tol
        else:
            gap = target + travel * rng.uniform(0.1, 0.9)
        pa = rng.uniform(-1, 1, 2)
        pb0 = pa + u * gap
        pb1 = pb0 - u * travel
        sa = np.array([0, 0, pa[0], pa[1], pa[0], pa[1], 0, 0], np.float32)
        sb = np.array([0, 0, pb0[0], pb0[1], pb1[0], pb1[1], 0, 0], np.float32)
        st, t = oracle.time_of_impact(model, fa, fb, sa, sb, slop)
        assert st == 3, (trial, st)  # TOUCHING
        # the proxies are the centres; the points separation function's axis is their direction at t = 0
        p0, p1, q = sb[2:4].astype(np.float64), sb[4:6].astype(np.float64), sa[2:4].astype(np.float64)
        axis = (p0 - q) / np.linalg.norm(p0 - q)
        s0, trav = float(np.dot(p0 - q, axis)), float(np.dot(p0 - p1, axis))
        miss = abs(s0 - 0.5 * trav - target)
        if abs(miss - tol) < 1e-5:
            continue  # too near the stopping test's edge for float64 to say which side float32 took
        if miss < tol:
            assert t == 0.5, (trial, t)
            halves += 1
        else:
            assert t == pytest.approx((s0 - target) / trav, rel=2e-6, abs=2e-7), (trial, t)
            roots += 1
    assert halves >= 20 and roots >= 150


def test_time_of_impact_contract(oracle):
    """b2TimeOfImpact: when it reports TOUCHING at t, the core shapes' distance at t is within target +- tol, target
    = max(slop, r_A + r_B - 3 slop), tol = slop / 4 (toi.py:372-375); when it reports SEPARATED at t = 1 they never
    came within target."""
    d = wd.WorldDef(S.stock())
    g = d.add_body(wd.STATIC)
    d.add_box(g, (0.5, 0.1))
    d.add_polygon(g, [(0, 0), (1, 0.2), (0.3, 0.8)])
    p = d.add_body(wd.DYNAMIC, (0, 3), mass=1, inertia=0.1)
    d.add_box(p, (0.2, 0.05))
    d.add_circle(p, 0.1, center=(0.3, 0))
    model, _ = d.build(4)
    slop = float(S.stock().linear_slop)
    rng = np.random.default_rng(7)
    touching = separated = 0
    for trial in range(300):
        fa = int(rng.integers(0, 2))
        fb = 2 + int(rng.integers(0, 2))
        ra, rb = float(model.radius[fa]), float(model.radius[fb])
        target = max(slop, ra + rb - 3 * slop)
        c0 = rng.uniform([-2, 1.5], [2, 3])
        c1 = rng.uniform([-1, -1.5], [1, 0.5])
        a0, a1 = rng.uniform(-3, 3), rng.uniform(-6, 6)
        sa = np.array([0, 0, 0, 0, 0, 0, 0, 0], np.float32)
        sb = np.array([0, 0, c0[0], c0[1], c1[0], c1[1], a0, a1], np.float32)
        state, t = oracle.time_of_impact(model, fa, fb, sa, sb, F32(slop))
        tol = 0.25 * slop
        dist = oracle.distance(model, fa, fb, _sweep_xf(sa, t), _sweep_xf(sb.astype(np.float64), t))
        if state == 3 and t > 0:  # reached by the root finder: the separation function is within target +- tol
            assert target - tol - 1e-4 <= dist < target + tol + 1e-4, (trial, t, dist, target)
            touching += 1
        elif state == 3:  # already closer than target + tol at t = 0 (but not overlapping)
            assert 0 < dist < target + tol + 1e-4
        elif state == 4:  # separated at the end of the sweep along the final axis, so the distance there exceeds it
            assert t == 1.0 and dist > target + tol - 1e-4
            separated += 1
    assert touching > 50 and separated > 20


# ---------------------------------------------------------------------------------------------------------------
# distance (GJK) and narrowphase vs brute force

def _poly_world(model, f, xf):
    n = int(model.count[f])
    v = model.verts[f, :n].astype(np.float64)
    c, s = float(xf[2]), float(xf[3])
    return np.stack([c * v[:, 0] - s * v[:, 1] + xf[0], s * v[:, 0] + c * v[:, 1] + xf[1]], 1)


def _seg_dist(p, a, b):
    ab = b - a
    t = np.clip(np.dot(p - a, ab) / max(np.dot(ab, ab), 1e-300), 0, 1)
    return float(np.linalg.norm(p - (a + t * ab)))


def _inside(p, poly):
    n = len(poly)
    return n >= 3 and all(_cross(poly[(i + 1) % n] - poly[i], p - poly[i]) >= 0 for i in range(n))


def _cross(a, b):
    return a[0] * b[1] - a[1] * b[0]


def _poly_dist(A, B):
    """Exact distance between convex polygons (vertex lists, CCW; 1 vertex = point): 0 if they overlap (no
    separating edge normal, or a point inside the polygon), else the minimum vertex-to-edge distance both ways."""
    if len(A) >= 3 and len(B) >= 3 and max(_sat(A, B), _sat(B, A)) <= 0:
        return 0.0
    if (len(B) == 1 and _inside(B[0], A)) or (len(A) == 1 and _inside(A[0], B)):
        return 0.0

    def edges(P):
        return [(P[i], P[(i + 1) % len(P)]) for i in range(len(P))] if len(P) > 1 else [(P[0], P[0])]
    dmin = min(_seg_dist(p, a, b) for p in A for (a, b) in edges(B))
    return min(dmin, min(_seg_dist(p, a, b) for p in B for (a, b) in edges(A)))


def _sat(A, B):
    """max over A's faces of min over B's vertices of the face separation (b2FindMaxSeparation, exhaustive)."""
    best = -np.inf
    for i in range(len(A)):
        e = A[(i + 1) % len(A)] - A[i]
        nrm = np.array([e[1], -e[0]]) / np.linalg.norm(e)
        best = max(best, min(np.dot(nrm, v - A[i]) for v in B))
    return best


@pytest.fixture(scope="module")
def shape_model():
    d = wd.WorldDef(S.stock())
    g = d.add_body(wd.STATIC)
    d.add_box(g, (0.6, 0.3))
    d.add_polygon(g, [(0, 0), (1, 0.2), (0.3, 0.8)])
    d.add_polygon(g, [(0, 0), (0.5, -0.1), (0.9, 0.3), (0.6, 0.7), (0.1, 0.6)])
    d.add_circle(g, 0.3)
    d.add_circle(g, 0.15, center=(0.2, -0.1))
    model, _ = d.build(2)
    return model


def _rand_xf(rng, spread=1.5):
    a = rng.uniform(-np.pi, np.pi)
    p = rng.uniform(-spread, spread, 2)
    return np.array([p[0], p[1], np.cos(a), np.sin(a)], np.float32)


def test_gjk_distance_vs_exhaustive(oracle, shape_model):
    m = shape_model
    rng = np.random.default_rng(11)
    for trial in range(400):
        fa, fb = (int(x) for x in rng.integers(0, 5, 2))
        xa, xb = _rand_xf(rng), _rand_xf(rng)
        got = oracle.distance(m, fa, fb, xa, xb)
        want = _poly_dist(_poly_world(m, fa, xa), _poly_world(m, fb, xb))
        if want == 0.0:
            assert got <= 1e-3, (trial, got)
        else:
            assert got == pytest.approx(want, abs=5e-5 + 5e-5 * want), (trial, fa, fb, got, want)


def _xf(x, y, a=0.0):
    return np.array([x, y, np.cos(F32(a)), np.sin(F32(a))], np.float32)


def test_polygon_manifold_known_answers(oracle):
    """b2CollidePolygons (collide.py:65-127) worked by hand on three box contacts, from the algorithm's definition:
    the reference face is A's unless B's separates by more than k_tol = 0.1 slop (then FACE_B and each point's
    feature swaps its A and B halves); the incident edge is the one of the other polygon most anti-parallel to the
    reference normal, its vertices keyed (reference edge, incident vertex, face, vertex); clipping against the
    reference face's side planes keys a new point (side vertex iv1 or iv2, the incoming point's vertex, vertex,
    face); key = indexA | indexB << 8 | typeA << 16 | typeB << 24 with vertex 0 and face 1 (collide.py:22-24).
    Boxes are b2PolygonShape::SetAsBox's: vertices (-h,-h), (h,-h), (h,h), (-h,h), edge i from vertex i.

    - rest: the unit box 0.015 above a (10, 0.5) slab. Reference A edge 2 (the slab's top), incident B edge 0,
      nothing clipped: (2, 0, F, V) = 65538 and (2, 1, F, V) = 65794 at B's vertices 0 and 1.
    - flip: the unit box turned 0.3 rad, its lowest corner (vertex 0) 0.01 above the slab, as fixture A. The box's
      faces separate from the slab's far corners by about -3 m, the slab's top by 0.01, so FACE_B; incident box
      edge 0; vertex 1 lies 0.31 above and drops out; one point, (2, 0, F, V) swapped to (0, 2, V, F) = 16777728.
    - clip: the unit box resting 0.01 above a (0.3, 0.3) box (A). Reference A edge 2 from (0.3, 0.3) to
      (-0.3, 0.3); B's edge 0 spans x = -0.5..0.5 and is clipped at x = +-(0.3 + 2 skins): side plane iv1 = 2 keys
      (2, 0, V, F) = 16777218 at x = 0.32, then iv2 = 3 keys (3, 0, V, F) = 16777219 at x = -0.32.
    - the k_tol hysteresis: with the unit box on the small one turned by t, B's face separates 0.2 t more than A's;
      t = 0.001 (0.0002 < k_tol) keeps FACE_A, t = 0.004 (0.0008) gives FACE_B, either sign of t.
    """
    d = wd.WorldDef(S.stock())
    g = d.add_body(wd.STATIC)
    d.add_box(g, (10, 0.5))
    d.add_box(g, (0.5, 0.5))
    d.add_box(g, (0.3, 0.3))
    model, _ = d.build(2)
    slop = S.stock()
    rest = oracle.evaluate(model, 0, 1, _xf(0, 0), _xf(0, 1.015), slop)
    assert (rest["mtype"], rest["count"]) == (1, 2) and rest["point_id"].tolist() == [65538, 65794]
    assert np.array_equal(rest["local_normal"], [0, 1]) and np.array_equal(rest["local_point"], [0, 0.5])
    assert np.array_equal(rest["point_local"], [[-0.5, -0.5], [0.5, -0.5]])
    t = 0.3
    flip = oracle.evaluate(model, 1, 0, _xf(0, 0.51 + 0.5 * (np.sin(t) + np.cos(t)), t), _xf(0, 0), slop)
    assert (flip["mtype"], flip["count"]) == (2, 1) and int(flip["point_id"][0]) == 16777728
    assert np.array_equal(flip["local_normal"], [0, 1]) and np.array_equal(flip["local_point"], [0, 0.5])
    assert np.allclose(flip["point_local"][0], [-0.5, -0.5], atol=1e-6)
    clip = oracle.evaluate(model, 2, 1, _xf(0, 0), _xf(0, 0.81), slop)
    assert (clip["mtype"], clip["count"]) == (1, 2) and clip["point_id"].tolist() == [16777218, 16777219]
    assert np.allclose(clip["point_local"], [[0.32, -0.5], [-0.32, -0.5]], atol=1e-6)
    for t, mtype in ((0.001, 1), (-0.001, 1), (0.004, 2), (-0.004, 2)):
        y = 0.31 + 0.5 * (np.cos(t) + abs(np.sin(t)))
        assert oracle.evaluate(model, 2, 1, _xf(0, 0), _xf(0, y, t), slop)["mtype"] == mtype, t


def test_narrowphase_vs_brute_force(oracle, shape_model):
    """Manifold point count against exhaustive geometry: circles touch iff |c1 - c2| <= r1 + r2; polygon-circle iff
    the centre is within r_p + r_c of the polygon; polygon pairs: no points when the exhaustive face separation
    exceeds r_A + r_B, some point when the true distance is below it; every manifold point's separation is at
    most r_A + r_B and no deeper than the exhaustive overlap allows."""
    m = shape_model
    rng = np.random.default_rng(12)
    slop = F32(0.005)
    seen = {"cc": [0, 0], "pc": [0, 0], "pp": [0, 0]}
    for trial in range(3000):
        fa, fb = (int(x) for x in rng.integers(0, 5, 2))
        ta, tb = int(m.shape_type[fa]), int(m.shape_type[fb])
        if ta == CIRCLE and tb == POLYGON:  # the contact always puts the polygon first
            fa, fb, ta, tb = fb, fa, tb, ta
        xa, xb = _rand_xf(rng, 0.8), _rand_xf(rng, 0.8)
        man = oracle.evaluate(m, fa, fb, xa, xb, slop)
        A, B = _poly_world(m, fa, xa), _poly_world(m, fb, xb)
        r = float(m.radius[fa]) + float(m.radius[fb])
        dist = _poly_dist(A, B)
        if abs(dist - r) < 1e-3:
            continue
        if ta == CIRCLE and tb == CIRCLE:
            kind = "cc"
            assert man["count"] == (1 if dist <= r else 0)
        elif tb == CIRCLE:
            kind = "pc"
            assert man["count"] == (1 if dist <= r else 0), (trial, dist, r, man)
        else:
            kind = "pp"
            sep = max(_sat(A, B), _sat(B, A))
            if sep > r + 1e-4:
                assert man["count"] == 0
            if dist < r - 1e-4:
                assert man["count"] >= 1
        seen[kind][man["count"] > 0] += 1
    assert all(a > 30 and b > 30 for a, b in seen.values()), seen


# ---------------------------------------------------------------------------------------------------------------
# broadphase: FindNewContacts vs a brute-force scan of the candidate list   (world.py:308-329, pairs.py:134-178)

def _overlap(a, b):
    return not (b[0] - a[2] > 0 or b[1] - a[3] > 0 or a[0] - b[2] > 0 or a[1] - b[3] > 0)


@pytest.mark.parametrize("cfg", [1, 3])
def test_find_new_contacts_vs_brute_force(oracle, cfg):
    """From an empty contact table, FindNewContacts creates exactly the candidates whose fat AABBs overlap (one body
    dynamic and awake-or-not, both active), in candidate order: the r-th overlapping candidate takes slot r and key
    next_key + r. Integer equality with a plain scan of Model.pair_a/pair_b."""
    s, model, state, c = b2.scenes.make_config(cfg, 64)
    st = oracle.copy(state)
    fat = wd.expand_state(model, st).fixtures.fat  # [N, F, 4] lower x, lower y, upper x, upper y
    oracle.collide_(model, st, s)
    pa, pb = np.asarray(model.pair_a), np.asarray(model.pair_b)
    fb_ = np.asarray(model.fixture_body)
    btype = np.asarray(state.bodies.type)
    for w in range(state.bodies.type.shape[0]):
        f = fat[w]
        want = []
        for p in range(pa.shape[0]):
            a, b = int(pa[p]), int(pb[p])
            if btype[w, fb_[a]] != wd.DYNAMIC and btype[w, fb_[b]] != wd.DYNAMIC:
                continue
            if _overlap(f[a], f[b]):
                want.append(p)
        C = st.contacts.pair.shape[1]
        got_pairs = st.contacts.pair[w]
        keep = want[:C]
        # Collide may destroy a fresh contact only if its fat AABBs stopped overlapping, which they cannot here.
        assert got_pairs[:len(keep)].tolist() == keep, w
        assert (got_pairs[len(keep):] == -1).all()
        assert st.contacts.key[w, :len(keep)].tolist() == list(range(len(keep)))
        assert int(st.next_key[w]) == len(keep)
        assert int(st.overflow[w]) == max(0, len(want) - C)


def test_find_new_contacts_keys_follow_candidate_order(oracle):
    """Later FindNewContacts calls (one per step with TOI off): surviving contacts keep their slot and key, and the
    contacts created in one call take keys next_key, next_key + 1, ... in candidate (pair index) order."""
    import dataclasses
    s, m, st0 = scene_defs.build_test_scene("pile", iterations=(8, 3))
    s = dataclasses.replace(s, continuous_physics=False)
    st = wd.batch(st0, 1)
    oracle.step_(m, st, s, F32(1 / 60))
    created = 0
    for _ in range(60):
        bp, bk, nk = st.contacts.pair[0].copy(), st.contacts.key[0].copy(), int(st.next_key[0])
        oracle.step_(m, st, s, F32(1 / 60))
        ap, ak = st.contacts.pair[0], st.contacts.key[0]
        kept = (bp >= 0) & (ap >= 0) & (ak < nk)
        assert (ap[kept] == bp[kept]).all() and (ak[kept] == bk[kept]).all()
        new = np.nonzero((ap >= 0) & (ak >= nk))[0]
        by_key = new[np.argsort(ak[new])]
        assert ak[by_key].tolist() == list(range(nk, nk + len(new)))
        assert ap[by_key].tolist() == sorted(ap[by_key].tolist())
        assert int(st.next_key[0]) == nk + len(new)
        created += len(new)
    assert created > 5


# ---------------------------------------------------------------------------------------------------------------
# islands: a plain sequential DFS from the rules of b2World::Solve   (island.py:1-19)

def _dfs_islands(model, st, w):
    """body_island, contact_order from the rules: seeds in descending body index (awake, active, not static,
    unvisited); pop LIFO; each popped body walks its touching contacts newest first (descending key), then its
    joints newest first (descending index); static bodies are never expanded."""
    bd, ct = st.bodies, st.contacts
    B, C = bd.type.shape[1], ct.pair.shape[1]
    fbody = np.asarray(model.fixture_body)
    isl = [-1] * B
    c_in = [False] * C
    order = []
    n = 0
    for seed in range(B - 1, -1, -1):
        if isl[seed] >= 0 or not bd.awake[w, seed] or not bd.active[w, seed] or bd.type[w, seed] == wd.STATIC:
            continue
        stack = [seed]
        isl[seed] = n
        while stack:
            b = stack.pop()
            if bd.type[w, b] == wd.STATIC:
                continue
            edges = [k for k in range(C) if ct.pair[w, k] >= 0 and ct.touching[w, k]
                     and b in (fbody[ct.fa[w, k]], fbody[ct.fb[w, k]])]
            for k in sorted(edges, key=lambda k: -int(ct.key[w, k])):
                if c_in[k]:
                    continue
                c_in[k] = True
                order.append(k)
                ba, bb = fbody[ct.fa[w, k]], fbody[ct.fb[w, k]]
                other = bb if ba == b else ba
                if isl[other] < 0 and bd.type[w, other] != wd.STATIC:
                    isl[other] = n
                    stack.append(other)
            for j in range(model.joint_type.shape[0] - 1, -1, -1):
                ja, jb = int(model.joint_a[j]), int(model.joint_b[j])
                if b not in (ja, jb):
                    continue
                other = jb if ja == b else ja
                if not bd.active[w, other]:
                    continue
                if isl[other] < 0 and bd.type[w, other] != wd.STATIC:
                    isl[other] = n
                    stack.append(other)
        n += 1
    return isl, order, n


@pytest.mark.parametrize("scene", ["pile", "joints", "island_walk"])
def test_islands_vs_sequential_dfs(oracle, scene):
    s, m, st0 = scene_defs.build_test_scene(scene, iterations=(8, 3))
    st = wd.batch(st0, 1)
    B, R, J, C = wd.dims(st)
    checked = 0
    for k in range(60):
        pre = oracle.copy(st)
        dbg = dict(body_island=np.zeros((B, 1), np.int32), contact_island=np.zeros((C, 1), np.int32),
                   contact_order=np.zeros((C, 1), np.int32), n_islands=np.zeros(1, np.int32))
        oracle.collide_(m, pre, s)  # the contact table Solve sees: after FindNewContacts and Collide
        oracle.step_(m, st, s, F32(1 / 60), debug=dbg)
        isl, order, n = _dfs_islands(m, pre, 0)
        if n == 0:
            continue
        assert dbg["n_islands"][0] == n
        assert dbg["body_island"][:, 0].tolist() == [i if pre.bodies.type[0, b] != wd.STATIC else -1
                                                     for b, i in enumerate(isl)]
        assert dbg["contact_order"][:len(order), 0].tolist() == order
        checked += 1
    assert checked > 10


# ---------------------------------------------------------------------------------------------------------------
# position rows: one pass of non-linear Gauss-Seidel   (contact_solver.py:307-354, joints.py:462-606)
#
# A position row moves its bodies by M^-1 J^T lambda, lambda chosen so that the constraint error, linearized at the
# current pose, becomes the row's target (zero for a joint's point and angle rows; the Baumgarte-scaled, slop-shifted
# and clamped separation for a contact point and a limit). These pins step one world once with no velocity pass and
# one position pass, a static body A and a dynamic body B placed with a known error, so that B's move is exactly that
# pass; they then check the two defining conditions on B's move (dc, da): the linearized error after it, and the
# direction M^-1 J^T (a rotation iB / mB times the moment of the linear move about the anchor). These conditions fix
# the move whatever the formula; a wrong effective mass, a sign, a dropped clamp or slop changes it.

def _pass_settings(**kw):
    import dataclasses
    return dataclasses.replace(S.stock(gravity=(0.0, 0.0), **kw), velocity_iterations=0, position_iterations=1,
                               allow_sleep=False)


def _one_pass(oracle, d, settings, body=1, capacity=4):
    """(c, a) of `body` before and after one step of a single world, float64."""
    model, state = d.build(capacity)
    cm = wd.compact_model(model, state)
    st = wd.batch(wd.compact_state(cm, state), 1)
    before = (st.bodies.c[0, body].astype(np.float64), float(st.bodies.a[0, body]))
    oracle.step_(cm, st, settings, F32(1 / 60))
    return before, (st.bodies.c[0, body].astype(np.float64), float(st.bodies.a[0, body])), st


def _rot(a, v):
    c, s = np.cos(np.float64(F32(a))), np.sin(np.float64(F32(a)))
    return np.array([c * v[0] - s * v[1], s * v[0] + c * v[1]])


def _perp(r):
    return np.array([-r[1], r[0]])


def _cross(a, b):
    return a[0] * b[1] - a[1] * b[0]


@pytest.mark.parametrize("v24", [True, False])
def test_revolute_point_row_is_one_newton_step(oracle, v24):
    """The revolute point row (joints.py:501-520, both solver versions): B's anchor misses A's by e = (0.04, -0.03),
    B's anchor offset rB = R(0.7)(0.6, 0.25), inverse mass 0.5, inverse inertia 4. After the pass the linearized
    anchor gap C + dc + da perp(rB) is zero and da = (iB / mB) cross(rB, dc)."""
    s = _pass_settings(revolute_v24=v24)
    d = wd.WorldDef(s)
    anchor = np.array([0.3, -0.2])
    a = d.add_body(wd.STATIC, tuple(anchor))
    lb, ang, e = (0.6, 0.25), 0.7, np.array([0.04, -0.03])
    rb = _rot(ang, lb)
    b = d.add_body(wd.DYNAMIC, tuple(anchor - rb + e), ang, mass=2.0, inertia=0.25)
    d.add_revolute(a, b, (0, 0), lb)
    (c0, a0), (c1, a1), _ = _one_pass(oracle, d, s)
    dc, da = c1 - c0, a1 - a0
    C = c0 + rb - anchor
    assert np.linalg.norm(C - e) < 1e-6 and np.linalg.norm(dc) > 1e-3
    assert np.linalg.norm(C + dc + da * _perp(rb)) < 2e-6
    assert abs(da - (4.0 / 0.5) * _cross(rb, dc)) < 2e-5


# (offset of the joint angle from the limit, limits) -> the angle after the pass: a violation beyond the slop is
# pulled back to the slop, a large one by at most max_angular_correction, equal limits to the limit itself
_LIMIT_CASES = [("below", -0.08, (-0.5, 0.4)), ("below_far", -0.5, (-0.5, 0.4)), ("above", 0.08, (-0.5, 0.4)),
                ("above_far", 0.5, (-0.5, 0.4)), ("inside", 0.3, (-0.5, 0.4)), ("equal", 0.05, (0.2, 0.2)),
                ("equal_far", 0.7, (0.2, 0.2))]


@pytest.mark.parametrize("v24", [True, False])
@pytest.mark.parametrize("name,off,limits", _LIMIT_CASES, ids=[c[0] for c in _LIMIT_CASES])
def test_revolute_limit_row(oracle, v24, name, off, limits):
    """The revolute limit row (joints.py:462-498): with B's anchor at its centre (rB = 0, so the point row leaves the
    angle alone) and static A, one pass moves the joint angle to lower - angular_slop (upper + slop) when it was
    below (above) by more than the slop, by at most max_angular_correction (8 degrees) when far, to the limit when
    lower == upper, and not at all inside the limits."""
    s = _pass_settings(revolute_v24=v24)
    lo, hi = limits
    ref = 0.1
    angle = (lo if off < 0 or name.startswith("equal") else hi if off > 0 and name != "inside" else 0.0) + off
    if name == "inside":
        angle = off
    d = wd.WorldDef(s)
    a = d.add_body(wd.STATIC, (1.0, 2.0))
    b = d.add_body(wd.DYNAMIC, (1.0, 2.0), ref + angle, mass=2.0, inertia=0.25)
    d.add_revolute(a, b, (0, 0), (0, 0), ref, limits=limits)
    (c0, a0), (c1, a1), _ = _one_pass(oracle, d, s)
    got = a1 - ref
    start = a0 - ref
    slop, mac = float(s.angular_slop), float(s.max_angular_correction)
    want = {"below": lo - slop, "below_far": start + mac, "above": hi + slop, "above_far": start - mac,
            "inside": start, "equal": lo, "equal_far": start - mac}[name]
    assert abs(got - want) < 2e-6, (got, want)
    assert np.array_equal(c1, c0)


@pytest.mark.parametrize("case", ["free", "lower", "lower_far", "upper"])
def test_prismatic_position_row(oracle, case):
    """The prismatic position row (joints.py:523-566): axis u at 0.7 rad on static A, B off the axis by 0.03, turned
    0.04 past the reference angle, at translation t along u. After the pass, the linearized perpendicular gap and
    angle error are zero: perp.d + perp.dc + cross(rB, perp) da = 0 and angle + da = 0; a slider inside its limits
    gets no impulse along u (u.dc = 0), one beyond a limit has its linearized translation change
    u.dc + cross(rB, u) da equal to minus the limit row's target clamp((t - lower) + slop, -0.2, 0) (or the upper
    one)."""
    s = _pass_settings()
    th = 0.7
    u = np.array([np.cos(th), np.sin(th)])
    pp = _perp(u)
    la, lb, ref = np.array([0.1, -0.2]), (0.2, -0.1), 0.3
    t = {"free": 0.4, "lower": -0.6, "lower_far": -1.2, "upper": 1.1}[case]
    lo, hi = -0.5, 1.0
    d = wd.WorldDef(s)
    a = d.add_body(wd.STATIC, (0.0, 0.0))
    ab = ref + 0.04
    rb = _rot(ab, lb)
    c_b = la + t * u + 0.03 * pp - rb
    b = d.add_body(wd.DYNAMIC, tuple(c_b), ab, mass=2.0, inertia=0.25)
    d.add_prismatic(a, b, tuple(la), lb, (np.cos(th), np.sin(th)), ref, limits=(lo, hi))
    (c0, a0), (c1, a1), _ = _one_pass(oracle, d, s)
    dc, da = c1 - c0, a1 - a0
    dvec = c0 + rb - la
    assert abs(pp @ dvec + pp @ dc + _cross(rb, pp) * da) < 3e-6
    assert abs((a0 - ref) + da) < 2e-6
    along = u @ dc + _cross(rb, u) * da
    tt = u @ dvec
    slop, mlc = float(s.linear_slop), float(s.max_linear_correction)
    if case == "free":
        assert abs(u @ dc) < 3e-6  # no impulse along the axis
    elif case == "upper":
        assert abs(along + min(max((tt - hi) - slop, 0.0), mlc)) < 3e-6
    else:
        assert abs(along + min(max((tt - lo) + slop, -mlc), 0.0)) < 3e-6
    assert np.linalg.norm(dc) > 1e-3


@pytest.mark.parametrize("soft", [False, True])
def test_weld_position_row(oracle, soft):
    """The weld position row (joints.py:569-595): B's anchor misses A's by (0.04, -0.03) and B is turned 0.05 past
    the reference angle. Rigid: the linearized anchor gap and angle error are both zero after the pass (three
    conditions for three unknowns). Soft (frequency > 0): only the anchor gap is corrected, along M^-1 J^T of the
    point row: da = (iB / mB) cross(rB, dc)."""
    s = _pass_settings()
    d = wd.WorldDef(s)
    anchor = np.array([-0.4, 0.5])
    a = d.add_body(wd.STATIC, tuple(anchor))
    lb, ref = (0.5, 0.3), 0.2
    ab = ref + 0.05
    rb = _rot(ab, lb)
    e = np.array([0.04, -0.03])
    b = d.add_body(wd.DYNAMIC, tuple(anchor - rb + e), ab, mass=2.0, inertia=0.25)
    d.add_weld(a, b, (0, 0), lb, ref, frequency=4.0 if soft else 0.0, damping=0.5)
    (c0, a0), (c1, a1), _ = _one_pass(oracle, d, s)
    dc, da = c1 - c0, a1 - a0
    C = c0 + rb - anchor
    assert np.linalg.norm(C + dc + da * _perp(rb)) < 3e-6
    if soft:
        assert abs(da - (4.0 / 0.5) * _cross(rb, dc)) < 2e-5
    else:
        assert abs((a0 - ref) + da) < 2e-6


@pytest.mark.parametrize("depth,clamped", [(0.03, False), (1.3, True)])
def test_contact_position_row_circle(oracle, depth, clamped):
    """The contact position row (contact_solver.py:307-354) on a circle (radius 1.5, inverse mass 1) embedded `depth`
    in a static slab's top face: separation sep = -depth - 0.01 (the slab's skin); the one point's target is
    clamp(baumgarte (sep + linear_slop), -max_linear_correction, 0) with Baumgarte 0.2 in Solve (not the TOI's 0.75);
    the contact point is the circle's centre, so the circle rises by exactly minus the target and does not turn."""
    s = _pass_settings()
    d = wd.WorldDef(s)
    g = d.add_body(wd.STATIC, (0.0, -0.5))
    d.add_box(g, (10.0, 0.5))
    r = 1.5
    b = d.add_body(wd.DYNAMIC, (0.0, r - depth), mass=1.0, inertia=1.0)
    d.add_circle(b, r)
    (c0, a0), (c1, a1), _ = _one_pass(oracle, d, s)
    sep = c0[1] - r - float(s.polygon_radius)
    target = min(max(float(s.baumgarte) * (sep + float(s.linear_slop)), -float(s.max_linear_correction)), 0.0)
    assert (target == -float(s.max_linear_correction)) == clamped
    assert abs((c1[1] - c0[1]) + target) < 1e-6 and c1[0] == c0[0] and a1 == a0


def test_contact_position_row_tilted_box(oracle):
    """The contact position row with rotation: a box (half extents 0.5 x 0.25, inverse mass 0.5, inverse inertia 10)
    turned 0.4 rad with its lowest corner 0.04 into a slab (one manifold point: the next corner is 0.35 above).
    The corner p is the contact point, n = +y, rB = p - cB. After the pass: dc is along n, da = (iB / mB)
    cross(rB, dc), and the corner's linearized rise n.dc + da n.perp(rB) equals minus the target
    clamp(0.2 (sep + slop), -0.2, 0), sep = -0.04 - 2 skins."""
    s = _pass_settings()
    d = wd.WorldDef(s)
    g = d.add_body(wd.STATIC, (0.0, -0.5))
    d.add_box(g, (10.0, 0.5))
    th, half = 0.4, (0.5, 0.25)
    corner = _rot(th, (-half[0], -half[1]))
    b = d.add_body(wd.DYNAMIC, (0.0, -corner[1] - 0.04), th, mass=2.0, inertia=0.1)
    d.add_box(b, half)
    (c0, a0), (c1, a1), st = _one_pass(oracle, d, s)
    assert int(st.contacts.count[0][st.contacts.pair[0] >= 0][0]) == 1
    dc, da = c1 - c0, a1 - a0
    rb = _rot(a0, (-half[0], -half[1]))
    sep = (c0[1] + rb[1]) - 2 * float(s.polygon_radius)
    target = min(max(0.2 * (sep + float(s.linear_slop)), -0.2), 0.0)
    assert abs(dc[0]) < 1e-7 and dc[1] > 1e-3
    assert abs(da - (10.0 / 0.5) * _cross(rb, dc)) < 2e-5
    assert abs(dc[1] + da * rb[0] + target) < 2e-6


# ---------------------------------------------------------------------------------------------------------------
# the block solver's condition test   (contact_solver.py:116-130)

def test_block_solver_condition_fallback(oracle):
    """A two-point contact uses the 2x2 block solver only while K is well conditioned (k11^2 < 1000 det K), else
    only its first point (contact_solver.py:116-130). A box 0.002 m wide on a slab has two manifold points 0.002 m
    apart: with inverse mass and inertia 1, det K = 4e-6 against k11^2 = 1, so one point carries the whole weight and
    the second point's normal impulse stays 0. A box 1 m wide (det K = 1) uses both points."""
    out = {}
    for name, hx in (("narrow", 0.001), ("wide", 0.5)):
        s = S.stock(gravity=(0.0, -10.0))
        d = wd.WorldDef(s)
        g = d.add_body(wd.STATIC, (0.0, -0.5))
        d.add_box(g, (10.0, 0.5))
        b = d.add_body(wd.DYNAMIC, (0.0, 0.2 + 0.015), mass=1.0, inertia=1.0)
        d.add_box(b, (hx, 0.2))
        model, state = d.build(4)
        st = wd.batch(state, 1)
        oracle.step_(model, st, s, F32(1 / 60))
        k = int(np.nonzero(st.contacts.pair[0] >= 0)[0][0])
        assert int(st.contacts.count[0, k]) == 2
        out[name] = st.contacts.normal_impulse[0, k]
    assert out["narrow"][0] > 0 and out["narrow"][1] == 0
    assert out["wide"][0] > 0 and out["wide"][1] > 0


# ---------------------------------------------------------------------------------------------------------------
# b2CollidePolygons under exact ties   (collide.py:32-42, 65-127)

def test_polygon_manifold_exact_ties(oracle):
    """Known answers worked by hand where the running maxima tie exactly (b2FindMaxSeparation keeps the first of equal
    separations, the incident edge search the first of equal dot products):

    - two unit boxes at the same pose: all eight face separations are -1, so the reference face is A's edge 0
      (normal -y, local point (0, -0.5)), no flip (B's -1 is not more than A's -1 + k_tol); B's incident edge is
      edge 2 (normal +y), both its vertices survive the side planes: points (0.5, 0.5) and (-0.5, 0.5) of B, keys
      (0, 2, F, V) = 66048 and (0, 3, F, V) = 66304;
    - a diamond (vertices (0.3, 0), (0, 0.3), (-0.3, 0), (0, -0.3)) centred on the top face of a unit box: A's top
      face (edge 2) separates by -0.3, the diamond's faces by -0.566; the diamond's lower edges 2 and 3 are equally
      anti-parallel to +y (normals (-k, -k) and (k, -k)), so edge 2 is incident: points (-0.3, 0) and (0, -0.3) of B
      (its vertices 2 and 3), keys (2, 2, F, V) = 66050 and (2, 3, F, V) = 66306."""
    d = wd.WorldDef(S.stock())
    g = d.add_body(wd.STATIC)
    d.add_box(g, (0.5, 0.5))
    d.add_box(g, (0.5, 0.5))
    d.add_polygon(g, [(0.3, 0.0), (0.0, 0.3), (-0.3, 0.0), (0.0, -0.3)], raw=True)
    model, _ = d.build(2)
    s = S.stock()
    same = oracle.evaluate(model, 0, 1, _xf(0.7, -0.4), _xf(0.7, -0.4), s)
    assert (same["mtype"], same["count"]) == (1, 2) and same["point_id"].tolist() == [66048, 66304]
    assert np.array_equal(same["local_normal"], [0, -1]) and np.array_equal(same["local_point"], [0, -0.5])
    assert np.allclose(same["point_local"], [[0.5, 0.5], [-0.5, 0.5]], atol=1e-6)  # rounding of the world round trip
    dia = oracle.evaluate(model, 0, 2, _xf(0.0, 0.0), _xf(0.0, 0.5), s)
    assert (dia["mtype"], dia["count"]) == (1, 2) and dia["point_id"].tolist() == [66050, 66306]
    assert np.array_equal(dia["local_normal"], [0, 1]) and np.array_equal(dia["local_point"], [0, 0.5])
    assert np.allclose(dia["point_local"], [[-0.3, 0.0], [0.0, -0.3]], atol=1e-7)


# ---------------------------------------------------------------------------------------------------------------
# the TOI event's island walk: order and contact cap   (toi.py:604-716)

def plank_over_bumps(n_bumps=40, capacity=48):
    """A flat plank (half extents 5.2 x 0.05) falling at 60 m/s onto a row of n_bumps equal static bumps 0.25 m
    apart, continuous physics on, one TOI event per step: the event's walk meets every bump's contact touching."""
    s = S.stock(gravity=(0.0, 0.0), continuous_physics=True, max_events=1)
    d = wd.WorldDef(s)
    g = d.add_body(wd.STATIC)
    for i in range(n_bumps):
        d.add_box(g, (0.05, 0.05), ((i - (n_bumps - 1) / 2) * 0.25, 0.0))
    p = d.add_body(wd.DYNAMIC, (0.0, 0.5), velocity=(0.0, -60.0), mass=1.0, inertia=1.0)
    d.add_box(p, (5.2, 0.05))
    model, state = d.build(capacity)
    cm = wd.compact_model(model, state)
    return s, cm, wd.batch(wd.compact_state(cm, state), 1)


def toi_trace(n, dims):
    return {k: np.full(shape, -7, np.int32) for k, shape in b2.debug_shapes(n, dims).items()}


def test_toi_island_walk_order_and_cap(oracle):
    """b2World::SolveTOI's island walk (toi.py:604-716): the event's contact is row 0, then bodyA's contacts and then
    bodyB's, each list newest first (descending key), skipping contacts already in the island and those that do not
    touch after the update, until the island holds b2_maxTOIContacts = 32 contacts. Here bodyA is the static ground
    (not walked) and bodyB the plank, whose 40 bump contacts all touch at the event's pose: the rows are the event's
    contact and then the 31 newest others. toi.solved marks exactly those 32 contacts. (The island's body cap,
    2 x 32, can never bind: each row adds at most one body to the pair.)"""
    s, m, st = plank_over_bumps()
    B, R, J, C = wd.dims(st)
    dbg = toi_trace(1, (B, R, J, C))
    oracle.step_(m, st, s, F32(1 / 60), debug=dbg)
    assert int(st.toi.events[0]) == 1
    slot = int(dbg["toi_event_slot"][0, 0])
    rows = dbg["toi_island_rows"][:32, 0].tolist()
    live = np.nonzero(st.contacts.pair[0] >= 0)[0]
    assert len(live) == 40 and slot in live.tolist()
    newest_first = sorted(live.tolist(), key=lambda c: -int(st.contacts.key[0, c]))
    want = [slot] + [c for c in newest_first if c != slot][:31]
    assert rows == want
    assert int(dbg["toi_event_island"][0, 0]) == 32 | (2 << 16)
    assert np.nonzero(st.toi.solved[0])[0].tolist() == sorted(want)
    assert dbg["toi_event_slot"][1:, 0].tolist() == [-1] * 7


# ---------------------------------------------------------------------------------------------------------------
# revolute velocity rows: the motor and the limits   (joints.py:257-343)
#
# With B's anchor at its centre (rB = 0) on a static A, the point row leaves B's spin alone, so one velocity pass
# (no position pass) shows the motor and limit rows alone in B's angular velocity after the step: the motor row
# drives the relative spin to the motor speed unless its accumulated impulse reaches max_motor_torque * dt; the
# v2.4.1 limits are speculative, their impulses never negative: a joint closing on a limit at distance C ahead ends
# the pass at -C / dt (it reaches the limit exactly at the step's end), one moving away is left alone; the v2.3.1
# limit at AT_LOWER / AT_UPPER stops the relative spin into the limit and releases a joint moving out of it.

_VEL_CASES = [  # (name, v24, angle offset from a limit, w0, motor (speed, max torque) or None, expected w)
    ("motor", True, None, -2.0, (3.0, 1000.0), lambda h: 3.0),
    ("motor_v23", False, None, -2.0, (3.0, 1000.0), lambda h: 3.0),
    ("motor_saturated", True, None, -2.0, (3.0, 6.0), lambda h: -2.0 + 4.0 * 6.0 * h),
    ("lower_closing", True, ("lower", 0.02), -5.0, None, lambda h: -0.02 / h),
    ("upper_closing", True, ("upper", -0.02), 5.0, None, lambda h: 0.02 / h),
    ("lower_opening", True, ("lower", 0.02), 1.0, None, lambda h: 1.0),
    ("at_lower_v23", False, ("lower", -0.01), -5.0, None, lambda h: 0.0),
    ("leaving_lower_v23", False, ("lower", -0.01), 2.0, None, lambda h: 2.0),
    ("at_upper_v23", False, ("upper", 0.01), 5.0, None, lambda h: 0.0),
]


@pytest.mark.parametrize("name,v24,where,w0,motor,want", _VEL_CASES, ids=[c[0] for c in _VEL_CASES])
def test_revolute_velocity_rows(oracle, name, v24, where, w0, motor, want):
    import dataclasses
    s = dataclasses.replace(S.stock(gravity=(0.0, 0.0), revolute_v24=v24), velocity_iterations=1,
                            position_iterations=0, allow_sleep=False)
    lo, hi, ref = -0.3, 0.5, 0.1
    angle = 0.0 if where is None else (lo if where[0] == "lower" else hi) + where[1]
    d = wd.WorldDef(s)
    a = d.add_body(wd.STATIC, (0.5, 0.5))
    b = d.add_body(wd.DYNAMIC, (0.5, 0.5), ref + angle, angular_velocity=w0, mass=2.0, inertia=0.25)
    kw = {} if motor is None else dict(motor_speed=motor[0], max_motor_torque=motor[1], enable_motor=True)
    d.add_revolute(a, b, (0, 0), (0, 0), ref, limits=None if where is None else (lo, hi), **kw)
    h = F32(1 / 60)
    model, state = d.build(4)
    st = wd.batch(state, 1)
    oracle.step_(model, st, s, h)
    assert abs(float(st.bodies.w[0, 1]) - want(float(h))) < 2e-5


# ---------------------------------------------------------------------------------------------------------------
# SynchronizeFixtures' re-fatten rule   (pairs.py:181-207, shapes.py:136-146; b2DynamicTree::MoveProxy)
#
# A body that moved has its fixture's swept AABB (the union of the AABBs at the sweep start (c0, a0) and at the
# new transform) checked against its fat AABB. If the fat box still holds it, nothing changes. Otherwise the new fat
# box is the swept box extended by b2_aabbExtension = 0.1 on every side, and then by b2_aabbMultiplier = 2 times the
# transform's displacement on the side the body moved to. A circle centred on its body has the AABB p +- r, so with
# no gravity and no contacts every number is fixed by the step's integration (semi-implicit Euler, pinned above).

def _moved_circle(oracle, p, v, r=0.5, dt=F32(1 / 60)):
    s = S.stock(gravity=(0.0, 0.0))
    d = wd.WorldDef(s)
    b = d.add_body(wd.DYNAMIC, p, velocity=v, mass=1.0, inertia=1.0)
    d.add_circle(b, r)
    model, state = d.build(4)
    cm = wd.compact_model(model, state)
    st = wd.batch(wd.compact_state(cm, state), 1)
    fat0 = st.fixtures.fat[0, 0].copy()
    oracle.step_(cm, st, s, dt)
    return fat0, st.bodies.xf_p[0, 0].copy(), st.bodies.c0[0, 0].copy(), st.fixtures.fat[0, 0].copy()


_SYNC_MOVES = [((0.25, 5.0), (12.0, -7.0)), ((-3.0, 1.0), (-15.0, 9.5)), ((7.5, -2.0), (0.5, 30.0)),
               ((0.0, 0.0), (-8.0, -0.25))]


@pytest.mark.parametrize("p,v", _SYNC_MOVES)
def test_synchronize_fixtures_refattens_a_moved_box(oracle, p, v):
    r = F32(0.5)
    fat0, p1, p0, fat = _moved_circle(oracle, p, v, r)
    assert np.array_equal(p0, np.array(p, F32))  # the sweep start is the step's start
    lo = np.minimum(p0 - r, p1 - r)
    hi = np.maximum(p0 + r, p1 + r)
    assert not (np.all(fat0[:2] <= lo) and np.all(hi <= fat0[2:]))  # the move leaves the old fat box
    e, d = F32(0.1), (p1 - p0).astype(F32)
    lo, hi = (lo - e).astype(F32), (hi + e).astype(F32)
    for i in range(2):
        dd = F32(F32(2.0) * d[i])
        if dd < 0:
            lo[i] = F32(lo[i] + dd)
        else:
            hi[i] = F32(hi[i] + dd)
    assert np.array_equal(fat, np.concatenate([lo, hi])), (fat, lo, hi)


@pytest.mark.parametrize("v", [(3.0, 1.0), (-5.5, 0.0), (0.0, -5.9)])
def test_synchronize_fixtures_keeps_a_fat_box_that_still_holds(oracle, v):
    """A move of under 0.1 m keeps the swept AABB inside the fat box from b2BroadPhase::CreateProxy (the AABB
    +- 0.1): the fat box stays the same to the bit."""
    fat0, p1, p0, fat = _moved_circle(oracle, (0.25, 5.0), v)
    assert 0 < np.abs(p1 - p0).max() < 0.1
    assert np.array_equal(fat, fat0)


# ---------------------------------------------------------------------------------------------------------------
# the TOI island's position passes   (toi.py:719-760; b2Island::SolveTOI)
#
# A circle (radius 0.5, no gravity) flies head-on into a static slab's face and would pass through it in one step.
# b2TimeOfImpact stops it where the core shapes are target = r_total - 3 slop apart, so the contact's separation is
# -3 slop (-0.015) at the event. Only the TOI pair has mass; the contact point lies on the line through the circle's
# centre along the normal, so the effective mass is the circle's inverse mass and each pass moves the circle by
# exactly -clamp(b (sep + slop), -max_linear_correction, 0) along the normal, b = toi_baumgarte, sep measured before
# the pass. A pass that measured sep >= -1.5 slop is the last one (its correction still applies). The TOI velocity
# pass then stops the circle (restitution 0), so it ends the step at the solved pose.
#
# With the stock b = 0.75 the second pass measures -0.0075 = -1.5 slop (the scheme is built to land there), so its
# outcome turns on the last bit of the TOI root; b = 0.6 keeps every decision 1e-3 away from its threshold.

def test_toi_position_passes_closed_form(oracle):
    s = S.stock(gravity=(0.0, 0.0), continuous_physics=True, toi_baumgarte=0.6)
    d = wd.WorldDef(s)
    g = d.add_body(wd.STATIC, (3.0, 0.0))
    d.add_box(g, (0.5, 2.0))  # face at x = 2.5, skin 0.01
    x0, vx, r = F32(1.2), F32(110.0), 0.5
    b = d.add_body(wd.DYNAMIC, (x0, 0.0), velocity=(vx, 0.0), mass=1.0, inertia=1.0)
    d.add_circle(b, r)
    model, state = d.build(4)
    cm = wd.compact_model(model, state)
    st = wd.batch(wd.compact_state(cm, state), 1)
    dbg = toi_trace(1, wd.dims(st))
    h = F32(1 / 60)
    oracle.step_(cm, st, s, h, debug=dbg)
    assert int(st.toi.events[0]) == 1
    alpha = dbg["toi_event_alpha"][0, 0].view(np.float32)
    x1 = F32(x0 + F32(h * vx))  # Solve's integration
    x = float(F32(x0 + F32(alpha * F32(x1 - x0))))  # b2Sweep::Advance to the event
    slop, b_toi = float(s.linear_slop), float(s.toi_baumgarte)
    seps = []
    for _ in range(20):
        sep = (2.5 - x) - (r + float(s.polygon_radius))
        seps.append(sep)
        x += max(b_toi * (sep + slop), -float(s.max_linear_correction))
        if sep >= -1.5 * slop:
            break
    assert abs(seps[0] + 3 * slop) < 2e-4  # the TOI target
    assert len(seps) == 3 and min(abs(q + 1.5 * slop) for q in seps) > 5e-4
    assert abs(float(st.bodies.c[0, 1, 0]) - x) < 2e-6, (st.bodies.c[0, 1, 0], x)
    assert st.bodies.c[0, 1, 1] == 0 and st.bodies.a[0, 1] == 0
    assert np.array_equal(st.bodies.c0[0, 1], st.bodies.c[0, 1])  # the leap of faith
    assert np.all(st.bodies.v[0, 1] == 0) and st.bodies.w[0, 1] == 0


# ---------------------------------------------------------------------------------------------------------------
# warm start's dtRatio   (contact_solver.py:165-184, step.py:34)
#
# b2ContactSolver scales the stored impulses by dtRatio = dt * inv_dt0 before warm-starting; with no velocity
# iteration StoreImpulses writes those scaled values back. At dt = 1/64 (inv_dt0 = 64 exactly) followed by a step of
# 1/128, dtRatio is exactly 1/2, so every stored impulse halves to the bit.

def test_warm_start_scales_impulses_by_dt_ratio(oracle):
    import dataclasses
    s = dataclasses.replace(S.stock(), allow_sleep=False)
    d = wd.WorldDef(s)
    g = d.add_body(wd.STATIC, (0.0, -0.5))
    d.add_box(g, (10.0, 0.5))
    b = d.add_body(wd.DYNAMIC, (0.0, 0.5), mass=2.0, inertia=F32(2) / F32(6))
    d.add_box(b, (0.5, 0.5))
    model, state = d.build(4)
    cm = wd.compact_model(model, state)
    st = wd.batch(wd.compact_state(cm, state), 1)
    for _ in range(20):
        oracle.step_(cm, st, s, F32(1 / 64))
    assert float(st.inv_dt0[0]) == 64.0
    ct = st.contacts
    k = int(np.nonzero((ct.pair[0] >= 0) & ct.touching[0])[0][0])
    ni, ti, ids = ct.normal_impulse[0, k].copy(), ct.tangent_impulse[0, k].copy(), ct.point_id[0, k].copy()
    assert int(ct.count[0, k]) == 2 and np.all(ni > 0.1)
    oracle.step_(cm, st, dataclasses.replace(s, velocity_iterations=0), F32(1 / 128))
    assert np.array_equal(ct.point_id[0, k], ids)  # the same features: the impulses carry over
    assert np.array_equal(ct.normal_impulse[0, k], ni * F32(0.5))
    assert np.array_equal(ct.tangent_impulse[0, k], ti * F32(0.5))
    assert float(st.inv_dt0[0]) == 128.0


# ---------------------------------------------------------------------------------------------------------------
# Solve's rotation clamp   (step.py:117-135)
#
# A free body whose step would turn it by more than max_rotation (stock pi/2) has its angular velocity scaled by
# max_rotation / |h w|: it turns by exactly max_rotation (to float rounding) and keeps the scaled spin.

@pytest.mark.parametrize("w0", [200.0, -150.0, 95.0])
def test_rotation_clamp(oracle, w0):
    s = S.stock(gravity=(0.0, 0.0))
    d = wd.WorldDef(s)
    b = d.add_body(wd.DYNAMIC, (0.0, 0.0), 0.3, angular_velocity=w0, mass=1.0, inertia=1.0)
    d.add_box(b, (0.5, 0.5))
    model, state = d.build(4)
    cm = wd.compact_model(model, state)
    st = wd.batch(wd.compact_state(cm, state), 1)
    h = F32(1 / 60)
    oracle.step_(cm, st, s, h)
    turn, max_r = float(st.bodies.a[0, 0]) - float(F32(0.3)), float(s.max_rotation)
    assert abs(float(h) * w0) > max_r
    assert abs(turn - np.sign(w0) * max_r) < 1e-6
    assert float(st.bodies.w[0, 0]) == pytest.approx(np.sign(w0) * max_r / float(h), rel=1e-6)
    assert np.all(st.bodies.v[0, 0] == 0)


def test_rotation_below_the_clamp_is_untouched(oracle):
    s = S.stock(gravity=(0.0, 0.0))
    d = wd.WorldDef(s)
    b = d.add_body(wd.DYNAMIC, (0.0, 0.0), 0.3, angular_velocity=90.0, mass=1.0, inertia=1.0)
    d.add_box(b, (0.5, 0.5))
    model, state = d.build(4)
    cm = wd.compact_model(model, state)
    st = wd.batch(wd.compact_state(cm, state), 1)
    h = F32(1 / 60)
    oracle.step_(cm, st, s, h)
    assert st.bodies.w[0, 0] == F32(90.0) and st.bodies.a[0, 0] == F32(F32(0.3) + F32(h * F32(90.0)))


# ---------------------------------------------------------------------------------------------------------------
# the position iterations' per-island exit   (step.py:197-251)
#
# Each island stops after the first position pass whose smallest separation is at least -3 slop and whose joints
# are within tolerance (that pass's corrections apply). Two boxes rest on one static slab, so they form two islands:
# box A overlaps the slab by 0.0125 (separation -0.0125, within -3 slop at the first pass), box B by 0.05. With no
# gravity and no velocity neither moves before the position passes. Box A must end the step exactly as with one
# position iteration, whatever the iteration count; box B keeps correcting.

def _two_islands(oracle, iterations):
    import dataclasses
    s = dataclasses.replace(S.stock(gravity=(0.0, 0.0)), position_iterations=iterations, allow_sleep=False)
    d = wd.WorldDef(s)
    g = d.add_body(wd.STATIC, (0.0, -0.5))
    d.add_box(g, (10.0, 0.5))
    a = d.add_body(wd.DYNAMIC, (-3.0, 0.5 + 0.0075), mass=1.0, inertia=0.2)  # separation 0.0075 - 2 skins
    d.add_box(a, (0.5, 0.5))
    bb = d.add_body(wd.DYNAMIC, (3.0, 0.5 - 0.03), mass=1.0, inertia=0.2)
    d.add_box(bb, (0.5, 0.5))
    model, state = d.build(4)
    cm = wd.compact_model(model, state)
    st = wd.batch(wd.compact_state(cm, state), 1)
    dbg = {k: np.full(shape, -7, np.int32) for k, shape in b2.debug_shapes(1, wd.dims(st)).items()}
    oracle.step_(cm, st, s, F32(1 / 60), debug=dbg)
    return st, dbg


def test_position_iterations_exit_per_island(oracle):
    runs = {n: _two_islands(oracle, n) for n in (1, 2, 3, 8)}
    st1, dbg1 = runs[1]
    isl = dbg1["body_island"][:, 0]
    assert isl[0] == -1 and isl[1] >= 0 and isl[2] >= 0 and isl[1] != isl[2]
    pose = lambda st, b: (st.bodies.c[0, b].tobytes(), st.bodies.a[0, b].tobytes(),  # noqa: E731
                          st.bodies.xf_p[0, b].tobytes(), st.bodies.xf_q[0, b].tobytes())
    assert float(st1.bodies.c[0, 1, 1]) > 0.5 + 0.0075  # the first pass moved box A
    for n in (2, 3, 8):
        st, _ = runs[n]
        assert pose(st, 1) == pose(st1, 1), n
    ys = [float(runs[n][0].bodies.c[0, 2, 1]) for n in (1, 2, 3, 8)]
    assert all(y1 < y2 for y1, y2 in zip(ys, ys[1:]))  # box B rises with every pass


# ---------------------------------------------------------------------------------------------------------------
# settings paths and per-step bookkeeping   (step.py:28-47, 73-194; contact_solver.py:32-147, 194-290)

def _single(d, capacity=4):
    model, state = d.build(capacity)
    cm = wd.compact_model(model, state)
    return cm, wd.batch(wd.compact_state(cm, state), 1)


def test_angular_damping_closed_form(oracle):
    """b2Island::Solve's angular damping, w <- w / (1 + h c_ang), apart from the linear one: a free spinning body
    with angular damping 0.3 and linear damping 0.05 follows the float32 recurrence to the bit."""
    import dataclasses
    s = dataclasses.replace(S.stock(gravity=(0.0, 0.0)), allow_sleep=False)
    d = wd.WorldDef(s)
    b = d.add_body(wd.DYNAMIC, (0.0, 0.0), 0.0, (2.0, 0.0), 7.0, mass=1.0, inertia=1.0, linear_damping=0.05,
                   angular_damping=0.3)
    d.add_circle(b, 0.5)
    m, st = _single(d)
    h = F32(1 / 60)
    w, v = F32(7.0), F32(2.0)
    wd_, vd_ = F32(1) / (F32(1) + h * F32(0.3)), F32(1) / (F32(1) + h * F32(0.05))
    for _ in range(50):
        oracle.step_(m, st, s, h)
        w, v = w * wd_, v * vd_
        assert st.bodies.w[0, 0] == w and st.bodies.v[0, 0, 0] == v


def test_clamps_per_second(oracle):
    """Settings.clamps_per_second: max_translation and max_rotation are per second, so a step may move at most
    max_translation * h and turn at most max_rotation * h (step.py:120-135)."""
    import dataclasses
    s = dataclasses.replace(S.stock(gravity=(0.0, 0.0), max_translation=120.0, max_rotation=30.0),
                            clamps_per_second=True, allow_sleep=False)
    d = wd.WorldDef(s)
    b = d.add_body(wd.DYNAMIC, (0.0, 0.0), 0.0, (300.0, 400.0), 50.0, mass=1.0, inertia=1.0)
    d.add_box(b, (0.5, 0.5))
    m, st = _single(d)
    h = F32(1 / 60)
    oracle.step_(m, st, s, h)
    assert float(np.hypot(*st.bodies.c[0, 0])) == pytest.approx(120.0 / 60.0, rel=2e-6)
    assert float(np.hypot(*st.bodies.v[0, 0])) == pytest.approx(120.0, rel=2e-6)
    assert float(st.bodies.a[0, 0]) == pytest.approx(30.0 / 60.0, rel=2e-6)
    assert float(st.bodies.w[0, 0]) == pytest.approx(30.0, rel=2e-6)
    # the same settings without clamps_per_second: 120 m and 30 rad per step bind nothing here
    m2, st2 = _single(d)
    oracle.step_(m2, st2, dataclasses.replace(s, clamps_per_second=False), h)
    assert float(np.hypot(*st2.bodies.v[0, 0])) == pytest.approx(500.0, rel=1e-6)


def test_restitution_velocity_threshold(oracle):
    """b2VelocityConstraintPoint::velocityBias = -e vRel only when vRel < -velocity_threshold: a ball with
    restitution 1 meeting the ground at 0.5 m/s (below the stock 1 m/s threshold) stops, one at 3 m/s bounces
    back at 3 m/s."""
    for speed, bounce in ((0.5, False), (3.0, True)):
        s = S.stock(gravity=(0.0, 0.0))
        d = wd.WorldDef(s)
        g = d.add_body(wd.STATIC, (0.0, -0.5))
        d.add_box(g, (10.0, 0.5), restitution=1.0)
        b = d.add_body(wd.DYNAMIC, (0.0, 0.5 + 0.005), 0.0, (0.0, -speed), mass=1.0, inertia=1.0)
        d.add_circle(b, 0.5, restitution=1.0)
        m, st = _single(d)
        oracle.step_(m, st, s, F32(1 / 60))
        vy = float(st.bodies.v[0, 1, 1])
        assert (vy == pytest.approx(speed, rel=1e-5)) if bounce else abs(vy) < 1e-6, (speed, vy)


def test_warm_starting_off(oracle):
    """Settings.warm_starting false: every contact starts the step with zero impulses, so with no velocity iteration
    the stored impulses are zero (contact_solver.py:160-164), while warm starting keeps them (dtRatio 1)."""
    import dataclasses
    s = dataclasses.replace(S.stock(), allow_sleep=False)
    d = wd.WorldDef(s)
    g = d.add_body(wd.STATIC, (0.0, -0.5))
    d.add_box(g, (10.0, 0.5))
    b = d.add_body(wd.DYNAMIC, (0.0, 0.5), mass=2.0, inertia=F32(2) / F32(6))
    d.add_box(b, (0.5, 0.5))
    m, st = _single(d)
    for _ in range(10):
        oracle.step_(m, st, s, F32(1 / 64))
    k = int(np.nonzero(st.contacts.touching[0])[0][0])
    ni = st.contacts.normal_impulse[0, k].copy()
    assert np.all(ni > 0.1)
    on, off = oracle.copy(st), oracle.copy(st)
    oracle.step_(m, on, dataclasses.replace(s, velocity_iterations=0), F32(1 / 64))
    oracle.step_(m, off, dataclasses.replace(s, velocity_iterations=0, warm_starting=False), F32(1 / 64))
    assert np.array_equal(on.contacts.normal_impulse[0, k], ni)
    assert np.all(off.contacts.normal_impulse[0, k] == 0) and np.all(off.contacts.tangent_impulse[0, k] == 0)


def test_inv_dt0_kept_for_non_positive_dt(oracle):
    """inv_dt0 becomes 1 / dt after a step with dt > 0 and is left alone by a step with dt <= 0 (step.py:41-44),
    so the next positive step's dtRatio still refers to the last real step."""
    d, box = resting_box()
    m, st = _single(d, 8)
    oracle.step_(m, st, d.settings, F32(1 / 64))
    assert float(st.inv_dt0[0]) == 64.0
    for dt in (0.0, -0.02):
        oracle.step_(m, st, d.settings, F32(dt))
        assert float(st.inv_dt0[0]) == 64.0


def test_sleep_needs_the_position_solve(oracle):
    """An island sleeps only when its bodies have been slow for time_to_sleep and its position iterations reached
    tolerance in the step (b2Island::Solve's positionSolved; step.py:153-168). With no position iteration an island
    is never position-solved: a box at rest in zero gravity then never sleeps; with one iteration it sleeps once its
    sleep time reaches 0.5 s (31 steps of 1/60: the sleep time is the float sum of the steps)."""
    import dataclasses
    for iters, sleeps in ((0, False), (1, True)):
        s = dataclasses.replace(S.stock(gravity=(0.0, 0.0)), position_iterations=iters)
        d = wd.WorldDef(s)
        b = d.add_body(wd.DYNAMIC, (0.0, 0.0), mass=1.0, inertia=1.0)
        d.add_box(b, (0.5, 0.5))
        m, st = _single(d)
        t = F32(0)
        asleep_at = None
        for k in range(40):
            oracle.step_(m, st, s, F32(1 / 60))
            t = t + F32(1 / 60)
            if asleep_at is None and not st.bodies.awake[0, 0]:
                asleep_at = k
        assert (asleep_at is not None) == sleeps, (iters, asleep_at)
        if sleeps:
            n = 0
            acc = F32(0)
            while acc < F32(0.5):
                acc = acc + F32(1 / 60)
                n += 1
            assert asleep_at == n - 1


def test_sleep_time_resets_when_moving(oracle):
    """A body slower than the sleep tolerances accumulates sleep time; one moving faster has it reset to 0 in the
    step (step.py:153-168)."""
    s = S.stock(gravity=(0.0, 0.0))
    d = wd.WorldDef(s)
    b = d.add_body(wd.DYNAMIC, (0.0, 0.0), mass=1.0, inertia=1.0)
    d.add_box(b, (0.5, 0.5))
    m, st = _single(d)
    for _ in range(10):
        oracle.step_(m, st, s, F32(1 / 60))
    assert float(st.bodies.sleep_time[0, 0]) > 0.15
    st.bodies.v[0, 0] = (0.5, 0.0)
    oracle.step_(m, st, s, F32(1 / 60))
    assert st.bodies.sleep_time[0, 0] == 0 and st.bodies.awake[0, 0]


@pytest.mark.parametrize("v24", [True, False])
def test_joint_warm_start_scales_by_dt_ratio(oracle, v24):
    """b2RevoluteJoint::InitVelocityConstraints scales every stored impulse (point, motor, limit) by dtRatio before
    warm-starting (joints.py:151-160). A bar hanging from a static pivot against its lower limit with a weak motor
    holding it: after steps of 1/64 s (inv_dt0 = 64 exactly), one step of 1/128 s with no velocity iteration stores
    exactly half of each impulse."""
    import dataclasses
    s = dataclasses.replace(S.stock(gravity=(0.0, -10.0)), revolute_v24=v24, allow_sleep=False)
    d = wd.WorldDef(s)
    g = d.add_body(wd.STATIC, (0.0, 0.0))
    b = d.add_body(wd.DYNAMIC, (1.0, 0.0), mass=2.0, inertia=0.5)
    d.add_box(b, (1.0, 0.1))
    d.add_revolute(g, b, (0.0, 0.0), (-1.0, 0.0), limits=(-0.1, 0.1), motor_speed=0.0, max_motor_torque=3.0,
                   enable_motor=True)
    m, st = _single(d)
    for _ in range(40):
        oracle.step_(m, st, s, F32(1 / 64))
    jt = st.joints
    imp, mot = jt.impulse[0, 0].copy(), jt.motor_impulse[0, 0].copy()
    low = jt.lower_impulse[0, 0].copy()
    assert abs(float(imp[1])) > 0.1 and abs(float(mot)) > 1e-3
    assert (float(low) > 1e-3) if v24 else (abs(float(imp[2])) > 1e-3)  # resting on the lower limit
    oracle.step_(m, st, dataclasses.replace(s, velocity_iterations=0), F32(1 / 128))
    half = F32(0.5)
    assert np.array_equal(jt.impulse[0, 0, :2], imp[:2] * half)
    assert jt.motor_impulse[0, 0] == mot * half
    if v24:
        assert jt.lower_impulse[0, 0] == low * half
    else:
        assert jt.impulse[0, 0, 2] == imp[2] * half


def test_tangent_speed_drives_the_contact(oracle):
    """contacts.tangent_speed (b2Contact::m_tangentSpeed, a conveyor belt): the friction rows solve for a relative
    tangential velocity dot(vB - vA, t) equal to it, t = cross(n, 1) (contact_solver.py:252-262). A box resting on a
    high-friction slab with tangent speed 1 set on its contact moves at +1 m/s along the slab after one step (either
    fixture order gives the same sign), and at -1 m/s for tangent speed -1; the box's inertia is so large that it
    does not turn, so the first friction row reaches the target and the second finds it reached."""
    import dataclasses
    s = dataclasses.replace(S.stock(gravity=(0.0, -10.0)), allow_sleep=False)
    d = wd.WorldDef(s)
    g = d.add_body(wd.STATIC, (0.0, -0.5))
    d.add_box(g, (10.0, 0.5), friction=100.0)
    b = d.add_body(wd.DYNAMIC, (0.0, 0.5), mass=1.0, inertia=1e6)  # (nearly) no rotation: the rows decouple
    d.add_box(b, (0.5, 0.5), friction=100.0)
    m, st = _single(d)
    for _ in range(20):
        oracle.step_(m, st, s, F32(1 / 60))
    k = int(np.nonzero(st.contacts.touching[0])[0][0])
    for speed in (1.0, -1.0):
        x = oracle.copy(st)
        x.contacts.tangent_speed[0, k] = speed
        oracle.step_(m, x, s, F32(1 / 60))
        assert float(x.bodies.v[0, 1, 0]) == pytest.approx(speed, abs=1e-3)
        assert abs(float(x.bodies.w[0, 1])) < 1e-3


def test_static_body_takes_the_last_islands_awake_flag(oracle):
    """A static body shared by several islands ends the step with the awake flag of the highest-numbered island that
    included it (step.py:173-194). Islands are numbered in seed order, newest body first (island.py:8-9). Two boxes
    on one frictionless slab: body 1 drops onto it and then slides (its contact is the newer), body 2 rests on it
    from the start and falls asleep after time_to_sleep. Body 1 is seeded last, so in the step where body 2's island
    falls asleep the slab follows body 1's island and stays awake, whatever the contacts' slot order."""
    s = S.stock(gravity=(0.0, -10.0))
    d = wd.WorldDef(s)
    g = d.add_body(wd.STATIC, (0.0, -0.5))
    d.add_box(g, (50.0, 0.5), friction=0.0)
    slide = d.add_body(wd.DYNAMIC, (0.0, 1.0), velocity=(2.0, 0.0), mass=1.0, inertia=F32(1) / F32(6))
    d.add_box(slide, (0.5, 0.5), friction=0.0)
    rest = d.add_body(wd.DYNAMIC, (-20.0, 0.5), mass=1.0, inertia=F32(1) / F32(6))
    d.add_box(rest, (0.5, 0.5), friction=0.0)
    m, st = _single(d)
    for _ in range(45):
        oracle.step_(m, st, s, F32(1 / 60))
        if not st.bodies.awake[0, rest]:
            break
    live = np.nonzero(st.contacts.touching[0])[0]
    by_body = {int(m.fixture_body[st.contacts.fb[0, k]]): int(k) for k in live}
    assert by_body[rest] < by_body[slide]  # the resting box's contact holds the lower slot
    assert not st.bodies.awake[0, rest] and st.bodies.awake[0, slide]
    assert st.bodies.awake[0, g]


@pytest.mark.parametrize("kind", ["revolute_v24", "revolute_v23", "prismatic", "weld"])
def test_joint_error_keeps_position_iterations_going(oracle, kind):
    """An island stops its position iterations only once its joints report both their linear error within
    linear_slop and their angular error within angular_slop (step.py:197-251, joints.py:462-606). A bar joined to a
    static body, with no linear error and an angular error far beyond angular_slop: a revolute pivoted at the bar's
    centre 0.8 rad past its upper limit (each pass turns it back by at most max_angular_correction and moves no
    anchor, so three passes leave less error than one, and eight less than three); a prismatic or weld joint at the
    bar's end turned 0.9 rad from its reference angle (one pass
    removes the angular error but, the anchor being off the bar's centre, leaves a linear one that the second pass
    corrects: one pass and three end in different poses)."""
    import dataclasses
    s = dataclasses.replace(S.stock(gravity=(0.0, 0.0)), revolute_v24=(kind != "revolute_v23"), allow_sleep=False)

    def run(iters):
        d = wd.WorldDef(dataclasses.replace(s, position_iterations=iters))
        g = d.add_body(wd.STATIC, (0.0, 0.0))
        ang = 0.9
        c, sn = np.cos(ang), np.sin(ang)
        b = d.add_body(wd.DYNAMIC, (c, sn), ang, mass=1.0, inertia=0.3)
        d.add_box(b, (1.0, 0.1))
        if kind.startswith("revolute"):  # pivot at the bar's centre: correcting the angle moves no anchor
            d.add_revolute(g, b, (c, sn), (0.0, 0.0), limits=(-0.1, 0.1))
        elif kind == "prismatic":
            d.add_prismatic(g, b, (0.0, 0.0), (-1.0, 0.0), axis=(c, sn))
        else:
            d.add_weld(g, b, (0.0, 0.0), (-1.0, 0.0))
        m, st = _single(d)
        oracle.step_(m, st, d.settings, F32(1 / 60))
        return np.concatenate([st.bodies.c[0, 1], st.bodies.a[0, 1:2]]).astype(np.float64)
    poses = [run(n) for n in (1, 3, 8)]
    if kind.startswith("revolute"):
        errs = [abs(p[2] - 0.1) for p in poses]
        assert errs[0] > errs[1] > errs[2], errs
    else:
        assert np.abs(poses[0] - poses[1]).max() > 1e-4, poses


# ---------------------------------------------------------------------------------------------------------------
# SolveTOI's bookkeeping: the sub-step cap, re-search after a move, the island walk's restore   (toi.py:462-716)

def _ball_between_walls(speed):
    s = S.stock(gravity=(0.0, 0.0), continuous_physics=True, max_translation=100.0)
    d = wd.WorldDef(s)
    g = d.add_body(wd.STATIC, (0.0, 0.0))
    d.add_box(g, (0.1, 2.0), center=(-0.45, 0.0), restitution=1.0)
    d.add_box(g, (0.1, 2.0), center=(0.45, 0.0), restitution=1.0)
    b = d.add_body(wd.DYNAMIC, (0.0, 0.0), velocity=(speed, 0.0), mass=1.0, inertia=1.0)
    d.add_circle(b, 0.1, restitution=1.0)
    m, st = _single(d)
    return s, m, st


def test_toi_sub_step_cap_and_re_search(oracle):
    """A ball (radius 0.1, restitution 1) at 700 m/s between two walls 0.7 apart: every TOI event reflects its
    velocity exactly, and after each event the moved ball's contacts get their TOIs searched again (the wall it now
    heads to included). A contact takes events while its count is at most b2_maxSubSteps = 8, so each wall takes 9
    events: 18 in the step, then both contacts are skipped and the ball leaves through a wall at full speed."""
    s, m, st = _ball_between_walls(700.0)
    oracle.step_(m, st, s, F32(1 / 60))
    assert int(st.toi.events[0]) == 18
    live = st.contacts.pair[0] >= 0
    assert sorted(st.toi.count[0][live].tolist()) == [9, 9]
    assert abs(float(st.bodies.c[0, 1, 0])) > 0.55 and abs(float(st.bodies.v[0, 1, 0])) == 700.0
    # slower, the same cage never reaches the cap: fewer events, all of them reflections
    s, m, st = _ball_between_walls(200.0)
    oracle.step_(m, st, s, F32(1 / 60))
    assert 2 <= int(st.toi.events[0]) < 18 and abs(float(st.bodies.c[0, 1, 0])) < 0.25


def test_toi_walk_restores_a_body_it_does_not_keep(oracle):
    """The TOI island walk advances each candidate neighbour to the event's alpha to update their contact, and puts
    it back where it was when the contact does not touch (toi.py:640-680). A bullet ball flies into a wall past a
    slowly rising box whose fat box its swept box overlaps (so they share a contact) but which it never touches: after
    the event the box stands exactly where Solve put it, c + h v."""
    s = S.stock(gravity=(0.0, 0.0), continuous_physics=True, max_translation=100.0)
    d = wd.WorldDef(s)
    g = d.add_body(wd.STATIC, (0.0, 0.0))
    d.add_box(g, (0.05, 2.0), center=(4.0, 0.0))
    ball = d.add_body(wd.DYNAMIC, (0.0, 0.0), velocity=(300.0, 0.0), mass=1.0, inertia=1.0, bullet=True)
    d.add_circle(ball, 0.1)
    box = d.add_body(wd.DYNAMIC, (2.0, 0.25), velocity=(0.0, 1.0), mass=1.0, inertia=1.0)
    d.add_box(box, (0.5, 0.1))
    m, st = _single(d, 8)
    h = F32(1 / 60)
    c0 = st.bodies.c[0, box].copy()
    dbg = toi_trace(1, wd.dims(st))
    oracle.step_(m, st, s, h, debug=dbg)
    assert int(st.toi.events[0]) >= 1
    slot = int(dbg["toi_event_slot"][0, 0])
    assert {int(m.fixture_body[st.contacts.fa[0, slot]]), int(m.fixture_body[st.contacts.fb[0, slot]])} == {0, ball}
    shared = [k for k in range(st.contacts.pair.shape[1]) if st.contacts.pair[0, k] >= 0 and
              {int(m.fixture_body[st.contacts.fa[0, k]]), int(m.fixture_body[st.contacts.fb[0, k]])} == {ball, box}]
    assert shared and not st.contacts.touching[0, shared[0]]
    want = np.array([c0[0] + h * F32(0.0), c0[1] + h * F32(1.0)], F32)  # semi-implicit Euler, no force
    assert np.array_equal(st.bodies.c[0, box], want)
    assert float(st.bodies.c[0, ball, 0]) < 3.95


def test_angular_sleep_tolerance_is_squared(oracle):
    """A body is slow enough to sleep when w^2 <= angular_sleep_tolerance^2 (2 degrees a second) and
    |v|^2 <= linear_sleep_tolerance^2 (step.py:153-168): spinning at 0.1 rad/s it never sleeps, at 0.02 rad/s it
    falls asleep after time_to_sleep."""
    s = S.stock(gravity=(0.0, 0.0))
    for w0, sleeps in ((0.1, False), (0.02, True)):
        d = wd.WorldDef(s)
        b = d.add_body(wd.DYNAMIC, (0.0, 0.0), 0.0, angular_velocity=w0, mass=1.0, inertia=1.0)
        d.add_box(b, (0.5, 0.5))
        m, st = _single(d)
        for _ in range(45):
            oracle.step_(m, st, s, F32(1 / 60))
        assert bool(st.bodies.awake[0, 0]) != sleeps, w0


def test_gravity_scale_and_lateral_gravity(oracle):
    """Integration uses gravity_scale x gravity on both axes (step.py:86-93): with gravity (3, -10) and a gravity
    scale of 0.5 a free body's velocity after one step is exactly h (0.5 g) in float32."""
    s = S.stock(gravity=(3.0, -10.0))
    d = wd.WorldDef(s)
    b = d.add_body(wd.DYNAMIC, (0.0, 0.0), mass=1.0, inertia=1.0, gravity_scale=0.5)
    d.add_box(b, (0.5, 0.5))
    m, st = _single(d)
    h = F32(1 / 60)
    oracle.step_(m, st, s, h)
    one = F32(1)
    want = [F32(F32(0) + h * (F32(0.5) * F32(3.0) + one * F32(0))),
            F32(F32(0) + h * (F32(0.5) * F32(-10.0) + one * F32(0)))]
    assert st.bodies.v[0, 0].tolist() == want


@pytest.mark.parametrize("damping", [0.0, 0.5])
def test_soft_weld_velocity_row(oracle, damping):
    """b2WeldJoint with frequency > 0 is a spring on the angle (joints.py:125-144, 375-400): with m = 1 / (iA + iB),
    omega = 2 pi f, d = 2 m zeta omega, k = m omega^2, gamma = 1 / (h (d + h k)) and bias = C h k gamma, one velocity
    pass from rest gives the angular impulse -(bias) / (invM + gamma). A box welded at its centre to a static body
    and turned 0.3 rad from the reference angle, no warm start, one velocity and no position iteration: its spin after
    the step is iB times that impulse (float64 closed form, to 1e-5)."""
    import dataclasses
    s = dataclasses.replace(S.stock(gravity=(0.0, 0.0)), velocity_iterations=1, position_iterations=0,
                            warm_starting=False, allow_sleep=False)
    d = wd.WorldDef(s)
    g = d.add_body(wd.STATIC, (0.0, 0.0))
    C, inertia, f = 0.3, 0.5, 2.0
    b = d.add_body(wd.DYNAMIC, (0.0, 0.0), C, mass=1.0, inertia=inertia)
    d.add_box(b, (0.5, 0.5))
    d.add_weld(g, b, (0.0, 0.0), (0.0, 0.0), frequency=f, damping=damping)
    m, st = _single(d)
    h = 1.0 / 60.0
    oracle.step_(m, st, s, F32(h))
    iB = 1.0 / float(F32(inertia))
    mass = 1.0 / iB
    omega = 2.0 * np.pi * f
    dd, kk = 2.0 * mass * damping * omega, mass * omega * omega
    gamma = 1.0 / (h * (dd + h * kk))
    bias = float(F32(C)) * h * kk * gamma
    want = iB * (-bias / (iB + gamma))
    assert float(st.bodies.w[0, 1]) == pytest.approx(want, rel=1e-5)


def test_toi_integration_clamp_is_per_step(oracle):
    """With clamps_per_second, the TOI island's integration over the rest of the step (h = (1 - alpha) dt) clamps
    the translation at max_translation x dt, the step's, not x h (toi.py:780-790). A ball at 50 m/s (max_translation
    50 m/s) meets a wall of restitution 3 and leaves at 150 m/s; over h the translation 150 h exceeds 50 dt, so its
    speed is scaled to exactly 50 dt / h = 50 / (1 - alpha)."""
    import dataclasses
    s = dataclasses.replace(S.stock(gravity=(0.0, 0.0), continuous_physics=True, max_translation=50.0),
                            clamps_per_second=True, allow_sleep=False)
    d = wd.WorldDef(s)
    g = d.add_body(wd.STATIC, (0.0, 0.0))
    d.add_box(g, (0.05, 2.0), center=(0.5, 0.0), restitution=3.0)
    ball = d.add_body(wd.DYNAMIC, (0.0, 0.0), velocity=(50.0, 0.0), mass=1.0, inertia=1.0)
    d.add_circle(ball, 0.1, restitution=3.0)
    m, st = _single(d)
    dbg = toi_trace(1, wd.dims(st))
    oracle.step_(m, st, s, F32(1 / 60), debug=dbg)
    assert int(st.toi.events[0]) >= 1
    alpha = float(dbg["toi_event_alpha"][0, 0].view(np.float32))
    assert alpha < 0.6
    assert float(st.bodies.v[0, 1, 0]) == pytest.approx(-50.0 / (1.0 - alpha), rel=1e-5)
