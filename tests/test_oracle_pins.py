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
