"""Small deterministic test scenes for the parity and pin tests (test inputs, not part of the package).

The scene inputs follow the reference's parity scenes (tests/box2d/box2d_scenes.py:21-355) and TOI scenes
(tests/box2d/test_toi.py:20-121), built with this package's WorldDef. `build_test_scene(name)` returns
(Settings, compact Model, compact single-world State).
"""
import importlib
import sys
from pathlib import Path

import numpy as np

if str(Path(__file__).resolve().parent.parent) not in sys.path:
    sys.path.insert(0, str(Path(__file__).resolve().parent.parent))
b2 = importlib.import_module("getting-over-it-rl_amd.box2d")
wd = b2.world
Settings = b2.Settings
F32 = np.float32


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


def scene_kinematic_wall(s):
    """A thin kinematic wall on x = 0 rising at 0.5 m/s (at x = -0 with tests/util.negative_zero_kinematic) and two
    boxes flying into it at 300 and 250 m/s, one from each side: TOI events whose side without mass is kinematic."""
    d = wd.WorldDef(s)
    k = d.add_body(wd.KINEMATIC, (0.0, 0.0), 0.0, (0.0, 0.5), 0.0)
    d.add_box(k, (0.05, 3.0))
    a = d.add_body(wd.DYNAMIC, (-3.0, 0.5), 0.2, (300.0, 10.0), 2.0, mass=1.0, inertia=0.02, continuous=True)
    d.add_box(a, (0.15, 0.1))
    b = d.add_body(wd.DYNAMIC, (3.0, -0.5), -0.3, (-250.0, -5.0), -3.0, mass=0.8, inertia=0.02, continuous=True)
    d.add_box(b, (0.1, 0.12))
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
    "kinematic_wall": (scene_kinematic_wall, lambda: _toi(unity=False, gravity=(0.0, 0.0)), 8),
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
