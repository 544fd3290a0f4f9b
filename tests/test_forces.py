"""Applied forces and torques (State leaves bodies.force / bodies.torque, world.py:87-88), CPU: the oracle against
b2Island::Solve's integration in closed form, with values chosen so that every float32 operation is exact
(h = 1/64, inverse mass 1/2, inverse inertia 4), and Settings.auto_clear_forces (step.py:44-46)."""
from dataclasses import replace

import numpy as np

from util import b2, wd

F32 = np.float32
H = 1.0 / 64.0


def _body(auto_clear):
    s = b2.Settings.stock(gravity=(0.0, 0.0), auto_clear_forces=auto_clear)
    d = wd.WorldDef(s)
    b = d.add_body(wd.DYNAMIC, (0.0, 0.0), mass=2.0, inertia=0.25)
    d.add_box(b, (0.5, 0.5))
    m, st = d.build(4)
    st = wd.batch(st, 1)
    st.bodies.force[0, b] = (3.0, -1.0)
    st.bodies.torque[0, b] = 4.0
    return s, m, st, b


def test_force_integration_closed_form(oracle):
    """One step: v = h F / m, w = h T / I, c = h v, a = h w (semi-implicit Euler), all exact here."""
    s, m, st, b = _body(True)
    oracle.step_(m, st, s, H)
    bd = st.bodies
    assert tuple(bd.v[0, b]) == (F32(3.0 / 128), F32(-1.0 / 128))
    assert bd.w[0, b] == F32(0.25)
    assert tuple(bd.c[0, b]) == (F32(3.0 / 8192), F32(-1.0 / 8192))
    assert bd.a[0, b] == F32(1.0 / 256)
    assert tuple(bd.force[0, b]) == (0.0, 0.0) and bd.torque[0, b] == 0.0


def test_auto_clear_forces(oracle):
    """With auto_clear_forces the second step coasts; without it the force acts again and the velocity doubles."""
    for clear, k in ((True, 1), (False, 2)):
        s, m, st, b = _body(clear)
        oracle.step_(m, st, s, H)
        oracle.step_(m, st, s, H)
        assert tuple(st.bodies.v[0, b]) == (F32(k * 3.0 / 128), F32(-k * 1.0 / 128)), clear
        assert st.bodies.w[0, b] == F32(k * 0.25), clear
        kept = (0.0, 0.0, 0.0) if clear else (3.0, -1.0, 4.0)
        assert (*st.bodies.force[0, b], st.bodies.torque[0, b]) == kept


def test_force_scales_with_gravity_scale(oracle):
    """Gravity enters scaled by the body's gravity_scale, the force by the inverse mass: v = h (gs g + F / m)."""
    s = b2.Settings.stock(gravity=(0.0, -8.0))
    d = wd.WorldDef(s)
    b = d.add_body(wd.DYNAMIC, (0.0, 0.0), mass=2.0, inertia=0.25, gravity_scale=0.5)
    d.add_box(b, (0.5, 0.5))
    m, st = d.build(4)
    st = wd.batch(st, 1)
    st.bodies.force[0, b] = (0.0, 2.0)
    oracle.step_(m, st, replace(s), H)
    assert tuple(st.bodies.v[0, b]) == (0.0, F32(H * (0.5 * -8.0 + 1.0)))
