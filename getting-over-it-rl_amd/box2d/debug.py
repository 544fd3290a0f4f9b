"""Host-side getters for debugging and parity dumps, the counterparts of the reference oracle's C API readers
(goi_jax/reference/capi.cpp:252-269 body records, :786-838 contact records with the world manifold).

They read a numpy State (a device State goes through layout.to_host first) and compute in float32 with Box2D's
operation order, so their world manifolds equal the device's (world_manifolds) bit for bit.
"""
import numpy as np

from . import world as wd

F32 = np.float32
# b2Body::m_flags bits that the State determines (the island, fixed-rotation and TOI bits are not State leaves)
AWAKE_FLAG, AUTO_SLEEP_FLAG, BULLET_FLAG, ACTIVE_FLAG = 0x0002, 0x0004, 0x0008, 0x0020


def _world(x, w):
    return np.asarray(x)[w] if np.asarray(x).ndim > 0 and w is not None else np.asarray(x)


def body_record(state, w, b):
    """goi_b2_body_get's 24 floats for body b of world w (capi.cpp:252-269): origin x, y, angle, centre x, y, vx, vy,
    w, awake, sleep time, type, active, mass, inverse mass, I about the centre, inverse I, local centre x, y, c0 x, y,
    a0, alpha0, flags (the awake, auto-sleep, bullet and active bits), bullet | continuous << 1."""
    bd = state.bodies
    g = lambda leaf: np.asarray(leaf)[w]  # noqa: E731
    flags = ((AWAKE_FLAG if g(bd.awake)[b] else 0) | (AUTO_SLEEP_FLAG if g(bd.allow_sleep)[b] else 0)
             | (BULLET_FLAG if g(bd.bullet)[b] else 0) | (ACTIVE_FLAG if g(bd.active)[b] else 0))
    return np.array([
        g(bd.xf_p)[b, 0], g(bd.xf_p)[b, 1], g(bd.a)[b], g(bd.c)[b, 0], g(bd.c)[b, 1], g(bd.v)[b, 0], g(bd.v)[b, 1],
        g(bd.w)[b], float(g(bd.awake)[b]), g(bd.sleep_time)[b], float(g(bd.type)[b]), float(g(bd.active)[b]),
        g(bd.mass)[b], g(bd.inv_mass)[b], g(bd.inertia)[b], g(bd.inv_inertia)[b], g(bd.local_center)[b, 0],
        g(bd.local_center)[b, 1], g(bd.c0)[b, 0], g(bd.c0)[b, 1], g(bd.a0)[b], np.asarray(state.toi.alpha0)[w][b],
        float(flags), float(int(g(bd.bullet)[b]) | (int(g(bd.continuous)[b]) << 1))], F32)


def _mul(q, p, v):
    """b2Mul(xf, v) in float32: (c x - s y) + px, (s x + c y) + py."""
    c, s = F32(q[0]), F32(q[1])
    return np.array([F32(F32(F32(c * v[0]) - F32(s * v[1])) + F32(p[0])),
                     F32(F32(F32(s * v[0]) + F32(c * v[1])) + F32(p[1]))], F32)


def _rot(q, v):
    c, s = F32(q[0]), F32(q[1])
    return np.array([F32(F32(c * v[0]) - F32(s * v[1])), F32(F32(s * v[0]) + F32(c * v[1]))], F32)


def _dot(a, b):
    return F32(F32(a[0] * b[0]) + F32(a[1] * b[1]))


def _scale(s, v):
    return np.array([F32(s * v[0]), F32(s * v[1])], F32)


def world_manifold(mtype, count, ln, lp, pl, xa, qa, xb, qb, ra, rb):
    """b2WorldManifold::Initialize (Box2D 2.3.1; contact_solver.py:60-104 computes the same inside prepare):
    (normal [2], points [2, 2], separations [2]); points and separations past `count` are zero."""
    eps = F32(1.1920928955078125e-7)
    normal = np.zeros(2, F32)
    pts = np.zeros((2, 2), F32)
    seps = np.zeros(2, F32)
    if count == 0:
        return normal, pts, seps
    ra, rb = F32(ra), F32(rb)
    if mtype == 0:
        normal = np.array([1, 0], F32)
        pa, pb = _mul(qa, xa, lp), _mul(qb, xb, pl[0])
        d = (pb - pa).astype(F32)
        if _dot(d, d) > F32(eps * eps):
            n = F32(np.sqrt(_dot(d, d)))
            if n >= eps:
                inv = F32(F32(1) / n)
                normal = np.array([F32(d[0] * inv), F32(d[1] * inv)], F32)
            else:
                normal = d
        ca = (pa + _scale(ra, normal)).astype(F32)
        cb = (pb - _scale(rb, normal)).astype(F32)
        pts[0] = _scale(F32(0.5), (ca + cb).astype(F32))
        seps[0] = _dot((cb - ca).astype(F32), normal)
        return normal, pts, seps
    face_a = mtype == 1
    q1, x1, q2, x2 = (qa, xa, qb, xb) if face_a else (qb, xb, qa, xa)
    r1, r2 = (ra, rb) if face_a else (rb, ra)
    normal = _rot(q1, ln)
    plane = _mul(q1, x1, lp)
    for i in range(count):
        clip = _mul(q2, x2, pl[i])
        c1 = (clip + _scale(F32(r1 - _dot((clip - plane).astype(F32), normal)), normal)).astype(F32)
        c2 = (clip - _scale(r2, normal)).astype(F32)
        pts[i] = _scale(F32(0.5), (c1 + c2).astype(F32))
        seps[i] = _dot((c2 - c1).astype(F32), normal)
    if not face_a:
        normal = (-normal).astype(F32)
    return normal, pts, seps


def contacts(model, state, w):
    """The live contacts of world w in Box2D's list order (newest first = descending key), as goi_b2_contacts
    reports them (capi.cpp:786-838): fixtures, bodies, slot, key, flags' touching / enabled bits, TOI count and
    time, friction, restitution, tangent speed, the manifold and, where it has points, the world manifold."""
    ct, bd, toi = state.contacts, state.bodies, state.toi
    g = lambda leaf: np.asarray(leaf)[w]  # noqa: E731
    live = [k for k in range(ct.pair.shape[-1]) if g(ct.pair)[k] >= 0]
    live.sort(key=lambda k: -int(g(ct.key)[k]))
    out = []
    for k in live:
        fa, fb = int(g(ct.fa)[k]), int(g(ct.fb)[k])
        ba, bb = int(model.fixture_body[fa]), int(model.fixture_body[fb])
        n = int(g(ct.count)[k])
        r = dict(slot=k, key=int(g(ct.key)[k]), candidate=int(g(ct.pair)[k]), fixtureA=fa, fixtureB=fb, bodyA=ba,
                 bodyB=bb, touching=bool(g(ct.touching)[k]), enabled=bool(g(toi.enabled)[k]),
                 toiCount=int(g(toi.count)[k]), toi=F32(g(toi.toi)[k]), friction=F32(g(ct.friction)[k]),
                 restitution=F32(g(ct.restitution)[k]), tangentSpeed=F32(g(ct.tangent_speed)[k]),
                 manifoldType=int(g(ct.mtype)[k]), pointCount=n, localNormal=g(ct.local_normal)[k].copy(),
                 localPoint=g(ct.local_point)[k].copy(), pointLocal=g(ct.point_local)[k][:n].copy(),
                 normalImpulse=g(ct.normal_impulse)[k][:n].copy(), tangentImpulse=g(ct.tangent_impulse)[k][:n].copy(),
                 pointKey=g(ct.point_id)[k][:n].copy())
        if n > 0:
            nrm, pts, seps = world_manifold(r["manifoldType"], n, r["localNormal"], r["localPoint"],
                                            g(ct.point_local)[k], g(bd.xf_p)[ba], g(bd.xf_q)[ba], g(bd.xf_p)[bb],
                                            g(bd.xf_q)[bb], model.radius[fa], model.radius[fb])
            r.update(worldNormal=nrm, worldPoints=pts[:n], separations=seps[:n])
        out.append(r)
    return out
