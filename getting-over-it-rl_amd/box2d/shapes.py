"""Host-side shape construction in float32, b2PolygonShape / b2CircleShape v2.3.1 op for op (mirror of
goi_jax/box2d/shapes.py:1-113), plus the thin-quad encoding of terrain edge segments.

A fixture holds one shape. Polygons store up to 8 vertices and edge normals, padded by repeating vertex 0 (pads are
masked by `count`); a circle stores its centre in vertex 0 and count 1.
"""
import math

import numpy as np

from .settings import EPSILON, MAX_POLYGON_VERTICES

F32 = np.float32
CIRCLE, POLYGON = 0, 2  # b2Shape::Type (shapes.py:13)


def host_sin_cos(a):
    """(float)sin((double)a), (float)cos((double)a) (math2d.py:321-325)."""
    a = float(F32(a))
    return F32(math.sin(a)), F32(math.cos(a))


def normalize_host(x, y):
    """b2Vec2::Normalize in float32 (shapes.py:19-25)."""
    x, y = F32(x), F32(y)
    n = F32(np.sqrt(F32(F32(x * x) + F32(y * y))))
    if n < EPSILON:
        return x, y
    inv = F32(F32(1.0) / n)
    return F32(x * inv), F32(y * inv)


def edge_normals(v):
    """b2PolygonShape::Set's normals: Normalize(b2Cross(v[i+1] - v[i], 1.0f)) (shapes.py:28-33)."""
    n = len(v)
    out = np.zeros((n, 2), F32)
    for i in range(n):
        j = i + 1 if i + 1 < n else 0
        ex, ey = F32(v[j][0] - v[i][0]), F32(v[j][1] - v[i][1])
        out[i] = normalize_host(F32(F32(1.0) * ey), F32(F32(-1.0) * ex))
    return out


def polygon_raw(vertices):
    """Vertices verbatim (strictly convex, CCW), normals as Set derives them (shapes.py:36-47)."""
    v = np.asarray(vertices, F32).reshape(-1, 2)
    if not 3 <= len(v) <= MAX_POLYGON_VERTICES:
        raise ValueError("polygon needs 3..8 vertices")
    for i in range(len(v)):
        e = v[(i + 1) % len(v)] - v[i]
        for k in range(2, len(v)):
            d = v[(i + k) % len(v)] - v[i]
            if F32(F32(e[0] * d[1]) - F32(e[1] * d[0])) <= 0:
                raise ValueError("polygon not strictly convex CCW")
    return v, edge_normals(v)


def polygon_set(vertices, linear_slop):
    """b2PolygonShape::Set v2.3.1: weld near points, gift-wrap from the rightmost (then lowest) point, CCW
    (shapes.py:50-89). Raises where Box2D would fall back to SetAsBox(1, 1)."""
    pts = [tuple(F32(c) for c in p) for p in np.asarray(vertices, F32).reshape(-1, 2)[:MAX_POLYGON_VERTICES]]
    weld = F32(F32(0.5) * F32(linear_slop))
    ps = []
    for v in pts:
        keep = True
        for q in ps:
            dx, dy = F32(v[0] - q[0]), F32(v[1] - q[1])
            if F32(F32(dx * dx) + F32(dy * dy)) < weld:
                keep = False
                break
        if keep:
            ps.append(v)
    n = len(ps)
    if n < 3:
        raise ValueError("degenerate polygon (Box2D would use SetAsBox(1, 1))")
    i0, x0 = 0, ps[0][0]
    for i in range(1, n):
        x = ps[i][0]
        if x > x0 or (x == x0 and ps[i][1] < ps[i0][1]):
            i0, x0 = i, x
    hull, ih = [], i0
    while True:
        hull.append(ih)
        ie = 0
        for j in range(1, n):
            if ie == ih:
                ie = j
                continue
            rx, ry = F32(ps[ie][0] - ps[hull[-1]][0]), F32(ps[ie][1] - ps[hull[-1]][1])
            vx, vy = F32(ps[j][0] - ps[hull[-1]][0]), F32(ps[j][1] - ps[hull[-1]][1])
            c = F32(F32(rx * vy) - F32(ry * vx))
            if c < 0:
                ie = j
            if c == 0 and F32(F32(vx * vx) + F32(vy * vy)) > F32(F32(rx * rx) + F32(ry * ry)):
                ie = j
        ih = ie
        if ie == i0:
            break
        if len(hull) > MAX_POLYGON_VERTICES:
            raise ValueError("hull did not close")
    if len(hull) < 3:
        raise ValueError("degenerate hull")
    v = np.array([ps[i] for i in hull], F32)
    return v, edge_normals(v)


def box(hx, hy, center=(0.0, 0.0), angle=0.0):
    """b2PolygonShape::SetAsBox(hx, hy, center, angle) (shapes.py:92-104)."""
    hx, hy = F32(hx), F32(hy)
    v = np.array([(-hx, -hy), (hx, -hy), (hx, hy), (-hx, hy)], F32)
    n = np.array([(0, -1), (1, 0), (0, 1), (-1, 0)], F32)
    s, c = host_sin_cos(angle)
    px, py = F32(center[0]), F32(center[1])
    for i in range(4):
        x, y = v[i]
        v[i] = (F32(F32(F32(c * x) - F32(s * y)) + px), F32(F32(F32(s * x) + F32(c * y)) + py))
        x, y = n[i]
        n[i] = (F32(F32(c * x) - F32(s * y)), F32(F32(s * x) + F32(c * y)))
    return v, n


def edge_quad(p0, p1, thickness=0.1):
    """A terrain edge segment [p0, p1] as a thin CCW quad {p0, p1, p1 - t n, p0 - t n} (n the segment's left normal,
    t the thickness), so the contact uses reference-defined polygon code. Raw vertices, Set's normals."""
    p0 = np.asarray(p0, np.float64)
    p1 = np.asarray(p1, np.float64)
    d = p1 - p0
    n = np.array([-d[1], d[0]]) / np.hypot(d[0], d[1])
    q = np.array([p0 - thickness * n, p1 - thickness * n, p1, p0], np.float64)  # CCW: bottom edge first
    return polygon_raw(q.astype(F32))


def pad(v, n):
    """(8, 2) vertex and normal arrays, padded with vertex/normal 0 (shapes.py:107-113)."""
    k = len(v)
    vv = np.repeat(np.asarray(v, F32)[:1], MAX_POLYGON_VERTICES, axis=0)
    nn = np.repeat(np.asarray(n, F32)[:1], MAX_POLYGON_VERTICES, axis=0)
    vv[:k], nn[:k] = v, n
    return vv, nn
