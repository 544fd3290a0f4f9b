"""Host-side shape construction in float32, b2PolygonShape / b2CircleShape v2.3.1 op for op (mirror of
goi_jax/box2d/shapes.py:1-113), the thin-quad encoding of terrain edge segments, and native b2EdgeShape /
b2ChainShape children (which the reference does not have, shapes.py:13).

A fixture holds one shape. Polygons store up to 8 vertices and edge normals, padded by repeating vertex 0 (pads are
masked by `count`); a circle stores its centre in vertex 0 and count 1; an edge stores m_vertex1, m_vertex2,
m_vertex0, m_vertex3 in vertices 0-3 with count 2, and its m_hasVertex0 / m_hasVertex3 in the fixture's edge flags.
"""
import math

import numpy as np

from .settings import EPSILON, MAX_POLYGON_VERTICES

F32 = np.float32
CIRCLE, EDGE, POLYGON = 0, 1, 2  # b2Shape::Type (shapes.py:13; the reference leaves out edge 1)
EDGE_HAS_V0, EDGE_HAS_V3, EDGE_CHAIN = 1, 2, 4  # edge flags; EDGE_CHAIN: a b2ChainShape child


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


def centroid_raw(v):
    """m_centroid of a raw polygon as the reference oracle's builder accumulates it: sum of (1/n) * v[i] in order
    (goi_jax/reference/capi.cpp:386-401)."""
    n = len(v)
    inv = F32(F32(1.0) / F32(n))
    cx, cy = F32(0), F32(0)
    for x, y in np.asarray(v, F32):
        cx, cy = F32(cx + F32(inv * x)), F32(cy + F32(inv * y))
    return np.array([cx, cy], F32)


def centroid_set(v):
    """ComputeCentroid of b2PolygonShape::Set v2.3.1: area-weighted triangle fan from the origin."""
    v = np.asarray(v, F32)
    n = len(v)
    cx, cy, area = F32(0), F32(0), F32(0)
    inv3 = F32(F32(1.0) / F32(3.0))
    for i in range(n):
        p2, p3 = v[i], v[i + 1] if i + 1 < n else v[0]
        e1x, e1y, e2x, e2y = p2[0], p2[1], p3[0], p3[1]  # p1 = (0, 0)
        d = F32(F32(e1x * e2y) - F32(e1y * e2x))
        tri = F32(F32(0.5) * d)
        area = F32(area + tri)
        w = F32(tri * inv3)
        sx, sy = F32(F32(F32(0) + p2[0]) + p3[0]), F32(F32(F32(0) + p2[1]) + p3[1])
        cx, cy = F32(cx + F32(w * sx)), F32(cy + F32(w * sy))
    inv = F32(F32(1.0) / area)
    return np.array([F32(inv * cx), F32(inv * cy)], F32)


def edge_shape(v1, v2, v0=None, v3=None):
    """b2EdgeShape::Set(v1, v2) with optional ghost vertices: ((4, 2) vertices v1, v2, v0, v3; flags)."""
    v = np.zeros((4, 2), F32)
    v[0], v[1] = v1, v2
    flags = 0
    if v0 is not None:
        v[2], flags = v0, flags | EDGE_HAS_V0
    if v3 is not None:
        v[3], flags = v3, flags | EDGE_HAS_V3
    if v[0][0] == v[1][0] and v[0][1] == v[1][1]:
        raise ValueError("degenerate edge")
    return v, flags


def chain_edges(points, loop=False, prev_vertex=None, next_vertex=None):
    """The child edges of b2ChainShape::CreateChain / CreateLoop (GetChildEdge): edge i runs from point i to i + 1,
    with ghosts at points i - 1 and i + 2 where they exist (the loop wraps; an open chain takes prev_vertex /
    next_vertex, b2ChainShape::SetPrevVertex / SetNextVertex, at its ends)."""
    p = [np.asarray(x, F32) for x in np.asarray(points, F32).reshape(-1, 2)]
    if loop:
        if len(p) < 3:
            raise ValueError("a loop needs 3 points")
        prev_vertex, next_vertex = p[-1], p[1]
        p = p + [p[0]]
    if len(p) < 2:
        raise ValueError("a chain needs 2 points")
    n = len(p)
    out = []
    for i in range(n - 1):
        v0 = p[i - 1] if i > 0 else prev_vertex
        v3 = p[i + 2] if i < n - 2 else next_vertex
        v, flags = edge_shape(p[i], p[i + 1], v0, v3)
        out.append((v, flags | EDGE_CHAIN))
    return out


def pad(v, n):
    """(8, 2) vertex and normal arrays, padded with vertex/normal 0 (shapes.py:107-113)."""
    k = len(v)
    vv = np.repeat(np.asarray(v, F32)[:1], MAX_POLYGON_VERTICES, axis=0)
    nn = np.repeat(np.asarray(n, F32)[:1], MAX_POLYGON_VERTICES, axis=0)
    vv[:k], nn[:k] = v, n
    return vv, nn
