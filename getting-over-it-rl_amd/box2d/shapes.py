"""Shape geometry built on the host in float32: polygons (raw and hull-built), boxes, circles, the thin-quad encoding
of terrain segments, and native b2EdgeShape / b2ChainShape children (which the reference does not have,
goi_jax/box2d/shapes.py:13).

Arithmetic. Every value is an IEEE binary32 rounded after each operation, in the operation order of Box2D 2.3.1's
b2PolygonShape / b2Math code that the reference restates (goi_jax/box2d/shapes.py:16-113). The code below works on
float32 numpy arrays: an elementwise float32 operation rounds once per element, so a vectorized expression gives the
same bits as Box2D's scalar loop as long as each element sees the same operations in the same order.

Storage. A fixture holds one shape in 8 vertex and 8 normal slots: a polygon's vertices and outward edge normals,
the unused slots repeating slot 0 (never read: `count` masks them); a circle's centre in slot 0 with count 1; an
edge's m_vertex1, m_vertex2, m_vertex0, m_vertex3 in slots 0-3 with count 2, its ghost flags in the fixture's edge
flags.
"""
import math

import numpy as np

from .settings import EPSILON, MAX_POLYGON_VERTICES

F32 = np.float32
CIRCLE, EDGE, POLYGON = 0, 1, 2  # b2Shape::Type (the reference's shapes.py:13 leaves out edge 1)
EDGE_HAS_V0, EDGE_HAS_V3, EDGE_CHAIN = 1, 2, 4  # edge flags; EDGE_CHAIN: a b2ChainShape child


def host_sin_cos(a):
    """(float)sin((double)a), (float)cos((double)a): the correctly rounded float pair (math2d.py:321-325)."""
    x = float(F32(a))
    return F32(math.sin(x)), F32(math.cos(x))


def _unit_rows(vx, vy):
    """b2Vec2::Normalize of each row (x, y) of two float32 arrays: length sqrt(x x + y y); a row shorter than
    b2_epsilon stays as it is, the others are multiplied by 1 / length."""
    vx, vy = np.asarray(vx, F32), np.asarray(vy, F32)
    length = np.sqrt(vx * vx + vy * vy)
    short = length < EPSILON
    inv = F32(1.0) / np.where(short, F32(1.0), length)
    return np.where(short, vx, vx * inv), np.where(short, vy, vy * inv)


def normalize_host(x, y):
    """b2Vec2::Normalize of one vector in float32; returns (x, y)."""
    ux, uy = _unit_rows(np.array([x], F32), np.array([y], F32))
    return F32(ux[0]), F32(uy[0])


def edge_normals(v):
    """Outward unit normals of a CCW polygon's edges, as b2PolygonShape::Set derives them: edge i runs from vertex i
    to vertex i + 1 (wrapping), and its normal is b2Cross(edge, 1) = (edge.y, -edge.x), normalized."""
    v = np.asarray(v, F32)
    ahead = np.roll(v, -1, axis=0)
    ex, ey = ahead[:, 0] - v[:, 0], ahead[:, 1] - v[:, 1]
    nx, ny = _unit_rows(ey, -ex)
    return np.stack([nx, ny], axis=1)


def _check_strictly_convex_ccw(v):
    """Every vertex j other than the ends of edge i lies strictly left of it: cross(edge_i, v_j - v_i) > 0, each
    term rounded as Box2D's b2Cross of float32 vectors."""
    n = len(v)
    start = v[:, None, :]                                    # (n, 1, 2): v_i
    edge = (np.roll(v, -1, axis=0) - v)[:, None, :]          # (n, 1, 2): v_{i+1} - v_i
    others = np.stack([np.roll(v, -k, axis=0) for k in range(2, n)], axis=1) - start  # (n, n-2, 2): v_{i+k} - v_i
    turn = edge[..., 0] * others[..., 1] - edge[..., 1] * others[..., 0]
    if not (turn > 0).all():
        raise ValueError("raw polygon vertices must turn strictly left (convex, counter-clockwise)")


def polygon_raw(vertices):
    """A polygon whose vertices are taken as given (3 to 8, strictly convex, counter-clockwise), with the normals
    b2PolygonShape::Set would compute (the reference oracle's raw polygons, capi.cpp:378-416). Returns
    (vertices (n, 2), normals (n, 2)) float32."""
    v = np.asarray(vertices, F32).reshape(-1, 2)
    if not 3 <= len(v) <= MAX_POLYGON_VERTICES:
        raise ValueError(f"a raw polygon takes 3 to {MAX_POLYGON_VERTICES} vertices, not {len(v)}")
    _check_strictly_convex_ccw(v)
    return v, edge_normals(v)


def _merge_close_points(pts, tol):
    """The points in order, skipping each one whose squared distance to a point already kept is below tol
    (b2PolygonShape::Set's weld of points closer than sqrt(0.5 * linearSlop))."""
    kept = np.zeros((0, 2), F32)
    for p in pts:
        d = kept - p
        if len(kept) == 0 or (d[:, 0] * d[:, 0] + d[:, 1] * d[:, 1] >= tol).all():
            kept = np.vstack([kept, p[None]])
    return kept


def _wrap_hull(pts):
    """Indices of the convex hull of pts in counter-clockwise order, by Box2D 2.3.1's gift wrap: start at the
    largest x (the lowest y among equal x); from each hull vertex h, scan the points in index order keeping a
    candidate c, which a point p replaces when p lies right of h->c (cross < 0), or on that line farther from h; the
    candidate is seeded with the first point other than h."""
    count = len(pts)
    first = 0
    for i in range(1, count):
        x, y = pts[i]
        if x > pts[first][0] or (x == pts[first][0] and y < pts[first][1]):
            first = i
    order = [first]
    while len(order) <= MAX_POLYGON_VERTICES:
        here = pts[order[-1]]
        pick = 0
        for i in range(1, count):
            if pick == order[-1]:
                pick = i
                continue
            to_pick = pts[pick] - here
            to_i = pts[i] - here
            turn = to_pick[0] * to_i[1] - to_pick[1] * to_i[0]
            if turn < 0:
                pick = i
            if turn == 0 and to_i[0] * to_i[0] + to_i[1] * to_i[1] > to_pick[0] * to_pick[0] + to_pick[1] * to_pick[1]:
                pick = i
        if pick == first:
            return order
        order.append(pick)
    raise ValueError("the gift wrap did not come back to its first vertex")


def polygon_set(vertices, linear_slop):
    """b2PolygonShape::Set (v2.3.1): the first 8 points, close points merged, their convex hull counter-clockwise,
    and the edge normals. Raises ValueError where Box2D would give up and build SetAsBox(1, 1) instead (fewer than 3
    distinct points, or a hull of fewer than 3 vertices). Returns (vertices, normals) float32."""
    pts = np.asarray(vertices, F32).reshape(-1, 2)[:MAX_POLYGON_VERTICES]
    pts = _merge_close_points(pts, F32(0.5) * F32(linear_slop))
    if len(pts) < 3:
        raise ValueError("fewer than 3 distinct points: b2PolygonShape::Set would fall back to a 1 x 1 box")
    hull = _wrap_hull(pts)
    if len(hull) < 3:
        raise ValueError("the points are collinear: b2PolygonShape::Set would fall back to a 1 x 1 box")
    v = pts[hull]
    return v, edge_normals(v)


def _rotate_rows(c, s, pts):
    """b2Mul(b2Rot, v) of each row: (c x - s y, s x + c y)."""
    x, y = pts[:, 0], pts[:, 1]
    return np.stack([c * x - s * y, s * x + c * y], axis=1)


def box(hx, hy, center=(0.0, 0.0), angle=0.0):
    """b2PolygonShape::SetAsBox(hx, hy, center, angle): the corners (-hx, -hy), (hx, -hy), (hx, hy), (-hx, hy) and
    the normals -y, +x, +y, -x, rotated by the correctly rounded b2Rot(angle), the corners then moved by center.
    Returns (vertices, normals) float32."""
    hx, hy = F32(hx), F32(hy)
    corners = np.array([[-hx, -hy], [hx, -hy], [hx, hy], [-hx, hy]], F32)
    normals = np.array([[0, -1], [1, 0], [0, 1], [-1, 0]], F32)
    s, c = host_sin_cos(angle)
    shift = np.array([center[0], center[1]], F32)
    return _rotate_rows(c, s, corners) + shift, _rotate_rows(c, s, normals)


def edge_quad(p0, p1, thickness=0.1):
    """A terrain segment [p0, p1] as a thin counter-clockwise quad {p0 - t n, p1 - t n, p1, p0} (n the segment's
    unit left normal, t the thickness; computed in float64, then rounded to float32), so that its contacts use
    reference-defined polygon code. Raw vertices, with Set's normals."""
    a, b = np.asarray(p0, np.float64), np.asarray(p1, np.float64)
    along = b - a
    left = np.array([-along[1], along[0]]) / np.hypot(along[0], along[1])
    drop = thickness * left
    return polygon_raw(np.array([a - drop, b - drop, b, a]).astype(F32))


def centroid_raw(v):
    """m_centroid of a raw polygon as the reference oracle's builder accumulates it: a running float32 sum of
    (1 / n) v_i over the vertices in order (capi.cpp:386-401)."""
    v = np.asarray(v, F32)
    weight = F32(1.0) / F32(len(v))
    acc = np.zeros(2, F32)
    for p in v:
        acc = acc + weight * p
    return acc


def centroid_set(v):
    """ComputeCentroid of b2PolygonShape::Set (v2.3.1): triangles fanned from the origin (its reference point p1 =
    (0, 0)), each of signed area 0.5 cross(v_i, v_{i+1}) adding area / 3 times (p1 + v_i + v_{i+1}); the sum over
    the total area."""
    v = np.asarray(v, F32)
    third = F32(1.0) / F32(3.0)
    acc, area = np.zeros(2, F32), F32(0.0)
    for p, q in zip(v, np.roll(v, -1, axis=0)):
        tri = F32(0.5) * (p[0] * q[1] - p[1] * q[0])
        area = area + tri
        acc = acc + (tri * third) * ((F32(0.0) + p) + q)
    return (F32(1.0) / area) * acc


def edge_shape(v1, v2, v0=None, v3=None):
    """b2EdgeShape::Set(v1, v2) with the optional ghost vertices v0 (before v1) and v3 (after v2): ((4, 2) float32
    slots v1, v2, v0, v3; the EDGE_HAS_V0 / EDGE_HAS_V3 flags of the ghosts given)."""
    slots = np.zeros((4, 2), F32)
    slots[0], slots[1] = v1, v2
    flags = 0
    for slot, ghost, flag in ((2, v0, EDGE_HAS_V0), (3, v3, EDGE_HAS_V3)):
        if ghost is not None:
            slots[slot] = ghost
            flags |= flag
    if (slots[0] == slots[1]).all():
        raise ValueError("an edge needs two distinct end points")
    return slots, flags


def chain_edges(points, loop=False, prev_vertex=None, next_vertex=None):
    """The child edges of b2ChainShape::CreateChain / CreateLoop (GetChildEdge): edge i runs from point i to point
    i + 1, with ghosts at points i - 1 and i + 2 where they exist. A loop closes back to its first point and wraps its
    ghosts; an open chain takes prev_vertex / next_vertex (b2ChainShape::SetPrevVertex / SetNextVertex) as the ghosts
    of its end edges. Returns [(slots, flags)], each flagged EDGE_CHAIN."""
    p = np.asarray(points, F32).reshape(-1, 2)
    if loop:
        if len(p) < 3:
            raise ValueError("a chain loop needs at least 3 points")
        prev_vertex, next_vertex = p[-1], p[1]
        p = np.vstack([p, p[:1]])
    if len(p) < 2:
        raise ValueError("a chain needs at least 2 points")
    last = len(p) - 2  # index of the last edge
    children = []
    for i in range(last + 1):
        before = p[i - 1] if i > 0 else prev_vertex
        after = p[i + 2] if i < last else next_vertex
        slots, flags = edge_shape(p[i], p[i + 1], before, after)
        children.append((slots, flags | EDGE_CHAIN))
    return children


def pad(v, n):
    """The (8, 2) vertex and normal slots of a shape: its rows, then copies of row 0."""
    v, n = np.asarray(v, F32), np.asarray(n, F32)
    fill = MAX_POLYGON_VERTICES - len(v)
    return (np.concatenate([v, np.repeat(v[:1], fill, axis=0)]),
            np.concatenate([n, np.repeat(n[:1], fill, axis=0)]))
