"""Native edge shapes: b2EdgeShape and b2ChainShape children, which the reference does not have
(goi_jax/box2d/shapes.py:13, __init__.py:53), so their parity with the reference is unpinned by construction. These
pins fix the CPU restatement of Box2D 2.3.1's b2CollideEdgeAndCircle and b2EPCollider (oracle/b2_oracle.c) by closed
forms, brute force, agreement with the thin-quad polygon path where both must agree, and the behaviour ghost
vertices exist for (no catching on the junctions of a flat chain). CPU only.
"""
import numpy as np
import pytest

from util import b2

F32 = np.float32
wd = b2.world
S = b2.Settings
sh = b2.shapes
CIRCLES, FACE_A, FACE_B = 0, 1, 2
SKIN = 0.01  # b2_polygonRadius at the stock linear slop


def xf(x, y, a=0.0):
    return np.array([x, y, np.cos(a), np.sin(a)], F32)


def _world_manifold(m, fa, fb, xa, xb, man):
    """b2WorldManifold::Initialize of an evaluated manifold: (world normal A->B, [separations]) in float64."""
    def mul(t, v):
        return np.array([t[2] * v[0] - t[3] * v[1] + t[0], t[3] * v[0] + t[2] * v[1] + t[1]], np.float64)

    def rot(t, v):
        return np.array([t[2] * v[0] - t[3] * v[1], t[3] * v[0] + t[2] * v[1]], np.float64)
    ra, rb = float(m.radius[fa]), float(m.radius[fb])
    xa, xb = xa.astype(np.float64), xb.astype(np.float64)
    seps = []
    if man["mtype"] == CIRCLES:
        pa, pb = mul(xa, man["local_point"]), mul(xb, man["point_local"][0])
        n = (pb - pa) / np.linalg.norm(pb - pa)
        return n, [float(np.dot(pb - pa, n)) - ra - rb]
    if man["mtype"] == FACE_A:
        n, plane, other = rot(xa, man["local_normal"]), mul(xa, man["local_point"]), xb
    else:
        n, plane, other = rot(xb, man["local_normal"]), mul(xb, man["local_point"]), xa
    for i in range(man["count"]):
        seps.append(float(np.dot(mul(other, man["point_local"][i]) - plane, n)) - ra - rb)
    return (n if man["mtype"] == FACE_A else -n), seps


@pytest.fixture(scope="module")
def edge_world():
    d = wd.WorldDef(S.stock())
    g = d.add_body(wd.STATIC)
    f = {}
    f["iso"] = d.add_segment(g, (-1, 0), (1, 0))
    f["flat"] = d.add_segment(g, (-1, 0), (1, 0), v0=(-2, 0), v3=(2, 0))
    f["down"] = d.add_segment(g, (-1, 0), (1, 0), v3=(2, -1))
    f["long"] = d.add_segment(g, (-2, 0), (2, 0))
    f["right_iso"] = d.add_segment(g, (0, 0), (2, 0))
    f["left_iso"] = d.add_segment(g, (-2, 0), (0, 0))
    f["left_child"], f["right_child"] = d.add_chain(g, [(-2, 0), (0, 0), (2, 0)])
    f["circle"] = d.add_circle(g, 0.5)
    f["box"] = d.add_box(g, (0.5, 0.25))
    model, _ = d.build(2)
    return model, f


def test_edge_circle_regions(oracle, edge_world):
    """Regions AB (two-sided face contact), A and B (vertex contacts), and the ghost vertices' suppression."""
    m, f = edge_world
    ev = lambda e, x, y: oracle.evaluate(m, f[e], f["circle"], xf(0, 0), xf(x, y), S.stock())  # noqa: E731
    top = ev("iso", 0.2, 0.4)
    assert (top["count"], top["mtype"]) == (1, FACE_A)
    assert tuple(top["local_normal"]) == (0.0, 1.0) and tuple(top["local_point"]) == (-1.0, 0.0)
    assert int(top["point_id"][0]) == 1 << 16  # face of A, vertex of B
    assert tuple(ev("iso", 0.2, -0.4)["local_normal"]) == (0.0, -1.0)
    assert ev("iso", 0.2, 0.52)["count"] == 0  # 0.52 > 0.5 + skin
    vb = ev("iso", 1.3, 0.1)
    assert (vb["count"], vb["mtype"], int(vb["point_id"][0])) == (1, CIRCLES, 1)
    assert tuple(vb["local_point"]) == (1.0, 0.0)
    va = ev("iso", -1.3, -0.1)
    assert (va["count"], va["mtype"], int(va["point_id"][0])) == (1, CIRCLES, 0)
    assert ev("iso", 1.6, 0.0)["count"] == 0
    # collinear neighbours own the circle beyond either vertex
    assert ev("flat", 1.3, 0.1)["count"] == 0 and ev("flat", -1.3, 0.1)["count"] == 0
    assert ev("flat", 0.3, 0.1)["count"] == 1
    # a convex corner downwards: the next edge owns only the circles on its face side
    assert ev("down", 1.3, 0.1)["count"] == 0
    corner = ev("down", 1.1, 0.45)
    assert (corner["count"], corner["mtype"]) == (1, CIRCLES) and tuple(corner["local_point"]) == (1.0, 0.0)


def _seg_dist(p, a, b):
    ab = b - a
    t = np.clip(np.dot(p - a, ab) / np.dot(ab, ab), 0.0, 1.0)
    return float(np.linalg.norm(p - (a + t * ab)))


def test_edge_circle_vs_brute_force(oracle):
    """An isolated edge touches a circle iff the segment distance is within the radii; the face normal points to
    the circle. Along a chain, ghosts only remove duplicates: some child edge touches the circle iff the chain's
    distance is within the radii."""
    rng = np.random.default_rng(21)
    pts = np.array([(-3, 0.5), (-1.5, -0.2), (0, 0), (1.2, 0.9), (2.5, 0.4), (3.5, 1.5)])
    d = wd.WorldDef(S.stock())
    g = d.add_body(wd.STATIC)
    chain = d.add_chain(g, pts)
    iso = [d.add_segment(g, pts[i], pts[i + 1]) for i in range(len(pts) - 1)]
    c = d.add_circle(g, 0.3)
    m, _ = d.build(2)
    r = 0.3 + SKIN
    seen = [0, 0]
    for _ in range(1500):
        q = rng.uniform((-3.5, -1.0), (4.0, 2.0)).astype(F32)
        dists = [_seg_dist(q.astype(np.float64), pts[i], pts[i + 1]) for i in range(len(pts) - 1)]
        if min(abs(x - r) for x in dists) < 1e-4:
            continue
        hits = []
        for i, (fc, fi) in enumerate(zip(chain, iso)):
            mi = oracle.evaluate(m, fi, c, xf(0, 0), xf(q[0], q[1]), S.stock())
            assert (mi["count"] == 1) == (dists[i] <= r)
            if mi["count"] and mi["mtype"] == FACE_A:
                assert np.dot(mi["local_normal"], q - pts[i]) > 0 and abs(np.linalg.norm(mi["local_normal"]) - 1) < 1e-6
            mc = oracle.evaluate(m, fc, c, xf(0, 0), xf(q[0], q[1]), S.stock())
            assert mc["count"] <= mi["count"]
            hits.append(mc["count"])
        assert (sum(hits) > 0) == (min(dists) <= r)
        seen[min(dists) <= r] += 1
    assert min(seen) > 100


def test_edge_polygon_closed_forms(oracle, edge_world):
    """A box resting on an edge (the back side of a left-to-right edge faces up), the skin 2 * b2_polygonRadius, the
    ghost collision that ghost vertices prevent (a box sunk 2 cm and just past a junction is pushed sideways by an
    isolated edge, whose polygon side becomes the reference face, but held up by the chain child), and the axis
    hysteresis."""
    m, f = edge_world
    ev = lambda e, x, y: oracle.evaluate(m, f[e], f["box"], xf(0, 0), xf(x, y), S.stock())  # noqa: E731
    rest = ev("long", 0.3, F32(0.245))
    assert (rest["count"], rest["mtype"]) == (2, FACE_A)
    assert tuple(rest["local_normal"]) == (0.0, 1.0) and tuple(rest["local_point"]) == (2.0, 0.0)
    assert [tuple(p) for p in rest["point_local"]] == [(-0.5, -0.25), (0.5, -0.25)]
    assert [int(i) for i in rest["point_id"]] == [1 << 16, (1 << 16) | (1 << 8)]
    n, seps = _world_manifold(m, f["long"], f["box"], xf(0, 0), xf(0.3, F32(0.245)), rest)
    assert np.allclose(n, (0, 1)) and np.allclose(seps, [-0.005 - 2 * SKIN] * 2, atol=1e-6)
    assert ev("long", 0.3, F32(0.25 + 0.015))["count"] == 2  # within the 2-cm skin
    assert ev("long", 0.3, F32(0.25 + 0.021))["count"] == 0
    below = ev("long", 0.3, F32(-0.245))
    assert (below["count"], below["mtype"], tuple(below["local_normal"])) == (2, FACE_A, (0.0, -1.0))
    for iso, child, x, side in (("right_iso", "right_child", -0.495, (1.0, 0.0)),
                                ("left_iso", "left_child", 0.495, (-1.0, 0.0))):
        caught = ev(iso, F32(x), F32(0.23))
        assert (caught["count"], caught["mtype"], tuple(caught["local_normal"])) == (1, FACE_B, side)
        held = ev(child, F32(x), F32(0.23))
        assert held["mtype"] == FACE_A and tuple(held["local_normal"]) == (0.0, 1.0) and held["count"] >= 1
    # hysteresis 0.98 / 0.001: a side face 1 mm shallower (-0.019) than the edge axis (-0.020) does not take over
    near = ev("right_iso", F32(-0.481), F32(0.23))
    assert (near["mtype"], tuple(near["local_normal"])) == (FACE_A, (0.0, 1.0))


def test_edge_polygon_matches_thin_quad(oracle):
    """Inside a long edge, a polygon touching its face gets the same world normal and separations from the edge
    collider as from b2CollidePolygons against the thin quad under the same segment (both skins are b2_polygonRadius);
    the incident vertices (feature index B) agree too."""
    rng = np.random.default_rng(5)

    def add_shapes(d, g):
        return [d.add_box(g, (0.4, 0.2)), d.add_polygon(g, [(0, 0), (0.6, 0.1), (0.2, 0.5)]),
                d.add_polygon(g, [(0.3 * np.cos(a), 0.3 * np.sin(a)) for a in np.arange(5) * 2 * np.pi / 5])]
    found = 0
    for ang in (0.0, 0.3):
        p0, p1 = np.array([-3 * np.cos(ang), -3 * np.sin(ang)]), np.array([3 * np.cos(ang), 3 * np.sin(ang)])
        d2 = wd.WorldDef(S.stock())
        g2 = d2.add_body(wd.STATIC)
        e = d2.add_segment(g2, p0, p1)
        q = d2.add_edge(g2, p0, p1)
        assert add_shapes(d2, g2) == [2, 3, 4]
        m, _ = d2.build(2)
        t, nrm = p1 / 3.0, np.array([-np.sin(ang), np.cos(ang)])
        for _ in range(300):
            k = 2 + int(rng.integers(0, 3))
            a = rng.uniform(-np.pi, np.pi)
            x = xf(0, 0, a)
            verts = m.verts[k, :m.count[k]].astype(np.float64)
            rv = np.stack([x[2] * verts[:, 0] - x[3] * verts[:, 1], x[3] * verts[:, 0] + x[2] * verts[:, 1]], 1)
            depth = rng.uniform(-0.012, 0.012)
            c = rng.uniform(-1.5, 1.5) * t + (depth - np.min(rv @ nrm)) * nrm
            xb = xf(c[0], c[1], a)
            me = oracle.evaluate(m, e, k, xf(0, 0), xb, S.stock())
            mq = oracle.evaluate(m, q, k, xf(0, 0), xb, S.stock())
            assert me["count"] == mq["count"]
            if me["count"] == 0:
                continue
            found += 1
            ne, se = _world_manifold(m, e, k, xf(0, 0), xb, me)
            nq, sq = _world_manifold(m, q, k, xf(0, 0), xb, mq)
            assert np.allclose(ne, nq, atol=1e-5) and np.allclose(sorted(se), sorted(sq), atol=1e-5)
            ib = lambda man: sorted((int(i) >> 8) & 0xFF for i in man["point_id"][:man["count"]])  # noqa: E731
            if me["mtype"] == FACE_A and mq["mtype"] == FACE_A:
                assert ib(me) == ib(mq)
    assert found > 300


def test_aabbs_and_candidate_order():
    """A chain child's fat box has no skin (b2ChainShape::ComputeAABB), a segment's has one (b2EdgeShape); every
    candidate names the edge first (b2Contact::Create), and two edges never pair."""
    d = wd.WorldDef(S.stock())
    g = d.add_body(wd.STATIC)
    seg = d.add_segment(g, (0, 0), (2, 1))
    ch = d.add_chain(g, [(3, 0), (4, 1), (5, 0)])
    b = d.add_body(wd.DYNAMIC, (0, 3), mass=1, inertia=0.1)
    circ = d.add_circle(b, 0.2)
    box = d.add_box(b, (0.2, 0.2))
    m, st = d.build(8)
    fat = st.fixtures.fat
    assert np.allclose(fat[seg], [-0.11, -0.11, 2.11, 1.11], atol=1e-6)
    assert np.allclose(fat[ch[0]], [2.9, -0.1, 4.1, 1.1], atol=1e-6)
    pairs = set(zip(m.pair_a.tolist(), m.pair_b.tolist()))
    assert pairs == {(e, s) for e in (seg, *ch) for s in (circ, box)}
    assert m.edge_flags[ch[0]] == sh.EDGE_HAS_V3 | sh.EDGE_CHAIN and m.edge_flags[ch[1]] == sh.EDGE_HAS_V0 | sh.EDGE_CHAIN
    assert m.edge_flags[seg] == 0 and list(m.count[[seg, *ch]]) == [2, 2, 2]
    loop = sh.chain_edges([(0, 0), (1, 0), (1, 1)], loop=True)
    assert len(loop) == 3 and all(fl == sh.EDGE_HAS_V0 | sh.EDGE_HAS_V3 | sh.EDGE_CHAIN for _, fl in loop)
    assert tuple(loop[0][0][2]) == (1.0, 1.0) and tuple(loop[2][0][3]) == (1.0, 0.0)
    with pytest.raises(ValueError):
        d.add_segment(b, (0, 0), (1, 0))


def test_polygon_centroids():
    """m_centroid by build path: Set's area-weighted fan (exact for a right triangle), the raw mean, a box's centre."""
    c = sh.centroid_set(np.array([(0, 0), (3, 0), (0, 3)], F32))
    assert np.allclose(c, (1, 1), atol=1e-6)
    v = np.array([(0, 0), (4, 0), (4, 1), (0, 1)], F32)
    assert np.allclose(sh.centroid_set(v), (2, 0.5), atol=1e-6) and np.allclose(sh.centroid_raw(v), (2, 0.5))
    d = wd.WorldDef(S.stock())
    g = d.add_body(wd.STATIC)
    d.add_box(g, (1, 2), center=(0.5, -0.25), angle=0.3)
    d.add_polygon(g, [(0, 0), (2, 0), (2, 1), (0, 3)])
    m, _ = d.build(2)
    assert tuple(m.centroid[0]) == (0.5, -0.25)
    # the quadrilateral (0,0) (2,0) (2,1) (0,3) = rectangle [0,2]x[0,1] (area 2, centre (1, 0.5)) + triangle
    # (0,1) (2,1) (0,3) (area 2, centroid (2/3, 5/3)): centroid (5/6, 13/12)
    assert np.allclose(m.centroid[1], (5 / 6, 13 / 12), atol=1e-6)


def _chain_ground(d, g, ghosts, x0=-10.0, x1=10.0, step=0.5):
    xs = np.arange(x0, x1 + 1e-9, step)
    if ghosts:
        d.add_chain(g, [(x, 0.0) for x in xs], friction=0.0)
    else:
        for a, b in zip(xs[:-1], xs[1:]):
            d.add_segment(g, (a, 0.0), (b, 0.0), friction=0.0)


def test_box_slides_over_chain_junctions(oracle):
    """A frictionless box sliding at 4 m/s across 24 junctions of a flat chain keeps its speed and height: ghost
    vertices stop the junctions from catching it (its motion is a closed form: constant velocity)."""
    d = wd.WorldDef(S.stock(gravity=(0.0, -10.0)))
    g = d.add_body(wd.STATIC)
    _chain_ground(d, g, ghosts=True)
    b = d.add_body(wd.DYNAMIC, (-8.0, 0.25), 0.0, (4.0, 0.0), mass=1.0, inertia=F32(1) / F32(24))
    d.add_box(b, (0.5, 0.25), friction=0.0)
    model, state = d.build(8)
    st = wd.batch(state, 1)
    for k in range(180):
        oracle.step_(model, st, d.settings, 1.0 / 60.0)
        if k >= 20:
            v, w, y = st.bodies.v[0, b], float(st.bodies.w[0, b]), float(st.bodies.c[0, b, 1])
            # resting height: half height + both skins - linear_slop = 0.25 + 0.02 - 0.005
            assert abs(v[0] - 4.0) < 0.02 and abs(v[1]) < 0.02 and abs(w) < 0.02 and abs(y - 0.265) < 2e-3, (k, v, w, y)
    assert float(st.bodies.c[0, b, 0]) > 3.5


def test_ball_rolls_down_chain_slope(oracle):
    """A ball rolling without slipping down a chain of collinear edges at slope a accelerates at (5/7) g sin a
    (solid disc: (2/3) g sin a) - rolling-friction-free closed form - across the junctions."""
    a = 0.2
    d = wd.WorldDef(S.stock(gravity=(0.0, -10.0)))
    g = d.add_body(wd.STATIC)
    pts = [(np.cos(a) * s, -np.sin(a) * s) for s in np.arange(0.0, 30.0, 0.4)]
    d.add_chain(g, pts, friction=1.0)
    r, mass = 0.25, 1.0
    c0 = np.array([np.cos(a) * 1.0, -np.sin(a) * 1.0]) + (r + 0.0) * np.array([np.sin(a), np.cos(a)])
    b = d.add_body(wd.DYNAMIC, tuple(c0), mass=mass, inertia=0.5 * mass * r * r)
    d.add_circle(b, r, friction=1.0)
    model, state = d.build(8)
    st = wd.batch(state, 1)
    dt, steps = 1.0 / 60.0, 120
    for _ in range(steps):
        oracle.step_(model, st, d.settings, dt)
    v = st.bodies.v[0, b].astype(np.float64)
    speed = float(np.linalg.norm(v))
    expect = (2.0 / 3.0) * 10.0 * np.sin(a) * dt * steps
    assert abs(speed - expect) / expect < 0.02, (speed, expect)
    along = np.array([np.cos(a), -np.sin(a)])
    assert abs(np.dot(v, along) - speed) < 1e-2 * speed  # moving along the slope, not bouncing
