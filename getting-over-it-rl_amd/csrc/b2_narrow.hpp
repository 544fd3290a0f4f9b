// b2_narrow.hpp - Box2D 2.3.1 narrowphase on the device: b2CollidePolygons, b2CollidePolygonAndCircle,
// b2CollideCircles (goi_jax/box2d/collide.py:22-207), and the edge colliders the reference leaves out. Only the
// collider of the slot's shape pair runs (the reference evaluates all three and selects, collide.py:197-207). Vertex
// loops run over the real count (<= 8) instead of masked (8 x 8) tiles; Box2D's strict `<` / `>` running extremes
// give the reference's first-index argmin/argmax.
//
// Manifold fields that the reference leaves as don't-care (collide.py:5-7) follow its values: on an early out only
// count = 0 matters (the caller keeps the old geometry, pairs.py:73-81); with one kept clip point, point slot 1 holds
// the second clip point (collide.py:122-127); polygon-circle and circle-circle write the circle centre and key 0 into
// both point slots (collide.py:168-170, 184-186).
#pragma once

#include "b2_view.hpp"

namespace goi {

enum { kCircles = 0, kFaceA = 1, kFaceB = 2 };

struct Manifold {
    int mtype, count;
    V2 ln, lp, pl0, pl1;
    int id0, id1;
};

GOI_D int feature_key(int ia, int ib, int ta, int tb) { return ia | (ib << 8) | (ta << 16) | (tb << 24); }

GOI_D V2 mvert(const DModel& m, int f, int i) { return m.poly[16 * f + i]; }
GOI_D V2 mnorm(const DModel& m, int f, int i) { return m.poly[16 * f + 8 + i]; }

// the smallest separation of poly2's first c2 vertices (of kN slots) from the plane through v1 with normal n
template <int kN>
GOI_D float face_min_separation(V2 n, V2 v1, const V2* v2s, int c2) {
    float si = kMaxFloat;
#pragma unroll
    for (int j = 0; j < kN; ++j) {
        if (j < c2) {
            const float sij = dot(n, v2s[j] - v1);
            if (sij < si) si = sij;
        }
    }
    return si;
}

// b2FindMaxSeparation: (edge of poly1, separation) over poly1's normals against poly2's vertices; poly1's normals
// split over the lane group. Most shapes are quads: their vertex loop runs over 4 slots, not 8.
template <class Grp>
GOI_D float max_separation(const DModel& m, int f1, const Xf& xf1, int f2, const Xf& xf2, int& edge, const Grp& g) {
    const int c1 = m.fix[f1].count, c2 = m.fix[f2].count;
    const Xf xf = mulT(xf2, xf1);
    // every slot of the padded [F, 8] tables is loaded, so the loads issue together with the counts' instead of
    // after them; the slots at or past a count are never used
    V2 v2s[kPoly];
#pragma unroll
    for (int j = 0; j < kPoly; ++j) v2s[j] = mvert(m, f2, j);
    int best = 0;
    float maxsep = -kMaxFloat;
#pragma unroll
    for (int i = g.sub(); i < kPoly; i += g.G()) {
        const V2 ni = mnorm(m, f1, i), vi = mvert(m, f1, i);
        if (i >= c1) break;
        const V2 n = mul(xf.q, ni);
        const V2 v1 = mul(xf, vi);
        float si;
        if (c2 <= 4) si = face_min_separation<4>(n, v1, v2s, c2);
        else si = face_min_separation<kPoly>(n, v1, v2s, c2);
        if (si > maxsep) {
            maxsep = si;
            best = i;
        }
    }
    group_argmax(g, maxsep, best);
    edge = best;
    return maxsep;
}

struct ClipV {
    V2 v;
    int ia, ib, ta, tb;
};

// b2ClipSegmentToLine for two input vertices; returns numOut
GOI_D int clip_line(ClipV& o0, ClipV& o1, const ClipV& i0, const ClipV& i1, V2 n, float offset, int vidx) {
    const float d0 = dot(n, i0.v) - offset;
    const float d1 = dot(n, i1.v) - offset;
    const bool in0 = d0 <= 0.0f, in1 = d1 <= 0.0f;
    int num = (int)in0 + (int)in1;
    ClipV x;
    x.v = mk(0.0f, 0.0f);
    x.ia = vidx; x.ib = i0.ib; x.ta = 0; x.tb = 1;  // vertex A hits edge B
    if (d0 * d1 < 0.0f) {
        const float interp = d0 / (d0 - d1);
        x.v = i0.v + interp * (i1.v - i0.v);
        ++num;
    }
    o0 = in0 ? i0 : i1;
    o1 = (in0 && in1) ? i1 : x;
    return num;
}

template <class Grp>
GOI_D void collide_polygons(const DModel& m, int fa, const Xf& xfa, int fb, const Xf& xfb, float linear_slop,
                            Manifold& out, const Grp& g) {
    out.count = 0;
    const float total_radius = m.fix[fa].radius + m.fix[fb].radius;
    int edge_a, edge_b;
    const float sep_a = max_separation(m, fa, xfa, fb, xfb, edge_a, g);
    if (sep_a > total_radius) return;
    const float sep_b = max_separation(m, fb, xfb, fa, xfa, edge_b, g);
    if (sep_b > total_radius) return;
    const float k_tol = 0.1f * linear_slop;
    const bool flip = sep_b > sep_a + k_tol;
    const int f1 = flip ? fb : fa, f2 = flip ? fa : fb;
    const Xf xf1 = flip ? xfb : xfa, xf2 = flip ? xfa : xfb;
    const int edge1 = flip ? edge_b : edge_a;
    out.mtype = flip ? kFaceB : kFaceA;

    // b2FindIncidentEdge
    const int c2 = m.fix[f2].count;
    const V2 n1 = mulT(xf2.q, mul(xf1.q, mnorm(m, f1, edge1)));
    int idx = 0;
    float mind = kMaxFloat;
#pragma unroll
    for (int i = g.sub(); i < kPoly; i += g.G()) {
        const V2 ni = mnorm(m, f2, i);
        if (i >= c2) break;
        const float d = dot(n1, ni);
        if (d < mind) {
            mind = d;
            idx = i;
        }
    }
    group_argmin(g, mind, idx);
    const int i2 = idx + 1 < c2 ? idx + 1 : 0;
    ClipV inc0, inc1;
    inc0.v = mul(xf2, mvert(m, f2, idx)); inc0.ia = edge1; inc0.ib = idx; inc0.ta = 1; inc0.tb = 0;
    inc1.v = mul(xf2, mvert(m, f2, i2));  inc1.ia = edge1; inc1.ib = i2;  inc1.ta = 1; inc1.tb = 0;

    const int c1 = m.fix[f1].count;
    const int iv1 = edge1, iv2 = edge1 + 1 < c1 ? edge1 + 1 : 0;
    V2 v11 = mvert(m, f1, iv1), v12 = mvert(m, f1, iv2);
    V2 lt = v12 - v11;
    normalize(lt);
    const V2 ln = cross(lt, 1.0f);
    const V2 plane = 0.5f * (v11 + v12);
    const V2 tangent = mul(xf1.q, lt);
    const V2 normal = cross(tangent, 1.0f);
    v11 = mul(xf1, v11);
    v12 = mul(xf1, v12);
    const float front = dot(normal, v11);
    const float side1 = -dot(tangent, v11) + total_radius;
    const float side2 = dot(tangent, v12) + total_radius;

    ClipV a0, a1, b0, b1;
    if (clip_line(a0, a1, inc0, inc1, -tangent, side1, iv1) < 2) return;
    if (clip_line(b0, b1, a0, a1, tangent, side2, iv2) < 2) return;

    out.ln = ln;
    out.lp = plane;
    const bool k0 = dot(normal, b0.v) - front <= total_radius;
    const bool k1 = dot(normal, b1.v) - front <= total_radius;
    const V2 p0 = mulT(xf2, b0.v), p1 = mulT(xf2, b1.v);
    const int id0 = flip ? feature_key(b0.ib, b0.ia, b0.tb, b0.ta) : feature_key(b0.ia, b0.ib, b0.ta, b0.tb);
    const int id1 = flip ? feature_key(b1.ib, b1.ia, b1.tb, b1.ta) : feature_key(b1.ia, b1.ib, b1.ta, b1.tb);
    out.count = (int)k0 + (int)k1;
    out.pl0 = k0 ? p0 : p1;
    out.id0 = k0 ? id0 : id1;
    out.pl1 = p1;
    out.id1 = id1;
}

// The face loop splits over the lane group; the early out on any separating face is the sequential one (nothing
// but count = 0 is written before it).
template <class Grp>
GOI_D void collide_polygon_circle(const DModel& m, int fa, const Xf& xfa, int fb, const Xf& xfb, Manifold& out,
                                  const Grp& g) {
    out.count = 0;
    const V2 cl = mulT(xfa, mul(xfb, mvert(m, fb, 0)));
    const float radius = m.fix[fa].radius + m.fix[fb].radius;
    const int n = m.fix[fa].count;
    int ni = 0;
    float sep = -kMaxFloat;
    bool apart = false;
    for (int i = g.sub(); i < n; i += g.G()) {
        const float s = dot(mnorm(m, fa, i), cl - mvert(m, fa, i));
        if (s > radius) {
            apart = true;
            break;
        }
        if (s > sep) {
            sep = s;
            ni = i;
        }
    }
    if (group_any(g, apart)) return;
    group_argmax(g, sep, ni);
    const int i2 = ni + 1 < n ? ni + 1 : 0;
    const V2 v1 = mvert(m, fa, ni), v2 = mvert(m, fa, i2);
    const V2 centre = mvert(m, fb, 0);
    out.mtype = kFaceA;
    out.pl0 = centre; out.pl1 = centre;
    out.id0 = 0; out.id1 = 0;
    if (sep < kEps) {
        out.count = 1;
        out.ln = mnorm(m, fa, ni);
        out.lp = 0.5f * (v1 + v2);
        return;
    }
    const float u1 = dot(cl - v1, v2 - v1);
    const float u2 = dot(cl - v2, v1 - v2);
    const float rr = radius * radius;
    if (u1 <= 0.0f) {
        V2 d = cl - v1;
        if (dot(d, d) > rr) return;
        normalize(d);
        out.count = 1; out.ln = d; out.lp = v1;
    } else if (u2 <= 0.0f) {
        V2 d = cl - v2;
        if (dot(d, d) > rr) return;
        normalize(d);
        out.count = 1; out.ln = d; out.lp = v2;
    } else {
        const V2 fc = 0.5f * (v1 + v2);
        if (dot(cl - fc, mnorm(m, fa, ni)) > radius) return;
        out.count = 1; out.ln = mnorm(m, fa, ni); out.lp = fc;
    }
}

GOI_D void collide_circles(const DModel& m, int fa, const Xf& xfa, int fb, const Xf& xfb, Manifold& out) {
    out.count = 0;
    const V2 d = mul(xfb, mvert(m, fb, 0)) - mul(xfa, mvert(m, fa, 0));
    const float r = m.fix[fa].radius + m.fix[fb].radius;
    if (dot(d, d) > r * r) return;
    out.mtype = kCircles;
    out.count = 1;
    out.ln = mk(0.0f, 0.0f);
    out.lp = mvert(m, fa, 0);
    out.pl0 = mvert(m, fb, 0); out.pl1 = out.pl0;
    out.id0 = 0; out.id1 = 0;
}

// Native edge shapes, which the reference does not have (goi_jax/box2d/shapes.py:13): Box2D 2.3.1's
// b2CollideEdgeAndCircle and b2EPCollider (b2CollideEdge.cpp). Edge fixture f holds m_vertex1, m_vertex2 in
// vertices 0-1 and the ghost vertices m_vertex0, m_vertex3 in vertices 2-3; edge_flags[f] says which ghosts exist.
// The unused point slot follows the polygon convention above.

// b2CollideEdgeAndCircle: regions A and B give vertex contacts unless the neighbouring edge owns the circle; region
// AB a face contact with the normal on the circle's side.
GOI_D void collide_edge_circle(const DModel& m, int fa, const Xf& xfa, int fb, const Xf& xfb, Manifold& out) {
    out.count = 0;
    const V2 q = mulT(xfa, mul(xfb, mvert(m, fb, 0)));
    const V2 a = mvert(m, fa, 0), b = mvert(m, fa, 1);
    const V2 e = b - a;
    const float u = dot(e, b - q), v = dot(e, q - a);  // barycentric coordinates
    const float radius = m.fix[fa].radius + m.fix[fb].radius;
    const int flags = m.fix[fa].edge_flags;
    out.pl0 = mvert(m, fb, 0); out.pl1 = out.pl0;
    out.mtype = kCircles;
    out.ln = mk(0.0f, 0.0f);
    if (v <= 0.0f) {  // region A
        const V2 d = q - a;
        if (dot(d, d) > radius * radius) return;
        if ((flags & GOI_EDGE_HAS_V0) && dot(a - mvert(m, fa, 2), a - q) > 0.0f) return;
        out.count = 1; out.lp = a;
        out.id0 = feature_key(0, 0, 0, 0); out.id1 = out.id0;
        return;
    }
    if (u <= 0.0f) {  // region B
        const V2 d = q - b;
        if (dot(d, d) > radius * radius) return;
        if ((flags & GOI_EDGE_HAS_V3) && dot(mvert(m, fa, 3) - b, q - b) > 0.0f) return;
        out.count = 1; out.lp = b;
        out.id0 = feature_key(1, 0, 0, 0); out.id1 = out.id0;
        return;
    }
    const float den = dot(e, e);  // region AB
    const V2 p = (1.0f / den) * (u * a + v * b);
    const V2 d = q - p;
    if (dot(d, d) > radius * radius) return;
    V2 n = mk(-e.y, e.x);
    if (dot(n, q - a) < 0.0f) n = mk(-n.x, -n.y);
    normalize(n);
    out.mtype = kFaceA; out.count = 1;
    out.ln = n; out.lp = a;
    out.id0 = feature_key(0, 0, 1, 0); out.id1 = out.id0;
}

// b2EPCollider::Collide: edge A against polygon B in A's frame. The polygon centroid's side of the edge and the
// neighbouring edges (ghost vertices) fix the collision normal and the admissible range of polygon normals; the
// edge axis or the deepest admissible polygon axis (hysteresis 0.98 / 0.001) gives the reference face, and the
// incident edge is clipped to its sides (no radius on the side planes). Skin radius 2 * b2_polygonRadius. Polygon
// B's vertices and normals are transformed into A's frame where used rather than staged in registers.
GOI_D void collide_edge_polygon(const DModel& m, int fa, const Xf& xfa, int fb, const Xf& xfb, const GoiSettings& s,
                                Manifold& out) {
    out.count = 0;
    const Xf xf = mulT(xfa, xfb);
    const V2 cb = mul(xf, m.fix[fb].centroid);
    const V2 v1 = mvert(m, fa, 0), v2 = mvert(m, fa, 1);
    const int flags = m.fix[fa].edge_flags;
    const bool has0 = (flags & GOI_EDGE_HAS_V0) != 0, has3 = (flags & GOI_EDGE_HAS_V3) != 0;
    V2 edge1 = v2 - v1;
    normalize(edge1);
    const V2 n1 = mk(edge1.y, -edge1.x);
    const float offset1 = dot(n1, cb - v1);
    float offset0 = 0.0f, offset2 = 0.0f;
    bool convex1 = false, convex2 = false;
    V2 n0 = mk(0.0f, 0.0f), n2 = mk(0.0f, 0.0f);
    if (has0) {
        const V2 v0 = mvert(m, fa, 2);
        V2 edge0 = v1 - v0;
        normalize(edge0);
        n0 = mk(edge0.y, -edge0.x);
        convex1 = cross(edge0, edge1) >= 0.0f;
        offset0 = dot(n0, cb - v0);
    }
    if (has3) {
        V2 edge2 = mvert(m, fa, 3) - v2;
        normalize(edge2);
        n2 = mk(edge2.y, -edge2.x);
        convex2 = cross(edge1, edge2) > 0.0f;
        offset2 = dot(n2, cb - v2);
    }
    bool front;
    V2 lower, upper;
    if (has0 && has3) {
        if (convex1 && convex2) {
            front = offset0 >= 0.0f || offset1 >= 0.0f || offset2 >= 0.0f;
            lower = front ? n0 : -n1; upper = front ? n2 : -n1;
        } else if (convex1) {
            front = offset0 >= 0.0f || (offset1 >= 0.0f && offset2 >= 0.0f);
            lower = front ? n0 : -n2; upper = front ? n1 : -n1;
        } else if (convex2) {
            front = offset2 >= 0.0f || (offset0 >= 0.0f && offset1 >= 0.0f);
            lower = front ? n1 : -n1; upper = front ? n2 : -n0;
        } else {
            front = offset0 >= 0.0f && offset1 >= 0.0f && offset2 >= 0.0f;
            lower = front ? n1 : -n2; upper = front ? n1 : -n0;
        }
    } else if (has0) {
        if (convex1) {
            front = offset0 >= 0.0f || offset1 >= 0.0f;
            lower = front ? n0 : n1; upper = -n1;
        } else {
            front = offset0 >= 0.0f && offset1 >= 0.0f;
            lower = n1; upper = front ? -n1 : -n0;
        }
    } else if (has3) {
        if (convex2) {
            front = offset1 >= 0.0f || offset2 >= 0.0f;
            lower = -n1; upper = front ? n2 : n1;
        } else {
            front = offset1 >= 0.0f && offset2 >= 0.0f;
            lower = front ? -n1 : -n2; upper = n1;
        }
    } else {
        front = offset1 >= 0.0f;
        lower = front ? -n1 : n1; upper = lower;
    }
    const V2 normal = front ? n1 : -n1;
    const int cnt = m.fix[fb].count;
    const float radius = 2.0f * s.polygon_radius;

    // ComputeEdgeSeparation (the edge axis is always known)
    float edge_sep = kMaxFloat;
    for (int i = 0; i < cnt; ++i) {
        const float sv = dot(normal, mul(xf, mvert(m, fb, i)) - v1);
        if (sv < edge_sep) edge_sep = sv;
    }
    if (edge_sep > radius) return;

    // ComputePolygonSeparation: the first separating polygon axis, else the deepest admissible one
    int poly_index = -1;
    float poly_sep = -kMaxFloat;
    const V2 perp = mk(-normal.y, normal.x);
    for (int i = 0; i < cnt; ++i) {
        const V2 n = -mul(xf.q, mnorm(m, fb, i));
        const V2 pv = mul(xf, mvert(m, fb, i));
        const float sv = bmin(dot(n, pv - v1), dot(n, pv - v2));
        if (sv > radius) {
            poly_index = i;
            poly_sep = sv;
            break;
        }
        const V2 lim = dot(n, perp) >= 0.0f ? upper : lower;
        if (dot(n - lim, normal) < -s.angular_slop) continue;
        if (sv > poly_sep) {
            poly_index = i;
            poly_sep = sv;
        }
    }
    if (poly_index >= 0 && poly_sep > radius) return;

    const bool edge_primary = poly_index < 0 || !(poly_sep > 0.98f * edge_sep + 0.001f);
    ClipV ie0, ie1;
    int rf_i1, rf_i2;
    V2 rf_v1, rf_v2, rf_n;
    if (edge_primary) {
        int best = 0;  // the polygon normal most anti-parallel to the edge normal
        float bestv = dot(normal, mul(xf.q, mnorm(m, fb, 0)));
        for (int i = 1; i < cnt; ++i) {
            const float val = dot(normal, mul(xf.q, mnorm(m, fb, i)));
            if (val < bestv) {
                bestv = val;
                best = i;
            }
        }
        const int i2 = best + 1 < cnt ? best + 1 : 0;
        ie0.v = mul(xf, mvert(m, fb, best)); ie0.ia = 0; ie0.ib = best; ie0.ta = 1; ie0.tb = 0;
        ie1.v = mul(xf, mvert(m, fb, i2));   ie1.ia = 0; ie1.ib = i2;   ie1.ta = 1; ie1.tb = 0;
        rf_i1 = front ? 0 : 1; rf_i2 = front ? 1 : 0;
        rf_v1 = front ? v1 : v2; rf_v2 = front ? v2 : v1;
        rf_n = normal;
    } else {
        ie0.v = v1; ie0.ia = 0; ie0.ib = poly_index; ie0.ta = 0; ie0.tb = 1;
        ie1.v = v2; ie1.ia = 0; ie1.ib = poly_index; ie1.ta = 0; ie1.tb = 1;
        rf_i1 = poly_index;
        rf_i2 = rf_i1 + 1 < cnt ? rf_i1 + 1 : 0;
        rf_v1 = mul(xf, mvert(m, fb, rf_i1));
        rf_v2 = mul(xf, mvert(m, fb, rf_i2));
        rf_n = mul(xf.q, mnorm(m, fb, rf_i1));
    }
    const V2 side1 = mk(rf_n.y, -rf_n.x);
    const V2 side2 = -side1;
    ClipV a0, a1, b0, b1;
    if (clip_line(a0, a1, ie0, ie1, side1, dot(side1, rf_v1), rf_i1) < 2) return;
    if (clip_line(b0, b1, a0, a1, side2, dot(side2, rf_v2), rf_i2) < 2) return;
    out.mtype = edge_primary ? kFaceA : kFaceB;
    out.ln = edge_primary ? rf_n : mnorm(m, fb, rf_i1);
    out.lp = edge_primary ? rf_v1 : mvert(m, fb, rf_i1);
    const bool k0 = dot(rf_n, b0.v - rf_v1) <= radius;
    const bool k1 = dot(rf_n, b1.v - rf_v1) <= radius;
    const V2 p0 = edge_primary ? mulT(xf, b0.v) : b0.v;
    const V2 p1 = edge_primary ? mulT(xf, b1.v) : b1.v;
    const int id0 = edge_primary ? feature_key(b0.ia, b0.ib, b0.ta, b0.tb) : feature_key(b0.ib, b0.ia, b0.tb, b0.ta);
    const int id1 = edge_primary ? feature_key(b1.ia, b1.ib, b1.ta, b1.tb) : feature_key(b1.ib, b1.ia, b1.tb, b1.ta);
    out.count = (int)k0 + (int)k1;
    out.pl0 = k0 ? p0 : p1;
    out.id0 = k0 ? id0 : id1;
    out.pl1 = p1;
    out.id1 = id1;
}

// b2Contact::Evaluate by shape types (b2Contact::Create puts a polygon before a circle and an edge before either)
template <class Grp>
GOI_D void evaluate(const DModel& m, int fa, int fb, const Xf& xfa, const Xf& xfb, const GoiSettings& s,
                    Manifold& out, const Grp& g) {
    const int ta = m.fix[fa].type, tb = m.fix[fb].type;
    if (ta == GOI_POLYGON && tb == GOI_POLYGON) collide_polygons(m, fa, xfa, fb, xfb, s.linear_slop, out, g);
    else if (ta == GOI_POLYGON) collide_polygon_circle(m, fa, xfa, fb, xfb, out, g);
    else if (!m.no_edges && ta == GOI_EDGE && tb == GOI_POLYGON) collide_edge_polygon(m, fa, xfa, fb, xfb, s, out);
    else if (!m.no_edges && ta == GOI_EDGE) collide_edge_circle(m, fa, xfa, fb, xfb, out);
    else collide_circles(m, fa, xfa, fb, xfb, out);
}
GOI_D void evaluate(const DModel& m, int fa, int fb, const Xf& xfa, const Xf& xfb, const GoiSettings& s,
                    Manifold& out) {
    evaluate(m, fa, fb, xfa, xfb, s, out, Solo{});
}

}  // namespace goi
