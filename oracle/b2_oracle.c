/* b2_oracle.c - CPU restatement of goi_jax.box2d's world step (TEST INFRASTRUCTURE ONLY).
 *
 * This is the parity oracle and the CPU baseline. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it; the product path (libgoi_b2.so) never links or calls it.
 *
 * It restates the reference's algorithm (the modules of goi_jax/box2d at the cited lines) as plain sequential C, one world
 * at a time, in Box2D 2.3.1's own loop structure: the contact list walked newest first, the island DFS, the
 * Gauss-Seidel sweeps, SolveTOI's event loop. The reference vectorises these walks (wake fixed point pairs.py:90-117,
 * prefix-sum DFS island.py:41-140, single-evaluation TOI walk toi.py:9-26) and documents each as exact against the
 * sequential semantics; this file follows the sequential semantics those docstrings state. Where the reference
 * deliberately differs from Box2D it is followed, not Box2D:
 *   - every contact counts as enabled in Solve; SolveTOI resets e_enabledFlag (toi.py:32-34, world.py:157-161);
 *   - at most max_events TOI events per step (toi.py:838-847);
 *   - Solve runs even when dt <= 0 (step.py:35-40; only SolveTOI checks dt, toi.py:841);
 *   - the don't-care fields of an updated manifold (point 1 when pointCount < 2, mtype on an early out) take the
 *     reference's values (collide.py:113-127, pairs.py:56-83), so whole State leaves can be compared bit for bit.
 *
 * Floating point: one rounding per C operation in C order (build with -ffp-contract=off, no fast-math), denormals
 * kept, sin/cos = (float)sin((double)x) from the C library (the reference oracle's trig_mode=1,
 * scripts/patches/box2d-2.3.1-trig.patch:17-23; math2d.py:291-310 reproduces it).
 *
 * Parity pinning (tests/test_oracle_pins.py, tests/test_edges.py; tests/test_oracle_mutants.py plants 50 slips and
 * shows each pin catching its slip): semi-implicit Euler closed form (tests/reference/test_box2d_reference.py:22-35),
 * resting-contact impulse m*g*dt and sqrt friction mix (:49-63), sleeping (:38-46), pendulum radius/energy (:90-110),
 * revolute limit and motor (:112-127), TOI ball stopped / discrete ball tunnels (test_toi.py:181-185,
 * test_box2d_reference.py:130-155); one pass of each position row (contact, revolute point and limit, prismatic,
 * rigid and soft weld) checked by the defining conditions of a non-linear Gauss-Seidel step (the linearized error
 * reaches the row's target, the move is along M^-1 J^T); the revolute velocity rows' motor and limit impulses; the
 * velocity rows' result by the constraint invariant; the block solver's result by the two-point LCP conditions and
 * its condition-number fallback; b2CollidePolygons known answers, exact face ties and incident-edge ties included;
 * the Collide wake cascade in list order; the TOI event island walk's order and 32-contact cap (with its trace), its
 * membership rule and the tie rules; b2TimeOfImpact's root steps and target contract; narrowphase, GJK and the
 * broadphase candidate scan against brute force; islands against an independent DFS.
 *
 * Parity unpinned: the reference commits no golden vectors for this path and can be run neither here (jax absent)
 * nor from source (Box2D 2.3.1 is fetched over the network). These parts are right only by faithful reading of the
 * cited reference text:
 *   - the block solver's choice among its four cases where two of them accept (only at exact float boundaries of
 *     the LCP's active set; the result is pinned by the LCP conditions) (contact_solver.py:236-279);
 *   - time_of_impact / distance iteration paths beyond the head-on root steps and the target contract
 *     (toi.py:230-459);
 *   - the native edge colliders collide_edge_circle / collide_edge_polygon, which have no reference function (the
 *     reference has no edge shape, shapes.py:13): they restate Box2D 2.3.1's b2CollideEdge.cpp and are pinned by
 *     closed forms, brute force and the thin-quad polygon path only (tests/test_edges.py).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "../include/goi_b2.h"

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------------------------------ constants */

#define EPS 1.1920928955078125e-7f /* b2_epsilon = FLT_EPSILON */
#define MAXF 3.40282346638528859812e+38f /* b2_maxFloat */
#define MAX_SUB_STEPS 8
#define MAX_TOI_CONTACTS 32
#define NPOLY GOI_MAX_POLY
#define CIRCLES 0
#define FACE_A 1
#define FACE_B 2
#define E_VERTEX 0
#define E_FACE 1
#define INACTIVE_LIMIT 0
#define AT_LOWER 1
#define AT_UPPER 2
#define EQUAL_LIMITS 3

/* ------------------------------------------------------------------------------------------------ math (math2d.py) */

typedef struct { float x, y; } V2;
typedef struct { float c, s; } Rot;
typedef struct { V2 p; Rot q; } Xf;

static inline V2 v2(float x, float y) { V2 r = {x, y}; return r; }
static inline V2 add(V2 a, V2 b) { return v2(a.x + b.x, a.y + b.y); }
static inline V2 sub(V2 a, V2 b) { return v2(a.x - b.x, a.y - b.y); }
static inline V2 neg(V2 a) { return v2(-a.x, -a.y); }
static inline V2 scl(float s, V2 a) { return v2(s * a.x, s * a.y); }          /* s * v */
static inline float dot(V2 a, V2 b) { return a.x * b.x + a.y * b.y; }          /* b2Dot */
static inline float crs(V2 a, V2 b) { return a.x * b.y - a.y * b.x; }          /* b2Cross(v, v) */
static inline V2 crs_vs(V2 a, float s) { return v2(s * a.y, -s * a.x); }       /* b2Cross(v, s) */
static inline V2 crs_sv(float s, V2 a) { return v2(-s * a.y, s * a.x); }       /* b2Cross(s, v) */
static inline V2 rmul(Rot q, V2 v) { return v2(q.c * v.x - q.s * v.y, q.s * v.x + q.c * v.y); }
static inline V2 rmulT(Rot q, V2 v) { return v2(q.c * v.x + q.s * v.y, -q.s * v.x + q.c * v.y); }
static inline V2 xmul(Xf t, V2 v) {
    return v2((t.q.c * v.x - t.q.s * v.y) + t.p.x, (t.q.s * v.x + t.q.c * v.y) + t.p.y);
}
static inline V2 xmulT(Xf t, V2 v) {
    float px = v.x - t.p.x, py = v.y - t.p.y;
    return v2(t.q.c * px + t.q.s * py, -t.q.s * px + t.q.c * py);
}
static inline Rot rmulT_rot(Rot q, Rot r) { /* b2MulT(q, r) */
    Rot o; o.s = q.c * r.s - q.s * r.c; o.c = q.c * r.c + q.s * r.s; return o;
}
static inline Xf xmulT_xf(Xf A, Xf B) { /* b2MulT(A, B) */
    Xf C; C.q = rmulT_rot(A.q, B.q); C.p = rmulT(A.q, sub(B.p, A.p)); return C;
}
static inline float len(V2 a) { return sqrtf(a.x * a.x + a.y * a.y); }
static inline float normalize(V2* a) { /* b2Vec2::Normalize (math2d.py:102-107) */
    float n = len(*a);
    if (n < EPS) return 0.0f;
    float inv = 1.0f / n;
    a->x *= inv; a->y *= inv;
    return n;
}
static inline float bmin(float a, float b) { return a < b ? a : b; }
static inline float bmax(float a, float b) { return a > b ? a : b; }
static inline float bclamp(float a, float lo, float hi) { return bmax(lo, bmin(a, hi)); }
static inline float babs(float a) { return a > 0.0f ? a : -a; }

/* correctly rounded float sin/cos: (float)sin((double)x), the trig patch's definition (math2d.py:291-310) */
static inline Rot rot_of(float a) { Rot q; q.s = (float)sin((double)a); q.c = (float)cos((double)a); return q; }

/* b2Mat22::Solve / b2Mat33::Solve22 (math2d.py:162-166) */
static inline V2 solve22(float a11, float a12, float a21, float a22, V2 b) {
    float det = a11 * a22 - a12 * a21;
    if (det != 0.0f) det = 1.0f / det;
    return v2(det * (a22 * b.x - a12 * b.y), det * (a11 * b.y - a21 * b.x));
}
typedef struct { float x, y, z; } V3;
static inline V3 v3(float x, float y, float z) { V3 r = {x, y, z}; return r; }
static inline float dot3(V3 a, V3 b) { return (a.x * b.x + a.y * b.y) + a.z * b.z; }
static inline V3 cross3(V3 a, V3 b) {
    return v3(a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x);
}
/* b2Mat33::Solve33 (math2d.py:175-182), columns ex, ey, ez */
static inline V3 solve33(V3 ex, V3 ey, V3 ez, V3 b) {
    float det = dot3(ex, cross3(ey, ez));
    if (det != 0.0f) det = 1.0f / det;
    return v3(det * dot3(b, cross3(ey, ez)), det * dot3(ex, cross3(b, ez)), det * dot3(ex, cross3(ey, b)));
}

/* ------------------------------------------------------------------------------------------------ per-world view */

typedef struct {
    int B, C, R, J;
    int32_t* b_type; uint8_t *b_active, *b_awake, *b_allow_sleep, *b_bullet, *b_continuous;
    float *b_sleep_time, *b_xf_p, *b_xf_q, *b_lc, *b_c0, *b_c, *b_a0, *b_a, *b_v, *b_w, *b_force, *b_torque;
    float *b_mass, *b_inv_mass, *b_inertia, *b_inv_inertia, *b_ld, *b_ad, *b_gs;
    float *f_friction, *f_restitution, *f_fat;
    uint8_t* j_enable_motor; float *j_motor_speed, *j_max_motor; uint8_t* j_enable_limit;
    float *j_lower, *j_upper, *j_frequency, *j_damping, *j_impulse, *j_motor_impulse;
    int32_t* j_limit_state; float *j_lower_impulse, *j_upper_impulse;
    int32_t *c_pair, *c_fa, *c_fb, *c_key; uint8_t* c_touching; int32_t *c_mtype, *c_count;
    float *c_ln, *c_lp, *c_pl; int32_t* c_pid; float *c_ni, *c_ti, *c_friction, *c_restitution, *c_tangent_speed;
    float *gravity, *inv_dt0; int32_t* next_key; uint8_t* new_fixture; int32_t* overflow;
    float* t_alpha0; int32_t* t_count; float* t_toi; uint8_t *t_flag, *t_enabled, *t_solved;
    float *t_ni, *t_ti; int32_t* t_events;
} W;

typedef struct {
    const GoiModelDesc* m;
    const GoiSettings* s;
    float dt;
    int compact; /* the State holds only the non-static fixture rows (world.py:400-403: a compact Model and fewer rows
                    than fixtures); otherwise every fixture has its row, whatever the Model's layout */
} Ctx;

/* body transform, sweep pieces */
static inline Xf body_xf(const W* w, int b) {
    Xf t; t.p = v2(w->b_xf_p[2 * b], w->b_xf_p[2 * b + 1]); t.q.c = w->b_xf_q[2 * b]; t.q.s = w->b_xf_q[2 * b + 1];
    return t;
}
static inline V2 getv(const float* a, int i) { return v2(a[2 * i], a[2 * i + 1]); }
static inline void setv(float* a, int i, V2 v) { a[2 * i] = v.x; a[2 * i + 1] = v.y; }

/* b2Body::SetAwake(true): sleep time zeroed only if it was asleep (pairs.py:126-131) */
static inline void wake(W* w, int b) {
    if (!w->b_awake[b]) { w->b_awake[b] = 1; w->b_sleep_time[b] = 0.0f; }
}

/* fixture accessors in either layout (world.py:413-434) */
static inline const float* fat_of(const Ctx* x, const W* w, int f) {
    const GoiModelDesc* m = x->m;
    if (x->compact) {
        int r = m->fixture_slot[f];
        return r >= 0 ? w->f_fat + 4 * r : m->static_fat + 4 * f;
    }
    return w->f_fat + 4 * f;
}
static inline float friction_of(const Ctx* x, const W* w, int f) {
    const GoiModelDesc* m = x->m;
    if (x->compact) {
        int r = m->fixture_slot[f];
        return r >= 0 ? w->f_friction[r] : m->static_friction[f];
    }
    return w->f_friction[f];
}
static inline float restitution_of(const Ctx* x, const W* w, int f) {
    const GoiModelDesc* m = x->m;
    if (x->compact) {
        int r = m->fixture_slot[f];
        return r >= 0 ? w->f_restitution[r] : m->static_restitution[f];
    }
    return w->f_restitution[f];
}
static inline V2 vert(const GoiModelDesc* m, int f, int i) {
    return v2(m->verts[(f * NPOLY + i) * 2], m->verts[(f * NPOLY + i) * 2 + 1]);
}
static inline V2 nrm(const GoiModelDesc* m, int f, int i) {
    return v2(m->normals[(f * NPOLY + i) * 2], m->normals[(f * NPOLY + i) * 2 + 1]);
}

/* ------------------------------------------------------------------------------------------------ AABBs (shapes.py) */

typedef struct { float lx, ly, ux, uy; } AABB;

/* b2Shape::ComputeAABB (shapes.py:118-133) */
static AABB shape_aabb(const GoiModelDesc* m, int f, Xf t) {
    AABB a;
    float r = m->radius[f];
    if (m->shape_type[f] == GOI_CIRCLE) {
        V2 p = add(t.p, rmul(t.q, vert(m, f, 0))); /* rotation first, then add */
        a.lx = p.x - r; a.ly = p.y - r; a.ux = p.x + r; a.uy = p.y + r;
        return a;
    }
    V2 lo = xmul(t, vert(m, f, 0)), hi = lo;
    for (int i = 1; i < m->count[f]; ++i) {
        V2 v = xmul(t, vert(m, f, i));
        lo.x = bmin(lo.x, v.x); lo.y = bmin(lo.y, v.y);
        hi.x = bmax(hi.x, v.x); hi.y = bmax(hi.y, v.y);
    }
    a.lx = lo.x - r; a.ly = lo.y - r; a.ux = hi.x + r; a.uy = hi.y + r;
    return a;
}

/* b2TestOverlap (shapes.py:149-153) */
static inline int overlap(const float* a, const float* b) {
    float d1x = b[0] - a[2], d1y = b[1] - a[3];
    float d2x = a[0] - b[2], d2y = a[1] - b[3];
    return !(d1x > 0.0f || d1y > 0.0f || d2x > 0.0f || d2y > 0.0f);
}

/* ------------------------------------------------------------------------------------------------ narrowphase (collide.py) */

typedef struct {
    int32_t mtype, count;
    V2 ln, lp, pl[2];
    int32_t id[2];
} Manifold;

static inline int32_t feature_key(int ia, int ib, int ta, int tb) { /* collide.py:22-24 */
    return ia | (ib << 8) | (ta << 16) | (tb << 24);
}

typedef struct { V2 v; int ia, ib, ta, tb; } ClipV;

/* b2FindMaxSeparation (collide.py:32-42) */
static float find_max_separation(const GoiModelDesc* m, int f1, Xf xf1, int f2, Xf xf2, int* edge) {
    int c1 = m->count[f1], c2 = m->count[f2];
    Xf xf = xmulT_xf(xf2, xf1);
    int best = 0;
    float maxsep = -MAXF;
    for (int i = 0; i < c1; ++i) {
        V2 n = rmul(xf.q, nrm(m, f1, i));
        V2 v1 = xmul(xf, vert(m, f1, i));
        float si = MAXF;
        for (int j = 0; j < c2; ++j) {
            float sij = dot(n, sub(vert(m, f2, j), v1));
            if (sij < si) si = sij;
        }
        if (si > maxsep) { maxsep = si; best = i; }
    }
    *edge = best;
    return maxsep;
}

/* b2ClipSegmentToLine (collide.py:45-62) */
static int clip_segment(ClipV out[2], const ClipV in[2], V2 n, float offset, int vertex_index_a) {
    int num = 0;
    float d0 = dot(n, in[0].v) - offset;
    float d1 = dot(n, in[1].v) - offset;
    if (d0 <= 0.0f) out[num++] = in[0];
    if (d1 <= 0.0f) out[num++] = in[1];
    if (d0 * d1 < 0.0f) {
        float interp = d0 / (d0 - d1);
        out[num].v = add(in[0].v, scl(interp, sub(in[1].v, in[0].v)));
        out[num].ia = vertex_index_a; out[num].ib = in[0].ib;
        out[num].ta = E_VERTEX; out[num].tb = E_FACE;
        ++num;
    }
    return num;
}

/* b2CollidePolygons (collide.py:65-127). Returns count; `out` follows the reference's field values (mtype and
 * geometry only meaningful when count > 0). */
static void collide_polygons(const GoiModelDesc* m, int fa, Xf xfa, int fb, Xf xfb, float linear_slop,
                             Manifold* out) {
    out->count = 0;
    float total_radius = m->radius[fa] + m->radius[fb];
    int edge_a = 0, edge_b = 0;
    float sep_a = find_max_separation(m, fa, xfa, fb, xfb, &edge_a);
    float sep_b = find_max_separation(m, fb, xfb, fa, xfa, &edge_b);
    /* The reference evaluates the whole manifold and masks count afterwards (collide.py:125); mtype, normal and
     * points are kept only where count > 0 (pairs.py:73-81), so an early out leaves them as don't-care. */
    if (sep_a > total_radius || sep_b > total_radius) return;
    float k_tol = 0.1f * linear_slop;
    int flip = sep_b > sep_a + k_tol;
    int f1 = flip ? fb : fa, f2 = flip ? fa : fb;
    Xf xf1 = flip ? xfb : xfa, xf2 = flip ? xfa : xfb;
    int edge1 = flip ? edge_b : edge_a;
    out->mtype = flip ? FACE_B : FACE_A;

    /* b2FindIncidentEdge */
    int c2 = m->count[f2];
    V2 n1 = rmulT(xf2.q, rmul(xf1.q, nrm(m, f1, edge1)));
    int index = 0;
    float mind = MAXF;
    for (int i = 0; i < c2; ++i) {
        float d = dot(n1, nrm(m, f2, i));
        if (d < mind) { mind = d; index = i; }
    }
    int i1 = index, i2 = i1 + 1 < c2 ? i1 + 1 : 0;
    ClipV inc[2];
    inc[0].v = xmul(xf2, vert(m, f2, i1)); inc[0].ia = edge1; inc[0].ib = i1; inc[0].ta = E_FACE; inc[0].tb = E_VERTEX;
    inc[1].v = xmul(xf2, vert(m, f2, i2)); inc[1].ia = edge1; inc[1].ib = i2; inc[1].ta = E_FACE; inc[1].tb = E_VERTEX;

    int c1 = m->count[f1];
    int iv1 = edge1, iv2 = edge1 + 1 < c1 ? edge1 + 1 : 0;
    V2 v11 = vert(m, f1, iv1), v12 = vert(m, f1, iv2);
    V2 tangent_l = sub(v12, v11);
    normalize(&tangent_l);
    V2 normal_l = crs_vs(tangent_l, 1.0f);
    V2 plane_point = scl(0.5f, add(v11, v12));
    V2 tangent = rmul(xf1.q, tangent_l);
    V2 normal = crs_vs(tangent, 1.0f);
    v11 = xmul(xf1, v11);
    v12 = xmul(xf1, v12);
    float front = dot(normal, v11);
    float side1 = -dot(tangent, v11) + total_radius;
    float side2 = dot(tangent, v12) + total_radius;

    ClipV cp1[2], cp2[2];
    int np = clip_segment(cp1, inc, neg(tangent), side1, iv1);
    if (np < 2) return;
    np = clip_segment(cp2, cp1, tangent, side2, iv2);
    if (np < 2) return;

    out->ln = normal_l;
    out->lp = plane_point;
    int keep[2];
    V2 pts[2];
    int32_t ids[2];
    for (int i = 0; i < 2; ++i) {
        float sep = dot(normal, cp2[i].v) - front;
        keep[i] = sep <= total_radius;
        pts[i] = xmulT(xf2, cp2[i].v);
        ids[i] = flip ? feature_key(cp2[i].ib, cp2[i].ia, cp2[i].tb, cp2[i].ta)
                      : feature_key(cp2[i].ia, cp2[i].ib, cp2[i].ta, cp2[i].tb);
    }
    out->count = keep[0] + keep[1];
    /* first kept clip point in slot 0; slot 1 holds the second clip point (collide.py:122-127) */
    out->pl[0] = keep[0] ? pts[0] : pts[1];
    out->id[0] = keep[0] ? ids[0] : ids[1];
    out->pl[1] = pts[1];
    out->id[1] = ids[1];
}

/* b2CollidePolygonAndCircle (collide.py:130-170) */
static void collide_polygon_circle(const GoiModelDesc* m, int fa, Xf xfa, int fb, Xf xfb, Manifold* out) {
    out->count = 0;
    V2 cpos = xmul(xfb, vert(m, fb, 0));
    V2 cl = xmulT(xfa, cpos);
    float radius = m->radius[fa] + m->radius[fb];
    int n = m->count[fa];
    int ni = 0;
    float separation = -MAXF;
    for (int i = 0; i < n; ++i) {
        float s = dot(nrm(m, fa, i), sub(cl, vert(m, fa, i)));
        if (s > radius) return;
        if (s > separation) { separation = s; ni = i; }
    }
    int i1 = ni, i2 = i1 + 1 < n ? i1 + 1 : 0;
    V2 v1 = vert(m, fa, i1), v2_ = vert(m, fa, i2);
    V2 pl = vert(m, fb, 0);
    out->mtype = FACE_A;
    out->pl[0] = pl; out->pl[1] = pl;
    out->id[0] = 0; out->id[1] = 0;
    if (separation < EPS) {
        out->count = 1;
        out->ln = nrm(m, fa, ni);
        out->lp = scl(0.5f, add(v1, v2_));
        return;
    }
    float u1 = dot(sub(cl, v1), sub(v2_, v1));
    float u2 = dot(sub(cl, v2_), sub(v1, v2_));
    float rr = radius * radius;
    if (u1 <= 0.0f) {
        V2 d = sub(cl, v1);
        if (dot(d, d) > rr) return;
        out->count = 1;
        normalize(&d);
        out->ln = d;
        out->lp = v1;
    } else if (u2 <= 0.0f) {
        V2 d = sub(cl, v2_);
        if (dot(d, d) > rr) return;
        out->count = 1;
        normalize(&d);
        out->ln = d;
        out->lp = v2_;
    } else {
        V2 fc = scl(0.5f, add(v1, v2_));
        float s = dot(sub(cl, fc), nrm(m, fa, i1));
        if (s > radius) return;
        out->count = 1;
        out->ln = nrm(m, fa, i1);
        out->lp = fc;
    }
}

/* b2CollideCircles (collide.py:173-186) */
static void collide_circles(const GoiModelDesc* m, int fa, Xf xfa, int fb, Xf xfb, Manifold* out) {
    out->count = 0;
    V2 pa = xmul(xfa, vert(m, fa, 0));
    V2 pb = xmul(xfb, vert(m, fb, 0));
    V2 d = sub(pb, pa);
    float r = m->radius[fa] + m->radius[fb];
    if (dot(d, d) > r * r) return;
    out->mtype = CIRCLES;
    out->count = 1;
    out->ln = v2(0.0f, 0.0f);
    out->lp = vert(m, fa, 0);
    out->pl[0] = vert(m, fb, 0); out->pl[1] = out->pl[0];
    out->id[0] = 0; out->id[1] = 0;
}

/* ---- native edge shapes. The reference has no edge shape (shapes.py:13, __init__.py:53); these restate Box2D
 * 2.3.1's b2CollideEdge.cpp (b2CollideEdgeAndCircle, b2EPCollider) from the published source of that release. An
 * edge fixture holds m_vertex1, m_vertex2 in vertices 0-1 and the ghosts m_vertex0, m_vertex3 in vertices 2-3, with
 * GOI_EDGE_HAS_V0 / GOI_EDGE_HAS_V3 in edge_flags. The manifold's unused point slot follows the polygon
 * convention above: slot 1 holds the second clip point; the circle cases write the key into both slots. */

static inline int edge_flags_of(const GoiModelDesc* m, int f) { return m->edge_flags ? m->edge_flags[f] : 0; }
static inline V2 centroid_of(const GoiModelDesc* m, int f) {
    return m->centroid ? v2(m->centroid[2 * f], m->centroid[2 * f + 1]) : v2(0.0f, 0.0f);
}

/* b2CollideEdgeAndCircle: regions A, B (vertex contacts, suppressed where the neighbouring edge owns the circle)
 * and AB (face contact, two-sided normal). */
static void collide_edge_circle(const GoiModelDesc* m, int fa, Xf xfa, int fb, Xf xfb, Manifold* out) {
    out->count = 0;
    V2 q = xmulT(xfa, xmul(xfb, vert(m, fb, 0)));
    V2 a = vert(m, fa, 0), b = vert(m, fa, 1);
    V2 e = sub(b, a);
    float u = dot(e, sub(b, q)); /* barycentric coordinates */
    float v = dot(e, sub(q, a));
    float radius = m->radius[fa] + m->radius[fb];
    int flags = edge_flags_of(m, fa);
    V2 pl = vert(m, fb, 0);
    out->pl[0] = pl; out->pl[1] = pl;
    if (v <= 0.0f) { /* region A */
        V2 d = sub(q, a);
        if (dot(d, d) > radius * radius) return;
        if (flags & GOI_EDGE_HAS_V0) {
            V2 e1 = sub(a, vert(m, fa, 2));
            if (dot(e1, sub(a, q)) > 0.0f) return; /* in region AB of the previous edge */
        }
        out->mtype = CIRCLES; out->count = 1;
        out->ln = v2(0.0f, 0.0f); out->lp = a;
        out->id[0] = out->id[1] = feature_key(0, 0, E_VERTEX, E_VERTEX);
        return;
    }
    if (u <= 0.0f) { /* region B */
        V2 d = sub(q, b);
        if (dot(d, d) > radius * radius) return;
        if (flags & GOI_EDGE_HAS_V3) {
            V2 e2 = sub(vert(m, fa, 3), b);
            if (dot(e2, sub(q, b)) > 0.0f) return; /* in region AB of the next edge */
        }
        out->mtype = CIRCLES; out->count = 1;
        out->ln = v2(0.0f, 0.0f); out->lp = b;
        out->id[0] = out->id[1] = feature_key(1, 0, E_VERTEX, E_VERTEX);
        return;
    }
    float den = dot(e, e); /* region AB */
    V2 p = scl(1.0f / den, add(scl(u, a), scl(v, b)));
    V2 d = sub(q, p);
    if (dot(d, d) > radius * radius) return;
    V2 n = v2(-e.y, e.x);
    if (dot(n, sub(q, a)) < 0.0f) n = v2(-n.x, -n.y);
    normalize(&n);
    out->mtype = FACE_A; out->count = 1;
    out->ln = n; out->lp = a;
    out->id[0] = out->id[1] = feature_key(0, 0, E_FACE, E_VERTEX);
}

/* b2EPCollider::Collide: edge A against polygon B in A's frame. Classify the centroid of B as in front of or behind
 * the edge and bound the admissible normals by the neighbouring edges (ghost vertices), take the edge axis or the
 * best admissible polygon axis (hysteresis 0.98 / 0.001), then clip the incident edge against the reference face's
 * sides (no radius on the side planes). Skin radius 2 * b2_polygonRadius. */
static void collide_edge_polygon(const GoiModelDesc* m, int fa, Xf xfa, int fb, Xf xfb, const GoiSettings* st,
                                 Manifold* out) {
    out->count = 0;
    Xf xf = xmulT_xf(xfa, xfb);
    V2 cb = xmul(xf, centroid_of(m, fb));
    V2 v0 = vert(m, fa, 2), v1 = vert(m, fa, 0), v2_ = vert(m, fa, 1), v3 = vert(m, fa, 3);
    int flags = edge_flags_of(m, fa);
    int has0 = (flags & GOI_EDGE_HAS_V0) != 0, has3 = (flags & GOI_EDGE_HAS_V3) != 0;
    V2 edge1 = sub(v2_, v1);
    normalize(&edge1);
    V2 n1 = v2(edge1.y, -edge1.x);
    float offset1 = dot(n1, sub(cb, v1));
    float offset0 = 0.0f, offset2 = 0.0f;
    int convex1 = 0, convex2 = 0;
    V2 n0 = v2(0.0f, 0.0f), n2 = v2(0.0f, 0.0f);
    if (has0) {
        V2 edge0 = sub(v1, v0);
        normalize(&edge0);
        n0 = v2(edge0.y, -edge0.x);
        convex1 = crs(edge0, edge1) >= 0.0f;
        offset0 = dot(n0, sub(cb, v0));
    }
    if (has3) {
        V2 edge2 = sub(v3, v2_);
        normalize(&edge2);
        n2 = v2(edge2.y, -edge2.x);
        convex2 = crs(edge1, edge2) > 0.0f;
        offset2 = dot(n2, sub(cb, v2_));
    }
    int front;
    V2 normal, lower, upper;
    if (has0 && has3) {
        if (convex1 && convex2) {
            front = offset0 >= 0.0f || offset1 >= 0.0f || offset2 >= 0.0f;
            if (front) { normal = n1; lower = n0; upper = n2; }
            else { normal = neg(n1); lower = neg(n1); upper = neg(n1); }
        } else if (convex1) {
            front = offset0 >= 0.0f || (offset1 >= 0.0f && offset2 >= 0.0f);
            if (front) { normal = n1; lower = n0; upper = n1; }
            else { normal = neg(n1); lower = neg(n2); upper = neg(n1); }
        } else if (convex2) {
            front = offset2 >= 0.0f || (offset0 >= 0.0f && offset1 >= 0.0f);
            if (front) { normal = n1; lower = n1; upper = n2; }
            else { normal = neg(n1); lower = neg(n1); upper = neg(n0); }
        } else {
            front = offset0 >= 0.0f && offset1 >= 0.0f && offset2 >= 0.0f;
            if (front) { normal = n1; lower = n1; upper = n1; }
            else { normal = neg(n1); lower = neg(n2); upper = neg(n0); }
        }
    } else if (has0) {
        if (convex1) {
            front = offset0 >= 0.0f || offset1 >= 0.0f;
            if (front) { normal = n1; lower = n0; upper = neg(n1); }
            else { normal = neg(n1); lower = n1; upper = neg(n1); }
        } else {
            front = offset0 >= 0.0f && offset1 >= 0.0f;
            if (front) { normal = n1; lower = n1; upper = neg(n1); }
            else { normal = neg(n1); lower = n1; upper = neg(n0); }
        }
    } else if (has3) {
        if (convex2) {
            front = offset1 >= 0.0f || offset2 >= 0.0f;
            if (front) { normal = n1; lower = neg(n1); upper = n2; }
            else { normal = neg(n1); lower = neg(n1); upper = n1; }
        } else {
            front = offset1 >= 0.0f && offset2 >= 0.0f;
            if (front) { normal = n1; lower = neg(n1); upper = n1; }
            else { normal = neg(n1); lower = neg(n2); upper = n1; }
        }
    } else {
        front = offset1 >= 0.0f;
        if (front) { normal = n1; lower = neg(n1); upper = neg(n1); }
        else { normal = neg(n1); lower = n1; upper = n1; }
    }

    /* polygon B in frame A */
    int cnt = m->count[fb];
    V2 pv[NPOLY], pn[NPOLY];
    for (int i = 0; i < cnt; ++i) {
        pv[i] = xmul(xf, vert(m, fb, i));
        pn[i] = rmul(xf.q, nrm(m, fb, i));
    }
    float radius = 2.0f * st->polygon_radius;

    /* ComputeEdgeSeparation: the edge axis is always known */
    float edge_sep = MAXF;
    for (int i = 0; i < cnt; ++i) {
        float sv = dot(normal, sub(pv[i], v1));
        if (sv < edge_sep) edge_sep = sv;
    }
    if (edge_sep > radius) return;

    /* ComputePolygonSeparation: the first separating polygon axis, else the deepest admissible one */
    int poly_known = 0, poly_index = -1;
    float poly_sep = -MAXF;
    V2 perp = v2(-normal.y, normal.x);
    for (int i = 0; i < cnt; ++i) {
        V2 n = neg(pn[i]);
        float s1 = dot(n, sub(pv[i], v1));
        float s2 = dot(n, sub(pv[i], v2_));
        float sv = bmin(s1, s2);
        if (sv > radius) { poly_known = 1; poly_index = i; poly_sep = sv; break; }
        if (dot(n, perp) >= 0.0f) {
            if (dot(sub(n, upper), normal) < -st->angular_slop) continue;
        } else {
            if (dot(sub(n, lower), normal) < -st->angular_slop) continue;
        }
        if (sv > poly_sep) { poly_known = 1; poly_index = i; poly_sep = sv; }
    }
    if (poly_known && poly_sep > radius) return;

    int edge_primary = !poly_known || !(poly_sep > 0.98f * edge_sep + 0.001f);
    ClipV ie[2];
    int rf_i1, rf_i2;
    V2 rf_v1, rf_v2, rf_n;
    if (edge_primary) {
        out->mtype = FACE_A;
        int best = 0; /* the polygon normal most anti-parallel to the edge normal */
        float bestv = dot(normal, pn[0]);
        for (int i = 1; i < cnt; ++i) {
            float val = dot(normal, pn[i]);
            if (val < bestv) { bestv = val; best = i; }
        }
        int i1 = best, i2 = i1 + 1 < cnt ? i1 + 1 : 0;
        ie[0].v = pv[i1]; ie[0].ia = 0; ie[0].ib = i1; ie[0].ta = E_FACE; ie[0].tb = E_VERTEX;
        ie[1].v = pv[i2]; ie[1].ia = 0; ie[1].ib = i2; ie[1].ta = E_FACE; ie[1].tb = E_VERTEX;
        if (front) { rf_i1 = 0; rf_i2 = 1; rf_v1 = v1; rf_v2 = v2_; rf_n = n1; }
        else { rf_i1 = 1; rf_i2 = 0; rf_v1 = v2_; rf_v2 = v1; rf_n = neg(n1); }
    } else {
        out->mtype = FACE_B;
        ie[0].v = v1; ie[0].ia = 0; ie[0].ib = poly_index; ie[0].ta = E_VERTEX; ie[0].tb = E_FACE;
        ie[1].v = v2_; ie[1].ia = 0; ie[1].ib = poly_index; ie[1].ta = E_VERTEX; ie[1].tb = E_FACE;
        rf_i1 = poly_index;
        rf_i2 = rf_i1 + 1 < cnt ? rf_i1 + 1 : 0;
        rf_v1 = pv[rf_i1]; rf_v2 = pv[rf_i2]; rf_n = pn[rf_i1];
    }
    V2 side1 = v2(rf_n.y, -rf_n.x);
    V2 side2 = neg(side1);
    float side_off1 = dot(side1, rf_v1);
    float side_off2 = dot(side2, rf_v2);
    ClipV cp1[2], cp2[2];
    if (clip_segment(cp1, ie, side1, side_off1, rf_i1) < 2) return;
    if (clip_segment(cp2, cp1, side2, side_off2, rf_i2) < 2) return;
    if (edge_primary) { out->ln = rf_n; out->lp = rf_v1; }
    else { out->ln = nrm(m, fb, rf_i1); out->lp = vert(m, fb, rf_i1); }
    int keep[2];
    V2 pts[2];
    int32_t ids[2];
    for (int i = 0; i < 2; ++i) {
        float sep = dot(rf_n, sub(cp2[i].v, rf_v1));
        keep[i] = sep <= radius;
        if (edge_primary) {
            pts[i] = xmulT(xf, cp2[i].v);
            ids[i] = feature_key(cp2[i].ia, cp2[i].ib, cp2[i].ta, cp2[i].tb);
        } else {
            pts[i] = cp2[i].v;
            ids[i] = feature_key(cp2[i].ib, cp2[i].ia, cp2[i].tb, cp2[i].ta);
        }
    }
    out->count = keep[0] + keep[1];
    out->pl[0] = keep[0] ? pts[0] : pts[1];
    out->id[0] = keep[0] ? ids[0] : ids[1];
    out->pl[1] = pts[1];
    out->id[1] = ids[1];
}

/* b2Contact::Evaluate by shape types (collide.py:189-207); b2Contact::Create puts the polygon before a circle and
 * an edge before either */
static void evaluate(const GoiModelDesc* m, int fa, int fb, Xf xfa, Xf xfb, const GoiSettings* st, Manifold* out) {
    int ta = m->shape_type[fa], tb = m->shape_type[fb];
    if (ta == GOI_POLYGON && tb == GOI_POLYGON) collide_polygons(m, fa, xfa, fb, xfb, st->linear_slop, out);
    else if (ta == GOI_POLYGON && tb == GOI_CIRCLE) collide_polygon_circle(m, fa, xfa, fb, xfb, out);
    else if (ta == GOI_EDGE && tb == GOI_POLYGON) collide_edge_polygon(m, fa, xfa, fb, xfb, st, out);
    else if (ta == GOI_EDGE && tb == GOI_CIRCLE) collide_edge_circle(m, fa, xfa, fb, xfb, out);
    else collide_circles(m, fa, xfa, fb, xfb, out);
}

/* ------------------------------------------------------------------------------------------------ contacts (pairs.py) */

/* Live slots in Box2D's contact-list order: newest first = descending key (pairs.py:12-13). Returns the count. */
static int list_order(const W* w, int* order) {
    int n = 0;
    for (int k = 0; k < w->C; ++k) {
        if (w->c_pair[k] < 0) continue;
        int j = n++;
        while (j > 0 && w->c_key[order[j - 1]] < w->c_key[k]) { order[j] = order[j - 1]; --j; }
        order[j] = k;
    }
    return n;
}

/* b2Contact::Update's manifold part (pairs.py:56-83, toi.py:567-594): new manifold, impulses carried over from the
 * first old point with the same feature key, touching flag. Returns 1 if touching flipped. */
static int contact_update(W* w, int k, const Manifold* mf) {
    int oldn = w->c_count[k];
    int32_t old0 = w->c_pid[2 * k], old1 = w->c_pid[2 * k + 1];
    float oni0 = w->c_ni[2 * k], oni1 = w->c_ni[2 * k + 1];
    float oti0 = w->c_ti[2 * k], oti1 = w->c_ti[2 * k + 1];
    int n = mf->count;
    float ni[2], ti[2];
    for (int i = 0; i < 2; ++i) {
        ni[i] = 0.0f; ti[i] = 0.0f;
        if (i >= n) continue;
        if (oldn > 0 && old0 == mf->id[i]) { ni[i] = oni0; ti[i] = oti0; }
        else if (oldn > 1 && old1 == mf->id[i]) { ni[i] = oni1; ti[i] = oti1; }
    }
    int touching = n > 0;
    int flip = touching != (int)w->c_touching[k];
    w->c_touching[k] = (uint8_t)touching;
    w->c_count[k] = n;
    if (n > 0) {
        w->c_mtype[k] = mf->mtype;
        setv(w->c_ln, k, mf->ln);
        setv(w->c_lp, k, mf->lp);
        setv(w->c_pl, 2 * k, mf->pl[0]);
        setv(w->c_pl, 2 * k + 1, mf->pl[1]);
        w->c_pid[2 * k] = mf->id[0];
        w->c_pid[2 * k + 1] = mf->id[1];
    }
    w->c_ni[2 * k] = ni[0]; w->c_ni[2 * k + 1] = ni[1];
    w->c_ti[2 * k] = ti[0]; w->c_ti[2 * k + 1] = ti[1];
    return flip;
}

/* b2ContactManager::FindNewContacts over the candidate list (pairs.py:134-178): every candidate whose fat AABBs
 * overlap, whose bodies may collide and that has no contact gets a slot, in candidate order, lowest free slot
 * first; keys ascend in that order; a full table drops the rest and counts them. */
static void find_new_contacts(const Ctx* x, W* w) {
    const GoiModelDesc* m = x->m;
    int P = m->P, C = w->C;
    if (P == 0) return;
    int next = 0;                 /* next free slot to fill (scan pointer) */
    int32_t rank = 0;             /* creation rank among the new pairs */
    int32_t base_key = *w->next_key;
    /* exists: candidates that already have a live slot */
    for (int p = 0; p < P; ++p) {
        int a = m->pair_a[p], b = m->pair_b[p];
        int ba = m->fixture_body[a], bb = m->fixture_body[b];
        if (!overlap(fat_of(x, w, a), fat_of(x, w, b))) continue;
        if (!((w->b_type[ba] == GOI_DYNAMIC) || (w->b_type[bb] == GOI_DYNAMIC))) continue;
        if (!(w->b_active[ba] && w->b_active[bb])) continue;
        int exists = 0;
        for (int k = 0; k < C; ++k)
            if (w->c_pair[k] == p) { exists = 1; break; }
        if (exists) continue;
        /* find the next free slot at or after `next` */
        while (next < C && w->c_pair[next] >= 0) ++next;
        if (next < C) {
            int k = next++;
            w->c_pair[k] = p; w->c_fa[k] = a; w->c_fb[k] = b;
            w->c_key[k] = base_key + rank;
            w->c_touching[k] = 0; w->c_count[k] = 0;
            w->c_ni[2 * k] = 0.0f; w->c_ni[2 * k + 1] = 0.0f;
            w->c_ti[2 * k] = 0.0f; w->c_ti[2 * k + 1] = 0.0f;
            w->c_pid[2 * k] = 0; w->c_pid[2 * k + 1] = 0;
            w->c_friction[k] = sqrtf(friction_of(x, w, a) * friction_of(x, w, b)); /* b2MixFriction */
            float ra = restitution_of(x, w, a), rb = restitution_of(x, w, b);
            w->c_restitution[k] = ra > rb ? ra : rb;                             /* b2MixRestitution */
            w->c_tangent_speed[k] = 0.0f;
            wake(w, ba); wake(w, bb); /* AddPair wakes both bodies */
        } else {
            *w->overflow += 1;
        }
        ++rank;
    }
    *w->next_key = base_key + rank;
}

/* b2ContactManager::Collide (pairs.py:38-87): the contact list newest first; a contact whose bodies are both
 * inactive (asleep or static) is skipped; fat AABBs no longer overlapping destroy it (waking both bodies if it
 * still had points, b2Contact::Destroy); the rest are updated (waking both bodies when touching flips). */
static void collide(const Ctx* x, W* w, int* order) {
    const GoiModelDesc* m = x->m;
    int n = list_order(w, order);
    for (int i = 0; i < n; ++i) {
        int k = order[i];
        int fa = w->c_fa[k], fb = w->c_fb[k];
        int ba = m->fixture_body[fa], bb = m->fixture_body[fb];
        int act_a = w->b_awake[ba] && w->b_type[ba] != GOI_STATIC;
        int act_b = w->b_awake[bb] && w->b_type[bb] != GOI_STATIC;
        if (!act_a && !act_b) continue;
        if (!overlap(fat_of(x, w, fa), fat_of(x, w, fb))) {
            if (w->c_count[k] > 0) { wake(w, ba); wake(w, bb); }
            w->c_pair[k] = -1; w->c_touching[k] = 0; w->c_count[k] = 0;
            continue;
        }
        Manifold mf;
        evaluate(m, fa, fb, body_xf(w, ba), body_xf(w, bb), x->s, &mf);
        if (contact_update(w, k, &mf)) { wake(w, ba); wake(w, bb); }
    }
}

/* b2Body::SynchronizeFixtures for the bodies in `moved` (pairs.py:181-207): swept AABB over the sweep start
 * (c0, a0) and the current transform; b2DynamicTree::MoveProxy re-fattens only if the fat box no longer holds it. */
static void synchronize_fixtures(const Ctx* x, W* w, const uint8_t* moved) {
    const GoiModelDesc* m = x->m;
    for (int f = 0; f < m->F; ++f) {
        int b = m->fixture_body[f];
        if (!moved[b]) continue;
        int row = x->compact ? m->fixture_slot[f] : f;
        if (row < 0) continue;
        Xf x1;
        x1.q = rot_of(w->b_a0[b]);
        x1.p = sub(getv(w->b_c0, b), rmul(x1.q, getv(w->b_lc, b)));
        Xf x2 = body_xf(w, b);
        AABB a1 = shape_aabb(m, f, x1), a2 = shape_aabb(m, f, x2);
        float lx = bmin(a1.lx, a2.lx), ly = bmin(a1.ly, a2.ly);
        float ux = bmax(a1.ux, a2.ux), uy = bmax(a1.uy, a2.uy);
        float* fat = w->f_fat + 4 * row;
        if (fat[0] <= lx && fat[1] <= ly && ux <= fat[2] && uy <= fat[3]) continue;
        V2 d = sub(x2.p, x1.p);
        float e = 0.1f; /* b2_aabbExtension */
        lx = lx - e; ly = ly - e; ux = ux + e; uy = uy + e;
        float ddx = 2.0f * d.x, ddy = 2.0f * d.y; /* b2_aabbMultiplier */
        if (ddx < 0.0f) lx = lx + ddx; else ux = ux + ddx;
        if (ddy < 0.0f) ly = ly + ddy; else uy = uy + ddy;
        fat[0] = lx; fat[1] = ly; fat[2] = ux; fat[3] = uy;
    }
}

/* ------------------------------------------------------------------------------------------------ per-world scratch */

typedef struct {
    int slot, ia, ib;
    float mA, mB, iA, iB;
    V2 n;
    float friction, tangent_speed;
    int count, pc_count, mtype;
    V2 rA[2], rB[2];
    float nmass[2], tmass[2], bias[2], ni[2], ti[2];
    float K[4], NM[4];            /* ex.x, ex.y, ey.x, ey.y */
    V2 ln, lp, pl[2], lcA, lcB;
    float radA, radB;
} CC;

typedef struct {
    int jid, type, ia, ib;
    float mA, mB, iA, iB;
    V2 rA, rB;
    V3 ex, ey, ez;
    float motor_mass;
    int limit_state, enable_motor, enable_limit, soft;
    float motor_speed, max_impulse;
    V2 axis, perp;
    float a1, a2, s1, s2, gamma, bias, angle, inv_dt;
    V2 la, lb, lx, ly;
    float ref, lower, upper;
    float imp[5], mimp;
} JR;

typedef struct {
    int cap_b, cap_c, cap_j;
    int *order, *stack, *corder, *jorder, *body_island, *contact_island, *joint_island;
    uint8_t *bflag, *cflag, *jflag, *moved, *done, *isl_sleep;
    float *vx, *vy, *w, *cx, *cy, *a, *min_sep, *min_st;
    int *jok, *last;
    CC* cc;
    JR* jr;
    /* TOI */
    float *bk;         /* body sweep backups: c0x c0y cx cy a0 a alpha0 per body */
    int *isl_bodies;
    int n_islands;
} Work;

static void work_init(Work* k, int B, int C, int J) {
    int nb = B > 0 ? B : 1, nc = C > 0 ? C : 1, nj = J > 0 ? J : 1;
    k->cap_b = nb; k->cap_c = nc; k->cap_j = nj;
    k->order = calloc(nc, sizeof(int)); k->corder = calloc(nc, sizeof(int));
    k->stack = calloc(2 * nb + 2 * nc + 4, sizeof(int));
    k->jorder = calloc(nj, sizeof(int)); k->body_island = calloc(nb, sizeof(int));
    k->contact_island = calloc(nc, sizeof(int)); k->joint_island = calloc(nj, sizeof(int));
    k->bflag = calloc(nb, 1); k->cflag = calloc(nc, 1); k->jflag = calloc(nj, 1); k->moved = calloc(nb, 1);
    k->done = calloc(nb, 1); k->isl_sleep = calloc(nb, 1);
    k->vx = calloc(nb, 4); k->vy = calloc(nb, 4); k->w = calloc(nb, 4);
    k->cx = calloc(nb, 4); k->cy = calloc(nb, 4); k->a = calloc(nb, 4);
    k->min_sep = calloc(nb, 4); k->min_st = calloc(nb, 4);
    k->jok = calloc(nb, sizeof(int)); k->last = calloc(nb, sizeof(int));
    k->cc = calloc(nc, sizeof(CC)); k->jr = calloc(nj, sizeof(JR));
    k->bk = calloc(7 * nb, 4); k->isl_bodies = calloc(nb, sizeof(int));
}

static void work_free(Work* k) {
    free(k->order); free(k->corder); free(k->stack); free(k->jorder); free(k->body_island);
    free(k->contact_island); free(k->joint_island); free(k->bflag); free(k->cflag); free(k->jflag);
    free(k->moved); free(k->done); free(k->isl_sleep); free(k->vx); free(k->vy); free(k->w); free(k->cx);
    free(k->cy); free(k->a); free(k->min_sep); free(k->min_st); free(k->jok); free(k->last); free(k->cc);
    free(k->jr); free(k->bk); free(k->isl_bodies);
}

/* ------------------------------------------------------------------------------------------------ islands (island.py) */

/* b2World::Solve's depth-first search (island.py:1-19, 41-140): seeds newest body first (descending index); a seed
 * is unvisited, awake, active and not static. Popping b wakes it, then walks b's contact edges newest first
 * (touching contacts not yet in an island join in that order and push their other body if it is unvisited and not
 * static), then b's joint edges newest first (descending joint index; joints to inactive bodies skipped). Island
 * ids count up in seed order; contacts/joints are appended to one solve order across islands. */
static int find_islands(const Ctx* x, W* w, Work* k, int* nc_out, int* nj_out) {
    const GoiModelDesc* m = x->m;
    int B = w->B, C = w->C, J = m->J;
    int n = list_order(w, k->order);
    for (int b = 0; b < B; ++b) { k->bflag[b] = 0; k->body_island[b] = -1; }
    for (int c = 0; c < C; ++c) { k->cflag[c] = 0; k->contact_island[c] = -1; }
    for (int j = 0; j < J; ++j) { k->jflag[j] = 0; k->joint_island[j] = -1; }
    int nisl = 0, nc = 0, nj = 0;
    for (int seed = B - 1; seed >= 0; --seed) {
        if (k->bflag[seed] || !w->b_awake[seed] || !w->b_active[seed] || w->b_type[seed] == GOI_STATIC) continue;
        int isl = nisl++;
        int sp = 0;
        k->stack[sp++] = seed;
        k->bflag[seed] = 1;
        while (sp > 0) {
            int b = k->stack[--sp];
            k->body_island[b] = isl;
            wake(w, b);
            for (int i = 0; i < n; ++i) {
                int c = k->order[i];
                int ba = m->fixture_body[w->c_fa[c]], bb = m->fixture_body[w->c_fb[c]];
                if (ba != b && bb != b) continue;
                if (k->cflag[c] || !w->c_touching[c]) continue;
                k->corder[nc++] = c;
                k->cflag[c] = 1;
                k->contact_island[c] = isl;
                int other = ba == b ? bb : ba;
                if (k->bflag[other] || w->b_type[other] == GOI_STATIC) continue;
                k->stack[sp++] = other;
                k->bflag[other] = 1;
            }
            for (int j = J - 1; j >= 0; --j) {
                int ja = m->joint_a[j], jb = m->joint_b[j];
                if (ja != b && jb != b) continue;
                if (k->jflag[j]) continue;
                int other = ja == b ? jb : ja;
                if (!w->b_active[other]) continue;
                k->jorder[nj++] = j;
                k->jflag[j] = 1;
                k->joint_island[j] = isl;
                if (k->bflag[other] || w->b_type[other] == GOI_STATIC) continue;
                k->stack[sp++] = other;
                k->bflag[other] = 1;
            }
        }
    }
    *nc_out = nc; *nj_out = nj;
    k->n_islands = nisl;
    return nisl;
}

/* ------------------------------------------------------------------------------------------------ contact solver */

/* b2ContactSolver constructor + InitializeVelocityConstraints for one ordered contact (contact_solver.py:32-147).
 * pos/vel are the island arrays after velocity integration; q the per-body rotations of the step-start angles. */
static void cs_prepare(const Ctx* x, const W* w, Work* k, CC* c, int slot, int warm, float dt_ratio,
                       const Rot* q) {
    const GoiModelDesc* m = x->m;
    int fa = w->c_fa[slot], fb = w->c_fb[slot];
    int ia = m->fixture_body[fa], ib = m->fixture_body[fb];
    c->slot = slot; c->ia = ia; c->ib = ib;
    c->mA = w->b_inv_mass[ia]; c->mB = w->b_inv_mass[ib];
    c->iA = w->b_inv_inertia[ia]; c->iB = w->b_inv_inertia[ib];
    c->lcA = getv(w->b_lc, ia); c->lcB = getv(w->b_lc, ib);
    c->radA = m->radius[fa]; c->radB = m->radius[fb];
    c->mtype = w->c_mtype[slot];
    c->pc_count = w->c_count[slot];
    c->ln = getv(w->c_ln, slot); c->lp = getv(w->c_lp, slot);
    c->pl[0] = getv(w->c_pl, 2 * slot); c->pl[1] = getv(w->c_pl, 2 * slot + 1);
    for (int j = 0; j < 2; ++j) {
        c->ni[j] = warm ? dt_ratio * w->c_ni[2 * slot + j] : 0.0f;
        c->ti[j] = warm ? dt_ratio * w->c_ti[2 * slot + j] : 0.0f;
    }
    c->friction = w->c_friction[slot];
    c->tangent_speed = w->c_tangent_speed[slot];
    float restitution = w->c_restitution[slot];
    V2 cA = v2(k->cx[ia], k->cy[ia]), cB = v2(k->cx[ib], k->cy[ib]);
    V2 vA = v2(k->vx[ia], k->vy[ia]), vB = v2(k->vx[ib], k->vy[ib]);
    float wA = k->w[ia], wB = k->w[ib];
    Xf xfA, xfB;
    xfA.q = q[ia]; xfB.q = q[ib];
    xfA.p = sub(cA, rmul(xfA.q, c->lcA));
    xfB.p = sub(cB, rmul(xfB.q, c->lcB));
    /* b2WorldManifold::Initialize */
    V2 n = v2(1.0f, 0.0f), pts[2];
    pts[0] = v2(0.0f, 0.0f); pts[1] = pts[0];
    int cnt = c->pc_count;
    if (c->mtype == CIRCLES) {
        V2 pA = xmul(xfA, c->lp), pB = xmul(xfB, c->pl[0]);
        V2 d = sub(pB, pA);
        if (dot(d, d) > EPS * EPS) { n = d; normalize(&n); }
        V2 ccA = add(pA, scl(c->radA, n)), ccB = sub(pB, scl(c->radB, n));
        pts[0] = scl(0.5f, add(ccA, ccB));
        pts[1] = pts[0];
    } else if (c->mtype == FACE_A) {
        n = rmul(xfA.q, c->ln);
        V2 pp = xmul(xfA, c->lp);
        for (int j = 0; j < 2; ++j) {
            V2 cp = xmul(xfB, c->pl[j]);
            V2 aA = add(cp, scl(c->radA - dot(sub(cp, pp), n), n));
            V2 aB = sub(cp, scl(c->radB, n));
            pts[j] = scl(0.5f, add(aA, aB));
        }
    } else {
        n = rmul(xfB.q, c->ln);
        V2 pp = xmul(xfB, c->lp);
        for (int j = 0; j < 2; ++j) {
            V2 cp = xmul(xfA, c->pl[j]);
            V2 bB = add(cp, scl(c->radB - dot(sub(cp, pp), n), n));
            V2 bA = sub(cp, scl(c->radA, n));
            pts[j] = scl(0.5f, add(bA, bB));
        }
        n = neg(n);
    }
    c->n = n;
    V2 t = crs_vs(n, 1.0f);
    float mA = c->mA, mB = c->mB, iA = c->iA, iB = c->iB;
    for (int j = 0; j < 2; ++j) {
        c->rA[j] = sub(pts[j], cA);
        c->rB[j] = sub(pts[j], cB);
        float rnA = crs(c->rA[j], n), rnB = crs(c->rB[j], n);
        float kn = ((mA + mB) + iA * rnA * rnA) + iB * rnB * rnB;
        float rtA = crs(c->rA[j], t), rtB = crs(c->rB[j], t);
        float kt = ((mA + mB) + iA * rtA * rtA) + iB * rtB * rtB;
        c->nmass[j] = kn > 0.0f ? 1.0f / kn : 0.0f;
        c->tmass[j] = kt > 0.0f ? 1.0f / kt : 0.0f;
        V2 dv = sub(sub(add(vB, crs_sv(wB, c->rB[j])), vA), crs_sv(wA, c->rA[j]));
        float vrel = dot(n, dv);
        c->bias[j] = vrel < -x->s->velocity_threshold ? -restitution * vrel : 0.0f;
    }
    c->count = cnt;
    for (int i = 0; i < 4; ++i) { c->K[i] = 0.0f; c->NM[i] = 0.0f; }
    if (cnt == 2) {
        float rn1A = crs(c->rA[0], n), rn1B = crs(c->rB[0], n);
        float rn2A = crs(c->rA[1], n), rn2B = crs(c->rB[1], n);
        float k11 = ((mA + mB) + iA * rn1A * rn1A) + iB * rn1B * rn1B;
        float k22 = ((mA + mB) + iA * rn2A * rn2A) + iB * rn2B * rn2B;
        float k12 = ((mA + mB) + iA * rn1A * rn2A) + iB * rn1B * rn2B;
        if (k11 * k11 < 1000.0f * (k11 * k22 - k12 * k12)) {
            float det = k11 * k22 - k12 * k12;
            if (det != 0.0f) det = 1.0f / det;
            c->K[0] = k11; c->K[1] = k12; c->K[2] = k12; c->K[3] = k22;
            c->NM[0] = det * k22; c->NM[1] = -det * k12; c->NM[2] = -det * k12; c->NM[3] = det * k11;
        } else {
            c->count = 1;
        }
    }
}

static void cs_warm_start(const CC* c, Work* k) {
    int ia = c->ia, ib = c->ib;
    V2 vA = v2(k->vx[ia], k->vy[ia]), vB = v2(k->vx[ib], k->vy[ib]);
    float wA = k->w[ia], wB = k->w[ib];
    V2 t = crs_vs(c->n, 1.0f);
    for (int j = 0; j < c->count; ++j) {
        V2 P = add(scl(c->ni[j], c->n), scl(c->ti[j], t));
        wA = wA - c->iA * crs(c->rA[j], P);
        vA = sub(vA, scl(c->mA, P));
        wB = wB + c->iB * crs(c->rB[j], P);
        vB = add(vB, scl(c->mB, P));
    }
    k->vx[ia] = vA.x; k->vy[ia] = vA.y; k->w[ia] = wA;
    k->vx[ib] = vB.x; k->vy[ib] = vB.y; k->w[ib] = wB;
}

static inline V2 rel_vel(V2 vB, float wB, V2 rB, V2 vA, float wA, V2 rA) {
    return sub(sub(add(vB, crs_sv(wB, rB)), vA), crs_sv(wA, rA));
}

/* b2ContactSolver::SolveVelocityConstraints for one contact (contact_solver.py:194-279) */
static void cs_solve_velocity(CC* c, Work* k) {
    int ia = c->ia, ib = c->ib;
    V2 vA = v2(k->vx[ia], k->vy[ia]), vB = v2(k->vx[ib], k->vy[ib]);
    float wA = k->w[ia], wB = k->w[ib];
    float mA = c->mA, mB = c->mB, iA = c->iA, iB = c->iB;
    V2 n = c->n, t = crs_vs(n, 1.0f);
    for (int j = 0; j < c->count; ++j) {
        V2 dv = rel_vel(vB, wB, c->rB[j], vA, wA, c->rA[j]);
        float vt = dot(dv, t) - c->tangent_speed;
        float lam = c->tmass[j] * (-vt);
        float maxf = c->friction * c->ni[j];
        float nw = bclamp(c->ti[j] + lam, -maxf, maxf);
        lam = nw - c->ti[j];
        c->ti[j] = nw;
        V2 P = scl(lam, t);
        vA = sub(vA, scl(mA, P)); wA = wA - iA * crs(c->rA[j], P);
        vB = add(vB, scl(mB, P)); wB = wB + iB * crs(c->rB[j], P);
    }
    if (c->count == 1) {
        V2 dv = rel_vel(vB, wB, c->rB[0], vA, wA, c->rA[0]);
        float vn = dot(dv, n);
        float lam = -c->nmass[0] * (vn - c->bias[0]);
        float nw = bmax(c->ni[0] + lam, 0.0f);
        lam = nw - c->ni[0];
        c->ni[0] = nw;
        V2 P = scl(lam, n);
        vA = sub(vA, scl(mA, P)); wA = wA - iA * crs(c->rA[0], P);
        vB = add(vB, scl(mB, P)); wB = wB + iB * crs(c->rB[0], P);
    } else if (c->count == 2) {
        float ax = c->ni[0], ay = c->ni[1];
        V2 dv1 = rel_vel(vB, wB, c->rB[0], vA, wA, c->rA[0]);
        V2 dv2 = rel_vel(vB, wB, c->rB[1], vA, wA, c->rA[1]);
        float vn1 = dot(dv1, n), vn2 = dot(dv2, n);
        float bx = vn1 - c->bias[0], by = vn2 - c->bias[1];
        bx = bx - (c->K[0] * ax + c->K[2] * ay);
        by = by - (c->K[1] * ax + c->K[3] * ay);
        float xx, xy;
        int ok = 0;
        /* case 1: both points */
        xx = -(c->NM[0] * bx + c->NM[2] * by);
        xy = -(c->NM[1] * bx + c->NM[3] * by);
        if (xx >= 0.0f && xy >= 0.0f) ok = 1;
        if (!ok) { /* case 2: point 1 only */
            xx = -c->nmass[0] * bx; xy = 0.0f;
            float v2n = c->K[1] * xx + by;
            if (xx >= 0.0f && v2n >= 0.0f) ok = 1;
        }
        if (!ok) { /* case 3: point 2 only */
            xx = 0.0f; xy = -c->nmass[1] * by;
            float v1n = c->K[2] * xy + bx;
            if (xy >= 0.0f && v1n >= 0.0f) ok = 1;
        }
        if (!ok) { /* case 4: neither */
            xx = 0.0f; xy = 0.0f;
            if (bx >= 0.0f && by >= 0.0f) ok = 1;
        }
        if (ok) {
            float dx = xx - ax, dy = xy - ay;
            V2 P1 = scl(dx, n), P2 = scl(dy, n);
            V2 P12 = add(P1, P2);
            vA = sub(vA, scl(mA, P12));
            wA = wA - iA * (crs(c->rA[0], P1) + crs(c->rA[1], P2));
            vB = add(vB, scl(mB, P12));
            wB = wB + iB * (crs(c->rB[0], P1) + crs(c->rB[1], P2));
            c->ni[0] = xx; c->ni[1] = xy;
        }
    }
    k->vx[ia] = vA.x; k->vy[ia] = vA.y; k->w[ia] = wA;
    k->vx[ib] = vB.x; k->vy[ib] = vB.y; k->w[ib] = wB;
}

/* b2ContactSolver::SolvePositionConstraints for one contact (contact_solver.py:307-354); returns its min separation
 * starting from 0. baumgarte is b2_baumgarte or b2_toiBaugarte; masses as given in c. */
static float cs_solve_position(const Ctx* x, const CC* c, Work* k, float baumgarte, float mA, float mB, float iA,
                               float iB) {
    const GoiSettings* s = x->s;
    int ia = c->ia, ib = c->ib;
    V2 cA = v2(k->cx[ia], k->cy[ia]), cB = v2(k->cx[ib], k->cy[ib]);
    float aA = k->a[ia], aB = k->a[ib];
    float min_sep = 0.0f;
    for (int j = 0; j < c->pc_count; ++j) {
        Xf xfA, xfB;
        xfA.q = rot_of(aA); xfB.q = rot_of(aB);
        xfA.p = sub(cA, rmul(xfA.q, c->lcA));
        xfB.p = sub(cB, rmul(xfB.q, c->lcB));
        V2 n, p;
        float sep;
        if (c->mtype == CIRCLES) {
            V2 pA = xmul(xfA, c->lp), pB = xmul(xfB, c->pl[0]);
            n = sub(pB, pA);
            normalize(&n);
            p = scl(0.5f, add(pA, pB));
            sep = (dot(sub(pB, pA), n) - c->radA) - c->radB;
        } else if (c->mtype == FACE_A) {
            n = rmul(xfA.q, c->ln);
            V2 pp = xmul(xfA, c->lp);
            V2 cp = xmul(xfB, c->pl[j]);
            sep = (dot(sub(cp, pp), n) - c->radA) - c->radB;
            p = cp;
        } else {
            n = rmul(xfB.q, c->ln);
            V2 pp = xmul(xfB, c->lp);
            V2 cp = xmul(xfA, c->pl[j]);
            sep = (dot(sub(cp, pp), n) - c->radA) - c->radB;
            p = cp;
            n = neg(n);
        }
        V2 rA = sub(p, cA), rB = sub(p, cB);
        min_sep = bmin(min_sep, sep);
        float C = bclamp(baumgarte * (sep + s->linear_slop), -s->max_linear_correction, 0.0f);
        float rnA = crs(rA, n), rnB = crs(rB, n);
        float K = ((mA + mB) + iA * rnA * rnA) + iB * rnB * rnB;
        float imp = K > 0.0f ? -C / K : 0.0f;
        V2 P = scl(imp, n);
        cA = sub(cA, scl(mA, P)); aA = aA - iA * crs(rA, P);
        cB = add(cB, scl(mB, P)); aB = aB + iB * crs(rB, P);
    }
    k->cx[ia] = cA.x; k->cy[ia] = cA.y; k->a[ia] = aA;
    k->cx[ib] = cB.x; k->cy[ib] = cB.y; k->a[ib] = aB;
    return min_sep;
}

/* ------------------------------------------------------------------------------------------------ joints (joints.py) */

/* InitVelocityConstraints minus the velocity writes (joints.py:61-174); impulses scaled by dtRatio or reset. */
static void jn_prepare(const Ctx* x, const W* w, Work* k, JR* r, int jid, float dt, float dt_ratio, int warm,
                       const Rot* q) {
    const GoiModelDesc* m = x->m;
    const GoiSettings* s = x->s;
    int v24 = s->revolute_v24;
    int type = m->joint_type[jid];
    int ia = m->joint_a[jid], ib = m->joint_b[jid];
    r->jid = jid; r->type = type; r->ia = ia; r->ib = ib;
    float mA = w->b_inv_mass[ia], mB = w->b_inv_mass[ib], iA = w->b_inv_inertia[ia], iB = w->b_inv_inertia[ib];
    r->mA = mA; r->mB = mB; r->iA = iA; r->iB = iB;
    V2 lcA = getv(w->b_lc, ia), lcB = getv(w->b_lc, ib);
    V2 cA = v2(k->cx[ia], k->cy[ia]), cB = v2(k->cx[ib], k->cy[ib]);
    float aA = k->a[ia], aB = k->a[ib];
    Rot qA = q[ia], qB = q[ib];
    r->la = sub(getv(m->local_anchor_a, jid), lcA);
    r->lb = sub(getv(m->local_anchor_b, jid), lcB);
    r->rA = rmul(qA, r->la);
    r->rB = rmul(qB, r->lb);
    r->ref = m->reference_angle[jid];
    r->lx = getv(m->local_axis_a, jid); r->ly = getv(m->local_yaxis_a, jid);
    r->enable_motor = w->j_enable_motor[jid]; r->enable_limit = w->j_enable_limit[jid];
    r->lower = w->j_lower[jid]; r->upper = w->j_upper[jid];
    r->motor_speed = w->j_motor_speed[jid];
    r->max_impulse = dt * w->j_max_motor[jid];
    r->inv_dt = dt > 0.0f ? 1.0f / dt : 0.0f;
    int state_in = w->j_limit_state[jid];
    float ix = w->j_impulse[3 * jid], iy = w->j_impulse[3 * jid + 1], iz = w->j_impulse[3 * jid + 2];
    float mimp = w->j_motor_impulse[jid];
    float lo = 0.0f, up = 0.0f;
    V2 rA = r->rA, rB = r->rB;
    r->soft = 0; r->gamma = 0.0f; r->bias = 0.0f; r->angle = 0.0f;
    r->a1 = r->a2 = r->s1 = r->s2 = 0.0f;
    r->axis = v2(0.0f, 0.0f); r->perp = v2(0.0f, 0.0f);
    if (type == GOI_REVOLUTE || type == GOI_WELD) {
        /* revolute / weld 3x3 effective mass, iA last in each product (joints.py:39-47) */
        float exx = ((mA + mB) + rA.y * rA.y * iA) + rB.y * rB.y * iB;
        float eyx = -rA.y * rA.x * iA - rB.y * rB.x * iB;
        float ezx = -rA.y * iA - rB.y * iB;
        float eyy = ((mA + mB) + rA.x * rA.x * iA) + rB.x * rB.x * iB;
        float ezy = rA.x * iA + rB.x * iB;
        float ezz = iA + iB;
        r->ex = v3(exx, eyx, ezx); r->ey = v3(eyx, eyy, ezy); r->ez = v3(ezx, ezy, ezz);
    }
    if (type == GOI_REVOLUTE) {
        int fixed = (iA + iB) == 0.0f;
        r->motor_mass = (iA + iB) > 0.0f ? 1.0f / (iA + iB) : 0.0f;
        if (!r->enable_motor || fixed) mimp = 0.0f;
        float angle = (aB - aA) - r->ref;
        r->angle = angle;
        int equal = babs(r->upper - r->lower) < 2.0f * s->angular_slop;
        int lim_on = r->enable_limit && !fixed;
        int st = !lim_on ? INACTIVE_LIMIT : equal ? EQUAL_LIMITS : angle <= r->lower ? AT_LOWER
                 : angle >= r->upper ? AT_UPPER : INACTIVE_LIMIT;
        r->limit_state = st;
        if (v24) {
            lo = lim_on ? w->j_lower_impulse[jid] : 0.0f;
            up = lim_on ? w->j_upper_impulse[jid] : 0.0f;
        } else if (lim_on && !equal && (st == INACTIVE_LIMIT || st != state_in)) {
            iz = 0.0f;
        }
    } else if (type == GOI_PRISMATIC) {
        V2 d = sub(add(sub(cB, cA), rB), rA);
        r->axis = rmul(qA, r->lx);
        r->a1 = crs(add(d, rA), r->axis);
        r->a2 = crs(rB, r->axis);
        float mm = ((mA + mB) + iA * r->a1 * r->a1) + iB * r->a2 * r->a2;
        r->motor_mass = mm > 0.0f ? 1.0f / mm : mm;
        r->perp = rmul(qA, r->ly);
        r->s1 = crs(add(d, rA), r->perp);
        r->s2 = crs(rB, r->perp);
        float s1 = r->s1, s2 = r->s2, a1 = r->a1, a2 = r->a2;
        float k11 = ((mA + mB) + iA * s1 * s1) + iB * s2 * s2;
        float k12 = iA * s1 + iB * s2;
        float k13 = iA * s1 * a1 + iB * s2 * a2;
        float k22 = iA + iB;
        if (k22 == 0.0f) k22 = 1.0f;
        float k23 = iA * a1 + iB * a2;
        float k33 = ((mA + mB) + iA * a1 * a1) + iB * a2 * a2;
        r->ex = v3(k11, k12, k13); r->ey = v3(k12, k22, k23); r->ez = v3(k13, k23, k33);
        float trans = dot(r->axis, d);
        int pequal = babs(r->upper - r->lower) < 2.0f * s->linear_slop;
        int st = !r->enable_limit ? INACTIVE_LIMIT : pequal ? EQUAL_LIMITS : trans <= r->lower ? AT_LOWER
                 : trans >= r->upper ? AT_UPPER : INACTIVE_LIMIT;
        r->limit_state = st;
        if (!r->enable_limit || (!pequal && (st == INACTIVE_LIMIT || st != state_in))) iz = 0.0f;
        if (!r->enable_motor) mimp = 0.0f;
    } else { /* weld (joints.py:125-144) */
        V3 ex = r->ex, ey = r->ey, ez = r->ez;
        r->soft = w->j_frequency[jid] > 0.0f;
        float invM = iA + iB;
        float wm = invM > 0.0f ? 1.0f / invM : 0.0f;
        float C = (aB - aA) - r->ref;
        float omega = (2.0f * 3.14159265359f) * w->j_frequency[jid];
        float dd = 2.0f * wm * w->j_damping[jid] * omega;
        float kk = wm * omega * omega;
        float h = dt;
        float gamma = h * (dd + h * kk);
        gamma = gamma != 0.0f ? 1.0f / gamma : 0.0f;
        float bias = C * h * kk * gamma;
        if (r->soft || ez.z == 0.0f) {
            float a = ex.x, b = ey.x, c = ex.y, d = ey.y;
            float det = a * d - b * c;
            if (det != 0.0f) det = 1.0f / det;
            r->ex = v3(det * d, -det * c, 0.0f);
            r->ey = v3(-det * b, det * a, 0.0f);
            r->ez = v3(0.0f, 0.0f, 0.0f);
        } else {
            float det = dot3(ex, cross3(ey, ez));
            if (det != 0.0f) det = 1.0f / det;
            float a11 = ex.x, a12 = ey.x, a13 = ez.x, a22 = ey.y, a23 = ez.y, a33 = ez.z;
            float exx = det * (a22 * a33 - a23 * a23);
            float exy = det * (a13 * a23 - a12 * a33);
            float exz = det * (a12 * a23 - a13 * a22);
            float eyy = det * (a11 * a33 - a13 * a13);
            float eyz = det * (a13 * a12 - a11 * a23);
            float ezz = det * (a11 * a22 - a12 * a12);
            r->ex = v3(exx, exy, exz); r->ey = v3(exy, eyy, eyz); r->ez = v3(exz, eyz, ezz);
        }
        if (r->soft) {
            float inv = invM + gamma;
            r->ez.z = inv != 0.0f ? 1.0f / inv : 0.0f;
        }
        r->gamma = r->soft ? gamma : 0.0f;
        r->bias = r->soft ? bias : 0.0f;
        r->limit_state = INACTIVE_LIMIT;
        r->motor_mass = 0.0f;
        mimp = 0.0f;
    }
    /* warm-start scaling or reset (joints.py:151-160) */
    r->imp[0] = warm ? ix * dt_ratio : 0.0f;
    r->imp[1] = warm ? iy * dt_ratio : 0.0f;
    r->imp[2] = (v24 && type == GOI_REVOLUTE) ? iz : (warm ? iz * dt_ratio : 0.0f);
    r->imp[3] = warm ? lo * dt_ratio : 0.0f;
    r->imp[4] = warm ? up * dt_ratio : 0.0f;
    r->mimp = warm ? mimp * dt_ratio : 0.0f;
}

/* the velocity part of InitVelocityConstraints (joints.py:202-248) */
static void jn_warm_start(const Ctx* x, const JR* r, Work* k) {
    int ia = r->ia, ib = r->ib;
    V2 vA = v2(k->vx[ia], k->vy[ia]), vB = v2(k->vx[ib], k->vy[ib]);
    float wA = k->w[ia], wB = k->w[ib];
    float ix = r->imp[0], iy = r->imp[1], iz = r->imp[2], mi = r->mimp;
    if (r->type == GOI_REVOLUTE) {
        V2 P = v2(ix, iy);
        float ax = x->s->revolute_v24 ? (mi + r->imp[3]) - r->imp[4] : 0.0f;
        vA = sub(vA, scl(r->mA, P));
        vB = add(vB, scl(r->mB, P));
        if (x->s->revolute_v24) {
            wA = wA - r->iA * (crs(r->rA, P) + ax);
            wB = wB + r->iB * (crs(r->rB, P) + ax);
        } else {
            wA = wA - r->iA * ((crs(r->rA, P) + mi) + iz);
            wB = wB + r->iB * ((crs(r->rB, P) + mi) + iz);
        }
    } else if (r->type == GOI_PRISMATIC) {
        float mz = mi + iz;
        V2 P = add(scl(ix, r->perp), scl(mz, r->axis));
        float LA = (ix * r->s1 + iy) + mz * r->a1;
        float LB = (ix * r->s2 + iy) + mz * r->a2;
        vA = sub(vA, scl(r->mA, P)); wA = wA - r->iA * LA;
        vB = add(vB, scl(r->mB, P)); wB = wB + r->iB * LB;
    } else {
        V2 P = v2(ix, iy);
        vA = sub(vA, scl(r->mA, P)); wA = wA - r->iA * (crs(r->rA, P) + iz);
        vB = add(vB, scl(r->mB, P)); wB = wB + r->iB * (crs(r->rB, P) + iz);
    }
    k->vx[ia] = vA.x; k->vy[ia] = vA.y; k->w[ia] = wA;
    k->vx[ib] = vB.x; k->vy[ib] = vB.y; k->w[ib] = wB;
}

/* SolveVelocityConstraints for one joint (joints.py:257-437) */
static void jn_solve_velocity(const Ctx* x, JR* r, Work* k) {
    int ia = r->ia, ib = r->ib;
    V2 vA = v2(k->vx[ia], k->vy[ia]), vB = v2(k->vx[ib], k->vy[ib]);
    float wA = k->w[ia], wB = k->w[ib];
    float mA = r->mA, mB = r->mB, iA = r->iA, iB = r->iB;
    float* imp = r->imp;
    if (r->type == GOI_REVOLUTE && x->s->revolute_v24) {
        int fixed = (iA + iB) == 0.0f;
        float am = r->motor_mass;
        if (r->enable_motor && !fixed) {
            float cdot = (wB - wA) - r->motor_speed;
            float impulse = -am * cdot;
            float old = r->mimp;
            r->mimp = bclamp(r->mimp + impulse, -r->max_impulse, r->max_impulse);
            impulse = r->mimp - old;
            wA = wA - iA * impulse;
            wB = wB + iB * impulse;
        }
        if (r->enable_limit && !fixed) {
            float C = r->angle - r->lower;
            float impulse = -am * ((wB - wA) + bmax(C, 0.0f) * r->inv_dt);
            float old = imp[3];
            imp[3] = bmax(imp[3] + impulse, 0.0f);
            impulse = imp[3] - old;
            wA = wA - iA * impulse;
            wB = wB + iB * impulse;
            C = r->upper - r->angle;
            impulse = -am * ((wA - wB) + bmax(C, 0.0f) * r->inv_dt);
            old = imp[4];
            imp[4] = bmax(imp[4] + impulse, 0.0f);
            impulse = imp[4] - old;
            wA = wA + iA * impulse;
            wB = wB - iB * impulse;
        }
        V2 c1 = rel_vel(vB, wB, r->rB, vA, wA, r->rA);
        V2 p = solve22(r->ex.x, r->ey.x, r->ex.y, r->ey.y, neg(c1));
        imp[0] = imp[0] + p.x; imp[1] = imp[1] + p.y;
        vA = sub(vA, scl(mA, p)); wA = wA - iA * crs(r->rA, p);
        vB = add(vB, scl(mB, p)); wB = wB + iB * crs(r->rB, p);
    } else if (r->type == GOI_REVOLUTE) {
        int fixed = (iA + iB) == 0.0f;
        int st = r->limit_state;
        if (r->enable_motor && st != EQUAL_LIMITS && !fixed) {
            float cdot = (wB - wA) - r->motor_speed;
            float impulse = -r->motor_mass * cdot;
            float old = r->mimp;
            r->mimp = bclamp(r->mimp + impulse, -r->max_impulse, r->max_impulse);
            impulse = r->mimp - old;
            wA = wA - iA * impulse;
            wB = wB + iB * impulse;
        }
        if (r->enable_limit && st != INACTIVE_LIMIT && !fixed) {
            V2 c1 = rel_vel(vB, wB, r->rB, vA, wA, r->rA);
            float c2 = wB - wA;
            V3 sv = solve33(r->ex, r->ey, r->ez, v3(c1.x, c1.y, c2));
            V3 j = v3(-sv.x, -sv.y, -sv.z);
            float new_z = imp[2] + j.z;
            int redo = (st == AT_LOWER && new_z < 0.0f) || (st == AT_UPPER && new_z > 0.0f);
            if (redo) {
                V2 rhs = v2(-c1.x + imp[2] * r->ez.x, -c1.y + imp[2] * r->ez.y);
                V2 red = solve22(r->ex.x, r->ey.x, r->ex.y, r->ey.y, rhs);
                j = v3(red.x, red.y, -imp[2]);
                imp[0] = imp[0] + red.x; imp[1] = imp[1] + red.y; imp[2] = 0.0f;
            } else {
                imp[0] = imp[0] + j.x; imp[1] = imp[1] + j.y; imp[2] = imp[2] + j.z;
            }
            V2 P = v2(j.x, j.y);
            vA = sub(vA, scl(mA, P)); wA = wA - iA * (crs(r->rA, P) + j.z);
            vB = add(vB, scl(mB, P)); wB = wB + iB * (crs(r->rB, P) + j.z);
        } else {
            V2 c1 = rel_vel(vB, wB, r->rB, vA, wA, r->rA);
            V2 p = solve22(r->ex.x, r->ey.x, r->ex.y, r->ey.y, neg(c1));
            imp[0] = imp[0] + p.x; imp[1] = imp[1] + p.y;
            vA = sub(vA, scl(mA, p)); wA = wA - iA * crs(r->rA, p);
            vB = add(vB, scl(mB, p)); wB = wB + iB * crs(r->rB, p);
        }
    } else if (r->type == GOI_PRISMATIC) {
        int st = r->limit_state;
        V2 axis = r->axis, perp = r->perp;
        if (r->enable_motor && st != EQUAL_LIMITS) {
            float cdot = (dot(axis, sub(vB, vA)) + r->a2 * wB) - r->a1 * wA;
            float impulse = r->motor_mass * (r->motor_speed - cdot);
            float old = r->mimp;
            r->mimp = bclamp(r->mimp + impulse, -r->max_impulse, r->max_impulse);
            impulse = r->mimp - old;
            V2 P = scl(impulse, axis);
            float LA = impulse * r->a1, LB = impulse * r->a2;
            vA = sub(vA, scl(mA, P)); wA = wA - iA * LA;
            vB = add(vB, scl(mB, P)); wB = wB + iB * LB;
        }
        float c1x = (dot(perp, sub(vB, vA)) + r->s2 * wB) - r->s1 * wA;
        float c1y = wB - wA;
        if (r->enable_limit && st != INACTIVE_LIMIT) {
            float c2 = (dot(axis, sub(vB, vA)) + r->a2 * wB) - r->a1 * wA;
            float f1x = imp[0], f1y = imp[1], f1z = imp[2];
            V3 df = solve33(r->ex, r->ey, r->ez, v3(-c1x, -c1y, -c2));
            float nx = f1x + df.x, ny = f1y + df.y, nz = f1z + df.z;
            (void)nx; (void)ny;
            if (st == AT_LOWER) nz = bmax(nz, 0.0f);
            else if (st == AT_UPPER) nz = bmin(nz, 0.0f);
            V2 b = v2(-c1x - (nz - f1z) * r->ez.x, -c1y - (nz - f1z) * r->ez.y);
            V2 f2 = solve22(r->ex.x, r->ey.x, r->ex.y, r->ey.y, b);
            f2 = v2(f2.x + f1x, f2.y + f1y);
            imp[0] = f2.x; imp[1] = f2.y; imp[2] = nz;
            float dfx = f2.x - f1x, dfy = f2.y - f1y, dfz = nz - f1z;
            V2 P = add(scl(dfx, perp), scl(dfz, axis));
            float LA = (dfx * r->s1 + dfy) + dfz * r->a1;
            float LB = (dfx * r->s2 + dfy) + dfz * r->a2;
            vA = sub(vA, scl(mA, P)); wA = wA - iA * LA;
            vB = add(vB, scl(mB, P)); wB = wB + iB * LB;
        } else {
            V2 df = solve22(r->ex.x, r->ey.x, r->ex.y, r->ey.y, v2(-c1x, -c1y));
            imp[0] = imp[0] + df.x; imp[1] = imp[1] + df.y;
            V2 P = scl(df.x, perp);
            float LA = df.x * r->s1 + df.y;
            float LB = df.x * r->s2 + df.y;
            vA = sub(vA, scl(mA, P)); wA = wA - iA * LA;
            vB = add(vB, scl(mB, P)); wB = wB + iB * LB;
        }
    } else { /* weld */
        if (r->soft) {
            float c2 = wB - wA;
            float i2 = -r->ez.z * ((c2 + r->bias) + r->gamma * imp[2]);
            imp[2] = imp[2] + i2;
            wA = wA - iA * i2;
            wB = wB + iB * i2;
            V2 c1 = rel_vel(vB, wB, r->rB, vA, wA, r->rA);
            V2 i1 = v2(-(r->ex.x * c1.x + r->ey.x * c1.y), -(r->ex.y * c1.x + r->ey.y * c1.y));
            imp[0] = imp[0] + i1.x; imp[1] = imp[1] + i1.y;
            vA = sub(vA, scl(mA, i1)); wA = wA - iA * crs(r->rA, i1);
            vB = add(vB, scl(mB, i1)); wB = wB + iB * crs(r->rB, i1);
        } else {
            V2 c1 = rel_vel(vB, wB, r->rB, vA, wA, r->rA);
            float c2 = wB - wA;
            float jx = -((c1.x * r->ex.x + c1.y * r->ey.x) + c2 * r->ez.x);
            float jy = -((c1.x * r->ex.y + c1.y * r->ey.y) + c2 * r->ez.y);
            float jz = -((c1.x * r->ex.z + c1.y * r->ey.z) + c2 * r->ez.z);
            imp[0] = imp[0] + jx; imp[1] = imp[1] + jy; imp[2] = imp[2] + jz;
            V2 P = v2(jx, jy);
            vA = sub(vA, scl(mA, P)); wA = wA - iA * (crs(r->rA, P) + jz);
            vB = add(vB, scl(mB, P)); wB = wB + iB * (crs(r->rB, P) + jz);
        }
    }
    k->vx[ia] = vA.x; k->vy[ia] = vA.y; k->w[ia] = wA;
    k->vx[ib] = vB.x; k->vy[ib] = vB.y; k->w[ib] = wB;
}

/* the point-to-point part of the revolute position solve (joints.py:501-520) */
static int rev_point_position(const Ctx* x, const JR* r, V2* cA, float* aA, V2* cB, float* aB, float ang_err) {
    const GoiSettings* s = x->s;
    float mA = r->mA, mB = r->mB, iA = r->iA, iB = r->iB;
    Rot qA = rot_of(*aA), qB = rot_of(*aB);
    V2 rA = rmul(qA, r->la), rB = rmul(qB, r->lb);
    V2 C = sub(sub(add(*cB, rB), *cA), rA);
    float pos_err = len(C);
    float kxx = ((mA + mB) + iA * rA.y * rA.y) + iB * rB.y * rB.y;
    float kxy = -iA * rA.x * rA.y - iB * rB.x * rB.y;
    float kyy = ((mA + mB) + iA * rA.x * rA.x) + iB * rB.x * rB.x;
    V2 j = solve22(kxx, kxy, kxy, kyy, C);
    j = neg(j);
    *cA = sub(*cA, scl(mA, j)); *aA = *aA - iA * crs(rA, j);
    *cB = add(*cB, scl(mB, j)); *aB = *aB + iB * crs(rB, j);
    return pos_err <= s->linear_slop && ang_err <= s->angular_slop;
}

/* SolvePositionConstraints for one joint (joints.py:462-606) */
static int jn_solve_position(const Ctx* x, const JR* r, Work* k) {
    const GoiSettings* s = x->s;
    int ia = r->ia, ib = r->ib;
    V2 cA = v2(k->cx[ia], k->cy[ia]), cB = v2(k->cx[ib], k->cy[ib]);
    float aA = k->a[ia], aB = k->a[ib];
    float mA = r->mA, mB = r->mB, iA = r->iA, iB = r->iB;
    int ok;
    float mac = s->max_angular_correction;
    if (r->type == GOI_REVOLUTE && s->revolute_v24) {
        int fixed = (iA + iB) == 0.0f;
        float ang_err = 0.0f;
        if (r->enable_limit && !fixed) {
            float angle = (aB - aA) - r->ref;
            float C = 0.0f;
            if (babs(r->upper - r->lower) < 2.0f * s->angular_slop)
                C = bclamp(angle - r->lower, -mac, mac);
            else if (angle <= r->lower)
                C = bclamp((angle - r->lower) + s->angular_slop, -mac, 0.0f);
            else if (angle >= r->upper)
                C = bclamp((angle - r->upper) - s->angular_slop, 0.0f, mac);
            float li = -r->motor_mass * C;
            aA = aA - iA * li;
            aB = aB + iB * li;
            ang_err = babs(C);
        }
        ok = rev_point_position(x, r, &cA, &aA, &cB, &aB, ang_err);
    } else if (r->type == GOI_REVOLUTE) {
        int fixed = (iA + iB) == 0.0f;
        int st = r->limit_state;
        float ang_err = 0.0f;
        if (r->enable_limit && st != INACTIVE_LIMIT && !fixed) {
            float angle = (aB - aA) - r->ref;
            float li = 0.0f;
            if (st == EQUAL_LIMITS) {
                float C = bclamp(angle - r->lower, -mac, mac);
                li = -r->motor_mass * C;
                ang_err = babs(C);
            } else if (st == AT_LOWER) {
                float C = angle - r->lower;
                ang_err = -C;
                C = bclamp(C + s->angular_slop, -mac, 0.0f);
                li = -r->motor_mass * C;
            } else {
                float C = angle - r->upper;
                ang_err = C;
                C = bclamp(C - s->angular_slop, 0.0f, mac);
                li = -r->motor_mass * C;
            }
            aA = aA - iA * li;
            aB = aB + iB * li;
        }
        ok = rev_point_position(x, r, &cA, &aA, &cB, &aB, ang_err);
    } else if (r->type == GOI_PRISMATIC) {
        Rot qA = rot_of(aA), qB = rot_of(aB);
        V2 rA = rmul(qA, r->la), rB = rmul(qB, r->lb);
        V2 d = sub(sub(add(cB, rB), cA), rA);
        V2 axis = rmul(qA, r->lx);
        float a1 = crs(add(d, rA), axis), a2 = crs(rB, axis);
        V2 perp = rmul(qA, r->ly);
        float s1 = crs(add(d, rA), perp), s2 = crs(rB, perp);
        float c1x = dot(perp, d);
        float c1y = (aB - aA) - r->ref;
        float lin_err = babs(c1x), ang_err = babs(c1y);
        int active = 0;
        float C2 = 0.0f;
        float mlc = s->max_linear_correction;
        if (r->enable_limit) {
            float t = dot(axis, d);
            if (babs(r->upper - r->lower) < 2.0f * s->linear_slop) {
                C2 = bclamp(t, -mlc, mlc);
                lin_err = bmax(lin_err, babs(t));
                active = 1;
            } else if (t <= r->lower) {
                C2 = bclamp((t - r->lower) + s->linear_slop, -mlc, 0.0f);
                lin_err = bmax(lin_err, r->lower - t);
                active = 1;
            } else if (t >= r->upper) {
                C2 = bclamp((t - r->upper) - s->linear_slop, 0.0f, mlc);
                lin_err = bmax(lin_err, t - r->upper);
                active = 1;
            }
        }
        float k11 = ((mA + mB) + iA * s1 * s1) + iB * s2 * s2;
        float k12 = iA * s1 + iB * s2;
        float k22 = iA + iB;
        if (k22 == 0.0f) k22 = 1.0f;
        V3 imp;
        if (active) {
            float k13 = iA * s1 * a1 + iB * s2 * a2;
            float k23 = iA * a1 + iB * a2;
            float k33 = ((mA + mB) + iA * a1 * a1) + iB * a2 * a2;
            imp = solve33(v3(k11, k12, k13), v3(k12, k22, k23), v3(k13, k23, k33), v3(-c1x, -c1y, -C2));
        } else {
            V2 i2 = solve22(k11, k12, k12, k22, v2(-c1x, -c1y));
            imp = v3(i2.x, i2.y, 0.0f);
        }
        V2 P = add(scl(imp.x, perp), scl(imp.z, axis));
        float LA = (imp.x * s1 + imp.y) + imp.z * a1;
        float LB = (imp.x * s2 + imp.y) + imp.z * a2;
        cA = sub(cA, scl(mA, P)); aA = aA - iA * LA;
        cB = add(cB, scl(mB, P)); aB = aB + iB * LB;
        ok = lin_err <= s->linear_slop && ang_err <= s->angular_slop;
    } else { /* weld */
        Rot qA = rot_of(aA), qB = rot_of(aB);
        V2 rA = rmul(qA, r->la), rB = rmul(qB, r->lb);
        float exx = ((mA + mB) + rA.y * rA.y * iA) + rB.y * rB.y * iB;
        float eyx = -rA.y * rA.x * iA - rB.y * rB.x * iB;
        float ezx = -rA.y * iA - rB.y * iB;
        float eyy = ((mA + mB) + rA.x * rA.x * iA) + rB.x * rB.x * iB;
        float ezy = rA.x * iA + rB.x * iB;
        float ezz = iA + iB;
        V3 ex = v3(exx, eyx, ezx), ey = v3(eyx, eyy, ezy), ez = v3(ezx, ezy, ezz);
        V2 C1 = sub(sub(add(cB, rB), cA), rA);
        float pos_err = len(C1), ang_err;
        V3 imp;
        if (r->soft) {
            ang_err = 0.0f;
            V2 p = solve22(ex.x, ey.x, ex.y, ey.y, C1);
            imp = v3(-p.x, -p.y, 0.0f);
            V2 P = v2(imp.x, imp.y);
            cA = sub(cA, scl(mA, P)); aA = aA - iA * crs(rA, P);
            cB = add(cB, scl(mB, P)); aB = aB + iB * crs(rB, P);
        } else {
            float C2 = (aB - aA) - r->ref;
            ang_err = babs(C2);
            if (ez.z > 0.0f) {
                V3 p = solve33(ex, ey, ez, v3(C1.x, C1.y, C2));
                imp = v3(-p.x, -p.y, -p.z);
            } else {
                V2 p = solve22(ex.x, ey.x, ex.y, ey.y, C1);
                imp = v3(-p.x, -p.y, 0.0f);
            }
            V2 P = v2(imp.x, imp.y);
            cA = sub(cA, scl(mA, P)); aA = aA - iA * (crs(rA, P) + imp.z);
            cB = add(cB, scl(mB, P)); aB = aB + iB * (crs(rB, P) + imp.z);
        }
        ok = pos_err <= s->linear_slop && ang_err <= s->angular_slop;
    }
    k->cx[ia] = cA.x; k->cy[ia] = cA.y; k->a[ia] = aA;
    k->cx[ib] = cB.x; k->cy[ib] = cB.y; k->a[ib] = aB;
    return ok;
}

static void jn_store(const Ctx* x, W* w, const JR* r) {
    int j = r->jid;
    w->j_impulse[3 * j] = r->imp[0]; w->j_impulse[3 * j + 1] = r->imp[1]; w->j_impulse[3 * j + 2] = r->imp[2];
    w->j_motor_impulse[j] = r->mimp;
    w->j_limit_state[j] = r->limit_state;
    if (x->s->revolute_v24) { w->j_lower_impulse[j] = r->imp[3]; w->j_upper_impulse[j] = r->imp[4]; }
}

/* ------------------------------------------------------------------------------------------------ Solve (step.py:73-182) */

static void solve(const Ctx* x, W* w, Work* k, float dt, float dt_ratio, GoiDebug* dbg, int wi, int pitch) {
    const GoiModelDesc* m = x->m;
    const GoiSettings* s = x->s;
    int B = w->B, C = w->C;
    int nc, nj;
    int nisl = find_islands(x, w, k, &nc, &nj);
    float h = dt;
    /* Integrate velocities (dynamic island bodies) and start the sweeps: c0 = c for every island body. */
    for (int b = 0; b < B; ++b) {
        k->vx[b] = w->b_v[2 * b]; k->vy[b] = w->b_v[2 * b + 1]; k->w[b] = w->b_w[b];
        k->cx[b] = w->b_c[2 * b]; k->cy[b] = w->b_c[2 * b + 1]; k->a[b] = w->b_a[b];
        if (k->body_island[b] < 0) continue;
        if (w->b_type[b] == GOI_DYNAMIC) {
            float ax = w->b_gs[b] * w->gravity[0] + w->b_inv_mass[b] * w->b_force[2 * b];
            float ay = w->b_gs[b] * w->gravity[1] + w->b_inv_mass[b] * w->b_force[2 * b + 1];
            float vx = w->b_v[2 * b] + h * ax;
            float vy = w->b_v[2 * b + 1] + h * ay;
            float ww = w->b_w[b] + h * w->b_inv_inertia[b] * w->b_torque[b];
            float ld = 1.0f / (1.0f + h * w->b_ld[b]);
            float ad = 1.0f / (1.0f + h * w->b_ad[b]);
            k->vx[b] = vx * ld; k->vy[b] = vy * ld; k->w[b] = ww * ad;
        }
        w->b_c0[2 * b] = w->b_c[2 * b]; w->b_c0[2 * b + 1] = w->b_c[2 * b + 1];
        w->b_a0[b] = w->b_a[b];
    }
    Rot q[64];
    Rot* qq = B <= 64 ? q : (Rot*)malloc(sizeof(Rot) * B);
    for (int b = 0; b < B; ++b) qq[b] = rot_of(k->a[b]);
    int warm = s->warm_starting;
    for (int i = 0; i < nc; ++i) cs_prepare(x, w, k, &k->cc[i], k->corder[i], warm, dt_ratio, qq);
    if (warm)
        for (int i = 0; i < nc; ++i) cs_warm_start(&k->cc[i], k);
    for (int i = 0; i < nj; ++i) jn_prepare(x, w, k, &k->jr[i], k->jorder[i], dt, dt_ratio, warm, qq);
    for (int i = 0; i < nj; ++i) jn_warm_start(x, &k->jr[i], k);
    if (qq != q) free(qq);
    for (int it = 0; it < s->velocity_iterations; ++it) {
        for (int i = 0; i < nj; ++i) jn_solve_velocity(x, &k->jr[i], k);
        for (int i = 0; i < nc; ++i) cs_solve_velocity(&k->cc[i], k);
    }
    /* StoreImpulses: points j < the velocity constraint's pointCount (contact_solver.py:293-304) */
    for (int i = 0; i < nc; ++i) {
        const CC* c = &k->cc[i];
        for (int j = 0; j < c->count; ++j) {
            w->c_ni[2 * c->slot + j] = c->ni[j];
            w->c_ti[2 * c->slot + j] = c->ti[j];
        }
    }
    for (int i = 0; i < nj; ++i) jn_store(x, w, &k->jr[i]);
    /* Integrate positions with the per-step translation / rotation clamps (step.py:120-135) */
    float max_t = s->clamps_per_second ? s->max_translation * h : s->max_translation;
    float max_r = s->clamps_per_second ? s->max_rotation * h : s->max_rotation;
    for (int b = 0; b < B; ++b) {
        if (k->body_island[b] < 0) continue;
        V2 v = v2(k->vx[b], k->vy[b]);
        float ww = k->w[b];
        V2 t = scl(h, v);
        if (dot(t, t) > max_t * max_t) {
            float ratio = max_t / len(t);
            v = v2(v.x * ratio, v.y * ratio);
        }
        float rot = h * ww;
        if (rot * rot > max_r * max_r) {
            float ratio = max_r / babs(rot);
            ww = ww * ratio;
        }
        k->cx[b] = k->cx[b] + h * v.x; k->cy[b] = k->cy[b] + h * v.y; k->a[b] = k->a[b] + h * ww;
        k->vx[b] = v.x; k->vy[b] = v.y; k->w[b] = ww;
    }
    /* Position iterations, each island stopping at its first pass within tolerance (step.py:197-251) */
    for (int i = 0; i < B; ++i) k->done[i] = i >= nisl;
    for (int it = 0; it < s->position_iterations; ++it) {
        int more = 0;
        for (int i = 0; i < nisl; ++i) more |= !k->done[i];
        if (!more) break;
        for (int i = 0; i < nisl; ++i) { k->min_sep[i] = 0.0f; k->jok[i] = 1; }
        for (int i = 0; i < nc; ++i) {
            const CC* c = &k->cc[i];
            int isl = k->contact_island[c->slot];
            if (k->done[isl]) continue;
            float ms = cs_solve_position(x, c, k, s->baumgarte, c->mA, c->mB, c->iA, c->iB);
            k->min_sep[isl] = bmin(k->min_sep[isl], ms);
        }
        for (int i = 0; i < nj; ++i) {
            const JR* r = &k->jr[i];
            int isl = k->joint_island[r->jid];
            if (k->done[isl]) continue;
            int ok = jn_solve_position(x, r, k);
            k->jok[isl] = k->jok[isl] && ok;
        }
        for (int i = 0; i < nisl; ++i)
            if (!k->done[i] && k->min_sep[i] >= -3.0f * s->linear_slop && k->jok[i]) k->done[i] = 1;
    }
    /* Write back + SynchronizeTransform (island bodies) */
    for (int b = 0; b < B; ++b) {
        if (k->body_island[b] < 0) continue;
        w->b_c[2 * b] = k->cx[b]; w->b_c[2 * b + 1] = k->cy[b]; w->b_a[b] = k->a[b];
        w->b_v[2 * b] = k->vx[b]; w->b_v[2 * b + 1] = k->vy[b]; w->b_w[b] = k->w[b];
        Rot qb = rot_of(k->a[b]);
        V2 r = rmul(qb, getv(w->b_lc, b));
        w->b_xf_p[2 * b] = k->cx[b] - r.x; w->b_xf_p[2 * b + 1] = k->cy[b] - r.y;
        w->b_xf_q[2 * b] = qb.c; w->b_xf_q[2 * b + 1] = qb.s;
    }
    /* Sleep, per island (step.py:153-168) */
    for (int i = 0; i < B; ++i) k->isl_sleep[i] = 0;
    if (s->allow_sleep) {
        float lin_tol = s->linear_sleep_tolerance * s->linear_sleep_tolerance;
        float ang_tol = s->angular_sleep_tolerance * s->angular_sleep_tolerance;
        for (int i = 0; i < nisl; ++i) k->min_st[i] = MAXF;
        for (int b = 0; b < B; ++b) {
            int isl = k->body_island[b];
            if (isl < 0 || w->b_type[b] == GOI_STATIC) continue;
            V2 v = getv(w->b_v, b);
            int moving = !w->b_allow_sleep[b] || w->b_w[b] * w->b_w[b] > ang_tol || dot(v, v) > lin_tol;
            if (moving) { w->b_sleep_time[b] = 0.0f; k->min_st[isl] = 0.0f; }
            else { w->b_sleep_time[b] = w->b_sleep_time[b] + h; k->min_st[isl] = bmin(k->min_st[isl], w->b_sleep_time[b]); }
        }
        for (int i = 0; i < nisl; ++i) k->isl_sleep[i] = k->min_st[i] >= s->time_to_sleep && k->done[i];
        for (int b = 0; b < B; ++b) {
            int isl = k->body_island[b];
            if (isl < 0 || w->b_type[b] == GOI_STATIC || !k->isl_sleep[isl]) continue;
            w->b_sleep_time[b] = 0.0f; w->b_awake[b] = 0;
            w->b_v[2 * b] = 0.0f; w->b_v[2 * b + 1] = 0.0f; w->b_w[b] = 0.0f;
            w->b_force[2 * b] = 0.0f; w->b_force[2 * b + 1] = 0.0f; w->b_torque[b] = 0.0f;
        }
    }
    /* Static bodies end with the awake flag of the last island that included them (step.py:173-194) */
    for (int b = 0; b < B; ++b) k->last[b] = -1;
    for (int c = 0; c < C; ++c) {
        int isl = k->contact_island[c];
        if (isl < 0) continue;
        int ba = m->fixture_body[w->c_fa[c]], bb = m->fixture_body[w->c_fb[c]];
        if (isl > k->last[ba]) k->last[ba] = isl;
        if (isl > k->last[bb]) k->last[bb] = isl;
    }
    for (int j = 0; j < m->J; ++j) {
        int isl = k->joint_island[j];
        if (isl < 0) continue;
        int ja = m->joint_a[j], jb = m->joint_b[j];
        if (isl > k->last[ja]) k->last[ja] = isl;
        if (isl > k->last[jb]) k->last[jb] = isl;
    }
    for (int b = 0; b < B; ++b) {
        if (w->b_type[b] != GOI_STATIC || k->last[b] < 0) continue;
        w->b_awake[b] = !k->isl_sleep[k->last[b]];
        w->b_sleep_time[b] = 0.0f;
    }
    if (dbg) {
        for (int b = 0; b < B; ++b) if (dbg->body_island) dbg->body_island[(size_t)b * pitch + wi] = k->body_island[b];
        for (int c = 0; c < C; ++c) {
            if (dbg->contact_island) dbg->contact_island[(size_t)c * pitch + wi] = k->contact_island[c];
            if (dbg->contact_order) dbg->contact_order[(size_t)c * pitch + wi] = c < nc ? k->corder[c] : -1;
        }
        if (dbg->n_islands) dbg->n_islands[wi] = nisl;
    }
    /* SynchronizeFixtures of island bodies that are not static, then FindNewContacts */
    for (int b = 0; b < B; ++b) k->moved[b] = k->body_island[b] >= 0 && w->b_type[b] != GOI_STATIC;
    synchronize_fixtures(x, w, k->moved);
    find_new_contacts(x, w);
}

/* ------------------------------------------------------------------------------------------------ TOI (toi.py) */

typedef struct { V2 lc, c0, c; float a0, a; } Sweep;

/* b2Sweep::GetTransform (toi.py:73-81) */
static Xf sweep_xf(const Sweep* sw, float beta) {
    Xf t;
    float omb = 1.0f - beta;
    t.p = v2(omb * sw->c0.x + beta * sw->c.x, omb * sw->c0.y + beta * sw->c.y);
    t.q = rot_of(omb * sw->a0 + beta * sw->a);
    t.p = sub(t.p, rmul(t.q, sw->lc));
    return t;
}

/* b2Sweep::Normalize (toi.py:92-97) */
static void sweep_normalize(Sweep* sw) {
    float two_pi = 2.0f * 3.14159265359f;
    float d = two_pi * floorf(sw->a0 / two_pi);
    sw->a0 = sw->a0 - d;
    sw->a = sw->a - d;
}

static Sweep body_sweep(const W* w, int b) {
    Sweep s;
    s.lc = getv(w->b_lc, b); s.c0 = getv(w->b_c0, b); s.c = getv(w->b_c, b);
    s.a0 = w->b_a0[b]; s.a = w->b_a[b];
    return s;
}

/* b2Sweep::Advance (toi.py:100-104), on the body's sweep */
static void sweep_advance(W* w, int b, float alpha) {
    float al0 = w->t_alpha0[b];
    float den = 1.0f - al0;
    float beta = (alpha - al0) / (den != 0.0f ? den : 1.0f);
    w->b_c0[2 * b] = w->b_c0[2 * b] + beta * (w->b_c[2 * b] - w->b_c0[2 * b]);
    w->b_c0[2 * b + 1] = w->b_c0[2 * b + 1] + beta * (w->b_c[2 * b + 1] - w->b_c0[2 * b + 1]);
    w->b_a0[b] = w->b_a0[b] + beta * (w->b_a[b] - w->b_a0[b]);
    w->t_alpha0[b] = alpha;
}

/* b2Body::SynchronizeTransform */
static void sync_transform(W* w, int b) {
    Rot q = rot_of(w->b_a[b]);
    V2 r = rmul(q, getv(w->b_lc, b));
    w->b_xf_p[2 * b] = w->b_c[2 * b] - r.x; w->b_xf_p[2 * b + 1] = w->b_c[2 * b + 1] - r.y;
    w->b_xf_q[2 * b] = q.c; w->b_xf_q[2 * b + 1] = q.s;
}

/* b2Body::Advance: sweep to alpha, the body at the new sweep start */
static void body_advance(W* w, int b, float alpha) {
    sweep_advance(w, b, alpha);
    w->b_c[2 * b] = w->b_c0[2 * b]; w->b_c[2 * b + 1] = w->b_c0[2 * b + 1];
    w->b_a[b] = w->b_a0[b];
    sync_transform(w, b);
}

static void backup_sweep(const W* w, Work* k, int b) {
    float* s = k->bk + 7 * b;
    s[0] = w->b_c0[2 * b]; s[1] = w->b_c0[2 * b + 1]; s[2] = w->b_c[2 * b]; s[3] = w->b_c[2 * b + 1];
    s[4] = w->b_a0[b]; s[5] = w->b_a[b]; s[6] = w->t_alpha0[b];
}
static void restore_sweep(W* w, const Work* k, int b) {
    const float* s = k->bk + 7 * b;
    w->b_c0[2 * b] = s[0]; w->b_c0[2 * b + 1] = s[1]; w->b_c[2 * b] = s[2]; w->b_c[2 * b + 1] = s[3];
    w->b_a0[b] = s[4]; w->b_a[b] = s[5]; w->t_alpha0[b] = s[6];
    sync_transform(w, b);
}

/* ---- b2Distance (toi.py:116-294) */

typedef struct { const float* v; int count; float radius; } Proxy;

static inline V2 pvert(const Proxy* p, int i) { return v2(p->v[2 * i], p->v[2 * i + 1]); }
static Proxy proxy_of(const GoiModelDesc* m, int f) {
    Proxy p; p.v = m->verts + (size_t)f * NPOLY * 2; p.count = m->count[f]; p.radius = m->radius[f]; return p;
}
/* b2DistanceProxy::GetSupport: first index of the largest b2Dot(v_i, d) */
static int support(const Proxy* p, V2 d) {
    int best = 0;
    float bv = dot(pvert(p, 0), d);
    for (int i = 1; i < p->count; ++i) {
        float v = dot(pvert(p, i), d);
        if (v > bv) { best = i; bv = v; }
    }
    return best;
}

typedef struct { V2 wA, wB, w; float a; int iA, iB; } SV;
typedef struct { float metric; int count; int iA[3], iB[3]; } Cache;

static float simplex_metric(const SV* v, int count) {
    if (count == 2) return len(sub(v[0].w, v[1].w));
    if (count == 3) return crs(sub(v[1].w, v[0].w), sub(v[2].w, v[0].w));
    return 0.0f;
}

static void make_vertex(SV* v, const Proxy* pA, Xf xA, int iA, const Proxy* pB, Xf xB, int iB) {
    v->iA = iA; v->iB = iB;
    v->wA = xmul(xA, pvert(pA, iA));
    v->wB = xmul(xB, pvert(pB, iB));
    v->w = sub(v->wB, v->wA);
}

static void solve2(SV* v, int* count) {
    V2 w1 = v[0].w, w2 = v[1].w;
    V2 e12 = sub(w2, w1);
    float d12_2 = -dot(w1, e12);
    if (d12_2 <= 0.0f) { v[0].a = 1.0f; *count = 1; return; }
    float d12_1 = dot(w2, e12);
    if (d12_1 <= 0.0f) { v[1].a = 1.0f; *count = 1; v[0] = v[1]; return; }
    float inv = 1.0f / (d12_1 + d12_2);
    v[0].a = d12_1 * inv; v[1].a = d12_2 * inv; *count = 2;
}

static void solve3(SV* v, int* count) {
    V2 w1 = v[0].w, w2 = v[1].w, w3 = v[2].w;
    V2 e12 = sub(w2, w1);
    float d12_1 = dot(w2, e12), d12_2 = -dot(w1, e12);
    V2 e13 = sub(w3, w1);
    float d13_1 = dot(w3, e13), d13_2 = -dot(w1, e13);
    V2 e23 = sub(w3, w2);
    float d23_1 = dot(w3, e23), d23_2 = -dot(w2, e23);
    float n123 = crs(e12, e13);
    float d123_1 = n123 * crs(w2, w3);
    float d123_2 = n123 * crs(w3, w1);
    float d123_3 = n123 * crs(w1, w2);
    if (d12_2 <= 0.0f && d13_2 <= 0.0f) { v[0].a = 1.0f; *count = 1; return; }
    if (d12_1 > 0.0f && d12_2 > 0.0f && d123_3 <= 0.0f) {
        float inv = 1.0f / (d12_1 + d12_2);
        v[0].a = d12_1 * inv; v[1].a = d12_2 * inv; *count = 2; return;
    }
    if (d13_1 > 0.0f && d13_2 > 0.0f && d123_2 <= 0.0f) {
        float inv = 1.0f / (d13_1 + d13_2);
        v[0].a = d13_1 * inv; v[2].a = d13_2 * inv; *count = 2; v[1] = v[2]; return;
    }
    if (d12_1 <= 0.0f && d23_2 <= 0.0f) { v[1].a = 1.0f; *count = 1; v[0] = v[1]; return; }
    if (d13_1 <= 0.0f && d23_1 <= 0.0f) { v[2].a = 1.0f; *count = 1; v[0] = v[2]; return; }
    if (d23_1 > 0.0f && d23_2 > 0.0f && d123_1 <= 0.0f) {
        float inv = 1.0f / (d23_1 + d23_2);
        v[1].a = d23_1 * inv; v[2].a = d23_2 * inv; *count = 2; v[0] = v[2]; return;
    }
    float inv = 1.0f / ((d123_1 + d123_2) + d123_3);
    v[0].a = d123_1 * inv; v[1].a = d123_2 * inv; v[2].a = d123_3 * inv; *count = 3;
}

/* b2Distance with useRadii = false; returns the distance and updates the cache */
static float distance(Cache* cache, const Proxy* pA, Xf xA, const Proxy* pB, Xf xB) {
    SV v[3];
    memset(v, 0, sizeof(v));
    int count = cache->count;
    for (int i = 0; i < count; ++i) {
        make_vertex(&v[i], pA, xA, cache->iA[i], pB, xB, cache->iB[i]);
        v[i].a = 0.0f;
    }
    if (count > 1) {
        float m1 = cache->metric, m2 = simplex_metric(v, count);
        if (m2 < 0.5f * m1 || 2.0f * m1 < m2 || m2 < EPS) count = 0;
    }
    if (count == 0) {
        make_vertex(&v[0], pA, xA, 0, pB, xB, 0);
        v[0].a = 1.0f;
        count = 1;
    }
    int saveA[3], saveB[3], iter = 0;
    while (iter < 20) {
        int save = count;
        for (int i = 0; i < save; ++i) { saveA[i] = v[i].iA; saveB[i] = v[i].iB; }
        if (count == 2) solve2(v, &count);
        else if (count == 3) solve3(v, &count);
        if (count == 3) break;
        V2 d;
        if (count == 1) d = neg(v[0].w);
        else {
            V2 e12 = sub(v[1].w, v[0].w);
            float sgn = crs(e12, neg(v[0].w));
            d = sgn > 0.0f ? crs_sv(1.0f, e12) : crs_vs(e12, 1.0f);
        }
        if (dot(d, d) < EPS * EPS) break;
        SV* nv = &v[count];
        float keep_a = nv->a; /* the tentative vertex's barycentric coordinate is not set */
        make_vertex(nv, pA, xA, support(pA, rmulT(xA.q, neg(d))), pB, xB, support(pB, rmulT(xB.q, d)));
        nv->a = keep_a;
        ++iter;
        int dup = 0;
        for (int i = 0; i < save; ++i)
            if (nv->iA == saveA[i] && nv->iB == saveB[i]) { dup = 1; break; }
        if (dup) break;
        ++count;
    }
    V2 pa, pb;
    if (count == 1) { pa = v[0].wA; pb = v[0].wB; }
    else if (count == 2) {
        pa = add(scl(v[0].a, v[0].wA), scl(v[1].a, v[1].wA));
        pb = add(scl(v[0].a, v[0].wB), scl(v[1].a, v[1].wB));
    } else {
        pa = add(add(scl(v[0].a, v[0].wA), scl(v[1].a, v[1].wA)), scl(v[2].a, v[2].wA));
        pb = pa;
    }
    float dist = len(sub(pa, pb));
    cache->metric = simplex_metric(v, count);
    cache->count = count;
    for (int i = 0; i < count; ++i) { cache->iA[i] = v[i].iA; cache->iB[i] = v[i].iB; }
    return dist;
}

/* ---- b2SeparationFunction (toi.py:299-359) */

enum { SEP_POINTS = 0, SEP_FACE_A = 1, SEP_FACE_B = 2 };
typedef struct { int type; V2 axis, lp; } SepFn;

static void sep_init(SepFn* f, const Cache* cache, const Proxy* pA, const Sweep* sA, const Proxy* pB,
                     const Sweep* sB, float t1) {
    Xf xA = sweep_xf(sA, t1), xB = sweep_xf(sB, t1);
    f->lp = v2(0.0f, 0.0f);
    if (cache->count == 1) {
        f->type = SEP_POINTS;
        V2 a = xmul(xA, pvert(pA, cache->iA[0])), b = xmul(xB, pvert(pB, cache->iB[0]));
        f->axis = sub(b, a);
        normalize(&f->axis);
    } else if (cache->iA[0] == cache->iA[1]) {
        f->type = SEP_FACE_B;
        V2 b1 = pvert(pB, cache->iB[0]), b2 = pvert(pB, cache->iB[1]);
        f->axis = crs_vs(sub(b2, b1), 1.0f);
        normalize(&f->axis);
        V2 n = rmul(xB.q, f->axis);
        f->lp = scl(0.5f, add(b1, b2));
        V2 pb = xmul(xB, f->lp);
        V2 pa = xmul(xA, pvert(pA, cache->iA[0]));
        float s = dot(sub(pa, pb), n);
        if (s < 0.0f) f->axis = neg(f->axis);
    } else {
        f->type = SEP_FACE_A;
        V2 a1 = pvert(pA, cache->iA[0]), a2 = pvert(pA, cache->iA[1]);
        f->axis = crs_vs(sub(a2, a1), 1.0f);
        normalize(&f->axis);
        V2 n = rmul(xA.q, f->axis);
        f->lp = scl(0.5f, add(a1, a2));
        V2 pa = xmul(xA, f->lp);
        V2 pb = xmul(xB, pvert(pB, cache->iB[0]));
        float s = dot(sub(pb, pa), n);
        if (s < 0.0f) f->axis = neg(f->axis);
    }
}

static float sep_eval(const SepFn* f, const Proxy* pA, const Sweep* sA, const Proxy* pB, const Sweep* sB, int iA,
                      int iB, float t) {
    Xf xA = sweep_xf(sA, t), xB = sweep_xf(sB, t);
    if (f->type == SEP_POINTS) {
        V2 a = xmul(xA, pvert(pA, iA)), b = xmul(xB, pvert(pB, iB));
        return dot(sub(b, a), f->axis);
    } else if (f->type == SEP_FACE_A) {
        V2 n = rmul(xA.q, f->axis);
        V2 a = xmul(xA, f->lp);
        V2 b = xmul(xB, pvert(pB, iB));
        return dot(sub(b, a), n);
    } else {
        V2 n = rmul(xB.q, f->axis);
        V2 b = xmul(xB, f->lp);
        V2 a = xmul(xA, pvert(pA, iA));
        return dot(sub(a, b), n);
    }
}

static float sep_find_min(const SepFn* f, const Proxy* pA, const Sweep* sA, const Proxy* pB, const Sweep* sB,
                          int* iA, int* iB, float t) {
    Xf xA = sweep_xf(sA, t), xB = sweep_xf(sB, t);
    if (f->type == SEP_POINTS) {
        *iA = support(pA, rmulT(xA.q, f->axis));
        *iB = support(pB, rmulT(xB.q, neg(f->axis)));
        V2 a = xmul(xA, pvert(pA, *iA)), b = xmul(xB, pvert(pB, *iB));
        return dot(sub(b, a), f->axis);
    } else if (f->type == SEP_FACE_A) {
        V2 n = rmul(xA.q, f->axis);
        V2 a = xmul(xA, f->lp);
        *iA = -1;
        *iB = support(pB, rmulT(xB.q, neg(n)));
        V2 b = xmul(xB, pvert(pB, *iB));
        return dot(sub(b, a), n);
    } else {
        V2 n = rmul(xB.q, f->axis);
        V2 b = xmul(xB, f->lp);
        *iB = -1;
        *iA = support(pA, rmulT(xA.q, neg(n)));
        V2 a = xmul(xA, pvert(pA, *iA));
        return dot(sub(a, b), n);
    }
}

enum { E_UNKNOWN = 0, E_FAILED = 1, E_OVERLAPPED = 2, E_TOUCHING = 3, E_SEPARATED = 4 };

/* b2TimeOfImpact with tMax = 1 (toi.py:364-457) */
static int time_of_impact(const Proxy* pA, Sweep sA, const Proxy* pB, Sweep sB, float linear_slop, float* t_out) {
    sweep_normalize(&sA);
    sweep_normalize(&sB);
    float total_radius = pA->radius + pB->radius;
    float target = bmax(linear_slop, total_radius - 3.0f * linear_slop);
    float tol = 0.25f * linear_slop;
    float t1 = 0.0f;
    int iter = 0;
    Cache cache;
    memset(&cache, 0, sizeof(cache));
    int state = E_UNKNOWN;
    float out_t = 1.0f;
    for (;;) {
        Xf xA = sweep_xf(&sA, t1), xB = sweep_xf(&sB, t1);
        float dist = distance(&cache, pA, xA, pB, xB);
        if (dist <= 0.0f) { state = E_OVERLAPPED; out_t = 0.0f; break; }
        if (dist < target + tol) { state = E_TOUCHING; out_t = t1; break; }
        SepFn f;
        sep_init(&f, &cache, pA, &sA, pB, &sB, t1);
        int done = 0;
        float t2 = 1.0f;
        int push = 0;
        for (;;) {
            int iA, iB;
            float s2 = sep_find_min(&f, pA, &sA, pB, &sB, &iA, &iB, t2);
            if (s2 > target + tol) { state = E_SEPARATED; out_t = 1.0f; done = 1; break; }
            if (s2 > target - tol) { t1 = t2; break; }
            float s1 = sep_eval(&f, pA, &sA, pB, &sB, iA, iB, t1);
            if (s1 < target - tol) { state = E_FAILED; out_t = t1; done = 1; break; }
            if (s1 <= target + tol) { state = E_TOUCHING; out_t = t1; done = 1; break; }
            int rc = 0;
            float a1 = t1, a2 = t2;
            for (;;) {
                float t;
                if (rc & 1) t = a1 + (target - s1) * (a2 - a1) / (s2 - s1);
                else t = 0.5f * (a1 + a2);
                ++rc;
                float s = sep_eval(&f, pA, &sA, pB, &sB, iA, iB, t);
                if (babs(s - target) < tol) { t2 = t; break; }
                if (s > target) { a1 = t; s1 = s; }
                else { a2 = t; s2 = s; }
                if (rc == 50) break;
            }
            ++push;
            if (push == NPOLY) break;
        }
        ++iter;
        if (done) break;
        if (iter == 20) { state = E_FAILED; out_t = t1; break; }
    }
    *t_out = out_t;
    return state;
}

/* ---- SolveTOI (toi.py:462-865) */

/* `collideA || collideB` plus, with unity_toi, b2UnityTOIPair (toi.py:462-470) */
static int pair_rule(const Ctx* x, const W* w, int a, int b) {
    int dyn_a = w->b_type[a] == GOI_DYNAMIC, dyn_b = w->b_type[b] == GOI_DYNAMIC;
    int stock = w->b_bullet[a] || !dyn_a || w->b_bullet[b] || !dyn_b;
    if (!x->s->unity_toi) return stock;
    int rule = w->b_bullet[a] || w->b_bullet[b] || (!dyn_b ? w->b_continuous[a] : (!dyn_a ? w->b_continuous[b] : 0));
    return stock && rule;
}

/* The min-TOI search (toi.py:488-558): the contact list newest first; a contact with a cached TOI keeps it,
 * otherwise (one body active, pair rule) the two sweeps are put on the same interval by advancing the one behind
 * and b2TimeOfImpact runs; the minimum is the first in list order (the last with toi_tie_oldest). */
static int toi_search(const Ctx* x, W* w, Work* k, int* min_slot, float* min_alpha) {
    const GoiModelDesc* m = x->m;
    int n = list_order(w, k->order);
    int best = -1;
    float best_alpha = 1.0f;
    for (int i = 0; i < n; ++i) {
        int c = k->order[i];
        if (!w->t_enabled[c] || w->t_count[c] > MAX_SUB_STEPS) continue;
        float alpha;
        if (w->t_flag[c]) {
            alpha = w->t_toi[c];
        } else {
            int fa = w->c_fa[c], fb = w->c_fb[c];
            int A = m->fixture_body[fa], Bb = m->fixture_body[fb];
            int act_a = w->b_awake[A] && w->b_type[A] != GOI_STATIC;
            int act_b = w->b_awake[Bb] && w->b_type[Bb] != GOI_STATIC;
            if (!act_a && !act_b) continue;
            if (!pair_rule(x, w, A, Bb)) continue;
            float alpha0 = w->t_alpha0[A];
            if (w->t_alpha0[A] < w->t_alpha0[Bb]) { alpha0 = w->t_alpha0[Bb]; sweep_advance(w, A, alpha0); }
            else if (w->t_alpha0[Bb] < w->t_alpha0[A]) { alpha0 = w->t_alpha0[A]; sweep_advance(w, Bb, alpha0); }
            Proxy pA = proxy_of(m, fa), pB = proxy_of(m, fb);
            float beta;
            int st = time_of_impact(&pA, body_sweep(w, A), &pB, body_sweep(w, Bb), x->s->linear_slop, &beta);
            alpha = st == E_TOUCHING ? bmin(alpha0 + (1.0f - alpha0) * beta, 1.0f) : 1.0f;
            w->t_toi[c] = alpha;
            w->t_flag[c] = 1;
        }
        if (alpha < 1.0f && (x->s->toi_tie_oldest ? alpha <= best_alpha : alpha < best_alpha)) {
            best = c;
            best_alpha = alpha;
        }
    }
    *min_slot = best;
    *min_alpha = best_alpha;
    float done_alpha = 1.0f - 10.0f * EPS;
    return best >= 0 && !(done_alpha < best_alpha);
}

/* b2Island::SolveTOI (toi.py:719-799) over the island bodies k->isl_bodies[0..nb) (TOI pair first) and the contacts
 * k->corder[0..nc). */
static void toi_solve_island(const Ctx* x, W* w, Work* k, int nb, int nc, float min_alpha) {
    const GoiSettings* s = x->s;
    int A = k->isl_bodies[0], Bb = k->isl_bodies[1];
    for (int i = 0; i < nb; ++i) {
        int b = k->isl_bodies[i];
        k->cx[b] = w->b_c[2 * b]; k->cy[b] = w->b_c[2 * b + 1]; k->a[b] = w->b_a[b];
        k->vx[b] = w->b_v[2 * b]; k->vy[b] = w->b_v[2 * b + 1]; k->w[b] = w->b_w[b];
    }
    Rot q[64];
    Rot* qq = w->B <= 64 ? q : (Rot*)malloc(sizeof(Rot) * w->B);
    /* position constraints (the velocity set-up below reads the solved positions) */
    for (int i = 0; i < nc; ++i) {
        CC* c = &k->cc[i];
        /* only the fields the position solve reads; masses are the TOI pair's */
        int slot = k->corder[i];
        int fa = w->c_fa[slot], fb = w->c_fb[slot];
        c->slot = slot; c->ia = x->m->fixture_body[fa]; c->ib = x->m->fixture_body[fb];
        c->pc_count = w->c_count[slot]; c->mtype = w->c_mtype[slot];
        c->ln = getv(w->c_ln, slot); c->lp = getv(w->c_lp, slot);
        c->pl[0] = getv(w->c_pl, 2 * slot); c->pl[1] = getv(w->c_pl, 2 * slot + 1);
        c->lcA = getv(w->b_lc, c->ia); c->lcB = getv(w->b_lc, c->ib);
        c->radA = x->m->radius[fa]; c->radB = x->m->radius[fb];
    }
    for (int it = 0; it < 20; ++it) {
        float min_sep = 0.0f;
        for (int i = 0; i < nc; ++i) {
            const CC* c = &k->cc[i];
            int ta = c->ia == A || c->ia == Bb, tb = c->ib == A || c->ib == Bb;
            float mA = ta ? w->b_inv_mass[c->ia] : 0.0f, iA = ta ? w->b_inv_inertia[c->ia] : 0.0f;
            float mB = tb ? w->b_inv_mass[c->ib] : 0.0f, iB = tb ? w->b_inv_inertia[c->ib] : 0.0f;
            float ms = cs_solve_position(x, c, k, s->toi_baumgarte, mA, mB, iA, iB);
            min_sep = bmin(min_sep, ms);
        }
        if (min_sep >= -1.5f * s->linear_slop) break;
    }
    /* leap of faith: the TOI bodies' sweep start is the solved pose */
    w->b_c0[2 * A] = k->cx[A]; w->b_c0[2 * A + 1] = k->cy[A]; w->b_a0[A] = k->a[A];
    w->b_c0[2 * Bb] = k->cx[Bb]; w->b_c0[2 * Bb + 1] = k->cy[Bb]; w->b_a0[Bb] = k->a[Bb];
    for (int i = 0; i < nb; ++i) { int b = k->isl_bodies[i]; qq[b] = rot_of(k->a[b]); }
    for (int i = 0; i < nc; ++i) cs_prepare(x, w, k, &k->cc[i], k->corder[i], 0, 1.0f, qq);
    if (qq != q) free(qq);
    for (int it = 0; it < s->velocity_iterations; ++it)
        for (int i = 0; i < nc; ++i) cs_solve_velocity(&k->cc[i], k);
    float h = (1.0f - min_alpha) * x->dt;
    float max_t = s->clamps_per_second ? s->max_translation * x->dt : s->max_translation;
    float max_r = s->clamps_per_second ? s->max_rotation * x->dt : s->max_rotation;
    for (int i = 0; i < nb; ++i) {
        int b = k->isl_bodies[i];
        V2 v = v2(k->vx[b], k->vy[b]);
        float ww = k->w[b];
        V2 t = scl(h, v);
        if (dot(t, t) > max_t * max_t) {
            float ratio = max_t / len(t);
            v = v2(v.x * ratio, v.y * ratio);
        }
        float rot = h * ww;
        if (rot * rot > max_r * max_r) {
            float ratio = max_r / babs(rot);
            ww = ww * ratio;
        }
        w->b_c[2 * b] = k->cx[b] + h * v.x; w->b_c[2 * b + 1] = k->cy[b] + h * v.y; w->b_a[b] = k->a[b] + h * ww;
        w->b_v[2 * b] = v.x; w->b_v[2 * b + 1] = v.y; w->b_w[b] = ww;
        sync_transform(w, b);
    }
    /* b2Island::Report: the impulses of the velocity constraints' points */
    for (int i = 0; i < nc; ++i) {
        const CC* c = &k->cc[i];
        for (int j = 0; j < 2; ++j) {
            w->t_ni[2 * c->slot + j] = j < c->count ? c->ni[j] : 0.0f;
            w->t_ti[2 * c->slot + j] = j < c->count ? c->ti[j] : 0.0f;
        }
        w->t_solved[c->slot] = 1;
    }
}

/* One TOI event (toi.py:604-716): advance the pair to min_alpha, update its contact; if it touches, the island walk
 * over bodyA's then bodyB's contact lists (at most 32 contacts / 64 bodies), b2Island::SolveTOI, fixture sync with
 * TOI invalidation of the moved bodies' contacts, FindNewContacts. */
/* The debug trace of event ev of world wi (GoiDebug's toi_* arrays, when given): slot, alpha bits, island size
 * (contacts | bodies << 16) and the island's contact slots in walk order, -1 beyond them. */
static void record_toi_event(GoiDebug* dbg, int wi, int pitch, int ev, int slot, float alpha, const int* rows, int nc,
                             int nb) {
    if (!dbg || !dbg->toi_event_slot || ev >= GOI_DEBUG_TOI_EVENTS) return;
    size_t P = (size_t)pitch;
    union { float f; int32_t i; } bits;
    bits.f = alpha;
    dbg->toi_event_slot[ev * P + wi] = slot;
    dbg->toi_event_alpha[ev * P + wi] = bits.i;
    dbg->toi_event_island[ev * P + wi] = nc | (nb << 16);
    for (int i = 0; i < GOI_DEBUG_TOI_ROWS; ++i)
        dbg->toi_island_rows[((size_t)ev * GOI_DEBUG_TOI_ROWS + i) * P + wi] = i < nc ? rows[i] : -1;
}

static void toi_event(const Ctx* x, W* w, Work* k, int min_slot, float min_alpha, int ev, GoiDebug* dbg, int wi,
                      int pitch) {
    const GoiModelDesc* m = x->m;
    int B = w->B, C = w->C;
    int fa = w->c_fa[min_slot], fb = w->c_fb[min_slot];
    int A = m->fixture_body[fa], Bb = m->fixture_body[fb];
    backup_sweep(w, k, A);
    backup_sweep(w, k, Bb);
    body_advance(w, A, min_alpha);
    body_advance(w, Bb, min_alpha);
    Manifold mf;
    evaluate(m, fa, fb, body_xf(w, A), body_xf(w, Bb), x->s, &mf);
    if (contact_update(w, min_slot, &mf)) { wake(w, A); wake(w, Bb); }
    w->t_flag[min_slot] = 0;
    w->t_count[min_slot] += 1;
    if (!w->c_touching[min_slot]) {
        w->t_enabled[min_slot] = 0;
        restore_sweep(w, k, A);
        restore_sweep(w, k, Bb);
        record_toi_event(dbg, wi, pitch, ev, min_slot, min_alpha, k->corder, 0, 0);
        return;
    }
    w->t_enabled[min_slot] = 1;
    wake(w, A); wake(w, Bb);
    for (int b = 0; b < B; ++b) k->bflag[b] = 0;
    for (int c = 0; c < C; ++c) k->cflag[c] = 0;
    int nb = 0, nc = 0;
    k->isl_bodies[nb++] = A; k->isl_bodies[nb++] = Bb;
    k->corder[nc++] = min_slot;
    k->bflag[A] = 1; k->bflag[Bb] = 1; k->cflag[min_slot] = 1;
    int n = list_order(w, k->order);
    int pair[2] = {A, Bb};
    for (int pi = 0; pi < 2; ++pi) {
        int body = pair[pi];
        if (w->b_type[body] != GOI_DYNAMIC) continue;
        for (int i = 0; i < n; ++i) {
            int c = k->order[i];
            int ca = m->fixture_body[w->c_fa[c]], cb = m->fixture_body[w->c_fb[c]];
            if (ca != body && cb != body) continue;
            if (nb == 2 * MAX_TOI_CONTACTS || nc == MAX_TOI_CONTACTS) break;
            if (k->cflag[c]) continue;
            int other = ca == body ? cb : ca;
            if (w->b_type[other] == GOI_DYNAMIC && !w->b_bullet[body] && !w->b_bullet[other]) continue;
            if (x->s->unity_toi && !pair_rule(x, w, body, other)) continue;
            backup_sweep(w, k, other);
            if (!k->bflag[other]) body_advance(w, other, min_alpha);
            Manifold mc;
            evaluate(m, w->c_fa[c], w->c_fb[c], body_xf(w, ca), body_xf(w, cb), x->s, &mc);
            if (contact_update(w, c, &mc)) { wake(w, ca); wake(w, cb); }
            w->t_enabled[c] = 1;
            if (!w->c_touching[c]) { restore_sweep(w, k, other); continue; }
            k->cflag[c] = 1;
            k->corder[nc++] = c;
            if (k->bflag[other]) continue;
            k->bflag[other] = 1;
            if (w->b_type[other] != GOI_STATIC) wake(w, other);
            k->isl_bodies[nb++] = other;
        }
    }
    record_toi_event(dbg, wi, pitch, ev, min_slot, min_alpha, k->corder, nc, nb);
    toi_solve_island(x, w, k, nb, nc, min_alpha);
    for (int b = 0; b < B; ++b) k->moved[b] = 0;
    for (int i = 0; i < nb; ++i) {
        int b = k->isl_bodies[i];
        if (w->b_type[b] == GOI_DYNAMIC) k->moved[b] = 1;
    }
    synchronize_fixtures(x, w, k->moved);
    for (int c = 0; c < C; ++c) {
        if (w->c_pair[c] < 0) continue;
        int ca = m->fixture_body[w->c_fa[c]], cb = m->fixture_body[w->c_fb[c]];
        if (k->moved[ca] || k->moved[cb]) w->t_flag[c] = 0;
    }
    /* FindNewContacts; a slot that received a new contact starts with fresh TOI state */
    int32_t* old_pair = (int32_t*)k->stack; /* stack has room for 2B + 2C ints */
    int32_t* old_key = old_pair + C;
    for (int c = 0; c < C; ++c) { old_pair[c] = w->c_pair[c]; old_key[c] = w->c_key[c]; }
    find_new_contacts(x, w);
    for (int c = 0; c < C; ++c) {
        if (w->c_pair[c] >= 0 && (old_pair[c] < 0 || old_key[c] != w->c_key[c])) {
            w->t_count[c] = 0; w->t_flag[c] = 0; w->t_enabled[c] = 1;
        }
    }
}

/* Returns 1 when the world stopped at max_events with another event pending (toi.py:838-842). */
static int solve_toi(const Ctx* x, W* w, Work* k, float dt, GoiDebug* dbg, int wi, int pitch) {
    const GoiModelDesc* m = x->m;
    int B = w->B, C = w->C;
    if (C == 0 || m->P == 0) return 0;
    if (x->s->unity_toi && m->toi_bodies) {
        int any = 0;
        for (int b = 0; b < B; ++b) any |= m->toi_bodies[b];
        if (!any) return 0;
    }
    for (int b = 0; b < B; ++b) w->t_alpha0[b] = 0.0f;
    for (int c = 0; c < C; ++c) {
        w->t_count[c] = 0; w->t_toi[c] = 1.0f; w->t_flag[c] = 0; w->t_enabled[c] = 1; w->t_solved[c] = 0;
        w->t_ni[2 * c] = 0.0f; w->t_ni[2 * c + 1] = 0.0f; w->t_ti[2 * c] = 0.0f; w->t_ti[2 * c + 1] = 0.0f;
    }
    *w->t_events = 0;
    if (!(dt > 0.0f)) return 0;
    int max_events = x->s->max_events >= 0 ? x->s->max_events : C * (MAX_SUB_STEPS + 1) + 8;
    int slot;
    float alpha;
    int found = toi_search(x, w, k, &slot, &alpha);
    while (found && *w->t_events < max_events) {
        toi_event(x, w, k, slot, alpha, *w->t_events, dbg, wi, pitch);
        *w->t_events += 1;
        found = toi_search(x, w, k, &slot, &alpha);
    }
    return found;
}

/* ------------------------------------------------------------------------------------------------ step (step.py:28-47) */

static void step_world(const Ctx* x, W* w, Work* k, GoiDebug* dbg, int wi, int pitch) {
    float dt = x->dt;
    int overflow0 = *w->overflow, capped = 0;
    if (*w->new_fixture) find_new_contacts(x, w);
    *w->new_fixture = 0;
    float inv_dt = dt > 0.0f ? 1.0f / dt : 0.0f;
    float dt_ratio = *w->inv_dt0 * dt;
    collide(x, w, k->order);
    solve(x, w, k, dt, dt_ratio, dbg, wi, pitch);
    if (dbg && dbg->toi_event_slot) /* the blank trace; SolveTOI's events overwrite their entries */
        for (int e = 0; e < GOI_DEBUG_TOI_EVENTS; ++e) record_toi_event(dbg, wi, pitch, e, -1, 0.0f, k->corder, 0, 0);
    if (x->s->continuous_physics) capped = solve_toi(x, w, k, dt, dbg, wi, pitch);
    if (dt > 0.0f) *w->inv_dt0 = inv_dt;
    if (x->s->auto_clear_forces) {
        for (int b = 0; b < w->B; ++b) { w->b_force[2 * b] = 0.0f; w->b_force[2 * b + 1] = 0.0f; w->b_torque[b] = 0.0f; }
    }
    if (dbg && dbg->status) { /* the step's failure counters as one word (GOI_STATUS_*) */
        int st = *w->overflow != overflow0 ? GOI_STATUS_OVERFLOW : 0, finite = 1;
        for (int b = 0; b < w->B; ++b)
            finite = finite && isfinite(w->b_c[2 * b]) && isfinite(w->b_c[2 * b + 1]) && isfinite(w->b_a[b]) &&
                     isfinite(w->b_v[2 * b]) && isfinite(w->b_v[2 * b + 1]) && isfinite(w->b_w[b]);
        if (!finite) st |= GOI_STATUS_NONFINITE;
        if (capped) st |= GOI_STATUS_TOI_CAPPED;
        if (x->s->continuous_physics && !(dt > 0.0f)) st |= GOI_STATUS_TOI_SKIPPED;
        dbg->status[wi] = st;
    }
}

/* ------------------------------------------------------------------------------------------------ batch entry */

/* leaves: GOI_NUM_LEAVES host pointers to batch-major contiguous arrays [N, inner...] */
static void bind_world(W* w, void* const* lv, int B, int C, int R, int J, size_t wi) {
    w->B = B; w->C = C; w->R = R; w->J = J;
#define P(T, L, n) ((T*)lv[L] + wi * (size_t)(n))
    w->b_type = P(int32_t, GOI_B_TYPE, B); w->b_active = P(uint8_t, GOI_B_ACTIVE, B);
    w->b_awake = P(uint8_t, GOI_B_AWAKE, B); w->b_allow_sleep = P(uint8_t, GOI_B_ALLOW_SLEEP, B);
    w->b_bullet = P(uint8_t, GOI_B_BULLET, B); w->b_continuous = P(uint8_t, GOI_B_CONTINUOUS, B);
    w->b_sleep_time = P(float, GOI_B_SLEEP_TIME, B); w->b_xf_p = P(float, GOI_B_XF_P, 2 * B);
    w->b_xf_q = P(float, GOI_B_XF_Q, 2 * B); w->b_lc = P(float, GOI_B_LOCAL_CENTER, 2 * B);
    w->b_c0 = P(float, GOI_B_C0, 2 * B); w->b_c = P(float, GOI_B_C, 2 * B);
    w->b_a0 = P(float, GOI_B_A0, B); w->b_a = P(float, GOI_B_A, B); w->b_v = P(float, GOI_B_V, 2 * B);
    w->b_w = P(float, GOI_B_W, B); w->b_force = P(float, GOI_B_FORCE, 2 * B); w->b_torque = P(float, GOI_B_TORQUE, B);
    w->b_mass = P(float, GOI_B_MASS, B); w->b_inv_mass = P(float, GOI_B_INV_MASS, B);
    w->b_inertia = P(float, GOI_B_INERTIA, B); w->b_inv_inertia = P(float, GOI_B_INV_INERTIA, B);
    w->b_ld = P(float, GOI_B_LINEAR_DAMPING, B); w->b_ad = P(float, GOI_B_ANGULAR_DAMPING, B);
    w->b_gs = P(float, GOI_B_GRAVITY_SCALE, B);
    w->f_friction = P(float, GOI_F_FRICTION, R); w->f_restitution = P(float, GOI_F_RESTITUTION, R);
    w->f_fat = P(float, GOI_F_FAT, 4 * R);
    w->j_enable_motor = P(uint8_t, GOI_J_ENABLE_MOTOR, J); w->j_motor_speed = P(float, GOI_J_MOTOR_SPEED, J);
    w->j_max_motor = P(float, GOI_J_MAX_MOTOR, J); w->j_enable_limit = P(uint8_t, GOI_J_ENABLE_LIMIT, J);
    w->j_lower = P(float, GOI_J_LOWER, J); w->j_upper = P(float, GOI_J_UPPER, J);
    w->j_frequency = P(float, GOI_J_FREQUENCY, J); w->j_damping = P(float, GOI_J_DAMPING, J);
    w->j_impulse = P(float, GOI_J_IMPULSE, 3 * J); w->j_motor_impulse = P(float, GOI_J_MOTOR_IMPULSE, J);
    w->j_limit_state = P(int32_t, GOI_J_LIMIT_STATE, J); w->j_lower_impulse = P(float, GOI_J_LOWER_IMPULSE, J);
    w->j_upper_impulse = P(float, GOI_J_UPPER_IMPULSE, J);
    w->c_pair = P(int32_t, GOI_C_PAIR, C); w->c_fa = P(int32_t, GOI_C_FA, C); w->c_fb = P(int32_t, GOI_C_FB, C);
    w->c_key = P(int32_t, GOI_C_KEY, C); w->c_touching = P(uint8_t, GOI_C_TOUCHING, C);
    w->c_mtype = P(int32_t, GOI_C_MTYPE, C); w->c_count = P(int32_t, GOI_C_COUNT, C);
    w->c_ln = P(float, GOI_C_LOCAL_NORMAL, 2 * C); w->c_lp = P(float, GOI_C_LOCAL_POINT, 2 * C);
    w->c_pl = P(float, GOI_C_POINT_LOCAL, 4 * C); w->c_pid = P(int32_t, GOI_C_POINT_ID, 2 * C);
    w->c_ni = P(float, GOI_C_NORMAL_IMPULSE, 2 * C); w->c_ti = P(float, GOI_C_TANGENT_IMPULSE, 2 * C);
    w->c_friction = P(float, GOI_C_FRICTION, C); w->c_restitution = P(float, GOI_C_RESTITUTION, C);
    w->c_tangent_speed = P(float, GOI_C_TANGENT_SPEED, C);
    w->gravity = P(float, GOI_S_GRAVITY, 2); w->inv_dt0 = P(float, GOI_S_INV_DT0, 1);
    w->next_key = P(int32_t, GOI_S_NEXT_KEY, 1); w->new_fixture = P(uint8_t, GOI_S_NEW_FIXTURE, 1);
    w->overflow = P(int32_t, GOI_S_OVERFLOW, 1);
    w->t_alpha0 = P(float, GOI_T_ALPHA0, B); w->t_count = P(int32_t, GOI_T_COUNT, C);
    w->t_toi = P(float, GOI_T_TOI, C); w->t_flag = P(uint8_t, GOI_T_FLAG, C);
    w->t_enabled = P(uint8_t, GOI_T_ENABLED, C); w->t_solved = P(uint8_t, GOI_T_SOLVED, C);
    w->t_ni = P(float, GOI_T_NORMAL_IMPULSE, 2 * C); w->t_ti = P(float, GOI_T_TANGENT_IMPULSE, 2 * C);
    w->t_events = P(int32_t, GOI_T_EVENTS, 1);
#undef P
}

/* One step of n worlds (batch-major host arrays), n_threads OpenMP threads (<= 0: all). Debug outputs, when given,
 * are worlds-minor with pitch n. Returns 0. */
int oracle_step(const GoiModelDesc* m, void* const* leaves, int32_t n, int32_t B, int32_t C, int32_t R, int32_t J,
                const GoiSettings* s, float dt, int32_t n_threads, GoiDebug* dbg) {
    Ctx x = {m, s, dt, m->fixture_slot != NULL && R != m->F};
#ifdef _OPENMP
    int nt = n_threads > 0 ? n_threads : omp_get_max_threads();
#pragma omp parallel num_threads(nt)
#endif
    {
        Work k;
        work_init(&k, B, C, J);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 16)
#endif
        for (int wi = 0; wi < n; ++wi) {
            W w;
            bind_world(&w, leaves, B, C, R, J, (size_t)wi);
            step_world(&x, &w, &k, dbg, wi, n);
        }
        work_free(&k);
    }
    (void)n_threads;
    return 0;
}

/* Broadphase + narrowphase only (config 2): start-of-step FindNewContacts where new_fixture, then Collide. */
int oracle_collide(const GoiModelDesc* m, void* const* leaves, int32_t n, int32_t B, int32_t C, int32_t R, int32_t J,
                   const GoiSettings* s, int32_t n_threads) {
    Ctx x = {m, s, 0.0f, m->fixture_slot != NULL && R != m->F};
#ifdef _OPENMP
    int nt = n_threads > 0 ? n_threads : omp_get_max_threads();
#pragma omp parallel num_threads(nt)
#endif
    {
        Work k;
        work_init(&k, B, C, J);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 16)
#endif
        for (int wi = 0; wi < n; ++wi) {
            W w;
            bind_world(&w, leaves, B, C, R, J, (size_t)wi);
            if (*w.new_fixture) find_new_contacts(&x, &w);
            *w.new_fixture = 0;
            collide(&x, &w, k.order);
        }
        work_free(&k);
    }
    (void)n_threads;
    return 0;
}

/* Test hooks: the narrowphase, the GJK distance and b2TimeOfImpact on one pair, for the brute-force checks. */
int oracle_evaluate(const GoiModelDesc* m, int fa, int fb, const float* xfa, const float* xfb,
                    const GoiSettings* settings, int32_t* mtype_count, float* geo, int32_t* ids) {
    Xf a, b;
    a.p = v2(xfa[0], xfa[1]); a.q.c = xfa[2]; a.q.s = xfa[3];
    b.p = v2(xfb[0], xfb[1]); b.q.c = xfb[2]; b.q.s = xfb[3];
    Manifold mf;
    memset(&mf, 0, sizeof(mf));
    evaluate(m, fa, fb, a, b, settings, &mf);
    mtype_count[0] = mf.mtype; mtype_count[1] = mf.count;
    geo[0] = mf.ln.x; geo[1] = mf.ln.y; geo[2] = mf.lp.x; geo[3] = mf.lp.y;
    geo[4] = mf.pl[0].x; geo[5] = mf.pl[0].y; geo[6] = mf.pl[1].x; geo[7] = mf.pl[1].y;
    ids[0] = mf.id[0]; ids[1] = mf.id[1];
    return 0;
}

float oracle_distance(const GoiModelDesc* m, int fa, int fb, const float* xfa, const float* xfb) {
    Xf a, b;
    a.p = v2(xfa[0], xfa[1]); a.q.c = xfa[2]; a.q.s = xfa[3];
    b.p = v2(xfb[0], xfb[1]); b.q.c = xfb[2]; b.q.s = xfb[3];
    Proxy pA = proxy_of(m, fa), pB = proxy_of(m, fb);
    Cache cache;
    memset(&cache, 0, sizeof(cache));
    return distance(&cache, &pA, a, &pB, b);
}

/* sweeps: lcx lcy c0x c0y cx cy a0 a for A then B; returns the b2TOIOutput state, *t the time */
int oracle_toi(const GoiModelDesc* m, int fa, int fb, const float* swa, const float* swb, float linear_slop,
               float* t) {
    Sweep a, b;
    a.lc = v2(swa[0], swa[1]); a.c0 = v2(swa[2], swa[3]); a.c = v2(swa[4], swa[5]); a.a0 = swa[6]; a.a = swa[7];
    b.lc = v2(swb[0], swb[1]); b.c0 = v2(swb[2], swb[3]); b.c = v2(swb[4], swb[5]); b.a0 = swb[6]; b.a = swb[7];
    Proxy pA = proxy_of(m, fa), pB = proxy_of(m, fb);
    return time_of_impact(&pA, a, &pB, b, linear_slop, t);
}

void oracle_sincos(const float* x, float* s, float* c, int32_t n) {
    for (int i = 0; i < n; ++i) { Rot q = rot_of(x[i]); s[i] = q.s; c[i] = q.c; }
}
