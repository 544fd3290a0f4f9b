// b2_solver.hpp - b2World::Solve on the device (goi_jax/box2d/step.py:73-251, island.py, contact_solver.py,
// joints.py): the island search, velocity integration, contact and joint constraint set-up, warm start, the
// Gauss-Seidel velocity sweeps, position integration with the per-step clamps, position sweeps with per-island
// early exit, transform sync, sleeping, fixture sync and FindNewContacts.
//
// Storage: the solver's body arrays (v, w, c, a per body) live in LDS as [field][body][world] so each world's random
// body index hits its own bank; the prepared constraint rows live in HBM scratch tiles, one per block
// ([row][field][world of the block]: a row's fields for the block's worlds are contiguous).
#pragma once

#include "b2_pairs.hpp"

namespace goi {

constexpr int kMaxB = 64;  // bodies per world the kernels handle (body sets are 64-bit masks)
constexpr int kMaxJ = 64;  // joints per world (joint sets are 64-bit masks)

// Per-lane view of the solver body arrays in LDS.
struct Bodies {
    float* s;  // LDS base + the world's index in the block
    int B;
    int st;    // worlds per block
    GOI_D float& at(int field, int b) const { return s[(field * B + b) * st]; }
    GOI_D float& vx(int b) const { return at(0, b); }
    GOI_D float& vy(int b) const { return at(1, b); }
    GOI_D float& w(int b) const { return at(2, b); }
    GOI_D float& cx(int b) const { return at(3, b); }
    GOI_D float& cy(int b) const { return at(4, b); }
    GOI_D float& a(int b) const { return at(5, b); }
    GOI_D V2 v(int b) const { return mk(vx(b), vy(b)); }
    GOI_D V2 c(int b) const { return mk(cx(b), cy(b)); }
    GOI_D void set_v(int b, V2 x, float ww) const { vx(b) = x.x; vy(b) = x.y; w(b) = ww; }
    GOI_D void set_c(int b, V2 x, float aa) const { cx(b) = x.x; cy(b) = x.y; a(b) = aa; }
};

// One lane's view of the bodies while the lanes of a world's group solve its islands side by side, each lane its own
// island (island.py:3-7: islands share no body but static ones). The island's bodies (`own`) are read and written;
// another body that a row touches, a static one, is only read: Box2D's update of it (x - 0 * P) leaves it unchanged
// unless an impulse is not finite or the value is -0, and a write that would change it raises the world's flag
// (`changed`) instead, after which the world solves its islands again one after another. Without such a write, every
// row saw the values it sees in Box2D's order, so the results are the same floats.
struct IslandBodies {
    Bodies bd;
    unsigned long long own;
    int* changed;
    GOI_D V2 v(int b) const { return bd.v(b); }
    GOI_D float w(int b) const { return bd.w(b); }
    GOI_D V2 c(int b) const { return bd.c(b); }
    GOI_D float a(int b) const { return bd.a(b); }
    GOI_D static bool differ(float x, float y) { return __float_as_uint(x) != __float_as_uint(y); }
    GOI_D void set_v(int b, V2 x, float ww) const {
        if ((own >> b) & 1ull) bd.set_v(b, x, ww);
        else if (differ(x.x, bd.vx(b)) || differ(x.y, bd.vy(b)) || differ(ww, bd.w(b))) *changed = 1;
    }
    GOI_D void set_c(int b, V2 x, float aa) const {
        if ((own >> b) & 1ull) bd.set_c(b, x, aa);
        else if (differ(x.x, bd.cx(b)) || differ(x.y, bd.cy(b)) || differ(aa, bd.a(b))) *changed = 1;
    }
};

GOI_D V2 rel_vel(V2 vB, float wB, V2 rB, V2 vA, float wA, V2 rA) {
    return ((vB + cross(wB, rB)) - vA) - cross(wA, rA);
}

// ---------------------------------------------------------------- islands (island.py:41-140)

// Solve order and island ids, stored in the world's LDS workspace.
struct Islands {
    const World& W;
    int nc, nj, n;
    GOI_D int& corder(int i) const { return W.corder(i); }
    GOI_D int& jorder(int i) const { return W.jorder(i); }
    GOI_D int& body_island(int b) const { return W.bisl(b); }
    GOI_D int& contact_island(int c) const { return W.cisl(c); }
    GOI_D int& joint_island(int j) const { return W.jisl(j); }
    // island k's contact rows [c0, c1) and joint rows [j0, j1) of the solve order (find_islands notes where each
    // island's rows start)
    GOI_D void rows_of(int k, int& c0, int& c1, int& j0, int& j1) const {
        const int s0 = W.ibuf(k), s1 = k + 1 < n ? W.ibuf(k + 1) : (nc | (nj << 16));
        c0 = s0 & 0xffff; j0 = s0 >> 16;
        c1 = s1 & 0xffff; j1 = s1 >> 16;
    }
    GOI_D unsigned long long bodies_of(int k) const {
        unsigned long long own = 0ull;
        for (int b = 0; b < W.B; ++b)
            if (body_island(b) == k) own |= 1ull << b;
        return own;
    }
};

// b2World::Solve's depth-first search: seeds newest body first; popping b wakes it, walks b's touching contacts
// newest first (each joins the island and pushes its unvisited non-static other body), then b's joints newest
// first (joints to inactive bodies skipped). Contacts and joints append to one solve order across islands.
GOI_D void find_islands(const DModel& m, const World& W, Islands& I) {
    const int n = list_order(W);
    unsigned long long bflag = 0ull, jflag = 0ull;
    for (int b = W.sub; b < W.B; b += W.G) I.body_island(b) = -1;  // split over the lane group
    for (int c = W.sub; c < W.C; c += W.G) I.contact_island(c) = -1;  // also the "in an island" flag of each contact
    for (int j = W.sub; j < W.J; j += W.G) I.joint_island(j) = -1;
    group_sync();
    int nisl = 0, nc = 0, nj = 0;
    for (int seed = W.B - 1; seed >= 0; --seed) {
        if ((bflag >> seed) & 1ull) continue;
        if (!W.awake(seed) || !W.active(seed) || W.is_static(seed)) continue;
        const int isl = nisl++;
        if (m.island_lanes) W.ibuf(isl) = nc | (nj << 16);  // the island's first rows (nc <= 256, nj <= 64)
        int sp = 0;
        W.stack(sp++) = seed;
        bflag |= 1ull << seed;
        while (sp > 0) {
            const int b = W.stack(--sp);
            I.body_island(b) = isl;
            W.wake(b);
            // b's touching contacts not yet in an island, newest first, a chunk of the list at a time (the walk
            // marks only the contact it visits, so the mask of the chunk's others stays exact)
            for (int q0 = 0; q0 < n; q0 += 64) {
                const unsigned long long hits = list_mask(W, q0, n, [&](int c) {
                    return (W.ba(c) == b || W.bb(c) == b) && I.contact_island(c) < 0 && W.touching(c);
                });
                for (unsigned long long left = hits; left; left &= left - 1) {
                    const int c = W.order(q0 + __builtin_ctzll(left));
                    const int ba = W.ba(c), bb = W.bb(c);
                    I.corder(nc++) = c;
                    I.contact_island(c) = isl;
                    const int other = ba == b ? bb : ba;
                    if (((bflag >> other) & 1ull) || W.is_static(other)) continue;
                    W.stack(sp++) = other;
                    bflag |= 1ull << other;
                }
                group_sync();
            }
            for (int j = W.J - 1; j >= 0; --j) {
                const int ja = m.joint[j].a, jb = m.joint[j].b;
                if (ja != b && jb != b) continue;
                if ((jflag >> j) & 1ull) continue;
                const int other = ja == b ? jb : ja;
                if (!W.active(other)) continue;
                I.jorder(nj++) = j;
                jflag |= 1ull << j;
                I.joint_island(j) = isl;
                if (((bflag >> other) & 1ull) || W.is_static(other)) continue;
                W.stack(sp++) = other;
                bflag |= 1ull << other;
            }
        }
    }
    I.nc = nc;
    I.nj = nj;
    I.n = nisl;
}

// ---------------------------------------------------------------- contact solver (contact_solver.py)

// b2ContactSolver constructor + InitializeVelocityConstraints for contact slot `slot` into row i
// (contact_solver.py:32-147). Body positions/velocities from the LDS arrays; qA/qB the bodies' rotations.
GOI_D void cs_prepare(const DModel& m, const World& W, const Bodies& bd, const Rows& R, int i, int slot, bool warm,
                      float dt_ratio, Rot qA, Rot qB, float velocity_threshold) {
    const int fa = W.fa(slot), fb = W.fb(slot);
    const int ia = W.ba(slot), ib = W.bb(slot);
    const float mA = W.f(GOI_B_INV_MASS, ia), mB = W.f(GOI_B_INV_MASS, ib);
    const float iA = W.f(GOI_B_INV_INERTIA, ia), iB = W.f(GOI_B_INV_INERTIA, ib);
    const V2 lcA = W.v2(GOI_B_LOCAL_CENTER, ia), lcB = W.v2(GOI_B_LOCAL_CENTER, ib);
    const float radA = m.fix[fa].radius, radB = m.fix[fb].radius;
    const int mtype = W.i32(GOI_C_MTYPE, slot);
    const int cnt = W.ccount(slot);
    const V2 ln = W.v2(GOI_C_LOCAL_NORMAL, slot), lp = W.v2(GOI_C_LOCAL_POINT, slot);
    const V2 pl0 = W.v2(GOI_C_POINT_LOCAL, 2 * slot), pl1 = W.v2(GOI_C_POINT_LOCAL, 2 * slot + 1);
    R.seti(i, CF_SLOT, slot); R.seti(i, CF_IA, ia); R.seti(i, CF_IB, ib);
    R.seti(i, CF_PC_COUNT, cnt); R.seti(i, CF_MTYPE, mtype);
    R.setf(i, CF_MA, mA); R.setf(i, CF_MB, mB); R.setf(i, CF_IIA, iA); R.setf(i, CF_IIB, iB);
    R.set2(i, CF_LN, ln); R.set2(i, CF_LP, lp); R.set2(i, CF_PL0, pl0); R.set2(i, CF_PL1, pl1);
    R.set2(i, CF_LCA, lcA); R.set2(i, CF_LCB, lcB); R.setf(i, CF_RADA, radA); R.setf(i, CF_RADB, radB);
    R.setf(i, CF_NI0, warm ? dt_ratio * W.f(GOI_C_NORMAL_IMPULSE, 2 * slot) : 0.0f);
    R.setf(i, CF_NI1, warm ? dt_ratio * W.f(GOI_C_NORMAL_IMPULSE, 2 * slot + 1) : 0.0f);
    R.setf(i, CF_TI0, warm ? dt_ratio * W.f(GOI_C_TANGENT_IMPULSE, 2 * slot) : 0.0f);
    R.setf(i, CF_TI1, warm ? dt_ratio * W.f(GOI_C_TANGENT_IMPULSE, 2 * slot + 1) : 0.0f);
    R.setf(i, CF_FRICTION, W.f(GOI_C_FRICTION, slot));
    R.setf(i, CF_TSPEED, W.f(GOI_C_TANGENT_SPEED, slot));
    const float restitution = W.f(GOI_C_RESTITUTION, slot);
    const V2 cA = bd.c(ia), cB = bd.c(ib);
    const V2 vA = bd.v(ia), vB = bd.v(ib);
    const float wA = bd.w(ia), wB = bd.w(ib);
    Xf xfA, xfB;
    xfA.q = qA; xfB.q = qB;
    xfA.p = cA - mul(qA, lcA);
    xfB.p = cB - mul(qB, lcB);
    // b2WorldManifold::Initialize
    V2 n = mk(1.0f, 0.0f), p0, p1;
    if (mtype == kCircles) {
        const V2 pA = mul(xfA, lp), pB = mul(xfB, pl0);
        const V2 d = pB - pA;
        if (dot(d, d) > kEps * kEps) {
            n = d;
            normalize(n);
        }
        const V2 ccA = pA + radA * n, ccB = pB - radB * n;
        p0 = 0.5f * (ccA + ccB);
        p1 = p0;
    } else {
        // face A or face B: the reference face's side (x1, r1) and the incident side (x2, r2) swap; the two
        // clip-point sums are the same float additions in either order (addition commutes exactly), so one path
        // serves both
        const bool fa = mtype == kFaceA;
        const Xf& x1 = fa ? xfA : xfB;
        const Xf& x2 = fa ? xfB : xfA;
        const float r1 = fa ? radA : radB, r2 = fa ? radB : radA;
        n = mul(x1.q, ln);
        const V2 pp = mul(x1, lp);
        const V2 q0 = mul(x2, pl0), q1 = mul(x2, pl1);
        p0 = 0.5f * ((q0 + (r1 - dot(q0 - pp, n)) * n) + (q0 - r2 * n));
        p1 = 0.5f * ((q1 + (r1 - dot(q1 - pp, n)) * n) + (q1 - r2 * n));
        if (!fa) n = -n;
    }
    R.set2(i, CF_NX, n);
    const V2 t = cross(n, 1.0f);
    const V2 pts[2] = {p0, p1};
    float rnA2[2], rnB2[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const V2 rA = pts[j] - cA, rB = pts[j] - cB;
        R.set2(i, CF_RA0 + 2 * j, rA);
        R.set2(i, CF_RB0 + 2 * j, rB);
        const float rnA = cross(rA, n), rnB = cross(rB, n);
        rnA2[j] = rnA;
        rnB2[j] = rnB;
        const float kn = ((mA + mB) + iA * rnA * rnA) + iB * rnB * rnB;
        const float rtA = cross(rA, t), rtB = cross(rB, t);
        const float kt = ((mA + mB) + iA * rtA * rtA) + iB * rtB * rtB;
        R.setf(i, CF_NMASS0 + j, kn > 0.0f ? 1.0f / kn : 0.0f);
        R.setf(i, CF_TMASS0 + j, kt > 0.0f ? 1.0f / kt : 0.0f);
        const float vrel = dot(n, rel_vel(vB, wB, rB, vA, wA, rA));
        R.setf(i, CF_BIAS0 + j, vrel < -velocity_threshold ? -restitution * vrel : 0.0f);
    }
    int vcount = cnt;
    float K0 = 0.0f, K1 = 0.0f, K2 = 0.0f, K3 = 0.0f, N0 = 0.0f, N1 = 0.0f, N2 = 0.0f, N3 = 0.0f;
    if (cnt == 2) {
        const float k11 = ((mA + mB) + iA * rnA2[0] * rnA2[0]) + iB * rnB2[0] * rnB2[0];
        const float k22 = ((mA + mB) + iA * rnA2[1] * rnA2[1]) + iB * rnB2[1] * rnB2[1];
        const float k12 = ((mA + mB) + iA * rnA2[0] * rnA2[1]) + iB * rnB2[0] * rnB2[1];
        if (k11 * k11 < 1000.0f * (k11 * k22 - k12 * k12)) {
            float det = k11 * k22 - k12 * k12;
            if (det != 0.0f) det = 1.0f / det;
            K0 = k11; K1 = k12; K2 = k12; K3 = k22;
            N0 = det * k22; N1 = -det * k12; N2 = -det * k12; N3 = det * k11;
        } else {
            vcount = 1;
        }
    }
    R.seti(i, CF_COUNT, vcount);
    R.setf(i, CF_K0, K0); R.setf(i, CF_K1, K1); R.setf(i, CF_K2, K2); R.setf(i, CF_K3, K3);
    R.setf(i, CF_NM0, N0); R.setf(i, CF_NM1, N1); R.setf(i, CF_NM2, N2); R.setf(i, CF_NM3, N3);
}

template <class BD>
GOI_D void cs_warm_start(const BD& bd, const Rows& R, int i) {
    const int ia = R.geti(i, CF_IA), ib = R.geti(i, CF_IB), cnt = R.geti(i, CF_COUNT);
    const float mA = R.getf(i, CF_MA), mB = R.getf(i, CF_MB), iA = R.getf(i, CF_IIA), iB = R.getf(i, CF_IIB);
    const V2 n = R.get2(i, CF_NX), t = cross(n, 1.0f);
    V2 vA = bd.v(ia), vB = bd.v(ib);
    float wA = bd.w(ia), wB = bd.w(ib);
    for (int j = 0; j < cnt; ++j) {
        const V2 P = R.getf(i, CF_NI0 + j) * n + R.getf(i, CF_TI0 + j) * t;
        wA = wA - iA * cross(R.get2(i, CF_RA0 + 2 * j), P);
        vA = vA - mA * P;
        wB = wB + iB * cross(R.get2(i, CF_RB0 + 2 * j), P);
        vB = vB + mB * P;
    }
    bd.set_v(ia, vA, wA);
    bd.set_v(ib, vB, wB);
}

// b2ContactSolver::SolveVelocityConstraints for row i (contact_solver.py:194-279)
// A contact row's velocity-solver fields, loaded in one batch (every field, whether or not the row's point count
// uses it) so that the next row can be fetched while the current one is solved.
struct VRow {
    int ia, ib, cnt;
    float mA, mB, iA, iB, friction, tspeed, tm0, tm1, nm0, nm1, b0, b1, K0, K1, K2, K3, N0, N1, N2, N3;
    V2 n, rA0, rA1, rB0, rB1;
    float ni0, ni1, ti0, ti1;
};

GOI_D VRow load_vrow(const Rows& R, int i) {
    VRow r;
    r.ia = R.geti(i, CF_IA); r.ib = R.geti(i, CF_IB); r.cnt = R.geti(i, CF_COUNT);
    r.mA = R.getf(i, CF_MA); r.mB = R.getf(i, CF_MB); r.iA = R.getf(i, CF_IIA); r.iB = R.getf(i, CF_IIB);
    r.n = R.get2(i, CF_NX); r.friction = R.getf(i, CF_FRICTION); r.tspeed = R.getf(i, CF_TSPEED);
    r.rA0 = R.get2(i, CF_RA0); r.rA1 = R.get2(i, CF_RA1); r.rB0 = R.get2(i, CF_RB0); r.rB1 = R.get2(i, CF_RB1);
    r.tm0 = R.getf(i, CF_TMASS0); r.tm1 = R.getf(i, CF_TMASS1);
    r.nm0 = R.getf(i, CF_NMASS0); r.nm1 = R.getf(i, CF_NMASS1);
    r.b0 = R.getf(i, CF_BIAS0); r.b1 = R.getf(i, CF_BIAS1);
    r.K0 = R.getf(i, CF_K0); r.K1 = R.getf(i, CF_K1); r.K2 = R.getf(i, CF_K2); r.K3 = R.getf(i, CF_K3);
    r.N0 = R.getf(i, CF_NM0); r.N1 = R.getf(i, CF_NM1); r.N2 = R.getf(i, CF_NM2); r.N3 = R.getf(i, CF_NM3);
    r.ni0 = R.getf(i, CF_NI0); r.ni1 = R.getf(i, CF_NI1); r.ti0 = R.getf(i, CF_TI0); r.ti1 = R.getf(i, CF_TI1);
    return r;
}

// b2ContactSolver::SolveVelocityConstraints for one row (contact_solver.py:194-290): tangent rows first, then the
// normal row or the 2-point block solver's four cases. Updates the row's impulses in r and the bodies in LDS.
template <class BD>
GOI_D void solve_vrow(const BD& bd, VRow& r) {
    const V2 n = r.n, t = cross(n, 1.0f);
    const float mA = r.mA, mB = r.mB, iA = r.iA, iB = r.iB;
    const V2 rA0 = r.rA0, rA1 = r.rA1, rB0 = r.rB0, rB1 = r.rB1;
    float ni0 = r.ni0, ni1 = r.ni1, ti0 = r.ti0, ti1 = r.ti1;
    V2 vA = bd.v(r.ia), vB = bd.v(r.ib);
    float wA = bd.w(r.ia), wB = bd.w(r.ib);
    // tangent constraints first
    if (r.cnt > 0) {
        const float vt = dot(rel_vel(vB, wB, rB0, vA, wA, rA0), t) - r.tspeed;
        float lam = r.tm0 * (-vt);
        const float maxf = r.friction * ni0;
        const float nw = bclamp(ti0 + lam, -maxf, maxf);
        lam = nw - ti0;
        ti0 = nw;
        const V2 P = lam * t;
        vA = vA - mA * P; wA = wA - iA * cross(rA0, P);
        vB = vB + mB * P; wB = wB + iB * cross(rB0, P);
    }
    if (r.cnt > 1) {
        const float vt = dot(rel_vel(vB, wB, rB1, vA, wA, rA1), t) - r.tspeed;
        float lam = r.tm1 * (-vt);
        const float maxf = r.friction * ni1;
        const float nw = bclamp(ti1 + lam, -maxf, maxf);
        lam = nw - ti1;
        ti1 = nw;
        const V2 P = lam * t;
        vA = vA - mA * P; wA = wA - iA * cross(rA1, P);
        vB = vB + mB * P; wB = wB + iB * cross(rB1, P);
    }
    if (r.cnt == 1) {
        const float vn = dot(rel_vel(vB, wB, rB0, vA, wA, rA0), n);
        float lam = -r.nm0 * (vn - r.b0);
        const float nw = bmax(ni0 + lam, 0.0f);
        lam = nw - ni0;
        ni0 = nw;
        const V2 P = lam * n;
        vA = vA - mA * P; wA = wA - iA * cross(rA0, P);
        vB = vB + mB * P; wB = wB + iB * cross(rB0, P);
    } else if (r.cnt == 2) {
        const float K0 = r.K0, K1 = r.K1, K2 = r.K2, K3 = r.K3;
        const float ax = ni0, ay = ni1;
        const float vn1 = dot(rel_vel(vB, wB, rB0, vA, wA, rA0), n);
        const float vn2 = dot(rel_vel(vB, wB, rB1, vA, wA, rA1), n);
        float bx = vn1 - r.b0, by = vn2 - r.b1;
        bx = bx - (K0 * ax + K2 * ay);
        by = by - (K1 * ax + K3 * ay);
        float xx = -(r.N0 * bx + r.N2 * by);
        float xy = -(r.N1 * bx + r.N3 * by);
        bool ok = xx >= 0.0f && xy >= 0.0f;
        if (!ok) {
            xx = -r.nm0 * bx;
            xy = 0.0f;
            ok = xx >= 0.0f && K1 * xx + by >= 0.0f;
        }
        if (!ok) {
            xx = 0.0f;
            xy = -r.nm1 * by;
            ok = xy >= 0.0f && K2 * xy + bx >= 0.0f;
        }
        if (!ok) {
            xx = 0.0f;
            xy = 0.0f;
            ok = bx >= 0.0f && by >= 0.0f;
        }
        if (ok) {
            const float dx = xx - ax, dy = xy - ay;
            const V2 P1 = dx * n, P2 = dy * n;
            vA = vA - mA * (P1 + P2);
            wA = wA - iA * (cross(rA0, P1) + cross(rA1, P2));
            vB = vB + mB * (P1 + P2);
            wB = wB + iB * (cross(rB0, P1) + cross(rB1, P2));
            ni0 = xx;
            ni1 = xy;
        }
    }
    r.ni0 = ni0; r.ni1 = ni1; r.ti0 = ti0; r.ti1 = ti1;
    bd.set_v(r.ia, vA, wA);
    bd.set_v(r.ib, vB, wB);
}

// ---- TOI velocity passes with one moving body
//
// b2Island::SolveTOI's velocity passes (toi.py:762-772) give every island body its mass. When one body M of the
// island has mass and every row pairs it with a body without mass (static or kinematic: mass and inertia 0), that
// side's updates v - 0 * P and w - 0 * cross(r, P) are identities when its v and w are finite and not -0 and P and
// cross(r, P) are finite; its velocity terms in the relative velocity are then constants of the row: for M on side
// B, ((vM + cross(wM, rM)) - vF) - cross(wF, rF), for M on side A, ((vF + cross(wF, rF)) - vM) - cross(wM, rM), with
// cross(wF, rF) and vF + cross(wF, rF) evaluated once. M's velocity stays in registers, its updates are
// v + ms * P and w + is * cross(r, P) (ms, is = +-m, +-i): solve_vrow's floats for M with fewer instructions. The
// guard (the fixed velocity and arms finite, not -0 and below 2^60 when the rows are built; every applied impulse
// below 2^60, as one running sum) fails over to solve_vrow's passes from the same velocities.
struct TVRow {
    V2 n, r0, r1;  // the normal and M's arms
    V2 f0, f1;     // the fixed side's term at each point (see above)
    V2 vF;         // M on side B: the fixed side's velocity
    float tm0, tm1, nm0, nm1, b0, b1, K0, K1, K2, K3, N0, N1, N2, N3, friction, tspeed, ms, is;
    float ni0, ni1, ti0, ti1;
    int cnt;
    bool mvB;
};

// Velocity row r as a TVRow for the moving body M; false when the row is not of the form above or fails the guard.
GOI_D bool make_tvrow(const Bodies& bd, const VRow& r, int M, TVRow& t) {
    const bool mvB = r.ib == M;
    if (mvB == (r.ia == M)) return false;
    const int f = mvB ? r.ia : r.ib;
    const V2 vF = bd.v(f);
    const float wF = bd.w(f);
    const V2 rF0 = mvB ? r.rA0 : r.rB0, rF1 = mvB ? r.rA1 : r.rB1;
    const float mF = mvB ? r.mA : r.mB, iF = mvB ? r.iA : r.iB;
    const auto sane = [](float x) { return fabsf(x) < 0x1p60f && __float_as_uint(x) != 0x80000000u; };
    const bool ok = mF == 0.0f && iF == 0.0f && sane(vF.x) && sane(vF.y) && sane(wF) && fabsf(rF0.x) < 0x1p60f &&
                    fabsf(rF0.y) < 0x1p60f && fabsf(rF1.x) < 0x1p60f && fabsf(rF1.y) < 0x1p60f &&
                    fabsf(r.n.x) < 4.0f && fabsf(r.n.y) < 4.0f;
    t.n = r.n;
    t.r0 = mvB ? r.rB0 : r.rA0;
    t.r1 = mvB ? r.rB1 : r.rA1;
    if (mvB) {
        t.vF = vF;
        t.f0 = cross(wF, rF0);
        t.f1 = cross(wF, rF1);
    } else {
        t.vF = mk(0.0f, 0.0f);
        t.f0 = vF + cross(wF, rF0);
        t.f1 = vF + cross(wF, rF1);
    }
    t.ms = mvB ? r.mB : -r.mA;
    t.is = mvB ? r.iB : -r.iA;
    t.tm0 = r.tm0; t.tm1 = r.tm1; t.nm0 = r.nm0; t.nm1 = r.nm1; t.b0 = r.b0; t.b1 = r.b1;
    t.K0 = r.K0; t.K1 = r.K1; t.K2 = r.K2; t.K3 = r.K3; t.N0 = r.N0; t.N1 = r.N1; t.N2 = r.N2; t.N3 = r.N3;
    t.friction = r.friction; t.tspeed = r.tspeed;
    t.ni0 = r.ni0; t.ni1 = r.ni1; t.ti0 = r.ti0; t.ti1 = r.ti1;
    t.cnt = r.cnt;
    t.mvB = mvB;
    return ok;
}

// solve_vrow on a TVRow, M's velocity (vM, wM) in registers; acc gathers the applied impulses' magnitudes.
template <bool kMvB>
GOI_D void solve_tvrow(TVRow& r, V2& vM, float& wM, float& acc) {
    const V2 n = r.n, t = cross(n, 1.0f);
    const auto dv = [&](V2 rM, V2 f) {
        if constexpr (kMvB) return ((vM + cross(wM, rM)) - r.vF) - f;
        else return (f - vM) - cross(wM, rM);
    };
    float ni0 = r.ni0, ni1 = r.ni1, ti0 = r.ti0, ti1 = r.ti1;
    if (r.cnt > 0) {
        const float vt = dot(dv(r.r0, r.f0), t) - r.tspeed;
        float lam = r.tm0 * (-vt);
        const float maxf = r.friction * ni0;
        const float nw = bclamp(ti0 + lam, -maxf, maxf);
        lam = nw - ti0;
        ti0 = nw;
        const V2 P = lam * t;
        vM = vM + r.ms * P;
        wM = wM + r.is * cross(r.r0, P);
        acc = acc + fabsf(lam);
    }
    if (r.cnt > 1) {
        const float vt = dot(dv(r.r1, r.f1), t) - r.tspeed;
        float lam = r.tm1 * (-vt);
        const float maxf = r.friction * ni1;
        const float nw = bclamp(ti1 + lam, -maxf, maxf);
        lam = nw - ti1;
        ti1 = nw;
        const V2 P = lam * t;
        vM = vM + r.ms * P;
        wM = wM + r.is * cross(r.r1, P);
        acc = acc + fabsf(lam);
    }
    if (r.cnt == 1) {
        const float vn = dot(dv(r.r0, r.f0), n);
        float lam = -r.nm0 * (vn - r.b0);
        const float nw = bmax(ni0 + lam, 0.0f);
        lam = nw - ni0;
        ni0 = nw;
        const V2 P = lam * n;
        vM = vM + r.ms * P;
        wM = wM + r.is * cross(r.r0, P);
        acc = acc + fabsf(lam);
    } else if (r.cnt == 2) {
        const float K0 = r.K0, K1 = r.K1, K2 = r.K2, K3 = r.K3;
        const float ax = ni0, ay = ni1;
        const float vn1 = dot(dv(r.r0, r.f0), n);
        const float vn2 = dot(dv(r.r1, r.f1), n);
        float bx = vn1 - r.b0, by = vn2 - r.b1;
        bx = bx - (K0 * ax + K2 * ay);
        by = by - (K1 * ax + K3 * ay);
        float xx = -(r.N0 * bx + r.N2 * by);
        float xy = -(r.N1 * bx + r.N3 * by);
        bool ok = xx >= 0.0f && xy >= 0.0f;
        if (!ok) {
            xx = -r.nm0 * bx;
            xy = 0.0f;
            ok = xx >= 0.0f && K1 * xx + by >= 0.0f;
        }
        if (!ok) {
            xx = 0.0f;
            xy = -r.nm1 * by;
            ok = xy >= 0.0f && K2 * xy + bx >= 0.0f;
        }
        if (!ok) {
            xx = 0.0f;
            xy = 0.0f;
            ok = bx >= 0.0f && by >= 0.0f;
        }
        if (ok) {
            const float dx = xx - ax, dy = xy - ay;
            const V2 P1 = dx * n, P2 = dy * n;
            vM = vM + r.ms * (P1 + P2);
            wM = wM + r.is * (cross(r.r0, P1) + cross(r.r1, P2));
            ni0 = xx;
            ni1 = xy;
            acc = acc + (fabsf(dx) + fabsf(dy));
        }
    }
    r.ni0 = ni0; r.ni1 = ni1; r.ti0 = ti0; r.ti1 = ti1;
}
GOI_D void solve_tvrow(TVRow& r, V2& vM, float& wM, float& acc) {
    if (r.mvB) solve_tvrow<true>(r, vM, wM, acc);
    else solve_tvrow<false>(r, vM, wM, acc);
}

GOI_D void store_vimpulses(const Rows& R, int i, const VRow& r) {
    R.setf(i, CF_NI0, r.ni0); R.setf(i, CF_NI1, r.ni1); R.setf(i, CF_TI0, r.ti0); R.setf(i, CF_TI1, r.ti1);
}

// rows i0..n-1 once each, in order, each loaded in one batch while the row before it is solved; two rows a loop
// iteration, so the two row buffers alternate without copies between them
template <class BD>
GOI_D void cs_solve_velocity_sweep(const BD& bd, const Rows& R, int i0, int n) {
    if (n <= i0) return;
    VRow a = load_vrow(R, i0), b;
    for (int i = i0; i < n; i += 2) {
        if (i + 1 < n) b = load_vrow(R, i + 1);
        solve_vrow(bd, a);
        store_vimpulses(R, i, a);
        if (i + 1 >= n) break;
        if (i + 2 < n) a = load_vrow(R, i + 2);
        solve_vrow(bd, b);
        store_vimpulses(R, i + 1, b);
    }
}

// A contact row's position-solver fields (b2ContactPositionConstraint), loaded in one batch.
struct PRow {
    int ia, ib, cnt, mtype;
    V2 lcA, lcB, ln, lp, pl0, pl1;
    float radA, radB, mA, mB, iA, iB;
};

GOI_D PRow load_prow(const Rows& R, int i) {
    PRow r;
    r.ia = R.geti(i, CF_IA); r.ib = R.geti(i, CF_IB); r.cnt = R.geti(i, CF_PC_COUNT); r.mtype = R.geti(i, CF_MTYPE);
    r.lcA = R.get2(i, CF_LCA); r.lcB = R.get2(i, CF_LCB); r.ln = R.get2(i, CF_LN); r.lp = R.get2(i, CF_LP);
    r.pl0 = R.get2(i, CF_PL0); r.pl1 = R.get2(i, CF_PL1);
    r.radA = R.getf(i, CF_RADA); r.radB = R.getf(i, CF_RADB);
    r.mA = R.getf(i, CF_MA); r.mB = R.getf(i, CF_MB); r.iA = R.getf(i, CF_IIA); r.iB = R.getf(i, CF_IIB);
    return r;
}

// b2ContactSolver::SolvePositionConstraints for one row (contact_solver.py:307-354); masses given (the TOI solve
// passes zero for bodies other than the TOI pair). Returns the row's min separation, starting at 0. The callers keep
// one rotation memo per side across rows and passes.
template <class BD>
GOI_D float solve_prow(const BD& bd, const PRow& r, float baumgarte, float mA, float mB, float iA, float iB,
                       float linear_slop, float max_linear_correction, RotMemo& qa, RotMemo& qb) {
    const V2 lcA = r.lcA, lcB = r.lcB, ln = r.ln, lp = r.lp;
    const float radA = r.radA, radB = r.radB;
    V2 cA = bd.c(r.ia), cB = bd.c(r.ib);
    float aA = bd.a(r.ia), aB = bd.a(r.ib);
    float min_sep = 0.0f;
    for (int j = 0; j < r.cnt; ++j) {
        Xf xfA, xfB;
        xfA.q = qa.of(aA);
        xfB.q = qb.of(aB);
        xfA.p = cA - mul(xfA.q, lcA);
        xfB.p = cB - mul(xfB.q, lcB);
        const V2 plj = j == 0 ? r.pl0 : r.pl1;
        V2 n, p;
        float sep;
        if (r.mtype == kCircles) {
            const V2 pA = mul(xfA, lp), pB = mul(xfB, r.pl0);
            n = pB - pA;
            normalize(n);
            p = 0.5f * (pA + pB);
            sep = (dot(pB - pA, n) - radA) - radB;
        } else {
            // face A or face B: the same operations with the reference and incident transforms swapped (one path
            // for both, so lanes of different manifold types do not diverge)
            const bool fa = r.mtype == kFaceA;
            const Xf& x1 = fa ? xfA : xfB;
            const Xf& x2 = fa ? xfB : xfA;
            n = mul(x1.q, ln);
            const V2 cp = mul(x2, plj);
            sep = (dot(cp - mul(x1, lp), n) - radA) - radB;
            p = cp;
            if (!fa) n = -n;
        }
        const V2 rA = p - cA, rB = p - cB;
        min_sep = bmin(min_sep, sep);
        const float C = bclamp(baumgarte * (sep + linear_slop), -max_linear_correction, 0.0f);
        const float rnA = cross(rA, n), rnB = cross(rB, n);
        const float K = ((mA + mB) + iA * rnA * rnA) + iB * rnB * rnB;
        const float imp = K > 0.0f ? -C / K : 0.0f;
        const V2 P = imp * n;
        cA = cA - mA * P; aA = aA - iA * cross(rA, P);
        cB = cB + mB * P; aB = aB + iB * cross(rB, P);
    }
    bd.set_c(r.ia, cA, aA);
    bd.set_c(r.ib, cB, aB);
    return min_sep;
}

// ---- TOI position passes with one moving body
//
// In b2Island::SolveTOI's position passes (toi.py:738-760) only the TOI pair has mass. When exactly one of the pair
// has mass (M; the other is static or kinematic, as in every event of a dynamic body against the terrain), every row
// has M on one side and a side without mass (mass and inertia 0) on the other. That side's updates c - 0 * P and
// a - 0 * cross(r, P), and its term 0 * rn * rn of K, are identities when its c and a are finite and not -0 and r,
// rn and P are finite. The passes then need only M's pose, kept in registers, and per row the fixed side's transform
// and the normal, plane point or clip points it alone determines, evaluated once per event: solve_prow's floats for M
// with half its instructions (a wave running one world's TOI events alone issues one instruction every few clocks,
// so the count is the time). K is m + i * rn * rn of M, M's update c + ms * P and a + is * cross(r, P) with
// ms, is = +-m, +-i (x - y is x + -y), and the face-B flip of the normal n folded into ms and is: with n = -n1,
// rn * rn, P = -(imp * n1) and cross(r, P) = -cross(r, imp * n1) are the same floats negated or not.
// The guard. When the rows are built: the fixed pose finite, below 2^40 and not -0; M's pose below 2^40 and its angle
// below 2^20; the local vectors and fixed points below 2^40 and the local normal below 4; M's mass in [2^-40, 2^40),
// its inertia in [0, 2^40); the max linear correction in [0, 2^10]. Then K >= m > 0 (solve_prow's K > 0 always
// holds), |C| <= max correction, so M moves by at most 2^13 a point and at most 2^24 over the passes (20 passes of at
// most 64 points), every point, r, rn and P stay finite. In the passes: each angle that sin/cos is taken of below 2^20
// (one running sum of |a| * 2^40, which an infinity or NaN also fails). When it fails, or a row does not have this
// form, solve_prow's passes run from the same poses.
struct TRow {
    V2 lc;      // M's local center
    V2 u0, u1;  // M's local vectors: kind 1 the local normal and point, kind 2 the two local points
    V2 k0, k1;  // the fixed side's: kind 1 the two clip points, kind 2 the normal (before the face-B flip) and the
                // plane point
    float radA, radB, ms, is;
    int bits;   // point count | 4 when M holds the reference face (kind 1; else kind 2, M holds the incident points)
};

// a TOI row in a row's velocity-solver fields (the event sets those up, impulses included, after the passes)
enum { TF_BITS = CF_RA0, TF_LC, TF_U0 = TF_LC + 2, TF_U1 = TF_U0 + 2, TF_K0 = TF_U1 + 2, TF_K1 = TF_K0 + 2,
       TF_RADA = TF_K1 + 2, TF_RADB, TF_MS, TF_IS, TF_END };
static_assert(TF_END <= CF_LN, "a TOI row must fit the velocity-solver fields");

GOI_D void store_trow(const Rows& R, int i, const TRow& t) {
    R.seti(i, TF_BITS, t.bits); R.set2(i, TF_LC, t.lc); R.set2(i, TF_U0, t.u0); R.set2(i, TF_U1, t.u1);
    R.set2(i, TF_K0, t.k0); R.set2(i, TF_K1, t.k1);
    R.setf(i, TF_RADA, t.radA); R.setf(i, TF_RADB, t.radB); R.setf(i, TF_MS, t.ms); R.setf(i, TF_IS, t.is);
}
GOI_D TRow load_trow(const Rows& R, int i) {
    TRow t;
    t.bits = R.geti(i, TF_BITS); t.lc = R.get2(i, TF_LC); t.u0 = R.get2(i, TF_U0); t.u1 = R.get2(i, TF_U1);
    t.k0 = R.get2(i, TF_K0); t.k1 = R.get2(i, TF_K1);
    t.radA = R.getf(i, TF_RADA); t.radB = R.getf(i, TF_RADB); t.ms = R.getf(i, TF_MS); t.is = R.getf(i, TF_IS);
    return t;
}

GOI_D bool below40(V2 v) { return fabsf(v.x) < 0x1p40f && fabsf(v.y) < 0x1p40f; }

// Row r as a TRow for the moving body M (mass m, inertia i; checked by the caller); false when the row is not of the
// form above or fails the guard.
GOI_D bool make_trow(const Bodies& bd, const PRow& r, int M, float m, float i, TRow& t) {
    const bool mvB = r.ib == M;
    if (mvB == (r.ia == M) || r.mtype == kCircles) return false;
    const int f = mvB ? r.ia : r.ib;
    const V2 cF = bd.c(f);
    const float aF = bd.a(f);
    Xf xf;
    xf.q = rot_of(aF);
    xf.p = cF - mul(xf.q, mvB ? r.lcA : r.lcB);
    const bool fa = r.mtype == kFaceA;
    const bool mref = fa != mvB;
    if (mref) {
        t.u0 = r.ln;
        t.u1 = r.lp;
        t.k0 = mul(xf, r.pl0);
        t.k1 = mul(xf, r.pl1);
    } else {
        t.u0 = r.pl0;
        t.u1 = r.pl1;
        t.k0 = mul(xf.q, r.ln);
        t.k1 = mul(xf, r.lp);
    }
    t.lc = mvB ? r.lcB : r.lcA;
    t.radA = r.radA;
    t.radB = r.radB;
    const float sg = fa ? 1.0f : -1.0f;
    t.ms = sg * (mvB ? m : -m);
    t.is = sg * (mvB ? i : -i);
    t.bits = r.cnt | (mref ? 4 : 0);
    return below40(cF) && fabsf(aF) < 0x1p40f && __float_as_uint(cF.x) != 0x80000000u &&
           __float_as_uint(cF.y) != 0x80000000u && __float_as_uint(aF) != 0x80000000u && fabsf(r.ln.x) < 4.0f &&
           fabsf(r.ln.y) < 4.0f && below40(t.lc) && below40(t.u0) && below40(t.u1) && below40(t.k0) &&
           below40(t.k1);
}

// One pass over a TRow of kind kKind on M's pose; acc gathers the guard's angles.
template <int kKind>
GOI_D float trow_pass(const TRow& t, float baumgarte, float linear_slop, float max_linear_correction, V2& cM,
                      float& aM, float& acc) {
    float min_sep = 0.0f;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        if (j >= (t.bits & 3)) break;
        Xf xf;
        xf.q = rot_of_small(aM);
        xf.p = cM - mul(xf.q, t.lc);
        V2 cp, n1;
        float sep;
        if constexpr (kKind == 1) {
            n1 = mul(xf.q, t.u0);
            cp = j == 0 ? t.k0 : t.k1;
            sep = (dot(cp - mul(xf, t.u1), n1) - t.radA) - t.radB;
        } else {
            n1 = t.k0;
            cp = mul(xf, j == 0 ? t.u0 : t.u1);
            sep = (dot(cp - t.k1, n1) - t.radA) - t.radB;
        }
        const V2 r = cp - cM;
        min_sep = bmin(min_sep, sep);
        const float C = bclamp(baumgarte * (sep + linear_slop), -max_linear_correction, 0.0f);
        const float rn = cross(r, n1);
        const float imp = -C / (fabsf(t.ms) + fabsf(t.is) * rn * rn);
        const V2 P = imp * n1;
        cM = cM + t.ms * P;
        aM = aM + t.is * cross(r, P);
        acc = fmaf(fabsf(aM), 0x1p40f, acc);
    }
    return min_sep;
}
GOI_D float trow_pass(const TRow& t, float baumgarte, float linear_slop, float max_linear_correction, V2& cM,
                      float& aM, float& acc) {
    return (t.bits & 4) ? trow_pass<1>(t, baumgarte, linear_slop, max_linear_correction, cM, aM, acc)
                        : trow_pass<2>(t, baumgarte, linear_slop, max_linear_correction, cM, aM, acc);
}

}  // namespace goi
