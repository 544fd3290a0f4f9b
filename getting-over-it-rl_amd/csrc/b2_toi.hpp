// b2_toi.hpp - continuous collision on the device: b2World::SolveTOI with b2TimeOfImpact, b2Distance (GJK),
// b2SeparationFunction, b2Sweep::Advance and b2Island::SolveTOI (goi_jax/box2d/toi.py:73-865). Each world's lane
// group runs its event loop; the sweeps live in the State leaves (c0, c, a0, a, toi.alpha0).
#pragma once

#include "b2_joints.hpp"

namespace goi {

struct Sweep {
    V2 lc, c0, c;
    float a0, a;
};

// b2Sweep::GetTransform (toi.py:73-81); the rotation through the sweep's memo
GOI_D Xf sweep_xf(const Sweep& sw, float beta, RotMemo& memo) {
    Xf t;
    const float omb = 1.0f - beta;
    t.q = memo.of(omb * sw.a0 + beta * sw.a);
    t.p = mk(omb * sw.c0.x + beta * sw.c.x, omb * sw.c0.y + beta * sw.c.y) - mul(t.q, sw.lc);
    return t;
}

GOI_D Sweep body_sweep(const World& W, int b) {
    Sweep s;
    s.lc = W.v2(GOI_B_LOCAL_CENTER, b);
    s.c0 = W.v2(GOI_B_C0, b);
    s.c = W.v2(GOI_B_C, b);
    s.a0 = W.f(GOI_B_A0, b);
    s.a = W.f(GOI_B_A, b);
    return s;
}

// b2Sweep::Advance on body b's sweep (toi.py:100-104)
GOI_D void sweep_advance(const World& W, int b, float alpha) {
    const float al0 = W.f(GOI_T_ALPHA0, b);
    const float den = 1.0f - al0;
    const float beta = (alpha - al0) / (den != 0.0f ? den : 1.0f);
    const V2 c0 = W.v2(GOI_B_C0, b), c = W.v2(GOI_B_C, b);
    W.set2(GOI_B_C0, b, c0 + beta * (c - c0));
    const float a0 = W.f(GOI_B_A0, b);
    W.f(GOI_B_A0, b) = a0 + beta * (W.f(GOI_B_A, b) - a0);
    W.f(GOI_T_ALPHA0, b) = alpha;
}

// b2Body::SynchronizeTransform
GOI_D void sync_transform(const World& W, int b) {
    const float a = W.f(GOI_B_A, b);
    Rot q;
    if (a == 0.0f) {  // a static body's usual angle: rot_of's result, sin = the angle itself (+-0), cos = 1
        q.s = a;
        q.c = 1.0f;
    } else {
        q = rot_of(a);
    }
    W.set2(GOI_B_XF_P, b, W.v2(GOI_B_C, b) - mul(q, W.v2(GOI_B_LOCAL_CENTER, b)));
    W.f(GOI_B_XF_Q, 2 * b) = q.c;
    W.f(GOI_B_XF_Q, 2 * b + 1) = q.s;
}

// b2Body::Advance
GOI_D void body_advance(const World& W, int b, float alpha) {
    sweep_advance(W, b, alpha);
    W.set2(GOI_B_C, b, W.v2(GOI_B_C0, b));
    W.f(GOI_B_A, b) = W.f(GOI_B_A0, b);
    sync_transform(W, b);
}

struct SweepBackup {
    V2 c0, c;
    float a0, a, alpha0;
};
GOI_D SweepBackup backup(const World& W, int b) {
    SweepBackup k;
    k.c0 = W.v2(GOI_B_C0, b); k.c = W.v2(GOI_B_C, b);
    k.a0 = W.f(GOI_B_A0, b); k.a = W.f(GOI_B_A, b); k.alpha0 = W.f(GOI_T_ALPHA0, b);
    return k;
}
GOI_D void restore(const World& W, int b, const SweepBackup& k) {
    W.set2(GOI_B_C0, b, k.c0); W.set2(GOI_B_C, b, k.c);
    W.f(GOI_B_A0, b) = k.a0; W.f(GOI_B_A, b) = k.a; W.f(GOI_T_ALPHA0, b) = k.alpha0;
    sync_transform(W, b);
}

// ---------------------------------------------------------------- distance proxies and GJK (toi.py:116-294)

// b2DistanceProxy held in registers: the fixture's 8 vertex slots are loaded once, in one batch (the slots past
// `count` are padding and never selected), so GJK's support searches and vertex lookups stay off memory.
struct Proxy {
    V2 v[kPoly];
    int count;
    float radius;
    // vertex i (0 <= i < count) without dynamic register indexing: a chain of selects that starts from a constant
    // (a chain of selects between loads would fold into one load from a selected address, which keeps the vertex
    // array in private scratch memory)
    GOI_D V2 at(int i) const {
        V2 r = mk(0.0f, 0.0f);
#pragma unroll
        for (int j = 0; j < kPoly; ++j)
            if (i == j) r = v[j];
        return r;
    }
};
GOI_D Proxy proxy_of(const DModel& m, int f) {
    Proxy p;
#pragma unroll
    for (int j = 0; j < kPoly; ++j) p.v[j] = m.poly[16 * f + j];
    p.count = m.fix[f].count;
    p.radius = m.fix[f].radius;
    return p;
}
// b2DistanceProxy::GetSupport and GetVertex together: the first index of the largest dot and its vertex, selected in
// the same pass over the slots (no select chain over the slots by index after it); a quad's pass covers 4 slots
struct Support {
    V2 v;
    int i;
};
template <int kN>
GOI_D Support support_over(const Proxy& p, V2 d) {
    Support s;
    s.i = 0;
    s.v = p.v[0];
    float bv = dot(p.v[0], d);
#pragma unroll
    for (int i = 1; i < kN; ++i) {
        const float v = dot(p.v[i], d);
        if (i < p.count && v > bv) {
            s.i = i;
            s.v = p.v[i];
            bv = v;
        }
    }
    return s;
}
GOI_D Support support(const Proxy& p, V2 d) {
    if (p.count <= 4) return support_over<4>(p, d);
    return support_over<kPoly>(p, d);
}

struct SVert {
    V2 wA, wB, w;
    float a;
    int iA, iB;
};
struct SimplexCache {
    float metric;
    int count;
    int iA[3], iB[3];
};

GOI_D float metric(const SVert* v, int count) {
    if (count == 2) return length(v[0].w - v[1].w);
    if (count == 3) return cross(v[1].w - v[0].w, v[2].w - v[0].w);
    return 0.0f;
}

GOI_D void set_vertex(SVert& v, const Xf& xA, int iA, V2 lA, const Xf& xB, int iB, V2 lB) {
    v.iA = iA;
    v.iB = iB;
    v.wA = mul(xA, lA);
    v.wB = mul(xB, lB);
    v.w = v.wB - v.wA;
}
GOI_D void set_vertex(SVert& v, const Proxy& pA, const Xf& xA, int iA, const Proxy& pB, const Xf& xB, int iB) {
    set_vertex(v, xA, iA, pA.at(iA), xB, iB, pB.at(iB));
}

GOI_D void simplex_solve2(SVert* v, int& count) {
    const V2 w1 = v[0].w, w2 = v[1].w, e12 = w2 - w1;
    const float d12_2 = -dot(w1, e12);
    if (d12_2 <= 0.0f) { v[0].a = 1.0f; count = 1; return; }
    const float d12_1 = dot(w2, e12);
    if (d12_1 <= 0.0f) { v[1].a = 1.0f; count = 1; v[0] = v[1]; return; }
    const float inv = 1.0f / (d12_1 + d12_2);
    v[0].a = d12_1 * inv;
    v[1].a = d12_2 * inv;
    count = 2;
}

GOI_D void simplex_solve3(SVert* v, int& count) {
    const V2 w1 = v[0].w, w2 = v[1].w, w3 = v[2].w;
    const V2 e12 = w2 - w1, e13 = w3 - w1, e23 = w3 - w2;
    const float d12_1 = dot(w2, e12), d12_2 = -dot(w1, e12);
    const float d13_1 = dot(w3, e13), d13_2 = -dot(w1, e13);
    const float d23_1 = dot(w3, e23), d23_2 = -dot(w2, e23);
    const float n123 = cross(e12, e13);
    const float d123_1 = n123 * cross(w2, w3), d123_2 = n123 * cross(w3, w1), d123_3 = n123 * cross(w1, w2);
    if (d12_2 <= 0.0f && d13_2 <= 0.0f) { v[0].a = 1.0f; count = 1; return; }
    if (d12_1 > 0.0f && d12_2 > 0.0f && d123_3 <= 0.0f) {
        const float inv = 1.0f / (d12_1 + d12_2);
        v[0].a = d12_1 * inv; v[1].a = d12_2 * inv; count = 2; return;
    }
    if (d13_1 > 0.0f && d13_2 > 0.0f && d123_2 <= 0.0f) {
        const float inv = 1.0f / (d13_1 + d13_2);
        v[0].a = d13_1 * inv; v[2].a = d13_2 * inv; count = 2; v[1] = v[2]; return;
    }
    if (d12_1 <= 0.0f && d23_2 <= 0.0f) { v[1].a = 1.0f; count = 1; v[0] = v[1]; return; }
    if (d13_1 <= 0.0f && d23_1 <= 0.0f) { v[2].a = 1.0f; count = 1; v[0] = v[2]; return; }
    if (d23_1 > 0.0f && d23_2 > 0.0f && d123_1 <= 0.0f) {
        const float inv = 1.0f / (d23_1 + d23_2);
        v[1].a = d23_1 * inv; v[2].a = d23_2 * inv; count = 2; v[0] = v[2]; return;
    }
    const float inv = 1.0f / ((d123_1 + d123_2) + d123_3);
    v[0].a = d123_1 * inv; v[1].a = d123_2 * inv; v[2].a = d123_3 * inv;
    count = 3;
}

// b2Distance (useRadii = false): the distance and the updated simplex cache. The simplex, the saved indices and
// the cache are indexed only by constants once the short loops are unrolled, so they stay in registers (a runtime
// index would put them in private scratch memory, one memory round trip per access).
GOI_D float gjk_distance(SimplexCache& cache, const Proxy& pA, const Xf& xA, const Proxy& pB, const Xf& xB) {
    SVert v[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        v[i].a = 0.0f;
        v[i].iA = 0; v[i].iB = 0;
        v[i].wA = mk(0.0f, 0.0f); v[i].wB = v[i].wA; v[i].w = v[i].wA;
    }
    int count = cache.count;
#pragma unroll
    for (int i = 0; i < 3; ++i)
        if (i < count) set_vertex(v[i], pA, xA, cache.iA[i], pB, xB, cache.iB[i]);
    if (count > 1) {
        const float m1 = cache.metric, m2 = metric(v, count);
        if (m2 < 0.5f * m1 || 2.0f * m1 < m2 || m2 < kEps) count = 0;
    }
    if (count == 0) {
        set_vertex(v[0], pA, xA, 0, pB, xB, 0);
        v[0].a = 1.0f;
        count = 1;
    }
    int saveA[3], saveB[3];
    for (int iter = 0; iter < 20;) {
        const int save = count;
#pragma unroll
        for (int i = 0; i < 3; ++i)
            if (i < save) { saveA[i] = v[i].iA; saveB[i] = v[i].iB; }
        if (count == 2) simplex_solve2(v, count);
        else if (count == 3) simplex_solve3(v, count);
        if (count == 3) break;
        V2 d;
        if (count == 1) {
            d = -v[0].w;
        } else {
            const V2 e12 = v[1].w - v[0].w;
            d = cross(e12, -v[0].w) > 0.0f ? cross(1.0f, e12) : cross(e12, 1.0f);
        }
        if (dot(d, d) < kEps * kEps) break;
        // the new vertex takes slot `count` (1 or 2); its barycentric coordinate is left as it was
        SVert nv;
        const Support sa = support(pA, mulT(xA.q, -d)), sb = support(pB, mulT(xB.q, d));
        set_vertex(nv, xA, sa.i, sa.v, xB, sb.i, sb.v);
        nv.a = count == 1 ? v[1].a : v[2].a;
        if (count == 1) v[1] = nv;
        else v[2] = nv;
        ++iter;
        bool dup = false;
#pragma unroll
        for (int i = 0; i < 3; ++i)
            if (i < save) dup |= (nv.iA == saveA[i] && nv.iB == saveB[i]);
        if (dup) break;
        ++count;
    }
    V2 pa, pb;
    if (count == 1) {
        pa = v[0].wA;
        pb = v[0].wB;
    } else if (count == 2) {
        pa = v[0].a * v[0].wA + v[1].a * v[1].wA;
        pb = v[0].a * v[0].wB + v[1].a * v[1].wB;
    } else {
        pa = (v[0].a * v[0].wA + v[1].a * v[1].wA) + v[2].a * v[2].wA;
        pb = pa;
    }
    cache.metric = metric(v, count);
    cache.count = count;
#pragma unroll
    for (int i = 0; i < 3; ++i)
        if (i < count) { cache.iA[i] = v[i].iA; cache.iB[i] = v[i].iB; }
    return length(pa - pb);
}

// ---------------------------------------------------------------- b2SeparationFunction and b2TimeOfImpact

enum { kSepPoints = 0, kSepFaceA = 1, kSepFaceB = 2 };
struct SepFn {
    int type;
    V2 axis, lp;
};

GOI_D SepFn sep_init(const SimplexCache& cache, const Proxy& pA, const Sweep& sA, const Proxy& pB, const Sweep& sB,
                     float t1, RotMemo& ma, RotMemo& mb) {
    const Xf xA = sweep_xf(sA, t1, ma), xB = sweep_xf(sB, t1, mb);
    SepFn f;
    f.lp = mk(0.0f, 0.0f);
    if (cache.count == 1) {
        f.type = kSepPoints;
        f.axis = mul(xB, pB.at(cache.iB[0])) - mul(xA, pA.at(cache.iA[0]));
        normalize(f.axis);
    } else if (cache.iA[0] == cache.iA[1]) {
        f.type = kSepFaceB;
        const V2 b1 = pB.at(cache.iB[0]), b2 = pB.at(cache.iB[1]);
        f.axis = cross(b2 - b1, 1.0f);
        normalize(f.axis);
        const V2 n = mul(xB.q, f.axis);
        f.lp = 0.5f * (b1 + b2);
        if (dot(mul(xA, pA.at(cache.iA[0])) - mul(xB, f.lp), n) < 0.0f) f.axis = -f.axis;
    } else {
        f.type = kSepFaceA;
        const V2 a1 = pA.at(cache.iA[0]), a2 = pA.at(cache.iA[1]);
        f.axis = cross(a2 - a1, 1.0f);
        normalize(f.axis);
        const V2 n = mul(xA.q, f.axis);
        f.lp = 0.5f * (a1 + a2);
        if (dot(mul(xB, pB.at(cache.iB[0])) - mul(xA, f.lp), n) < 0.0f) f.axis = -f.axis;
    }
    return f;
}

// b2SeparationFunction::Evaluate at the support vertices lA = pA.at(iA), lB = pB.at(iB) that FindMinSeparation chose
// (those of a face's own proxy unused), looked up once by the caller for all the root finder's steps
GOI_D float sep_eval(const SepFn& f, const Sweep& sA, const Sweep& sB, V2 lA, V2 lB, float t, RotMemo& ma,
                     RotMemo& mb) {
    const Xf xA = sweep_xf(sA, t, ma), xB = sweep_xf(sB, t, mb);
    if (f.type == kSepPoints) return dot(mul(xB, lB) - mul(xA, lA), f.axis);
    if (f.type == kSepFaceA) return dot(mul(xB, lB) - mul(xA, f.lp), mul(xA.q, f.axis));
    return dot(mul(xA, lA) - mul(xB, f.lp), mul(xB.q, f.axis));
}

// b2SeparationFunction::FindMinSeparation; lA, lB its support vertices (lA = (0, 0) for face A, lB for face B)
GOI_D float sep_find_min(const SepFn& f, const Proxy& pA, const Sweep& sA, const Proxy& pB, const Sweep& sB, V2& lA,
                         V2& lB, float t, RotMemo& ma, RotMemo& mb) {
    const Xf xA = sweep_xf(sA, t, ma), xB = sweep_xf(sB, t, mb);
    if (f.type == kSepPoints) {
        lA = support(pA, mulT(xA.q, f.axis)).v;
        lB = support(pB, mulT(xB.q, -f.axis)).v;
        return dot(mul(xB, lB) - mul(xA, lA), f.axis);
    }
    if (f.type == kSepFaceA) {
        const V2 n = mul(xA.q, f.axis);
        lA = mk(0.0f, 0.0f);
        lB = support(pB, mulT(xB.q, -n)).v;
        return dot(mul(xB, lB) - mul(xA, f.lp), n);
    }
    const V2 n = mul(xB.q, f.axis);
    lB = mk(0.0f, 0.0f);
    lA = support(pA, mulT(xA.q, -n)).v;
    return dot(mul(xA, lA) - mul(xB, f.lp), n);
}

enum { kToiUnknown = 0, kToiFailed = 1, kToiOverlapped = 2, kToiTouching = 3, kToiSeparated = 4 };

// b2TimeOfImpact with tMax = 1 (toi.py:364-457): separating axes (20), push-backs (8), root finder (50 steps of
// alternating bisection and secant)
GOI_D int time_of_impact(const Proxy& pA, Sweep sA, const Proxy& pB, Sweep sB, float linear_slop, float& t_out) {
    const float two_pi = 2.0f * kPi;
    {
        const float d = two_pi * floorf(sA.a0 / two_pi);
        sA.a0 = sA.a0 - d; sA.a = sA.a - d;
    }
    {
        const float d = two_pi * floorf(sB.a0 / two_pi);
        sB.a0 = sB.a0 - d; sB.a = sB.a - d;
    }
    const float total_radius = pA.radius + pB.radius;
    const float target = bmax(linear_slop, total_radius - 3.0f * linear_slop);
    const float tol = 0.25f * linear_slop;
    float t1 = 0.0f;
    SimplexCache cache;
    cache.count = 0;
    cache.metric = 0.0f;
    int state = kToiUnknown;
    t_out = 1.0f;
    RotMemo ma, mb;
    for (int iter = 0;;) {
        const float dist = gjk_distance(cache, pA, sweep_xf(sA, t1, ma), pB, sweep_xf(sB, t1, mb));
        if (dist <= 0.0f) { state = kToiOverlapped; t_out = 0.0f; break; }
        if (dist < target + tol) { state = kToiTouching; t_out = t1; break; }
        const SepFn f = sep_init(cache, pA, sA, pB, sB, t1, ma, mb);
        bool done = false;
        float t2 = 1.0f;
        for (int push = 0;;) {
            V2 lA, lB;
            float s2 = sep_find_min(f, pA, sA, pB, sB, lA, lB, t2, ma, mb);
            if (s2 > target + tol) { state = kToiSeparated; t_out = 1.0f; done = true; break; }
            if (s2 > target - tol) { t1 = t2; break; }
            float s1 = sep_eval(f, sA, sB, lA, lB, t1, ma, mb);
            if (s1 < target - tol) { state = kToiFailed; t_out = t1; done = true; break; }
            if (s1 <= target + tol) { state = kToiTouching; t_out = t1; done = true; break; }
            float a1 = t1, a2 = t2;
            for (int rc = 0;;) {
                const float t = (rc & 1) ? a1 + (target - s1) * (a2 - a1) / (s2 - s1) : 0.5f * (a1 + a2);
                ++rc;
                const float s = sep_eval(f, sA, sB, lA, lB, t, ma, mb);
                if (babs(s - target) < tol) { t2 = t; break; }
                if (s > target) { a1 = t; s1 = s; }
                else { a2 = t; s2 = s; }
                if (rc == 50) break;
            }
            if (++push == kPoly) break;
        }
        ++iter;
        if (done) break;
        if (iter == 20) { state = kToiFailed; t_out = t1; break; }
    }
    return state;
}

}  // namespace goi
