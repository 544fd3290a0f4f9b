// b2_joints.hpp - revolute (Box2D v2.4.1 solver and stock 2.3.1), prismatic and weld joints on the device
// (goi_jax/box2d/joints.py:39-622; scripts/patches/box2d-2.3.1-revolute24.patch:78-330). One joint row per ordered
// joint in HBM scratch (Rows, JF_* fields); each row's branch runs only its own joint type.
#pragma once

#include "b2_solver.hpp"

namespace goi {

enum { kInactive = 0, kAtLower = 1, kAtUpper = 2, kEqual = 3 };

GOI_D V3 jcol(const Rows& R, int i, int f) { return mk3(R.getf(i, f), R.getf(i, f + 1), R.getf(i, f + 2)); }
GOI_D void set_jcol(const Rows& R, int i, int f, V3 v) { R.setf(i, f, v.x); R.setf(i, f + 1, v.y); R.setf(i, f + 2, v.z); }

// InitVelocityConstraints minus the velocity writes (joints.py:61-174): row i for joint jid.
GOI_D void jn_prepare(const DModel& m, const World& W, const Bodies& bd, const Rows& R, int i, int jid,
                      const GoiSettings& s, float dt, float dt_ratio, bool warm, Rot qA, Rot qB) {
    const int type = m.rev_only ? (int)GOI_REVOLUTE : m.joint[jid].type;
    const int ia = m.joint[jid].a, ib = m.joint[jid].b;
    const float mA = W.f(GOI_B_INV_MASS, ia), mB = W.f(GOI_B_INV_MASS, ib);
    const float iA = W.f(GOI_B_INV_INERTIA, ia), iB = W.f(GOI_B_INV_INERTIA, ib);
    const V2 la = m.joint[jid].anchor_a - W.v2(GOI_B_LOCAL_CENTER, ia);
    const V2 lb = m.joint[jid].anchor_b - W.v2(GOI_B_LOCAL_CENTER, ib);
    const V2 rA = mul(qA, la), rB = mul(qB, lb);
    const float ref = m.joint[jid].reference_angle;
    const bool emotor = W.u8(GOI_J_ENABLE_MOTOR, jid) != 0, elimit = W.u8(GOI_J_ENABLE_LIMIT, jid) != 0;
    const float lower = W.f(GOI_J_LOWER, jid), upper = W.f(GOI_J_UPPER, jid);
    const int state_in = W.i32(GOI_J_LIMIT_STATE, jid);
    float ix = W.f(GOI_J_IMPULSE, 3 * jid), iy = W.f(GOI_J_IMPULSE, 3 * jid + 1), iz = W.f(GOI_J_IMPULSE, 3 * jid + 2);
    float mimp = W.f(GOI_J_MOTOR_IMPULSE, jid);
    float lo = 0.0f, up = 0.0f;
    const V2 cA = bd.c(ia), cB = bd.c(ib);
    const float aA = bd.a(ia), aB = bd.a(ib);
    R.seti(i, JF_JID, jid); R.seti(i, JF_TYPE, type); R.seti(i, JF_IA, ia); R.seti(i, JF_IB, ib);
    R.seti(i, JF_EMOTOR, emotor); R.seti(i, JF_ELIMIT, elimit);
    R.setf(i, JF_MA, mA); R.setf(i, JF_MB, mB); R.setf(i, JF_IIA, iA); R.setf(i, JF_IIB, iB);
    R.set2(i, JF_RA, rA); R.set2(i, JF_RB, rB); R.set2(i, JF_LA, la); R.set2(i, JF_LB, lb);
    R.set2(i, JF_LX, m.joint[jid].axis_a); R.set2(i, JF_LY, m.joint[jid].yaxis_a);
    R.setf(i, JF_REF, ref); R.setf(i, JF_LOWER, lower); R.setf(i, JF_UPPER, upper);
    R.setf(i, JF_MSPEED, W.f(GOI_J_MOTOR_SPEED, jid));
    R.setf(i, JF_MAXIMP, dt * W.f(GOI_J_MAX_MOTOR, jid));
    R.setf(i, JF_INVDT, dt > 0.0f ? 1.0f / dt : 0.0f);
    int state = kInactive, soft = 0;
    float mmass = 0.0f, gamma = 0.0f, bias = 0.0f, angle = 0.0f;
    if (type == GOI_REVOLUTE || type == GOI_WELD) {
        const float exx = ((mA + mB) + rA.y * rA.y * iA) + rB.y * rB.y * iB;
        const float eyx = -rA.y * rA.x * iA - rB.y * rB.x * iB;
        const float ezx = -rA.y * iA - rB.y * iB;
        const float eyy = ((mA + mB) + rA.x * rA.x * iA) + rB.x * rB.x * iB;
        const float ezy = rA.x * iA + rB.x * iB;
        const float ezz = iA + iB;
        V3 ex = mk3(exx, eyx, ezx), ey = mk3(eyx, eyy, ezy), ez = mk3(ezx, ezy, ezz);
        if (type == GOI_REVOLUTE) {
            const bool fixed = (iA + iB) == 0.0f;
            mmass = (iA + iB) > 0.0f ? 1.0f / (iA + iB) : 0.0f;
            if (!emotor || fixed) mimp = 0.0f;
            angle = (aB - aA) - ref;
            const bool equal = babs(upper - lower) < 2.0f * s.angular_slop;
            const bool lim_on = elimit && !fixed;
            state = !lim_on ? kInactive : equal ? kEqual : angle <= lower ? kAtLower
                    : angle >= upper ? kAtUpper : kInactive;
            if (s.revolute_v24) {
                lo = lim_on ? W.f(GOI_J_LOWER_IMPULSE, jid) : 0.0f;
                up = lim_on ? W.f(GOI_J_UPPER_IMPULSE, jid) : 0.0f;
            } else if (lim_on && !equal && (state == kInactive || state != state_in)) {
                iz = 0.0f;
            }
        } else {
            soft = W.f(GOI_J_FREQUENCY, jid) > 0.0f;
            const float invM = iA + iB;
            const float wm = invM > 0.0f ? 1.0f / invM : 0.0f;
            const float C = (aB - aA) - ref;
            const float omega = (2.0f * kPi) * W.f(GOI_J_FREQUENCY, jid);
            const float d = 2.0f * wm * W.f(GOI_J_DAMPING, jid) * omega;
            const float k = wm * omega * omega;
            const float h = dt;
            float g = h * (d + h * k);
            g = g != 0.0f ? 1.0f / g : 0.0f;
            const float bs = C * h * k * g;
            if (soft || ez.z == 0.0f) {  // b2Mat33::GetInverse22
                const float a = ex.x, b = ey.x, c = ex.y, dd = ey.y;
                float det = a * dd - b * c;
                if (det != 0.0f) det = 1.0f / det;
                ex = mk3(det * dd, -det * c, 0.0f);
                ey = mk3(-det * b, det * a, 0.0f);
                ez = mk3(0.0f, 0.0f, 0.0f);
            } else {  // b2Mat33::GetSymInverse33
                float det = dot(ex, cross(ey, ez));
                if (det != 0.0f) det = 1.0f / det;
                const float a11 = ex.x, a12 = ey.x, a13 = ez.x, a22 = ey.y, a23 = ez.y, a33 = ez.z;
                const float m11 = det * (a22 * a33 - a23 * a23);
                const float m12 = det * (a13 * a23 - a12 * a33);
                const float m13 = det * (a12 * a23 - a13 * a22);
                const float m22 = det * (a11 * a33 - a13 * a13);
                const float m23 = det * (a13 * a12 - a11 * a23);
                const float m33 = det * (a11 * a22 - a12 * a12);
                ex = mk3(m11, m12, m13); ey = mk3(m12, m22, m23); ez = mk3(m13, m23, m33);
            }
            if (soft) {
                const float inv = invM + g;
                ez.z = inv != 0.0f ? 1.0f / inv : 0.0f;
                gamma = g;
                bias = bs;
            }
            mimp = 0.0f;
        }
        set_jcol(R, i, JF_EXX, ex); set_jcol(R, i, JF_EYX, ey); set_jcol(R, i, JF_EZX, ez);
    } else {  // prismatic
        const V2 d = ((cB - cA) + rB) - rA;
        const V2 axis = mul(qA, m.joint[jid].axis_a);
        const float a1 = cross(d + rA, axis), a2 = cross(rB, axis);
        const float mm = ((mA + mB) + iA * a1 * a1) + iB * a2 * a2;
        mmass = mm > 0.0f ? 1.0f / mm : mm;
        const V2 perp = mul(qA, m.joint[jid].yaxis_a);
        const float s1 = cross(d + rA, perp), s2 = cross(rB, perp);
        const float k11 = ((mA + mB) + iA * s1 * s1) + iB * s2 * s2;
        const float k12 = iA * s1 + iB * s2;
        const float k13 = iA * s1 * a1 + iB * s2 * a2;
        float k22 = iA + iB;
        if (k22 == 0.0f) k22 = 1.0f;
        const float k23 = iA * a1 + iB * a2;
        const float k33 = ((mA + mB) + iA * a1 * a1) + iB * a2 * a2;
        set_jcol(R, i, JF_EXX, mk3(k11, k12, k13));
        set_jcol(R, i, JF_EYX, mk3(k12, k22, k23));
        set_jcol(R, i, JF_EZX, mk3(k13, k23, k33));
        R.set2(i, JF_AX, axis); R.set2(i, JF_PX, perp);
        R.setf(i, JF_A1, a1); R.setf(i, JF_A2, a2); R.setf(i, JF_S1, s1); R.setf(i, JF_S2, s2);
        const float trans = dot(axis, d);
        const bool pequal = babs(upper - lower) < 2.0f * s.linear_slop;
        state = !elimit ? kInactive : pequal ? kEqual : trans <= lower ? kAtLower : trans >= upper ? kAtUpper : kInactive;
        if (!elimit || (!pequal && (state == kInactive || state != state_in))) iz = 0.0f;
        if (!emotor) mimp = 0.0f;
    }
    R.seti(i, JF_STATE, state); R.seti(i, JF_SOFT, soft);
    R.setf(i, JF_MMASS, mmass); R.setf(i, JF_GAMMA, gamma); R.setf(i, JF_BIAS, bias); R.setf(i, JF_ANGLE, angle);
    R.setf(i, JF_IMP0, warm ? ix * dt_ratio : 0.0f);
    R.setf(i, JF_IMP1, warm ? iy * dt_ratio : 0.0f);
    R.setf(i, JF_IMP2, (s.revolute_v24 && type == GOI_REVOLUTE) ? iz : (warm ? iz * dt_ratio : 0.0f));
    R.setf(i, JF_IMP3, warm ? lo * dt_ratio : 0.0f);
    R.setf(i, JF_IMP4, warm ? up * dt_ratio : 0.0f);
    R.setf(i, JF_MIMP, warm ? mimp * dt_ratio : 0.0f);
}

// the velocity part of InitVelocityConstraints (joints.py:202-248)
template <class BD>
GOI_D void jn_warm_start(const BD& bd, const Rows& R, int i, bool v24, bool rev_only) {
    const int type = rev_only ? (int)GOI_REVOLUTE : R.geti(i, JF_TYPE), ia = R.geti(i, JF_IA), ib = R.geti(i, JF_IB);
    const float mA = R.getf(i, JF_MA), mB = R.getf(i, JF_MB), iA = R.getf(i, JF_IIA), iB = R.getf(i, JF_IIB);
    const float ix = R.getf(i, JF_IMP0), iy = R.getf(i, JF_IMP1), iz = R.getf(i, JF_IMP2), mi = R.getf(i, JF_MIMP);
    V2 vA = bd.v(ia), vB = bd.v(ib);
    float wA = bd.w(ia), wB = bd.w(ib);
    if (type == GOI_PRISMATIC) {
        const float mz = mi + iz;
        const V2 P = ix * R.get2(i, JF_PX) + mz * R.get2(i, JF_AX);
        const float LA = (ix * R.getf(i, JF_S1) + iy) + mz * R.getf(i, JF_A1);
        const float LB = (ix * R.getf(i, JF_S2) + iy) + mz * R.getf(i, JF_A2);
        vA = vA - mA * P; wA = wA - iA * LA;
        vB = vB + mB * P; wB = wB + iB * LB;
    } else {
        const V2 P = mk(ix, iy);
        const V2 rA = R.get2(i, JF_RA), rB = R.get2(i, JF_RB);
        vA = vA - mA * P;
        vB = vB + mB * P;
        if (type == GOI_REVOLUTE && v24) {
            const float axial = (mi + R.getf(i, JF_IMP3)) - R.getf(i, JF_IMP4);
            wA = wA - iA * (cross(rA, P) + axial);
            wB = wB + iB * (cross(rB, P) + axial);
        } else if (type == GOI_REVOLUTE) {
            wA = wA - iA * ((cross(rA, P) + mi) + iz);
            wB = wB + iB * ((cross(rB, P) + mi) + iz);
        } else {
            wA = wA - iA * (cross(rA, P) + iz);
            wB = wB + iB * (cross(rB, P) + iz);
        }
    }
    bd.set_v(ia, vA, wA);
    bd.set_v(ib, vB, wB);
}

// SolveVelocityConstraints for joint row i (joints.py:257-437, revolute24.patch:166-240)
template <class BD>
GOI_D void jn_solve_velocity(const BD& bd, const Rows& R, int i, bool v24, bool rev_only) {
    const int type = rev_only ? (int)GOI_REVOLUTE : R.geti(i, JF_TYPE), ia = R.geti(i, JF_IA), ib = R.geti(i, JF_IB);
    const float mA = R.getf(i, JF_MA), mB = R.getf(i, JF_MB), iA = R.getf(i, JF_IIA), iB = R.getf(i, JF_IIB);
    const bool emotor = R.geti(i, JF_EMOTOR) != 0, elimit = R.geti(i, JF_ELIMIT) != 0;
    const int st = R.geti(i, JF_STATE);
    const V3 ex = jcol(R, i, JF_EXX), ey = jcol(R, i, JF_EYX), ez = jcol(R, i, JF_EZX);
    float i0 = R.getf(i, JF_IMP0), i1 = R.getf(i, JF_IMP1), i2 = R.getf(i, JF_IMP2);
    float i3 = R.getf(i, JF_IMP3), i4 = R.getf(i, JF_IMP4), mi = R.getf(i, JF_MIMP);
    const float maximp = R.getf(i, JF_MAXIMP), mspeed = R.getf(i, JF_MSPEED), mmass = R.getf(i, JF_MMASS);
    // the revolute fields load with the rest, in one batch (a branch would serialize them behind it)
    const V2 jrA = R.get2(i, JF_RA), jrB = R.get2(i, JF_RB);
    const float jangle = R.getf(i, JF_ANGLE), jinv_dt = R.getf(i, JF_INVDT);
    const float jlower = R.getf(i, JF_LOWER), jupper = R.getf(i, JF_UPPER);
    V2 vA = bd.v(ia), vB = bd.v(ib);
    float wA = bd.w(ia), wB = bd.w(ib);
    if (type == GOI_REVOLUTE) {
        const V2 rA = jrA, rB = jrB;
        const bool fixed = (iA + iB) == 0.0f;
        if (v24) {
            if (emotor && !fixed) {
                float impulse = -mmass * ((wB - wA) - mspeed);
                const float old = mi;
                mi = bclamp(mi + impulse, -maximp, maximp);
                impulse = mi - old;
                wA = wA - iA * impulse;
                wB = wB + iB * impulse;
            }
            if (elimit && !fixed) {
                const float angle = jangle, inv_dt = jinv_dt;
                float C = angle - jlower;
                float impulse = -mmass * ((wB - wA) + bmax(C, 0.0f) * inv_dt);
                float old = i3;
                i3 = bmax(i3 + impulse, 0.0f);
                impulse = i3 - old;
                wA = wA - iA * impulse;
                wB = wB + iB * impulse;
                C = jupper - angle;
                impulse = -mmass * ((wA - wB) + bmax(C, 0.0f) * inv_dt);
                old = i4;
                i4 = bmax(i4 + impulse, 0.0f);
                impulse = i4 - old;
                wA = wA + iA * impulse;
                wB = wB - iB * impulse;
            }
            const V2 p = solve22(ex.x, ey.x, ex.y, ey.y, -rel_vel(vB, wB, rB, vA, wA, rA));
            i0 = i0 + p.x;
            i1 = i1 + p.y;
            vA = vA - mA * p; wA = wA - iA * cross(rA, p);
            vB = vB + mB * p; wB = wB + iB * cross(rB, p);
        } else {
            if (emotor && st != kEqual && !fixed) {
                float impulse = -mmass * ((wB - wA) - mspeed);
                const float old = mi;
                mi = bclamp(mi + impulse, -maximp, maximp);
                impulse = mi - old;
                wA = wA - iA * impulse;
                wB = wB + iB * impulse;
            }
            const V2 c1 = rel_vel(vB, wB, rB, vA, wA, rA);
            if (elimit && st != kInactive && !fixed) {
                const V3 sv = solve33(ex, ey, ez, mk3(c1.x, c1.y, wB - wA));
                V3 j = mk3(-sv.x, -sv.y, -sv.z);
                const float nz = i2 + j.z;
                if ((st == kAtLower && nz < 0.0f) || (st == kAtUpper && nz > 0.0f)) {
                    const V2 red = solve22(ex.x, ey.x, ex.y, ey.y, mk(-c1.x + i2 * ez.x, -c1.y + i2 * ez.y));
                    j = mk3(red.x, red.y, -i2);
                    i0 = i0 + red.x; i1 = i1 + red.y; i2 = 0.0f;
                } else {
                    i0 = i0 + j.x; i1 = i1 + j.y; i2 = i2 + j.z;
                }
                const V2 P = mk(j.x, j.y);
                vA = vA - mA * P; wA = wA - iA * (cross(rA, P) + j.z);
                vB = vB + mB * P; wB = wB + iB * (cross(rB, P) + j.z);
            } else {
                const V2 p = solve22(ex.x, ey.x, ex.y, ey.y, -c1);
                i0 = i0 + p.x; i1 = i1 + p.y;
                vA = vA - mA * p; wA = wA - iA * cross(rA, p);
                vB = vB + mB * p; wB = wB + iB * cross(rB, p);
            }
        }
    } else if (type == GOI_PRISMATIC) {
        const V2 axis = R.get2(i, JF_AX), perp = R.get2(i, JF_PX);
        const float a1 = R.getf(i, JF_A1), a2 = R.getf(i, JF_A2), s1 = R.getf(i, JF_S1), s2 = R.getf(i, JF_S2);
        if (emotor && st != kEqual) {
            const float cdot = (dot(axis, vB - vA) + a2 * wB) - a1 * wA;
            float impulse = mmass * (mspeed - cdot);
            const float old = mi;
            mi = bclamp(mi + impulse, -maximp, maximp);
            impulse = mi - old;
            const V2 P = impulse * axis;
            vA = vA - mA * P; wA = wA - iA * (impulse * a1);
            vB = vB + mB * P; wB = wB + iB * (impulse * a2);
        }
        const float c1x = (dot(perp, vB - vA) + s2 * wB) - s1 * wA;
        const float c1y = wB - wA;
        if (elimit && st != kInactive) {
            const float c2 = (dot(axis, vB - vA) + a2 * wB) - a1 * wA;
            const float f1x = i0, f1y = i1, f1z = i2;
            const V3 df = solve33(ex, ey, ez, mk3(-c1x, -c1y, -c2));
            float nz = f1z + df.z;
            if (st == kAtLower) nz = bmax(nz, 0.0f);
            else if (st == kAtUpper) nz = bmin(nz, 0.0f);
            const V2 b = mk(-c1x - (nz - f1z) * ez.x, -c1y - (nz - f1z) * ez.y);
            V2 f2 = solve22(ex.x, ey.x, ex.y, ey.y, b);
            f2 = mk(f2.x + f1x, f2.y + f1y);
            i0 = f2.x; i1 = f2.y; i2 = nz;
            const float dfx = f2.x - f1x, dfy = f2.y - f1y, dfz = nz - f1z;
            const V2 P = dfx * perp + dfz * axis;
            const float LA = (dfx * s1 + dfy) + dfz * a1;
            const float LB = (dfx * s2 + dfy) + dfz * a2;
            vA = vA - mA * P; wA = wA - iA * LA;
            vB = vB + mB * P; wB = wB + iB * LB;
        } else {
            const V2 df = solve22(ex.x, ey.x, ex.y, ey.y, mk(-c1x, -c1y));
            i0 = i0 + df.x; i1 = i1 + df.y;
            const V2 P = df.x * perp;
            const float LA = df.x * s1 + df.y, LB = df.x * s2 + df.y;
            vA = vA - mA * P; wA = wA - iA * LA;
            vB = vB + mB * P; wB = wB + iB * LB;
        }
    } else {  // weld
        const V2 rA = R.get2(i, JF_RA), rB = R.get2(i, JF_RB);
        if (R.geti(i, JF_SOFT)) {
            const float imp2 = -ez.z * (((wB - wA) + R.getf(i, JF_BIAS)) + R.getf(i, JF_GAMMA) * i2);
            i2 = i2 + imp2;
            wA = wA - iA * imp2;
            wB = wB + iB * imp2;
            const V2 c1 = rel_vel(vB, wB, rB, vA, wA, rA);
            const V2 i1v = mk(-(ex.x * c1.x + ey.x * c1.y), -(ex.y * c1.x + ey.y * c1.y));
            i0 = i0 + i1v.x; i1 = i1 + i1v.y;
            vA = vA - mA * i1v; wA = wA - iA * cross(rA, i1v);
            vB = vB + mB * i1v; wB = wB + iB * cross(rB, i1v);
        } else {
            const V2 c1 = rel_vel(vB, wB, rB, vA, wA, rA);
            const float c2 = wB - wA;
            const float jx = -((c1.x * ex.x + c1.y * ey.x) + c2 * ez.x);
            const float jy = -((c1.x * ex.y + c1.y * ey.y) + c2 * ez.y);
            const float jz = -((c1.x * ex.z + c1.y * ey.z) + c2 * ez.z);
            i0 = i0 + jx; i1 = i1 + jy; i2 = i2 + jz;
            const V2 P = mk(jx, jy);
            vA = vA - mA * P; wA = wA - iA * (cross(rA, P) + jz);
            vB = vB + mB * P; wB = wB + iB * (cross(rB, P) + jz);
        }
    }
    R.setf(i, JF_IMP0, i0); R.setf(i, JF_IMP1, i1); R.setf(i, JF_IMP2, i2);
    R.setf(i, JF_IMP3, i3); R.setf(i, JF_IMP4, i4); R.setf(i, JF_MIMP, mi);
    bd.set_v(ia, vA, wA);
    bd.set_v(ib, vB, wB);
}

// A revolute joint's velocity-solve fields for the v2.4.1 solver (revolute24.patch:166-240), loaded in one batch.
// A revolute-only model's joint passes load joint i + 1's row while joint i is solved (rev_velocity_sweep); the
// operations are those of jn_solve_velocity's v2.4.1 revolute branch.
struct RevVRow {
    int ia, ib;
    bool emotor, elimit;
    float mA, mB, iA, iB, k11, k12, k21, k22, i0, i1, i3, i4, mi, maximp, mspeed, mmass, angle, inv_dt, lower, upper;
    V2 rA, rB;
};
GOI_D RevVRow load_rev_vrow(const Rows& R, int i) {
    RevVRow r;
    r.ia = R.geti(i, JF_IA); r.ib = R.geti(i, JF_IB);
    r.emotor = R.geti(i, JF_EMOTOR) != 0; r.elimit = R.geti(i, JF_ELIMIT) != 0;
    r.mA = R.getf(i, JF_MA); r.mB = R.getf(i, JF_MB); r.iA = R.getf(i, JF_IIA); r.iB = R.getf(i, JF_IIB);
    r.k11 = R.getf(i, JF_EXX); r.k21 = R.getf(i, JF_EXX + 1); r.k12 = R.getf(i, JF_EYX); r.k22 = R.getf(i, JF_EYX + 1);
    r.i0 = R.getf(i, JF_IMP0); r.i1 = R.getf(i, JF_IMP1); r.i3 = R.getf(i, JF_IMP3); r.i4 = R.getf(i, JF_IMP4);
    r.mi = R.getf(i, JF_MIMP);
    r.maximp = R.getf(i, JF_MAXIMP); r.mspeed = R.getf(i, JF_MSPEED); r.mmass = R.getf(i, JF_MMASS);
    r.rA = R.get2(i, JF_RA); r.rB = R.get2(i, JF_RB);
    r.angle = R.getf(i, JF_ANGLE); r.inv_dt = R.getf(i, JF_INVDT);
    r.lower = R.getf(i, JF_LOWER); r.upper = R.getf(i, JF_UPPER);
    return r;
}
template <class BD>
GOI_D void solve_rev_vrow(const BD& bd, RevVRow& r) {
    V2 vA = bd.v(r.ia), vB = bd.v(r.ib);
    float wA = bd.w(r.ia), wB = bd.w(r.ib);
    const float mA = r.mA, mB = r.mB, iA = r.iA, iB = r.iB;
    const bool fixed = (iA + iB) == 0.0f;
    if (r.emotor && !fixed) {
        float impulse = -r.mmass * ((wB - wA) - r.mspeed);
        const float old = r.mi;
        r.mi = bclamp(r.mi + impulse, -r.maximp, r.maximp);
        impulse = r.mi - old;
        wA = wA - iA * impulse;
        wB = wB + iB * impulse;
    }
    if (r.elimit && !fixed) {
        float C = r.angle - r.lower;
        float impulse = -r.mmass * ((wB - wA) + bmax(C, 0.0f) * r.inv_dt);
        float old = r.i3;
        r.i3 = bmax(r.i3 + impulse, 0.0f);
        impulse = r.i3 - old;
        wA = wA - iA * impulse;
        wB = wB + iB * impulse;
        C = r.upper - r.angle;
        impulse = -r.mmass * ((wA - wB) + bmax(C, 0.0f) * r.inv_dt);
        old = r.i4;
        r.i4 = bmax(r.i4 + impulse, 0.0f);
        impulse = r.i4 - old;
        wA = wA + iA * impulse;
        wB = wB - iB * impulse;
    }
    const V2 p = solve22(r.k11, r.k12, r.k21, r.k22, -rel_vel(vB, wB, r.rB, vA, wA, r.rA));
    r.i0 = r.i0 + p.x;
    r.i1 = r.i1 + p.y;
    vA = vA - mA * p; wA = wA - iA * cross(r.rA, p);
    vB = vB + mB * p; wB = wB + iB * cross(r.rB, p);
    bd.set_v(r.ia, vA, wA);
    bd.set_v(r.ib, vB, wB);
}
// the impulses the solve changes (the revolute v2.4.1 branch leaves impulse z as it is)
GOI_D void store_rev_impulses(const Rows& R, int i, const RevVRow& r) {
    R.setf(i, JF_IMP0, r.i0); R.setf(i, JF_IMP1, r.i1);
    R.setf(i, JF_IMP3, r.i3); R.setf(i, JF_IMP4, r.i4); R.setf(i, JF_MIMP, r.mi);
}
// joint rows i0..n-1 of a revolute-only model under the v2.4.1 solver, once each, in order
template <class BD>
GOI_D void rev_velocity_sweep(const BD& bd, const Rows& R, int i0, int n) {
    if (n <= i0) return;
    RevVRow a = load_rev_vrow(R, i0), b;
    for (int i = i0; i < n; i += 2) {  // as cs_solve_velocity_sweep: joint i + 1 in flight while joint i is solved
        if (i + 1 < n) b = load_rev_vrow(R, i + 1);
        solve_rev_vrow(bd, a);
        store_rev_impulses(R, i, a);
        if (i + 1 >= n) break;
        if (i + 2 < n) a = load_rev_vrow(R, i + 2);
        solve_rev_vrow(bd, b);
        store_rev_impulses(R, i + 1, b);
    }
}

// the point part of the revolute position solve (joints.py:501-520)
GOI_D bool rev_point(float mA, float mB, float iA, float iB, V2 la, V2 lb, V2& cA, float& aA, V2& cB, float& aB,
                     float ang_err, const GoiSettings& s) {
    const V2 rA = mul(rot_of(aA), la), rB = mul(rot_of(aB), lb);
    const V2 C = ((cB + rB) - cA) - rA;
    const float pos_err = length(C);
    const float kxx = ((mA + mB) + iA * rA.y * rA.y) + iB * rB.y * rB.y;
    const float kxy = -iA * rA.x * rA.y - iB * rB.x * rB.y;
    const float kyy = ((mA + mB) + iA * rA.x * rA.x) + iB * rB.x * rB.x;
    const V2 j = -solve22(kxx, kxy, kxy, kyy, C);
    cA = cA - mA * j; aA = aA - iA * cross(rA, j);
    cB = cB + mB * j; aB = aB + iB * cross(rB, j);
    return pos_err <= s.linear_slop && ang_err <= s.angular_slop;
}

// SolvePositionConstraints for joint row i (joints.py:462-606); returns the joint's ok flag
template <class BD>
GOI_D bool jn_solve_position(const BD& bd, const Rows& R, int i, const GoiSettings& s, bool rev_only) {
    const int type = rev_only ? (int)GOI_REVOLUTE : R.geti(i, JF_TYPE), ia = R.geti(i, JF_IA), ib = R.geti(i, JF_IB);
    const float mA = R.getf(i, JF_MA), mB = R.getf(i, JF_MB), iA = R.getf(i, JF_IIA), iB = R.getf(i, JF_IIB);
    const bool elimit = R.geti(i, JF_ELIMIT) != 0;
    const float lower = R.getf(i, JF_LOWER), upper = R.getf(i, JF_UPPER), ref = R.getf(i, JF_REF);
    // the revolute fields load with the rest, in one batch
    const float jmmass = R.getf(i, JF_MMASS);
    const int jst = R.geti(i, JF_STATE);
    const V2 jla = R.get2(i, JF_LA), jlb = R.get2(i, JF_LB);
    const float mac = s.max_angular_correction;
    V2 cA = bd.c(ia), cB = bd.c(ib);
    float aA = bd.a(ia), aB = bd.a(ib);
    bool ok;
    if (type == GOI_REVOLUTE) {
        const bool fixed = (iA + iB) == 0.0f;
        const float mmass = jmmass;
        float ang_err = 0.0f;
        if (s.revolute_v24) {
            if (elimit && !fixed) {
                const float angle = (aB - aA) - ref;
                float C = 0.0f;
                if (babs(upper - lower) < 2.0f * s.angular_slop) C = bclamp(angle - lower, -mac, mac);
                else if (angle <= lower) C = bclamp((angle - lower) + s.angular_slop, -mac, 0.0f);
                else if (angle >= upper) C = bclamp((angle - upper) - s.angular_slop, 0.0f, mac);
                const float li = -mmass * C;
                aA = aA - iA * li;
                aB = aB + iB * li;
                ang_err = babs(C);
            }
        } else {
            const int st = jst;
            if (elimit && st != kInactive && !fixed) {
                const float angle = (aB - aA) - ref;
                float li;
                if (st == kEqual) {
                    const float C = bclamp(angle - lower, -mac, mac);
                    li = -mmass * C;
                    ang_err = babs(C);
                } else if (st == kAtLower) {
                    float C = angle - lower;
                    ang_err = -C;
                    C = bclamp(C + s.angular_slop, -mac, 0.0f);
                    li = -mmass * C;
                } else {
                    float C = angle - upper;
                    ang_err = C;
                    C = bclamp(C - s.angular_slop, 0.0f, mac);
                    li = -mmass * C;
                }
                aA = aA - iA * li;
                aB = aB + iB * li;
            }
        }
        ok = rev_point(mA, mB, iA, iB, jla, jlb, cA, aA, cB, aB, ang_err, s);
    } else if (type == GOI_PRISMATIC) {
        const Rot qA = rot_of(aA), qB = rot_of(aB);
        const V2 rA = mul(qA, R.get2(i, JF_LA)), rB = mul(qB, R.get2(i, JF_LB));
        const V2 d = ((cB + rB) - cA) - rA;
        const V2 axis = mul(qA, R.get2(i, JF_LX));
        const float a1 = cross(d + rA, axis), a2 = cross(rB, axis);
        const V2 perp = mul(qA, R.get2(i, JF_LY));
        const float s1 = cross(d + rA, perp), s2 = cross(rB, perp);
        const float c1x = dot(perp, d), c1y = (aB - aA) - ref;
        float lin_err = babs(c1x);
        const float ang_err = babs(c1y);
        bool active = false;
        float C2 = 0.0f;
        const float mlc = s.max_linear_correction;
        if (elimit) {
            const float t = dot(axis, d);
            if (babs(upper - lower) < 2.0f * s.linear_slop) {
                C2 = bclamp(t, -mlc, mlc); lin_err = bmax(lin_err, babs(t)); active = true;
            } else if (t <= lower) {
                C2 = bclamp((t - lower) + s.linear_slop, -mlc, 0.0f); lin_err = bmax(lin_err, lower - t); active = true;
            } else if (t >= upper) {
                C2 = bclamp((t - upper) - s.linear_slop, 0.0f, mlc); lin_err = bmax(lin_err, t - upper); active = true;
            }
        }
        const float k11 = ((mA + mB) + iA * s1 * s1) + iB * s2 * s2;
        const float k12 = iA * s1 + iB * s2;
        float k22 = iA + iB;
        if (k22 == 0.0f) k22 = 1.0f;
        V3 imp;
        if (active) {
            const float k13 = iA * s1 * a1 + iB * s2 * a2;
            const float k23 = iA * a1 + iB * a2;
            const float k33 = ((mA + mB) + iA * a1 * a1) + iB * a2 * a2;
            imp = solve33(mk3(k11, k12, k13), mk3(k12, k22, k23), mk3(k13, k23, k33), mk3(-c1x, -c1y, -C2));
        } else {
            const V2 i2 = solve22(k11, k12, k12, k22, mk(-c1x, -c1y));
            imp = mk3(i2.x, i2.y, 0.0f);
        }
        const V2 P = imp.x * perp + imp.z * axis;
        const float LA = (imp.x * s1 + imp.y) + imp.z * a1;
        const float LB = (imp.x * s2 + imp.y) + imp.z * a2;
        cA = cA - mA * P; aA = aA - iA * LA;
        cB = cB + mB * P; aB = aB + iB * LB;
        ok = lin_err <= s.linear_slop && ang_err <= s.angular_slop;
    } else {  // weld
        const V2 rA = mul(rot_of(aA), R.get2(i, JF_LA)), rB = mul(rot_of(aB), R.get2(i, JF_LB));
        const float exx = ((mA + mB) + rA.y * rA.y * iA) + rB.y * rB.y * iB;
        const float eyx = -rA.y * rA.x * iA - rB.y * rB.x * iB;
        const float ezx = -rA.y * iA - rB.y * iB;
        const float eyy = ((mA + mB) + rA.x * rA.x * iA) + rB.x * rB.x * iB;
        const float ezy = rA.x * iA + rB.x * iB;
        const float ezz = iA + iB;
        const V3 ex = mk3(exx, eyx, ezx), ey = mk3(eyx, eyy, ezy), ez = mk3(ezx, ezy, ezz);
        const V2 C1 = ((cB + rB) - cA) - rA;
        const float pos_err = length(C1);
        float ang_err;
        if (R.geti(i, JF_SOFT)) {
            ang_err = 0.0f;
            const V2 P = -solve22(ex.x, ey.x, ex.y, ey.y, C1);
            cA = cA - mA * P; aA = aA - iA * cross(rA, P);
            cB = cB + mB * P; aB = aB + iB * cross(rB, P);
        } else {
            const float C2 = (aB - aA) - ref;
            ang_err = babs(C2);
            V3 imp;
            if (ez.z > 0.0f) {
                const V3 p = solve33(ex, ey, ez, mk3(C1.x, C1.y, C2));
                imp = mk3(-p.x, -p.y, -p.z);
            } else {
                const V2 p = solve22(ex.x, ey.x, ex.y, ey.y, C1);
                imp = mk3(-p.x, -p.y, 0.0f);
            }
            const V2 P = mk(imp.x, imp.y);
            cA = cA - mA * P; aA = aA - iA * (cross(rA, P) + imp.z);
            cB = cB + mB * P; aB = aB + iB * (cross(rB, P) + imp.z);
        }
        ok = pos_err <= s.linear_slop && ang_err <= s.angular_slop;
    }
    bd.set_c(ia, cA, aA);
    bd.set_c(ib, cB, aB);
    return ok;
}

GOI_D void jn_store(const World& W, const Rows& R, int i, bool v24) {
    const int j = R.geti(i, JF_JID);
    W.f(GOI_J_IMPULSE, 3 * j) = R.getf(i, JF_IMP0);
    W.f(GOI_J_IMPULSE, 3 * j + 1) = R.getf(i, JF_IMP1);
    W.f(GOI_J_IMPULSE, 3 * j + 2) = R.getf(i, JF_IMP2);
    W.f(GOI_J_MOTOR_IMPULSE, j) = R.getf(i, JF_MIMP);
    W.i32(GOI_J_LIMIT_STATE, j) = R.geti(i, JF_STATE);
    if (v24) {
        W.f(GOI_J_LOWER_IMPULSE, j) = R.getf(i, JF_IMP3);
        W.f(GOI_J_UPPER_IMPULSE, j) = R.getf(i, JF_IMP4);
    }
}

}  // namespace goi
