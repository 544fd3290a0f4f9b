// b2_math.hpp - float32 b2Math for gfx950 device code, one rounding per C operation in C order.
//
// The whole library is compiled with -ffp-contract=off (no FMA contraction), IEEE-correct division and square root,
// and f32 denormals kept, so every expression below rounds exactly as Box2D 2.3.1 built with -ffp-contract=off does
// (goi_jax/box2d/math2d.py:1-13, scripts/build_box2d.sh:11). C's `a + b + c` is `(a + b) + c`; products are written
// in the source order of b2Math.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define GOI_D __device__ __forceinline__
#define GOI_HD __host__ __device__ __forceinline__

namespace goi {

constexpr float kEps = 1.1920928955078125e-7f;       // b2_epsilon
constexpr float kMaxFloat = 3.40282346638528859812e+38f;  // b2_maxFloat
constexpr float kPi = 3.14159265359f;                // b2_pi
constexpr int kMaxSubSteps = 8;
constexpr int kMaxToiContacts = 32;
constexpr int kPoly = 8;

struct V2 { float x, y; };
struct Rot { float c, s; };
struct Xf { V2 p; Rot q; };
struct V3 { float x, y, z; };

GOI_D V2 mk(float x, float y) { V2 r; r.x = x; r.y = y; return r; }
GOI_D V3 mk3(float x, float y, float z) { V3 r; r.x = x; r.y = y; r.z = z; return r; }
GOI_D V2 operator+(V2 a, V2 b) { return mk(a.x + b.x, a.y + b.y); }
GOI_D V2 operator-(V2 a, V2 b) { return mk(a.x - b.x, a.y - b.y); }
GOI_D V2 operator-(V2 a) { return mk(-a.x, -a.y); }
GOI_D V2 operator*(float s, V2 a) { return mk(s * a.x, s * a.y); }
GOI_D float dot(V2 a, V2 b) { return a.x * b.x + a.y * b.y; }
GOI_D float cross(V2 a, V2 b) { return a.x * b.y - a.y * b.x; }
GOI_D V2 cross(V2 a, float s) { return mk(s * a.y, -s * a.x); }
GOI_D V2 cross(float s, V2 a) { return mk(-s * a.y, s * a.x); }
GOI_D V2 mul(Rot q, V2 v) { return mk(q.c * v.x - q.s * v.y, q.s * v.x + q.c * v.y); }
GOI_D V2 mulT(Rot q, V2 v) { return mk(q.c * v.x + q.s * v.y, -q.s * v.x + q.c * v.y); }
GOI_D V2 mul(const Xf& t, V2 v) { return mk((t.q.c * v.x - t.q.s * v.y) + t.p.x, (t.q.s * v.x + t.q.c * v.y) + t.p.y); }
GOI_D V2 mulT(const Xf& t, V2 v) {
    float px = v.x - t.p.x, py = v.y - t.p.y;
    return mk(t.q.c * px + t.q.s * py, -t.q.s * px + t.q.c * py);
}
GOI_D Xf mulT(const Xf& A, const Xf& B) {
    Xf C;
    C.q.s = A.q.c * B.q.s - A.q.s * B.q.c;
    C.q.c = A.q.c * B.q.c + A.q.s * B.q.s;
    C.p = mulT(A.q, B.p - A.p);
    return C;
}
GOI_D float length(V2 a) { return sqrtf(a.x * a.x + a.y * a.y); }
// b2Vec2::Normalize: unchanged below b2_epsilon
GOI_D float normalize(V2& a) {
    float n = length(a);
    if (n < kEps) return 0.0f;
    float inv = 1.0f / n;
    a.x *= inv;
    a.y *= inv;
    return n;
}
GOI_D float bmin(float a, float b) { return a < b ? a : b; }   // b2Min keeps b on ties and NaN
GOI_D float bmax(float a, float b) { return a > b ? a : b; }
GOI_D float bclamp(float a, float lo, float hi) { return bmax(lo, bmin(a, hi)); }
GOI_D float babs(float a) { return a > 0.0f ? a : -a; }
GOI_D float fdiv(float a, float b) { return a / b; }
GOI_D float fsqrt(float a) { return sqrtf(a); }  // IEEE sqrt under -fhip-fp32-correctly-rounded-divide-sqrt

// The library's double sin/cos, out of line: only angles of magnitude 2^20 and above, infinities and NaN take it.
__device__ __noinline__ double2 sincos_lib(double x) {
    double s, c;
    sincos(x, &s, &c);
    return make_double2(s, c);
}

// Correctly rounded float32 sin/cos: (float)sin((double)x), the value the reference computes with a float-float
// series (math2d.py:291-310) and its oracle with the C library (scripts/patches/box2d-2.3.1-trig.patch:17-23).
// Evaluated on the FP64 units: the double result is within about an ulp of the exact value, so rounding it to float
// gives the correctly rounded float except when sin x lies within ~2^-52 relative of a float rounding boundary.
//
// Method (Cody and Waite's additive range reduction, then Taylor series): k = nearest integer to x * 2/pi and
// r = x - k * pi/2 with pi/2 split into three doubles, each step one fused multiply-add (exact for the first part,
// since x and k * P1 agree in their leading bits; then one rounding of the exact remainder per part, so r keeps about
// an ulp of relative accuracy even when x is close to a multiple of pi/2); on |r| <= pi/4 the series of sin to r^17
// and of cos to r^16 (truncation below 2^-62 relative) by Horner's rule in fused multiply-adds; the quadrant k mod 4
// picks and signs the pair. Inline everywhere (about 30 double operations); |x| >= 2^20 calls the library. Checked
// bit for bit against (float)sin((double)x) of the C library on 24M inputs over +-8 .. +-1e6 and sweeps of every
// exponent (no difference), and by the known-answer test on the device.
GOI_D Rot rot_of(float a) {
    Rot q;
    if (a == 0.0f) {  // a static body at its rest angle, the common case; sin(+-0) = +-0, cos = 1
        q.s = a;
        q.c = 1.0f;
        return q;
    }
    const double x = (double)a;
    double s, c;
    if (!(fabs(x) < 1048576.0)) {
        const double2 sc = sincos_lib(x);
        s = sc.x;
        c = sc.y;
    } else {
        constexpr double kTwoOverPi = 0x1.45f306dc9c883p-1;
        constexpr double kP1 = 0x1.921fb54442d18p+0, kP2 = 0x1.1a62633145c07p-54, kP3 = -0x1.f1976b7ed8fbcp-110;
        const double k = rint(x * kTwoOverPi);
        double r = fma(-k, kP1, x);
        r = fma(-k, kP2, r);
        r = fma(-k, kP3, r);
        const double r2 = r * r;
        // sin r = r + r^3 (-1/3! + r^2 (1/5! - ...)), cos r = 1 + r^2 (-1/2! + r^2 (1/4! - ...)): coefficients 1/n!
        double ps = 0x1.952c77030ad4ap-49;           //  1/17!
        ps = fma(ps, r2, -0x1.ae7f3e733b81fp-41);    // -1/15!
        ps = fma(ps, r2, 0x1.6124613a86d09p-33);     //  1/13!
        ps = fma(ps, r2, -0x1.ae64567f544e4p-26);    // -1/11!
        ps = fma(ps, r2, 0x1.71de3a556c734p-19);     //  1/9!
        ps = fma(ps, r2, -0x1.a01a01a01a01ap-13);    // -1/7!
        ps = fma(ps, r2, 0x1.1111111111111p-7);      //  1/5!
        ps = fma(ps, r2, -0x1.5555555555555p-3);     // -1/3!
        double pc = 0x1.ae7f3e733b81fp-45;           //  1/16!
        pc = fma(pc, r2, -0x1.93974a8c07c9dp-37);    // -1/14!
        pc = fma(pc, r2, 0x1.1eed8eff8d898p-29);     //  1/12!
        pc = fma(pc, r2, -0x1.27e4fb7789f5cp-22);    // -1/10!
        pc = fma(pc, r2, 0x1.a01a01a01a01ap-16);     //  1/8!
        pc = fma(pc, r2, -0x1.6c16c16c16c17p-10);    // -1/6!
        pc = fma(pc, r2, 0x1.5555555555555p-5);      //  1/4!
        pc = fma(pc, r2, -0.5);                      // -1/2!
        const double sr = fma(r * r2, ps, r), cr = fma(r2, pc, 1.0);
        const int qd = (int)k & 3;
        s = (qd & 1) ? cr : sr;
        c = (qd & 1) ? sr : cr;
        if (qd == 1 || qd == 2) c = -c;
        if (qd >= 2) s = -s;
    }
    q.s = (float)s;
    q.c = (float)c;
    return q;
}

// One remembered rotation. sin/cos are pure functions of the angle's bits, so an angle met again (bit for bit)
// reuses the rotation computed for it: the terrain's constant angle in the position solver and in b2TimeOfImpact's
// sweeps, and a body angle that a zero impulse left unchanged. The initial key is a NaN payload (all ones) that
// arithmetic never generates (generated NaNs are 0x7fc00000); its rotation is NaN, as rot_of's would be.
struct RotMemo {
    uint32_t bits = 0x7fffffffu;
    Rot q{__uint_as_float(0x7fffffffu), __uint_as_float(0x7fffffffu)};
    GOI_D Rot of(float a) {
        const uint32_t b = __float_as_uint(a);
        if (b != bits) {
            q = rot_of(a);
            bits = b;
        }
        return q;
    }
};

// ---- lane groups
//
// The lanes that run one world together: a group of G consecutive lanes (G a power of two, aligned to G), every lane
// on the same data. A loop over a shape's vertices splits over the group (lane `sub` takes i = sub, sub + G, ...), and
// a reduction over the group gives every lane the result of the sequential loop. Solo is the one-lane case (a
// block-cooperative task), for which the split loop is the plain loop and the reductions vanish.
struct Solo {
    GOI_D int sub() const { return 0; }
    GOI_D int G() const { return 1; }
};
struct Group {
    int s, g;
    GOI_D int sub() const { return s; }
    GOI_D int G() const { return g; }
};

template <class Grp>
GOI_D int group_max(const Grp& g, int x) {
    for (int d = 1; d < g.G(); d <<= 1) x = max(x, __shfl_xor(x, d, 64));
    return x;
}
template <class Grp>
GOI_D int group_sum(const Grp& g, int x) {
    for (int d = 1; d < g.G(); d <<= 1) x += __shfl_xor(x, d, 64);
    return x;
}
template <class Grp>
GOI_D unsigned long long group_or(const Grp& g, unsigned long long x) {
    for (int d = 1; d < g.G(); d <<= 1) {
        const unsigned lo = __shfl_xor((unsigned)x, d, 64), hi = __shfl_xor((unsigned)(x >> 32), d, 64);
        x |= ((unsigned long long)hi << 32) | lo;
    }
    return x;
}

// Orders the memory accesses of a lane group: what one lane of the wavefront wrote before it (global or LDS) is
// what every lane reads after it. The lanes of a wavefront execute in lockstep, so this only keeps the compiler from
// moving accesses across it.
GOI_D void group_sync() { __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront"); }

// The sequential running maximum `if (v > best) { best = v; at = i; }` over i in ascending order, started from
// (best, at), equals the group's combination of each lane's running maximum over its own indices (started from the
// same (best, at)) when a larger value wins and equal values keep the smaller index: NaN never wins (its compares
// are false), and among equal maxima the first index is the sequential winner. Same for the minimum.
template <class Grp>
GOI_D void group_argmax(const Grp& g, float& v, int& at) {
    for (int d = 1; d < g.G(); d <<= 1) {
        const float ov = __shfl_xor(v, d, 64);
        const int oi = __shfl_xor(at, d, 64);
        if (ov > v || (ov == v && oi < at)) {
            v = ov;
            at = oi;
        }
    }
}
template <class Grp>
GOI_D void group_argmin(const Grp& g, float& v, int& at) {
    for (int d = 1; d < g.G(); d <<= 1) {
        const float ov = __shfl_xor(v, d, 64);
        const int oi = __shfl_xor(at, d, 64);
        if (ov < v || (ov == v && oi < at)) {
            v = ov;
            at = oi;
        }
    }
}
template <class Grp>
GOI_D bool group_any(const Grp& g, bool p) {
    int x = p ? 1 : 0;
    for (int d = 1; d < g.G(); d <<= 1) x |= __shfl_xor(x, d, 64);
    return x != 0;
}

// b2Mat22::Solve / b2Mat33::Solve22
GOI_D V2 solve22(float a11, float a12, float a21, float a22, V2 b) {
    float det = a11 * a22 - a12 * a21;
    if (det != 0.0f) det = fdiv(1.0f, det);
    return mk(det * (a22 * b.x - a12 * b.y), det * (a11 * b.y - a21 * b.x));
}
GOI_D float dot(V3 a, V3 b) { return (a.x * b.x + a.y * b.y) + a.z * b.z; }
GOI_D V3 cross(V3 a, V3 b) { return mk3(a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x); }
// b2Mat33::Solve33 with columns ex, ey, ez
GOI_D V3 solve33(V3 ex, V3 ey, V3 ez, V3 b) {
    float det = dot(ex, cross(ey, ez));
    if (det != 0.0f) det = fdiv(1.0f, det);
    return mk3(det * dot(b, cross(ey, ez)), det * dot(ex, cross(b, ez)), det * dot(ex, cross(ey, b)));
}

}  // namespace goi
