// b2_math.hpp - float32 b2Math for gfx950 device code, one rounding per C operation in C order.
//
// The whole library is compiled with -ffp-contract=off (no FMA contraction), IEEE-correct division and square root,
// and f32 denormals kept, so every expression below rounds exactly as Box2D 2.3.1 built with -ffp-contract=off does
// (goi_jax/box2d/math2d.py:1-13, scripts/build_box2d.sh:11). C's `a + b + c` is `(a + b) + c`; products are written
// in the source order of b2Math.h.
#pragma once

#ifdef GOI_HOST_BUILD
#include "host_shim.hpp"  // the sequential host build (tests): host definitions of the HIP surface used below
#else
#include <hip/hip_runtime.h>
#endif
#include <stdint.h>

#include "b2_sincos_table.h"

#define GOI_D __device__ __forceinline__
#define GOI_HD __host__ __device__ __forceinline__

namespace goi {

constexpr float kEps = 1.1920928955078125e-7f;       // b2_epsilon
constexpr float kMaxFloat = 3.40282346638528859812e+38f;  // b2_maxFloat
constexpr float kNaN = __builtin_nanf("");
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
static __device__ __noinline__ double2 sincos_lib(double x) {
    double s, c;
    sincos(x, &s, &c);
    return make_double2(s, c);
}

// sin(j pi/32), cos(j pi/32) for j = 0..63 (b2_sincos_table.h), and the block's copy in LDS, which every kernel that
// evaluates rot_of loads first (sincos_table_load).
__device__ const double kSinCosTable[128] = {GOI_SINCOS_TABLE};
#ifdef GOI_HOST_BUILD
inline
#endif
__shared__ __align__(16) double g_sincos_lds[128];

// This lane's index in its wavefront (a block is one wavefront), read from the hardware at the call: a fresh value,
// not one carried from earlier code (the mask goes through an empty asm statement, so the compiler recomputes the
// count at every call instead of reusing an earlier one).
GOI_D int lane_now() {
#ifdef GOI_HOST_BUILD
    return (int)threadIdx.x;
#else
    unsigned mask = ~0u;
    asm volatile("" : "+s"(mask));
    return (int)__builtin_amdgcn_mbcnt_hi(mask, __builtin_amdgcn_mbcnt_lo(mask, 0u));
#endif
}

// A clock for timing a block's work (the GPU's constant-rate real-time counter; 0 in the host build); nothing the step
// computes depends on it.
GOI_D uint64_t block_clock() {
#ifdef GOI_HOST_BUILD
    return 0;
#else
    return __builtin_amdgcn_s_memrealtime();
#endif
}

// The wave's instruction-issue priority among the waves of its SIMD (0 to 3); nothing else depends on it.
template <int kPrio>
GOI_D void wave_priority() {
#ifndef GOI_HOST_BUILD
    __builtin_amdgcn_s_setprio(kPrio);
#endif
}

// v itself, as a value the compiler cannot see through: what is computed from it after this point is computed there,
// not earlier (a multi-step loop then holds no per-lane address of one step across the next).
GOI_D int opaque(int v) {
#ifndef GOI_HOST_BUILD
    asm volatile("" : "+v"(v));
#endif
    return v;
}

// Copies the table into the block's LDS; called by every lane of the block before its first rot_of.
GOI_D void sincos_table_load() {
#ifdef GOI_HOST_BUILD
    for (int i = 0; i < 128; ++i) g_sincos_lds[i] = kSinCosTable[i];  // threads run one after another there
#else
    for (int i = threadIdx.x; i < 128; i += blockDim.x) g_sincos_lds[i] = kSinCosTable[i];
    __syncthreads();
#endif
}

// Correctly rounded float32 sin/cos: (float)sin((double)x), the value the reference computes with a float-float
// series (math2d.py:291-310) and its oracle with the C library (scripts/patches/box2d-2.3.1-trig.patch:17-23).
//
// Method (constants in b2_sincos_table.h): k = nearest integer to x * 32/pi, r = x - k pi/32 by Cody and Waite's
// three-part reduction in fused multiply-adds (the first exact: x and k * P1 agree in their leading bits and the
// difference fits 53 bits for |x| < 2^20); short series of sin r and cos r - 1 on |r| <= pi/64; then the addition
// formulas with the tabulated St = sin(k pi/32), Ct = cos(k pi/32) (k mod 64), the table value added last:
// sin x = St + (St (cos r - 1) + Ct sin r), cos x = Ct + (Ct (cos r - 1) - St sin r). Rounded to float, the result
// equals the C library's (float)sin((double)x) and (float)cos((double)x) for every float with |x| < 2^20 (all
// 2 x 1.23e9 of them, checked by tests/sincos_check.c, which restates these operations on the CPU; the factored form
// St cos r + Ct sin r misses one). sin(-0) = -0 is kept by returning a zero angle itself. Angles of magnitude 2^20
// and above, infinities and NaN call the library's double sin/cos.
// sin x and cos x in double by the table method above, for |x| < 2^20. The table row, k mod 64, is the low bits of
// k + 1.5 * 2^52 (exact for |k| < 2^51); for any other x, infinities and NaN included, it is some row in 0 .. 63.
GOI_D void sincos_table(double x, double& s, double& c) {
    const double k = rint(x * GOI_SC_32_OVER_PI);
    const int row = (int)(__double_as_longlong(k + 6755399441055744.0) & 63);
    double r = fma(-k, GOI_SC_P1, x);
    r = fma(-k, GOI_SC_P2, r);
    r = fma(-k, GOI_SC_P3, r);
    const double r2 = r * r;
    double ps = GOI_SC_S9;
    ps = fma(ps, r2, GOI_SC_S7);
    ps = fma(ps, r2, GOI_SC_S5);
    ps = fma(ps, r2, GOI_SC_S3);
    double pc = GOI_SC_C8;
    pc = fma(pc, r2, GOI_SC_C6);
    pc = fma(pc, r2, GOI_SC_C4);
    pc = fma(pc, r2, GOI_SC_C2);
    const double sr = fma(r * r2, ps, r), cm1 = r2 * pc;
    const double2 t = reinterpret_cast<const double2*>(g_sincos_lds)[row];  // St, Ct
    s = t.x + fma(t.x, cm1, t.y * sr);
    c = t.y + fma(t.y, cm1, -(t.x * sr));
}

GOI_D Rot rot_of(float a) {
    const double x = (double)a;
    double s, c;
    if (!(fabs(x) < 1048576.0)) {
        const double2 sc = sincos_lib(x);
        s = sc.x;
        c = sc.y;
    } else {
        sincos_table(x, s, c);
    }
    Rot q;
    q.s = a == 0.0f ? a : (float)s;
    q.c = (float)c;
    return q;
}

// rot_of for an angle its caller checks to be below 2^20 in magnitude, without the branch to the library (a larger
// angle, an infinity or NaN gives some rotation, which the caller discards).
GOI_D Rot rot_of_small(float a) {
    double s, c;
    sincos_table((double)a, s, c);
    Rot q;
    q.s = a == 0.0f ? a : (float)s;
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

// The partner's value in round d (1, 2, 4, ...) of a lane group's butterfly. Groups are aligned runs of G lanes
// (G a power of two). Up to G = 16 the exchange is one DPP move inside the lane's row of 16: lanes i and i ^ 1, then
// i ^ 2 (quad permutes), then the mirror inside 8 lanes (i and 7 - i), then inside 16 (i and 15 - i). After the
// rounds below d every lane of an aligned run of d lanes holds that run's combination, so any pairing that joins two
// such runs completes the next level, and every combiner here is commutative and associative (or a total order on
// its (value, index) pairs). Wider rounds go through the LDS crossbar (ds_bpermute).
template <int kCtrl>
GOI_D int dpp_mov(int v) { return __builtin_amdgcn_update_dpp(0, v, kCtrl, 0xf, 0xf, false); }
GOI_D int lane_partner(int v, int d) {
    switch (d) {
        case 1: return dpp_mov<0xb1>(v);   // quad_perm [1, 0, 3, 2]
        case 2: return dpp_mov<0x4e>(v);   // quad_perm [2, 3, 0, 1]
        case 4: return dpp_mov<0x141>(v);  // row_half_mirror
        case 8: return dpp_mov<0x140>(v);  // row_mirror
        default: return __shfl_xor(v, d, 64);
    }
}
GOI_D float lane_partner(float v, int d) { return __int_as_float(lane_partner(__float_as_int(v), d)); }
GOI_D unsigned lane_partner(unsigned v, int d) { return (unsigned)lane_partner((int)v, d); }

template <class Grp>
GOI_D int group_max(const Grp& g, int x) {
    for (int d = 1; d < g.G(); d <<= 1) x = max(x, lane_partner(x, d));
    return x;
}
template <class Grp>
GOI_D int group_sum(const Grp& g, int x) {
    for (int d = 1; d < g.G(); d <<= 1) x += lane_partner(x, d);
    return x;
}
template <class Grp>
GOI_D unsigned long long group_or(const Grp& g, unsigned long long x) {
    for (int d = 1; d < g.G(); d <<= 1) {
        const unsigned lo = lane_partner((unsigned)x, d), hi = lane_partner((unsigned)(x >> 32), d);
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
        const float ov = lane_partner(v, d);
        const int oi = lane_partner(at, d);
        if (ov > v || (ov == v && oi < at)) {
            v = ov;
            at = oi;
        }
    }
}
template <class Grp>
GOI_D void group_argmin(const Grp& g, float& v, int& at) {
    for (int d = 1; d < g.G(); d <<= 1) {
        const float ov = lane_partner(v, d);
        const int oi = lane_partner(at, d);
        if (ov < v || (ov == v && oi < at)) {
            v = ov;
            at = oi;
        }
    }
}
template <class Grp>
GOI_D bool group_any(const Grp& g, bool p) {
    int x = p ? 1 : 0;
    for (int d = 1; d < g.G(); d <<= 1) x |= lane_partner(x, d);
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
