// goi_b2.hip - the MI355X batched Box2D 2.3.1 world step (libgoi_b2.so) and its C ABI (include/goi_b2.h).
//
// Execution model: a step is one launch (k_step) of 64-lane wavefronts, each stepping S worlds; each world runs on a
// group of 64 / S lanes (8 lanes at 16384 worlds) that execute its sequential code together and split its
// independent loops (vertex, slot, body and row loops, list filters):
//   start-of-step FindNewContacts where new_fixture, then Collide           (step.py:30-35, pairs.py:38-178)
//   b2World::Solve: islands, solver, sleep, fixture sync, FindNewContacts   (step.py:73-182)
//   b2World::SolveTOI's event loop, then inv_dt0 and ClearForces             (toi.py:827-865, step.py:41-46)
// goi_collide launches k_collide (the first part only). Box2D's sequential orders inside a world (contact list
// newest first, island DFS, Gauss-Seidel sweeps, TOI events) are kept exactly; the parallelism is across worlds and
// within the independent parts of a world's work. State leaves are read and written in place in the
// worlds-minor layout; the solver's body arrays sit in LDS ([field][body][lane]), its constraint rows in a
// per-block HBM scratch tile ([row][field][world]); the static terrain is a BVH over the static fixtures' fat AABBs,
// shared by every world and read through L2.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/goi_b2.h"
#include "b2_launch.hpp"

using namespace goi;

namespace {

thread_local std::string g_error;
thread_local GoiLaunchInfo g_last_launch{};  // goi_last_launch

int fail(int code, const std::string& msg) {
    g_error = msg;
    return code;
}

#define HIP_TRY(expr)                                                                      \
    do {                                                                                   \
        hipError_t e_ = (expr);                                                            \
        if (e_ != hipSuccess) return fail(GOI_E_HIP, std::string(#expr) + ": " + hipGetErrorString(e_)); \
    } while (0)

// ---------------------------------------------------------------- kernels

// Start-of-step FindNewContacts where new_fixture, then Collide (unless start_only). All lanes of the block take
// part in Collide's manifold evaluations.
__global__ void __launch_bounds__(kBlock) k_collide(DModel m, Launch L, int start_only) {
    GOI_DYNAMIC_LDS(lds);
    sincos_table_load();
    const int lane = threadIdx.x;
    const int w0 = xcd_group() * L.wpw;
    const LaneMap lm = lane_map(L, w0, lane);
    // W is used only where lm.valid
    const World W = make_world(m, L, lm.valid ? w0 + lm.wl : w0, lds, lm.valid ? lm.wl : 0, lm.sub, lm.G);
    const BlockCopy bc = block_copy(L.leaf, L.pitch, L.n, L.B, L.C, L.J, L.R, L.wpw, lds, w0, lane, kBlock);
    load_mirror_block(m, bc);
    build_order_block(bc);
    if (lm.valid) {
        if (W.u8(GOI_S_NEW_FIXTURE, 0)) find_new_contacts(m, W);
        W.u8(GOI_S_NEW_FIXTURE, 0) = 0;
    }
    if (!start_only) {
        const LaneViews v = fresh_views(m, L, lds, w0);  // the search above is a world's own phase
        collide_block(m, v.co, v.W, v.lm.valid, v.lm.leader, L.s);
    }
    store_mirror_block(fresh_views(m, L, lds, w0).bc);
}

template <bool kMulti>
__global__ void __launch_bounds__(kBlock, 2) k_step(DModel m, Launch L) {
    step_block<kMulti, true>(m, L);  // SolveTOI's views re-derived in each event iteration
}

// b2WorldManifold::Initialize (Box2D 2.3.1; the solver's prepare computes the same, contact_solver.py:60-104) of
// every slot of every world from the bodies' transforms, one thread per (slot, world): normal [C, 2], points
// [C, 2, 2], separations [C, 2], worlds-minor with the State's pitch; zeros for a free slot, a slot without points
// and the points past a manifold's count.
__global__ void k_world_manifold(DModel m, Launch L, float* normal, float* points, float* seps) {
    const int w = blockIdx.x * blockDim.x + threadIdx.x, c = blockIdx.y;
    if (w >= L.n || c >= L.C) return;
    const uint32_t P = (uint32_t)L.pitch;
    const auto at_i = [&](int leaf, int i) { return reinterpret_cast<const int*>(L.leaf[leaf])[(uint32_t)i * P + w]; };
    const auto at_f = [&](int leaf, int i) { return reinterpret_cast<const float*>(L.leaf[leaf])[(uint32_t)i * P + w]; };
    const auto put = [&](float* out, int i, float v) { out[(uint32_t)i * P + w] = v; };
    V2 n = mk(0.0f, 0.0f), p[2] = {mk(0.0f, 0.0f), mk(0.0f, 0.0f)};
    float sep[2] = {0.0f, 0.0f};
    const int cnt = at_i(GOI_C_PAIR, c) >= 0 ? at_i(GOI_C_COUNT, c) : 0;
    if (cnt > 0) {
        const int fa = at_i(GOI_C_FA, c), fb = at_i(GOI_C_FB, c);
        const int ba = m.fix[fa].body, bb = m.fix[fb].body;
        Xf xa, xb;
        xa.p = mk(at_f(GOI_B_XF_P, 2 * ba), at_f(GOI_B_XF_P, 2 * ba + 1));
        xa.q.c = at_f(GOI_B_XF_Q, 2 * ba); xa.q.s = at_f(GOI_B_XF_Q, 2 * ba + 1);
        xb.p = mk(at_f(GOI_B_XF_P, 2 * bb), at_f(GOI_B_XF_P, 2 * bb + 1));
        xb.q.c = at_f(GOI_B_XF_Q, 2 * bb); xb.q.s = at_f(GOI_B_XF_Q, 2 * bb + 1);
        const float ra = m.fix[fa].radius, rb = m.fix[fb].radius;
        const int mtype = at_i(GOI_C_MTYPE, c);
        const V2 ln = mk(at_f(GOI_C_LOCAL_NORMAL, 2 * c), at_f(GOI_C_LOCAL_NORMAL, 2 * c + 1));
        const V2 lp = mk(at_f(GOI_C_LOCAL_POINT, 2 * c), at_f(GOI_C_LOCAL_POINT, 2 * c + 1));
        const V2 pl0 = mk(at_f(GOI_C_POINT_LOCAL, 4 * c), at_f(GOI_C_POINT_LOCAL, 4 * c + 1));
        const V2 pl1 = mk(at_f(GOI_C_POINT_LOCAL, 4 * c + 2), at_f(GOI_C_POINT_LOCAL, 4 * c + 3));
        if (mtype == kCircles) {
            n = mk(1.0f, 0.0f);
            const V2 pa = mul(xa, lp), pb = mul(xb, pl0);
            const V2 d = pb - pa;
            if (dot(d, d) > kEps * kEps) {
                n = d;
                normalize(n);
            }
            const V2 ca = pa + ra * n, cb = pb - rb * n;
            p[0] = 0.5f * (ca + cb);
            sep[0] = dot(cb - ca, n);
        } else {
            const bool face_a = mtype == kFaceA;
            const Xf x1 = face_a ? xa : xb, x2 = face_a ? xb : xa;
            const float r1 = face_a ? ra : rb, r2 = face_a ? rb : ra;
            n = mul(x1.q, ln);
            const V2 plane = mul(x1, lp);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                if (i < cnt) {
                    const V2 clip = mul(x2, i == 0 ? pl0 : pl1);
                    const V2 c1 = clip + (r1 - dot(clip - plane, n)) * n, c2 = clip - r2 * n;
                    p[i] = 0.5f * (face_a ? c1 + c2 : c2 + c1);  // 0.5 (cA + cB)
                    sep[i] = dot(c2 - c1, n);                     // faceA: cB - cA; faceB: cA - cB
                }
            }
            if (!face_a) n = -n;
        }
    }
    put(normal, 2 * c, n.x); put(normal, 2 * c + 1, n.y);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        put(points, 4 * c + 2 * i, p[i].x); put(points, 4 * c + 2 * i + 1, p[i].y);
        put(seps, 2 * c + i, sep[i]);
    }
}

// The block order of a launch that runs its blocks in more than one round: the longest blocks first, so that they
// start in the first round and the shorter ones fill the rounds after them. A world group's expected time is its
// block's time in the previous launch on this stream (`cost`, clock ticks, 0 where unknown), in classes a factor of
// sqrt(2) apart below the longest; without any such time, its worlds' largest TOI event count of the previous step
// (the State's toi.events: 8 or more, 3 or more, the rest). Each XCD keeps the contiguous range of groups xcd_group
// gives it (block b runs on XCD b % 8): within the range, chunks of groups that share the State's 128-byte lines
// (32 worlds) are ordered by class, each class in chunk order, so that a line's worlds stay in one XCD's L2. One
// wavefront: per XCD, lane i takes a run of consecutive chunks, and the lanes' class sizes are scanned across the
// wavefront. The step's results do not depend on the order.
__global__ void __launch_bounds__(kBlock) k_group_order(const int* events, const int* cost, int n, int wpw, int groups,
                                                        int* order) {
    constexpr int kClasses = 8;
    const int lane = threadIdx.x, lanes = blockDim.x;
    int top = 0;  // the longest block time of the previous launch
    for (int g = lane; g < groups; g += lanes) top = max(top, cost[g]);
    for (int d = 1; d < lanes; d <<= 1) top = max(top, __shfl_xor(top, d, 64));
    const int cg = wpw < 32 ? 32 / wpw : 1;  // groups per chunk
    const int q = groups >> 3, r = groups & 7;
    for (int x = 0; x < 8; ++x) {
        const int base = x * q + min(x, r), size = q + (x < r ? 1 : 0);  // XCD x's groups
        const int chunks = (size + cg - 1) / cg;
        const int per = (chunks + lanes - 1) / lanes;
        const int k0 = min(lane * per, chunks), k1 = min(k0 + per, chunks);
        const auto span = [&](int k) { return min(cg, size - k * cg); };  // groups in chunk k
        const auto cls = [&](int k) {
            const int g0 = base + k * cg, g1 = g0 + span(k);
            if (top > 0) {
                int t = 0;
                for (int g = g0; g < g1; ++g) t = max(t, cost[g]);
                return t > 0 ? min(kClasses - 1, (int)(2.0f * log2f((float)top / (float)t))) : kClasses - 1;
            }
            int mx = 0;
            for (int w = g0 * wpw; w < min(n, g1 * wpw); ++w) mx = max(mx, events[w]);
            return mx >= 8 ? 0 : mx >= 3 ? 1 : 2;
        };
        int cnt[kClasses];  // this lane's groups per class
#pragma unroll
        for (int c = 0; c < kClasses; ++c) cnt[c] = 0;
        for (int k = k0; k < k1; ++k) {
            const int c = cls(k), g = span(k);
#pragma unroll
            for (int e = 0; e < kClasses; ++e) cnt[e] += e == c ? g : 0;
        }
        int pos[kClasses];  // this lane's first position in each class
        int before = 0;     // the groups of the classes before
#pragma unroll
        for (int c = 0; c < kClasses; ++c) {
            int incl = cnt[c];
            for (int d = 1; d < lanes; d <<= 1) {
                const int v = __shfl_up(incl, d, 64);
                if (lane >= d) incl += v;
            }
            pos[c] = before + incl - cnt[c];
            before += __shfl(incl, lanes - 1, 64);
        }
        for (int k = k0; k < k1; ++k) {
            const int c = cls(k), g = span(k);
            int p = 0;
#pragma unroll
            for (int e = 0; e < kClasses; ++e) p = e == c ? pos[e] : p;
            for (int i = 0; i < g; ++i) order[8 * (p + i) + x] = base + k * cg + i;  // XCD x's (p + i)-th block
#pragma unroll
            for (int e = 0; e < kClasses; ++e) pos[e] += e == c ? g : 0;
        }
    }
}

// The action-driven motor of joint `joint` in every world: motor_speed = gs * a_x, max_motor = gt * |a| (float32,
// one rounding per operation, |a| by IEEE square root), into the State's worlds-minor joint leaves.
__global__ void k_motor_actions(const float* a, float* speed, float* torque, int n, int pitch, int joint, float gs,
                                float gt) {
    const int w = blockIdx.x * blockDim.x + threadIdx.x;
    if (w >= n) return;
    const float ax = a[2 * w], ay = a[2 * w + 1];
    const uint32_t i = (uint32_t)joint * (uint32_t)pitch + (uint32_t)w;
    speed[i] = gs * ax;
    torque[i] = gt * sqrtf(ax * ax + ay * ay);
}

__global__ void k_sincos(const float* x, float* s, float* c, int n) {
    sincos_table_load();
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const Rot q = rot_of(x[i]);
    s[i] = q.s;
    c[i] = q.c;
}

}  // namespace

// ---------------------------------------------------------------- model upload and the static BVH

// The constraint and task rows of the launches one stream makes with a model: allocated on the stream's first call,
// grown (after the stream's earlier work has finished) when a larger batch arrives on it.
struct StreamScratch {
    hipStream_t stream;
    uint32_t* rows;
    size_t words;
};

struct GoiModel {
    DModel d;
    std::vector<void*> allocs;
    int C;
    int device = 0;
    // One scratch buffer per stream, so that calls on different streams never share rows. `mu` is held from the
    // lookup through the launch, so a buffer is never freed between another call's lookup and its launch.
    std::mutex mu;
    std::vector<StreamScratch> scratch;
};

// ---------------------------------------------------------------- the allocation-free entry point's rows
//
// goi_step_n_noalloc keeps its constraint and task rows in this array instead of a buffer it allocates: 2^25 words
// (128 MiB), which every device the library runs on holds until the process ends. Host code never uses the array's
// name as an address (on the host it is only a stand-in): goi_model_create looks up its address on the model's device
// once (static_scratch_setup) and the entry point passes that address to the kernels. Calls that overlap on one device
// share the array and race.
constexpr size_t kStaticScratchWords = size_t(1) << 25;
static __device__ __align__(256) uint32_t scratch[kStaticScratchWords];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_static_mu;
uint32_t* g_static_rows[kMaxDevices];  // the address of `scratch` on each device, once looked up

// Looks up the address of `scratch` on `device`, the current device, once per device.
int static_scratch_setup(int device) {
    if (device < 0 || device >= kMaxDevices) return fail(GOI_E_UNSUPPORTED, "device index above 63");
    std::lock_guard<std::mutex> hold(g_static_mu);
    if (g_static_rows[device]) return GOI_OK;
    void* p = nullptr;
    HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    g_static_rows[device] = static_cast<uint32_t*>(p);
    return GOI_OK;
}

uint32_t* static_rows(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> hold(g_static_mu);
    return g_static_rows[device];
}

template <typename T>
int upload(GoiModel* M, const T* host, size_t n, const T*& dev, hipStream_t st) {
    if (n == 0 || host == nullptr) {
        dev = nullptr;
        return GOI_OK;
    }
    void* p = nullptr;
    HIP_TRY(hipMalloc(&p, n * sizeof(T)));
    M->allocs.push_back(p);
    HIP_TRY(hipMemcpyAsync(p, host, n * sizeof(T), hipMemcpyHostToDevice, st));
    dev = static_cast<const T*>(p);
    return GOI_OK;
}

// The static fixtures' 8-wide tree (DModel::wnode): a node splits its entries by three rounds of median
// splits on the longer axis of their centroid bounds (a range of at most 8 entries is not split further) into up to
// 8 children; a child of at most 8 entries is a leaf, a larger one an inner node. Entries end in leaf order.
struct WideBuild {
    const float* fat;  // [F, 4]
    std::vector<int> leaf;
    std::vector<float4> box;  // 8 per node
    std::vector<int> ref;     // 8 per node
    int max_depth = 0;

    float4 bounds(int lo, int hi) const {
        float4 b = make_float4(3.4e38f, 3.4e38f, -3.4e38f, -3.4e38f);
        for (int i = lo; i < hi; ++i) {
            const float* f = fat + 4 * leaf[i];
            b.x = std::min(b.x, f[0]); b.y = std::min(b.y, f[1]);
            b.z = std::max(b.z, f[2]); b.w = std::max(b.w, f[3]);
        }
        return b;
    }
    int split(int lo, int hi) {
        float cx0 = 3.4e38f, cy0 = 3.4e38f, cx1 = -3.4e38f, cy1 = -3.4e38f;
        for (int i = lo; i < hi; ++i) {
            const float* f = fat + 4 * leaf[i];
            const float cx = 0.5f * (f[0] + f[2]), cy = 0.5f * (f[1] + f[3]);
            cx0 = std::min(cx0, cx); cx1 = std::max(cx1, cx);
            cy0 = std::min(cy0, cy); cy1 = std::max(cy1, cy);
        }
        const int axis = (cx1 - cx0) >= (cy1 - cy0) ? 0 : 1;
        const int mid = (lo + hi) / 2;
        std::nth_element(leaf.begin() + lo, leaf.begin() + mid, leaf.begin() + hi, [&](int a, int b) {
            const float* fa = fat + 4 * a;
            const float* fb = fat + 4 * b;
            const float ca = fa[axis] + fa[axis + 2], cb = fb[axis] + fb[axis + 2];
            return ca < cb || (ca == cb && a < b);
        });
        return mid;
    }
    // node over entries [lo, hi) at `depth` levels below the root; returns its index
    int build(int lo, int hi, int depth) {
        max_depth = std::max(max_depth, depth);
        const int node = (int)(box.size() / 8);
        box.resize(box.size() + 8, make_float4(3.4e38f, 3.4e38f, -3.4e38f, -3.4e38f));
        ref.resize(ref.size() + 8, 0);
        std::vector<int2> parts{make_int2(lo, hi)};
        for (int round = 0; round < 3; ++round) {
            std::vector<int2> next;
            for (const int2 r : parts) {
                if (r.y - r.x <= 8) {
                    next.push_back(r);
                    continue;
                }
                const int mid = split(r.x, r.y);
                next.push_back(make_int2(r.x, mid));
                next.push_back(make_int2(mid, r.y));
            }
            parts.swap(next);
        }
        for (size_t j = 0; j < parts.size(); ++j) {
            const int a = parts[j].x, b = parts[j].y;
            const int child = b - a <= 8 ? ~((a << 4) | (b - a)) : build(a, b, depth + 1);
            box[8 * node + j] = bounds(a, b);
            ref[8 * node + j] = child;
        }
        return node;
    }
};

}  // namespace

extern "C" {

int32_t goi_abi_version(void) { return GOI_ABI_VERSION; }

const char* goi_last_error(void) { return g_error.c_str(); }

int32_t goi_model_create(const GoiModelDesc* desc, int32_t contact_capacity, void* hip_stream, GoiModel** out) {
    if (!desc || !out) return fail(GOI_E_ARG, "goi_model_create: null argument");
    *out = nullptr;
    const int F = desc->F, J = desc->J, P = desc->P, B = desc->B;
    if (F < 0 || J < 0 || P < 0 || B <= 0) return fail(GOI_E_ARG, "goi_model_create: negative or zero sizes");
    if (!desc->fixture_slot || !desc->static_fat || !desc->body_type)
        return fail(GOI_E_UNSUPPORTED, "goi_model_create: the device step needs the compact fixture layout and body types");
    if (B > kMaxB) return fail(GOI_E_UNSUPPORTED, "goi_model_create: more than 64 bodies per world");
    if (J > kMaxJ) return fail(GOI_E_UNSUPPORTED, "goi_model_create: more than 64 joints per world");
    if (contact_capacity < 0 || contact_capacity > kMaxC)
        return fail(GOI_E_UNSUPPORTED, "goi_model_create: contact capacity above 256");
    for (int j = 0; j < J; ++j) {
        const int t = desc->joint_type[j];
        if (t != GOI_REVOLUTE && t != GOI_PRISMATIC && t != GOI_WELD)
            return fail(GOI_E_UNSUPPORTED, "goi_model_create: unknown joint type");
    }
    bool any_edge = false;
    for (int f = 0; f < F; ++f) {
        if (desc->fixture_slot[f] >= 0) continue;
        if (!desc->static_friction || !desc->static_restitution)
            return fail(GOI_E_ARG, "goi_model_create: static fixtures need their friction and restitution");
        const float* b = desc->static_fat + 4 * f;
        // the static tree's bounds and its empty child slots (lower > upper) need finite, ordered boxes
        if (!(std::isfinite(b[0]) && std::isfinite(b[1]) && std::isfinite(b[2]) && std::isfinite(b[3]) &&
              b[0] <= b[2] && b[1] <= b[3]))
            return fail(GOI_E_ARG, "goi_model_create: a static fixture's fat AABB is not finite and ordered");
    }
    for (int f = 0; f < F; ++f) {
        const int t = desc->shape_type[f], c = desc->count[f];
        if ((t != GOI_CIRCLE && t != GOI_POLYGON && t != GOI_EDGE) || c < 1 || c > GOI_MAX_POLY)
            return fail(GOI_E_UNSUPPORTED, "goi_model_create: bad shape");
        if (desc->fixture_body[f] < 0 || desc->fixture_body[f] >= B) return fail(GOI_E_ARG, "goi_model_create: bad fixture body");
        if (t == GOI_EDGE) {
            if (c != 2) return fail(GOI_E_ARG, "goi_model_create: an edge fixture has count 2");
            if (desc->body_type[desc->fixture_body[f]] != GOI_STATIC)
                return fail(GOI_E_UNSUPPORTED, "goi_model_create: edge fixtures belong to static bodies");
            any_edge = true;
        }
    }
    if (any_edge && !desc->centroid)
        return fail(GOI_E_ARG, "goi_model_create: edge fixtures need the polygon centroids");
    for (int p = 0; p < P; ++p) {
        const int a = desc->pair_a[p], b = desc->pair_b[p];
        if (a >= 0 && a < F && b >= 0 && b < F && desc->shape_type[b] == GOI_EDGE)
            return fail(GOI_E_ARG, "goi_model_create: a candidate pair names its edge fixture first");
    }
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    GoiModel* M = new GoiModel();
    M->C = contact_capacity;
    HIP_TRY(hipGetDevice(&M->device));
    DModel& d = M->d;
    d.F = F; d.J = J; d.P = P; d.B = B;
    // non-static rows
    std::vector<int> slot_fixture;
    for (int f = 0; f < F; ++f)
        if (desc->fixture_slot[f] >= 0) slot_fixture.push_back(f);
    for (size_t r = 0; r < slot_fixture.size(); ++r)
        if (desc->fixture_slot[slot_fixture[r]] != (int)r) {
            delete M;
            return fail(GOI_E_ARG, "goi_model_create: fixture_slot rows must ascend with the fixture index");
        }
    const int R = (int)slot_fixture.size();
    if (R > 64) { delete M; return fail(GOI_E_UNSUPPORTED, "goi_model_create: more than 64 non-static fixtures"); }
    d.R = R;
    // candidate tables
    std::vector<int> cand((size_t)F * std::max(R, 1), -1), dd;
    for (int p = 0; p < P; ++p) {
        const int a = desc->pair_a[p], b = desc->pair_b[p];
        if (a < 0 || a >= F || b < 0 || b >= F) { delete M; return fail(GOI_E_ARG, "goi_model_create: bad candidate pair"); }
        const int ra = desc->fixture_slot[a], rb = desc->fixture_slot[b];
        if (ra >= 0 && rb >= 0) dd.push_back(p);
        else if (ra < 0 && rb >= 0) cand[(size_t)a * R + rb] = p;
        else if (rb < 0 && ra >= 0) cand[(size_t)b * R + ra] = p;
        else { delete M; return fail(GOI_E_UNSUPPORTED, "goi_model_create: candidate between two static fixtures"); }
    }
    // the static tree
    WideBuild tree;
    tree.fat = desc->static_fat;
    for (int f = 0; f < F; ++f)
        if (desc->fixture_slot[f] < 0) tree.leaf.push_back(f);
    if (tree.leaf.size() >= (1u << 26)) {
        delete M;
        return fail(GOI_E_UNSUPPORTED, "goi_model_create: static terrain too large for the tree");
    }
    if (!tree.leaf.empty()) tree.build(0, (int)tree.leaf.size(), 0);
    if (tree.max_depth >= kWideDepth) {
        delete M;
        return fail(GOI_E_UNSUPPORTED, "goi_model_create: static tree deeper than its traversal allows");
    }
    d.n_wnodes = (int)(tree.box.size() / 8);
    // per leaf entry: fat box, body, candidate row
    const size_t n_leaf = tree.leaf.size();
    std::vector<MLeaf> leaf(std::max<size_t>(n_leaf, 1), MLeaf{});
    std::vector<int> leaf_cand(std::max<size_t>(n_leaf * R, 1), -1);
    for (size_t i = 0; i < n_leaf; ++i) {
        const int f = tree.leaf[i], b = desc->fixture_body[f];
        leaf[i].fat = make_float4(desc->static_fat[4 * f], desc->static_fat[4 * f + 1], desc->static_fat[4 * f + 2],
                                  desc->static_fat[4 * f + 3]);
        leaf[i].info = b | ((desc->body_type[b] == GOI_DYNAMIC ? 1 : 0) << 16);
        for (int r = 0; r < R; ++r) leaf_cand[i * R + r] = cand[(size_t)f * R + r];
    }
    std::vector<MNode> wnode(std::max<size_t>(d.n_wnodes, 1), MNode{});
    for (int k = 0; k < d.n_wnodes; ++k)
        for (int j = 0; j < 8; ++j) {
            wnode[k].box[j] = tree.box[8 * k + j];
            wnode[k].ref[j] = tree.ref[8 * k + j];
        }
    // per row: its fixture, body and whether the body is dynamic
    std::vector<MRow> row(std::max(R, 1), MRow{});
    for (int r = 0; r < R; ++r) {
        row[r].fixture = slot_fixture[r];
        row[r].body = desc->fixture_body[slot_fixture[r]];
        row[r].dynamic = desc->body_type[row[r].body] == GOI_DYNAMIC;
    }
    d.n_dd = (int)dd.size();
    int any = desc->toi_bodies ? 0 : 1;
    if (desc->toi_bodies)
        for (int b = 0; b < B; ++b) any |= desc->toi_bodies[b] ? 1 : 0;
    d.any_toi_body = any;
    d.rev_only = 1;
    for (int j = 0; j < J; ++j) d.rev_only &= desc->joint_type[j] == GOI_REVOLUTE ? 1 : 0;
    d.no_edges = any_edge ? 0 : 1;
    // joint components of the non-static bodies (union-find): more than one, and a world can hold several islands
    std::vector<int> root(B);
    for (int b = 0; b < B; ++b) root[b] = b;
    const auto find = [&](int b) {
        while (root[b] != b) b = root[b] = root[root[b]];
        return b;
    };
    for (int j = 0; j < J; ++j) {
        const int a = desc->joint_a[j], b = desc->joint_b[j];
        if (desc->body_type[a] != GOI_STATIC && desc->body_type[b] != GOI_STATIC) root[find(a)] = find(b);
    }
    int components = 0;
    for (int b = 0; b < B; ++b) components += desc->body_type[b] != GOI_STATIC && find(b) == b ? 1 : 0;
    d.island_lanes = components > 1 ? 1 : 0;
    // per fixture: its scalars, its static fat box and its vertex and normal slots
    std::vector<MFixture> fix(std::max(F, 1), MFixture{});
    std::vector<V2> poly((size_t)std::max(F, 1) * 16, V2{0.0f, 0.0f});
    for (int f = 0; f < F; ++f) {
        MFixture& x = fix[f];
        x.body = desc->fixture_body[f];
        x.type = desc->shape_type[f];
        x.radius = desc->radius[f];
        x.count = desc->count[f];
        x.slot = desc->fixture_slot[f];
        if (x.slot < 0) {  // checked above: present when a static fixture exists
            x.friction = desc->static_friction[f];
            x.restitution = desc->static_restitution[f];
        }
        x.edge_flags = desc->edge_flags ? desc->edge_flags[f] : 0;
        x.fat = make_float4(desc->static_fat[4 * f], desc->static_fat[4 * f + 1], desc->static_fat[4 * f + 2],
                            desc->static_fat[4 * f + 3]);
        if (desc->centroid) x.centroid = V2{desc->centroid[2 * f], desc->centroid[2 * f + 1]};
        for (int i = 0; i < kPoly; ++i) {
            poly[16 * (size_t)f + i] = V2{desc->verts[2 * (kPoly * f + i)], desc->verts[2 * (kPoly * f + i) + 1]};
            poly[16 * (size_t)f + 8 + i] =
                V2{desc->normals[2 * (kPoly * f + i)], desc->normals[2 * (kPoly * f + i) + 1]};
        }
    }
    std::vector<MJoint> joint(std::max(J, 1), MJoint{});
    for (int j = 0; j < J; ++j) {
        MJoint& x = joint[j];
        x.type = desc->joint_type[j];
        x.a = desc->joint_a[j];
        x.b = desc->joint_b[j];
        x.reference_angle = desc->reference_angle[j];
        x.anchor_a = V2{desc->local_anchor_a[2 * j], desc->local_anchor_a[2 * j + 1]};
        x.anchor_b = V2{desc->local_anchor_b[2 * j], desc->local_anchor_b[2 * j + 1]};
        x.axis_a = V2{desc->local_axis_a[2 * j], desc->local_axis_a[2 * j + 1]};
        x.yaxis_a = V2{desc->local_yaxis_a[2 * j], desc->local_yaxis_a[2 * j + 1]};
    }
    std::vector<int2> pair(std::max(P, 1), int2{});
    for (int p = 0; p < P; ++p) pair[p] = make_int2(desc->pair_a[p], desc->pair_b[p]);
    std::vector<int4> dd_info(std::max<size_t>(dd.size(), 1));
    for (size_t i = 0; i < dd.size(); ++i) {
        const int p = dd[i], a = desc->pair_a[p], b = desc->pair_b[p];
        dd_info[i] = make_int4(p, desc->fixture_slot[a] | (desc->fixture_slot[b] << 8),
                               desc->fixture_body[a] | (desc->fixture_body[b] << 8), 0);
    }
    int rc = GOI_OK;
    // the host tables above live until the stream synchronises below
#define UP(field, host, n) \
    if (rc == GOI_OK) rc = upload(M, host, (size_t)(n), d.field, st)
    UP(fix, fix.data(), F);
    UP(poly, poly.data(), (size_t)F * 16);
    UP(joint, joint.data(), J);
    UP(pair, pair.data(), P);
    UP(row, row.data(), R);
    UP(body_type, desc->body_type, B);
    UP(wnode, wnode.data(), d.n_wnodes);
    UP(leaf, leaf.data(), n_leaf);
    UP(leaf_cand, leaf_cand.data(), n_leaf * R);
    UP(dd_info, dd_info.data(), dd.size());
#undef UP
    if (rc == GOI_OK) {
        hipError_t e = hipStreamSynchronize(st);
        if (e != hipSuccess) rc = fail(GOI_E_HIP, std::string("goi_model_create: ") + hipGetErrorString(e));
    }
    if (rc == GOI_OK) rc = static_scratch_setup(M->device);
    if (rc != GOI_OK) {
        goi_model_destroy(M);
        return rc;
    }
    *out = M;
    return GOI_OK;
}

int32_t goi_model_destroy(GoiModel* M) {
    if (!M) return GOI_OK;
    // every launch that read the model's tables or its rows has finished before they are freed
    int cur = 0;
    const bool switch_dev = hipGetDevice(&cur) == hipSuccess && cur != M->device;
    if (switch_dev) (void)hipSetDevice(M->device);
    (void)hipDeviceSynchronize();
    for (void* p : M->allocs) (void)hipFree(p);
    for (StreamScratch& s : M->scratch) (void)hipFree(s.rows);
    if (switch_dev) (void)hipSetDevice(cur);
    delete M;
    return GOI_OK;
}

int32_t goi_model_release_rows(GoiModel* M) {
    if (!M) return fail(GOI_E_ARG, "goi_model_release_rows: null argument");
    std::lock_guard<std::mutex> hold(M->mu);
    if (M->scratch.empty()) return GOI_OK;
    // every launch that reads a buffer has finished before it is freed (the streams themselves may be gone)
    int cur = 0;
    const bool switch_dev = hipGetDevice(&cur) == hipSuccess && cur != M->device;
    if (switch_dev) (void)hipSetDevice(M->device);
    hipError_t e = hipDeviceSynchronize();
    for (StreamScratch& s : M->scratch)
        if (e == hipSuccess) e = hipFree(s.rows);
    if (switch_dev) (void)hipSetDevice(cur);
    if (e != hipSuccess) return fail(GOI_E_HIP, std::string("goi_model_release_rows: ") + hipGetErrorString(e));
    M->scratch.clear();
    return GOI_OK;
}

static int check_view(const GoiModel* M, const GoiStateView* v, const char* who) {
    if (!M || !v) return fail(GOI_E_ARG, std::string(who) + ": null argument");
    if (v->n_worlds < 0 || v->pitch < v->n_worlds) return fail(GOI_E_ARG, std::string(who) + ": bad n_worlds/pitch");
    // R: the model's non-static fixture rows (the compact fixture layout) or all its fixtures (the full layout)
    if (v->B != M->d.B || (v->R != M->d.R && v->R != M->d.F) || v->J != M->d.J || v->C != M->C)
        return fail(GOI_E_SHAPE, std::string(who) + ": state capacities differ from the model's (B, R or F, J, C)");
    for (int i = 0; i < GOI_NUM_LEAVES; ++i) {
        // leaves over an empty axis (no joints, no non-static fixtures, no slots) may be null
        const bool by_j = i >= GOI_J_ENABLE_MOTOR && i <= GOI_J_UPPER_IMPULSE;
        const bool by_r = i >= GOI_F_FRICTION && i <= GOI_F_FAT;
        const bool by_c = (i >= GOI_C_PAIR && i <= GOI_C_TANGENT_SPEED) ||
                          (i >= GOI_T_COUNT && i <= GOI_T_TANGENT_IMPULSE);
        const bool empty = (by_j && v->J == 0) || (by_r && v->R == 0) || (by_c && v->C == 0);
        if (!v->leaf[i] && v->n_worlds > 0 && !empty)
            return fail(GOI_E_ARG, std::string(who) + ": null leaf pointer");
    }
    // the kernels address leaf elements and scratch-row words with 32-bit offsets
    const uint64_t per_world = std::max<uint64_t>({4ull * v->C, 4ull * v->R, 3ull * v->J, 2ull * v->B, 1ull});
    const uint64_t row_words = (uint64_t)v->C * CF_N + (uint64_t)v->J * JF_N;
    if (per_world * (uint64_t)v->pitch >= (1ull << 32) || row_words * ((uint64_t)v->pitch + 64) >= (1ull << 32))
        return fail(GOI_E_UNSUPPORTED, std::string(who) + ": pitch too large for 32-bit element offsets");
    return GOI_OK;
}

// Compute units of the current device, looked up once per device (256, the MI355X's count, if the query fails).
static int cu_count() {
    static std::atomic<int> cached[kMaxDevices];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
    int n = cached[dev].load(std::memory_order_relaxed);
    if (n <= 0) {
        int v = 0;
        n = hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0 ? v : 256;
        cached[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// LDS workspace bytes per world (Workspace::layout) and the block budget it is held to.
constexpr size_t kStaticLdsBytes = sizeof(g_sincos_lds);      // each block's static LDS: the sin/cos table
constexpr size_t kMaxLdsBytes = 64 * 1024 - kStaticLdsBytes;   // workspaces + scan space of one block
constexpr size_t kCuLdsBytes = 160 * 1024;                      // LDS per CU (gfx950)
constexpr long kBlocksPerCu = 8;                                // k_step's register budget: two waves per SIMD
static size_t workspace_bytes(int B, int C, int J, int R) {
    return (size_t)Workspace::layout(B, C, J, R).words * sizeof(int);
}

// Worlds per 64-lane wavefront. One lane runs one world's whole step (a long serial chain of dependent work), so
// a launch wants at least a few wavefronts per SIMD (256 CUs x 4 SIMDs) even when that leaves lanes idle.
// GOI_WORLDS_PER_WAVE overrides (1..64).
static int worlds_per_wave(int n, size_t ws_bytes_per_world) {
    const char* e = getenv("GOI_WORLDS_PER_WAVE");  // read per call: tests vary it within one process
    int forced = e ? atoi(e) : 0;
    if (forced < 0 || forced > kBlock) forced = 0;
    if (forced > 0)
        return std::min<long>(forced, std::max<long>(1, (kMaxLdsBytes - kBlock * sizeof(int)) / ws_bytes_per_world));
    // Fewer worlds per wave fill more SIMDs, shrink the slowest lane a wave waits for and give each world more lanes
    // in the block-cooperative passes, but past the waves a SIMD can hold (k_step's register budget allows two) the
    // launch needs a second round. Measured at 16384 worlds of the 4-body rig, two waves per SIMD: 16 -> 1.32 ms,
    // 8 -> 1.25 (one wave per SIMD: 32 -> 1.56, 16 -> 1.48). Aim for two waves per SIMD (8 per CU).
    //
    // A CU's 160 KB of LDS can hold fewer blocks than that when the worlds' workspaces are large, so among the wave
    // sizes that fit, take the one with the most worlds resident per CU (blocks per CU x worlds per block), the
    // smaller on a tie (more lanes per world). The 4-body rig with 40 slots: 8 worlds per wave, 8 blocks per CU. The
    // rig with 12 boxes and 128 slots: 4 worlds per wave (30.6 KB, 5 blocks per CU: 20 worlds) rather than 8 (61 KB,
    // 2 blocks: 16 worlds), measured 35% faster at 65536 worlds.
    int top = kBlock;
    while (top > 1 && (long)n / top < 8L * cu_count()) top /= 2;
    int wpw = 0;
    long best = -1;
    for (int w = top; w >= 1; w /= 2) {
        const size_t lds = ws_bytes_per_world * w + kBlock * sizeof(int);
        if (lds > kMaxLdsBytes) continue;
        const long blocks = std::min<long>(kBlocksPerCu, (long)(kCuLdsBytes / (lds + kStaticLdsBytes)));
        const long resident = blocks * w;
        if (resident >= best) {  // >=: the smaller wave wins a tie
            best = resident;
            wpw = w;
        }
    }
    return wpw > 0 ? wpw : 1;
}

// The buffer of a packed State (all leaves at their packed_word offsets from leaf 0, pitch a multiple of 64, every
// element offset within 32 bits), else null.
static char* packed_state(const GoiStateView* v) {
    if (v->pitch <= 0 || v->pitch % 64 != 0) return nullptr;
    const uint64_t words = (uint64_t)packed_word(GOI_NUM_LEAVES, v->B, v->C, v->J, v->R);
    if (4u * words * (uint64_t)v->pitch > 0xffffffffull) return nullptr;
    char* base = static_cast<char*>(v->leaf[0]);
    for (int l = 0; l < GOI_NUM_LEAVES; ++l)
        if (static_cast<char*>(v->leaf[l]) != base + 4 * (size_t)packed_word(l, v->B, v->C, v->J, v->R) * v->pitch)
            return nullptr;
    return base;
}

// The dynamic LDS of one block of launch L: the worlds' workspaces (words x wpw ints), then 64 ints of scan space.
static size_t block_lds_bytes(const Launch& L) {
    const int words = Workspace::layout(L.B, L.C, L.J, L.R).words;
    return ((size_t)words * L.wpw + kBlock) * sizeof(int);
}

// A State in the full fixture layout (a row per fixture: v->R is the model's F, not its R non-static rows) runs with
// full_rows set: the kernels then address non-static row r at the fixture's own row and never touch the static rows
// (a static fixture's fat AABB, friction and restitution are the Model's; a step never changes them).
static void fill_launch(Launch& L, const GoiModel* M, const GoiStateView* v, const GoiSettings* s, float dt) {
    std::memcpy(L.leaf, v->leaf, sizeof(L.leaf));
    L.n_steps = 1;
    L.n = v->n_worlds;
    L.pitch = v->pitch;
    L.B = v->B;
    L.C = v->C;
    L.R = M->d.R;
    L.J = v->J;
    L.full_rows = v->R != M->d.R;
    L.s = *s;
    L.dt = dt;
    std::memset(&L.dbg, 0, sizeof(L.dbg));
    L.scratch = nullptr;
    L.order = nullptr;
    L.cost = nullptr;
    L.wpw = worlds_per_wave(v->n_worlds, workspace_bytes(L.B, L.C, L.J, L.R));
    L.packed = !L.full_rows && packed_state(v) != nullptr;
}

// Words of constraint and task rows a launch over `state` uses: per world C contact rows and J joint rows, in tiles of
// wpw worlds, so at most pitch + 63 world columns (the kernels' 32-bit offsets are checked by check_view).
static size_t scratch_words(const GoiStateView* state) {
    return ((size_t)state->C * CF_N + (size_t)state->J * JF_N) * ((size_t)state->pitch + 64);
}

// The rows of stream st's launches with model M (M->mu held): the stream's buffer, allocated on its first call and
// replaced by a larger one when this batch needs more. The old buffer is freed only after the stream's earlier work,
// the only work that reads it, has finished. Past the rows, pitch + 64 words hold a launch's block order and as many
// its blocks' times (k_group_order), zero in a new buffer.
static int stream_rows(GoiModel* M, const GoiStateView* state, hipStream_t st, uint32_t** rows) {
    const size_t words = scratch_words(state) + 2 * ((size_t)state->pitch + 64);
    StreamScratch* e = nullptr;
    for (StreamScratch& s : M->scratch)
        if (s.stream == st) e = &s;
    if (!e) {
        M->scratch.push_back(StreamScratch{st, nullptr, 0});
        e = &M->scratch.back();
    }
    if (words > e->words) {
        if (e->rows) {
            HIP_TRY(hipStreamSynchronize(st));
            HIP_TRY(hipFree(e->rows));
            e->rows = nullptr;
            e->words = 0;
        }
        HIP_TRY(hipMalloc(&e->rows, words * sizeof(uint32_t)));
        e->words = words;
        const size_t times = scratch_words(state) + (size_t)state->pitch + 64;  // the blocks' times: none yet
        HIP_TRY(hipMemsetAsync(e->rows + times, 0, (words - times) * sizeof(uint32_t), st));
    }
    *rows = e->rows;
    return GOI_OK;
}

int32_t goi_step(const GoiModel* model, const GoiStateView* state, const GoiSettings* settings, float dt,
                 void* hip_stream, const GoiDebug* debug) {
    return goi_step_n(model, state, settings, dt, 1, hip_stream, debug);
}

static int check_step_args(const GoiModel* model, const GoiStateView* state, const GoiSettings* settings,
                           int32_t n_steps, const char* who) {
    int rc = check_view(model, state, who);
    if (rc != GOI_OK) return rc;
    if (!settings) return fail(GOI_E_ARG, std::string(who) + ": null settings");
    if (settings->velocity_iterations < 0 || settings->position_iterations < 0)
        return fail(GOI_E_ARG, std::string(who) + ": negative iteration counts");
    if (n_steps < 0) return fail(GOI_E_ARG, std::string(who) + ": negative step count");
    return GOI_OK;
}

// Launches n_steps steps of every world of `state` with the constraint rows at `rows` (scratch_words(state) words).
// order_buf: room for the block order (pitch + 64 words), or null (the blocks then run in the XCD order). A launch
// whose blocks do not all fit on the GPU at once, with TOI on, first orders its blocks (k_group_order).
static int launch_step(const GoiModel* M, const GoiStateView* state, const GoiSettings* settings, float dt,
                       int32_t n_steps, hipStream_t st, const GoiDebug* debug, uint32_t* rows, int* order_buf) {
    Launch L;
    fill_launch(L, M, state, settings, dt);
    L.scratch = rows;
    L.n_steps = n_steps;
#ifdef GOI_HOST_BUILD
    goi_host_poison(rows, scratch_words(state) * sizeof(uint32_t));  // no launch may read rows an earlier one wrote
#endif
    if (debug) L.dbg = *debug;
    const int grid = (state->n_worlds + L.wpw - 1) / L.wpw;
    const size_t lds = block_lds_bytes(L);
    // the fixed instances write no debug arrays (it frees the scalar registers their pointers would hold)
    const GoiDebug& D = L.dbg;
    const bool dbg = D.body_island || D.contact_island || D.contact_order || D.n_islands || D.toi_event_slot ||
                     D.toi_event_alpha || D.toi_event_island || D.toi_island_rows;
    const bool rig = L.B == kRigB && L.C == kRigC && L.J == kRigJ && L.R == kRigR && L.wpw == kRigS &&
                     M->d.B == kRigB && M->d.J == kRigJ && M->d.R == kRigR && L.packed && !dbg;
    const dim3 g(grid), b(kBlock);
    const bool plain = M->d.rev_only && M->d.no_edges && settings->revolute_v24;
    const bool island = L.B == kIslandB && L.C == kIslandC && L.J == kIslandJ && L.R == kIslandR &&
                        L.wpw == kIslandS && M->d.B == kIslandB && M->d.J == kIslandJ && M->d.R == kIslandR &&
                        L.packed && plain && !dbg;
    g_last_launch = GoiLaunchInfo{L.wpw, grid, (int32_t)lds,
                                  rig ? GOI_KERNEL_RIG : island ? GOI_KERNEL_ISLAND : GOI_KERNEL_GENERIC};
    const long resident = (long)cu_count() * std::min<long>(kBlocksPerCu, (long)(kCuLdsBytes / (lds + kStaticLdsBytes)));
    if (order_buf && settings->continuous_physics && grid > resident) {
        int* cost = order_buf + state->pitch + 64;
        hipLaunchKernelGGL(k_group_order, dim3(1), dim3(kBlock), 0, st,
                           static_cast<const int*>(state->leaf[GOI_T_EVENTS]), cost, state->n_worlds, L.wpw, grid,
                           order_buf);
        HIP_TRY(hipGetLastError());
        L.order = order_buf;
        L.cost = cost;
    }
    if (rig) {
        const hipError_t e = launch_rig_step(M->d, L, n_steps != 1, plain, g, lds, st);
        if (e != hipSuccess) return fail(GOI_E_HIP, std::string("launch_rig_step: ") + hipGetErrorString(e));
    } else if (island) {
        const hipError_t e = launch_island_step(M->d, L, n_steps != 1, g, lds, st);
        if (e != hipSuccess) return fail(GOI_E_HIP, std::string("launch_island_step: ") + hipGetErrorString(e));
    } else if (n_steps == 1) {
        hipLaunchKernelGGL(k_step<false>, g, b, lds, st, M->d, L);
    } else {
        hipLaunchKernelGGL(k_step<true>, g, b, lds, st, M->d, L);
    }
    HIP_TRY(hipGetLastError());
    return GOI_OK;
}

int32_t goi_step_n(const GoiModel* model, const GoiStateView* state, const GoiSettings* settings, float dt,
                   int32_t n_steps, void* hip_stream, const GoiDebug* debug) {
    int rc = check_step_args(model, state, settings, n_steps, "goi_step");
    if (rc != GOI_OK) return rc;
    if (state->n_worlds == 0 || n_steps == 0) return GOI_OK;
    // the handle's only mutable part is its per-stream scratch table, guarded by its mutex
    GoiModel* M = const_cast<GoiModel*>(model);
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    std::lock_guard<std::mutex> hold(M->mu);
    uint32_t* rows = nullptr;
    rc = stream_rows(M, state, st, &rows);
    if (rc != GOI_OK) return rc;
    return launch_step(M, state, settings, dt, n_steps, st, debug, rows,
                       reinterpret_cast<int*>(rows + scratch_words(state)));
}

int32_t goi_step_n_noalloc(const GoiModel* model, const GoiStateView* state, const GoiSettings* settings, float dt,
                           int32_t n_steps, void* hip_stream, const GoiDebug* debug) {
    int rc = check_step_args(model, state, settings, n_steps, "goi_step_n_noalloc");
    if (rc != GOI_OK) return rc;
    if (state->n_worlds == 0 || n_steps == 0) return GOI_OK;
    if (scratch_words(state) > kStaticScratchWords)
        return fail(GOI_E_UNSUPPORTED, "goi_step_n_noalloc: the batch needs " + std::to_string(scratch_words(state)) +
                                           " words of constraint rows, above the static maximum of " +
                                           std::to_string(kStaticScratchWords) +
                                           " ((C * 54 + J * 57) * (pitch + 64) words); use goi_step_n");
    uint32_t* rows = static_rows(model->device);
    if (!rows) return fail(GOI_E_ARG, "goi_step_n_noalloc: the model's device has no static rows set up");
    return launch_step(model, state, settings, dt, n_steps, static_cast<hipStream_t>(hip_stream), debug, rows,
                       nullptr);
}

int32_t goi_collide(const GoiModel* model, const GoiStateView* state, const GoiSettings* settings, void* hip_stream) {
    int rc = check_view(model, state, "goi_collide");
    if (rc != GOI_OK) return rc;
    if (!settings) return fail(GOI_E_ARG, "goi_collide: null settings");
    if (state->n_worlds == 0) return GOI_OK;
    GoiModel* M = const_cast<GoiModel*>(model);
    hipStream_t st = static_cast<hipStream_t>(hip_stream);
    std::lock_guard<std::mutex> hold(M->mu);
    Launch L;
    fill_launch(L, M, state, settings, 0.0f);
    const int grid = (state->n_worlds + L.wpw - 1) / L.wpw;
    rc = stream_rows(M, state, st, &L.scratch);
    if (rc != GOI_OK) return rc;
#ifdef GOI_HOST_BUILD
    goi_host_poison(L.scratch, scratch_words(state) * sizeof(uint32_t));
#endif
    const size_t lds = block_lds_bytes(L);
    g_last_launch = GoiLaunchInfo{L.wpw, grid, (int32_t)lds, GOI_KERNEL_COLLIDE};
    hipLaunchKernelGGL(k_collide, dim3(grid), dim3(kBlock), lds, st, M->d, L, 0);
    HIP_TRY(hipGetLastError());
    return GOI_OK;
}

int32_t goi_world_manifold(const GoiModel* model, const GoiStateView* state, float* normal, float* points,
                           float* separations, void* hip_stream) {
    int rc = check_view(model, state, "goi_world_manifold");
    if (rc != GOI_OK) return rc;
    if (state->n_worlds == 0 || state->C == 0) return GOI_OK;
    if (!normal || !points || !separations) return fail(GOI_E_ARG, "goi_world_manifold: null output");
    Launch L;
    const GoiSettings none{};
    fill_launch(L, model, state, &none, 0.0f);
    hipLaunchKernelGGL(k_world_manifold, dim3((state->n_worlds + 255) / 256, state->C), dim3(256), 0,
                       static_cast<hipStream_t>(hip_stream), model->d, L, normal, points, separations);
    HIP_TRY(hipGetLastError());
    return GOI_OK;
}

int32_t goi_apply_motor_actions(const float* actions, float* motor_speed, float* max_motor, int32_t n_worlds,
                                int32_t pitch, int32_t joint, float speed_gain, float torque_gain, void* hip_stream) {
    if (n_worlds < 0 || pitch < n_worlds || joint < 0)
        return fail(GOI_E_ARG, "goi_apply_motor_actions: bad n_worlds/pitch/joint");
    if (n_worlds == 0) return GOI_OK;
    if (!actions || !motor_speed || !max_motor) return fail(GOI_E_ARG, "goi_apply_motor_actions: null pointer");
    if ((uint64_t)(joint + 1) * (uint64_t)pitch >= (1ull << 32))
        return fail(GOI_E_UNSUPPORTED, "goi_apply_motor_actions: pitch too large for 32-bit element offsets");
    hipLaunchKernelGGL(k_motor_actions, dim3((n_worlds + 255) / 256), dim3(256), 0,
                       static_cast<hipStream_t>(hip_stream), actions, motor_speed, max_motor, n_worlds, pitch, joint,
                       speed_gain, torque_gain);
    HIP_TRY(hipGetLastError());
    return GOI_OK;
}

int32_t goi_packed_layout(int32_t B, int32_t C, int32_t J, int32_t R, int32_t* words) {
    if (B < 0 || C < 0 || J < 0 || R < 0 || !words) return fail(GOI_E_ARG, "goi_packed_layout: bad arguments");
    for (int l = 0; l <= GOI_NUM_LEAVES; ++l) words[l] = packed_word(l, B, C, J, R);
    return GOI_OK;
}

int32_t goi_last_launch(GoiLaunchInfo* out) {
    if (!out) return fail(GOI_E_ARG, "goi_last_launch: null argument");
    *out = g_last_launch;
    return GOI_OK;
}

int32_t goi_sincos(const float* x, float* s, float* c, int32_t n, void* hip_stream) {
    if (n < 0 || (n > 0 && (!x || !s || !c))) return fail(GOI_E_ARG, "goi_sincos: bad arguments");
    if (n == 0) return GOI_OK;
    hipLaunchKernelGGL(k_sincos, dim3((n + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(hip_stream), x, s, c, n);
    HIP_TRY(hipGetLastError());
    return GOI_OK;
}

}  // extern "C"
