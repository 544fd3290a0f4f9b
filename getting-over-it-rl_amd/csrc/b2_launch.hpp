// b2_launch.hpp - the launch-side device code shared by the step's translation units: the kernel argument block
// (Launch), the mapping of a block's lanes to worlds, the world views and the whole step of a block (step_block).
// goi_b2.hip instantiates it for any State (leaf pointers); goi_b2_rig.hip, compiled with GOI_PACKED_STATE = 1, for
// the 4-body rig's fixed dimensions on packed States.
#pragma once

#include "../../include/goi_b2.h"
#include "b2_step.hpp"

namespace goi {

#ifdef GOI_HOST_BUILD
constexpr int kBlock = 1;  // the sequential host build runs one lane per block
#define GOI_DYNAMIC_LDS(name) int* const name = goi_host_lds
#else
constexpr int kBlock = 64;
#define GOI_DYNAMIC_LDS(name) extern __shared__ int name[]
#endif
static_assert(kBlock == kCoopLanes, "the cooperative passes span the block");

struct Launch {
    void* leaf[GOI_NUM_LEAVES];
    int packed;  // the leaves are the consecutive parts of leaf[0]'s buffer (goi_packed_layout)
    int full_rows;  // the fixture leaves have a row per fixture (the full layout); R counts the non-static ones
    int n, pitch, B, C, R, J;
    int wpw;  // worlds per wavefront: lanes >= wpw idle, so small batches still spread over every SIMD
    uint32_t* scratch;  // contact rows then joint rows
    GoiSettings s;
    float dt;
    int n_steps;  // consecutive steps of every world in this launch (>= 1)
    GoiDebug dbg;
    const int* order;  // block b steps world group order[b] (k_group_order), or null: the XCD mapping (xcd_group)
    int* cost;         // with order: each group's block time in this launch (clock ticks), for the next launch's order
};


// World w on lane `lane` of its block; the block's LDS workspace holds L.wpw lanes.
__device__ __forceinline__ World make_world(const DModel& m, const Launch& L, int w, int* lds, int lane, int sub,
                                           int G) {
    World W;
    W.pitch = L.pitch;
    W.B = L.B;
    W.C = L.C;
    W.R = L.R;
    W.J = L.J;
    W.lv = L.leaf;
    W.w = w;
    W.k = Workspace::layout(L.B, L.C, L.J, L.R);
    W.ws = lds + lane;
    W.S = L.wpw;
    W.sub = sub;
    W.G = G;
    W.frow_map = L.full_rows ? m.row : nullptr;
    W.init_masks(m);
    return W;
}

// The scratch rows of world w0 + wl of this block (tile = the block's world group): the contact rows' tiles, then
// the joint rows' tiles, each region gridDim.x tiles long.
__device__ __forceinline__ Rows contact_rows(const Launch& L, int w0, int wl) {
    return rows_of(L.scratch, L.C, CF_N, L.wpw, w0 / L.wpw, wl);
}
// The contact rows' tile read world-major, for SolveTOI (Solve's rows are dead by then).
__device__ __forceinline__ Rows toi_rows(const Launch& L, int w0, int wl) {
    return rows_world_major(L.scratch, L.C, CF_N, L.wpw, w0 / L.wpw, wl);
}
__device__ __forceinline__ Rows joint_rows(const Launch& L, int w0, int wl) {
    uint32_t* region = L.scratch + (size_t)L.C * CF_N * ((size_t)gridDim.x * L.wpw);
    return rows_of(region, L.J, JF_N, L.wpw, w0 / L.wpw, wl);
}

// ---------------------------------------------------------------- kernels

// Lanes and worlds of a block: the block's L.wpw worlds each take G consecutive lanes (its lane group; G is the
// largest power of two with G * wpw <= 64).
// Every lane of a group runs the world's sequential code on the same data (same loads, same stores of the same
// values), so the group's lanes stay together on every branch; `leader` is the group's first lane, which alone
// reports the world's task counts to coop_run.
struct LaneMap {
    int G;        // lanes per world
    int wl;       // this lane's world in the block
    int sub;      // this lane's place in its world's group
    bool valid;   // the lane runs a world (wl < wpw and w0 + wl < n)
    bool leader;  // valid and sub == 0
};
__device__ __forceinline__ LaneMap lane_map(const Launch& L, int w0, int lane) {
    int G = kBlock;
    while (G * L.wpw > kBlock) G >>= 1;
    LaneMap lm;
    lm.G = G;
    lm.wl = lane / G;
    lm.sub = lane - lm.wl * G;
    lm.valid = lm.wl < L.wpw && w0 + lm.wl < L.n;  // wpw need not divide 64: lanes past G * wpw stay idle
    lm.leader = lm.valid && lm.sub == 0;
    return lm;
}

// World group of this block. Blocks are dealt to the 8 XCDs round robin (block b on XCD b % 8), and each XCD has its
// own L2; numbering the groups so that every XCD holds one contiguous range keeps neighbouring worlds, which share
// 128-byte lines of every State leaf, behind the same L2. A bijection on [0, gridDim.x) for any grid.
__device__ __forceinline__ int xcd_group() {
    const int nb = gridDim.x, b = blockIdx.x, x = b & 7, q = nb >> 3, r = nb & 7;
    return x * q + min(x, r) + (b >> 3);
}

// The world group of this block of launch L.
__device__ __forceinline__ int block_group(const Launch& L) { return L.order ? L.order[blockIdx.x] : xcd_group(); }

// The block's cooperative view (Coop) for lanes whose world is W (or lane 0's, for lanes without one).
__device__ __forceinline__ Coop block_coop(const Launch& L, const World& W, int* lds, int w0) {
    Coop co;
    co.base = W;
    co.lds = lds;
    co.scan = lds + W.k.words * L.wpw;
    co.rows = L.scratch;
    co.w0 = w0;
    co.lanes = kBlock;
    co.G = lane_map(L, w0, 0).G;
    return co;
}

// A lane's views of its block: its world's State and workspace, the block's cooperative queues, the solver's body
// arrays and constraint rows, and the block's State copy.
struct LaneViews {
    LaneMap lm;
    World W;  // used if lm.valid
    Coop co;
    Bodies bd;
    Rows CR;
    Rows TR;  // CR's tile world-major (toi_rows)
    BlockCopy bc;
};
__device__ __forceinline__ LaneViews lane_views(const DModel& m, const Launch& L, int* lds, int w0, int lane) {
    LaneViews v;
    v.lm = lane_map(L, w0, lane);
    const bool valid = v.lm.valid;
    v.W = make_world(m, L, valid ? w0 + v.lm.wl : w0, lds, valid ? v.lm.wl : 0, v.lm.sub, v.lm.G);
    v.co = block_coop(L, v.W, lds, w0);
    v.bd.s = reinterpret_cast<float*>(lds) + v.W.k.o_body * v.W.S + (valid ? v.lm.wl : 0);
    v.bd.B = L.B;
    v.bd.st = v.W.S;
    v.CR = contact_rows(L, w0, valid ? v.lm.wl : 0);
    v.TR = toi_rows(L, w0, valid ? v.lm.wl : 0);
    v.bc = block_copy(L.leaf, L.pitch, L.n, L.B, L.C, L.J, L.R, L.wpw, lds, w0, lane, kBlock);
    return v;
}

// The lane's views set up afresh from lane_now(), where block-cooperative code follows code that some lanes skipped
// (a world's own phases, which lanes without a world and the lanes of other worlds do not run). A per-lane value
// carried across such code was seen to be lost, in some builds, for the lanes that skipped it: lanes without a world
// (in a block's last, partly filled group of worlds, or at wave sizes that leave lanes idle) then ran cooperative
// tasks and block copies with a broken view and wrote over their block's worlds.
__device__ __forceinline__ LaneViews fresh_views(const DModel& m, const Launch& L, int* lds, int w0) {
    return lane_views(m, L, lds, w0, lane_now());
}

// The wave's issue priority for a step: the largest TOI event count of its worlds in the previous step (the State's
// toi.events), up to 3. The kernel ends with its slowest wave, and the slowest waves are those with a world on a long
// chain of TOI events, which recurs from step to step; with priority such a wave issues ahead of the other wave on its
// SIMD from the start of the step, not only once it runs alone (2.5% faster). Results do not depend on it.
__device__ __forceinline__ void prioritise_wave(const World& W, bool valid) {
    const int ev = valid ? W.i32(GOI_T_EVENTS, 0) : 0;
    if (__any(ev >= 3)) wave_priority<3>();
    else if (__any(ev >= 2)) wave_priority<2>();
    else if (__any(ev >= 1)) wave_priority<1>();
    else wave_priority<0>();
}

// inv_dt0, ClearForces and the debug status word of the lane's world after its step (step.py:41-47)
__device__ __forceinline__ void finish_step(const Launch& L, const LaneViews& v, int overflow0, bool capped) {
    if (!v.lm.valid) return;
    const World& W = v.W;
    const float dt = L.dt;
    if (dt > 0.0f) W.f(GOI_S_INV_DT0, 0) = 1.0f / dt;
    if (L.s.auto_clear_forces)
        for (int b = 0; b < W.B; ++b) {
            W.set2(GOI_B_FORCE, b, mk(0.0f, 0.0f));
            W.f(GOI_B_TORQUE, b) = 0.0f;
        }
    if (L.dbg.status) L.dbg.status[W.w] = step_status(W, overflow0, capped, dt, L.s);
}

// One b2World::Step (step.py:28-47) of each world of the block on its lane group, on the workspace mirror:
// FindNewContacts where new_fixture, Collide, Solve, SolveTOI, inv_dt0, ClearForces. Lanes without a world stay to
// share the block's manifold and TOI work. Each block-cooperative phase sets up the lane's views afresh (fresh_views).
template <bool kOpaqueToi>
__device__ __forceinline__ void step_worlds(const DModel& m, const Launch& L, int* lds, int w0) {
    const LaneViews v = fresh_views(m, L, lds, w0);
    prioritise_wave(v.W, v.lm.valid);
    const int overflow0 = v.lm.valid && L.dbg.status ? v.W.i32(GOI_S_OVERFLOW, 0) : 0;
    build_order_block(v.bc);
    if (v.lm.valid) {
        if (v.W.u8(GOI_S_NEW_FIXTURE, 0)) find_new_contacts(m, v.W);
        v.W.u8(GOI_S_NEW_FIXTURE, 0) = 0;
    }
    const LaneViews c = fresh_views(m, L, lds, w0);
    collide_block(m, c.co, c.W, c.lm.valid, c.lm.leader, L.s);
    if (c.lm.valid) {
        solve_world(m, c.W, c.bd, c.CR, joint_rows(L, w0, c.lm.wl), L.s, L.dt, L.dbg);
        clear_toi_trace(c.W, L.dbg);
    }
    bool capped = false;
    if (L.s.continuous_physics) {
        const LaneViews t = fresh_views(m, L, lds, w0);
        capped = solve_toi_world<kOpaqueToi>(m, t.W, t.bd, t.TR, L.s, L.dt, t.lm.valid,
                                             [&] { return fresh_views(m, L, lds, w0); }, L.dbg);
    }
    finish_step(L, fresh_views(m, L, lds, w0), overflow0, capped);
}

// The block's worlds: the State into the workspace mirror, one step (kMulti false) or L.n_steps steps, the mirror
// back. Across the steps of a multi-step launch the mirror stays in LDS (it is the State's current value; every access
// to a mirrored leaf inside a step goes through the workspace), so the worlds need neither a store nor a reload between
// steps, and the block never waits for other blocks' steps. The lane's views are set up afresh (fresh_views) for each
// block-cooperative phase and for the mirror's load and store.
// At most 256 registers (two waves per SIMD): the second wave hides the latency chains of the first.
template <bool kMulti, bool kOpaqueToi = false>  // kOpaqueToi: solve_toi_world's kOpaqueViews
__device__ __forceinline__ void step_block(const DModel& m, const Launch& L) {
    GOI_DYNAMIC_LDS(lds);
    const uint64_t t_start = block_clock();
    sincos_table_load();
    const int w0 = block_group(L) * L.wpw;
    const auto fresh_bc = [&] {
        return block_copy(L.leaf, L.pitch, L.n, L.B, L.C, L.J, L.R, L.wpw, lds, w0, lane_now(), kBlock);
    };
    if constexpr (!kMulti) {
        // step_worlds' sequence written out, a world's own views set up once (2% faster than a call of step_worlds);
        // the cooperative phases take theirs afresh
        const int lane = lane_now();
        const LaneMap lm = lane_map(L, w0, lane);
        const bool valid = lm.valid;
        const World W = make_world(m, L, valid ? w0 + lm.wl : w0, lds, valid ? lm.wl : 0, lm.sub, lm.G);  // if valid
        Bodies bd;
        bd.s = reinterpret_cast<float*>(lds) + W.k.o_body * W.S + (valid ? lm.wl : 0);
        bd.B = L.B;
        bd.st = W.S;
        const Rows CR = contact_rows(L, w0, valid ? lm.wl : 0);
        load_mirror_block(m, fresh_bc());
        prioritise_wave(W, valid);
        const int overflow0 = valid && L.dbg.status ? W.i32(GOI_S_OVERFLOW, 0) : 0;
        for (int step = 0; step < 1; ++step) {
            build_order_block(fresh_bc());
            if (valid) {
                if (W.u8(GOI_S_NEW_FIXTURE, 0)) find_new_contacts(m, W);
                W.u8(GOI_S_NEW_FIXTURE, 0) = 0;
            }
            {
                const LaneViews c = fresh_views(m, L, lds, w0);
                collide_block(m, c.co, c.W, c.lm.valid, c.lm.leader, L.s);
            }
            if (valid) {
                solve_world(m, W, bd, CR, joint_rows(L, w0, lm.wl), L.s, L.dt, L.dbg);
                clear_toi_trace(W, L.dbg);
            }
            bool capped = false;
            if (L.s.continuous_physics) {
                const LaneViews t = fresh_views(m, L, lds, w0);
                capped = solve_toi_world<kOpaqueToi>(m, t.W, t.bd, t.TR, L.s, L.dt, t.lm.valid,
                                                     [&] { return fresh_views(m, L, lds, w0); }, L.dbg);
            }
            finish_step(L, fresh_views(m, L, lds, w0), overflow0, capped);
        }
        store_mirror_block(fresh_bc());
    } else {
        load_mirror_block(m, fresh_bc());
        for (int step = 0; step < L.n_steps; ++step) {
            if (step > 0) __syncthreads();  // the worlds' workspace writes of the previous step
            step_worlds<kOpaqueToi>(m, L, lds, w0);
        }
        store_mirror_block(fresh_bc());
    }
    if (L.cost && lane_now() == 0) {
        const uint64_t dt = block_clock() - t_start;
        L.cost[block_group(L)] = dt < 0x7fffffffull ? (int)dt : 0x7fffffff;
    }
}

// The 4-body rig's dimensions (5 bodies, 40 contact slots, 3 joints, 4 fixture rows, 8 worlds per wave) and its
// fixed-dimension step on a packed State (goi_b2_rig.hip): kernel instance per (n_steps > 1, revolute-only plain
// model). Returns the launch's HIP error. The fixed-dimension instances need the worlds per wave they were compiled
// for; worlds_per_wave picks it for these dimensions at full batches.
constexpr int kRigB = 5, kRigC = 40, kRigJ = 3, kRigR = 4;
constexpr int kRigS = kBlock == 64 ? 8 : 1;  // one world a block in the sequential host build
hipError_t launch_rig_step(const DModel& d, const Launch& L, bool multi, bool plain, dim3 grid, size_t lds,
                           hipStream_t st);

// The rig with 12 boxes (17 bodies, 128 contact slots, 3 joints, 16 fixture rows, 4 worlds per wave) and its
// fixed-dimension step on a packed State with a plain Model (goi_b2_island.hip), per n_steps > 1.
constexpr int kIslandB = 17, kIslandC = 128, kIslandJ = 3, kIslandR = 16;
constexpr int kIslandS = kBlock == 64 ? 4 : 1;
hipError_t launch_island_step(const DModel& d, const Launch& L, bool multi, dim3 grid, size_t lds, hipStream_t st);

}  // namespace goi
