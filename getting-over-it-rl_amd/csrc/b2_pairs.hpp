// b2_pairs.hpp - contact management on the device: the contact list order, b2Contact::Update, Collide,
// FindNewContacts through the static-terrain BVH, SynchronizeFixtures (goi_jax/box2d/pairs.py:38-207).
#pragma once

#include "b2_narrow.hpp"

namespace goi {

// Upper bound on contact slots per world the kernels handle (State capacity C <= kMaxC). Sets of list positions are
// 64-bit masks over one chunk of 64 positions at a time, so the walks below take the list in chunks.
constexpr int kMaxC = 256;

// The contact list (Box2D's m_contactList: newest first = descending key, pairs.py:12-13) is kept in the
// workspace as W.order(0 .. nlive-1). build_order_block ranks the live slots once per step; Collide's destructions
// and FindNewContacts' creations then update it in place (see collide_walk, find_new_contacts).

// Live slots in contact-list order: W.order(0 .. n-1); returns n.
GOI_D int list_order(const World& W) { return W.nlive(); }

// The list positions q0 <= i < min(q0 + 64, n) whose slot W.order(i) satisfies pred(slot), as a bit mask (bit i - q0):
// the lane group tests them together; a walk then visits the set bits in list order. pred must not depend on what
// that walk changes for the other positions of the chunk.
template <class F>
GOI_D unsigned long long list_mask(const World& W, int q0, int n, F&& pred) {
    unsigned long long mk = 0ull;
    const int e = min(q0 + 64, n);
    for (int i = q0 + W.sub; i < e; i += W.G)
        if (pred(W.order(i))) mk |= 1ull << (i - q0);
    return group_or(W.grp(), mk);
}

// A slot's old manifold points (their feature keys and impulses, State leaves), loaded by the caller before it
// evaluates the new manifold so that the loads are in flight meanwhile.
struct OldPoints {
    int o0, o1;
    float n0, n1, t0, t1;
};
GOI_D OldPoints old_points(const World& W, int k) {
    OldPoints p;
    p.o0 = W.i32(GOI_C_POINT_ID, 2 * k); p.o1 = W.i32(GOI_C_POINT_ID, 2 * k + 1);
    p.n0 = W.f(GOI_C_NORMAL_IMPULSE, 2 * k); p.n1 = W.f(GOI_C_NORMAL_IMPULSE, 2 * k + 1);
    p.t0 = W.f(GOI_C_TANGENT_IMPULSE, 2 * k); p.t1 = W.f(GOI_C_TANGENT_IMPULSE, 2 * k + 1);
    return p;
}

// b2Contact::Update's manifold part: new manifold, impulses carried over from the first old point with the same
// feature key, touching flag (pairs.py:56-83). Returns whether touching flipped.
GOI_D bool contact_update(const World& W, int k, const Manifold& mf, const OldPoints& old) {
    const int oldn = W.ccount(k);
    const int o0 = old.o0, o1 = old.o1;
    const float n0 = old.n0, n1 = old.n1, t0 = old.t0, t1 = old.t1;
    const int n = mf.count;
    float ni0 = 0.0f, ti0 = 0.0f, ni1 = 0.0f, ti1 = 0.0f;
    if (n > 0) {
        if (oldn > 0 && o0 == mf.id0) { ni0 = n0; ti0 = t0; }
        else if (oldn > 1 && o1 == mf.id0) { ni0 = n1; ti0 = t1; }
    }
    if (n > 1) {
        if (oldn > 0 && o0 == mf.id1) { ni1 = n0; ti1 = t0; }
        else if (oldn > 1 && o1 == mf.id1) { ni1 = n1; ti1 = t1; }
    }
    const bool touching = n > 0;
    const bool flip = touching != W.touching(k);
    W.set_touch_count(k, touching, n);
    if (n > 0) {
        W.i32(GOI_C_MTYPE, k) = mf.mtype;
        W.set2(GOI_C_LOCAL_NORMAL, k, mf.ln);
        W.set2(GOI_C_LOCAL_POINT, k, mf.lp);
        W.set2(GOI_C_POINT_LOCAL, 2 * k, mf.pl0);
        W.set2(GOI_C_POINT_LOCAL, 2 * k + 1, mf.pl1);
        W.i32(GOI_C_POINT_ID, 2 * k) = mf.id0;
        W.i32(GOI_C_POINT_ID, 2 * k + 1) = mf.id1;
    }
    // written only where the bits change (a contact that stays apart keeps its zeros): no store, no dirty line
    if (__float_as_uint(ni0) != __float_as_uint(n0)) W.f(GOI_C_NORMAL_IMPULSE, 2 * k) = ni0;
    if (__float_as_uint(ni1) != __float_as_uint(n1)) W.f(GOI_C_NORMAL_IMPULSE, 2 * k + 1) = ni1;
    if (__float_as_uint(ti0) != __float_as_uint(t0)) W.f(GOI_C_TANGENT_IMPULSE, 2 * k) = ti0;
    if (__float_as_uint(ti1) != __float_as_uint(t1)) W.f(GOI_C_TANGENT_IMPULSE, 2 * k + 1) = ti1;
    return flip;
}
GOI_D bool contact_update(const World& W, int k, const Manifold& mf) {
    return contact_update(W, k, mf, old_points(W, k));
}

// ---------------------------------------------------------------- block-cooperative task runs
//
// A block is one wavefront of S worlds, each run by G = 64 / S consecutive lanes (its lane group: every lane of the
// group runs the world's sequential code on the same data, and a few phases split their loops over the group). All
// 64 lanes share the work of task lists the worlds build (TOIs to compute, manifolds to evaluate). Each world numbers
// its tasks 0..n-1 and keeps their inputs in its workspace or its contact rows; coop_run hands task i of world o (the
// block's o-th) to some lane of the block.
struct Coop {
    World base;      // world 0's view (the fields common to the block)
    int* lds;        // the block's LDS workspace (world 0's base)
    int* scan;       // 64 ints after the workspaces
    uint32_t* rows;  // contact rows (Launch.scratch)
    int w0;          // the block's first world
    int lanes;       // lanes sharing the tasks (the block size)
    int G;           // lanes per world
    GOI_D World world(int o) const {
        World W = base;
        W.ws = lds + o;
        W.w = w0 + o;
        W.sub = 0;  // a task runs on one lane
        W.G = 1;
        return W;
    }
    GOI_D Rows task_rows(int o) const { return rows_of(rows, base.C, CF_N, base.S, w0 / base.S, o); }
    // world o's rows in SolveTOI (rows_world_major over the same tile)
    GOI_D Rows toi_rows(int o) const { return rows_world_major(rows, base.C, CF_N, base.S, w0 / base.S, o); }
};

// Called by all lanes of the block together; `my` = this lane's task count: the world's count on the first lane of
// its group, 0 on every other lane.
#ifdef GOI_HOST_BUILD
constexpr int kCoopLanes = 1;  // the block's lanes (one in the sequential host build)
#else
constexpr int kCoopLanes = 64;
#endif
template <typename F>
GOI_D void coop_run(const Coop& co, int my, F&& task) {
    const int lane = threadIdx.x;
    int incl = my;
    for (int d = 1; d < kCoopLanes; d <<= 1) {
        const int v = __shfl_up(incl, d, 64);
        if (lane >= d) incl += v;
    }
    const int total = __shfl(incl, kCoopLanes - 1, 64);
    if (total == 0) return;
    co.scan[lane] = incl;
    __syncthreads();  // scan entries and the owners' task inputs visible to the whole block
    for (int t = lane; t < total; t += co.lanes) {
        int lo = 0, hi = kCoopLanes - 1;  // owner: the first lane whose inclusive count exceeds t
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (co.scan[mid] > t) hi = mid; else lo = mid + 1;
        }
        task(lo / co.G, t - (lo ? co.scan[lo - 1] : 0));
    }
    __syncthreads();  // the results visible to their owners
}

// manifold fields of a Collide task in a contact row
enum { MT_MTYPE = 0, MT_COUNT, MT_LN, MT_LP = MT_LN + 2, MT_PL0 = MT_LP + 2, MT_PL1 = MT_PL0 + 2, MT_ID0 = MT_PL1 + 2,
       MT_ID1, MT_N };
static_assert(MT_N <= CF_N, "a manifold must fit a contact row");

// b2ContactManager::Collide (pairs.py:38-87): the list newest first, a contact with both bodies inactive skipped,
// separated fat AABBs destroy it (waking both bodies if it still had points), the rest updated (waking both bodies
// when touching flips). Wakes change which later contacts are visited, as in Box2D's walk.
//
// The manifolds are pure functions of the fixtures and the body transforms, which Collide does not change, so the
// walk runs in three passes with the same results: each world marks the live contacts with overlapping fat AABBs
// (W.cisl(k) = task index, or -1), the block evaluates all their manifolds (coop_run), and each world walks its list
// with the wake cascade, taking the precomputed manifold of each contact it updates. A contact the walk skips (both
// bodies asleep) had its manifold evaluated for nothing, which changes no result.
// The overlap tests split over the lane group; a contact's task index is the number of overlapping contacts before
// it in the list.
GOI_D int collide_mark(const DModel& m, const World& W) {
    const int n = list_order(W);
    int t0 = 0;  // overlapping contacts before the chunk
    for (int q0 = 0; q0 < n; q0 += 64) {
        const unsigned long long hits =
            list_mask(W, q0, n, [&](int k) { return overlap(fat_of(m, W, W.fa(k)), fat_of(m, W, W.fb(k))); });
        for (int i = q0 + W.sub; i < min(q0 + 64, n); i += W.G) {
            const int k = W.order(i), b = i - q0;
            if ((hits >> b) & 1ull) {
                const int t = t0 + __popcll(hits & ((1ull << b) - 1ull));
                W.newp(t) = k;
                W.cisl(k) = t;
            } else {
                W.cisl(k) = -1;
            }
        }
        t0 += __popcll(hits);
    }
    group_sync();
    return t0;
}

GOI_D void collide_task(const DModel& m, const Coop& co, int o, int i, const GoiSettings& s) {
    const World W = co.world(o);
    const Rows R = co.task_rows(o);
    const int k = W.newp(i);
    const int fa = W.fa(k), fb = W.fb(k);
    Manifold mf;
    evaluate(m, fa, fb, W.xf(W.ba(k)), W.xf(W.bb(k)), s, mf);
    R.seti(i, MT_MTYPE, mf.mtype);
    R.seti(i, MT_COUNT, mf.count);
    R.set2(i, MT_LN, mf.ln);
    R.set2(i, MT_LP, mf.lp);
    R.set2(i, MT_PL0, mf.pl0);
    R.set2(i, MT_PL1, mf.pl1);
    R.seti(i, MT_ID0, mf.id0);
    R.seti(i, MT_ID1, mf.id1);
}

GOI_D void collide_apply(const DModel& m, const World& W, const Rows& R) {
    const int n = list_order(W);
    // The list in chunks of 64 positions, in order. A chunk's passes read and write only its own positions' slots,
    // and the walk's wake state (awake) carries from one chunk to the next, as in Box2D's single walk.
    unsigned long long awake = 0ull;
    for (int b = 0; b < W.B; ++b) awake |= (unsigned long long)(W.awake(b) != 0) << b;
    const unsigned long long woken0 = awake;
    int removed = 0;  // destroyed contacts in the chunks before
    for (int q0 = 0; q0 < n; q0 += 64) {
        const int e = min(q0 + 64, n);
        // 1. per list position (split over the lane group): the contact is destroyed (its fat boxes separated), and
        //    visiting it wakes its bodies (a destroyed contact that had points; an update that flips touching)
        unsigned long long gone = 0ull, wakes = 0ull;
        for (int i = q0 + W.sub; i < e; i += W.G) {
            const int k = W.order(i);
            const int t = W.cisl(k);
            const bool g = t < 0;
            const bool wk = g ? W.ccount(k) > 0 : (R.geti(t, MT_COUNT) > 0) != W.touching(k);
            gone |= (unsigned long long)g << (i - q0);
            wakes |= (unsigned long long)wk << (i - q0);
        }
        gone = group_or(W.grp(), gone);
        wakes = group_or(W.grp(), wakes);
        // 2. Box2D's walk with its wake cascade, on bit masks: a contact is visited when one of its bodies is awake
        //    and not static, and a visit that wakes makes both bodies awake for the rest of the walk
        unsigned long long visit = 0ull;
        for (int i = q0; i < e; ++i) {
            const int k = W.order(i);
            const unsigned long long pair = (1ull << W.ba(k)) | (1ull << W.bb(k));
            if (!(awake & pair & ~W.smask)) continue;
            visit |= 1ull << (i - q0);
            if ((wakes >> (i - q0)) & 1ull) awake |= pair;
        }
        // 3. the visited contacts' destructions and updates (each touches only its own slot), split over the group
        for (int i = q0 + W.sub; i < e; i += W.G) {
            if (!((visit >> (i - q0)) & 1ull)) continue;
            const int k = W.order(i);
            if ((gone >> (i - q0)) & 1ull) {
                W.pair(k) = -1;
                W.mark_slot_changed(k);
                W.set_touch_count(k, false, 0);
                continue;
            }
            const int t = W.cisl(k);
            Manifold mf;
            mf.mtype = R.geti(t, MT_MTYPE);
            mf.count = R.geti(t, MT_COUNT);
            mf.ln = R.get2(t, MT_LN);
            mf.lp = R.get2(t, MT_LP);
            mf.pl0 = R.get2(t, MT_PL0);
            mf.pl1 = R.get2(t, MT_PL1);
            mf.id0 = R.geti(t, MT_ID0);
            mf.id1 = R.geti(t, MT_ID1);
            contact_update(W, k, mf);
        }
        group_sync();
        // 4. the destroyed contacts leave the list, the rest keep their order: a position moves down by the number of
        //    destroyed positions before it, below every position the group has yet to read (this chunk's reads are
        //    done, later chunks start above it)
        const unsigned long long dead = visit & gone;
        for (int i = q0 + W.sub; i < e; i += W.G) {
            if ((dead >> (i - q0)) & 1ull) continue;
            const int k = W.order(i);
            W.order(i - removed - __popcll(dead & ((1ull << (i - q0)) - 1ull))) = k;
        }
        group_sync();
        removed += __popcll(dead);
    }
    // the wakes (b2Body::SetAwake restarts the sleep timer only of a body that was asleep)
    for (int b = W.sub; b < W.B; b += W.G)
        if (((awake & ~woken0) >> b) & 1ull) W.wake(b);
    group_sync();
    W.nlive() = n - removed;
}

// Collide for the block: called by all lanes together; `valid` marks the lanes that run a world, `leader` the first
// lane of each world's group.
GOI_D void collide_block(const DModel& m, const Coop& co, const World& W, bool valid, bool leader,
                         const GoiSettings& s) {
    const int nt = valid ? collide_mark(m, W) : 0;
    coop_run(co, leader ? nt : 0, [&](int o, int i) { collide_task(m, co, o, i, s); });
    if (valid) collide_apply(m, W, co.task_rows(W.w - co.w0));
}

// Sorted buffer (the workspace's newp array) of the smallest new candidate indices of one FindNewContacts call,
// plus the count of all of them.
struct NewPairs {
    const World& W;
    int kept, total, cap;
    GOI_D void add(int p) {
        ++total;
        if (kept == cap && (cap == 0 || W.newp(kept - 1) < p)) return;
        int j = kept < cap ? kept++ : kept - 1;
        while (j > 0) {
            const int prev = W.newp(j - 1);
            if (!(prev > p)) break;
            W.newp(j) = prev;
            --j;
        }
        W.newp(j) = p;
    }
};

// whether a slot holds candidate p (the slots split over the lane group)
GOI_D bool slot_has_pair(const World& W, int p) {
    bool has = false;
    for (int k = W.sub; k < W.C; k += W.G) has |= W.pair(k) == p;
    return group_any(W.grp(), has);
}

// b2ContactManager::FindNewContacts (pairs.py:134-178) without scanning the candidate list: one walk of the static
// BVH with the union of the world's non-static fat AABBs; at a leaf, each entry is tested against each row's box and
// a hit maps to its candidate index through leaf_cand; the few non-static/non-static candidates are tested directly.
// New pairs (overlapping, a dynamic body, both active, no contact yet) take the lowest free slots in ascending
// candidate order with keys in that order, and enter the contact list at its head (newest first); a full table
// counts the rest in overflow. Every (leaf entry, row) is met once, so no candidate is found twice.
//
// query_rows restricts the search to candidates with at least one of the given non-static rows. The result is the
// full scan's as long as every candidate without such a row was decided by an earlier call of the same step whose
// boxes it still has and whose contacts still exist, and no earlier call dropped a candidate (overflow still 0):
// true after a TOI event, which moves only the rows it re-fattens and destroys no contact.
GOI_D void find_new_contacts(const DModel& m, const World& W, unsigned long long query_rows = ~0ull) {
    if (m.P == 0 || query_rows == 0ull) return;
    int n_free = 0;
    for (int k = W.sub; k < W.C; k += W.G) n_free += W.pair(k) < 0;
    n_free = group_sum(W.grp(), n_free);
    NewPairs np{W, 0, 0, n_free};
    // the pairs of this lane's slots (sub, sub + G, ...) in registers for the membership tests below, when they fit
    constexpr int kHeld = 8;
    const bool held_all = W.C <= kHeld * W.G;
    int held[kHeld];
#pragma unroll
    for (int j = 0; j < kHeld; ++j) {
        const int k = W.sub + j * W.G;
        held[j] = held_all && k < W.C ? W.pair(k) : -1;
    }
    const auto has_pair = [&](int p) {
        if (!held_all) return slot_has_pair(W, p);
        bool has = false;
#pragma unroll
        for (int j = 0; j < kHeld; ++j) has |= held[j] == p;
        return group_any(W.grp(), has);
    };
    // the fat boxes of all rows into the workspace; the queried rows on active bodies and a box around them
    unsigned long long rows = 0ull;
    float4 U = make_float4(kMaxFloat, kMaxFloat, -kMaxFloat, -kMaxFloat);
    bool nan_query = false;
    const auto row_box = [&](int r) {
        const int fr = 4 * W.frow(r);
        const float4 q = make_float4(W.f(GOI_F_FAT, fr), W.f(GOI_F_FAT, fr + 1), W.f(GOI_F_FAT, fr + 2),
                                     W.f(GOI_F_FAT, fr + 3));
        W.set_qbox(r, q);
        if (!((query_rows >> r) & 1ull) || !W.active(m.row[r].body)) return;
        rows |= 1ull << r;
        U.x = fminf(U.x, q.x); U.y = fminf(U.y, q.y); U.z = fmaxf(U.z, q.z); U.w = fmaxf(U.w, q.w);
        nan_query |= q.x != q.x || q.y != q.y || q.z != q.z || q.w != q.w;
    };
    if (m.R > 8) {
        // many rows: one a lane of the group, the results combined over it (the union box in any order: it only
        // filters the tree walk, and each of its hits is tested against the rows' own boxes)
        for (int r = W.sub; r < m.R; r += W.G) row_box(r);
        rows = group_or(W.grp(), rows);
        nan_query = group_or(W.grp(), nan_query ? 1ull : 0ull) != 0ull;
        for (int d = 1; d < W.G; d <<= 1) {
            U.x = fminf(U.x, lane_partner(U.x, d)); U.y = fminf(U.y, lane_partner(U.y, d));
            U.z = fmaxf(U.z, lane_partner(U.z, d)); U.w = fmaxf(U.w, lane_partner(U.w, d));
        }
        group_sync();  // the boxes one lane wrote are read by all
    } else {
        for (int r = 0; r < m.R; ++r) row_box(r);
    }
    // b2TestOverlap finds a box with a NaN coordinate overlapping every box, so such a row meets every static leaf:
    // a NaN union box then passes every node and leaf test below (and the row's own tests decide)
    if (nan_query) U = make_float4(kNaN, kNaN, kNaN, kNaN);
    // the static tree, depth first: the lane group tests a node's 8 child boxes together against the union box; per
    // level, the node and the mask of its overlapping children not yet visited (registers, selected by level). An
    // unused child slot holds an empty box (lower > upper), which a NaN union box would pass: the hit needs a
    // non-empty box too (the Model's static boxes are finite, checked at goi_model_create).
    if (rows && m.n_wnodes > 0) {
        int path[kWideDepth];
        unsigned masks[kWideDepth];
#pragma unroll
        for (int l = 0; l < kWideDepth; ++l) { path[l] = 0; masks[l] = 0u; }
        const auto children = [&](int nd) {
            unsigned hit = 0u;
            for (int j = W.sub; j < 8; j += W.G) {
                const float4 b = m.wnode[nd].box[j];
                if (overlap(U, b) && b.x <= b.z) hit |= 1u << j;
            }
            return group_or(W.grp(), hit);
        };
        masks[0] = children(0);
        int level = 0;
        for (;;) {
            int nd = 0;
            unsigned cm = 0u;
#pragma unroll
            for (int l = 0; l < kWideDepth; ++l)
                if (l == level) { nd = path[l]; cm = masks[l]; }
            if (cm == 0u) {
                if (level == 0) break;
                --level;
                continue;
            }
            const int k = __builtin_ctz(cm);
#pragma unroll
            for (int l = 0; l < kWideDepth; ++l)
                if (l == level) masks[l] = cm & (cm - 1u);
            const int ref = m.wnode[nd].ref[k];
            if (ref >= 0) {  // an inner node one level down
                const unsigned hit = children(ref);
                ++level;
#pragma unroll
                for (int l = 0; l < kWideDepth; ++l)
                    if (l == level) { path[l] = ref; masks[l] = hit; }
                continue;
            }
            // a leaf's entries (at most 8, one per lane) take the cheap union-box test; the few that pass are then
            // tested row by row (one copy of that code, not one per entry), and only a hit reads its candidate index
            const int first = (~ref) >> 4, cnt = (~ref) & 15;
            unsigned hits = 0u;
            for (int j = W.sub; j < cnt; j += W.G)
                if (overlap(m.leaf[first + j].fat, U) && W.active(m.leaf[first + j].info & 0xffff)) hits |= 1u << j;
            hits = group_or(W.grp(), hits);
            for (; hits; hits &= hits - 1u) {
                const int j = __builtin_ctz(hits);
                const float4 fj = m.leaf[first + j].fat;
                const int ij = m.leaf[first + j].info;
                for (unsigned long long left = rows; left; left &= left - 1) {
                    const int r = __builtin_ctzll(left);
                    if (!overlap(fj, W.get_qbox(r))) continue;
                    if (!(m.row[r].dynamic || (ij >> 16))) continue;
                    const int p = m.leaf_cand[(size_t)(first + j) * m.R + r];
                    if (p < 0 || has_pair(p)) continue;
                    np.add(p);
                }
            }
        }
    }
    // non-static x non-static candidates
    const auto dd_passes = [&](int i) {  // the tests that depend on candidate i alone
        const int4 d = m.dd_info[i];     // candidate, rows, bodies
        const int ra = d.y & 0xff, rb = d.y >> 8, ba = d.z & 0xff, bb = d.z >> 8;
        return (((query_rows >> ra) | (query_rows >> rb)) & 1ull) && overlap(W.get_qbox(ra), W.get_qbox(rb)) &&
               (W.is_dynamic(ba) || W.is_dynamic(bb)) && W.active(ba) && W.active(bb);
    };
    if (m.R > 8) {
        // many rows, so many candidates: those tests split over the group, 64 candidates at a time; the ones that
        // pass then take the membership test and join the new pairs in order
        for (int q0 = 0; q0 < m.n_dd; q0 += 64) {
            const int e = min(q0 + 64, m.n_dd);
            unsigned long long mk = 0ull;
            for (int i = q0 + W.sub; i < e; i += W.G)
                if (dd_passes(i)) mk |= 1ull << (i - q0);
            for (unsigned long long left = group_or(W.grp(), mk); left; left &= left - 1) {
                const int p = m.dd_info[q0 + __builtin_ctzll(left)].x;
                if (!has_pair(p)) np.add(p);
            }
        }
    } else {
        for (int i = 0; i < m.n_dd; ++i)
            if (dd_passes(i) && !has_pair(m.dd_info[i].x)) np.add(m.dd_info[i].x);
    }
    if (np.total == 0) return;
    const int base_key = W.i32(GOI_S_NEXT_KEY, 0);
    // the new contacts (keys base_key .. base_key + kept - 1) go to the head of the list, newest first
    const int nl = W.nlive();
    for (int i = nl - 1; i >= 0; --i) W.order(i + np.kept) = W.order(i);
    W.nlive() = nl + np.kept;
    int k = 0;
    for (int i = 0; i < np.kept; ++i) {
        while (W.pair(k) >= 0) ++k;
        W.order(np.kept - 1 - i) = k;
        const int p = W.newp(i);
        const int2 ab = m.pair[p];
        const int a = ab.x, b = ab.y;
        W.pair(k) = p;
        W.fa(k) = a;
        W.fb(k) = b;
        W.key(k) = base_key + i;
        W.mark_slot_changed(k);
        W.set_touch_count(k, false, 0);
        W.f(GOI_C_NORMAL_IMPULSE, 2 * k) = 0.0f;
        W.f(GOI_C_NORMAL_IMPULSE, 2 * k + 1) = 0.0f;
        W.f(GOI_C_TANGENT_IMPULSE, 2 * k) = 0.0f;
        W.f(GOI_C_TANGENT_IMPULSE, 2 * k + 1) = 0.0f;
        W.i32(GOI_C_POINT_ID, 2 * k) = 0;
        W.i32(GOI_C_POINT_ID, 2 * k + 1) = 0;
        W.f(GOI_C_FRICTION, k) = fsqrt(friction_of(m, W, a) * friction_of(m, W, b));  // b2MixFriction
        const float ra = restitution_of(m, W, a), rb = restitution_of(m, W, b);
        W.f(GOI_C_RESTITUTION, k) = ra > rb ? ra : rb;                                // b2MixRestitution
        W.f(GOI_C_TANGENT_SPEED, k) = 0.0f;
        const int ba = m.fix[a].body, bb = m.fix[b].body;
        W.set_bodies(k, ba, bb);
        W.wake(ba);
        W.wake(bb);
        ++k;
    }
    W.i32(GOI_S_NEXT_KEY, 0) = base_key + np.total;
    W.i32(GOI_S_OVERFLOW, 0) += np.total - np.kept;
}

// the bounds of vertices 1 .. n-1 (of kN slots) under transforms t1 and t2, joined to (lo1, hi1) and (lo2, hi2)
template <int kN>
GOI_D void aabb2_over(const V2* vs, int n, const Xf& t1, const Xf& t2, V2& lo1, V2& hi1, V2& lo2, V2& hi2) {
#pragma unroll
    for (int i = 1; i < kN; ++i) {
        if (i < n) {
            const V2 v1 = mul(t1, vs[i]), v2 = mul(t2, vs[i]);
            lo1.x = bmin(lo1.x, v1.x); lo1.y = bmin(lo1.y, v1.y);
            hi1.x = bmax(hi1.x, v1.x); hi1.y = bmax(hi1.y, v1.y);
            lo2.x = bmin(lo2.x, v2.x); lo2.y = bmin(lo2.y, v2.y);
            hi2.x = bmax(hi2.x, v2.x); hi2.y = bmax(hi2.y, v2.y);
        }
    }
}

// b2Shape::ComputeAABB of fixture f under transforms t1 and t2 (a1, a2). The fixture's vertex slots (all kPoly of
// them: the Model pads every shape) load in one batch with its type, count and radius.
GOI_D void shape_aabb2(const DModel& m, int f, const Xf& t1, const Xf& t2, float4& a1, float4& a2) {
    const float r = m.fix[f].radius;
    const int type = m.fix[f].type, n = m.fix[f].count;
    V2 vs[kPoly];
#pragma unroll
    for (int i = 0; i < kPoly; ++i) vs[i] = mvert(m, f, i);
    if (type == GOI_CIRCLE) {
        const V2 p1 = t1.p + mul(t1.q, vs[0]), p2 = t2.p + mul(t2.q, vs[0]);
        a1 = make_float4(p1.x - r, p1.y - r, p1.x + r, p1.y + r);
        a2 = make_float4(p2.x - r, p2.y - r, p2.x + r, p2.y + r);
        return;
    }
    V2 lo1 = mul(t1, vs[0]), hi1 = lo1, lo2 = mul(t2, vs[0]), hi2 = lo2;
    if (n <= 4) aabb2_over<4>(vs, n, t1, t2, lo1, hi1, lo2, hi2);  // a quad's loop covers 4 slots
    else aabb2_over<kPoly>(vs, n, t1, t2, lo1, hi1, lo2, hi2);
    a1 = make_float4(lo1.x - r, lo1.y - r, hi1.x + r, hi1.y + r);
    a2 = make_float4(lo2.x - r, lo2.y - r, hi2.x + r, hi2.y + r);
}

// b2Body::SynchronizeFixtures (pairs.py:181-207) for one non-static row r (fixture f) of a body moved from transform
// x1 (its sweep start) to x2: the swept AABB over both; b2DynamicTree::MoveProxy re-fattens only if the fat box no
// longer contains it. Returns whether it re-fattened. A body's rows are independent, so callers take one a lane.
GOI_D bool sync_row(const DModel& m, const World& W, int r, int f, const Xf& x1, const Xf& x2) {
    float4 a1, a2;
    shape_aabb2(m, f, x1, x2, a1, a2);
    float lx = bmin(a1.x, a2.x), ly = bmin(a1.y, a2.y);
    float ux = bmax(a1.z, a2.z), uy = bmax(a1.w, a2.w);
    const int fr = 4 * W.frow(r);
    const float fx0 = W.f(GOI_F_FAT, fr), fy0 = W.f(GOI_F_FAT, fr + 1);
    const float fx1 = W.f(GOI_F_FAT, fr + 2), fy1 = W.f(GOI_F_FAT, fr + 3);
    if (fx0 <= lx && fy0 <= ly && ux <= fx1 && uy <= fy1) return false;
    const V2 d = x2.p - x1.p;
    lx = lx - 0.1f; ly = ly - 0.1f; ux = ux + 0.1f; uy = uy + 0.1f;  // b2_aabbExtension
    const float ddx = 2.0f * d.x, ddy = 2.0f * d.y;                  // b2_aabbMultiplier
    if (ddx < 0.0f) lx = lx + ddx; else ux = ux + ddx;
    if (ddy < 0.0f) ly = ly + ddy; else uy = uy + ddy;
    W.f(GOI_F_FAT, fr) = lx;
    W.f(GOI_F_FAT, fr + 1) = ly;
    W.f(GOI_F_FAT, fr + 2) = ux;
    W.f(GOI_F_FAT, fr + 3) = uy;
    return true;
}

// the sweep-start transform of body b: q(a0), c0 - q * localCenter
GOI_D Xf sweep_start_xf(const World& W, int b) {
    Xf t;
    t.q = rot_of(W.f(GOI_B_A0, b));
    t.p = W.v2(GOI_B_C0, b) - mul(t.q, W.v2(GOI_B_LOCAL_CENTER, b));
    return t;
}

}  // namespace goi
