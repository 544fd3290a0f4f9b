// b2_step.hpp - the world-level phases of b2World::Step for one world (run by its lane group): Solve
// (step.py:73-251) and SolveTOI (toi.py:462-865), on top of the narrowphase, contact, solver, joint and TOI primitives.
#pragma once

#include "b2_toi.hpp"

namespace goi {

// ---------------------------------------------------------------- b2World::Solve for one world

// b2Island::Solve's warm start and velocity iterations (step.py:96-117) for island k alone, on its rows
GOI_D void island_velocities(const IslandBodies& ib, const Islands& I, const Rows& CR, const Rows& JRw, int k,
                             bool warm, bool v24, bool rev_only, int iterations) {
    int c0, c1, j0, j1;
    I.rows_of(k, c0, c1, j0, j1);
    if (warm)
        for (int i = c0; i < c1; ++i) cs_warm_start(ib, CR, i);
    for (int i = j0; i < j1; ++i) jn_warm_start(ib, JRw, i, v24, rev_only);
    for (int it = 0; it < iterations; ++it) {
        if (rev_only && v24)
            rev_velocity_sweep(ib, JRw, j0, j1);
        else
            for (int i = j0; i < j1; ++i) jn_solve_velocity(ib, JRw, i, v24, rev_only);
        cs_solve_velocity_sweep(ib, CR, c0, c1);
    }
}

// b2Island::Solve's position iterations (step.py:197-251) for island k alone; returns its positionSolved
GOI_D bool island_positions(const IslandBodies& ib, const Islands& I, const Rows& CR, const Rows& JRw, int k,
                            const GoiSettings& s, bool rev_only) {
    int c0, c1, j0, j1;
    I.rows_of(k, c0, c1, j0, j1);
    RotMemo qa, qb;
    for (int it = 0; it < s.position_iterations; ++it) {
        float min_sep = 0.0f;
        for (int i = c0; i < c1; ++i) {
            const PRow r = load_prow(CR, i);
            min_sep = bmin(min_sep, solve_prow(ib, r, s.baumgarte, r.mA, r.mB, r.iA, r.iB, s.linear_slop,
                                               s.max_linear_correction, qa, qb));
        }
        bool jok = true;
        for (int i = j0; i < j1; ++i)
            if (!jn_solve_position(ib, JRw, i, s, rev_only)) jok = false;
        if (min_sep >= -3.0f * s.linear_slop && jok) return true;
    }
    return false;
}

GOI_D void solve_world(const DModel& m, const World& W, const Bodies& bd, const Rows& CR, const Rows& JRw,
                            const GoiSettings& s, float dt, const GoiDebug& dbg) {
    const float dt_ratio = W.f(GOI_S_INV_DT0, 0) * dt;
    Islands I{W, 0, 0, 0};
    find_islands(m, W, I);
    const float h = dt;
    const float gx = W.f(GOI_S_GRAVITY, 0), gy = W.f(GOI_S_GRAVITY, 1);
    const bool warm = s.warm_starting != 0;
    const bool v24 = s.revolute_v24 != 0;
    // A world of several islands has its group's lanes solve them side by side (lane sub takes islands sub, sub + G,
    // ...; IslandBodies). If a row would change a static body, the world's velocity phase runs again from the
    // integration below with the islands one after another, as is its position phase from the integrated poses.
    bool par = m.island_lanes && I.n > 1;
    int* const changed = &W.stack(0);  // the flag (the search's stack is free after find_islands)
    for (;;) {
        // integrate velocities of dynamic island bodies; the sweep starts at the current pose (bodies are independent
        // here and in the other per-body loops below: one body per lane of the group)
        for (int b = W.sub; b < W.B; b += W.G) {
            V2 v = W.v2(GOI_B_V, b);
            float w = W.f(GOI_B_W, b);
            const V2 c = W.v2(GOI_B_C, b);
            const float a = W.f(GOI_B_A, b);
            if (I.body_island(b) >= 0) {
                if (W.is_dynamic(b)) {
                    const float gs = W.f(GOI_B_GRAVITY_SCALE, b), im = W.f(GOI_B_INV_MASS, b);
                    const float ax = gs * gx + im * W.f(GOI_B_FORCE, 2 * b);
                    const float ay = gs * gy + im * W.f(GOI_B_FORCE, 2 * b + 1);
                    const float vx = v.x + h * ax, vy = v.y + h * ay;
                    const float ww = w + h * W.f(GOI_B_INV_INERTIA, b) * W.f(GOI_B_TORQUE, b);
                    const float ld = 1.0f / (1.0f + h * W.f(GOI_B_LINEAR_DAMPING, b));
                    const float ad = 1.0f / (1.0f + h * W.f(GOI_B_ANGULAR_DAMPING, b));
                    v = mk(vx * ld, vy * ld);
                    w = ww * ad;
                }
                W.set2(GOI_B_C0, b, c);
                W.f(GOI_B_A0, b) = a;
            }
            bd.set_v(b, v, w);
            bd.set_c(b, c, a);
            const Rot q = rot_of(a);
            bd.at(6, b) = q.c;
            bd.at(7, b) = q.s;
        }
        group_sync();
        // the constraint rows are independent of each other: the world's lane group prepares them together (one row
        // per lane), then every lane warm-starts them in order
        for (int i = W.sub; i < I.nc; i += W.G) {
            const int slot = I.corder(i);
            const int ia = W.ba(slot), ib = W.bb(slot);
            Rot qA, qB;
            qA.c = bd.at(6, ia); qA.s = bd.at(7, ia);
            qB.c = bd.at(6, ib); qB.s = bd.at(7, ib);
            cs_prepare(m, W, bd, CR, i, slot, warm, dt_ratio, qA, qB, s.velocity_threshold);
        }
        for (int i = W.sub; i < I.nj; i += W.G) {
            const int jid = I.jorder(i);
            const int ia = m.joint[jid].a, ib = m.joint[jid].b;
            Rot qA, qB;
            qA.c = bd.at(6, ia); qA.s = bd.at(7, ia);
            qB.c = bd.at(6, ib); qB.s = bd.at(7, ib);
            jn_prepare(m, W, bd, JRw, i, jid, s, dt, dt_ratio, warm, qA, qB);
        }
        group_sync();  // rows written by one lane of the group are read by all
        if (par) {
            *changed = 0;
            group_sync();
            for (int k = W.sub; k < I.n; k += W.G)
                island_velocities(IslandBodies{bd, I.bodies_of(k), changed}, I, CR, JRw, k, warm, v24, m.rev_only,
                                  s.velocity_iterations);
            group_sync();
            if (*changed == 0) break;
            par = false;
            group_sync();
            continue;
        }
        if (warm)
            for (int i = 0; i < I.nc; ++i) cs_warm_start(bd, CR, i);
        for (int i = 0; i < I.nj; ++i) jn_warm_start(bd, JRw, i, v24, m.rev_only);
        for (int it = 0; it < s.velocity_iterations; ++it) {
            if (m.rev_only && v24)
                rev_velocity_sweep(bd, JRw, 0, I.nj);
            else
                for (int i = 0; i < I.nj; ++i) jn_solve_velocity(bd, JRw, i, v24, m.rev_only);
            cs_solve_velocity_sweep(bd, CR, 0, I.nc);
        }
        break;
    }
    // StoreImpulses (contact_solver.py:293-304), rows split over the lane group
    for (int i = W.sub; i < I.nc; i += W.G) {
        const int slot = CR.geti(i, CF_SLOT), cnt = CR.geti(i, CF_COUNT);
        if (cnt > 0) {
            W.f(GOI_C_NORMAL_IMPULSE, 2 * slot) = CR.getf(i, CF_NI0);
            W.f(GOI_C_TANGENT_IMPULSE, 2 * slot) = CR.getf(i, CF_TI0);
        }
        if (cnt > 1) {
            W.f(GOI_C_NORMAL_IMPULSE, 2 * slot + 1) = CR.getf(i, CF_NI1);
            W.f(GOI_C_TANGENT_IMPULSE, 2 * slot + 1) = CR.getf(i, CF_TI1);
        }
    }
    for (int i = W.sub; i < I.nj; i += W.G) jn_store(W, JRw, i, v24);
    group_sync();
    // integrate positions with the per-step clamps (step.py:120-135)
    const float max_t = s.clamps_per_second ? s.max_translation * h : s.max_translation;
    const float max_r = s.clamps_per_second ? s.max_rotation * h : s.max_rotation;
    for (int b = W.sub; b < W.B; b += W.G) {
        if (I.body_island(b) < 0) continue;
        V2 v = bd.v(b);
        float w = bd.w(b);
        const V2 t = h * v;
        if (dot(t, t) > max_t * max_t) {
            const float ratio = max_t / length(t);
            v = mk(v.x * ratio, v.y * ratio);
        }
        const float rot = h * w;
        if (rot * rot > max_r * max_r) w = w * (max_r / babs(rot));
        bd.set_c(b, bd.c(b) + h * v, bd.a(b) + h * w);
        bd.set_v(b, v, w);
    }
    group_sync();
    // position iterations with per-island early exit (step.py:197-251)
    unsigned long long done = 0ull, all = I.n >= 64 ? ~0ull : ((1ull << I.n) - 1ull);
    if (par) {
        *changed = 0;
        group_sync();
        for (int k = W.sub; k < I.n; k += W.G)
            if (island_positions(IslandBodies{bd, I.bodies_of(k), changed}, I, CR, JRw, k, s, m.rev_only))
                done |= 1ull << k;
        done = group_or(W.grp(), done);
        group_sync();
        if (*changed != 0) {  // from the integrated poses again, the islands one after another
            for (int b = W.sub; b < W.B; b += W.G)
                if (I.body_island(b) >= 0) bd.set_c(b, W.v2(GOI_B_C, b) + h * bd.v(b), W.f(GOI_B_A, b) + h * bd.w(b));
            group_sync();
            done = 0ull;
            par = false;
        }
    }
    RotMemo qa, qb;
    for (int it = 0; !par && it < s.position_iterations && done != all; ++it) {
        unsigned long long jbad = 0ull;
        for (int i = 0; i < I.n; ++i) W.fwork(i) = 0.0f;  // min separation per island
        for (int i = 0; i < I.nc; ++i) {
            const int isl = I.contact_island(I.corder(i));
            if ((done >> isl) & 1ull) continue;
            const PRow r = load_prow(CR, i);
            W.fwork(isl) = bmin(W.fwork(isl), solve_prow(bd, r, s.baumgarte, r.mA, r.mB, r.iA, r.iB, s.linear_slop,
                                                         s.max_linear_correction, qa, qb));
        }
        for (int i = 0; i < I.nj; ++i) {
            const int isl = I.joint_island(JRw.geti(i, JF_JID));
            if ((done >> isl) & 1ull) continue;
            if (!jn_solve_position(bd, JRw, i, s, m.rev_only)) jbad |= 1ull << isl;
        }
        const float okay_sep = -3.0f * s.linear_slop;
        for (int i = 0; i < I.n; ++i)
            if (!((done >> i) & 1ull) && W.fwork(i) >= okay_sep && !((jbad >> i) & 1ull)) done |= 1ull << i;
    }
    // write back + SynchronizeTransform
    for (int b = W.sub; b < W.B; b += W.G) {
        if (I.body_island(b) < 0) continue;
        const V2 c = bd.c(b);
        const float a = bd.a(b);
        W.set2(GOI_B_C, b, c);
        W.f(GOI_B_A, b) = a;
        W.set2(GOI_B_V, b, bd.v(b));
        W.f(GOI_B_W, b) = bd.w(b);
        const Rot q = rot_of(a);
        W.set2(GOI_B_XF_P, b, c - mul(q, W.v2(GOI_B_LOCAL_CENTER, b)));
        W.f(GOI_B_XF_Q, 2 * b) = q.c;
        W.f(GOI_B_XF_Q, 2 * b + 1) = q.s;
    }
    group_sync();
    // sleep per island (step.py:153-168)
    unsigned long long isl_sleep = 0ull;
    if (s.allow_sleep) {
        const float lin_tol = s.linear_sleep_tolerance * s.linear_sleep_tolerance;
        const float ang_tol = s.angular_sleep_tolerance * s.angular_sleep_tolerance;
        for (int i = 0; i < I.n; ++i) W.fwork(i) = kMaxFloat;  // min sleep time per island
        for (int b = 0; b < W.B; ++b) {
            const int isl = I.body_island(b);
            if (isl < 0 || W.is_static(b)) continue;
            const V2 v = W.v2(GOI_B_V, b);
            const float w = W.f(GOI_B_W, b);
            const bool moving = !W.u8(GOI_B_ALLOW_SLEEP, b) || w * w > ang_tol || dot(v, v) > lin_tol;
            if (moving) {
                W.f(GOI_B_SLEEP_TIME, b) = 0.0f;
                W.fwork(isl) = 0.0f;
            } else {
                const float st = W.f(GOI_B_SLEEP_TIME, b) + h;
                W.f(GOI_B_SLEEP_TIME, b) = st;
                W.fwork(isl) = bmin(W.fwork(isl), st);
            }
        }
        for (int i = 0; i < I.n; ++i)
            if (W.fwork(i) >= s.time_to_sleep && ((done >> i) & 1ull)) isl_sleep |= 1ull << i;
        for (int b = 0; b < W.B; ++b) {
            const int isl = I.body_island(b);
            if (isl < 0 || W.is_static(b) || !((isl_sleep >> isl) & 1ull)) continue;
            W.f(GOI_B_SLEEP_TIME, b) = 0.0f;
            W.awake(b) = 0;
            W.set2(GOI_B_V, b, mk(0.0f, 0.0f));
            W.f(GOI_B_W, b) = 0.0f;
            W.set2(GOI_B_FORCE, b, mk(0.0f, 0.0f));
            W.f(GOI_B_TORQUE, b) = 0.0f;
        }
    }
    // static bodies end with the awake flag of the last island that included them (step.py:173-194)
    for (int b = 0; b < W.B; ++b) {
        if (!W.is_static(b)) continue;
        int last = -1;
        for (int c = W.sub; c < W.C; c += W.G) {  // slots split over the lane group
            const int isl = I.contact_island(c);
            if (isl < 0) continue;
            if (W.ba(c) == b || W.bb(c) == b) last = max(last, isl);
        }
        last = group_max(W.grp(), last);
        for (int j = 0; j < W.J; ++j) {
            const int isl = I.joint_island(j);
            if (isl >= 0 && (m.joint[j].a == b || m.joint[j].b == b)) last = max(last, isl);
        }
        if (last < 0) continue;
        W.awake(b) = !((isl_sleep >> last) & 1ull);
        W.f(GOI_B_SLEEP_TIME, b) = 0.0f;
    }
    if (dbg.body_island)
        for (int b = 0; b < W.B; ++b) dbg.body_island[(size_t)b * W.pitch + W.w] = I.body_island(b);
    if (dbg.contact_island)
        for (int c = 0; c < W.C; ++c) dbg.contact_island[(size_t)c * W.pitch + W.w] = I.contact_island(c);
    if (dbg.contact_order)
        for (int c = 0; c < W.C; ++c) dbg.contact_order[(size_t)c * W.pitch + W.w] = c < I.nc ? I.corder(c) : -1;
    if (dbg.n_islands) dbg.n_islands[W.w] = I.n;
    // SynchronizeFixtures of the non-static island bodies, then FindNewContacts for the rows it re-fattened: Box2D's
    // move buffer (b2BroadPhase::m_moveBuffer), empty at the end of every step. A candidate between rows whose fat
    // AABBs did not change was decided by the last search of the previous step and its contact, if any, still exists
    // (Collide destroys only contacts whose fat AABBs separated), so the result is the full scan's; a world that ever
    // dropped a candidate (overflow) keeps scanning all rows, since its dropped pairs may now find a slot.
    unsigned long long refat = 0ull;
    for (int r = W.sub; r < m.R; r += W.G) {  // the rows are independent: one per lane of the group
        const MRow row = m.row[r];
        const int b = row.body;
        if (I.body_island(b) < 0 || W.is_static(b)) continue;
        if (sync_row(m, W, r, row.fixture, sweep_start_xf(W, b), W.xf(b))) refat |= 1ull << r;
    }
    refat = group_or(W.grp(), refat);
    group_sync();
    find_new_contacts(m, W, W.i32(GOI_S_OVERFLOW, 0) == 0 ? refat : ~0ull);
}

// ---------------------------------------------------------------- b2World::SolveTOI for one world

GOI_D bool pair_rule(const DModel& m, const World& W, const GoiSettings& s, int a, int b) {
    const bool dyn_a = W.is_dynamic(a), dyn_b = W.is_dynamic(b);
    const bool bul_a = W.bullet(a), bul_b = W.bullet(b);
    const bool stock = bul_a || !dyn_a || bul_b || !dyn_b;
    if (!s.unity_toi) return stock;
    const bool rule = bul_a || bul_b ||
                      (!dyn_b ? W.continuous(a) : (!dyn_a ? W.continuous(b) : false));
    return stock && rule;
}

// ---------------------------------------------------------------- the min-TOI search (toi.py:488-558)
//
// Box2D's search walks the contact list once: for each contact without a cached TOI it aligns the two sweeps
// (b2Sweep::Advance of the body with the smaller alpha0) and computes the TOI, then keeps the minimum. Alignments
// depend only on alpha0 values, never on TOI results, so the walk splits into three passes with the same results:
//   1. toi_search_prepare (each world, list order): the alignments, and the list of the contacts that need a TOI
//      (the world's newp array);
//   2. toi_task under coop_run (the whole wavefront): the TOIs of all worlds of the block, over all 64 lanes;
//   3. toi_search_pick (each world, list order): the minimum with the reference's tie rule.
// A TOI's inputs are the two sweeps as aligned at its contact. They stay the bodies' sweeps in the workspace until
// one of the two bodies is advanced again later in the walk: only then (rarely: a body met by bodies of two larger
// alpha0 values) are the task's sweeps and alpha0 copied into its row of the world's TOI rows (the task is frozen,
// kFrozenTask in its newp entry), before the advance. Pass 2 reads the sweeps of the other tasks from the workspace.

// task snapshot fields in a TOI row
enum { TT_ALPHA0 = 0, TT_SA, TT_SB = TT_SA + 8, TT_N = TT_SB + 8 };
static_assert(TT_N <= CF_N, "TOI task snapshot must fit a contact row");
constexpr int kFrozenTask = 1 << 30;  // newp flag of a task whose inputs are in its row

GOI_D void put_sweep(const Rows& R, int row, int f, const Sweep& sw) {
    R.set2(row, f, sw.lc); R.set2(row, f + 2, sw.c0); R.set2(row, f + 4, sw.c);
    R.setf(row, f + 6, sw.a0); R.setf(row, f + 7, sw.a);
}
GOI_D Sweep get_sweep(const Rows& R, int row, int f) {
    Sweep sw;
    sw.lc = R.get2(row, f); sw.c0 = R.get2(row, f + 2); sw.c = R.get2(row, f + 4);
    sw.a0 = R.getf(row, f + 6); sw.a = R.getf(row, f + 7);
    return sw;
}

// freezes tasks 0 .. nt-1 that involve body b and are not frozen yet (b is about to be advanced)
GOI_D void freeze_tasks(const World& W, const Rows& CR, int nt, int b) {
    for (int t = 0; t < nt; ++t) {
        const int k = W.newp(t);
        if (k & kFrozenTask) continue;
        const int A = W.ba(k), Bb = W.bb(k);
        if (A != b && Bb != b) continue;
        CR.setf(t, TT_ALPHA0, W.f(GOI_T_ALPHA0, A));  // both bodies' alpha0 since the task's alignment
        put_sweep(CR, t, TT_SA, body_sweep(W, A));
        put_sweep(CR, t, TT_SB, body_sweep(W, Bb));
        W.newp(t) = k | kFrozenTask;
    }
}

// pass 1; returns the number of TOI tasks, whose slots are W.newp(0 .. n-1) (with kFrozenTask on frozen ones)
GOI_D int toi_search_prepare(const DModel& m, const World& W, const Rows& CR, const GoiSettings& s) {
    const int n = list_order(W);
    int nt = 0;
    for (int q0 = 0; q0 < n; q0 += 64) {
        // the chunk's contacts that need a TOI (the lane group tests them together; the walk below changes only the
        // flag of the contact it visits), then the alignments in list order
        const unsigned long long need = list_mask(W, q0, n, [&](int c) {
            if (!W.ten(c) || W.tcount(c) > kMaxSubSteps || W.tflag(c)) return false;
            const int A = W.ba(c), Bb = W.bb(c);
            const bool act_a = W.awake(A) && !W.is_static(A);
            const bool act_b = W.awake(Bb) && !W.is_static(Bb);
            return (act_a || act_b) && pair_rule(m, W, s, A, Bb);
        });
        // No alignment happens when no needed contact's bodies differ in alpha0 (the first search of a step, where
        // every body starts at 0): the chunk's tasks are then its needed contacts in list order, which the lane group
        // sets up together, each lane at its own positions.
        const int e = min(q0 + 64, n);
        bool align = false;
        for (int i = q0 + W.sub; i < e; i += W.G) {
            if (!((need >> (i - q0)) & 1ull)) continue;
            const int c = W.order(i);
            align |= W.f(GOI_T_ALPHA0, W.ba(c)) != W.f(GOI_T_ALPHA0, W.bb(c));
        }
        if (!group_any(W.grp(), align)) {
            for (int i = q0 + W.sub; i < e; i += W.G) {
                if (!((need >> (i - q0)) & 1ull)) continue;
                const int c = W.order(i);
                W.newp(nt + __popcll(need & ((1ull << (i - q0)) - 1ull))) = c;
                W.set_tflag(c, 1);  // the toi itself arrives in pass 2
            }
            nt += __popcll(need);
            group_sync();
            continue;
        }
        for (unsigned long long left = need; left; left &= left - 1) {
            const int c = W.order(q0 + __builtin_ctzll(left));
            const int A = W.ba(c), Bb = W.bb(c);
            const float alA = W.f(GOI_T_ALPHA0, A), alB = W.f(GOI_T_ALPHA0, Bb);
            if (alA < alB) {
                freeze_tasks(W, CR, nt, A);
                sweep_advance(W, A, alB);
            } else if (alB < alA) {
                freeze_tasks(W, CR, nt, Bb);
                sweep_advance(W, Bb, alA);
            }
            W.newp(nt++) = c;
            W.set_tflag(c, 1);  // the toi itself arrives in pass 2
        }
        group_sync();
    }
    return nt;
}

// pass 2: the TOI of task i of the block's world o
GOI_D void toi_task(const DModel& m, const Coop& co, int o, int i, float linear_slop) {
    const World W = co.world(o);
    const int k = W.newp(i);
    const int c = k & ~kFrozenTask;
    const int A = W.ba(c), Bb = W.bb(c);
    Sweep sa, sb;
    float alpha0;
    if (k & kFrozenTask) {
        const Rows R = co.toi_rows(o);
        alpha0 = R.getf(i, TT_ALPHA0);
        sa = get_sweep(R, i, TT_SA);
        sb = get_sweep(R, i, TT_SB);
    } else {
        alpha0 = W.f(GOI_T_ALPHA0, A);
        sa = body_sweep(W, A);
        sb = body_sweep(W, Bb);
    }
    float beta;
    const int st = time_of_impact(proxy_of(m, W.fa(c)), sa, proxy_of(m, W.fb(c)), sb, linear_slop, beta);
    W.ttoi(c) = st == kToiTouching ? bmin(alpha0 + (1.0f - alpha0) * beta, 1.0f) : 1.0f;
}

// pass 3; returns whether an event was found
GOI_D bool toi_search_pick(const World& W, const GoiSettings& s, int& min_slot, float& min_alpha) {
    const int n = list_order(W);
    // the list walk's running minimum, over the lane group: each lane walks its own positions, then the lanes combine
    // (smaller alpha wins; equal alphas keep the earlier position, or the later one under toi_tie_oldest)
    int at = -1;
    float best_alpha = 1.0f;
    for (int i = W.sub; i < n; i += W.G) {
        const int c = W.order(i);
        if (!W.ten(c) || W.tcount(c) > kMaxSubSteps || !W.tflag(c)) continue;
        const float alpha = W.ttoi(c);
        if (alpha < 1.0f && (s.toi_tie_oldest ? alpha <= best_alpha : alpha < best_alpha)) {
            at = i;
            best_alpha = alpha;
        }
    }
    for (int d = 1; d < W.G; d <<= 1) {
        const float oa = lane_partner(best_alpha, d);
        const int oi = lane_partner(at, d);
        const bool later = oi > at;
        if (oi >= 0 && (oa < best_alpha || (oa == best_alpha && (at < 0 || (s.toi_tie_oldest ? later : !later))))) {
            best_alpha = oa;
            at = oi;
        }
    }
    const int best = at >= 0 ? W.order(at) : -1;
    min_slot = best;
    min_alpha = best_alpha;
    const float done_alpha = 1.0f - 10.0f * kEps;
    return best >= 0 && !(done_alpha < best_alpha);
}

// position-constraint fields of contact slot `slot` into row i (the TOI island's b2ContactPositionConstraint); mf is
// the touching manifold the slot was just updated with (its State leaves hold the same values)
GOI_D void cs_position_row(const DModel& m, const World& W, const Rows& R, int i, int slot, const Manifold& mf) {
    const int fa = W.fa(slot), fb = W.fb(slot);
    const int ia = W.ba(slot), ib = W.bb(slot);
    R.seti(i, CF_SLOT, slot); R.seti(i, CF_IA, ia); R.seti(i, CF_IB, ib);
    R.seti(i, CF_PC_COUNT, mf.count); R.seti(i, CF_MTYPE, mf.mtype);
    R.set2(i, CF_LN, mf.ln); R.set2(i, CF_LP, mf.lp);
    R.set2(i, CF_PL0, mf.pl0); R.set2(i, CF_PL1, mf.pl1);
    R.set2(i, CF_LCA, W.v2(GOI_B_LOCAL_CENTER, ia)); R.set2(i, CF_LCB, W.v2(GOI_B_LOCAL_CENTER, ib));
    R.setf(i, CF_RADA, m.fix[fa].radius); R.setf(i, CF_RADB, m.fix[fb].radius);
}

// The debug trace of event `ev` of a world (GoiDebug's toi_* arrays, when given): its slot, alpha and island size,
// and the slots of its nc island rows (-1 beyond them); the group's lanes split the rows.
GOI_D void record_toi_event(const World& W, const GoiDebug& dbg, int ev, int slot, float alpha, int nc, int nb,
                            const Rows& CR) {
    if (!dbg.toi_event_slot || ev >= GOI_DEBUG_TOI_EVENTS) return;
    const size_t P = (size_t)W.pitch;
    if (W.sub == 0) {
        dbg.toi_event_slot[ev * P + W.w] = slot;
        dbg.toi_event_alpha[ev * P + W.w] = (int)__float_as_uint(alpha);
        dbg.toi_event_island[ev * P + W.w] = nc | (nb << 16);
    }
    for (int i = W.sub; i < GOI_DEBUG_TOI_ROWS; i += W.G)
        dbg.toi_island_rows[((size_t)ev * GOI_DEBUG_TOI_ROWS + i) * P + W.w] = i < nc ? CR.geti(i, CF_SLOT) : -1;
}

// The blank trace (no event) of every event entry of a world, written before SolveTOI.
GOI_D void clear_toi_trace(const World& W, const GoiDebug& dbg) {
    if (!dbg.toi_event_slot) return;
    const size_t P = (size_t)W.pitch;
    for (int e = W.sub; e < GOI_DEBUG_TOI_EVENTS; e += W.G) {
        dbg.toi_event_slot[e * P + W.w] = -1;
        dbg.toi_event_alpha[e * P + W.w] = 0;
        dbg.toi_event_island[e * P + W.w] = 0;
    }
    for (int i = W.sub; i < GOI_DEBUG_TOI_EVENTS * GOI_DEBUG_TOI_ROWS; i += W.G) dbg.toi_island_rows[i * P + W.w] = -1;
}

// b2Island::SolveTOI's position passes (toi.py:738-760) on the island's nc rows, the poses in bd: at most 20 passes,
// each over the rows in order, until the smallest separation is at least -1.5 linear slop. Only the TOI pair (A, Bb)
// has mass. The rows do not change across the passes: the first two (most islands have one or two) stay in
// registers, loaded once, each with its own rotation memos (a static side's rotation is then computed once per
// event); rows past them are read from the row tile in each pass and share a pair of memos.
GOI_D void toi_positions(const Bodies& bd, const Rows& CR, int nc, int A, int Bb, float mA_, float iA_, float mB_,
                         float iB_, const GoiSettings& s) {
    const PRow r0 = load_prow(CR, 0);
    const PRow r1 = nc > 1 ? load_prow(CR, 1) : r0;
    const auto masses = [&](const PRow& r, float& mA, float& mB, float& iA, float& iB) {
        const bool ta = r.ia == A || r.ia == Bb, tb = r.ib == A || r.ib == Bb;
        mA = ta ? (r.ia == A ? mA_ : mB_) : 0.0f;
        iA = ta ? (r.ia == A ? iA_ : iB_) : 0.0f;
        mB = tb ? (r.ib == A ? mA_ : mB_) : 0.0f;
        iB = tb ? (r.ib == A ? iA_ : iB_) : 0.0f;
    };
    float m0A, m0B, i0A, i0B, m1A, m1B, i1A, i1B;
    masses(r0, m0A, m0B, i0A, i0B);
    masses(r1, m1A, m1B, i1A, i1B);
    RotMemo qa0, qb0, qa1, qb1, qa, qb;
    for (int it = 0; it < 20; ++it) {
        float min_sep = solve_prow(bd, r0, s.toi_baumgarte, m0A, m0B, i0A, i0B, s.linear_slop, s.max_linear_correction,
                                   qa0, qb0);
        if (nc > 1)
            min_sep = bmin(min_sep, solve_prow(bd, r1, s.toi_baumgarte, m1A, m1B, i1A, i1B, s.linear_slop,
                                               s.max_linear_correction, qa1, qb1));
        for (int i = 2; i < nc; ++i) {
            const PRow cur = load_prow(CR, i);
            float mA, mB, iA, iB;
            masses(cur, mA, mB, iA, iB);
            min_sep = bmin(min_sep, solve_prow(bd, cur, s.toi_baumgarte, mA, mB, iA, iB, s.linear_slop,
                                               s.max_linear_correction, qa, qb));
        }
        if (min_sep >= -1.5f * s.linear_slop) break;
    }
}

// The same passes when exactly one of the TOI pair has mass (TRow): its pose in registers, rows 0 and 1 as TRows in
// registers, the others as TRows in the row tile. Returns false, with bd untouched, when the event is not of that
// form or the guard fails; toi_positions then runs the passes.
GOI_D bool toi_positions_one_body(const Bodies& bd, const Rows& CR, int nc, int A, int Bb, float mA_, float iA_,
                                  float mB_, float iB_, const GoiSettings& s) {
    const bool movA = mA_ != 0.0f || iA_ != 0.0f, movB = mB_ != 0.0f || iB_ != 0.0f;
    if (movA == movB) return false;
    const int M = movA ? A : Bb;
    const float mM = movA ? mA_ : mB_, iM = movA ? iA_ : iB_;
    const float maxc = s.max_linear_correction;
    if (!(mM >= 0x1p-40f && mM < 0x1p40f && iM >= 0.0f && iM < 0x1p40f && maxc >= 0.0f && maxc <= 1024.0f))
        return false;
    V2 cM = bd.c(M);
    float aM = bd.a(M);
    if (!below40(cM)) return false;
    TRow t0, t1;
    bool ok = make_trow(bd, load_prow(CR, 0), M, mM, iM, t0);
    if (nc > 1) ok = make_trow(bd, load_prow(CR, 1), M, mM, iM, t1) && ok;
    for (int i = 2; i < nc; ++i) {
        TRow t;
        ok = make_trow(bd, load_prow(CR, i), M, mM, iM, t) && ok;
        store_trow(CR, i, t);  // each lane of the group stores and reads back its own copy of the same words
    }
    if (!ok) return false;
    float acc = fabsf(aM) * 0x1p40f;
    const float b = s.toi_baumgarte, slop = s.linear_slop;
    for (int it = 0; it < 20; ++it) {
        float min_sep = trow_pass(t0, b, slop, maxc, cM, aM, acc);
        if (nc > 1) min_sep = bmin(min_sep, trow_pass(t1, b, slop, maxc, cM, aM, acc));
        for (int i = 2; i < nc; ++i) min_sep = bmin(min_sep, trow_pass(load_trow(CR, i), b, slop, maxc, cM, aM, acc));
        if (min_sep >= -1.5f * slop) break;
    }
    if (!(acc < 0x1p60f)) return false;
    bd.set_c(M, cM, aM);
    return true;
}

// b2Island::SolveTOI's velocity passes (toi.py:762-772) for an island of at most two rows whose only body with mass
// is one of the TOI pair (TVRow): its velocity in registers. Returns false, with bd and the rows untouched, when the
// island is not of that form or the guard fails; the event then runs solve_vrow's passes.
GOI_D bool toi_velocities_one_body(const Bodies& bd, const Rows& CR, int nc, int A, int Bb, float mA_, float iA_,
                                   float mB_, float iB_, int iterations) {
    const bool movA = mA_ != 0.0f || iA_ != 0.0f, movB = mB_ != 0.0f || iB_ != 0.0f;
    if (nc > 2 || movA == movB) return false;
    const int M = movA ? A : Bb;
    TVRow t0, t1;
    bool ok = make_tvrow(bd, load_vrow(CR, 0), M, t0);
    if (nc > 1) ok = make_tvrow(bd, load_vrow(CR, 1), M, t1) && ok;
    if (!ok) return false;
    V2 vM = bd.v(M);
    float wM = bd.w(M), acc = 0.0f;
    for (int it = 0; it < iterations; ++it) {
        solve_tvrow(t0, vM, wM, acc);
        if (nc > 1) solve_tvrow(t1, vM, wM, acc);
    }
    if (!(acc < 0x1p60f)) return false;
    CR.setf(0, CF_NI0, t0.ni0); CR.setf(0, CF_NI1, t0.ni1); CR.setf(0, CF_TI0, t0.ti0); CR.setf(0, CF_TI1, t0.ti1);
    if (nc > 1) {
        CR.setf(1, CF_NI0, t1.ni0); CR.setf(1, CF_NI1, t1.ni1); CR.setf(1, CF_TI0, t1.ti0); CR.setf(1, CF_TI1, t1.ti1);
    }
    bd.set_v(M, vM, wM);
    return true;
}

// one TOI event (toi.py:604-716) on min_slot at min_alpha, the step's event number `ev`: the event island's contacts
// are marked with a stamp distinct for each event of the step (-2 - ev) in the workspace's cisl array, whose island
// ids Solve no longer needs
GOI_D void toi_event(const DModel& m, const World& W, const Bodies& bd, const Rows& CR, const GoiSettings& s,
                          float dt, int min_slot, float min_alpha, int ev, const GoiDebug& dbg) {
    const int stamp = -2 - ev;
    const int fa = W.fa(min_slot), fb = W.fb(min_slot);
    const int A = W.ba(min_slot), Bb = W.bb(min_slot);
    const SweepBackup bkA = backup(W, A), bkB = backup(W, Bb);
    body_advance(W, A, min_alpha);
    body_advance(W, Bb, min_alpha);
    const OldPoints old0 = old_points(W, min_slot);  // in flight during the narrowphase
    Manifold mf0;
    evaluate(m, fa, fb, W.xf(A), W.xf(Bb), s, mf0, W.grp());
    if (contact_update(W, min_slot, mf0, old0)) { W.wake(A); W.wake(Bb); }
    W.set_tflag(min_slot, 0);
    W.set_tcount(min_slot, W.tcount(min_slot) + 1);
    if (!W.touching(min_slot)) {
        W.set_ten(min_slot, 0);
        restore(W, A, bkA);
        restore(W, Bb, bkB);
        record_toi_event(W, dbg, ev, min_slot, min_alpha, 0, 0, CR);
        return;
    }
    W.set_ten(min_slot, 1);
    W.wake(A);
    W.wake(Bb);
    // the island walk: bodyA's then bodyB's contact lists, newest first, at most 32 contacts / 64 bodies; island
    // bodies (distinct, so at most B) in the workspace's ibuf
    int nb = 0, nc = 0;
    unsigned long long bflag = (1ull << A) | (1ull << Bb);
    W.cisl(min_slot) = stamp;
    W.ibuf(nb++) = A;
    W.ibuf(nb++) = Bb;
    cs_position_row(m, W, CR, nc++, min_slot, mf0);
    const int n = list_order(W);
    for (int pi = 0; pi < 2; ++pi) {
        const int body = pi == 0 ? A : Bb;
        if (!W.is_dynamic(body)) continue;
        const bool bullet = W.bullet(body);
        bool full = false;
        // the contacts of `body` in list order that the walk does not skip, a chunk of the list at a time (found by
        // the lane group together). The skips test flags that the walk does not change, and stamps: a contact in the
        // chunk is stamped only when the walk visits it. A skipped contact does nothing, so leaving it out of the walk
        // changes nothing either, the island-full stop included (it stops at the next contact not skipped instead).
        for (int q0 = 0; q0 < n && !full; q0 += 64) {
            const unsigned long long hits = list_mask(W, q0, n, [&](int c) {
                const int ca = W.ba(c), cb = W.bb(c);
                if (ca != body && cb != body) return false;
                if (W.cisl(c) == stamp) return false;
                const int other = ca == body ? cb : ca;
                if (W.is_dynamic(other) && !bullet && !W.bullet(other)) return false;
                return !s.unity_toi || pair_rule(m, W, s, body, other);
            });
            for (unsigned long long left = hits; left; left &= left - 1) {
                const int c = W.order(q0 + __builtin_ctzll(left));
                const int ca = W.ba(c), cb = W.bb(c);
                if (nb == 2 * kMaxToiContacts || nc == kMaxToiContacts) {
                    full = true;
                    break;
                }
                const int other = ca == body ? cb : ca;
                const SweepBackup bk = backup(W, other);
                if (!((bflag >> other) & 1ull)) body_advance(W, other, min_alpha);
                const OldPoints old = old_points(W, c);  // in flight during the narrowphase
                Manifold mf;
                evaluate(m, W.fa(c), W.fb(c), W.xf(ca), W.xf(cb), s, mf, W.grp());
                if (contact_update(W, c, mf, old)) { W.wake(ca); W.wake(cb); }
                W.set_ten(c, 1);
                if (!W.touching(c)) {
                    restore(W, other, bk);
                    continue;
                }
                W.cisl(c) = stamp;
                cs_position_row(m, W, CR, nc++, c, mf);
                if ((bflag >> other) & 1ull) continue;
                bflag |= 1ull << other;
                if (!W.is_static(other)) W.wake(other);
                W.ibuf(nb++) = other;
            }
            group_sync();
        }
    }
    group_sync();
    record_toi_event(W, dbg, ev, min_slot, min_alpha, nc, nb, CR);
    // b2Island::SolveTOI (toi.py:719-799)
    for (int i = 0; i < nb; ++i) {
        const int b = W.ibuf(i);
        bd.set_c(b, W.v2(GOI_B_C, b), W.f(GOI_B_A, b));
        bd.set_v(b, W.v2(GOI_B_V, b), W.f(GOI_B_W, b));
    }
    const float mA_ = W.f(GOI_B_INV_MASS, A), iA_ = W.f(GOI_B_INV_INERTIA, A);
    const float mB_ = W.f(GOI_B_INV_MASS, Bb), iB_ = W.f(GOI_B_INV_INERTIA, Bb);
    if (!toi_positions_one_body(bd, CR, nc, A, Bb, mA_, iA_, mB_, iB_, s))
        toi_positions(bd, CR, nc, A, Bb, mA_, iA_, mB_, iB_, s);
    // leap of faith: the TOI pair's sweep start is the solved pose
    W.set2(GOI_B_C0, A, bd.c(A)); W.f(GOI_B_A0, A) = bd.a(A);
    W.set2(GOI_B_C0, Bb, bd.c(Bb)); W.f(GOI_B_A0, Bb) = bd.a(Bb);
    for (int i = W.sub; i < nc; i += W.G) {  // independent rows, one per lane of the group
        const int slot = CR.geti(i, CF_SLOT);
        const int ia = CR.geti(i, CF_IA), ib = CR.geti(i, CF_IB);
        cs_prepare(m, W, bd, CR, i, slot, false, 1.0f, rot_of(bd.a(ia)), rot_of(bd.a(ib)), s.velocity_threshold);
    }
    group_sync();
    if (!toi_velocities_one_body(bd, CR, nc, A, Bb, mA_, iA_, mB_, iB_, s.velocity_iterations)) {
        // rows 0 (the TOI contact, which every island has) and 1 stay in registers through the passes; rows past them
        // are read from the row tile in each pass
        VRow r0 = load_vrow(CR, 0);
        VRow r1 = nc > 1 ? load_vrow(CR, 1) : r0;
        for (int it = 0; it < s.velocity_iterations; ++it) {
            solve_vrow(bd, r0);
            if (nc > 1) solve_vrow(bd, r1);
            for (int i = 2; i < nc; ++i) {
                VRow r = load_vrow(CR, i);
                solve_vrow(bd, r);
                store_vimpulses(CR, i, r);
            }
        }
        store_vimpulses(CR, 0, r0);
        if (nc > 1) store_vimpulses(CR, 1, r1);
    }
    const float h = (1.0f - min_alpha) * dt;
    const float max_t = s.clamps_per_second ? s.max_translation * dt : s.max_translation;
    const float max_r = s.clamps_per_second ? s.max_rotation * dt : s.max_rotation;
    for (int i = W.sub; i < nb; i += W.G) {  // the island's bodies are independent here: one per lane of the group
        const int b = W.ibuf(i);
        V2 v = bd.v(b);
        float w = bd.w(b);
        const V2 t = h * v;
        if (dot(t, t) > max_t * max_t) {
            const float ratio = max_t / length(t);
            v = mk(v.x * ratio, v.y * ratio);
        }
        const float rot = h * w;
        if (rot * rot > max_r * max_r) w = w * (max_r / babs(rot));
        W.set2(GOI_B_C, b, bd.c(b) + h * v);
        W.f(GOI_B_A, b) = bd.a(b) + h * w;
        W.set2(GOI_B_V, b, v);
        W.f(GOI_B_W, b) = w;
        sync_transform(W, b);
    }
    group_sync();
    // b2Island::Report, rows split over the lane group
    for (int i = W.sub; i < nc; i += W.G) {
        const int slot = CR.geti(i, CF_SLOT), cnt = CR.geti(i, CF_COUNT);
        W.f(GOI_T_NORMAL_IMPULSE, 2 * slot) = cnt > 0 ? CR.getf(i, CF_NI0) : 0.0f;
        W.f(GOI_T_NORMAL_IMPULSE, 2 * slot + 1) = cnt > 1 ? CR.getf(i, CF_NI1) : 0.0f;
        W.f(GOI_T_TANGENT_IMPULSE, 2 * slot) = cnt > 0 ? CR.getf(i, CF_TI0) : 0.0f;
        W.f(GOI_T_TANGENT_IMPULSE, 2 * slot + 1) = cnt > 1 ? CR.getf(i, CF_TI1) : 0.0f;
        W.u8(GOI_T_SOLVED, slot) = 1;
    }
    group_sync();
    // fixture sync of the island's dynamic bodies and TOI invalidation of their contacts
    unsigned long long moved = 0ull, refat = 0ull;
    for (int i = W.sub; i < nb; i += W.G) {  // the island's dynamic bodies, combined over the group
        const int b = W.ibuf(i);
        if (W.is_dynamic(b)) moved |= 1ull << b;
    }
    moved = group_or(W.grp(), moved);
    for (int r = W.sub; r < m.R; r += W.G) {  // their rows, one per lane of the group
        const MRow row = m.row[r];
        const int b = row.body;
        if (((moved >> b) & 1ull) && sync_row(m, W, r, row.fixture, sweep_start_xf(W, b), W.xf(b))) refat |= 1ull << r;
    }
    refat = group_or(W.grp(), refat);
    // the slot loops below split over the lane group (slots are independent)
    // FindNewContacts; a slot that received a new contact starts with fresh TOI state. Before it, the workspace's
    // corder array (Solve's island order is no longer needed) takes each live slot's key, and for a free slot a mark
    // no new contact's key can equal: the search gives keys next_key, next_key + 1, ... (fewer than C of them), so
    // next_key - 1 (unsigned wrap) differs from each; a live slot that keeps its contact keeps its key.
    const int mark = (int)((unsigned)W.i32(GOI_S_NEXT_KEY, 0) - 1u);
    for (int c = W.sub; c < W.C; c += W.G) {
        if (W.pair(c) >= 0) {
            const int ca = W.ba(c), cb = W.bb(c);
            if (((moved >> ca) & 1ull) || ((moved >> cb) & 1ull)) W.set_tflag(c, 0);
        }
        W.corder(c) = W.pair(c) >= 0 ? W.key(c) : mark;
    }
    group_sync();
    find_new_contacts(m, W, W.i32(GOI_S_OVERFLOW, 0) == 0 ? refat : ~0ull);
    for (int c = W.sub; c < W.C; c += W.G) {
        if (W.pair(c) >= 0 && W.corder(c) != W.key(c)) {
            W.set_tcount(c, 0);
            W.set_tflag(c, 0);
            W.set_ten(c, 1);
        }
    }
    group_sync();
}

// b2World::SolveTOI (toi.py:827-865). Called by every lane of the block (the reset, the TOI searches and the final
// copy are cooperative); `valid` marks the lanes that run a world. fresh() returns the lane's views set up afresh
// (W, the cooperative view co, the block copy bc, the lane map lm with the group's leader) for every cooperative
// phase: each search, which follows events that the lanes of other worlds and lanes without a world skipped, and the
// stores after the event loop.
// kOpaqueViews: each iteration of the event loop re-derives the world's views through an offset the compiler cannot
// see through, so that no per-lane address is held (spilled) from one iteration to the next. The island instance's
// spilled registers go (816 to 16 B of scratch per lane, 3.5% faster), and most of the generic kernel's (960 to 160 B,
// 8% faster on the rig at 4 worlds per wave); the rig instance, with few spills, measured slower with it.
// Returns true when the world stopped at max_events with another event pending.
template <bool kOpaqueViews = false, class Fresh>
GOI_D bool solve_toi_world(const DModel& m, const World& W, const Bodies& bd, const Rows& CR, const GoiSettings& s,
                           float dt, bool valid, const Fresh& fresh, const GoiDebug& dbg) {
    if (W.C == 0 || m.P == 0) return false;
    if (s.unity_toi && !m.any_toi_body) return false;
    reset_toi_block(fresh().bc);
    int events = 0;
    bool capped = false;
    if (dt > 0.0f) {
        const int max_events = s.max_events >= 0 ? s.max_events : W.C * (kMaxSubSteps + 1) + 8;
        int slot = -1;
        float alpha = 1.0f;
        const auto search = [&](int nt) {
            const auto v = fresh();
            coop_run(v.co, v.lm.leader ? nt : 0, [&](int o, int i) { toi_task(m, v.co, o, i, s.linear_slop); });
        };
        search(valid ? toi_search_prepare(m, W, CR, s) : 0);
        bool found = valid && toi_search_pick(W, s, slot, alpha);
        // the block iterates while any world has an event to process; the others take part in the searches only
        while (__any(found && events < max_events)) {
            const bool act = found && events < max_events;
            if constexpr (kOpaqueViews) {
                const int z = opaque(0);
                World Wi = W;
                Wi.w = W.w + z;
                Wi.ws = W.ws + z;
                Bodies bdi = bd;
                bdi.s = bd.s + z;
                Rows CRi = CR;
                CRi.base = CR.base + z;
                if (act) {
                    toi_event(m, Wi, bdi, CRi, s, dt, slot, alpha, events, dbg);
                    ++events;
                }
                search(act ? toi_search_prepare(m, Wi, CRi, s) : 0);
                found = act && toi_search_pick(Wi, s, slot, alpha);
            } else {
                if (act) {
                    toi_event(m, W, bd, CR, s, dt, slot, alpha, events, dbg);
                    ++events;
                }
                search(act ? toi_search_prepare(m, W, CR, s) : 0);
                found = act && toi_search_pick(W, s, slot, alpha);
            }
        }
        capped = found && events >= max_events;
    }
    const auto v = fresh();
    if (v.lm.valid) v.W.i32(GOI_T_EVENTS, 0) = events;
    store_toi_block(v.bc);
    return capped;
}

// GoiDebug::status of a world after its step: overflow0 is State.overflow before the step, capped what
// solve_toi_world returned.
GOI_D int step_status(const World& W, int overflow0, bool capped, float dt, const GoiSettings& s) {
    int st = W.i32(GOI_S_OVERFLOW, 0) != overflow0 ? GOI_STATUS_OVERFLOW : 0;
    bool finite = true;
    for (int b = 0; b < W.B; ++b) {
        const V2 c = W.v2(GOI_B_C, b), v = W.v2(GOI_B_V, b);
        const float a = W.f(GOI_B_A, b), w = W.f(GOI_B_W, b);
        finite = finite && isfinite(c.x) && isfinite(c.y) && isfinite(a) && isfinite(v.x) && isfinite(v.y) &&
                 isfinite(w);
    }
    if (!finite) st |= GOI_STATUS_NONFINITE;
    if (capped) st |= GOI_STATUS_TOI_CAPPED;
    if (s.continuous_physics && !(dt > 0.0f)) st |= GOI_STATUS_TOI_SKIPPED;
    return st;
}

}  // namespace goi
