"""The pins have teeth: each case plants one plausible slip in a copy of the CPU restatement (oracle/b2_oracle.c,
rebuilt into a temporary directory), loads it in place of the real oracle and shows that the named pin of
test_oracle_pins now fails. CPU only; the real oracle is untouched.
"""
import subprocess
from pathlib import Path

import pytest

import test_edges as E
import test_oracle_pins as P
from oracle import oracle as O

SRC = Path(O.__file__).resolve().parent / "b2_oracle.c"
INC = SRC.parent.parent / "include"

# (name, text in b2_oracle.c, replacement, the pin that must fail)
MUTANTS = [
    ("damping_as_1_minus_hc", "float ld = 1.0f / (1.0f + h * w->b_ld[b]);", "float ld = 1.0f - h * w->b_ld[b];",
     lambda o: P.test_free_fall_is_semi_implicit_euler_bit_exact(o, 0.2)),
    ("friction_mix_max", "sqrtf(friction_of(x, w, a) * friction_of(x, w, b))",
     "fmaxf(friction_of(x, w, a), friction_of(x, w, b))",
     lambda o: P.test_contact_impulses_carry_the_weight(o)),
    ("restitution_mix_min", "w->c_restitution[k] = ra > rb ? ra : rb;", "w->c_restitution[k] = ra < rb ? ra : rb;",
     lambda o: P.test_restitution_mix_is_max(o)),
    ("toi_target_one_slop", "float target = bmax(linear_slop, total_radius - 3.0f * linear_slop);",
     "float target = bmax(linear_slop, total_radius - 1.0f * linear_slop);",
     lambda o: P.test_time_of_impact_contract(o)),
    ("contact_list_oldest_first", "while (j > 0 && w->c_key[order[j - 1]] < w->c_key[k])",
     "while (j > 0 && w->c_key[order[j - 1]] > w->c_key[k])",
     lambda o: P.test_islands_vs_sequential_dfs(o, "pile")),
    ("toi_tie_rules_swapped", "toi_tie_oldest ? alpha <= best_alpha : alpha < best_alpha",
     "toi_tie_oldest ? alpha < best_alpha : alpha <= best_alpha", lambda o: P.test_toi_tie_rule(o)),
    ("toi_search_slot_order", "int c = k->order[i];\n        if (!w->t_enabled[c]",
     "int c = i;\n        if (!w->t_enabled[c]", lambda o: P.test_toi_tie_rule(o)),
    ("toi_walk_takes_dynamic_neighbours",
     "if (w->b_type[other] == GOI_DYNAMIC && !w->b_bullet[body] && !w->b_bullet[other]) continue;",
     "if (0) continue;", lambda o: P.test_toi_island_membership(o)),
    ("toi_walk_bullet_of_walked_body_only",
     "if (w->b_type[other] == GOI_DYNAMIC && !w->b_bullet[body] && !w->b_bullet[other]) continue;",
     "if (w->b_type[other] == GOI_DYNAMIC && !w->b_bullet[body]) continue;",
     lambda o: P.test_toi_island_membership(o)),
    ("toi_walk_body_a_only", "for (int pi = 0; pi < 2; ++pi) {\n        int body = pair[pi];",
     "for (int pi = 0; pi < 1; ++pi) {\n        int body = pair[pi];", lambda o: P.test_toi_island_membership(o)),
    ("block_solver_diagonal_inverse",
     "c->NM[0] = det * k22; c->NM[1] = -det * k12; c->NM[2] = -det * k12; c->NM[3] = det * k11;",
     "c->NM[0] = 1.0f / k11; c->NM[1] = 0.0f; c->NM[2] = 0.0f; c->NM[3] = 1.0f / k22;",
     lambda o: P.test_block_solver_solves_the_two_point_lcp(o, 8)),
    ("block_solver_warm_sign", "bx = bx - (c->K[0] * ax + c->K[2] * ay);", "bx = bx + (c->K[0] * ax + c->K[2] * ay);",
     lambda o: P.test_block_solver_solves_the_two_point_lcp(o, 8)),
    ("collide_touch_flip_wakes_nobody", "if (contact_update(w, k, &mf)) { wake(w, ba); wake(w, bb); }",
     "contact_update(w, k, &mf);", lambda o: P.test_collide_wake_cascade_in_list_order(o, True)),
    ("collide_walk_to_fixed_point",
     "    for (int i = 0; i < n; ++i) {\n        int k = order[i];\n        int fa = w->c_fa[k], fb = w->c_fb[k];\n"
     "        int ba = m->fixture_body[fa], bb = m->fixture_body[fb];\n        int act_a",
     "    for (int i = 0; i < 2 * n; ++i) {\n        int k = order[i % n];\n        int fa = w->c_fa[k], fb = w->c_fb[k];\n"
     "        int ba = m->fixture_body[fa], bb = m->fixture_body[fb];\n        int act_a",
     lambda o: P.test_collide_wake_cascade_in_list_order(o, False)),
    ("joint_point_mass_uncoupled",
     "(joints.py:39-47) */\n        float exx = ((mA + mB) + rA.y * rA.y * iA) + rB.y * rB.y * iB;\n"
     "        float eyx = -rA.y * rA.x * iA - rB.y * rB.x * iB;",
     "(joints.py:39-47) */\n        float exx = ((mA + mB) + rA.y * rA.y * iA) + rB.y * rB.y * iB;\n"
     "        float eyx = 0.0f;",
     lambda o: P.test_joint_velocity_rows_solve_the_constraint(o, "revolute", True)),
    ("prismatic_mass_uncoupled", "float k12 = iA * s1 + iB * s2;\n        float k13",
     "float k12 = 0.0f;\n        float k13",
     lambda o: P.test_joint_velocity_rows_solve_the_constraint(o, "prismatic", True)),
    ("toi_root_secant_first", "if (rc & 1) t = a1 + (target - s1) * (a2 - a1) / (s2 - s1);",
     "if (!(rc & 1)) t = a1 + (target - s1) * (a2 - a1) / (s2 - s1);",
     lambda o: P.test_time_of_impact_head_on_circles_root_steps(o)),
    ("toi_root_bisection_only", "if (rc & 1) t = a1 + (target - s1) * (a2 - a1) / (s2 - s1);",
     "if (0) t = a1 + (target - s1) * (a2 - a1) / (s2 - s1);",
     lambda o: P.test_time_of_impact_head_on_circles_root_steps(o)),
    ("feature_key_types_swapped", "return ia | (ib << 8) | (ta << 16) | (tb << 24);",
     "return ia | (ib << 8) | (tb << 16) | (ta << 24);", lambda o: P.test_polygon_manifold_known_answers(o)),
    ("flip_keeps_feature_halves", "ids[i] = flip ? feature_key(cp2[i].ib, cp2[i].ia, cp2[i].tb, cp2[i].ta)",
     "ids[i] = flip ? feature_key(cp2[i].ia, cp2[i].ib, cp2[i].ta, cp2[i].tb)",
     lambda o: P.test_polygon_manifold_known_answers(o)),
    ("clip_second_side_keyed_iv1", "np = clip_segment(cp2, cp1, tangent, side2, iv2);",
     "np = clip_segment(cp2, cp1, tangent, side2, iv1);", lambda o: P.test_polygon_manifold_known_answers(o)),
    ("no_reference_face_hysteresis", "int flip = sep_b > sep_a + k_tol;", "int flip = sep_b > sep_a;",
     lambda o: P.test_polygon_manifold_known_answers(o)),
    ("circle_radius_dropped", "float r = m->radius[fa] + m->radius[fb];", "float r = m->radius[fa];",
     lambda o: P.test_narrowphase_vs_brute_force(o, P.shape_model.__wrapped__())),
    ("edge_circle_ghost_sign", "if (dot(e1, sub(a, q)) > 0.0f) return;", "if (dot(e1, sub(a, q)) < 0.0f) return;",
     lambda o: E.test_edge_circle_regions(o, E.edge_world.__wrapped__())),
    ("edge_polygon_limits_swapped", "if (dot(n, perp) >= 0.0f) {", "if (dot(n, perp) < 0.0f) {",
     lambda o: E.test_edge_polygon_closed_forms(o, E.edge_world.__wrapped__())),
    ("edge_polygon_one_skin", "float radius = 2.0f * st->polygon_radius;", "float radius = st->polygon_radius;",
     lambda o: E.test_edge_polygon_closed_forms(o, E.edge_world.__wrapped__())),
    ("edge_polygon_no_hysteresis", "!(poly_sep > 0.98f * edge_sep + 0.001f)", "!(poly_sep > edge_sep)",
     lambda o: E.test_edge_polygon_closed_forms(o, E.edge_world.__wrapped__())),
    # position rows (one pass of non-linear Gauss-Seidel)
    ("revolute_point_mass_uncoupled", "float kxy = -iA * rA.x * rA.y - iB * rB.x * rB.y;", "float kxy = 0.0f;",
     lambda o: P.test_revolute_point_row_is_one_newton_step(o, True)),
    ("revolute_point_sign", "    j = neg(j);\n", "    (void)0;\n",
     lambda o: P.test_revolute_point_row_is_one_newton_step(o, False)),
    ("revolute_point_angular_operands", "*aB = *aB + iB * crs(rB, j);", "*aB = *aB + iB * crs(j, rB);",
     lambda o: P.test_revolute_point_row_is_one_newton_step(o, True)),
    ("revolute_limit_slop_omitted", "C = bclamp((angle - r->lower) + s->angular_slop, -mac, 0.0f);",
     "C = bclamp(angle - r->lower, -mac, 0.0f);",
     lambda o: P.test_revolute_limit_row(o, True, "below", -0.08, (-0.5, 0.4))),
    ("revolute_limit_unclamped", "C = bclamp((angle - r->upper) - s->angular_slop, 0.0f, mac);",
     "C = (angle - r->upper) - s->angular_slop;",
     lambda o: P.test_revolute_limit_row(o, True, "above_far", 0.5, (-0.5, 0.4))),
    ("revolute_limit_sign", "float li = -r->motor_mass * C;", "float li = r->motor_mass * C;",
     lambda o: P.test_revolute_limit_row(o, True, "below", -0.08, (-0.5, 0.4))),
    ("prismatic_position_unclamped", "C2 = bclamp((t - r->lower) + s->linear_slop, -mlc, 0.0f);",
     "C2 = (t - r->lower) + s->linear_slop;", lambda o: P.test_prismatic_position_row(o, "lower_far")),
    ("prismatic_position_uncoupled", "float k12 = iA * s1 + iB * s2;\n        float k22 = iA + iB;",
     "float k12 = 0.0f;\n        float k22 = iA + iB;", lambda o: P.test_prismatic_position_row(o, "free")),
    ("weld_position_diagonal_mass",
     "V3 ex = v3(exx, eyx, ezx), ey = v3(eyx, eyy, ezy), ez = v3(ezx, ezy, ezz);\n        V2 C1",
     "V3 ex = v3(exx, 0.0f, 0.0f), ey = v3(0.0f, eyy, 0.0f), ez = v3(0.0f, 0.0f, ezz);\n        V2 C1",
     lambda o: P.test_weld_position_row(o, False)),
    ("position_uses_toi_baumgarte",
     "float ms = cs_solve_position(x, c, k, s->baumgarte, c->mA, c->mB, c->iA, c->iB);",
     "float ms = cs_solve_position(x, c, k, s->toi_baumgarte, c->mA, c->mB, c->iA, c->iB);",
     lambda o: P.test_contact_position_row_circle(o, 0.03, False)),
    ("position_slop_omitted",
     "float C = bclamp(baumgarte * (sep + s->linear_slop), -s->max_linear_correction, 0.0f);",
     "float C = bclamp(baumgarte * sep, -s->max_linear_correction, 0.0f);",
     lambda o: P.test_contact_position_row_circle(o, 0.03, False)),
    ("position_unclamped",
     "float C = bclamp(baumgarte * (sep + s->linear_slop), -s->max_linear_correction, 0.0f);",
     "float C = bmin(baumgarte * (sep + s->linear_slop), 0.0f);",
     lambda o: P.test_contact_position_row_circle(o, 1.3, True)),
    ("position_mass_without_rotation", "float K = ((mA + mB) + iA * rnA * rnA) + iB * rnB * rnB;",
     "float K = mA + mB;", lambda o: P.test_contact_position_row_tilted_box(o)),
    # the block solver's condition test, exact ties, the TOI island walk
    ("block_solver_condition_inverted", "k11 * k11 < 1000.0f * (k11 * k22 - k12 * k12)",
     "k11 * k11 >= 1000.0f * (k11 * k22 - k12 * k12)", lambda o: P.test_block_solver_condition_fallback(o)),
    ("max_separation_last_index_wins", "if (si > maxsep) { maxsep = si; best = i; }",
     "if (si >= maxsep) { maxsep = si; best = i; }", lambda o: P.test_polygon_manifold_exact_ties(o)),
    ("incident_edge_last_index_wins", "if (d < mind) { mind = d; index = i; }",
     "if (d <= mind) { mind = d; index = i; }", lambda o: P.test_polygon_manifold_exact_ties(o)),
    ("toi_walk_oldest_first",
     "for (int i = 0; i < n; ++i) {\n            int c = k->order[i];\n            int ca = m->fixture_body",
     "for (int i = n - 1; i >= 0; --i) {\n            int c = k->order[i];\n            int ca = m->fixture_body",
     lambda o: P.test_toi_island_walk_order_and_cap(o)),
    ("toi_walk_cap_31", "nc == MAX_TOI_CONTACTS", "nc == MAX_TOI_CONTACTS - 1",
     lambda o: P.test_toi_island_walk_order_and_cap(o)),
    ("toi_walk_cap_33", "nc == MAX_TOI_CONTACTS", "nc == MAX_TOI_CONTACTS + 1",
     lambda o: P.test_toi_island_walk_order_and_cap(o)),
    # revolute velocity rows
    ("revolute_limit_not_speculative", "float impulse = -am * ((wB - wA) + bmax(C, 0.0f) * r->inv_dt);",
     "float impulse = -am * (wB - wA);", lambda o: P.test_revolute_velocity_rows(o, *_vel("lower_closing"))),
    ("revolute_lower_impulse_may_pull", "imp[3] = bmax(imp[3] + impulse, 0.0f);", "imp[3] = imp[3] + impulse;",
     lambda o: P.test_revolute_velocity_rows(o, *_vel("lower_opening"))),
    ("revolute_motor_unclamped",
     "float impulse = -am * cdot;\n            float old = r->mimp;\n"
     "            r->mimp = bclamp(r->mimp + impulse, -r->max_impulse, r->max_impulse);",
     "float impulse = -am * cdot;\n            float old = r->mimp;\n            r->mimp = r->mimp + impulse;",
     lambda o: P.test_revolute_velocity_rows(o, *_vel("motor_saturated"))),
    ("revolute_v23_limit_never_releases",
     "int redo = (st == AT_LOWER && new_z < 0.0f) || (st == AT_UPPER && new_z > 0.0f);", "int redo = 0;",
     lambda o: P.test_revolute_velocity_rows(o, *_vel("leaving_lower_v23"))),
    # SynchronizeFixtures, the TOI position passes, warm start, the rotation clamp, the per-island exit
    ("sync_multiplier_one", "float ddx = 2.0f * d.x, ddy = 2.0f * d.y;", "float ddx = 1.0f * d.x, ddy = 1.0f * d.y;",
     lambda o: P.test_synchronize_fixtures_refattens_a_moved_box(o, *P._SYNC_MOVES[0])),
    ("sync_always_refattens", "if (fat[0] <= lx && fat[1] <= ly && ux <= fat[2] && uy <= fat[3]) continue;",
     "if (0) continue;", lambda o: P.test_synchronize_fixtures_keeps_a_fat_box_that_still_holds(o, (3.0, 1.0))),
    ("sync_extension_0_2", "float e = 0.1f; /* b2_aabbExtension */", "float e = 0.2f;",
     lambda o: P.test_synchronize_fixtures_refattens_a_moved_box(o, *P._SYNC_MOVES[0])),
    ("toi_position_stops_at_3_slop", "if (min_sep >= -1.5f * s->linear_slop) break;",
     "if (min_sep >= -3.0f * s->linear_slop) break;", lambda o: P.test_toi_position_passes_closed_form(o)),
    ("toi_position_uses_baumgarte", "float ms = cs_solve_position(x, c, k, s->toi_baumgarte, mA, mB, iA, iB);",
     "float ms = cs_solve_position(x, c, k, s->baumgarte, mA, mB, iA, iB);",
     lambda o: P.test_toi_position_passes_closed_form(o)),
    ("warm_start_without_dt_ratio", "c->ni[j] = warm ? dt_ratio * w->c_ni[2 * slot + j] : 0.0f;",
     "c->ni[j] = warm ? w->c_ni[2 * slot + j] : 0.0f;", lambda o: P.test_warm_start_scales_impulses_by_dt_ratio(o)),
    ("rotation_clamp_removed",
     "if (rot * rot > max_r * max_r) {\n            float ratio = max_r / babs(rot);\n            ww = ww * ratio;\n"
     "        }\n        k->cx[b]",
     "if (0) {\n            float ratio = max_r / babs(rot);\n            ww = ww * ratio;\n        }\n        k->cx[b]",
     lambda o: P.test_rotation_clamp(o, 200.0)),
    ("position_exit_at_1_5_slop", "k->min_sep[i] >= -3.0f * s->linear_slop && k->jok[i]",
     "k->min_sep[i] >= -1.5f * s->linear_slop && k->jok[i]", lambda o: P.test_position_iterations_exit_per_island(o)),
    ("position_exit_all_islands_together", "if (k->done[isl]) continue;\n            float ms",
     "if (!more) continue;\n            float ms", lambda o: P.test_position_iterations_exit_per_island(o)),
    # settings paths and per-step bookkeeping
    ("sleep_without_position_solve", "k->isl_sleep[i] = k->min_st[i] >= s->time_to_sleep && k->done[i];",
     "k->isl_sleep[i] = k->min_st[i] >= s->time_to_sleep;", lambda o: P.test_sleep_needs_the_position_solve(o)),
    ("restitution_without_threshold", "c->bias[j] = vrel < -x->s->velocity_threshold ? -restitution * vrel : 0.0f;",
     "c->bias[j] = vrel < 0.0f ? -restitution * vrel : 0.0f;", lambda o: P.test_restitution_velocity_threshold(o)),
    ("angular_damping_uses_linear", "float ad = 1.0f / (1.0f + h * w->b_ad[b]);",
     "float ad = 1.0f / (1.0f + h * w->b_ld[b]);", lambda o: P.test_angular_damping_closed_form(o)),
    ("tangent_speed_sign", "float vt = dot(dv, t) - c->tangent_speed;", "float vt = dot(dv, t) + c->tangent_speed;",
     lambda o: P.test_tangent_speed_drives_the_contact(o)),
    ("inv_dt0_on_any_dt", "if (dt > 0.0f) *w->inv_dt0 = inv_dt;", "*w->inv_dt0 = inv_dt;",
     lambda o: P.test_inv_dt0_kept_for_non_positive_dt(o)),
    ("clamps_per_second_ignored",
     "float max_t = s->clamps_per_second ? s->max_translation * h : s->max_translation;",
     "float max_t = s->max_translation;", lambda o: P.test_clamps_per_second(o)),
    ("sleep_time_kept_when_moving", "if (moving) { w->b_sleep_time[b] = 0.0f; k->min_st[isl] = 0.0f; }",
     "if (moving) { k->min_st[isl] = 0.0f; }", lambda o: P.test_sleep_time_resets_when_moving(o)),
    ("warm_starting_flag_ignored", "c->ni[j] = warm ? dt_ratio * w->c_ni[2 * slot + j] : 0.0f;",
     "c->ni[j] = dt_ratio * w->c_ni[2 * slot + j];", lambda o: P.test_warm_starting_off(o)),
    ("joint_warm_without_dt_ratio", "    r->imp[0] = warm ? ix * dt_ratio : 0.0f;", "    r->imp[0] = warm ? ix : 0.0f;",
     lambda o: P.test_joint_warm_start_scales_by_dt_ratio(o, True)),
    ("motor_warm_without_dt_ratio", "    r->mimp = warm ? mimp * dt_ratio : 0.0f;", "    r->mimp = warm ? mimp : 0.0f;",
     lambda o: P.test_joint_warm_start_scales_by_dt_ratio(o, True)),
    ("limit_warm_without_dt_ratio", "    r->imp[3] = warm ? lo * dt_ratio : 0.0f;", "    r->imp[3] = warm ? lo : 0.0f;",
     lambda o: P.test_joint_warm_start_scales_by_dt_ratio(o, True)),
    ("static_awake_from_first_island", "        if (isl > k->last[ba]) k->last[ba] = isl;",
     "        if (k->last[ba] < 0) k->last[ba] = isl;", lambda o: P.test_static_body_takes_the_last_islands_awake_flag(o)),
    ("revolute_exit_ignores_limit_error", "    return pos_err <= s->linear_slop && ang_err <= s->angular_slop;",
     "    return pos_err <= s->linear_slop;", lambda o: P.test_joint_error_keeps_position_iterations_going(o, "revolute_v24")),
    ("prismatic_exit_ignores_angle", "        ok = lin_err <= s->linear_slop && ang_err <= s->angular_slop;",
     "        ok = lin_err <= s->linear_slop;", lambda o: P.test_joint_error_keeps_position_iterations_going(o, "prismatic")),
    ("weld_exit_ignores_angle", "        ok = pos_err <= s->linear_slop && ang_err <= s->angular_slop;",
     "        ok = pos_err <= s->linear_slop;", lambda o: P.test_joint_error_keeps_position_iterations_going(o, "weld")),
    # SolveTOI's bookkeeping
    ("toi_sub_step_cap_at_8", "w->t_count[c] > MAX_SUB_STEPS", "w->t_count[c] >= MAX_SUB_STEPS",
     lambda o: P.test_toi_sub_step_cap_and_re_search(o)),
    ("toi_re_search_body_a_only", "if (k->moved[ca] || k->moved[cb]) w->t_flag[c] = 0;",
     "if (k->moved[ca]) w->t_flag[c] = 0;", lambda o: P.test_toi_sub_step_cap_and_re_search(o)),
    ("toi_walk_keeps_advanced_neighbour", "if (!w->c_touching[c]) { restore_sweep(w, k, other); continue; }",
     "if (!w->c_touching[c]) { continue; }", lambda o: P.test_toi_walk_restores_a_body_it_does_not_keep(o)),
    ("angular_sleep_tolerance_not_squared",
     "float ang_tol = s->angular_sleep_tolerance * s->angular_sleep_tolerance;",
     "float ang_tol = s->angular_sleep_tolerance;", lambda o: P.test_angular_sleep_tolerance_is_squared(o)),
    ("gravity_scale_ignored_x", "w->b_gs[b] * w->gravity[0]", "w->gravity[0]",
     lambda o: P.test_gravity_scale_and_lateral_gravity(o)),
    ("soft_weld_gamma_without_h", "        float gamma = h * (dd + h * kk);", "        float gamma = dd + h * kk;",
     lambda o: P.test_soft_weld_velocity_row(o, 0.5)),
    ("soft_weld_bias_sign", "        float bias = C * h * kk * gamma;", "        float bias = -C * h * kk * gamma;",
     lambda o: P.test_soft_weld_velocity_row(o, 0.0)),
    ("toi_integration_clamp_over_h",
     "    float max_t = s->clamps_per_second ? s->max_translation * x->dt : s->max_translation;",
     "    float max_t = s->clamps_per_second ? s->max_translation * h : s->max_translation;",
     lambda o: P.test_toi_integration_clamp_is_per_step(o)),
]


def _vel(name):
    return next(c for c in P._VEL_CASES if c[0] == name)


def _build(tmp, name, old, new):
    text = SRC.read_text()
    assert text.count(old) == 1, f"{name}: the planted text must occur exactly once"
    src = tmp / f"{name}.c"
    src.write_text(text.replace(old, new))
    lib = tmp / f"lib{name}.so"
    subprocess.run(["gcc", "-O1", "-std=c11", "-ffp-contract=off", "-fno-fast-math", "-fopenmp", "-fPIC",
                    "-shared", f"-I{INC}", f"-I{SRC.parent}", str(src), "-o", str(lib), "-lm"], check=True)
    return lib


@pytest.mark.parametrize("name,old,new,pin", MUTANTS, ids=[m[0] for m in MUTANTS])
def test_pin_catches_planted_mistake(tmp_path, monkeypatch, oracle, name, old, new, pin):
    pin(oracle)  # passes on the real restatement
    monkeypatch.setattr(O, "_L", O.load(_build(tmp_path, name, old, new)))
    with pytest.raises(AssertionError):
        pin(O)
