// b2_view.hpp - device-side views of the shared Model and of one world's State in the worlds-minor SoA layout.
//
// State leaf `L` of per-world inner shape S is a device array; element (i, w) is at L[i * pitch + w] (include/goi_b2.h).
// Lane w of a launch owns world w, so every per-world access of a wavefront touches 64 consecutive words of one leaf
// row: fully coalesced 256-byte segments.
#pragma once

#include "../../include/goi_b2.h"
#include "b2_math.hpp"

namespace goi {

// Device copy of the Model plus the static-terrain acceleration structures built by goi_model_create.
struct DModel {
    int F, J, P, B, R;  // R = non-static fixture rows (compact layout)
    const int* fixture_body;
    const int* shape_type;
    const float* radius;
    const int* count;
    const V2* verts;    // [F * 8]
    const V2* normals;  // [F * 8]
    const int* joint_type;
    const int* joint_a;
    const int* joint_b;
    const V2* local_anchor_a;
    const V2* local_anchor_b;
    const V2* local_axis_a;
    const V2* local_yaxis_a;
    const float* reference_angle;
    const int* pair_a;
    const int* pair_b;
    const int* fixture_slot;    // [F] State row or -1 (static)
    const int* slot_fixture;    // [R]
    const float4* static_fat;   // [F] (rows of static fixtures)
    const float* static_friction;
    const float* static_restitution;
    const int* body_type;       // [B]
    int any_toi_body;           // Model.toi_bodies has a set entry (or is absent)
    // Static BVH over the static fixtures' fat AABBs (node 0 = root). Internal node: child[0], child[1] >= 0.
    // Leaf: child[0] = ~first (index into leaf_fixture), child[1] = count.
    int n_nodes;
    const float4* node_box;     // [n_nodes] lx ly ux uy
    const int2* node_child;     // [n_nodes]
    const int* leaf_fixture;    // static fixture ids in leaf order
    const int* cand_static;     // [F * R]: candidate index of (static fixture f, row r), -1 if none
    int n_dd;                   // candidates whose fixtures are both non-static
    const int* dd_cand;         // [n_dd] candidate indices (ascending)
};

// One world's State: leaf pointers already offset by the lane's world index.
struct World {
    int pitch;
    int B, C, R, J;
    void* const* lv;  // leaf base pointers (kernel argument block)
    int w;

    template <typename T>
    GOI_D T& at(int leaf, int i) const {
        return reinterpret_cast<T*>(lv[leaf])[(size_t)i * pitch + w];
    }
    GOI_D float& f(int leaf, int i) const { return at<float>(leaf, i); }
    GOI_D int& i32(int leaf, int i) const { return at<int>(leaf, i); }
    GOI_D uint8_t& u8(int leaf, int i) const { return at<uint8_t>(leaf, i); }
    GOI_D V2 v2(int leaf, int i) const { return mk(f(leaf, 2 * i), f(leaf, 2 * i + 1)); }
    GOI_D void set2(int leaf, int i, V2 v) const {
        f(leaf, 2 * i) = v.x;
        f(leaf, 2 * i + 1) = v.y;
    }
    GOI_D Xf xf(int b) const {
        Xf t;
        t.p = v2(GOI_B_XF_P, b);
        t.q.c = f(GOI_B_XF_Q, 2 * b);
        t.q.s = f(GOI_B_XF_Q, 2 * b + 1);
        return t;
    }
    // b2Body::SetAwake(true): the sleep timer restarts only if the body was asleep
    GOI_D void wake(int b) const {
        if (!u8(GOI_B_AWAKE, b)) {
            u8(GOI_B_AWAKE, b) = 1;
            f(GOI_B_SLEEP_TIME, b) = 0.0f;
        }
    }
    GOI_D int body_of(const DModel& m, int fixture) const { return m.fixture_body[fixture]; }
};

// Fat AABB of a fixture in the compact layout: the world's own row, or the Model's shared static box.
GOI_D float4 fat_of(const DModel& m, const World& W, int fixture) {
    int r = m.fixture_slot[fixture];
    if (r < 0) return m.static_fat[fixture];
    return make_float4(W.f(GOI_F_FAT, 4 * r), W.f(GOI_F_FAT, 4 * r + 1), W.f(GOI_F_FAT, 4 * r + 2),
                       W.f(GOI_F_FAT, 4 * r + 3));
}
GOI_D float friction_of(const DModel& m, const World& W, int fixture) {
    int r = m.fixture_slot[fixture];
    return r < 0 ? m.static_friction[fixture] : W.f(GOI_F_FRICTION, r);
}
GOI_D float restitution_of(const DModel& m, const World& W, int fixture) {
    int r = m.fixture_slot[fixture];
    return r < 0 ? m.static_restitution[fixture] : W.f(GOI_F_RESTITUTION, r);
}

// b2TestOverlap
GOI_D bool overlap(float4 a, float4 b) {
    float d1x = b.x - a.z, d1y = b.y - a.w;
    float d2x = a.x - b.z, d2y = a.y - b.w;
    return !(d1x > 0.0f || d1y > 0.0f || d2x > 0.0f || d2y > 0.0f);
}

}  // namespace goi
