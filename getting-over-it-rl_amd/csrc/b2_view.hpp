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
constexpr int kWideDepth = 8;  // levels of the static tree below its root, at most

// The Model's per-fixture, per-joint and per-row data are records, so that the kernel keeps a few base pointers in
// scalar registers (one per record table) rather than one per field.
struct MFixture {       // 64 bytes
    int body, type;
    float radius;
    int count;
    int slot;           // the fixture's State row, -1 for a static fixture
    float friction, restitution;  // a static fixture's (a row's live in the State)
    int edge_flags;     // edge ghost flags; 0 when absent
    float4 fat;         // a static fixture's fat AABB
    V2 centroid;        // polygon centroid (edge-polygon contacts); zeros when the Model has no edges
    int pad_[2];
};
struct MJoint {         // 48 bytes
    int type, a, b;
    float reference_angle;
    V2 anchor_a, anchor_b, axis_a, yaxis_a;
};
struct MRow {           // a non-static fixture row
    int fixture, body, dynamic, pad_;
};
// Static 8-wide tree node: child j has the box box[j] and the reference ref[j], either a child node (>= 0) or a leaf,
// ~(first << 4 | count), of count (1..8) consecutive entries of DModel::leaf from first; an unused child slot holds an
// empty box (lx > ux), which overlaps nothing.
struct MNode {          // 160 bytes
    float4 box[8];
    int ref[8];
};
struct MLeaf {          // a static fixture in the tree: its fat AABB and its body | (body is dynamic) << 16
    float4 fat;
    int info, pad_[3];
};

static_assert(sizeof(MFixture) == 64 && sizeof(MJoint) == 48 && sizeof(MNode) == 160 && sizeof(MLeaf) == 32,
              "the Model's records are packed without holes");

struct DModel {
    int F, J, P, B, R;  // R = non-static fixture rows (compact layout)
    const MFixture* fix;  // [F]
    const V2* poly;       // [F * 16]: fixture f's vertices at 16 f + i, its edge normals at 16 f + 8 + i
    const MJoint* joint;  // [J]
    const int2* pair;     // [P] the candidate pairs' fixtures
    const MRow* row;      // [R]
    const int* body_type; // [B]
    int any_toi_body;     // Model.toi_bodies has a set entry (or is absent)
    int rev_only;         // every joint is revolute
    int no_edges;         // no edge fixture
    int island_lanes;     // the non-static bodies are not all joined by joints: a world may hold several islands,
                          // which its lane group then solves side by side
    // the static fixtures' 8-wide tree (node 0 = the root); nodes lie at most kWideDepth levels below the root
    int n_wnodes;         // 0 without static fixtures
    const MNode* wnode;   // [n_wnodes]
    const MLeaf* leaf;    // [n_leaf]
    const int* leaf_cand; // [n_leaf * R]: candidate index of (leaf entry i, row r), -1 if none
    int n_dd;             // candidates whose fixtures are both non-static
    const int4* dd_info;  // [n_dd] ascending: candidate, row_a | row_b << 8, body_a | body_b << 8, 0
};

// Float body leaves mirrored in the workspace for the whole step: the leaf's per-body element count and the
// multiple of B at which its elements start (-1 for leaves that stay in the State only).
GOI_HD constexpr int body_mirror_coef(int leaf) {
    return leaf == GOI_B_C0 ? 0 : leaf == GOI_B_C ? 2 : leaf == GOI_B_A0 ? 4 : leaf == GOI_B_A ? 5 : leaf == GOI_B_V ? 6
         : leaf == GOI_B_W ? 8 : leaf == GOI_B_XF_P ? 9 : leaf == GOI_B_XF_Q ? 11 : leaf == GOI_T_ALPHA0 ? 13
         : leaf == GOI_B_LOCAL_CENTER ? 14 : leaf == GOI_B_INV_MASS ? 16 : leaf == GOI_B_INV_INERTIA ? 17
         : leaf == GOI_B_SLEEP_TIME ? 18 : -1;
}
constexpr int kBodyMirrorWords = 19;  // per body
// the mirrored leaves with their per-body widths; the first `kBodyMirrorMutable` change during a step
constexpr int kBodyMirrorLeaves[13] = {GOI_B_C0, GOI_B_C, GOI_B_A0, GOI_B_A, GOI_B_V, GOI_B_W, GOI_B_XF_P, GOI_B_XF_Q,
                                       GOI_T_ALPHA0, GOI_B_SLEEP_TIME, GOI_B_LOCAL_CENTER, GOI_B_INV_MASS,
                                       GOI_B_INV_INERTIA};
constexpr int kBodyMirrorWidth[13] = {2, 2, 1, 1, 2, 1, 2, 2, 1, 1, 2, 1, 1};
constexpr int kBodyMirrorMutable = 10;

// Per-world workspace in LDS. Every array is [index][world] with the block's world count S as stride: world l's
// element i of an array at offset o sits at base[(o + i) * S + l], so one index across a block is consecutive words.
// It mirrors the per-world contact metadata (pair, key, fixtures), the awake flags and the TOI bookkeeping for the
// whole step (loaded once, written back once) and holds the per-world work arrays (contact list order, island
// lists and stacks, new-pair buffer), which would otherwise live in private scratch memory.
//
// A slot's small fields share one word (o_meta): its bodies (fixture_body of fa and fb), contacts.touching and
// contacts.count, and the TOI flag, enabled flag and count (SolveTOI's reset, world.py:157-161).
constexpr int kMetaBodyA = 0, kMetaBodyB = 6;  // 6 bits each (at most 64 bodies)
constexpr int kMetaTouch = 12;                 // 1 bit
constexpr int kMetaCount = 13;                 // 2 bits (manifold point count, 0..2)
constexpr int kMetaTFlag = 15, kMetaTEn = 16;  // 1 bit each
constexpr int kMetaTCount = 17;                // 4 bits (at most b2_maxSubSteps + 1 = 9)
constexpr int kMetaSlotChanged = 21;           // 1 bit: the slot's contact was created or destroyed since the load
constexpr int kMetaOddLoad = 22;               // 1 bit: the State's touching or count was not 0/1, 0..2 at the load
struct Workspace {
    int o_pair, o_key, o_fa, o_fb, o_meta, o_ttoi, o_order, o_newp, o_corder, o_cisl;  // [C]
    int o_awake, o_active, o_bisl, o_stack, o_fwork, o_ibuf;                            // [B]
    int o_qbox;                                                                         // [4 R]
    int o_nlive;                                                                        // [1]
    int o_jorder, o_jisl;                                                               // [J]
    int o_body;  // 8 solver body fields x B
    int o_bm;    // mirrored body leaves, kBodyMirrorWords x B
    int words;   // per lane
    GOI_HD static Workspace layout(int B, int C, int J, int R) {
        Workspace k;
        int o = 0;
        k.o_body = o; o += 8 * B;
        k.o_bm = o; o += kBodyMirrorWords * B;
        k.o_pair = o; o += C; k.o_key = o; o += C; k.o_fa = o; o += C; k.o_fb = o; o += C; k.o_meta = o; o += C;
        k.o_ttoi = o; o += C;
        k.o_order = o; o += C; k.o_newp = o; o += C; k.o_corder = o; o += C; k.o_cisl = o; o += C;
        k.o_awake = o; o += B; k.o_active = o; o += B; k.o_bisl = o; o += B; k.o_stack = o; o += B; k.o_fwork = o; o += B; k.o_ibuf = o; o += B;
        k.o_jorder = o; o += J; k.o_jisl = o; o += J;
        k.o_qbox = o; o += 4 * R;
        k.o_nlive = o; o += 1;
        k.words = o;
        return k;
    }
};

// ---- State leaf shapes and the packed layout
//
// Per-world element count of each leaf: dim (0 = B, 1 = R, 2 = J, 3 = C, 4 = one per world) times mult, of `bytes`
// each (the enum GoiLeaf table of goi_b2.h). A packed State holds its leaves as consecutive parts of one device
// buffer in leaf order, leaf l taking leaf_words(l) x pitch 4-byte words (its per-world bytes rounded up to a
// multiple of 4); with the pitch a multiple of 64, element (i, w) of leaf l is then element
// ((4 / bytes) packed_word(l) + i) x pitch + w of the buffer viewed with the leaf's element type, one base pointer
// for every leaf.
struct LeafDim {
    unsigned char dim, mult, bytes;
};
constexpr LeafDim kLeafDims[GOI_NUM_LEAVES] = {
    {0, 1, 4}, {0, 1, 1}, {0, 1, 1}, {0, 1, 1}, {0, 1, 1}, {0, 1, 1}, {0, 1, 4}, {0, 2, 4}, {0, 2, 4}, {0, 2, 4},
    {0, 2, 4}, {0, 2, 4}, {0, 1, 4}, {0, 1, 4}, {0, 2, 4}, {0, 1, 4}, {0, 2, 4}, {0, 1, 4}, {0, 1, 4}, {0, 1, 4},
    {0, 1, 4}, {0, 1, 4}, {0, 1, 4}, {0, 1, 4}, {0, 1, 4},                                    // bodies
    {1, 1, 4}, {1, 1, 4}, {1, 4, 4},                                                          // fixtures
    {2, 1, 1}, {2, 1, 4}, {2, 1, 4}, {2, 1, 1}, {2, 1, 4}, {2, 1, 4}, {2, 1, 4}, {2, 1, 4}, {2, 3, 4}, {2, 1, 4},
    {2, 1, 4}, {2, 1, 4}, {2, 1, 4},                                                          // joints
    {3, 1, 4}, {3, 1, 4}, {3, 1, 4}, {3, 1, 4}, {3, 1, 1}, {3, 1, 4}, {3, 1, 4}, {3, 2, 4}, {3, 2, 4}, {3, 4, 4},
    {3, 2, 4}, {3, 2, 4}, {3, 2, 4}, {3, 1, 4}, {3, 1, 4}, {3, 1, 4},                         // contacts
    {4, 2, 4}, {4, 1, 4}, {4, 1, 4}, {4, 1, 1}, {4, 1, 4},                                    // world scalars
    {0, 1, 4}, {3, 1, 4}, {3, 1, 4}, {3, 1, 1}, {3, 1, 1}, {3, 1, 1}, {3, 2, 4}, {3, 2, 4}, {4, 1, 4},  // ContactTOI
};
static_assert(kLeafDims[GOI_S_NEW_FIXTURE].bytes == 1 && kLeafDims[GOI_C_POINT_LOCAL].mult == 4 &&
                  kLeafDims[GOI_J_IMPULSE].mult == 3 && kLeafDims[GOI_T_EVENTS].dim == 4 &&
                  kLeafDims[GOI_T_EVENTS].bytes == 4 && kLeafDims[GOI_T_SOLVED].bytes == 1,
              "kLeafDims follows enum GoiLeaf");
GOI_HD constexpr int leaf_count(int l, int B, int C, int J, int R) {
    const int d = kLeafDims[l].dim;
    return (d == 0 ? B : d == 1 ? R : d == 2 ? J : d == 3 ? C : 1) * kLeafDims[l].mult;
}
GOI_HD constexpr int leaf_words(int l, int B, int C, int J, int R) {
    return (leaf_count(l, B, C, J, R) * kLeafDims[l].bytes + 3) / 4;
}
// Words per unit of pitch before leaf l, as a closed form (coefficients of B, C, J, R, of the rounded-up quarters of
// the u8 leaves' counts, and a constant), so that it folds to a constant wherever the dimensions are constants.
struct PackedCoef {
    int b, c, j, r, one, ub, uc, uj;
};
struct PackedTable {
    PackedCoef k[GOI_NUM_LEAVES + 1];
};
constexpr PackedTable make_packed_table() {
    PackedTable t{};
    PackedCoef acc{};
    for (int l = 0; l < GOI_NUM_LEAVES; ++l) {
        t.k[l] = acc;
        const LeafDim d = kLeafDims[l];
        if (d.bytes == 4) {
            if (d.dim == 0) acc.b += d.mult;
            else if (d.dim == 1) acc.r += d.mult;
            else if (d.dim == 2) acc.j += d.mult;
            else if (d.dim == 3) acc.c += d.mult;
            else acc.one += d.mult;
        } else {  // u8 leaves have mult 1
            if (d.dim == 0) acc.ub += 1;
            else if (d.dim == 2) acc.uj += 1;
            else if (d.dim == 3) acc.uc += 1;
            else acc.one += (d.mult + 3) / 4;
        }
    }
    t.k[GOI_NUM_LEAVES] = acc;
    return t;
}
constexpr PackedTable kPackedTable = make_packed_table();
GOI_HD constexpr int packed_word(int l, int B, int C, int J, int R) {
    const PackedCoef& k = kPackedTable.k[l];
    return k.b * B + k.c * C + k.j * J + k.r * R + k.one + k.ub * ((B + 3) / 4) + k.uc * ((C + 3) / 4) +
           k.uj * ((J + 3) / 4);
}
constexpr int packed_word_sum(int l, int B, int C, int J, int R) {
    int k = 0;
    for (int j = 0; j < l; ++j) k += leaf_words(j, B, C, J, R);
    return k;
}
static_assert(packed_word(GOI_NUM_LEAVES, 5, 40, 3, 4) == packed_word_sum(GOI_NUM_LEAVES, 5, 40, 3, 4) &&
                  packed_word(GOI_C_TOUCHING, 7, 13, 2, 9) == packed_word_sum(GOI_C_TOUCHING, 7, 13, 2, 9) &&
                  packed_word(GOI_T_EVENTS, 1, 1, 1, 1) == packed_word_sum(GOI_T_EVENTS, 1, 1, 1, 1),
              "the closed form sums the leaves' words");
constexpr bool u8_leaves_have_mult_1() {
    for (int l = 0; l < GOI_NUM_LEAVES; ++l)
        if (kLeafDims[l].bytes == 1 && kLeafDims[l].dim != 4 && kLeafDims[l].mult != 1) return false;
    return true;
}
static_assert(u8_leaves_have_mult_1(), "the closed form assumes single-element u8 leaves");

#ifndef GOI_PACKED_STATE
#define GOI_PACKED_STATE 0  // 1 in the translation unit of the kernels that take packed States only
#endif
// One world's State: leaf pointers already offset by the world's index, plus the world's LDS workspace.
struct World {
    int pitch;
    int B, C, R, J;
    void* const* lv;  // leaf base pointers (kernel argument block)
    int w;
    int* ws;          // LDS workspace base + the world's index in the block
    int S;            // workspace stride (worlds per block)
    Workspace k;
    unsigned long long smask, dmask;  // static and dynamic bodies (Model.body_type, the same in every world)
    int sub, G;       // the lane's place in the world's lane group, and the group's size
    const MRow* frow_map;  // non-null for a State in the full fixture layout (DModel::row)

    // The State row of non-static fixture row r: r itself in the compact fixture layout, the fixture's own index in
    // the full layout, where every fixture has a row (world.py:98-101, 400-403; the static rows are never read: their
    // fat AABB, friction and restitution are the Model's).
    GOI_D int frow(int r) const {
#if GOI_PACKED_STATE
        return r;
#else
        return frow_map ? frow_map[r].fixture : r;
#endif
    }

    GOI_D Group grp() const { return Group{sub, G}; }

    GOI_D bool is_static(int b) const { return (smask >> b) & 1ull; }
    GOI_D bool is_dynamic(int b) const { return (dmask >> b) & 1ull; }

    GOI_D int& wi(int off, int i) const { return ws[(off + i) * S]; }
    GOI_D float& wf(int off, int i) const { return reinterpret_cast<float*>(ws)[(off + i) * S]; }
    // mirrored State leaves
    GOI_D int& pair(int c) const { return wi(k.o_pair, c); }      // contacts.pair
    GOI_D int& key(int c) const { return wi(k.o_key, c); }        // contacts.key
    GOI_D int& fa(int c) const { return wi(k.o_fa, c); }          // contacts.fa
    GOI_D int& fb(int c) const { return wi(k.o_fb, c); }          // contacts.fb
    // the slot's packed word (see Workspace): bodies of a live slot's fixtures, touching and point count, TOI state
    GOI_D int meta(int c) const { return wi(k.o_meta, c); }
    GOI_D void set_meta_bits(int c, int shift, int width, int v) const {
        int& m = wi(k.o_meta, c);
        const int mask = ((1 << width) - 1) << shift;
        m = (m & ~mask) | ((v << shift) & mask);
    }
    GOI_D int ba(int c) const { return (meta(c) >> kMetaBodyA) & 63; }
    GOI_D int bb(int c) const { return (meta(c) >> kMetaBodyB) & 63; }
    GOI_D void set_bodies(int c, int a, int b) const { set_meta_bits(c, kMetaBodyA, 12, a | (b << 6)); }
    // contacts.pair / key / fa / fb of the slot changed (the mirror's store writes back only such slots)
    GOI_D void mark_slot_changed(int c) const { set_meta_bits(c, kMetaSlotChanged, 1, 1); }
    // contacts.touching and contacts.count, read from the workspace and written through to the State
    GOI_D bool touching(int c) const { return (meta(c) >> kMetaTouch) & 1; }
    GOI_D int ccount(int c) const { return (meta(c) >> kMetaCount) & 3; }
    GOI_D void set_touch_count(int c, bool t, int n) const {
        // the State holds what the workspace held (both loaded together, every change made here): write only changes
        const int was = meta(c);
        const bool odd = (was >> kMetaOddLoad) & 1;
        set_meta_bits(c, kMetaTouch, 3, (t ? 1 : 0) | (n << 1));
        set_meta_bits(c, kMetaOddLoad, 1, 0);
        if (odd || ((was >> kMetaTouch) & 1) != (t ? 1 : 0)) u8(GOI_C_TOUCHING, c) = t ? 1 : 0;
        if (odd || ((was >> kMetaCount) & 3) != n) i32(GOI_C_COUNT, c) = n;
    }
    GOI_D int& awake(int b) const { return wi(k.o_awake, b); }    // bodies.awake
    // bodies.active, .bullet and .continuous (read-only in a step), one word per body: bits 0, 1 and 2
    GOI_D bool active(int b) const { return wi(k.o_active, b) & 1; }
    GOI_D bool bullet(int b) const { return (wi(k.o_active, b) >> 1) & 1; }
    GOI_D bool continuous(int b) const { return (wi(k.o_active, b) >> 2) & 1; }
    // toi.flag, toi.enabled and toi.count of a slot
    GOI_D int tflag(int c) const { return (meta(c) >> kMetaTFlag) & 1; }
    GOI_D int ten(int c) const { return (meta(c) >> kMetaTEn) & 1; }
    GOI_D int tcount(int c) const { return (meta(c) >> kMetaTCount) & 15; }
    GOI_D void set_tflag(int c, int v) const { set_meta_bits(c, kMetaTFlag, 1, v ? 1 : 0); }
    GOI_D void set_ten(int c, int v) const { set_meta_bits(c, kMetaTEn, 1, v ? 1 : 0); }
    GOI_D void set_tcount(int c, int v) const { set_meta_bits(c, kMetaTCount, 4, v); }
    GOI_D float& ttoi(int c) const { return wf(k.o_ttoi, c); }    // toi.toi
    // work arrays
    GOI_D int& order(int i) const { return wi(k.o_order, i); }
    GOI_D int& newp(int i) const { return wi(k.o_newp, i); }
    GOI_D int& corder(int i) const { return wi(k.o_corder, i); }
    GOI_D int& cisl(int c) const { return wi(k.o_cisl, c); }
    GOI_D int& bisl(int b) const { return wi(k.o_bisl, b); }
    GOI_D int& stack(int i) const { return wi(k.o_stack, i); }
    GOI_D float& fwork(int i) const { return wf(k.o_fwork, i); }
    GOI_D int& ibuf(int i) const { return wi(k.o_ibuf, i); }
    GOI_D int& jorder(int i) const { return wi(k.o_jorder, i); }
    GOI_D int& jisl(int j) const { return wi(k.o_jisl, j); }
    GOI_D int& nlive() const { return wi(k.o_nlive, 0); }   // length of the contact list in order()
    GOI_D void set_qbox(int r, float4 q) const {
        wf(k.o_qbox, 4 * r) = q.x; wf(k.o_qbox, 4 * r + 1) = q.y; wf(k.o_qbox, 4 * r + 2) = q.z; wf(k.o_qbox, 4 * r + 3) = q.w;
    }
    GOI_D float4 get_qbox(int r) const {
        return make_float4(wf(k.o_qbox, 4 * r), wf(k.o_qbox, 4 * r + 1), wf(k.o_qbox, 4 * r + 2), wf(k.o_qbox, 4 * r + 3));
    }

    // element (i, w) of a leaf; the element offset fits 32 bits (checked at launch), so the address is the leaf's
    // base plus one 32-bit product and sum
    template <typename T>
    GOI_D T& at(int leaf, int i) const {
#if GOI_PACKED_STATE
        // a packed State: every leaf from leaf 0's base, at its constant packed offset
        const uint32_t row = (uint32_t)(4 / sizeof(T)) * (uint32_t)packed_word(leaf, B, C, J, R) + (uint32_t)i;
        return reinterpret_cast<T*>(lv[0])[row * (uint32_t)pitch + (uint32_t)w];
#else
        return reinterpret_cast<T*>(lv[leaf])[(uint32_t)i * (uint32_t)pitch + (uint32_t)w];
#endif
    }
    GOI_D float& f(int leaf, int i) const {
        const int c = body_mirror_coef(leaf);  // a constant at every call site
        if (c >= 0) return wf(k.o_bm + c * B, i);
        return at<float>(leaf, i);
    }
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
        if (!awake(b)) {
            awake(b) = 1;
            f(GOI_B_SLEEP_TIME, b) = 0.0f;
        }
    }
    GOI_D void init_masks(const DModel& m) {
        smask = dmask = 0ull;
        for (int b = 0; b < B; ++b) {
            const int t = m.body_type[b];
            if (t == GOI_STATIC) smask |= 1ull << b;
            if (t == GOI_DYNAMIC) dmask |= 1ull << b;
        }
    }
};

// ---- block-cooperative copies between the State and the block's workspaces
//
// The per-world phases leave most lanes of a block idle, and a lane copying its own world's mirror would pay one
// memory round trip per element. Instead every lane of the block copies: lane l serves world j = l % S at rows r0 =
// l / S, r0 + stride, ... (stride = lanes / S), so one load or store instruction moves `stride` rows of every world,
// and each batch issues all its loads before the first use. A lane whose world lies beyond the batch stays idle.
struct BlockCopy {
    void* const* lv;   // the State's leaf base pointers
    int pitch, B, C, J, R, S;
    Workspace k;
    int* lds;          // the block's workspace base (world 0, word 0)
    int w, j, r0, stride;
    bool on;           // this lane copies for world w (= the block's world j)

    template <typename T>
    GOI_D T& at(int leaf, int i) const {
#if GOI_PACKED_STATE
        const uint32_t row = (uint32_t)(4 / sizeof(T)) * (uint32_t)packed_word(leaf, B, C, J, R) + (uint32_t)i;
        return reinterpret_cast<T*>(lv[0])[row * (uint32_t)pitch + (uint32_t)w];
#else
        return reinterpret_cast<T*>(lv[leaf])[(uint32_t)i * (uint32_t)pitch + (uint32_t)w];
#endif
    }
    // Streaming reads and writes of State words that the step touches once here (the mirror's load and store, the
    // TOI reset and store): non-temporal, so the L2 evicts these lines before the constraint rows and contact data
    // that the step reuses.
    template <typename T>
    GOI_D T ld(int leaf, int i) const { return __builtin_nontemporal_load(&at<T>(leaf, i)); }
    template <typename T>
    GOI_D void st(int leaf, int i, T v) const { __builtin_nontemporal_store(v, &at<T>(leaf, i)); }
    GOI_D int& wi(int off) const { return lds[off * S + j]; }
    GOI_D float& wf(int off) const { return reinterpret_cast<float*>(lds)[off * S + j]; }
};

// lanes: the block's lanes taking part (the whole block on the device, 1 for a sequential host build)
GOI_HD BlockCopy block_copy(void* const* lv, int pitch, int n, int B, int C, int J, int R, int S, int* lds, int w0,
                            int lane, int lanes) {
    BlockCopy bc;
    bc.lv = lv; bc.pitch = pitch; bc.B = B; bc.C = C; bc.J = J; bc.R = R; bc.S = S;
    bc.k = Workspace::layout(B, C, J, R);
    bc.lds = lds;
    bc.stride = lanes / S > 0 ? lanes / S : 1;
    bc.j = lane % S;
    bc.r0 = lane / S;
    bc.w = w0 + bc.j;
    bc.on = bc.r0 < bc.stride && bc.w < n;
    return bc;
}

constexpr int kCopyU = 8;  // rows per lane and leaf in one batch

// The mirrored leaves of the block's worlds into their workspaces (contact metadata, awake and active flags, the
// mirrored float body leaves, the bodies of every live slot). Called by every lane of the block.
GOI_D void load_mirror_block(const DModel& m, const BlockCopy& bc) {
    const Workspace& k = bc.k;
    if (bc.on) {
        // pair first; a free slot's other fields are never read in a step (every use is behind pair >= 0) and are
        // written back only if a contact is created there, so only live slots load them. A free slot starts with
        // the load-time flag set, so its first touching / count write goes through whatever the State held.
        for (int c0 = bc.r0; c0 < bc.C; c0 += kCopyU * bc.stride) {
            int p[kCopyU], ky[kCopyU], fa[kCopyU], fb[kCopyU], n[kCopyU];
            uint8_t t[kCopyU];
#pragma unroll
            for (int u = 0; u < kCopyU; ++u) p[u] = bc.ld<int>(GOI_C_PAIR, min(c0 + u * bc.stride, bc.C - 1));
#pragma unroll
            for (int u = 0; u < kCopyU; ++u) {
                const int c = min(c0 + u * bc.stride, bc.C - 1);
                ky[u] = fa[u] = fb[u] = n[u] = 0;
                t[u] = 2;  // a free slot: flagged below
                if (p[u] >= 0) {
                    ky[u] = bc.ld<int>(GOI_C_KEY, c);
                    fa[u] = bc.ld<int>(GOI_C_FA, c);
                    fb[u] = bc.ld<int>(GOI_C_FB, c);
                    t[u] = bc.ld<uint8_t>(GOI_C_TOUCHING, c);
                    n[u] = bc.ld<int>(GOI_C_COUNT, c);
                }
            }
#pragma unroll
            for (int u = 0; u < kCopyU; ++u) {
                const int c = c0 + u * bc.stride;
                if (c < bc.C) {
                    bc.wi(k.o_pair + c) = p[u];
                    bc.wi(k.o_key + c) = ky[u];
                    bc.wi(k.o_fa + c) = fa[u];
                    bc.wi(k.o_fb + c) = fb[u];
                    const bool odd = t[u] > 1 || (unsigned)n[u] > 2u;
                    const bool touch = p[u] >= 0 && t[u] != 0;
                    bc.wi(k.o_meta + c) = ((touch ? 1 : 0) << kMetaTouch) | ((n[u] & 3) << kMetaCount) |
                                          ((odd ? 1 : 0) << kMetaOddLoad);
                }
            }
        }
        // the float body leaves: rows i < width * B of each, at word coef * B + i
        for (int i0 = bc.r0; i0 < 2 * bc.B; i0 += 2 * bc.stride) {
            float v[13][2];
            uint8_t aw[2], ac[2], bu[2], co[2];
#pragma unroll
            for (int l = 0; l < 13; ++l) {
                const int rows = kBodyMirrorWidth[l] * bc.B;
#pragma unroll
                for (int u = 0; u < 2; ++u) v[l][u] = bc.ld<float>(kBodyMirrorLeaves[l], min(i0 + u * bc.stride, rows - 1));
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int b = min(i0 + u * bc.stride, bc.B - 1);
                aw[u] = bc.ld<uint8_t>(GOI_B_AWAKE, b);
                ac[u] = bc.ld<uint8_t>(GOI_B_ACTIVE, b);
                bu[u] = bc.ld<uint8_t>(GOI_B_BULLET, b);
                co[u] = bc.ld<uint8_t>(GOI_B_CONTINUOUS, b);
            }
#pragma unroll
            for (int l = 0; l < 13; ++l) {
                const int rows = kBodyMirrorWidth[l] * bc.B, off = k.o_bm + body_mirror_coef(kBodyMirrorLeaves[l]) * bc.B;
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int i = i0 + u * bc.stride;
                    if (i < rows) bc.wf(off + i) = v[l][u];
                }
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int b = i0 + u * bc.stride;
                if (b < bc.B) {
                    bc.wi(k.o_awake + b) = aw[u];
                    bc.wi(k.o_active + b) = (ac[u] != 0 ? 1 : 0) | (bu[u] != 0 ? 2 : 0) | (co[u] != 0 ? 4 : 0);
                }
            }
        }
    }
    __syncthreads();
    // the bodies of each live slot's fixtures
    if (bc.on) {
        for (int c0 = bc.r0; c0 < bc.C; c0 += kCopyU * bc.stride) {
            int ba[kCopyU], bb[kCopyU];
            bool live[kCopyU];
#pragma unroll
            for (int u = 0; u < kCopyU; ++u) {
                const int c = c0 + u * bc.stride, cc = min(c, bc.C - 1);
                live[u] = c < bc.C && bc.wi(k.o_pair + cc) >= 0;
                ba[u] = m.fix[live[u] ? bc.wi(k.o_fa + cc) : 0].body;
                bb[u] = m.fix[live[u] ? bc.wi(k.o_fb + cc) : 0].body;
            }
#pragma unroll
            for (int u = 0; u < kCopyU; ++u)
                if (live[u]) bc.wi(k.o_meta + c0 + u * bc.stride) |= (ba[u] << kMetaBodyA) | (bb[u] << kMetaBodyB);
        }
    }
    __syncthreads();
}

// Box2D's contact list of the block's worlds (newest first = descending key, pairs.py:12-13) into each workspace's
// order(0 .. nlive-1): each live slot's position is the number of live slots with a larger key (keys of live slots
// are distinct). Every lane ranks its rows of its world. Called by every lane after load_mirror_block.
// The ranks read each world's keys from a contiguous copy in its newp rows (free until FindNewContacts), a free
// slot's key replaced by INT32_MIN, which no key is below: one comparison per slot, four slots per load.
GOI_D void build_order_block(const BlockCopy& bc) {
    const Workspace& k = bc.k;
    int* const keys = bc.lds + k.o_newp * bc.S + bc.j * bc.C;
    if (bc.on)
        for (int c = bc.r0; c < bc.C; c += bc.stride)
            keys[c] = bc.wi(k.o_pair + c) >= 0 ? bc.wi(k.o_key + c) : INT32_MIN;
    __syncthreads();
    if (bc.on) {
        const bool by4 = bc.C % 4 == 0 && (k.o_newp * bc.S) % 4 == 0;  // every world's copy 16-byte aligned
        for (int c = bc.r0; c < bc.C; c += bc.stride) {
            if (bc.wi(k.o_pair + c) < 0) continue;
            const int key = keys[c];
            int rank = 0;
            if (by4) {
                const int4* const k4 = reinterpret_cast<const int4*>(keys);
                for (int q = 0; q < bc.C / 4; ++q) {
                    const int4 t = k4[q];
                    rank += (t.x > key ? 1 : 0) + (t.y > key ? 1 : 0) + (t.z > key ? 1 : 0) + (t.w > key ? 1 : 0);
                }
            } else {
                for (int i = 0; i < bc.C; ++i) rank += keys[i] > key ? 1 : 0;
            }
            bc.wi(k.o_order + rank) = c;
        }
        if (bc.r0 == 0) {
            int n = 0;
#pragma unroll 8
            for (int i = 0; i < bc.C; ++i) n += bc.wi(k.o_pair + i) >= 0 ? 1 : 0;
            bc.wi(k.o_nlive) = n;
        }
    }
    __syncthreads();
}

// The workspaces' mutable mirrored leaves back into the State (contact metadata, awake flags, the first
// kBodyMirrorMutable float body leaves). Called by every lane of the block after the worlds' last writes.
GOI_D void store_mirror_block(const BlockCopy& bc) {
    __syncthreads();
    if (!bc.on) return;
    const Workspace& k = bc.k;
    for (int c = bc.r0; c < bc.C; c += bc.stride) {
        // a slot whose contact was neither created nor destroyed holds the values the State already has
        if (!((bc.wi(k.o_meta + c) >> kMetaSlotChanged) & 1)) continue;
        bc.st<int>(GOI_C_PAIR, c, bc.wi(k.o_pair + c));
        bc.st<int>(GOI_C_KEY, c, bc.wi(k.o_key + c));
        bc.st<int>(GOI_C_FA, c, bc.wi(k.o_fa + c));
        bc.st<int>(GOI_C_FB, c, bc.wi(k.o_fb + c));
    }
    for (int b = bc.r0; b < bc.B; b += bc.stride) bc.st<uint8_t>(GOI_B_AWAKE, b, (uint8_t)bc.wi(k.o_awake + b));
#pragma unroll
    for (int l = 0; l < kBodyMirrorMutable; ++l) {
        const int rows = kBodyMirrorWidth[l] * bc.B, off = k.o_bm + body_mirror_coef(kBodyMirrorLeaves[l]) * bc.B;
        for (int i = bc.r0; i < rows; i += bc.stride) bc.st<float>(kBodyMirrorLeaves[l], i, bc.wf(off + i));
    }
}

// SolveTOI's reset (world.py:157-161, toi.py:837) of the block's worlds: alpha0 = 0, count 0, toi 1, flag off,
// enabled, not solved, report impulses 0. Called by every lane; the barriers order it after the worlds' last writes
// of their slots' packed words and before their next reads.
GOI_D void reset_toi_block(const BlockCopy& bc) {
    __syncthreads();
    if (bc.on) {
        const Workspace& k = bc.k;
        const int oa = k.o_bm + body_mirror_coef(GOI_T_ALPHA0) * bc.B;
        for (int b = bc.r0; b < bc.B; b += bc.stride) bc.wf(oa + b) = 0.0f;
        for (int c = bc.r0; c < bc.C; c += bc.stride) {
            // count 0, enabled, no flag; the slot's other fields stay
            int& mt = bc.wi(k.o_meta + c);
            mt = (mt & ~((1 << kMetaTFlag) | (1 << kMetaTEn) | (15 << kMetaTCount))) | (1 << kMetaTEn);
            bc.wf(k.o_ttoi + c) = 1.0f;
            bc.st<uint8_t>(GOI_T_SOLVED, c, 0);
        }
        for (int i = bc.r0; i < 2 * bc.C; i += bc.stride) {
            bc.st<float>(GOI_T_NORMAL_IMPULSE, i, 0.0f);
            bc.st<float>(GOI_T_TANGENT_IMPULSE, i, 0.0f);
        }
    }
    __syncthreads();
}

// The TOI bookkeeping of the block's worlds into the State. Called by every lane after SolveTOI.
GOI_D void store_toi_block(const BlockCopy& bc) {
    __syncthreads();
    if (!bc.on) return;
    const Workspace& k = bc.k;
    for (int c = bc.r0; c < bc.C; c += bc.stride) {
        const int t = bc.wi(k.o_meta + c);
        bc.st<uint8_t>(GOI_T_FLAG, c, (uint8_t)((t >> kMetaTFlag) & 1));
        bc.st<uint8_t>(GOI_T_ENABLED, c, (uint8_t)((t >> kMetaTEn) & 1));
        bc.st<int>(GOI_T_COUNT, c, (t >> kMetaTCount) & 15);
        bc.st<float>(GOI_T_TOI, c, bc.wf(k.o_ttoi + c));
    }
}

// Fat AABB of a fixture in the compact layout: the world's own row, or the Model's shared static box.
GOI_D float4 fat_of(const DModel& m, const World& W, int fixture) {
    const int r = m.fix[fixture].slot;
    if (r < 0) return m.fix[fixture].fat;
    const int i = 4 * W.frow(r);
    return make_float4(W.f(GOI_F_FAT, i), W.f(GOI_F_FAT, i + 1), W.f(GOI_F_FAT, i + 2), W.f(GOI_F_FAT, i + 3));
}
GOI_D float friction_of(const DModel& m, const World& W, int fixture) {
    const int r = m.fix[fixture].slot;
    return r < 0 ? m.fix[fixture].friction : W.f(GOI_F_FRICTION, W.frow(r));
}
GOI_D float restitution_of(const DModel& m, const World& W, int fixture) {
    const int r = m.fix[fixture].slot;
    return r < 0 ? m.fix[fixture].restitution : W.f(GOI_F_RESTITUTION, W.frow(r));
}

// b2TestOverlap
GOI_D bool overlap(float4 a, float4 b) {
    float d1x = b.x - a.z, d1y = b.y - a.w;
    float d2x = a.x - b.z, d2y = a.y - b.w;
    return !(d1x > 0.0f || d1y > 0.0f || d2x > 0.0f || d2y > 0.0f);
}

// Per-world HBM scratch rows, in tiles: the S worlds of a block share one tile of nrows x nf x S words, and element
// (row, field) of the block's world `lane` is tile[(row * nf + field) * S + lane]. A row's fields for the block's
// worlds are contiguous (one row is a few 128-byte lines, not one line per field), and the field offsets fold into the
// load and store instructions. Word offsets fit 32 bits (checked at launch).
struct Rows {
    uint32_t* base;  // the tile's word 0 of this world
    int nf, S;
    // the row's word 0 first, then the field in it: a constant field becomes a constant offset from one row address
    // (one address computation per row, not one per field)
    GOI_D uint32_t& u(int row, int field) const {
        uint32_t* const r = base + (uint32_t)row * (uint32_t)(nf * S);
        return r[(uint32_t)field * (uint32_t)S];
    }
    GOI_D float getf(int row, int field) const { return __uint_as_float(u(row, field)); }
    GOI_D void setf(int row, int field, float v) const { u(row, field) = __float_as_uint(v); }
    GOI_D int geti(int row, int field) const { return (int)u(row, field); }
    GOI_D void seti(int row, int field, int v) const { u(row, field) = (uint32_t)v; }
    GOI_D V2 get2(int row, int field) const { return mk(getf(row, field), getf(row, field + 1)); }
    GOI_D void set2(int row, int field, V2 v) const { setf(row, field, v.x); setf(row, field + 1, v.y); }
};
// The rows of world `lane` of tile `tile` in a region of tiles of nrows x nf x S words.
GOI_D Rows rows_of(uint32_t* region, int nrows, int nf, int S, int tile, int lane) {
    Rows R;
    R.base = region + (size_t)tile * ((size_t)nrows * nf * S) + lane;
    R.nf = nf;
    R.S = S;
    return R;
}
// The same tile read world-major: world `lane` owns words [lane * nrows * nf, (lane + 1) * nrows * nf) of it, a row's
// fields contiguous. For rows that one world writes while the block's other worlds write none (SolveTOI's task
// snapshots and event islands): its stores then fill whole lines instead of one 4-byte word in each 32 bytes.
GOI_D Rows rows_world_major(uint32_t* region, int nrows, int nf, int S, int tile, int lane) {
    Rows R;
    R.base = region + (size_t)tile * ((size_t)nrows * nf * S) + (size_t)lane * ((size_t)nrows * nf);
    R.nf = nf;
    R.S = 1;
    return R;
}

// contact constraint row fields
enum {
    CF_SLOT, CF_IA, CF_IB, CF_COUNT, CF_PC_COUNT, CF_MTYPE,
    CF_MA, CF_MB, CF_IIA, CF_IIB, CF_NX, CF_NY, CF_FRICTION, CF_TSPEED,
    CF_RA0, CF_RA0Y, CF_RA1, CF_RA1Y, CF_RB0, CF_RB0Y, CF_RB1, CF_RB1Y,
    CF_NMASS0, CF_NMASS1, CF_TMASS0, CF_TMASS1, CF_BIAS0, CF_BIAS1,
    CF_NI0, CF_NI1, CF_TI0, CF_TI1, CF_K0, CF_K1, CF_K2, CF_K3, CF_NM0, CF_NM1, CF_NM2, CF_NM3,
    CF_LN, CF_LNY, CF_LP, CF_LPY, CF_PL0, CF_PL0Y, CF_PL1, CF_PL1Y, CF_LCA, CF_LCAY, CF_LCB, CF_LCBY,
    CF_RADA, CF_RADB,
    CF_N
};

// joint row fields
enum {
    JF_JID, JF_TYPE, JF_IA, JF_IB, JF_STATE, JF_EMOTOR, JF_ELIMIT, JF_SOFT,
    JF_MA, JF_MB, JF_IIA, JF_IIB, JF_RA, JF_RAY, JF_RB, JF_RBY,
    JF_EXX, JF_EXY, JF_EXZ, JF_EYX, JF_EYY, JF_EYZ, JF_EZX, JF_EZY, JF_EZZ,
    JF_MMASS, JF_MSPEED, JF_MAXIMP, JF_AX, JF_AXY, JF_PX, JF_PXY, JF_A1, JF_A2, JF_S1, JF_S2,
    JF_GAMMA, JF_BIAS, JF_ANGLE, JF_INVDT, JF_LA, JF_LAY, JF_LB, JF_LBY, JF_LX, JF_LXY, JF_LY, JF_LYY,
    JF_REF, JF_LOWER, JF_UPPER, JF_IMP0, JF_IMP1, JF_IMP2, JF_IMP3, JF_IMP4, JF_MIMP,
    JF_N
};


}  // namespace goi
