/* goi_b2.h - C ABI of the MI355X batched Box2D 2.3.1 world step (libgoi_b2.so).
 *
 * The library steps N independent worlds that share one Model, on the GPU, in place, on caller-owned device
 * buffers. It replaces the reference's operator boundary for this path:
 *   - goi_jax/box2d/step.py:28          step(model, state, settings, dt, axis_name=None)
 *   - goi_jax/box2d/step.py:36-40       Settings.solver dispatch to the batched kernels
 *   - goi_jax/box2d/gpu/kernel.py:573-598, gpu/pairs.py:242-263, gpu/toi_loop.py:66-130
 *                                      the custom_vmap rules that receive the whole batch and run one kernel
 *   - goi_jax/reference/capi.cpp:184-189 goi_b2_world_step (int return codes, ids in creation order)
 *
 * Data layout. A State is the reference pytree (goi_jax/box2d/world.py:70-174) flattened in field order into
 * GOI_NUM_LEAVES leaves (enum GoiLeaf below). Each leaf of per-world inner shape S (e.g. contacts.point_local has
 * S = [C, 2, 2]) is one device array stored worlds-minor: element (inner index i, world w) lives at
 * leaf[i * pitch + w]. Bools are uint8 (0/1), ints int32, floats IEEE binary32. The leaves may live anywhere; a
 * State whose leaves are the consecutive parts of one buffer (goi_packed_layout) with a pitch that is a multiple of 64
 * is "packed", and the step addresses every leaf from one base pointer (the fast instance of the 4-body rig needs it).
 *
 * Return codes (capi.cpp style): 0 ok, GOI_E_ARG bad argument, GOI_E_SHAPE capacity/shape mismatch, GOI_E_HIP a HIP
 * runtime error, GOI_E_UNSUPPORTED settings or model the kernels do not cover. goi_last_error() returns a
 * thread-local message for the last failure. Contact-table overflow is not an error: it is counted in the overflow
 * leaf (world.py:173), as the reference does.
 *
 * Threading: calls are stream-ordered and asynchronous on the given hipStream_t (NULL = default stream). A model
 * handle may be shared by calls on different streams and from different host threads. Its shape tables are
 * read-only after creation; its one mutable part is the scratch memory of goi_step, goi_step_n and goi_collide (the
 * constraint and task rows), which it keeps per stream: one device buffer per stream handle, allocated on that
 * stream's first call and replaced by a larger one when a larger batch arrives on that stream (the old buffer is
 * freed after that stream's earlier work has finished). The buffers stay until goi_model_release_rows or
 * goi_model_destroy, so each stream a handle was used on holds one. Calls on different streams therefore never share rows, and
 * calls on one stream are ordered by it. A mutex in the handle covers the table from lookup through launch. A state
 * must not be stepped by two calls at once. goi_model_destroy waits for the device to finish (hipDeviceSynchronize)
 * before freeing, and must not overlap other calls on the same handle.
 */
#ifndef GOI_B2_H
#define GOI_B2_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GOI_ABI_VERSION 5

#define GOI_OK 0
#define GOI_E_ARG (-1)
#define GOI_E_SHAPE (-2)
#define GOI_E_HIP (-3)
#define GOI_E_UNSUPPORTED (-4)

/* Box2D enums as the reference numbers them (world.py:24-27, shapes.py:13, collide.py:18). */
#define GOI_STATIC 0
#define GOI_KINEMATIC 1
#define GOI_DYNAMIC 2
#define GOI_REVOLUTE 1
#define GOI_PRISMATIC 2
#define GOI_WELD 8
#define GOI_CIRCLE 0
#define GOI_POLYGON 2
#define GOI_MAX_POLY 8
/* b2Shape::e_edge, which the reference does not use (shapes.py:13: "edge 1 and chain 3 are not used by the game").
 * An edge fixture holds b2EdgeShape: verts[f][0..1] = m_vertex1, m_vertex2 and count[f] = 2 (its distance proxy),
 * verts[f][2] = m_vertex0 and verts[f][3] = m_vertex3 (the ghost vertices), edge_flags[f] = GOI_EDGE_HAS_V0 |
 * GOI_EDGE_HAS_V3 as m_hasVertex0 / m_hasVertex3 are set. A b2ChainShape is its child edges (b2ChainShape::
 * GetChildEdge), one edge fixture each, in child order, flagged GOI_EDGE_CHAIN (their fat AABBs, which the caller
 * computes, have no skin radius: b2ChainShape::ComputeAABB). Edge fixtures belong to static bodies only, and a
 * candidate pair names the edge first (b2Contact::Create). */
#define GOI_EDGE 1
#define GOI_EDGE_HAS_V0 1
#define GOI_EDGE_HAS_V3 2
#define GOI_EDGE_CHAIN 4

/* The State leaves in pytree order (world.py:70-174). Per-world inner shapes in brackets: B bodies, R fixture rows
 * (F in the full layout, the non-static fixtures in the compact layout, world.py:400-434), J joints, C slots. */
enum GoiLeaf {
    /* Bodies (world.py:70-95) */
    GOI_B_TYPE = 0,       /* i32[B]   */
    GOI_B_ACTIVE,         /* u8[B]    */
    GOI_B_AWAKE,          /* u8[B]    */
    GOI_B_ALLOW_SLEEP,    /* u8[B]    */
    GOI_B_BULLET,         /* u8[B]    */
    GOI_B_CONTINUOUS,     /* u8[B]    */
    GOI_B_SLEEP_TIME,     /* f32[B]   */
    GOI_B_XF_P,           /* f32[B,2] */
    GOI_B_XF_Q,           /* f32[B,2] (cos, sin) */
    GOI_B_LOCAL_CENTER,   /* f32[B,2] */
    GOI_B_C0,             /* f32[B,2] */
    GOI_B_C,              /* f32[B,2] */
    GOI_B_A0,             /* f32[B]   */
    GOI_B_A,              /* f32[B]   */
    GOI_B_V,              /* f32[B,2] */
    GOI_B_W,              /* f32[B]   */
    GOI_B_FORCE,          /* f32[B,2] */
    GOI_B_TORQUE,         /* f32[B]   */
    GOI_B_MASS,           /* f32[B]   */
    GOI_B_INV_MASS,       /* f32[B]   */
    GOI_B_INERTIA,        /* f32[B]   */
    GOI_B_INV_INERTIA,    /* f32[B]   */
    GOI_B_LINEAR_DAMPING, /* f32[B]   */
    GOI_B_ANGULAR_DAMPING,/* f32[B]   */
    GOI_B_GRAVITY_SCALE,  /* f32[B]   */
    /* Fixtures (world.py:98-101) */
    GOI_F_FRICTION,       /* f32[R]   */
    GOI_F_RESTITUTION,    /* f32[R]   */
    GOI_F_FAT,            /* f32[R,4] lower x, lower y, upper x, upper y */
    /* Joints (world.py:104-118) */
    GOI_J_ENABLE_MOTOR,   /* u8[J]    */
    GOI_J_MOTOR_SPEED,    /* f32[J]   (the action-driven motor target) */
    GOI_J_MAX_MOTOR,      /* f32[J]   */
    GOI_J_ENABLE_LIMIT,   /* u8[J]    */
    GOI_J_LOWER,          /* f32[J]   */
    GOI_J_UPPER,          /* f32[J]   */
    GOI_J_FREQUENCY,      /* f32[J]   */
    GOI_J_DAMPING,        /* f32[J]   */
    GOI_J_IMPULSE,        /* f32[J,3] */
    GOI_J_MOTOR_IMPULSE,  /* f32[J]   */
    GOI_J_LIMIT_STATE,    /* i32[J]   */
    GOI_J_LOWER_IMPULSE,  /* f32[J]   */
    GOI_J_UPPER_IMPULSE,  /* f32[J]   */
    /* Contacts (world.py:121-139) */
    GOI_C_PAIR,           /* i32[C]   candidate index, -1 empty slot */
    GOI_C_FA,             /* i32[C]   */
    GOI_C_FB,             /* i32[C]   */
    GOI_C_KEY,            /* i32[C]   */
    GOI_C_TOUCHING,       /* u8[C]    */
    GOI_C_MTYPE,          /* i32[C]   */
    GOI_C_COUNT,          /* i32[C]   */
    GOI_C_LOCAL_NORMAL,   /* f32[C,2] */
    GOI_C_LOCAL_POINT,    /* f32[C,2] */
    GOI_C_POINT_LOCAL,    /* f32[C,2,2] */
    GOI_C_POINT_ID,       /* i32[C,2] */
    GOI_C_NORMAL_IMPULSE, /* f32[C,2] */
    GOI_C_TANGENT_IMPULSE,/* f32[C,2] */
    GOI_C_FRICTION,       /* f32[C]   */
    GOI_C_RESTITUTION,    /* f32[C]   */
    GOI_C_TANGENT_SPEED,  /* f32[C]   */
    /* World scalars (world.py:169-173) */
    GOI_S_GRAVITY,        /* f32[2]   */
    GOI_S_INV_DT0,        /* f32[]    */
    GOI_S_NEXT_KEY,       /* i32[]    */
    GOI_S_NEW_FIXTURE,    /* u8[]     */
    GOI_S_OVERFLOW,       /* i32[]    */
    /* ContactTOI (world.py:142-154) */
    GOI_T_ALPHA0,         /* f32[B]   */
    GOI_T_COUNT,          /* i32[C]   */
    GOI_T_TOI,            /* f32[C]   */
    GOI_T_FLAG,           /* u8[C]    */
    GOI_T_ENABLED,        /* u8[C]    */
    GOI_T_SOLVED,         /* u8[C]    */
    GOI_T_NORMAL_IMPULSE, /* f32[C,2] */
    GOI_T_TANGENT_IMPULSE,/* f32[C,2] */
    GOI_T_EVENTS,         /* i32[]    */
    GOI_NUM_LEAVES
};

/* Settings (settings.py:42-107) as a POD. The step reads gravity from the State (world.py:169), as the reference
 * does. max_events < 0 selects the reference default C * (b2_maxSubSteps + 1) + 8 (toi.py:838-840). */
typedef struct GoiSettings {
    int32_t velocity_iterations;
    int32_t position_iterations;
    float linear_slop;
    float angular_slop;
    float polygon_radius;
    float velocity_threshold;
    float max_linear_correction;
    float max_angular_correction;
    float max_translation;
    float max_rotation;
    float baumgarte;
    float toi_baumgarte;
    float time_to_sleep;
    float linear_sleep_tolerance;
    float angular_sleep_tolerance;
    int32_t clamps_per_second;
    int32_t allow_sleep;
    int32_t warm_starting;
    int32_t continuous_physics;
    int32_t unity_toi;
    int32_t toi_tie_oldest;
    int32_t auto_clear_forces;
    int32_t revolute_v24;
    int32_t max_events;
} GoiSettings;

/* The shared Model (world.py:30-67), host pointers. fixture_slot == NULL is the full fixture layout; otherwise the
 * compact layout (world.py:437-472): fixture_slot[f] is the State row of fixture f or -1 for a static body's
 * fixture, whose fat AABB, friction and restitution are static_fat/static_friction/static_restitution[f].
 * body_type[B] are the body types every world shares (the compact layout requires it, world.py:447-450).
 * toi_bodies[B] (nullable) is Model.toi_bodies (world.py:48-50).
 * centroid[F,2] and edge_flags[F] exist only for edge fixtures (GOI_EDGE): b2PolygonShape::m_centroid of each
 * polygon, which edge-polygon contacts read, and each edge's ghost flags. Both may be NULL when no fixture is an
 * edge. */
typedef struct GoiModelDesc {
    int32_t F, J, P, B;
    const int32_t* fixture_body;   /* [F] */
    const int32_t* shape_type;     /* [F] */
    const float* radius;           /* [F] */
    const int32_t* count;          /* [F] */
    const float* verts;            /* [F,8,2] */
    const float* normals;          /* [F,8,2] */
    const int32_t* joint_type;     /* [J] */
    const int32_t* joint_a;        /* [J] */
    const int32_t* joint_b;        /* [J] */
    const float* local_anchor_a;   /* [J,2] */
    const float* local_anchor_b;   /* [J,2] */
    const float* local_axis_a;     /* [J,2] */
    const float* local_yaxis_a;    /* [J,2] */
    const float* reference_angle;  /* [J] */
    const int32_t* pair_a;         /* [P] */
    const int32_t* pair_b;         /* [P] */
    const int32_t* fixture_slot;   /* [F] or NULL */
    const float* static_fat;       /* [F,4] or NULL */
    const float* static_friction;  /* [F] or NULL */
    const float* static_restitution; /* [F] or NULL */
    const int32_t* body_type;      /* [B] */
    const uint8_t* toi_bodies;     /* [B] or NULL */
    const float* centroid;         /* [F,2] or NULL (required when an edge fixture exists) */
    const int32_t* edge_flags;     /* [F] or NULL (no ghost vertices) */
} GoiModelDesc;

/* A batch of States on the device: GOI_NUM_LEAVES device pointers, worlds-minor with the given pitch (>= n). R is the
 * fixture rows of the fixture leaves: the model's non-static fixtures (the compact layout) or all F of its fixtures
 * (the full layout that WorldDef.build returns, world.py:98-101; a reader tells the two apart by the row count, as
 * world.py:400-403 does). In the full layout the step reads and writes only the non-static fixtures' rows: the
 * static rows stay as they are, their values taken from the model, which must have been made from them
 * (compact_model checks that they agree in every world). */
typedef struct GoiStateView {
    int32_t n_worlds;
    int32_t pitch;
    int32_t B, C, R, J;
    void* leaf[GOI_NUM_LEAVES];
} GoiStateView;

/* Optional per-world integer outputs that are not State leaves: Solve's islands and solve order, and a trace of
 * SolveTOI's first GOI_DEBUG_TOI_EVENTS events (which contact, when, and the island the event's walk built,
 * toi.py:604-716). Each pointer may be NULL; a non-NULL one receives its array worlds-minor with the view's pitch
 * (element (i, w) at [i * pitch + w]; the rows of event e at i = e * GOI_DEBUG_TOI_ROWS + row). Event entries past
 * the step's last event hold slot -1, alpha 0, island 0 and rows -1. */
#define GOI_DEBUG_TOI_EVENTS 8
#define GOI_DEBUG_TOI_ROWS 32 /* b2_maxTOIContacts: an event island's contact cap */
typedef struct GoiDebug {
    int32_t* body_island;      /* [B] island of each body after Solve's search, -1 none (island.py:33) */
    int32_t* contact_island;   /* [C] (island.py:34) */
    int32_t* contact_order;    /* [C] slots in solve order, -1 padded (island.py:29) */
    int32_t* n_islands;        /* [] */
    int32_t* toi_event_slot;   /* [E] the event's contact slot (the TOI search's minimum) */
    int32_t* toi_event_alpha;  /* [E] the bits of its float minAlpha */
    int32_t* toi_event_island; /* [E] island contacts | island bodies << 16; 0 when the contact stopped touching */
    int32_t* toi_island_rows;  /* [E, 32] the island's contact slots in walk order (the event's contact first), -1 padded */
    int32_t* status;           /* [] the world's GOI_STATUS_* bits for the step (below) */
} GoiDebug;

/* GoiDebug::status bits, the failure counters of a step as one word per world (the reference keeps them as State
 * counters and bench checks: world.py:154, 173; toi.py:838-842; bench_gpu.py:135-136). */
#define GOI_STATUS_OVERFLOW 1    /* FindNewContacts dropped a pair on a full contact table (State.overflow grew) */
#define GOI_STATUS_NONFINITE 2   /* a body's position, angle or velocity is not finite after the step */
#define GOI_STATUS_TOI_CAPPED 4  /* SolveTOI stopped at max_events with another event pending (toi.py:838-842) */
#define GOI_STATUS_TOI_SKIPPED 8 /* continuous physics on but dt <= 0, so SolveTOI did not run (toi.py:841) */

typedef struct GoiModel GoiModel;

/* ABI version of the loaded library (GOI_ABI_VERSION). */
int32_t goi_abi_version(void);

/* Upload the shared Model to the current device and build the static-terrain acceleration structures: the
 * bounding-volume hierarchy over static fixtures' fat AABBs and the candidate-index table. The library owns *out.
 * Replaces the host build of world.py:331-386 + compact_model (world.py:437-472) for the device. */
int32_t goi_model_create(const GoiModelDesc* desc, int32_t contact_capacity, void* hip_stream, GoiModel** out);
int32_t goi_model_destroy(GoiModel* model);

/* Frees the handle's per-stream constraint and task rows (goi_step, goi_step_n and goi_collide keep one buffer per
 * stream handle they were called on, (C * 54 + J * 57 + 2) * (pitch + 64) 4-byte words each, the last 2 * (pitch +
 * 64) of them a launch's block order and its blocks' times: about 153 MB for 16,384 worlds of the 4-body rig, until
 * goi_model_destroy). A caller that steps on many short-lived or pooled streams calls
 * it to return that memory; the next call on a stream allocates its buffer again. Waits for the model's device to
 * finish first (hipDeviceSynchronize). Must not overlap other calls on the same handle. No counterpart in the
 * reference. */
int32_t goi_model_release_rows(GoiModel* model);

/* One b2World::Step (step.py:28-47) of every world in place. dt in seconds. debug may be NULL. */
int32_t goi_step(const GoiModel* model, const GoiStateView* state, const GoiSettings* settings, float dt,
                 void* hip_stream, const GoiDebug* debug);

/* n_steps consecutive b2World::Steps of every world in one launch, the same as n_steps goi_step calls with the
 * State's joint motor commands and forces left as they are between them (bit for bit). No counterpart in the
 * reference's step(): it is the loop a caller runs for several physics sub-steps per action (the game's K physics
 * sub-steps per environment step, goi_jax/box2d/gpu/graph.py:8). Each block keeps its worlds' workspaces in LDS
 * across the sub-steps and never waits for other blocks. debug (may be NULL) receives the last sub-step's values.
 * n_steps = 0 does nothing. */
int32_t goi_step_n(const GoiModel* model, const GoiStateView* state, const GoiSettings* settings, float dt,
                   int32_t n_steps, void* hip_stream, const GoiDebug* debug);

/* goi_step_n without any allocation: the same launches and results (bit for bit), with the constraint and task rows
 * in a static device array of the library (2^25 words = 128 MiB per device, held until the process ends) instead of
 * the handle's per-stream buffers. No counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). It calls no hipMalloc,
 * hipFree or allocating library routine. A batch needing more than the maximum, (C * 54 + J * 57) * (pitch + 64)
 * words (about 14,300 worlds of the 4-body rig with its 40 slots, so the 16,384-world benchmark batch is refused),
 * returns GOI_E_UNSUPPORTED before anything is launched. Every call on a device
 * shares that device's array: calls that overlap on one device (on different streams, or from different threads)
 * race and must not be made. */
int32_t goi_step_n_noalloc(const GoiModel* model, const GoiStateView* state, const GoiSettings* settings, float dt,
                           int32_t n_steps, void* hip_stream, const GoiDebug* debug);

/* Broadphase and narrowphase only (the collide-only workload): start-of-step FindNewContacts where new_fixture
 * (step.py:50-70), then Collide (pairs.py:38-87). */
int32_t goi_collide(const GoiModel* model, const GoiStateView* state, const GoiSettings* settings,
                    void* hip_stream);

/* b2WorldManifold::Initialize of every contact slot of every world (Box2D 2.3.1; the solver computes the same
 * in prepare, contact_solver.py:60-104), from the bodies' transforms: normal [C,2], points [C,2,2] and separations
 * [C,2], device buffers laid out worlds-minor with the view's pitch; zeros for free slots, slots without points and
 * points past a manifold's count. The counterpart of the reference oracle's contact readers for debugging and
 * parity dumps (goi_jax/reference/capi.cpp:786-838). */
int32_t goi_world_manifold(const GoiModel* model, const GoiStateView* state, float* normal, float* points,
                           float* separations, void* hip_stream);

/* The action-driven motor: writes every world's action a = (a_x, a_y) into joint `joint` of the
 * State's joint leaves, motor_speed = speed_gain * a_x and max_motor = torque_gain * |a| (float32, |a| by IEEE
 * square root). actions: device [n_worlds, 2] contiguous; motor_speed, max_motor: the State's joints.motor_speed and
 * joints.max_motor leaves (worlds-minor, element (j, w) at [j * pitch + w]). One launch for what a caller of the
 * reference does by writing State.joints.motor_speed / max_motor before each step (goi_jax/box2d/world.py:105-107,
 * used by joints.py:308-316); the mapping itself is this build's, the reference leaves it to its caller
 * (README.md:22-24). Returns GOI_E_ARG for n_worlds < 0, pitch < n_worlds, joint < 0 or a null pointer. */
int32_t goi_apply_motor_actions(const float* actions, float* motor_speed, float* max_motor, int32_t n_worlds,
                                int32_t pitch, int32_t joint, float speed_gain, float torque_gain, void* hip_stream);

/* Correctly rounded float32 sin/cos of n values on the device, as the step computes them (math2d.py:291-310):
 * s[i] = (float)sin((double)x[i]), c[i] = (float)cos((double)x[i]). Device pointers. */
int32_t goi_sincos(const float* x, float* s, float* c, int32_t n, void* hip_stream);

/* The packed State layout for capacities B, C, J, R: words[l] (l = 0 .. GOI_NUM_LEAVES) = the 4-byte words per unit of
 * pitch before leaf l, each leaf taking its per-world bytes rounded up to a multiple of 4 (words[0] = 0, words[l + 1]
 * - words[l] = that rounding for leaf l, words[GOI_NUM_LEAVES] = the whole). A packed State's leaf l starts at byte
 * 4 * words[l] * pitch of one device buffer, with the pitch a multiple of 64. No counterpart in the reference (whose
 * State is a pytree of separate arrays): it describes this library's fast layout, for callers that allocate States.
 * Returns GOI_E_ARG for a negative capacity or a null `words`. */
int32_t goi_packed_layout(int32_t B, int32_t C, int32_t J, int32_t R, int32_t* words);

/* The shape of the calling thread's last launch of goi_step, goi_step_n, goi_step_n_noalloc or goi_collide: the
 * worlds each 64-lane wavefront stepped (GOI_WORLDS_PER_WAVE may ask for another count; the library lowers a request
 * whose workspaces do not fit a block's LDS), the blocks launched, the dynamic LDS of a block in bytes and the kernel
 * instance that ran. No counterpart in the reference: it is for tests and profiling. Returns GOI_E_ARG for a null
 * `out`; all zero before the thread's first launch. */
#define GOI_KERNEL_GENERIC 1 /* the step for any dimensions */
#define GOI_KERNEL_RIG 2     /* the step compiled for the 4-body rig (5 bodies, 40 slots, 3 joints, 4 rows) */
#define GOI_KERNEL_ISLAND 3  /* the step compiled for the rig with 12 boxes (17 bodies, 128 slots, 3 joints, 16 rows) */
#define GOI_KERNEL_COLLIDE 4 /* goi_collide's kernel */
typedef struct GoiLaunchInfo {
    int32_t worlds_per_wave;
    int32_t blocks;
    int32_t lds_bytes;
    int32_t kernel;
} GoiLaunchInfo;
int32_t goi_last_launch(GoiLaunchInfo* out);

/* Thread-local message of the last failed call ("" if none). */
const char* goi_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* GOI_B2_H */
