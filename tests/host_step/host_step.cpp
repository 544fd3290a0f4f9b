// host_step.cpp - steps a batch of worlds through the library's step compiled for the host (GOI_HOST_BUILD: the
// kernels run their blocks and lanes one after another on heap memory of exactly the requested sizes) and through
// the oracle, side by side, and compares every State leaf bit for bit after every launch. Built with AddressSanitizer
// and UBSan (Makefile beside this file), so an out-of-bounds access or undefined operation in the step's code stops
// the run at its source line, which a fault on the device does not give.
//
// Usage: host_step <scenario file> <mode> [plant], mode "step" (goi_step), "step_n:K" (goi_step_n, K steps a
// launch) or "noalloc:K" (goi_step_n_noalloc); "plant" moves the last world's first body by one ulp in the oracle's
// copy only, so that run must end in a mismatch. The scenario file (written by tests/test_host_sanitized.py,
// little-endian):
//   "GOISCN02", int32 F J P B, then the 24 GoiModelDesc arrays in declaration order, each an int64 byte count
//   (-1 = NULL) and the bytes; int32 sizeof(GoiSettings) and the struct; float dt; int32 n_steps, n, B R J C,
//   contact_capacity, packed, n_leaves; per leaf: int32 name length, name, int32 element size, int64 elements per
//   world, int32 kind (1 float, 0 integer or bool), n * that many elements batch-major; int32 motor joint (-1: no actions), float speed gain, torque gain,
//   then n_steps * n * 2 float actions.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "../../include/goi_b2.h"

extern "C" int oracle_step(const GoiModelDesc* m, void* const* leaves, int32_t n, int32_t B, int32_t C, int32_t R,
                           int32_t J, const GoiSettings* s, float dt, int32_t n_threads, GoiDebug* dbg);

namespace {

[[noreturn]] void die(const std::string& msg) {
    std::fprintf(stderr, "host_step: %s\n", msg.c_str());
    std::exit(2);
}

// Owns every buffer; each is a separate heap block of exactly its size, so the sanitizer bounds each one.
std::vector<std::unique_ptr<uint8_t[]>> g_keep;

uint8_t* block(size_t n) {
    g_keep.emplace_back(new uint8_t[n]);
    return g_keep.back().get();
}

struct Reader {
    FILE* f;
    void raw(void* p, size_t n) {
        if (n && std::fread(p, 1, n, f) != n) die("scenario file truncated");
    }
    template <typename T> T get() {
        T v;
        raw(&v, sizeof(T));
        return v;
    }
    const void* array() {  // an int64 byte count (-1 = NULL), then the bytes
        const int64_t n = get<int64_t>();
        if (n < 0) return nullptr;
        uint8_t* p = block((size_t)n);
        raw(p, (size_t)n);
        return p;
    }
};

struct Leaf {
    std::string name;
    int esize;
    int64_t per_world;
    bool is_float;
    uint8_t* ref;  // the oracle's copy, batch-major [n][per_world]
    uint8_t* dev;  // the library's copy, worlds-minor [per_world][pitch]
};

}  // namespace

int main(int argc, char** argv) {
    if (argc != 3 && !(argc == 4 && std::strcmp(argv[3], "plant") == 0))
        die("usage: host_step <scenario> <step | step_n:K | noalloc:K> [plant]");
    const std::string mode = argv[2];
    const bool plant = argc == 4;  // nudge the oracle's input by one ulp: the run must then report a mismatch
    int per_launch = 1;
    bool noalloc = false, step_n = false;
    if (mode.rfind("step_n:", 0) == 0) {
        step_n = true;
        per_launch = std::atoi(mode.c_str() + 7);
    } else if (mode.rfind("noalloc:", 0) == 0) {
        noalloc = true;
        per_launch = std::atoi(mode.c_str() + 8);
    } else if (mode != "step") {
        die("unknown mode " + mode);
    }
    if (per_launch < 1) die("steps per launch must be positive");

    Reader r{std::fopen(argv[1], "rb")};
    if (!r.f) die(std::string("cannot open ") + argv[1]);
    char magic[8];
    r.raw(magic, 8);
    if (std::memcmp(magic, "GOISCN02", 8) != 0) die("not a scenario file");

    GoiModelDesc d{};
    d.F = r.get<int32_t>();
    d.J = r.get<int32_t>();
    d.P = r.get<int32_t>();
    d.B = r.get<int32_t>();
    d.fixture_body = (const int32_t*)r.array();
    d.shape_type = (const int32_t*)r.array();
    d.radius = (const float*)r.array();
    d.count = (const int32_t*)r.array();
    d.verts = (const float*)r.array();
    d.normals = (const float*)r.array();
    d.joint_type = (const int32_t*)r.array();
    d.joint_a = (const int32_t*)r.array();
    d.joint_b = (const int32_t*)r.array();
    d.local_anchor_a = (const float*)r.array();
    d.local_anchor_b = (const float*)r.array();
    d.local_axis_a = (const float*)r.array();
    d.local_yaxis_a = (const float*)r.array();
    d.reference_angle = (const float*)r.array();
    d.pair_a = (const int32_t*)r.array();
    d.pair_b = (const int32_t*)r.array();
    d.fixture_slot = (const int32_t*)r.array();
    d.static_fat = (const float*)r.array();
    d.static_friction = (const float*)r.array();
    d.static_restitution = (const float*)r.array();
    d.body_type = (const int32_t*)r.array();
    d.toi_bodies = (const uint8_t*)r.array();
    d.centroid = (const float*)r.array();
    d.edge_flags = (const int32_t*)r.array();

    if (r.get<int32_t>() != (int32_t)sizeof(GoiSettings)) die("GoiSettings size differs from the writer's");
    const GoiSettings s = r.get<GoiSettings>();
    const float dt = r.get<float>();
    const int n_steps = r.get<int32_t>();
    const int n = r.get<int32_t>();
    const int B = r.get<int32_t>(), R = r.get<int32_t>(), J = r.get<int32_t>(), C = r.get<int32_t>();
    const int capacity = r.get<int32_t>();
    const bool packed = r.get<int32_t>() != 0;
    const int n_leaves = r.get<int32_t>();
    if (n_leaves != GOI_NUM_LEAVES) die("leaf count differs from GOI_NUM_LEAVES");
    if (n < 1 || n_steps < 1) die("empty scenario");

    // packed: one buffer, leaf l at words[l] * pitch words with a pitch a multiple of 64 (the layout the library
    // recognises); otherwise one exactly-sized buffer per leaf with pitch n
    const int pitch = packed ? (n + 63) / 64 * 64 : n;
    int32_t words[GOI_NUM_LEAVES + 1];
    if (goi_packed_layout(B, C, J, R, words) != GOI_OK) die(std::string("goi_packed_layout: ") + goi_last_error());
    const size_t packed_bytes = packed ? (size_t)words[GOI_NUM_LEAVES] * pitch * 4 : 0;
    uint8_t* base = packed ? block(packed_bytes) : nullptr;
    if (packed) std::memset(base, 0, packed_bytes);  // the padding between leaves and past world n
    std::vector<Leaf> leaves(n_leaves);
    for (int l = 0; l < n_leaves; ++l) {
        Leaf& L = leaves[l];
        L.name.resize(r.get<int32_t>());
        r.raw(&L.name[0], L.name.size());
        L.esize = r.get<int32_t>();
        L.per_world = r.get<int64_t>();
        L.is_float = r.get<int32_t>() == 1;
        const size_t bytes = (size_t)n * L.per_world * L.esize;
        L.ref = block(bytes);
        r.raw(L.ref, bytes);
        L.dev = packed ? base + (size_t)words[l] * pitch * 4 : block((size_t)L.per_world * pitch * L.esize);
        for (int w = 0; w < n; ++w)
            for (int64_t i = 0; i < L.per_world; ++i)
                std::memcpy(L.dev + ((size_t)i * pitch + w) * L.esize, L.ref + ((size_t)w * L.per_world + i) * L.esize,
                            L.esize);
    }
    const int motor = r.get<int32_t>();
    const float speed_gain = r.get<float>(), torque_gain = r.get<float>();
    float* actions = nullptr;
    if (motor >= 0) {
        actions = (float*)block((size_t)n_steps * n * 2 * sizeof(float));
        r.raw(actions, (size_t)n_steps * n * 2 * sizeof(float));
    }
    std::fclose(r.f);

    auto leaf_index = [&](const char* name) {
        for (int l = 0; l < n_leaves; ++l)
            if (leaves[l].name == name) return l;
        die(std::string("no leaf ") + name);
    };
    const int l_speed = leaf_index("joints.motor_speed"), l_torque = leaf_index("joints.max_motor");
    if (plant) {
        const Leaf& L = leaves[leaf_index("bodies.c")];
        float* c = (float*)L.ref + (size_t)(n - 1) * L.per_world;
        c[0] = std::nextafter(c[0], INFINITY);
    }

    GoiModel* model = nullptr;
    if (goi_model_create(&d, capacity, nullptr, &model) != GOI_OK)
        die(std::string("goi_model_create: ") + goi_last_error());
    GoiStateView view{};
    view.n_worlds = n;
    view.pitch = pitch;
    view.B = B;
    view.C = C;
    view.R = R;
    view.J = J;
    std::vector<void*> ref_leaves(n_leaves);
    for (int l = 0; l < n_leaves; ++l) {
        view.leaf[l] = leaves[l].dev;
        ref_leaves[l] = leaves[l].ref;
    }

    long compared = 0;
    for (int k0 = 0; k0 < n_steps; k0 += per_launch) {
        const int k1 = std::min(n_steps, k0 + per_launch);
        if (actions && k1 - k0 != 1) die("actions need one step per launch");
        if (actions) {
            // the device side through the library's action kernel, the oracle side with the same float32 operations
            const float* a = actions + (size_t)k0 * n * 2;
            if (goi_apply_motor_actions(a, (float*)leaves[l_speed].dev, (float*)leaves[l_torque].dev, n, pitch, motor,
                                        speed_gain, torque_gain, nullptr) != GOI_OK)
                die(std::string("goi_apply_motor_actions: ") + goi_last_error());
            float* sp = (float*)leaves[l_speed].ref;
            float* tq = (float*)leaves[l_torque].ref;
            for (int w = 0; w < n; ++w) {
                const float ax = a[2 * w], ay = a[2 * w + 1];
                sp[(size_t)w * J + motor] = speed_gain * ax;
                tq[(size_t)w * J + motor] = torque_gain * std::sqrt(ax * ax + ay * ay);
            }
        }
        int rc;
        if (noalloc)
            rc = goi_step_n_noalloc(model, &view, &s, dt, k1 - k0, nullptr, nullptr);
        else if (step_n)
            rc = goi_step_n(model, &view, &s, dt, k1 - k0, nullptr, nullptr);
        else
            rc = goi_step(model, &view, &s, dt, nullptr, nullptr);
        if (rc != GOI_OK) die(std::string("step: ") + goi_last_error());
        for (int k = k0; k < k1; ++k)
            if (oracle_step(&d, ref_leaves.data(), n, B, C, R, J, &s, dt, 1, nullptr) != 0) die("oracle_step failed");
        for (const Leaf& L : leaves)
            for (int w = 0; w < n; ++w)
                for (int64_t i = 0; i < L.per_world; ++i) {
                    const uint8_t* a = L.ref + ((size_t)w * L.per_world + i) * L.esize;
                    const uint8_t* b = L.dev + ((size_t)i * pitch + w) * L.esize;
                    // float elements compare bit for bit, except that any two NaNs are equal: a NaN's sign and
                    // payload follow the operand order of the operations that made it, which neither IEEE 754 nor
                    // the reference fixes
                    float fa = 0.0f, fb = 0.0f;
                    if (L.is_float) {
                        std::memcpy(&fa, a, 4);
                        std::memcpy(&fb, b, 4);
                    }
                    if (std::memcmp(a, b, L.esize) != 0 && !(L.is_float && std::isnan(fa) && std::isnan(fb))) {
                        uint32_t ua = 0, ub = 0;
                        std::memcpy(&ua, a, L.esize);
                        std::memcpy(&ub, b, L.esize);
                        std::printf("MISMATCH after step %d: leaf %s world %d element %lld (oracle 0x%08x, step 0x%08x)\n",
                                    k1, L.name.c_str(), w, (long long)i, ua, ub);
                        std::fflush(stdout);
                        goi_model_destroy(model);
                        return 1;
                    }
                    ++compared;
                }
        std::printf("step %d equal\n", k1);
        std::fflush(stdout);
    }
    goi_model_destroy(model);
    // the regime the run reached: contacts dropped by full tables (overflow) and TOI events of the last step
    long overflow = 0, events = 0;
    const int32_t* ovf = (const int32_t*)leaves[leaf_index("overflow")].ref;
    const int32_t* ev = (const int32_t*)leaves[leaf_index("toi.events")].ref;
    for (int w = 0; w < n; ++w) {
        overflow += ovf[w];
        events += ev[w];
    }
    std::printf("overflow %ld events %ld\n", overflow, events);
    std::printf("PASS %d worlds, %d steps, %ld elements compared (%s, %s State)\n", n, n_steps, compared, mode.c_str(),
                packed ? "packed" : "one buffer per leaf");
    return 0;
}
