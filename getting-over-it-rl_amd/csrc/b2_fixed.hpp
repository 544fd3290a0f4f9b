// b2_fixed.hpp - the step with the world dimensions and the worlds per wave fixed at compile time, for a translation
// unit that defines GOI_PACKED_STATE 1 (World and BlockCopy then address every State leaf from leaf 0's base at the
// leaf's constant packed offset, so the kernel holds one base pointer where the general step holds 71).
#pragma once

#if !GOI_PACKED_STATE
#error "b2_fixed.hpp: define GOI_PACKED_STATE 1 before including it"
#endif
#include "b2_launch.hpp"

namespace goi {
namespace {

// Every workspace offset, loop bound and leaf offset folds into the instructions, which frees the scalar registers
// the runtime dimensions and the 71 leaf pointers would hold (spilled scalars come back through v_readlane on every
// use). kPlain: revolute joints only (the v2.4.1 solver) and no edge shapes, so the other joint and collider code
// drops out. Launches with debug arrays take k_step, so the debug writes drop out too. kIslands: worlds of several
// islands solve them on separate lanes of the group (DModel::island_lanes); without it that path drops out, for
// models whose bodies are joined into one island (the rig). The results are those of k_step.
template <int kB, int kC, int kJ, int kR, int kS, bool kMulti, bool kPlain, bool kIslands>
__global__ void __launch_bounds__(kBlock, 2) k_step_fixed(DModel m, Launch L) {
    L.B = kB; L.C = kC; L.J = kJ; L.R = kR; L.wpw = kS;
    if (!kIslands) m.island_lanes = 0;
    L.full_rows = 0;  // the launch takes these instances for compact packed States only
    L.dbg = GoiDebug{};
    m.B = kB; m.J = kJ; m.R = kR;
    if (kPlain) {
        m.rev_only = 1;
        m.no_edges = 1;
        L.s.revolute_v24 = 1;
    }
    step_block<kMulti, (kC > 64)>(m, L);  // the island instance (128 slots) re-derives its SolveTOI views
}

}  // namespace
}  // namespace goi
