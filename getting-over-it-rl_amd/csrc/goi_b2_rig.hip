// goi_b2_rig.hip - the step of the 4-body rig (5 bodies, 40 contact slots, 3 joints, 4 fixture rows, 8 worlds per
// wave) on packed States: World and BlockCopy address every State leaf from leaf 0's base at the leaf's constant
// packed offset (GOI_PACKED_STATE), so the kernel holds one base pointer where the general step holds 71.
#define GOI_PACKED_STATE 1
#include "b2_launch.hpp"

namespace goi {
namespace {

// The same step with the world dimensions and the worlds per wave fixed at compile time (the 4-body rig with 40
// contact slots, 8 worlds per wave) on a packed State: every workspace offset, loop bound and leaf offset folds into
// the instructions, which frees the scalar registers the runtime dimensions and the 71 leaf pointers would hold
// (spilled scalars come back through v_readlane on every use). The results are those of k_step.
template <int kB, int kC, int kJ, int kR, int kS, bool kMulti, bool kPlain>
__global__ void __launch_bounds__(kBlock, 2) k_step_fixed(DModel m, Launch L) {
    L.B = kB; L.C = kC; L.J = kJ; L.R = kR; L.wpw = kS;
    m.B = kB; m.J = kJ; m.R = kR;
    if (kPlain) {  // revolute joints only (the v2.4.1 solver), no edge shapes: the other joint and collider code drops out
        m.rev_only = 1;
        m.no_edges = 1;
        L.s.revolute_v24 = 1;
    }
    step_block<kMulti>(m, L);
}

}  // namespace

hipError_t launch_rig_step(const DModel& d, const Launch& L, bool multi, bool plain, dim3 grid, size_t lds,
                           hipStream_t st) {
    const dim3 b(kBlock);
    if (!multi && plain)
        hipLaunchKernelGGL((k_step_fixed<kRigB, kRigC, kRigJ, kRigR, kRigS, false, true>), grid, b, lds, st, d, L);
    else if (!multi)
        hipLaunchKernelGGL((k_step_fixed<kRigB, kRigC, kRigJ, kRigR, kRigS, false, false>), grid, b, lds, st, d, L);
    else if (plain)
        hipLaunchKernelGGL((k_step_fixed<kRigB, kRigC, kRigJ, kRigR, kRigS, true, true>), grid, b, lds, st, d, L);
    else
        hipLaunchKernelGGL((k_step_fixed<kRigB, kRigC, kRigJ, kRigR, kRigS, true, false>), grid, b, lds, st, d, L);
    return hipGetLastError();
}

}  // namespace goi
