// goi_b2_rig.hip - the step of the 4-body rig (5 bodies, 40 contact slots, 3 joints, 4 fixture rows, 8 worlds per
// wave) on packed States, compiled for those dimensions (b2_fixed.hpp).
#define GOI_PACKED_STATE 1
#include "b2_fixed.hpp"

namespace goi {

hipError_t launch_rig_step(const DModel& d, const Launch& L, bool multi, bool plain, dim3 grid, size_t lds,
                           hipStream_t st) {
    const dim3 b(kBlock);
    if (!multi && plain)
        hipLaunchKernelGGL((k_step_fixed<kRigB, kRigC, kRigJ, kRigR, kRigS, false, true, false>), grid, b, lds, st, d, L);
    else if (!multi)
        hipLaunchKernelGGL((k_step_fixed<kRigB, kRigC, kRigJ, kRigR, kRigS, false, false, false>), grid, b, lds, st, d, L);
    else if (plain)
        hipLaunchKernelGGL((k_step_fixed<kRigB, kRigC, kRigJ, kRigR, kRigS, true, true, false>), grid, b, lds, st, d, L);
    else
        hipLaunchKernelGGL((k_step_fixed<kRigB, kRigC, kRigJ, kRigR, kRigS, true, false, false>), grid, b, lds, st, d, L);
    return hipGetLastError();
}

}  // namespace goi
