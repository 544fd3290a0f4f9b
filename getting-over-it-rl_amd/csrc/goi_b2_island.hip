// goi_b2_island.hip - the step of the rig with 12 boxes (17 bodies, 128 contact slots, 3 joints, 16 fixture rows, 4
// worlds per wave) on packed States with a plain Model (revolute joints only, no edge shapes), compiled for those
// dimensions (b2_fixed.hpp).
#define GOI_PACKED_STATE 1
#include "b2_fixed.hpp"

namespace goi {

hipError_t launch_island_step(const DModel& d, const Launch& L, bool multi, dim3 grid, size_t lds, hipStream_t st) {
    const dim3 b(kBlock);
    if (!multi)
        hipLaunchKernelGGL((k_step_fixed<kIslandB, kIslandC, kIslandJ, kIslandR, kIslandS, false, true, true>), grid, b, lds,
                           st, d, L);
    else
        hipLaunchKernelGGL((k_step_fixed<kIslandB, kIslandC, kIslandJ, kIslandR, kIslandS, true, true, true>), grid, b, lds,
                           st, d, L);
    return hipGetLastError();
}

}  // namespace goi
