// k_drone.hip -- instantiates the generic rollout kernels with (DRONE, BOXES) = (true, false)
// for the scalar type SWARP_T (the build compiles this unit once per dtype).
#include "generic.hpp"

namespace swarp {
template void launch_fwd<SWARP_T, true, false>(int, const Cst<SWARP_T> &, const Args<SWARP_T> &,
                                         unsigned, hipStream_t);
template void launch_bwd<SWARP_T, true, false>(int, const Cst<SWARP_T> &, const Args<SWARP_T> &,
                                         unsigned, size_t, hipStream_t);
}  // namespace swarp
