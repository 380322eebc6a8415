// k_wbodies.hip -- instantiates the movable-body rollout kernels of envs of more than 64
// agents (and of grid-ordered lists) for the scalar type SWARP_T.
#include "wide_bodies.hpp"

namespace swarp {
template void launch_wbody_fwd<SWARP_T>(bool, const Cst<SWARP_T> &, const Args<SWARP_T> &,
                                        const ObTab<SWARP_T> &, const ObIO<SWARP_T> &,
                                        hipStream_t);
template void launch_wbody_bwd<SWARP_T>(bool, const Cst<SWARP_T> &, const Args<SWARP_T> &,
                                        const ObTab<SWARP_T> &, const ObIO<SWARP_T> &,
                                        hipStream_t);
}  // namespace swarp
