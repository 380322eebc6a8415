// k_bodies.hip -- instantiates the movable-body rollout kernels for the scalar type SWARP_T.
#include "bodies.hpp"

namespace swarp {
template void launch_body_fwd<SWARP_T>(int, const Cst<SWARP_T> &, const Args<SWARP_T> &,
                                       const ObTab<SWARP_T> &, const ObIO<SWARP_T> &, unsigned,
                                       hipStream_t);
template void launch_body_bwd<SWARP_T>(int, const Cst<SWARP_T> &, const Args<SWARP_T> &,
                                       const ObTab<SWARP_T> &, const ObIO<SWARP_T> &, unsigned,
                                       size_t, hipStream_t);
}  // namespace swarp
