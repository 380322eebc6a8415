// k_bodies.hip -- instantiates the movable-body rollout kernels for the scalar type SWARP_T.
#include "bodies.hpp"

namespace swarp {
template void launch_body_fwd<SWARP_T>(int, const Cst<SWARP_T> &, const Args<SWARP_T> &,
                                       const ObTab<SWARP_T> &, const ObIO<SWARP_T> &, unsigned,
                                       bool, hipStream_t);
template void launch_body_bwd<SWARP_T>(int, const Cst<SWARP_T> &, const Args<SWARP_T> &,
                                       const ObTab<SWARP_T> &, const ObIO<SWARP_T> &, unsigned,
                                       bool, size_t, hipStream_t);
template size_t body_bwd_lds_of<SWARP_T>(int, int, int, bool, bool);
}  // namespace swarp
