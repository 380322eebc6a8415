// k_wide2.hip -- instantiates the wide-env rollout kernels with 2 agents per thread (envs
// of more than 1024 agents) for the scalar type SWARP_T.
#include "wide.hpp"

namespace swarp {
template void launch_wide_fwd_apt<SWARP_T, 2>(bool, bool, const Cst<SWARP_T> &,
                                              const Args<SWARP_T> &, hipStream_t);
template void launch_wide_bwd_apt<SWARP_T, 2>(bool, bool, const Cst<SWARP_T> &,
                                              const Args<SWARP_T> &, hipStream_t);
}  // namespace swarp
