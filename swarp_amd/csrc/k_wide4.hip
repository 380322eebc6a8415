// k_wide4.hip -- instantiates the wide-env rollout kernels with 4 agents per thread (envs
// of more than 2048 agents) for the scalar type SWARP_T.
#include "wide.hpp"

namespace swarp {
template void launch_wide_fwd_apt<SWARP_T, 4>(bool, bool, const Cst<SWARP_T> &,
                                              const Args<SWARP_T> &, hipStream_t);
template void launch_wide_bwd_apt<SWARP_T, 4>(bool, bool, const Cst<SWARP_T> &,
                                              const Args<SWARP_T> &, hipStream_t);
}  // namespace swarp
