// k_wide.hip -- instantiates the wide-env list builder and grid frame (every wide env) and
// the rollout kernels with one agent per thread (envs of up to 1024 agents) for the scalar
// type SWARP_T.
#include "wide.hpp"

namespace swarp {
template void launch_wide_lists<SWARP_T>(const Cst<SWARP_T> &, const SWARP_T *, const SWARP_T *,
                                         int32_t *, int32_t *, int32_t *, hipStream_t);
template void launch_grid_frame<SWARP_T>(const SWARP_T *, int64_t, SWARP_T, int, SWARP_T *,
                                         hipStream_t);
template void launch_wide_fwd_apt<SWARP_T, 1>(bool, bool, const Cst<SWARP_T> &,
                                              const Args<SWARP_T> &, hipStream_t);
template void launch_wide_bwd_apt<SWARP_T, 1>(bool, bool, const Cst<SWARP_T> &,
                                              const Args<SWARP_T> &, hipStream_t);
}  // namespace swarp
