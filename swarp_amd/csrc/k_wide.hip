// k_wide.hip -- instantiates the wide-env kernels (envs of up to 1024 agents, uniform-grid
// list order) for the scalar type SWARP_T.
#include "wide.hpp"

namespace swarp {
template void launch_wide_lists<SWARP_T>(const Cst<SWARP_T> &, const SWARP_T *, const SWARP_T *,
                                         int32_t *, int32_t *, int32_t *, hipStream_t);
template void launch_grid_frame<SWARP_T>(const SWARP_T *, int64_t, SWARP_T, int, SWARP_T *,
                                         hipStream_t);
template void launch_wide_fwd<SWARP_T>(bool, bool, const Cst<SWARP_T> &, const Args<SWARP_T> &,
                                       hipStream_t);
template void launch_wide_bwd<SWARP_T>(bool, bool, const Cst<SWARP_T> &, const Args<SWARP_T> &,
                                       hipStream_t);
}  // namespace swarp
