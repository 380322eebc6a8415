// k_holo.hip -- instantiates the specialised holonomic rollout kernels (with and without
// the rollout tape) for the scalar type SWARP_T.
#include "lean.hpp"

namespace swarp {
template void launch_holo_fwd<SWARP_T, true>(int, const Cst<SWARP_T> &, const Args<SWARP_T> &,
                                             const Tape<SWARP_T> &, hipStream_t);
template void launch_holo_fwd<SWARP_T, false>(int, const Cst<SWARP_T> &, const Args<SWARP_T> &,
                                              const Tape<SWARP_T> &, hipStream_t);
template void launch_holo_bwd<SWARP_T, true>(int, const Cst<SWARP_T> &, const Args<SWARP_T> &,
                                             const Tape<SWARP_T> &, size_t, hipStream_t);
template void launch_holo_bwd<SWARP_T, false>(int, const Cst<SWARP_T> &, const Args<SWARP_T> &,
                                              const Tape<SWARP_T> &, size_t, hipStream_t);
}  // namespace swarp
