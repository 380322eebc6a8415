// k_nav.hip -- instantiates the fused navigation pass and the neighbour-list kernel for the
// scalar type SWARP_T; the float unit also defines the COO edge kernel's launcher.
#if SWARP_T_IS_F32
#define SWARP_EDGE_INDEX_IMPL 1
#endif
#include "nav.hpp"
#include "neighbors.hpp"

namespace swarp {
template void launch_nav<SWARP_T>(int, const Cst<SWARP_T> &, const NavArgs<SWARP_T> &, unsigned,
                                  hipStream_t);
template void launch_neighbors<SWARP_T>(int, const Cst<SWARP_T> &, const SWARP_T *, int32_t *,
                                        int32_t *, int32_t *, hipStream_t);
}  // namespace swarp
