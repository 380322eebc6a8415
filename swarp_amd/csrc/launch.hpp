// launch.hpp -- the kernel launchers each family unit (k_*.hip) instantiates, declared
// `extern` for the host unit (swarp_hip.hip) so that it compiles no kernel itself.
#pragma once
#include "generic.hpp"
#include "lean.hpp"
#include "bodies.hpp"
#include "nav.hpp"
#include "neighbors.hpp"
#include "wide.hpp"
#include "wide_bodies.hpp"

#define SWARP_EXTERN_LAUNCHERS(T)                                                            \
    extern template void launch_fwd<T, false, false>(int, const Cst<T> &, const Args<T> &,   \
                                                     unsigned, hipStream_t);                 \
    extern template void launch_fwd<T, true, false>(int, const Cst<T> &, const Args<T> &,    \
                                                    unsigned, hipStream_t);                  \
    extern template void launch_fwd<T, false, true>(int, const Cst<T> &, const Args<T> &,    \
                                                    unsigned, hipStream_t);                  \
    extern template void launch_bwd<T, false, false>(int, const Cst<T> &, const Args<T> &,   \
                                                     unsigned, size_t, hipStream_t);         \
    extern template void launch_bwd<T, true, false>(int, const Cst<T> &, const Args<T> &,    \
                                                    unsigned, size_t, hipStream_t);          \
    extern template void launch_bwd<T, false, true>(int, const Cst<T> &, const Args<T> &,    \
                                                    unsigned, size_t, hipStream_t);          \
    extern template void launch_holo_fwd<T, true>(int, const Cst<T> &, const Args<T> &,      \
                                                  const Tape<T> &, hipStream_t);             \
    extern template void launch_holo_fwd<T, false>(int, const Cst<T> &, const Args<T> &,     \
                                                   const Tape<T> &, hipStream_t);            \
    extern template void launch_holo_bwd<T, true>(int, const Cst<T> &, const Args<T> &,      \
                                                  const Tape<T> &, size_t, hipStream_t);     \
    extern template void launch_holo_bwd<T, false>(int, const Cst<T> &, const Args<T> &,     \
                                                   const Tape<T> &, size_t, hipStream_t);    \
    extern template void launch_body_fwd<T>(int, const Cst<T> &, const Args<T> &,            \
                                            const ObTab<T> &, const ObIO<T> &, unsigned,     \
                                            bool, hipStream_t);                              \
    extern template void launch_body_bwd<T>(int, const Cst<T> &, const Args<T> &,            \
                                            const ObTab<T> &, const ObIO<T> &, unsigned,     \
                                            bool, size_t, hipStream_t);                      \
    extern template size_t body_bwd_lds_of<T>(int, int, int, bool, bool);                    \
    extern template void launch_nav<T>(int, const Cst<T> &, const NavArgs<T> &, unsigned,    \
                                       hipStream_t);                                         \
    extern template void launch_neighbors<T>(int, const Cst<T> &, const T *, int32_t *,      \
                                             int32_t *, int32_t *, hipStream_t);             \
    extern template void launch_wide_lists<T>(const Cst<T> &, const T *, const T *, int32_t *,\
                                              int32_t *, int32_t *, hipStream_t);            \
    extern template void launch_grid_frame<T>(const T *, int64_t, T, int, T *, hipStream_t);  \
    extern template void launch_wide_fwd_apt<T, 1>(bool, bool, const Cst<T> &, const Args<T> &, \
                                                   hipStream_t);                             \
    extern template void launch_wide_fwd_apt<T, 2>(bool, bool, const Cst<T> &, const Args<T> &, \
                                                   hipStream_t);                             \
    extern template void launch_wide_fwd_apt<T, 4>(bool, bool, const Cst<T> &, const Args<T> &, \
                                                   hipStream_t);                             \
    extern template void launch_wide_bwd_apt<T, 1>(bool, bool, const Cst<T> &, const Args<T> &, \
                                                   hipStream_t);                             \
    extern template void launch_wide_bwd_apt<T, 2>(bool, bool, const Cst<T> &, const Args<T> &, \
                                                   hipStream_t);                             \
    extern template void launch_wide_bwd_apt<T, 4>(bool, bool, const Cst<T> &, const Args<T> &, \
                                                   hipStream_t);                             \
    extern template void launch_wbody_fwd<T>(bool, const Cst<T> &, const Args<T> &,           \
                                             const ObTab<T> &, const ObIO<T> &, hipStream_t); \
    extern template void launch_wbody_bwd<T>(bool, const Cst<T> &, const Args<T> &,           \
                                             const ObTab<T> &, const ObIO<T> &, hipStream_t);

namespace swarp {
SWARP_EXTERN_LAUNCHERS(float)
SWARP_EXTERN_LAUNCHERS(double)
}  // namespace swarp
