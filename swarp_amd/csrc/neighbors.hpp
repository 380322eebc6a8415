// neighbors.hpp -- padded radius-neighbour lists of one state and the COO radius graph.
#pragma once
#include "common.hpp"

namespace swarp {

// --------------------------------------------------------------- neighbour lists

template <typename T, int PA>
__global__ __launch_bounds__(64) void k_neighbors(const Cst<T> C, const T *pos, int32_t *idx,
                                                  int32_t *cnt, int32_t *tru)
{
    typedef typename MaskT<PA>::type M;
    constexpr int EPW = 64 / PA;
    __shared__ T lx[64], ly[64];
    const int lane = threadIdx.x, agent = lane % PA, base = lane - agent;
    const int env = blockIdx.x * EPW + lane / PA;
    const bool active = agent < C.A && env < C.E;
    const size_t i = active ? (size_t)env * C.A + agent : 0;
    const bool real = agent < C.A;
    const T px = real ? pos[2 * i] : (T)__builtin_nan(""), py = real ? pos[2 * i + 1] : (T)__builtin_nan("");
    lx[lane] = px;
    ly[lane] = py;
    __syncthreads();
    M cd;
    const M incl = scan_all<T, PA>(lx, ly, base, C.A, agent, px, py, C.t_nbr, C.t_nbr, cd);
    if (!active) return;
    M m = cap_list(incl, C.K);
    const int n = m_popc(m);
    int32_t *row = idx + i * C.K;
    for (int k = 0; k < C.K; ++k) {
        int v = 0;
        if (k < n) {
            v = m_ctz(m);
            m &= m - 1;
        }
        row[k] = v;
    }
    cnt[i] = n;
    if (tru) tru[i] = m_popc(incl);
}


template <typename T>
void launch_neighbors(int PA, const Cst<T> &C, const T *p, int32_t *idx, int32_t *cnt,
                      int32_t *tru, hipStream_t st)
{
    const dim3 grid((C.E + (64 / PA) - 1) / (64 / PA));
    switch (PA) {
    case 4: hipLaunchKernelGGL((k_neighbors<T, 4>), grid, dim3(64), 0, st, C, p, idx, cnt, tru); break;
    case 8: hipLaunchKernelGGL((k_neighbors<T, 8>), grid, dim3(64), 0, st, C, p, idx, cnt, tru); break;
    case 16: hipLaunchKernelGGL((k_neighbors<T, 16>), grid, dim3(64), 0, st, C, p, idx, cnt, tru); break;
    case 32: hipLaunchKernelGGL((k_neighbors<T, 32>), grid, dim3(64), 0, st, C, p, idx, cnt, tru); break;
    default: hipLaunchKernelGGL((k_neighbors<T, 64>), grid, dim3(64), 0, st, C, p, idx, cnt, tru); break;
    }
}

void launch_edge_index(int E, int A, int K, const int32_t *idx, const int32_t *cnt,
                       const int64_t *off, int64_t n_edges, int64_t *out, hipStream_t st);

#ifdef SWARP_EDGE_INDEX_IMPL
__global__ void k_edge_index(int E, int A, int K, const int32_t *idx, const int32_t *cnt,
                             const int64_t *off, int64_t n_edges, int64_t *out)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)E * A) return;
    const int64_t e = (int64_t)(i / A);
    const int64_t n = cnt[i];
    const int64_t o = off[i];
    for (int64_t s = 0; s < n && o + s < n_edges; ++s) {
        out[o + s] = e * A + idx[i * K + s];
        out[n_edges + o + s] = (int64_t)i;
    }
}

void launch_edge_index(int E, int A, int K, const int32_t *idx, const int32_t *cnt,
                       const int64_t *off, int64_t n_edges, int64_t *out, hipStream_t st)
{
    const size_t n = (size_t)E * A;
    hipLaunchKernelGGL(k_edge_index, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, E, A,
                       K, idx, cnt, off, n_edges, out);
}
#endif

}  // namespace swarp
