// neighbors.hpp -- padded radius-neighbour lists of one state and the COO radius graph.
#pragma once
#include "common.hpp"

namespace swarp {

// --------------------------------------------------------------- neighbour lists

// Padded lists of one state (NeighborGrid.query_into's brute-force order).  Each lane
// builds the K slots of its row; with STAGE the rows are staged in LDS in (env, agent)
// order -- the order of the output -- and the wave stores its envs' rows, one contiguous
// block of idx, with coalesced 16-byte stores (4-byte ones when the block is not 16-byte
// aligned) instead of K scattered 4-byte stores per lane.  STAGE = false (rows too long
// for the LDS) writes each row directly.
template <typename T, int PA, bool STAGE>
__global__ __launch_bounds__(64) void k_neighbors(const Cst<T> C, const T *pos, int32_t *idx,
                                                  int32_t *cnt, int32_t *tru)
{
    typedef typename MaskT<PA>::type M;
    constexpr int EPW = 64 / PA;
    __shared__ T lx[64], ly[64];
    extern __shared__ __align__(16) unsigned char smem[];
    int32_t *const srows = (int32_t *)smem;  // [EPW * A][K] (STAGE)
    const int lane = threadIdx.x, agent = lane % PA, base = lane - agent;
    const int e0 = blockIdx.x * EPW;
    const int env = e0 + lane / PA;
    const bool active = agent < C.A && env < C.E;
    const size_t i = active ? (size_t)env * C.A + agent : 0;
    const bool real = agent < C.A;
    const T px = real ? pos[2 * i] : (T)__builtin_nan(""), py = real ? pos[2 * i + 1] : (T)__builtin_nan("");
    lx[lane] = px;
    ly[lane] = py;
    __syncthreads();
    M cd;
    const M incl = scan_all<T, PA>(lx, ly, base, C.A, agent, px, py, C.t_nbr, C.t_nbr, cd);
    M m = cap_list(incl, C.K);
    const int n = m_popc(m);
    int32_t *row = STAGE ? srows + ((size_t)(lane / PA) * C.A + agent) * C.K : idx + i * C.K;
    if (active) {
        int k = 0;
        if (STAGE && (C.K & 3) == 0) {
            // 16-byte LDS writes: a row of K words at a stride of K words per lane puts
            // every lane's k-th word in the same few banks, and one 16-byte write per four
            // slots quarters the conflicting writes
            for (; k < C.K; k += 4) {
                int w[4];
                for (int u = 0; u < 4; ++u) {
                    w[u] = 0;
                    if (k + u < n) {
                        w[u] = m_ctz(m);
                        m &= m - 1;
                    }
                }
                *(int4 *)(row + k) = make_int4(w[0], w[1], w[2], w[3]);
            }
        }
        for (; k < C.K; ++k) {
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
    if (STAGE) {
        wave_lds_sync();  // the workgroup is this one wave
        const int ne = C.E - e0 < EPW ? C.E - e0 : EPW;
        const size_t nb = (size_t)ne * C.A * C.K;  // rows of the wave's active envs
        int32_t *dst = idx + (size_t)e0 * C.A * C.K;
        if (((uintptr_t)dst & 15u) == 0u && (nb & 3u) == 0u) {
            const int4 *s4 = (const int4 *)srows;
            int4 *d4 = (int4 *)dst;
            for (size_t q = lane; q < nb / 4; q += 64) d4[q] = s4[q];
        } else {
            for (size_t q = lane; q < nb; q += 64) dst[q] = srows[q];
        }
    }
}

// LDS bytes of the staged rows of one wave (0: rows too long to stage: with the kernel's
// static position arrays lx / ly, a workgroup's LDS stays within 64 KiB).
inline size_t neighbors_stage_bytes(int PA, int A, int K, size_t tsize)
{
    const size_t b = (size_t)(64 / PA) * A * K * sizeof(int32_t);
    return b + 2 * 64 * tsize <= 65536 ? b : 0;
}

template <typename T>
void launch_neighbors(int PA, const Cst<T> &C, const T *p, int32_t *idx, int32_t *cnt,
                      int32_t *tru, hipStream_t st)
{
    const dim3 grid((C.E + (64 / PA) - 1) / (64 / PA));
    const size_t shm = neighbors_stage_bytes(PA, C.A, C.K, sizeof(T));
#define SWARP_NBR(PA_)                                                                             \
    if (shm)                                                                                       \
        hipLaunchKernelGGL((k_neighbors<T, PA_, true>), grid, dim3(64), shm, st, C, p, idx, cnt, tru); \
    else                                                                                           \
        hipLaunchKernelGGL((k_neighbors<T, PA_, false>), grid, dim3(64), 0, st, C, p, idx, cnt, tru);
    switch (PA) {
    case 4: SWARP_NBR(4) break;
    case 8: SWARP_NBR(8) break;
    case 16: SWARP_NBR(16) break;
    case 32: SWARP_NBR(32) break;
    default: SWARP_NBR(64) break;
    }
#undef SWARP_NBR
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
