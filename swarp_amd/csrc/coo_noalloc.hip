// coo_noalloc.hip -- swarp_edge_index_noalloc: the COO radius graph of padded neighbour
// lists without any allocation, for callers that cannot allocate device memory (code
// under HIP graph capture, tight serving loops).
//
// swarp_edge_index takes the exclusive prefix sum of the list counts from the caller (a
// workspace the caller allocates and fills) and the edge count (a host value, so a host
// sync).  This variant computes the prefix sums itself, three launches on the caller's
// stream, with its per-block partial sums in the file-scope array `scratch` below, and
// reports the edge count on the device:
//   k_coo_block_sums  block b of 256 agents: the sum of its counts -> scratch[b]
//   k_coo_scan        one workgroup: exclusive scan of scratch[0 .. nb) in place, the
//                     total -> *n_edges
//   k_coo_write       block b: its agents' exclusive offsets (block-local scan in LDS
//                     plus scratch[b]), then each agent's edges
// Every scratch entry the later kernels read is written earlier in the same call, so
// nothing needs clearing.  Calls that overlap on one GPU share its scratch and race.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "swarp_hip.h"

namespace swarp {
int set_error(const char *msg);  // swarp_hip.hip: the message swarp_last_error() returns
}

#define COO_SCRATCH_BLOCKS 65536  // partial sums: 512 KiB per GPU

// The per-block partial sums.  Host code never passes this name to a kernel: each GPU
// holds its own copy, whose device address scratch_ptr() looks up.
static __device__ __align__(256) int64_t scratch[COO_SCRATCH_BLOCKS];

namespace {

constexpr int COO_BLOCK = 256;

// A list count as the number of valid slots of its row (counts from the neighbour
// kernels already lie in [0, K]).
__device__ __forceinline__ int64_t clamp_count(int32_t c, int32_t K)
{
    return c < 0 ? 0 : (c > K ? (int64_t)K : (int64_t)c);
}

__global__ __launch_bounds__(COO_BLOCK) void k_coo_block_sums(int64_t n, int32_t K,
                                                              const int32_t *cnt, int64_t *part)
{
    __shared__ int64_t red[COO_BLOCK / 64];
    const int64_t i = (int64_t)blockIdx.x * COO_BLOCK + threadIdx.x;
    int64_t v = i < n ? clamp_count(cnt[i], K) : 0;
    for (int d = 32; d > 0; d >>= 1) v += __shfl_down(v, d, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    if (threadIdx.x == 0) {
        int64_t s = 0;
        for (int w = 0; w < COO_BLOCK / 64; ++w) s += red[w];
        part[blockIdx.x] = s;
    }
}

// Inclusive scan of one value per thread over a workgroup of 1024 (16 waves).
__device__ __forceinline__ int64_t block_scan_1024(int64_t v, int64_t *wsum)
{
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    for (int d = 1; d < 64; d <<= 1) {
        const int64_t y = __shfl_up(v, d, 64);
        if (lane >= d) v += y;
    }
    if (lane == 63) wsum[wv] = v;
    __syncthreads();
    int64_t before = 0;
    for (int w = 0; w < wv; ++w) before += wsum[w];
    __syncthreads();
    return v + before;
}

__global__ __launch_bounds__(1024) void k_coo_scan(int nb, int64_t *part, int64_t *n_edges)
{
    __shared__ int64_t wsum[16];
    __shared__ int64_t carry;
    if (threadIdx.x == 0) carry = 0;
    __syncthreads();
    for (int base = 0; base < nb; base += 1024) {
        const int i = base + (int)threadIdx.x;
        const int64_t v = i < nb ? part[i] : 0;
        const int64_t inc = block_scan_1024(v, wsum);
        const int64_t c = carry;
        if (i < nb) part[i] = c + inc - v;  // exclusive
        __syncthreads();
        if (threadIdx.x == 1023) carry = c + inc;
        __syncthreads();
    }
    if (threadIdx.x == 0) *n_edges = carry;
}

__global__ __launch_bounds__(COO_BLOCK) void k_coo_write(int64_t n, int32_t A, int32_t K,
                                                         const int32_t *idx, const int32_t *cnt,
                                                         const int64_t *part, int64_t capacity,
                                                         int64_t *out)
{
    __shared__ int64_t wsum[COO_BLOCK / 64];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int64_t i = (int64_t)blockIdx.x * COO_BLOCK + threadIdx.x;
    const int64_t c = i < n ? clamp_count(cnt[i], K) : 0;
    int64_t v = c;
    for (int d = 1; d < 64; d <<= 1) {
        const int64_t y = __shfl_up(v, d, 64);
        if (lane >= d) v += y;
    }
    if (lane == 63) wsum[wv] = v;
    __syncthreads();
    int64_t before = part[blockIdx.x];
    for (int w = 0; w < wv; ++w) before += wsum[w];
    if (i >= n) return;
    const int64_t o = before + v - c;  // this agent's first edge
    const int64_t e = i / A;
    for (int64_t s = 0; s < c && o + s < capacity; ++s) {
        out[o + s] = e * A + idx[i * K + s];
        out[capacity + o + s] = i;
    }
}

int fail(const char *msg) { return swarp::set_error(msg); }

// Device address of `scratch` per device, looked up once per device with it current.
constexpr int MAX_DEVICES = 64;
void *g_ptr[MAX_DEVICES];
std::mutex g_mu;

int scratch_ptr(void **ptr)
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail("hipGetDevice failed");
    if (dev < 0 || dev >= MAX_DEVICES) return fail("device ordinal out of range");
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_ptr[dev]) {
        // The lookup is not a stream operation, but a caller may be capturing a graph in
        // the global capture mode, which refuses calls of this kind from any thread: this
        // thread's mode is relaxed around the lookup and restored after it.
        hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
        const bool swapped = hipThreadExchangeStreamCaptureMode(&mode) == hipSuccess;
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (swapped) (void)hipThreadExchangeStreamCaptureMode(&mode);
        if (e != hipSuccess || !p) {
            char m[160];
            snprintf(m, sizeof m, "hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
            return fail(m);
        }
        g_ptr[dev] = p;
    }
    *ptr = g_ptr[dev];
    return 0;
}

}  // namespace

extern "C" {

int swarp_edge_index_noalloc(int32_t n_envs, int32_t n_agents, int32_t max_neighbors,
                             const int32_t *idx, const int32_t *cnt, int64_t capacity,
                             int64_t *edge_index, int64_t *n_edges, void *stream)
{
    swarp::set_error("");
    if (n_envs < 1 || n_agents < 1 || max_neighbors < 1) return fail("bad sizes");
    if (capacity < 0) return fail("capacity must be >= 0");
    if (!idx || !cnt || !n_edges || (capacity > 0 && !edge_index))
        return fail("pointer arguments must be set");
    const int64_t n = (int64_t)n_envs * n_agents;
    const int64_t nb = (n + COO_BLOCK - 1) / COO_BLOCK;
    if (nb > COO_SCRATCH_BLOCKS) {
        char m[160];
        snprintf(m, sizeof m,
                 "n_envs * n_agents = %lld exceeds the allocation-free limit of %lld agents",
                 (long long)n, (long long)COO_SCRATCH_BLOCKS * COO_BLOCK);
        return fail(m);
    }
    void *sp = nullptr;
    if (scratch_ptr(&sp)) return -1;
    int64_t *part = (int64_t *)sp;
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(k_coo_block_sums, dim3((unsigned)nb), dim3(COO_BLOCK), 0, st, n,
                       max_neighbors, cnt, part);
    hipLaunchKernelGGL(k_coo_scan, dim3(1), dim3(1024), 0, st, (int)nb, part, n_edges);
    hipLaunchKernelGGL(k_coo_write, dim3((unsigned)nb), dim3(COO_BLOCK), 0, st, n, n_agents,
                       max_neighbors, idx, cnt, (const int64_t *)part, capacity, edge_index);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(hipGetErrorString(e));
    return 0;
}

}  // extern "C"
