// Host emulation of the parts of the HIP device model the swarp kernels use, for a CPU
// build of the kernels under AddressSanitizer / UndefinedBehaviorSanitizer (test
// infrastructure only: tests/test_asan_kernels.py).  It is found before the real
// <hip/hip_runtime.h> by include order and never reaches the product build.
//
// Execution model: a launch runs its blocks one after the other; a block runs one host
// thread per work-item.  __syncthreads is a barrier of the block's threads; the wave
// collectives (__ballot, __shfl*, readlane) are exchanges among the 64 threads of a wave
// through a per-wave buffer between two wave barriers.  Every barrier times out after
// 60 s and aborts the process with a message, so a collective reached by only part of a
// wave (which real hardware would evaluate over the active lanes) fails loudly instead of
// hanging.  Dynamic LDS is a fresh heap block of exactly the launch's size, and each
// `__shared__` array becomes a static object, so the sanitizer sees the true extent of
// every device-memory, LDS and argument access.  DPP and other intrinsics of the
// specialised kernels abort if called: those kernels are not emulated.
#pragma once
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <chrono>
#include <condition_variable>
#include <mutex>
#include <thread>
#include <vector>

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __align__(n) alignas(n)
#define __shared__ static

struct dim3 {
    unsigned x, y, z;
    dim3(unsigned a = 1, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};
struct alignas(16) uint4 {
    unsigned x, y, z, w;
};
typedef struct ihipStream_t *hipStream_t;
typedef int hipError_t;
#define hipSuccess 0
#define hipErrorLaunchFailure 719

namespace emu {

struct Barrier {
    std::mutex mu;
    std::condition_variable cv;
    int n = 0, waiting = 0;
    unsigned long gen = 0;
    void init(int count)
    {
        n = count;
        waiting = 0;
    }
    void wait(const char *what)
    {
        std::unique_lock<std::mutex> lk(mu);
        const unsigned long g = gen;
        if (++waiting == n) {
            waiting = 0;
            ++gen;
            cv.notify_all();
            return;
        }
        if (!cv.wait_for(lk, std::chrono::seconds(60), [&] { return gen != g; })) {
            fprintf(stderr, "emu: %s barrier timed out (%d of %d threads arrived): a barrier "
                            "or wave collective reached by only part of its group\n",
                    what, waiting, n);
            abort();
        }
    }
};

struct Wave {
    Barrier bar;
    uint64_t slot[64];
};

struct Block {
    Barrier bar;
    std::vector<Wave> waves;
    std::vector<unsigned char> *lds = nullptr;
};

inline thread_local dim3 tIdx, bIdx;
inline dim3 bDim, gDim;
inline Block *block = nullptr;
inline int last_error = 0;

inline unsigned char *dyn_lds() { return block->lds->empty() ? nullptr : block->lds->data(); }

inline Wave &my_wave() { return block->waves[tIdx.x / 64]; }

// every lane of the wave publishes `v`; returns the 64 published values
inline void exchange(uint64_t v, uint64_t (&out)[64])
{
    Wave &w = my_wave();
    w.slot[tIdx.x % 64] = v;
    w.bar.wait("wave");
    memcpy(out, w.slot, sizeof out);
    w.bar.wait("wave");
}

template <typename K, typename... A>
void launch(K kernel, dim3 grid, dim3 blk, size_t shm, A... args)
{
    const int nt = (int)(blk.x * blk.y * blk.z);
    if (nt % 64 != 0 && nt != 1) {
        fprintf(stderr, "emu: block of %d threads (not whole waves)\n", nt);
        abort();
    }
    gDim = grid;
    bDim = blk;
    for (unsigned bx = 0; bx < grid.x; ++bx) {
        Block B;
        B.bar.init(nt);
        B.waves = std::vector<Wave>((nt + 63) / 64);
        for (auto &w : B.waves) w.bar.init(nt < 64 ? nt : 64);
        std::vector<unsigned char> lds(shm);
        B.lds = &lds;
        block = &B;
        std::vector<std::thread> th;
        th.reserve(nt);
        for (int t = 0; t < nt; ++t)
            th.emplace_back([=] {
                tIdx = dim3(t, 0, 0);
                bIdx = dim3(bx, 0, 0);
                kernel(args...);
            });
        for (auto &t : th) t.join();
        block = nullptr;
    }
}

}  // namespace emu

#define threadIdx (::emu::tIdx)
#define blockIdx (::emu::bIdx)
#define blockDim (::emu::bDim)
#define gridDim (::emu::gDim)
#define hipLaunchKernelGGL(K, G, B, SHM, ST, ...) ::emu::launch(K, dim3(G), dim3(B), (size_t)(SHM), __VA_ARGS__)

inline hipError_t hipGetLastError() { return ::emu::last_error; }
inline const char *hipGetErrorString(hipError_t) { return "emulated launch failure"; }

inline void __syncthreads() { ::emu::block->bar.wait("block"); }

inline uint64_t __ballot(int pred)
{
    uint64_t v[64], m = 0;
    ::emu::exchange(pred ? 1u : 0u, v);
    const int n = (int)::emu::bDim.x < 64 ? (int)::emu::bDim.x : 64;
    for (int l = 0; l < n; ++l) m |= v[l] ? (1ull << l) : 0ull;
    return m;
}

template <typename T> inline uint64_t emu_bits(T x)
{
    uint64_t b = 0;
    memcpy(&b, &x, sizeof x);
    return b;
}
template <typename T> inline T emu_from(uint64_t b)
{
    T x;
    memcpy(&x, &b, sizeof x);
    return x;
}

template <typename T> inline T __shfl(T x, int src, int width = 64)
{
    uint64_t v[64];
    ::emu::exchange(emu_bits(x), v);
    const int l = (int)(::emu::tIdx.x % 64), base = l - l % width;
    return emu_from<T>(v[base + ((src % width) + width) % width]);
}
template <typename T> inline T __shfl_xor(T x, int mask, int width = 64)
{
    uint64_t v[64];
    ::emu::exchange(emu_bits(x), v);
    const int l = (int)(::emu::tIdx.x % 64), base = l - l % width;
    const int src = l ^ mask;
    return (src >= base && src < base + width) ? emu_from<T>(v[src]) : x;
}
template <typename T> inline T __shfl_up(T x, unsigned d, int width = 64)
{
    uint64_t v[64];
    ::emu::exchange(emu_bits(x), v);
    const int l = (int)(::emu::tIdx.x % 64), lw = l % width;
    return (lw >= (int)d) ? emu_from<T>(v[l - (int)d]) : x;
}
template <typename T> inline T __shfl_down(T x, unsigned d, int width = 64)
{
    uint64_t v[64];
    ::emu::exchange(emu_bits(x), v);
    const int l = (int)(::emu::tIdx.x % 64), lw = l % width;
    return (lw + (int)d < width) ? emu_from<T>(v[l + (int)d]) : x;
}

inline int __builtin_amdgcn_readlane(int x, int l)
{
    uint64_t v[64];
    ::emu::exchange((uint32_t)x, v);
    return (int)(uint32_t)v[l];
}

inline float __int_as_float(int x) { return emu_from<float>((uint32_t)x); }
inline int __float_as_int(float x) { return (int)(uint32_t)emu_bits(x); }
inline double __longlong_as_double(long long x) { return emu_from<double>((uint64_t)x); }
inline long long __double_as_longlong(double x) { return (long long)emu_bits(x); }

inline int min(int a, int b) { return a < b ? a : b; }
inline int max(int a, int b) { return a > b ? a : b; }
inline long long min(long long a, long long b) { return a < b ? a : b; }
inline long long max(long long a, long long b) { return a > b ? a : b; }

inline int atomicAdd(int *p, int v) { return __atomic_fetch_add(p, v, __ATOMIC_SEQ_CST); }

inline float __builtin_amdgcn_sqrtf(float x) { return sqrtf(x); }
inline double __builtin_amdgcn_rcp(double x) { return 1.0 / x; }
inline float __builtin_amdgcn_rcpf(float x) { return 1.0f / x; }
inline float rsqrtf(float x) { return 1.0f / sqrtf(x); }
inline double rsqrt(double x) { return 1.0 / sqrt(x); }
#define __builtin_assume(x) ((void)0)

// intrinsics of the specialised (DPP) kernels: not emulated
[[noreturn]] inline void emu_not_emulated(const char *what)
{
    fprintf(stderr, "emu: %s is not emulated (the specialised kernels do not run here)\n", what);
    abort();
}
inline int __builtin_amdgcn_update_dpp(int, int, int, int, int, bool) { emu_not_emulated("DPP"); }
inline int __builtin_amdgcn_mov_dpp(int, int, int, int, bool) { emu_not_emulated("DPP"); }
inline unsigned __builtin_amdgcn_ubfe(unsigned, unsigned, unsigned) { emu_not_emulated("ubfe"); }
inline void __builtin_amdgcn_s_waitcnt(int) {}
inline void __builtin_amdgcn_s_barrier() { emu_not_emulated("s_barrier"); }
// The hardware executes one wave's LDS instructions in issue order, so the lanes of a
// wave exchange values through LDS behind a wavefront-scope fence (a compiler fence
// only).  The emulated work-items run as concurrent threads, so here the fence is a
// barrier of the calling thread's wave.
inline void __builtin_amdgcn_wave_barrier() {}
inline void __builtin_amdgcn_fence(int, const char *scope)
{
    if (scope && strcmp(scope, "wavefront") == 0) ::emu::my_wave().bar.wait("wave fence");
}
struct alignas(16) int4 {
    int x, y, z, w;
};
inline int4 make_int4(int x, int y, int z, int w) { return int4{x, y, z, w}; }
inline uint64_t __builtin_amdgcn_read_exec() { emu_not_emulated("read_exec"); }
inline int __builtin_amdgcn_readfirstlane(int x) { return __builtin_amdgcn_readlane(x, 0); }
// issue priority between waves: nothing to order on the host
inline void __builtin_amdgcn_s_setprio(int) {}

inline unsigned __builtin_amdgcn_mbcnt_lo(unsigned, unsigned) { emu_not_emulated("mbcnt"); }
inline unsigned __builtin_amdgcn_mbcnt_hi(unsigned, unsigned) { emu_not_emulated("mbcnt"); }
inline int __builtin_amdgcn_ds_bpermute(int, int) { emu_not_emulated("ds_bpermute"); }
inline int __builtin_amdgcn_ds_swizzle(int, int) { emu_not_emulated("ds_swizzle"); }
