// occupancy_probe.hip -- calibration program for the occupancy figures of the counter
// profiles (not part of libswarp_hip.so).  Every wave of `blocks` one-wave workgroups
// spins on s_memtime for a fixed number of ticks (a bounded wait: a tick budget and an
// iteration cap), so while they all run the mean number of resident waves per SIMD is
// blocks / 1024 on MI355X (256 CUs x 4 SIMDs).  Profiled with SQ_WAVE_CYCLES and
// SQ_BUSY_CYCLES, it fixes the unit of their ratio:
//     mean resident waves per SIMD = SQ_WAVE_CYCLES / SQ_BUSY_CYCLES / 8.
// Build and run: hipcc --offload-arch=gfx950 -O3 -o occ_probe occupancy_probe.hip
//                ./occ_probe BLOCKS TICKS
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>

__global__ void k_spin(uint64_t ticks, uint32_t *out)
{
    const uint64_t t0 = __builtin_amdgcn_s_memtime();
    uint64_t t = t0;
    for (int n = 0; t - t0 < ticks && n < (1 << 26); ++n) t = __builtin_amdgcn_s_memtime();
    if (threadIdx.x == 0) out[blockIdx.x] = (uint32_t)(t - t0);
}

int main(int argc, char **argv)
{
    const int blocks = argc > 1 ? atoi(argv[1]) : 1024;
    const uint64_t ticks = argc > 2 ? strtoull(argv[2], nullptr, 10) : 200000;
    if (blocks < 1 || blocks > (1 << 20)) return 1;
    uint32_t *o = nullptr;
    if (hipMalloc(&o, (size_t)blocks * sizeof(uint32_t)) != hipSuccess) return 2;
    for (int r = 0; r < 3; ++r) hipLaunchKernelGGL(k_spin, dim3(blocks), dim3(64), 0, 0, ticks, o);
    if (hipDeviceSynchronize() != hipSuccess) return 3;
    uint32_t first = 0;
    if (hipMemcpy(&first, o, sizeof first, hipMemcpyDeviceToHost) != hipSuccess) return 4;
    printf("blocks %d ticks %llu spun %u\n", blocks, (unsigned long long)ticks, first);
    return hipFree(o) == hipSuccess ? 0 : 5;
}
