// Test helper, not part of the product: a bounded kernel that holds compute
// units while another stream's work runs, so that a GPU test can run the
// attention backward with only part of its grid resident.
//
// Each workgroup is one wave holding 128 KiB of LDS, so a CU (160 KiB of LDS)
// hosts one of them and no workgroup of the backward (about 49 KiB each)
// beside it. Every workgroup counts itself in `started`, then sleeps until
// `microseconds` of wall-clock time have passed since it started, and ends.
#include <hip/hip_runtime.h>

namespace {

constexpr int kHoldFloats = 32768;  // 128 KiB

__global__ __launch_bounds__(64) void occupy_kernel(long long ticks, int *started, float *sink)
{
    __shared__ float hold[kHoldFloats];
    hold[kHoldFloats - 1 - threadIdx.x] = (float)threadIdx.x;
    if (threadIdx.x == 0)
        atomicAdd(started, 1);
    const long long t0 = (long long)wall_clock64();
    while ((long long)wall_clock64() - t0 < ticks)
        __builtin_amdgcn_s_sleep(64);
    __syncthreads();
    if (threadIdx.x == 0 && blockIdx.x == 0)
        sink[0] = hold[kHoldFloats - 1];  // keeps the LDS allocation
}

}  // namespace

extern "C" int gpt_test_occupy(int n_workgroups, long long microseconds, int *started, float *sink, void *stream)
{
    if (n_workgroups <= 0 || microseconds < 0 || microseconds > 5000000 || !started || !sink)
        return -1;
    int dev = 0, khz = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess || khz <= 0)
        return -2;
    const long long ticks = microseconds * (long long)khz / 1000;
    hipLaunchKernelGGL(occupy_kernel, dim3((unsigned)n_workgroups), dim3(64), 0,
                       reinterpret_cast<hipStream_t>(stream), ticks, started, sink);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}
