// Plain device-to-device copy kernel of a known size: the calibration point
// for HBM byte counters (rocprofv3 FETCH_SIZE / WRITE_SIZE read on this kernel
// against its exact 2 x bytes of traffic) and the achievable-bandwidth
// reference for the weight-streaming kernels.
//
//   benchmark_hbm_copy [--mib 1024] [--iters 20]
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdlib>
#include <iostream>
#include <string>

#define HIP_OK(expr)                                                                                     \
    do {                                                                                                 \
        const hipError_t e_ = (expr);                                                                    \
        if (e_ != hipSuccess) {                                                                          \
            std::cerr << "HIP error " << hipGetErrorString(e_) << " at " << __FILE__ << ":" << __LINE__ \
                      << std::endl;                                                                      \
            std::exit(1);                                                                                \
        }                                                                                                \
    } while (0)

__global__ __launch_bounds__(256) void copy16(const uint4* __restrict__ src, uint4* __restrict__ dst, int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

int main(int argc, char** argv) {
    int64_t mib = 1024;
    int iters = 20;
    for (int i = 1; i + 1 < argc; i += 2) {
        const std::string a = argv[i];
        if (a == "--mib") mib = std::stoll(argv[i + 1]);
        else if (a == "--iters") iters = std::stoi(argv[i + 1]);
    }
    const int64_t bytes = mib << 20;
    const int64_t n = bytes / 16;
    void *src, *dst;
    HIP_OK(hipMalloc(&src, bytes));
    HIP_OK(hipMalloc(&dst, bytes));
    HIP_OK(hipMemset(src, 1, bytes));
    const int grid = 256 * 32;
    hipEvent_t t0, t1;
    HIP_OK(hipEventCreate(&t0));
    HIP_OK(hipEventCreate(&t1));
    hipLaunchKernelGGL(copy16, dim3(grid), dim3(256), 0, 0, static_cast<const uint4*>(src), static_cast<uint4*>(dst), n);
    HIP_OK(hipDeviceSynchronize());
    HIP_OK(hipEventRecord(t0, 0));
    for (int i = 0; i < iters; ++i)
        hipLaunchKernelGGL(copy16, dim3(grid), dim3(256), 0, 0, static_cast<const uint4*>(src), static_cast<uint4*>(dst), n);
    HIP_OK(hipEventRecord(t1, 0));
    HIP_OK(hipEventSynchronize(t1));
    float ms = 0.f;
    HIP_OK(hipEventElapsedTime(&ms, t0, t1));
    ms /= iters;
    std::cout << "copy " << mib << " MiB: " << ms << " ms/launch, read+write " << 2.0 * bytes / ms / 1e6 << " GB/s"
              << " (bytes per launch: read " << bytes << ", write " << bytes << ")" << std::endl;
    HIP_OK(hipFree(src));
    HIP_OK(hipFree(dst));
    return 0;
}
