// Plain device-to-device copy kernel of a known size: the calibration point
// for HBM byte counters (rocprofv3 FETCH_SIZE / WRITE_SIZE read on this kernel
// against its exact 2 x bytes of traffic) and the achievable-bandwidth
// reference for the weight-streaming kernels.
//
//   benchmark_hbm_copy [--mib 1024] [--iters 20]
//   benchmark_hbm_copy --read-sweep   read-only streaming kernel over 16.8 MB,
//       67 MB and 268 MB buffers, cycling 24 buffers so that the 256 MB
//       Infinity Cache cannot serve them: the per-call floor a weight-streaming
//       kernel of that size can reach (launch + ramp + drain included)
//   benchmark_hbm_copy --read-bytes B  the same floor for one size of B bytes
//   benchmark_hbm_copy --read-bytes B --graph  the same 24 launches captured
//       once in a HIP graph and replayed (the launch method of a graph-replay
//       timing of the GEMM)
//   benchmark_hbm_copy --strip-probe [--n N] [--k K]  the lean small-M
//       kernel's memory traffic without its arithmetic (M=16, 16-column
//       strips, one 16-wave workgroup per strip, four 64-K stages in flight
//       per wave), 24 rotated (K/16, N, 16) weights, back to back: the weight
//       strip alone, the same bytes read contiguously per workgroup, the strip
//       plus the activation copies into LDS in the kernel's order, the copies
//       alone, and three other orders of the same loads
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdlib>
#include <initializer_list>
#include <iostream>
#include <string>

#include "../csrc/lds_dma.h"

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

__global__ __launch_bounds__(256) void read16(const uint4* __restrict__ src, int64_t n, uint32_t* __restrict__ sink) {
    uint32_t acc = 0;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x * 4;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x * 4 + threadIdx.x; i < n; i += stride) {
        uint4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = i + u * 256 < n ? src[i + u * 256] : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (int u = 0; u < 4; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x9e3779b9u) sink[0] = acc;  // keeps the loads live
}

int read_sweep(const std::initializer_list<int64_t>& sizes, bool graph = false) {
    const int nbuf = 24;
    uint32_t* sink;
    HIP_OK(hipMalloc(&sink, 4));
    hipEvent_t t0, t1;
    HIP_OK(hipEventCreate(&t0));
    HIP_OK(hipEventCreate(&t1));
    for (const int64_t bytes0 : sizes) {
        const int64_t bytes = (bytes0 + 15) / 16 * 16;
        void* bufs[nbuf];
        for (auto& b : bufs) {
            HIP_OK(hipMalloc(&b, bytes));
            HIP_OK(hipMemset(b, 1, bytes));
        }
        const int64_t n = bytes / 16;
        const int grid = 1024;
        for (int i = 0; i < nbuf; ++i)
            hipLaunchKernelGGL(read16, dim3(grid), dim3(256), 0, 0, static_cast<const uint4*>(bufs[i]), n, sink);
        HIP_OK(hipDeviceSynchronize());
        float ms = 0.f;
        if (graph) {
            hipStream_t s;
            HIP_OK(hipStreamCreate(&s));
            hipGraph_t g;
            hipGraphExec_t ge;
            HIP_OK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
            for (int i = 0; i < nbuf; ++i)
                hipLaunchKernelGGL(read16, dim3(grid), dim3(256), 0, s, static_cast<const uint4*>(bufs[i]), n, sink);
            HIP_OK(hipStreamEndCapture(s, &g));
            HIP_OK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
            for (int r = 0; r < 10; ++r) HIP_OK(hipGraphLaunch(ge, s));
            HIP_OK(hipStreamSynchronize(s));
            HIP_OK(hipEventRecord(t0, s));
            for (int r = 0; r < 40; ++r) HIP_OK(hipGraphLaunch(ge, s));
            HIP_OK(hipEventRecord(t1, s));
            HIP_OK(hipEventSynchronize(t1));
            HIP_OK(hipEventElapsedTime(&ms, t0, t1));
            ms /= 40 * nbuf;
            HIP_OK(hipGraphExecDestroy(ge));
            HIP_OK(hipGraphDestroy(g));
            HIP_OK(hipStreamDestroy(s));
        } else {
            HIP_OK(hipEventRecord(t0, 0));
            for (int i = 0; i < 10 * nbuf; ++i)
                hipLaunchKernelGGL(read16, dim3(grid), dim3(256), 0, 0, static_cast<const uint4*>(bufs[i % nbuf]), n,
                                   sink);
            HIP_OK(hipEventRecord(t1, 0));
            HIP_OK(hipEventSynchronize(t1));
            HIP_OK(hipEventElapsedTime(&ms, t0, t1));
            ms /= 10 * nbuf;
        }
        std::cout << "read " << bytes << " B" << (graph ? " (graph replay)" : "") << ": " << ms * 1000.0
                  << " us/call, " << bytes / ms / 1e6 << " GB/s" << std::endl;
        for (auto& b : bufs) HIP_OK(hipFree(b));
    }
    HIP_OK(hipFree(sink));
    return 0;
}

// Probe kinds of --strip-probe. Wave w of workgroup b takes stages w, w + 16,
// w + 32, w + 48 (64 K each) of 16-column strip b, like the lean small-M kernel.
enum StripProbe {
    kStrip = 0,        // weight strip only: per stage one 16-byte load per lane, 4 K groups x 16 columns
    kContiguous,       // the same byte count, each workgroup reading its own contiguous 64 KB
    kStripCopies,      // strip + activation copies (rows 0-15 of the stage into LDS), copies issued first
    kCopies,           // activation copies only
    kRotated,          // kStripCopies with the stage order rotated per workgroup
    kWeightsFirst,     // kStripCopies with the weight loads issued before the copies
    kInterleaved,      // per stage: weight load, then its copies
    kNumStripProbes
};
const char* const kStripProbeName[kNumStripProbes] = {"weight strip only", "contiguous 64 KB per workgroup",
                                                       "strip + activation copies (kernel order)",
                                                       "activation copies only", "strip + copies, rotated stages",
                                                       "strip + copies, weights first",
                                                       "strip + copies, interleaved per stage"};

template <int KIND>
__global__ __launch_bounds__(1024) void strip_probe(const uint16_t* __restrict__ A, const uint8_t* __restrict__ B,
                                                    int N, int K, uint32_t* __restrict__ sink) {
    constexpr int U = 4;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[16 * U * 2048];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int lr = lane & 15, lg = lane >> 4;
    const int nst = K >> 6;
    const int n0 = blockIdx.x * 16;
    const uint32_t slab = feather::lds_addr_of(smem) + wave * (U * 2048);
    const uint32_t cchunk = static_cast<uint32_t>((lane & 7) * 16);
    auto stage_of = [&](int st) { return KIND == kRotated ? (st + 4 * static_cast<int>(blockIdx.x)) % nst : st; };
    auto weight = [&](int st) -> uint4 {
        if (KIND == kContiguous)
            return *reinterpret_cast<const uint4*>(B + static_cast<int64_t>(blockIdx.x) * (K / 16) * 256 +
                                                   static_cast<int64_t>(st) * 1024 + lane * 16);
        return *reinterpret_cast<const uint4*>(B + (static_cast<int64_t>(st * 4 + lg) * N + n0 + lr) * 16);
    };
    auto copies = [&](int st, int u) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
            feather::dma16_lds(A, static_cast<uint32_t>(8 * j + (lane >> 3)) * static_cast<uint32_t>(K) * 2u +
                                      static_cast<uint32_t>(st) * 128u + cchunk,
                               slab + u * 2048 + j * 1024);
    };
    constexpr bool kW = KIND != kCopies;
    constexpr bool kC = KIND != kStrip && KIND != kContiguous;
    uint32_t acc = 0;
    for (int base = wave; base < nst; base += 16 * U) {
        uint4 v[U];
        if (KIND == kWeightsFirst) {
#pragma unroll
            for (int u = 0; u < U; ++u) v[u] = weight(base + u * 16);
        }
        if (KIND == kInterleaved) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                v[u] = weight(base + u * 16);
                copies(base + u * 16, u);
            }
        } else {
            if (kC) {
#pragma unroll
                for (int u = 0; u < U; ++u)
                    if (base + u * 16 < nst) copies(stage_of(base + u * 16), u);
            }
            if (kW && KIND != kWeightsFirst) {
#pragma unroll
                for (int u = 0; u < U; ++u) v[u] = weight(stage_of(base + u * 16));
            }
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        if (kW) {
#pragma unroll
            for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
        }
        if (kC) acc ^= *reinterpret_cast<const uint32_t*>(smem + wave * (U * 2048) + lane * 16);
    }
    if (acc == 0x9e3779b9u) sink[0] = acc;  // keeps the loads live
}

int strip_probe_run(int N, int K) {
    if (N % 16 != 0 || K % 4096 != 0) {
        std::cerr << "--strip-probe: N % 16 == 0 and K % 4096 == 0 (whole rounds of 64 stages)" << std::endl;
        return 1;
    }
    const int nbuf = 24;
    const int64_t bytes = static_cast<int64_t>(N) * K;
    uint8_t* bufs[nbuf];
    for (auto& b : bufs) {
        HIP_OK(hipMalloc(&b, bytes));
        HIP_OK(hipMemset(b, 1, bytes));
    }
    uint16_t* a;
    HIP_OK(hipMalloc(&a, static_cast<size_t>(16) * K * 2));
    HIP_OK(hipMemset(a, 0, static_cast<size_t>(16) * K * 2));
    uint32_t* sink;
    HIP_OK(hipMalloc(&sink, 4));
    hipEvent_t t0, t1;
    HIP_OK(hipEventCreate(&t0));
    HIP_OK(hipEventCreate(&t1));
    auto launch = [&](int kind, const uint8_t* b) {
        const dim3 grid(N / 16), block(1024);
        switch (kind) {
            case kStrip: hipLaunchKernelGGL(strip_probe<kStrip>, grid, block, 0, 0, a, b, N, K, sink); break;
            case kContiguous: hipLaunchKernelGGL(strip_probe<kContiguous>, grid, block, 0, 0, a, b, N, K, sink); break;
            case kStripCopies: hipLaunchKernelGGL(strip_probe<kStripCopies>, grid, block, 0, 0, a, b, N, K, sink); break;
            case kCopies: hipLaunchKernelGGL(strip_probe<kCopies>, grid, block, 0, 0, a, b, N, K, sink); break;
            case kRotated: hipLaunchKernelGGL(strip_probe<kRotated>, grid, block, 0, 0, a, b, N, K, sink); break;
            case kWeightsFirst: hipLaunchKernelGGL(strip_probe<kWeightsFirst>, grid, block, 0, 0, a, b, N, K, sink); break;
            default: hipLaunchKernelGGL(strip_probe<kInterleaved>, grid, block, 0, 0, a, b, N, K, sink); break;
        }
    };
    std::cout << "strip probe M=16 N=" << N << " K=" << K << ", " << nbuf << " rotated weights, back to back" << std::endl;
    for (int rep = 0; rep < 2; ++rep)
        for (int kind = 0; kind < kNumStripProbes; ++kind) {
            for (int i = 0; i < 1000; ++i) launch(kind, bufs[i % nbuf]);
            HIP_OK(hipEventRecord(t0, 0));
            for (int i = 0; i < 5000; ++i) launch(kind, bufs[i % nbuf]);
            HIP_OK(hipEventRecord(t1, 0));
            HIP_OK(hipEventSynchronize(t1));
            float ms = 0.f;
            HIP_OK(hipEventElapsedTime(&ms, t0, t1));
            std::cout << "  " << kStripProbeName[kind] << ": " << ms * 1000.0 / 5000 << " us/call" << std::endl;
        }
    for (auto& b : bufs) HIP_OK(hipFree(b));
    HIP_OK(hipFree(a));
    HIP_OK(hipFree(sink));
    return 0;
}

int main(int argc, char** argv) {
    int64_t mib = 1024;
    int iters = 20;
    for (int i = 1; i < argc; ++i)
        if (std::string(argv[i]) == "--strip-probe") {
            int n = 4096, k = 4096;
            for (int j = 1; j + 1 < argc; ++j) {
                if (std::string(argv[j]) == "--n") n = std::stoi(argv[j + 1]);
                if (std::string(argv[j]) == "--k") k = std::stoi(argv[j + 1]);
            }
            return strip_probe_run(n, k);
        }
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        if (a == "--read-sweep") return read_sweep({int64_t(16777216), int64_t(67108864), int64_t(268435456)});
        if (a == "--read-bytes" && i + 1 < argc) {
            const int64_t b = std::stoll(argv[++i]);
            if (b <= 0 || b > (int64_t(1) << 32)) {
                std::cerr << "--read-bytes takes 1 .. 2^32" << std::endl;
                return 1;
            }
            const bool graph = i + 1 < argc && std::string(argv[i + 1]) == "--graph";
            return read_sweep({b}, graph);
        }
        if (i + 1 >= argc) break;
        if (a == "--mib") mib = std::stoll(argv[++i]);
        else if (a == "--iters") iters = std::stoi(argv[++i]);
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
