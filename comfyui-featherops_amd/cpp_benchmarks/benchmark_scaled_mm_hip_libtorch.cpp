// libtorch flavour of the C++ bench of launch_scaled_mm: operands are ATen
// tensors on the GPU (allocated and filled by torch's own kernels), the launch
// goes to the C ABI of libfeatherops_amd.so on torch's current HIP stream.
//
// Same command line and report as the reference's
// cpp_benchmarks/benchmark_scaled_mm_hip_libtorch.cpp: --m --n --k --warmup
// --iters --warps_m --warps_n --unroll --repeat_m --repeat_n; prints avg/std/
// min/max ms, TFLOP/s and GB/s with GB = 2*M*K + N*K + 2*M*N bytes. Inputs:
// A ~ N(0, 1) fp16, B random e5m2 codes of N(0, 1) values (torch's fp8 cast),
// scale 2.34, bias ~ N(0, 1) fp16. Additions: --out fp16|bf16 and --check,
// which compares C with a float64 evaluation of the same contract (torch on
// the device) and exits non-zero on a mismatch.
#include <ATen/ATen.h>
#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <iomanip>
#include <iostream>
#include <numeric>
#include <string>
#include <vector>

#include "featherops_amd.h"

#define HIP_OK(expr)                                                                                     \
    do {                                                                                                 \
        const hipError_t e_ = (expr);                                                                    \
        if (e_ != hipSuccess) {                                                                          \
            std::cerr << "HIP error " << hipGetErrorString(e_) << " at " << __FILE__ << ":" << __LINE__ \
                      << std::endl;                                                                      \
            std::exit(1);                                                                                \
        }                                                                                                \
    } while (0)

namespace {

struct Opts {
    int64_t m = 8192, n = 8192, k = 8192;
    int warmup = 10, iters = 100;
    int wm = 2, wn = 4, u = 4, rm = 8, rn = 4;
    bool out_bf16 = false;
    bool check = false;
};

Opts parse(int argc, char** argv) {
    Opts o;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        auto val = [&]() -> std::string {
            if (i + 1 >= argc) {
                std::cerr << "Missing value for " << a << std::endl;
                std::exit(1);
            }
            return argv[++i];
        };
        if (a == "--m") o.m = std::stoll(val());
        else if (a == "--n") o.n = std::stoll(val());
        else if (a == "--k") o.k = std::stoll(val());
        else if (a == "--warmup") o.warmup = std::stoi(val());
        else if (a == "--iters") o.iters = std::stoi(val());
        else if (a == "--warps_m") o.wm = std::stoi(val());
        else if (a == "--warps_n") o.wn = std::stoi(val());
        else if (a == "--unroll") o.u = std::stoi(val());
        else if (a == "--repeat_m") o.rm = std::stoi(val());
        else if (a == "--repeat_n") o.rn = std::stoi(val());
        else if (a == "--out") o.out_bf16 = val() == "bf16";
        else if (a == "--check") o.check = true;
        else {
            std::cout << "Usage: " << argv[0]
                      << " [--m M] [--n N] [--k K] [--warmup W] [--iters I] [--warps_m M] [--warps_n N] [--unroll U]"
                         " [--repeat_m RM] [--repeat_n RN] [--out fp16|bf16] [--check]\n";
            std::exit(a == "--help" || a == "-h" ? 0 : 1);
        }
    }
    if (o.m <= 0 || o.n <= 0 || o.k <= 0 || o.k % 16 != 0 || o.warmup < 0 || o.iters <= 0) {
        std::cerr << "sizes and iters must be positive, K a multiple of 16" << std::endl;
        std::exit(1);
    }
    return o;
}

}  // namespace

int main(int argc, char** argv) {
    const Opts o = parse(argc, argv);
    const at::Device dev(at::kCUDA, 0);
    const at::ScalarType out_t = o.out_bf16 ? at::kBFloat16 : at::kHalf;
    at::manual_seed(42);
    const at::Tensor a = at::randn({o.m, o.k}, at::TensorOptions().dtype(at::kFloat).device(dev)).to(at::kHalf);
    // (K, N) e5m2 values, prepacked to (K/16, N, 16): element (k, n) at [k/16][n][k%16]
    const at::Tensor b_kn = at::randn({o.k, o.n}, at::TensorOptions().dtype(at::kFloat).device(dev))
                                .to(at::kFloat8_e5m2);
    const at::Tensor bp = b_kn.view({o.k / 16, 16, o.n}).permute({0, 2, 1}).contiguous();
    const at::Tensor scale = at::full({1}, 2.34, at::TensorOptions().dtype(at::kFloat).device(dev));
    const at::Tensor bias = at::randn({o.n}, at::TensorOptions().dtype(at::kFloat).device(dev)).to(out_t);
    at::Tensor c = at::empty({o.m, o.n}, at::TensorOptions().dtype(out_t).device(dev));
    const hipStream_t stream = c10::hip::getCurrentHIPStream(dev.index()).stream();

    const size_t ws_bytes = feather_scaled_mm_workspace_size(o.m, o.n, o.k, o.wm, o.wn, o.u, o.rm, o.rn);
    at::Tensor ws = at::zeros({static_cast<int64_t>(std::max<size_t>(ws_bytes, 16))},
                              at::TensorOptions().dtype(at::kByte).device(dev));
    auto run = [&]() {
        const bool ok = feather_launch_scaled_mm_ws(
            a.data_ptr(), static_cast<const uint8_t*>(bp.data_ptr()), static_cast<const float*>(scale.data_ptr()),
            static_cast<const uint16_t*>(bias.data_ptr()), static_cast<uint16_t*>(c.data_ptr()), o.m, o.n, o.k, 1, 1,
            o.wm, o.wn, o.u, o.rm, o.rn, FEATHER_B_E5M2, o.out_bf16 ? 1 : 0, ws.data_ptr(), ws_bytes, stream);
        if (!ok) {
            std::cerr << "Failed to launch kernel: unsupported config" << std::endl;
            std::exit(1);
        }
    };
    for (int i = 0; i < o.warmup; ++i) run();
    HIP_OK(hipGetLastError());
    HIP_OK(hipStreamSynchronize(stream));

    hipEvent_t t0, t1;
    HIP_OK(hipEventCreate(&t0));
    HIP_OK(hipEventCreate(&t1));
    std::vector<float> ms(o.iters);
    for (int i = 0; i < o.iters; ++i) {
        HIP_OK(hipEventRecord(t0, stream));
        run();
        HIP_OK(hipEventRecord(t1, stream));
        HIP_OK(hipEventSynchronize(t1));
        HIP_OK(hipEventElapsedTime(&ms[i], t0, t1));
    }
    HIP_OK(hipEventDestroy(t0));
    HIP_OK(hipEventDestroy(t1));

    const double bytes = 2.0 * o.m * o.k + 1.0 * o.k * o.n + 2.0 * o.m * o.n;
    const double flops = 2.0 * o.m * o.n * o.k;
    const double avg = std::accumulate(ms.begin(), ms.end(), 0.0) / ms.size();
    double var = 0.0;
    for (float x : ms) var += (x - avg) * (x - avg);
    std::cout << std::fixed << std::setprecision(3);
    std::cout << "scaled_mm libtorch benchmark\n";
    std::cout << "  problem: m=" << o.m << " n=" << o.n << " k=" << o.k << (o.out_bf16 ? " out=bf16" : " out=fp16")
              << "\n";
    std::cout << "  config: warps_m=" << o.wm << " warps_n=" << o.wn << " unroll_k=" << o.u << " repeat_m=" << o.rm
              << " repeat_n=" << o.rn << " kernel_id="
              << feather_scaled_mm_kernel_id(o.m, o.n, o.k, o.wm, o.wn, o.u, o.rm, o.rn) << "\n";
    std::cout << "  memory footprint: " << bytes / (1024.0 * 1024.0) << " MiB\n";
    std::cout << "  avg ms: " << avg << "\n  std ms: " << std::sqrt(var / ms.size()) << "\n";
    std::cout << "  min ms: " << *std::min_element(ms.begin(), ms.end()) << "\n";
    std::cout << "  max ms: " << *std::max_element(ms.begin(), ms.end()) << "\n";
    std::cout << "  avg TFLOP/s: " << flops / avg / 1e9 << "\n";
    std::cout << "  avg GB/s: " << bytes / avg / 1e6 << std::endl;

    if (o.check) {
        // the kernel contract in float64: scale on the float32-rounded sum, one rounding to the
        // output type, bias added in the output type
        const at::Tensor acc = at::matmul(a.to(at::kDouble), b_kn.to(at::kDouble)).to(at::kFloat) * 2.34f;
        const at::Tensor want = (acc.to(out_t).to(at::kFloat) + bias.to(at::kFloat)).to(out_t);
        const at::Tensor d = (c.to(at::kDouble) - want.to(at::kDouble)).abs();
        const at::Tensor r = want.to(at::kDouble).abs();
        const int mant = o.out_bf16 ? 7 : 10;
        const at::Tensor ulp = at::exp2(at::floor(at::log2(at::clamp_min(r, std::ldexp(1.0, -14)))) - mant);
        const at::Tensor tol = at::clamp_min(2.0 * ulp * 1.0001, 2e-2);
        const double worst = (d / tol).max().item<double>();
        const double fro = (d.norm() / at::clamp_min(r.norm(), 1e-6)).item<double>();
        std::cout << "  check: max |diff|/tol " << worst << ", rel-Fro " << fro << (worst <= 1.0 && fro <= 1e-3 ? " ok" : " FAILED")
                  << std::endl;
        if (!(worst <= 1.0 && fro <= 1e-3)) return 2;
    }
    return 0;
}
