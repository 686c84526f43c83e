// Standalone C++ bench of launch_scaled_mm (no torch), linking libfeatherops_amd.so.
//
// Same command line and report as the reference's
// cpp_benchmarks/benchmark_scaled_mm_hip.cpp: --m --n --k --warmup --iters
// --warps_m --warps_n --unroll --repeat_m --repeat_n; prints avg/std/min/max
// ms, TFLOP/s and GB/s with GB = 2*M*K + N*K + 2*M*N bytes. Inputs follow the
// same recipe (A uniform in [-1, 1) from mt19937(42); B drawn from the nine
// e5m2 codes {0, +-0.25, +-0.5, +-0.75, +-1}; scale 2.34; bias uniform).
// Calls go through feather_launch_scaled_mm_ws with the workspace the call
// can use (the small-M split-K path), allocated once and reused.
// Additions: --out fp16|bf16, --rotate R (cycle through R distinct weight
// buffers so that a weight larger than the 256 MB Infinity Cache in total is
// streamed from HBM), --b e5m2|e4m3. Default config is the gfx950 256x256
// tile (2,4,4,8,4).
// --quant: time feather_quantize_prepack_e5m2_ws (the torch op's entry) on an
// N x K fp16 weight instead: one pass (3 bytes per element: the weight read
// once, the codes written) where the weight fits the registers of the chip,
// else an amax pass + a quantize/prepack pass (5 bytes per element: 2 read for
// the amax, 2 read + 1 written for the codes); rates are printed for both byte
// counts. --quant-two-pass: the same through feather_quantize_prepack_e5m2,
// always two passes.
// --lora-down R: time feather_lora_down instead, T (M x R) = x (M x K) . D^T
// with bf16 x ~ U[-1, 1) rotated over --rotate buffers and D (R x K), GB/s on
// the bytes of x, D and T.
// --convert rtz|rne: time feather_bf16_to_fp16 (round toward zero, the
// reference's kernel/convert.py) or feather_bf16_to_fp16_rne on an N x N bf16
// matrix (randn), GB/s on 4 bytes per element (2 read + 2 written), the
// reference benchmark_convert.py's measure; --rotate buffers in and out.
// --dequant: time feather_dequantize_e5m2 of an (K/16, N, 16) e5m2 weight to an
// N x K fp16 matrix, GB/s on 3 bytes per element (1 read + 2 written).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <iomanip>
#include <iostream>
#include <numeric>
#include <random>
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
    int out_bf16 = 0;
    int b_dtype = FEATHER_B_E5M2;
    int rotate = 1;
    bool quant = false;
    bool quant_two_pass = false;
    int64_t lora_rank = 0;
    int convert = 0;  // 1 rtz, 2 rne
    bool dequant = false;
};

void usage(const char* argv0) {
    std::cout << "Usage: " << argv0
              << " [--m M] [--n N] [--k K] [--warmup W] [--iters I] [--warps_m M] [--warps_n N] [--unroll U]"
                 " [--repeat_m RM] [--repeat_n RN] [--out fp16|bf16] [--b e5m2|e4m3] [--rotate R] [--quant] [--quant-two-pass]"
                 " [--lora-down R] [--convert rtz|rne] [--dequant]\n";
}

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
        else if (a == "--b") o.b_dtype = val() == "e4m3" ? FEATHER_B_E4M3FN : FEATHER_B_E5M2;
        else if (a == "--rotate") o.rotate = std::max(1, std::stoi(val()));
        else if (a == "--quant") o.quant = true;
        else if (a == "--quant-two-pass") o.quant = o.quant_two_pass = true;
        else if (a == "--lora-down") o.lora_rank = std::stoll(val());
        else if (a == "--convert") o.convert = val() == "rne" ? 2 : 1;
        else if (a == "--dequant") o.dequant = true;
        else if (a == "--help" || a == "-h") {
            usage(argv[0]);
            std::exit(0);
        } else {
            std::cerr << "Unknown argument: " << a << std::endl;
            usage(argv[0]);
            std::exit(1);
        }
    }
    if (o.m <= 0 || o.n <= 0 || o.k <= 0 || o.warmup < 0 || o.iters <= 0) {
        std::cerr << "sizes and iters must be positive, warmup non-negative" << std::endl;
        std::exit(1);
    }
    return o;
}

uint16_t to_half_bits(float f) {
    const _Float16 h = static_cast<_Float16>(f);
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
}

// Quantize + prepack of an N x K fp16 weight with a computed per-tensor scale
// (the load path of the reference's quant.py:52-74 with no checkpoint scale).
int run_quant(const Opts& o) {
    const size_t nw = static_cast<size_t>(o.n) * o.k;
    std::mt19937 gen(42);
    std::normal_distribution<float> nrm(0.f, 0.02f);
    std::vector<uint16_t> hw(nw);
    for (auto& x : hw) x = to_half_bits(nrm(gen));
    std::vector<void*> dw(o.rotate);
    for (auto& p : dw) {
        HIP_OK(hipMalloc(&p, nw * 2));
        HIP_OK(hipMemcpy(p, hw.data(), nw * 2, hipMemcpyHostToDevice));
    }
    uint8_t* dq;
    float* dscale;
    void* dws;
    const size_t ws_bytes = feather_quantize_workspace_size();
    HIP_OK(hipMalloc(&dq, nw));
    HIP_OK(hipMalloc(&dscale, sizeof(float)));
    HIP_OK(hipMalloc(&dws, ws_bytes));
    HIP_OK(hipMemset(dws, 0, ws_bytes));  // the _ws entry's counters start at zero
    hipStream_t stream;
    hipEvent_t t0, t1;
    HIP_OK(hipStreamCreate(&stream));
    HIP_OK(hipEventCreate(&t0));
    HIP_OK(hipEventCreate(&t1));
    auto run = [&](int i) {
        const int rc = o.quant_two_pass
                           ? feather_quantize_prepack_e5m2(dw[i % o.rotate], FEATHER_DTYPE_F16, o.n, o.k, nullptr, 0,
                                                           dq, dscale, static_cast<uint32_t*>(dws), stream)
                           : feather_quantize_prepack_e5m2_ws(dw[i % o.rotate], FEATHER_DTYPE_F16, o.n, o.k, nullptr,
                                                              0, dq, dscale, dws, ws_bytes, stream);
        if (rc != FEATHER_OK) {
            std::cerr << "quantize failed: " << feather_status_string(rc) << std::endl;
            std::exit(1);
        }
    };
    for (int i = 0; i < o.warmup; ++i) run(i);
    HIP_OK(hipStreamSynchronize(stream));
    HIP_OK(hipEventRecord(t0, stream));
    for (int i = 0; i < o.iters; ++i) run(i);
    HIP_OK(hipEventRecord(t1, stream));
    HIP_OK(hipEventSynchronize(t1));
    float ms = 0.f;
    HIP_OK(hipEventElapsedTime(&ms, t0, t1));
    ms /= o.iters;
    const double bytes = 5.0 * static_cast<double>(nw);
    std::cout << std::fixed << std::setprecision(4);
    std::cout << "quantize_prepack_e5m2 benchmark\n  problem: n=" << o.n << " k=" << o.k << " fp16 rotate=" << o.rotate
              << (o.quant_two_pass ? " two-pass entry" : "") << "\n  back-to-back ms: " << ms << "  (GB/s "
              << bytes / ms / 1e6 << " on 5 B/element, " << 0.6 * bytes / ms / 1e6
              << " on 3 B/element: the weight read once, the codes written once)" << std::endl;
    for (auto p : dw) HIP_OK(hipFree(p));
    HIP_OK(hipFree(dq));
    HIP_OK(hipFree(dscale));
    HIP_OK(hipFree(dws));
    HIP_OK(hipEventDestroy(t0));
    HIP_OK(hipEventDestroy(t1));
    HIP_OK(hipStreamDestroy(stream));
    return 0;
}

uint16_t to_bf16_bits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// T = x . D^T through feather_lora_down (bf16), x rotated over o.rotate buffers.
int run_lora_down(const Opts& o) {
    const int64_t M = o.m, K = o.k, R = o.lora_rank;
    const size_t nx = static_cast<size_t>(M) * K, nd = static_cast<size_t>(R) * K, nt = static_cast<size_t>(M) * R;
    std::mt19937 gen(42);
    std::uniform_real_distribution<float> uni(-1.f, 1.f);
    std::vector<uint16_t> hx(nx), hd(nd);
    for (auto& v : hx) v = to_bf16_bits(uni(gen));
    for (auto& v : hd) v = to_bf16_bits(0.05f * uni(gen));
    std::vector<void*> dx(o.rotate);
    for (auto& p : dx) {
        HIP_OK(hipMalloc(&p, nx * 2));
        HIP_OK(hipMemcpy(p, hx.data(), nx * 2, hipMemcpyHostToDevice));
    }
    void *dd, *dt, *dws = nullptr;
    HIP_OK(hipMalloc(&dd, nd * 2));
    HIP_OK(hipMalloc(&dt, nt * 2));
    HIP_OK(hipMemcpy(dd, hd.data(), nd * 2, hipMemcpyHostToDevice));
    const size_t ws = feather_lora_down_workspace_size(M, K, R);
    if (ws) {
        HIP_OK(hipMalloc(&dws, ws));
        HIP_OK(hipMemset(dws, 0, ws));
    }
    hipStream_t stream;
    hipEvent_t t0, t1;
    HIP_OK(hipStreamCreate(&stream));
    HIP_OK(hipEventCreate(&t0));
    HIP_OK(hipEventCreate(&t1));
    auto run = [&](int i) {
        const int rc = feather_lora_down(dx[i % o.rotate], FEATHER_DTYPE_BF16, dd, dt, M, K, R, dws, ws, stream);
        if (rc != FEATHER_OK) {
            std::cerr << "lora_down failed: " << feather_status_string(rc) << std::endl;
            std::exit(1);
        }
    };
    for (int i = 0; i < o.warmup; ++i) run(i);
    HIP_OK(hipStreamSynchronize(stream));
    HIP_OK(hipEventRecord(t0, stream));
    for (int i = 0; i < o.iters; ++i) run(i);
    HIP_OK(hipEventRecord(t1, stream));
    HIP_OK(hipEventSynchronize(t1));
    float ms = 0.f;
    HIP_OK(hipEventElapsedTime(&ms, t0, t1));
    ms /= o.iters;
    const double bytes = 2.0 * (nx + nd + nt);
    std::cout << std::fixed << std::setprecision(4);
    std::cout << "lora_down benchmark\n  problem: m=" << M << " k=" << K << " rank=" << R << " bf16 rotate=" << o.rotate
              << " workspace=" << ws << "\n  back-to-back ms: " << ms << "  (GB/s " << bytes / ms / 1e6
              << " on x + D + T)" << std::endl;
    for (auto p : dx) HIP_OK(hipFree(p));
    HIP_OK(hipFree(dd));
    HIP_OK(hipFree(dt));
    if (dws) HIP_OK(hipFree(dws));
    HIP_OK(hipEventDestroy(t0));
    HIP_OK(hipEventDestroy(t1));
    HIP_OK(hipStreamDestroy(stream));
    return 0;
}

// One HBM-bound auxiliary kernel, back to back over o.rotate (input, output)
// pairs: --convert (bf16 -> fp16 of an N x N matrix) or --dequant (an N x K
// e5m2 weight to fp16).
int run_aux(const Opts& o) {
    const bool conv = o.convert != 0;
    const size_t n = conv ? static_cast<size_t>(o.n) * o.n : static_cast<size_t>(o.n) * o.k;
    const size_t in_bytes = conv ? 2 * n : n;
    const size_t out_bytes = 2 * n;
    std::mt19937 gen(42);
    std::vector<uint8_t> host(in_bytes);
    if (conv) {
        std::normal_distribution<float> nrm(0.f, 1.f);
        for (size_t i = 0; i < n; ++i) {
            const uint16_t b = to_bf16_bits(nrm(gen));
            std::memcpy(&host[2 * i], &b, 2);
        }
    } else {
        // e5m2 codes of finite values (exponent field below 31)
        std::uniform_int_distribution<int> code(0, 255);
        for (auto& c : host) {
            int v = code(gen);
            if ((v & 0x7c) == 0x7c) v &= 0xbb;
            c = static_cast<uint8_t>(v);
        }
    }
    std::vector<void*> din(o.rotate), dout(o.rotate);
    for (int i = 0; i < o.rotate; ++i) {
        HIP_OK(hipMalloc(&din[i], in_bytes));
        HIP_OK(hipMemcpy(din[i], host.data(), in_bytes, hipMemcpyHostToDevice));
        HIP_OK(hipMalloc(&dout[i], out_bytes));
    }
    float* dscale;
    HIP_OK(hipMalloc(&dscale, sizeof(float)));
    const float hs = 0.0125f;
    HIP_OK(hipMemcpy(dscale, &hs, sizeof(float), hipMemcpyHostToDevice));
    hipStream_t stream;
    hipEvent_t t0, t1;
    HIP_OK(hipStreamCreate(&stream));
    HIP_OK(hipEventCreate(&t0));
    HIP_OK(hipEventCreate(&t1));
    auto run = [&](int i) {
        const int j = i % o.rotate;
        int rc;
        if (o.convert == 1)
            rc = feather_bf16_to_fp16(static_cast<const uint16_t*>(din[j]), static_cast<uint16_t*>(dout[j]), n, stream);
        else if (o.convert == 2)
            rc = feather_bf16_to_fp16_rne(static_cast<const uint16_t*>(din[j]), static_cast<uint16_t*>(dout[j]), n,
                                          stream);
        else
            rc = feather_dequantize_e5m2(static_cast<const uint8_t*>(din[j]), dscale, dout[j], FEATHER_DTYPE_F16, o.n,
                                         o.k, stream);
        if (rc != FEATHER_OK) {
            std::cerr << "launch failed: " << feather_status_string(rc) << std::endl;
            std::exit(1);
        }
    };
    for (int i = 0; i < o.warmup; ++i) run(i);
    HIP_OK(hipStreamSynchronize(stream));
    HIP_OK(hipEventRecord(t0, stream));
    for (int i = 0; i < o.iters; ++i) run(i);
    HIP_OK(hipEventRecord(t1, stream));
    HIP_OK(hipEventSynchronize(t1));
    float ms = 0.f;
    HIP_OK(hipEventElapsedTime(&ms, t0, t1));
    ms /= o.iters;
    const double bytes = static_cast<double>(in_bytes + out_bytes);
    std::cout << std::fixed << std::setprecision(4);
    if (conv)
        std::cout << "bf16_to_fp16" << (o.convert == 2 ? "_rne" : "") << " benchmark\n  problem: n=" << o.n
                  << " (n x n) rotate=" << o.rotate;
    else
        std::cout << "dequantize_e5m2 benchmark\n  problem: n=" << o.n << " k=" << o.k << " fp16 out rotate=" << o.rotate;
    std::cout << "\n  back-to-back us: " << ms * 1e3 << "  (GB/s " << bytes / ms / 1e6 << " on " << (conv ? 4 : 3)
              << " B/element)" << std::endl;
    for (int i = 0; i < o.rotate; ++i) {
        HIP_OK(hipFree(din[i]));
        HIP_OK(hipFree(dout[i]));
    }
    HIP_OK(hipFree(dscale));
    HIP_OK(hipEventDestroy(t0));
    HIP_OK(hipEventDestroy(t1));
    HIP_OK(hipStreamDestroy(stream));
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    const Opts o = parse(argc, argv);
    if (o.quant) return run_quant(o);
    if (o.convert || o.dequant) return run_aux(o);
    if (o.lora_rank > 0) return run_lora_down(o);
    if (o.k % (16 * o.u) != 0) {
        std::cerr << "K must be divisible by 16 * unroll_k (" << 16 * o.u << ")" << std::endl;
        return 1;
    }
    const size_t na = static_cast<size_t>(o.m) * o.k, nb = static_cast<size_t>(o.k) * o.n,
                 nc = static_cast<size_t>(o.m) * o.n;
    const double bytes = 2.0 * na + 1.0 * nb + 2.0 * nc;
    const double flops = 2.0 * o.m * o.n * o.k;

    std::mt19937 gen(42);
    std::uniform_real_distribution<float> uni(-1.f, 1.f);
    std::vector<uint16_t> ha(na), hbias(o.n);
    for (auto& x : ha) x = to_half_bits(uni(gen));
    for (auto& x : hbias) x = to_half_bits(uni(gen));
    static const uint8_t kCodes[] = {0xbc, 0xba, 0xb8, 0xb4, 0x00, 0x34, 0x38, 0x3a, 0x3c};
    std::uniform_int_distribution<int> pick(0, 8);
    std::vector<uint8_t> hb(nb);
    for (auto& x : hb) x = kCodes[pick(gen)];

    void *da, *dbias, *dc;
    float* dscale;
    std::vector<uint8_t*> db(o.rotate);
    HIP_OK(hipMalloc(&da, na * 2));
    HIP_OK(hipMalloc(&dbias, o.n * 2));
    HIP_OK(hipMalloc(&dc, nc * 2));
    HIP_OK(hipMalloc(&dscale, sizeof(float)));
    for (auto& p : db) {
        HIP_OK(hipMalloc(&p, nb));
        HIP_OK(hipMemcpy(p, hb.data(), nb, hipMemcpyHostToDevice));
    }
    HIP_OK(hipMemcpy(da, ha.data(), na * 2, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dbias, hbias.data(), o.n * 2, hipMemcpyHostToDevice));
    const float hs = 2.34f;
    HIP_OK(hipMemcpy(dscale, &hs, sizeof(float), hipMemcpyHostToDevice));

    // workspace for the small-M split-K path (zero-filled, reused by every call)
    const size_t ws_bytes = feather_scaled_mm_workspace_size(o.m, o.n, o.k, o.wm, o.wn, o.u, o.rm, o.rn);
    void* dws = nullptr;
    if (ws_bytes) {
        HIP_OK(hipMalloc(&dws, ws_bytes));
        HIP_OK(hipMemset(dws, 0, ws_bytes));
    }

    hipStream_t stream;
    hipEvent_t t0, t1;
    HIP_OK(hipStreamCreate(&stream));
    HIP_OK(hipEventCreate(&t0));
    HIP_OK(hipEventCreate(&t1));

    auto run = [&](int i) {
        const bool ok = feather_launch_scaled_mm_ws(da, db[i % o.rotate], dscale, static_cast<const uint16_t*>(dbias),
                                                    static_cast<uint16_t*>(dc), o.m, o.n, o.k, 1, 1, o.wm, o.wn, o.u,
                                                    o.rm, o.rn, o.b_dtype, o.out_bf16, dws, ws_bytes, stream);
        if (!ok) {
            std::cerr << "Failed to launch kernel: unsupported config" << std::endl;
            std::exit(1);
        }
    };
    for (int i = 0; i < o.warmup; ++i) run(i);
    HIP_OK(hipGetLastError());
    HIP_OK(hipStreamSynchronize(stream));

    std::vector<float> ms(o.iters);
    for (int i = 0; i < o.iters; ++i) {
        HIP_OK(hipEventRecord(t0, stream));
        run(i);
        HIP_OK(hipEventRecord(t1, stream));
        HIP_OK(hipEventSynchronize(t1));
        HIP_OK(hipEventElapsedTime(&ms[i], t0, t1));
    }
    // back-to-back launches, one event pair: the steady-state rate without per-call event gaps
    HIP_OK(hipEventRecord(t0, stream));
    for (int i = 0; i < o.iters; ++i) run(i);
    HIP_OK(hipEventRecord(t1, stream));
    HIP_OK(hipEventSynchronize(t1));
    float stream_ms = 0.f;
    HIP_OK(hipEventElapsedTime(&stream_ms, t0, t1));
    stream_ms /= o.iters;

    const double avg = std::accumulate(ms.begin(), ms.end(), 0.0) / ms.size();
    double var = 0.0;
    for (float x : ms) var += (x - avg) * (x - avg);
    const double sd = std::sqrt(var / ms.size());
    std::cout << std::fixed << std::setprecision(3);
    std::cout << "scaled_mm benchmark\n";
    std::cout << "  problem: m=" << o.m << " n=" << o.n << " k=" << o.k << (o.out_bf16 ? " out=bf16" : " out=fp16")
              << " rotate=" << o.rotate << "\n";
    std::cout << "  config: warps_m=" << o.wm << " warps_n=" << o.wn << " unroll_k=" << o.u << " repeat_m=" << o.rm
              << " repeat_n=" << o.rn << " kernel_id="
              << feather_scaled_mm_kernel_id(o.m, o.n, o.k, o.wm, o.wn, o.u, o.rm, o.rn) << "\n";
    std::cout << "  memory footprint: " << bytes / (1024.0 * 1024.0) << " MiB\n";
    std::cout << "  avg ms: " << avg << "\n  std ms: " << sd << "\n";
    std::cout << "  min ms: " << *std::min_element(ms.begin(), ms.end()) << "\n";
    std::cout << "  max ms: " << *std::max_element(ms.begin(), ms.end()) << "\n";
    std::cout << "  avg TFLOP/s: " << flops / avg / 1e9 << "\n";
    std::cout << "  avg GB/s: " << bytes / avg / 1e6 << "\n";
    std::cout << "  back-to-back ms: " << stream_ms << "  (TFLOP/s " << flops / stream_ms / 1e9 << ", GB/s "
              << bytes / stream_ms / 1e6 << ")" << std::endl;
    std::cout << "  back-to-back us: " << stream_ms * 1e3 << std::endl;
    if (o.rotate > 1) {
        // the rotate launches captured once in a HIP graph and replayed
        hipGraph_t g;
        hipGraphExec_t ge;
        HIP_OK(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
        for (int i = 0; i < o.rotate; ++i) run(i);
        HIP_OK(hipStreamEndCapture(stream, &g));
        HIP_OK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
        const int reps = std::max(1, o.iters / o.rotate);
        for (int r = 0; r < std::max(1, reps / 4); ++r) HIP_OK(hipGraphLaunch(ge, stream));
        HIP_OK(hipStreamSynchronize(stream));
        HIP_OK(hipEventRecord(t0, stream));
        for (int r = 0; r < reps; ++r) HIP_OK(hipGraphLaunch(ge, stream));
        HIP_OK(hipEventRecord(t1, stream));
        HIP_OK(hipEventSynchronize(t1));
        float gms = 0.f;
        HIP_OK(hipEventElapsedTime(&gms, t0, t1));
        std::cout << "  graph-replay us: " << gms * 1e3 / (reps * o.rotate) << std::endl;
        HIP_OK(hipGraphExecDestroy(ge));
        HIP_OK(hipGraphDestroy(g));
    }

    HIP_OK(hipEventDestroy(t0));
    HIP_OK(hipEventDestroy(t1));
    HIP_OK(hipStreamDestroy(stream));
    for (auto p : db) HIP_OK(hipFree(p));
    if (dws) HIP_OK(hipFree(dws));
    HIP_OK(hipFree(da));
    HIP_OK(hipFree(dbias));
    HIP_OK(hipFree(dc));
    HIP_OK(hipFree(dscale));
    return 0;
}
