// Small-M (M <= 64) fp16 x fp8 GEMM for gfx950: the weight-streaming regime.
//
// Same contract as the tile kernel (reference kernel/hip/hip_kernel.cu:133-420:
// fp32 accumulation, scale on the accumulator, rounding to the output type,
// bias added in the output type). At M <= 64 the weight bytes dominate HBM
// traffic (M=16, K=N=4096: 16.8 MB of weight vs 0.26 MB of activations and
// output), so the kernel is built to stream Bp once at full bandwidth:
//   * one workgroup per 16-column strip of N, 16 waves splitting K between
//     them (split-K inside the workgroup); every wave keeps several 64-K stages
//     of 16-byte weight loads in flight;
//   * the contraction of each 16 x 64 slice runs on the 16x16x32 fp16 MFMA:
//     the wave64 VALU (v_dot2_f32_f16: 256 flop/clk/CU, 157 TFLOP/s chip-wide)
//     would need 3.4 us for M=16, K=N=4096, above the 3.0 us budget of 70% of
//     HBM bandwidth, while the MFMA does it in a fraction of the load time;
//   * partial sums of the 16 waves are reduced through LDS in a fixed order
//     (deterministic), then the epilogue applies scale, rounding and bias.
#include "feather_common.h"
#include "scaled_mm_dispatch.h"

namespace feather {
namespace {

constexpr int kWaves = 16;

template <int MT, bool kBf16, bool kE4m3>
__global__ __launch_bounds__(64 * kWaves) void scaled_mm_smallm_kernel(
    const uint16_t* __restrict__ A, const uint8_t* __restrict__ Bp, const float* __restrict__ scale,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ C, int M, int N, int K, int has_scale, int has_bias) {
    constexpr int U = MT <= 2 ? 4 : 2;  // stages in flight per wave
    constexpr int kRows = MT * 16;
    constexpr int kRedStride = 17;      // floats per reduction row (16 + 1 pad)
    __shared__ float red[kWaves][kRows][kRedStride];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int lr = lane & 15;
    const int lg = lane >> 4;
    const int n0 = blockIdx.x * 16;
    const int col = n0 + lr;
    const int kgroups = K >> 4;
    const int nst = (K + 63) >> 6;

    f32x4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int base = wave; base < nst; base += kWaves * U) {
        uint4 braw[U];
        uint4 araw[U][MT][2];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kg = (base + u * kWaves) * 4 + lg;
            const bool kval = kg < kgroups;
            braw[u] = kval ? *reinterpret_cast<const uint4*>(Bp + (static_cast<int64_t>(kg) * N + col) * 16)
                           : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int row = mt * 16 + lr;
                if (kval && row < M) {
                    const uint4* ap = reinterpret_cast<const uint4*>(A + static_cast<int64_t>(row) * K + kg * 16);
                    araw[u][mt][0] = ap[0];
                    araw[u][mt][1] = ap[1];
                } else {
                    araw[u][mt][0] = make_uint4(0u, 0u, 0u, 0u);
                    araw[u][mt][1] = make_uint4(0u, 0u, 0u, 0u);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (base + u * kWaves < nst) {
                const half8_t b0 = widen_fp8x8<kE4m3>(braw[u].x, braw[u].y);
                const half8_t b1 = widen_fp8x8<kE4m3>(braw[u].z, braw[u].w);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    acc[mt] = mfma16x16x32(as_half8(araw[u][mt][0]), b0, acc[mt]);
                    acc[mt] = mfma16x16x32(as_half8(araw[u][mt][1]), b1, acc[mt]);
                }
            }
        }
    }

    // accumulator element i of lane (lr, lg) is (row 4*lg + i, col lr) of its 16x16 tile
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave][mt * 16 + 4 * lg + i][lr] = acc[mt][i];
    __syncthreads();

    const float s = has_scale ? scale[0] : 1.0f;
    for (int e = tid; e < M * 16; e += 64 * kWaves) {
        const int r = e >> 4;
        const int c = e & 15;
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) sum += red[w][r][c];
        const float v = kE4m3 ? (sum * 256.0f) * s : sum * s;
        uint16_t o = f32_to_out_bits<kBf16>(v);
        if (has_bias) o = f32_to_out_bits<kBf16>(out_bits_to_f32<kBf16>(o) + out_bits_to_f32<kBf16>(bias[n0 + c]));
        C[static_cast<int64_t>(r) * N + n0 + c] = o;
    }
}

template <int MT>
void launch_mt(const MmArgs& p, hipStream_t stream) {
    const dim3 grid(static_cast<uint32_t>(p.N / 16));
    const dim3 block(64 * kWaves);
#define FEATHER_SMALLM_LAUNCH(BF, E4)                                                                                 \
    hipLaunchKernelGGL((scaled_mm_smallm_kernel<MT, BF, E4>), grid, block, 0, stream, p.a, p.b, p.scale, p.bias, p.c, \
                       static_cast<int>(p.M), static_cast<int>(p.N), static_cast<int>(p.K), p.has_scale, p.has_bias)
    if (p.out_bf16) {
        if (p.b_e4m3) FEATHER_SMALLM_LAUNCH(true, true);
        else FEATHER_SMALLM_LAUNCH(true, false);
    } else {
        if (p.b_e4m3) FEATHER_SMALLM_LAUNCH(false, true);
        else FEATHER_SMALLM_LAUNCH(false, false);
    }
#undef FEATHER_SMALLM_LAUNCH
}

}  // namespace

bool launch_smallm_kernel(const MmArgs& p, hipStream_t stream) {
    if (p.M <= 0 || p.M > 64) return false;
    const int mt = static_cast<int>((p.M + 15) / 16);
    switch (mt) {
        case 1: launch_mt<1>(p, stream); return true;
        case 2: launch_mt<2>(p, stream); return true;
        case 3: launch_mt<3>(p, stream); return true;
        case 4: launch_mt<4>(p, stream); return true;
        default: return false;
    }
}

}  // namespace feather
