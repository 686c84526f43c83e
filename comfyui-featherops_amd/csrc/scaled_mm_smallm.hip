// Small-M (M <= 64) fp16 x fp8 GEMM for gfx950: the weight-streaming regime.
//
// Same contract as the tile kernels (reference kernel/hip/hip_kernel.cu:133-420:
// fp32 accumulation, scale on the accumulator, rounding to the output type,
// bias added in the output type). At M <= 64 the weight bytes dominate HBM
// traffic (M=16, K=N=4096: 16.8 MB of weight vs 0.26 MB of activations and
// output), so the kernel is built to stream Bp once at full bandwidth:
//   * a workgroup owns a strip of 16 * CT columns and one of `ksplit` K
//     ranges; its 16 waves split that K range again and keep several 64-K
//     stages of 16-byte weight loads in flight each;
//   * a wave reuses each A fragment for its CT column tiles, so activations
//     are re-read from L2 once per 16 * CT columns (not once per 16);
//   * the contraction of each 16 x 64 slice runs on the 16x16x32 fp16 MFMA:
//     the wave64 VALU (v_dot2_f32_f16: 256 flop/clk/CU, 157 TFLOP/s chip-wide)
//     would need 3.4 us for M=16, K=N=4096, more than the whole weight stream;
//   * the 16 waves' partial sums are reduced through LDS in a fixed order;
//   * with ksplit > 1 each workgroup stores its fp32 partial in a caller
//     workspace and bumps the strip's arrival counter; the workgroup that
//     arrives last adds the ksplit partials in split order (deterministic,
//     no waiting on other workgroups), applies the epilogue and re-zeroes the
//     counter for the next call. Partials and counters use device-coherent
//     (agent-scope) loads, stores and atomics; the splits of a strip are also
//     placed on one XCD (workgroup p runs on XCD p % 8).
#include <cstdlib>

#include "feather_common.h"
#include "lds_dma.h"
#include "scaled_mm_dispatch.h"

namespace feather {
namespace {

constexpr int kWaves = 16;

// Bytes of LDS A slab per wave and stage: MT row tiles of 16 rows x 128 bytes.
constexpr int kSlabTile = 16 * 128;

template <int MT, int CT, bool kLdsA, bool kBf16, bool kE4m3, bool kABf16>
__global__ __launch_bounds__(64 * kWaves) void scaled_mm_smallm_kernel(
    const uint16_t* __restrict__ A, const uint8_t* __restrict__ Bp, const float* __restrict__ scale,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ C, int M, int N, int K, int has_scale, int has_bias,
    int nstrips, int ksplit, float* __restrict__ partials, uint32_t* __restrict__ counters) {
    // stages in flight per wave (within the 128 VGPRs a 16-wave workgroup allows)
    // and, with A through LDS, within 16 waves x U x MT x 2 KB of slabs
    constexpr int U0 = (MT * 2 + CT) <= 4 ? 4 : (MT * 2 + CT) < 10 ? 2 : 1;
    constexpr int U = kLdsA && U0 * MT > 4 ? 4 / MT : U0;
    constexpr int kRows = MT * 16;
    constexpr int kCols = CT * 16;
    constexpr int kRedStride = kCols + 1;  // floats per reduction row (+1 pad)
    constexpr int kRedBytes = kWaves * kRows * kRedStride * 4;
    constexpr int kSlabBytes = kLdsA ? kWaves * U * MT * kSlabTile : 0;
    static_assert(kRedBytes <= 160 * 1024 && kSlabBytes <= 160 * 1024, "LDS budget");
    // the per-wave A slabs and the reduction buffer share one LDS block
    __shared__ __attribute__((aligned(1024))) uint8_t smem[kRedBytes > kSlabBytes ? kRedBytes : kSlabBytes];
    float(*red)[kRows][kRedStride] = reinterpret_cast<float(*)[kRows][kRedStride]>(smem);
    __shared__ int last_flag;

    // ---- workgroup -> (strip, K split); splits of a strip share an XCD ----
    const int pid = blockIdx.x;
    int strip, q;
    if (nstrips % kNumXcd == 0) {
        const int j = pid / kNumXcd;
        q = j % ksplit;
        strip = (j / ksplit) * kNumXcd + pid % kNumXcd;
    } else {
        strip = pid / ksplit;
        q = pid % ksplit;
    }

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int lr = lane & 15;
    const int lg = lane >> 4;
    const int n0 = strip * kCols;
    const int kgroups = K >> 4;
    const int nst = (K + 63) >> 6;
    const int per_split = (nst + ksplit - 1) / ksplit;
    const int st_begin = q * per_split;
    const int st_end = st_begin + per_split < nst ? st_begin + per_split : nst;

    f32x4 acc[MT][CT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) acc[mt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int base = st_begin + wave; base < st_end; base += kWaves * U) {
        uint4 braw[U][CT];
        uint4 araw[U][MT][2];
        if constexpr (kLdsA) {
            // A through LDS: each copy instruction fetches 8 rows x 128 bytes
            // (whole cache lines), which costs half the L1 lookups of loading
            // the MFMA layout (16 rows x 2 separate 16-byte pieces) directly.
            // Row r of a 16-row tile holds its 64-K stage as 8 chunks of 16
            // bytes, chunk c at position c ^ swz(r). Each wave uses its own
            // slab, so only this wave's copy count is waited for.
            const uint32_t slab = lds_addr_of(smem) + wave * (U * MT * kSlabTile);
            if (base > st_begin + wave) __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): last slab reads done
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int st = base + u * kWaves;
                if (st < st_end) {
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
                        for (int j = 0; j < 2; ++j) {
                            const int r16 = 8 * j + (lane >> 3);
                            const int row = mt * 16 + r16 < M ? mt * 16 + r16 : M - 1;
                            int c = (lane & 7) ^ swz(r16);
                            if (st * 4 + (c >> 1) >= kgroups) c = 0;  // past K: any in-row chunk (zeroed below)
                            dma16_lds(A, (static_cast<uint32_t>(row) * static_cast<uint32_t>(K) + st * 64 + c * 8) * 2u,
                                      slab + (u * MT + mt) * kSlabTile + j * 1024);
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int st = base + u * kWaves;
            const int kg = st * 4 + lg;
            const bool kval = st < st_end && kg < kgroups;
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
                const int col = n0 + ct * 16 + lr;
                braw[u][ct] = (kval && col < N)
                                  ? *reinterpret_cast<const uint4*>(Bp + (static_cast<int64_t>(kg) * N + col) * 16)
                                  : make_uint4(0u, 0u, 0u, 0u);
            }
            if constexpr (!kLdsA) {
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
        }
        if constexpr (kLdsA) {
            wait_vmcnt<0>();
            const uint8_t* slab = smem + wave * (U * MT * kSlabTile);
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int st = base + u * kWaves;
                const bool kval = st < st_end && st * 4 + lg < kgroups;
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const uint4 v = *reinterpret_cast<const uint4*>(
                            slab + (u * MT + mt) * kSlabTile + lr * 128 + (((2 * lg + h) ^ swz(lr)) << 4));
                        araw[u][mt][h] = kval ? v : make_uint4(0u, 0u, 0u, 0u);
                    }
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (base + u * kWaves < st_end) {
#pragma unroll
                for (int ct = 0; ct < CT; ++ct) {
                    const half8_t b0 = widen_fp8x8<kE4m3>(braw[u][ct].x, braw[u][ct].y);
                    const half8_t b1 = widen_fp8x8<kE4m3>(braw[u][ct].z, braw[u][ct].w);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        acc[mt][ct] = mfma16x16x32(b0, a_frag<kABf16>(araw[u][mt][0]), acc[mt][ct]);
                        acc[mt][ct] = mfma16x16x32(b1, a_frag<kABf16>(araw[u][mt][1]), acc[mt][ct]);
                    }
                }
            }
        }
    }

    if constexpr (kLdsA) __syncthreads();  // the reduction buffer overlays other waves' slabs
    // weights are the MFMA's first operand, activations its second (as in the
    // large-tile kernel), so accumulator element i of lane (lr, lg) is
    // (row lr, col 4*lg + i) of its 16x16 tile
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[wave][mt * 16 + lr][ct * 16 + 4 * lg + i] = acc[mt][ct][i];
    __syncthreads();

    const int tile_elems = M * kCols;
    if (ksplit > 1) {
        // Partials are written and read only as relaxed agent-scope atomics
        // (sc1 stores and loads: coherent across XCDs with no L2 write-back or
        // invalidate). Each wave's vmcnt wait returns once its stores are
        // visible at agent scope, before the barrier after which the arrival
        // RMW is issued; the last arrival's loads depend on the RMW's result
        // (through LDS and a barrier), so they are issued after it returned.
        // A release/acquire RMW instead adds an L2 write-back per workgroup
        // and an invalidate per last arrival (measured: M=16 N=5120 K=13824
        // 17 -> 18 us, M=64 N=13824 K=5120 on the split-K tiles 25 -> 38 us).
        float* my_part = partials + (static_cast<int64_t>(strip) * ksplit + q) * tile_elems;
        for (int e = tid; e < tile_elems; e += 64 * kWaves) {
            float sum = 0.f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) sum += red[w][e / kCols][e % kCols];
            __hip_atomic_store(&my_part[e], sum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __syncthreads();
        if (tid == 0)
            last_flag = __hip_atomic_fetch_add(&counters[strip], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                        static_cast<uint32_t>(ksplit - 1);
        __syncthreads();
        if (!last_flag) return;
    }

    const float s = has_scale ? scale[0] : 1.0f;
    for (int e = tid; e < tile_elems; e += 64 * kWaves) {
        const int r = e / kCols;
        const int c = e % kCols;
        if (n0 + c >= N) continue;
        float sum = 0.f;
        if (ksplit > 1) {
            const float* strip_parts = partials + static_cast<int64_t>(strip) * ksplit * tile_elems;
            for (int qq = 0; qq < ksplit; ++qq)
                sum += __hip_atomic_load(&strip_parts[static_cast<int64_t>(qq) * tile_elems + e], __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
        } else {
#pragma unroll
            for (int w = 0; w < kWaves; ++w) sum += red[w][r][c];
        }
        const float v = opaque_f32(sum * s);
        uint16_t o = f32_to_out_bits<kBf16>(v);
        if (has_bias) o = f32_to_out_bits<kBf16>(out_bits_to_f32<kBf16>(o) + out_bits_to_f32<kBf16>(bias[n0 + c]));
        C[static_cast<int64_t>(r) * N + n0 + c] = o;
    }
    if (ksplit > 1 && tid == 0)  // ready for the next call on this stream
        __hip_atomic_store(&counters[strip], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Lean variant for the most common small-M calls: M <= 32 (MT = 1 or 2 row
// tiles of 16), K % 64 == 0, one 16-column strip per workgroup with the whole
// K range (no split across workgroups). Same arithmetic and summation order as
// scaled_mm_smallm_kernel with CT = 1 and the same MT (wave w multiplies
// stages w, w + 16, ... in order, the 16 waves' sums are added in wave
// order), with less work around the stream:
//   * scale and the strip's 16 bias values are read before the first copy
//     is issued, so the epilogue waits on nothing in memory;
//   * each stage is one copy instruction of A per 8 rows (only rows < M are
//     copied: an output row depends on its own A row alone, and rows >= M are
//     never stored) and one 16-byte weight load, with no per-lane K or N
//     bounds (K % 64 == 0, N % 16 == 0);
//   * a round's A copies are issued before its weight loads (the other order
//     measured ~0.4 us slower at M=16, K=N=4096).
// M=16, K=N=4096, 24 rotated weights, back-to-back launches: 5.87 us against
// 6.45 us for the general kernel on the same box.
template <int MT, bool kBf16, bool kE4m3, bool kABf16>
__global__ __launch_bounds__(64 * kWaves) void scaled_mm_m16_kernel(const uint16_t* __restrict__ A,
                                                                     const uint8_t* __restrict__ Bp,
                                                                     const float* __restrict__ scale,
                                                                     const uint16_t* __restrict__ bias,
                                                                     uint16_t* __restrict__ C, int M, int N, int K,
                                                                     int has_scale, int has_bias) {
    constexpr int U = 4 / MT;  // stages in flight per wave (the slabs fill 128 KB of LDS)
    constexpr int kStageSlab = MT * kSlabTile;
    constexpr int kRedStride = 17;
    static_assert(kWaves * 16 * MT * kRedStride * 4 <= kWaves * U * kStageSlab, "reduction fits the slabs");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[kWaves * U * kStageSlab];
    // one row tile: the cross-wave reduction buffer beside the slabs (17 KB;
    // 145 KB in all), so a wave writes its sums as soon as it is done; two
    // row tiles overlay it on the slabs (there is no room beside them)
    constexpr bool kOwnRed = MT == 1;
    __shared__ __attribute__((aligned(16))) float red_own[kOwnRed ? kWaves * 16 * MT * kRedStride : 1];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int lr = lane & 15;
    const int lg = lane >> 4;
    const int n0 = blockIdx.x * 16;
    const int nst = K >> 6;

    // The scale and lane l's bias value (column n0 + l % 16, the column the
    // epilogue thread on that lane stores) are loaded first, as vector loads with
    // no branch around them (an absent scale or bias reads A's first bytes and
    // is not used), so nothing waits for them before the stream starts: they
    // complete ahead of the round's copies and weights, in issue order, and
    // are selected in the epilogue. (Read under has_scale / has_bias, the
    // compiler waited for both -- a memory round trip -- before issuing the
    // first copy; a scalar load of the scale would be waited for with the
    // kernel arguments.)
    const uint32_t scale_raw = __builtin_amdgcn_raw_buffer_load_b32(
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(has_scale ? static_cast<const void*>(scale)
                                                                      : static_cast<const void*>(A)),
                                          0, 4, 0x00020000),
        0, 0, 0);
    const uint16_t bias_raw = *(has_bias ? bias + n0 + (lane & 15) : A);

    // copy j of a stage: rows 8 j .. 8 j + 7, lane -> (row 8 j + lane / 8, chunk lane % 8);
    // the swizzle depends on row % 16 only
    const int crow = lane >> 3;
    const uint32_t cchunk0 = static_cast<uint32_t>(((lane & 7) ^ swz(crow)) * 16);
    const uint32_t cchunk1 = static_cast<uint32_t>(((lane & 7) ^ swz(crow + 8)) * 16);
    const uint32_t slab = lds_addr_of(smem) + wave * (U * kStageSlab);
    const uint8_t* myslab = smem + wave * (U * kStageSlab);
    const uint8_t* bcol = Bp + (static_cast<int64_t>(lg) * N + n0 + lr) * 16;
    const int64_t kg_stride = static_cast<int64_t>(N) * 16;  // bytes per K-group row of Bp

    f32x4 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int base = wave; base < nst; base += kWaves * U) {
        if (base > wave) __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): last round's slab reads done
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int st = base + u * kWaves;
            if (st < nst) {
                const uint32_t koff = static_cast<uint32_t>(st) * 128u;
#pragma unroll
                for (int j = 0; j < 2 * MT; ++j) {
                    const int row = 8 * j + crow;
                    if (8 * j < M && row < M)
                        dma16_lds(A, static_cast<uint32_t>(row) * static_cast<uint32_t>(K) * 2u + koff +
                                         ((j & 1) ? cchunk1 : cchunk0),
                                  slab + u * kStageSlab + j * 1024);
                }
            }
        }
        auto stage_mfmas = [&](int u, const uint4& w) {
            const half8_t b0 = widen_fp8x8<kE4m3>(w.x, w.y);
            const half8_t b1 = widen_fp8x8<kE4m3>(w.z, w.w);
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const uint8_t* sl = myslab + u * kStageSlab + t * kSlabTile + lr * 128;
                const uint4 a0 = *reinterpret_cast<const uint4*>(sl + (((2 * lg) ^ swz(lr)) << 4));
                const uint4 a1 = *reinterpret_cast<const uint4*>(sl + (((2 * lg + 1) ^ swz(lr)) << 4));
                acc[t] = mfma16x16x32(b0, a_frag<kABf16>(a0), acc[t]);
                acc[t] = mfma16x16x32(b1, a_frag<kABf16>(a1), acc[t]);
            }
        };
        uint4 braw[U];
        if (MT == 1 && base + (U - 1) * kWaves < nst) {
            // a full round of one row tile: all U weight loads, issued after
            // the round's A copies; loads complete in issue order, so stage
            // u's copies and weights are in once at most U - 1 - u loads are
            // outstanding, and its MFMAs start while later stages still arrive
            // (the compiler waits for the weight registers itself; the explicit
            // wait covers the copies, which it does not see). M=16 K=N=4096, 24
            // rotated weights, back to back: 5.88 vs 6.07 us (M=1 5.36 vs 5.48
            // us); two row tiles (U = 2) measured slower this way (8.58 vs 8.34
            // us at M=32) and wait for the whole round
#pragma unroll
            for (int u = 0; u < U; ++u)
                braw[u] = *reinterpret_cast<const uint4*>(bcol + static_cast<int64_t>(base + u * kWaves) * 4 * kg_stride);
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (U - 1 - u >= 3) wait_vmcnt<3>();
                else if (U - 1 - u == 2) wait_vmcnt<2>();
                else if (U - 1 - u == 1) wait_vmcnt<1>();
                else wait_vmcnt<0>();
                stage_mfmas(u, braw[u]);
            }
        } else {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int st = base + u * kWaves;
                braw[u] = st < nst ? *reinterpret_cast<const uint4*>(bcol + static_cast<int64_t>(st) * 4 * kg_stride)
                                   : make_uint4(0u, 0u, 0u, 0u);
            }
            wait_vmcnt<0>();
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (base + u * kWaves < nst) stage_mfmas(u, braw[u]);
        }
    }

    const float s = has_scale ? __uint_as_float(scale_raw) : 1.0f;
    const uint16_t bias_c = has_bias ? bias_raw : static_cast<uint16_t>(0);
    if constexpr (!kOwnRed) __syncthreads();  // the reduction buffer overlays other waves' slabs
    float* red = kOwnRed ? red_own : reinterpret_cast<float*>(smem);  // [wave][row][kRedStride]
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[(wave * 16 * MT + t * 16 + lr) * kRedStride + 4 * lg + i] = acc[t][i];
    __syncthreads();
    if (tid < 256 * MT) {
        const int r = tid >> 4;
        const int c = tid & 15;  // = lane & 15: this lane's bias_c is column n0 + c's
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) sum += red[(w * 16 * MT + r) * kRedStride + c];
        const uint16_t b = bias_c;
        if (r < M) {
            uint16_t o = f32_to_out_bits<kBf16>(opaque_f32(sum * s));
            if (has_bias) o = f32_to_out_bits<kBf16>(out_bits_to_f32<kBf16>(o) + out_bits_to_f32<kBf16>(b));
            C[static_cast<int64_t>(r) * N + n0 + c] = o;
        }
    }
}

template <int MT>
bool launch_m16(const MmArgs& p, hipStream_t stream) {
    const dim3 grid(static_cast<uint32_t>(p.N / 16));
    const dim3 block(64 * kWaves);
#define FEATHER_M16_LAUNCH(BF, E4, AB)                                                                             \
    hipLaunchKernelGGL((scaled_mm_m16_kernel<MT, BF, E4, AB>), grid, block, 0, stream, p.a, p.b, p.scale, p.bias, \
                       p.c, static_cast<int>(p.M), static_cast<int>(p.N), static_cast<int>(p.K), p.has_scale,       \
                       p.has_bias)
    if (p.a_bf16) {
        if (p.b_e4m3) return false;  // bf16 activations: e5m2 weights only, as on the other small-M routes
        if (p.out_bf16) FEATHER_M16_LAUNCH(true, false, true);
        else FEATHER_M16_LAUNCH(false, false, true);
        return true;
    }
    if (p.out_bf16) {
        if (p.b_e4m3) FEATHER_M16_LAUNCH(true, true, false);
        else FEATHER_M16_LAUNCH(true, false, false);
    } else {
        if (p.b_e4m3) FEATHER_M16_LAUNCH(false, true, false);
        else FEATHER_M16_LAUNCH(false, false, false);
    }
#undef FEATHER_M16_LAUNCH
    return true;
}

// Shape policy for M > 32 (measured on MI355X, weights rotated past the
// MALL): strips of 32 columns with K split across workgroups up to the
// workgroup target, or 16-column strips when K is too short to split (or no
// workspace is given). For M <= 32 see smallm_plan's cost model.
constexpr int kSplitMinMt = 3;
constexpr int ct_split(int mt) { return mt <= 2 ? 4 : 2; }

template <int MT, int CT, bool LDSA = false>
bool launch_mt(const MmArgs& p, int ksplit, float* partials, uint32_t* counters, hipStream_t stream) {
    const int nstrips = static_cast<int>((p.N + 16 * CT - 1) / (16 * CT));
    const dim3 grid(static_cast<uint32_t>(nstrips * ksplit));
    const dim3 block(64 * kWaves);
#define FEATHER_SMALLM_LAUNCH(BF, E4, AB)                                                                          \
    hipLaunchKernelGGL((scaled_mm_smallm_kernel<MT, CT, LDSA, BF, E4, AB>), grid, block, 0, stream, p.a, p.b,       \
                       p.scale, p.bias, p.c, static_cast<int>(p.M), static_cast<int>(p.N), static_cast<int>(p.K),   \
                       p.has_scale, p.has_bias, nstrips, ksplit, partials, counters)
    if (p.a_bf16) {
        // bf16 activations: the LDS-activation variants, e5m2 weights
        if constexpr (LDSA) {
            if (p.b_e4m3) return false;
            if (p.out_bf16) FEATHER_SMALLM_LAUNCH(true, false, true);
            else FEATHER_SMALLM_LAUNCH(false, false, true);
            return true;
        }
        return false;
    }
    if (p.out_bf16) {
        if (p.b_e4m3) FEATHER_SMALLM_LAUNCH(true, true, false);
        else FEATHER_SMALLM_LAUNCH(true, false, false);
    } else {
        if (p.b_e4m3) FEATHER_SMALLM_LAUNCH(false, true, false);
        else FEATHER_SMALLM_LAUNCH(false, false, false);
    }
#undef FEATHER_SMALLM_LAUNCH
    return true;
}

int mt_of(int64_t M) { return static_cast<int>((M + 15) / 16); }

}  // namespace

struct SmallmPlan {
    int ct;  // column tiles per strip (strip = 16 * ct columns)
    int ks;  // workgroups per strip (K split)
};

// Cost model for M <= 32, in microseconds, from MI355X runs with rotated
// weights. A workgroup holds 128 KB of LDS, so one runs per CU and a grid
// larger than the CU count runs in rounds; each wave keeps a fixed number of
// 16-byte weight loads in flight, so a workgroup streams at a rate bounded by
// its bytes in flight over the loaded HBM latency. For one row tile (M <= 16)
// the terms are fitted per kernel: a fixed cost, a cost per round (launch,
// first-load latency, reduction, epilogue; a K split adds its partials and
// arrival counter here), a cost per KB one CU streams that grows with the rows
// of A (the A copies and MFMA issue of a stage), and a cost per MB of weight
// (the whole-chip share). For two row tiles: a 16-column strip streams 1 KB of
// weight per ~0.052 us, a 64-column strip (twice the loads in flight) per
// ~0.027 us, ~3.1 us per round, a whole-chip ceiling of ~7 TB/s, and ~2.6 us
// for a K split across workgroups.
double smallm_cost_us(int64_t M, int64_t N, int64_t nst, int ct, int ks, int cus) {
    const int64_t nstrips = (N + 16 * ct - 1) / (16 * ct);
    const int64_t groups = nstrips * ks;
    const int64_t rounds = (groups + cus - 1) / cus;
    const double kb_per_group = static_cast<double>(ct) * static_cast<double>((nst + ks - 1) / ks);
    const double work = static_cast<double>(rounds) * kb_per_group;  // KB one CU streams
    const double mb = static_cast<double>(nst) * static_cast<double>(N) * 1024.0 / 16.0 / 1.0e6;  // MB of weight
    if (M <= 16) {
        // one row tile: least-squares fits of measured back-to-back times
        // (M = 1..16, N = 2048..13824, K = 5120..16384), one per kernel: the
        // lean kernel (16-column strips, no split), the general kernel with
        // 16-column strips split over K, and 64-column strips split over K
        struct Fit { double c0, round, kb, kb_row, mb; };
        constexpr Fit kLean{0.05, 1.80, 0.0213, 0.0012, 0.086};
        constexpr Fit kStripSplit{1.51, 2.70, 0.0184, 0.0009, 0.122};
        constexpr Fit kWideSplit{2.57, 2.99, 0.0108, 0.0003, 0.116};
        const Fit& f = ct >= 4 ? kWideSplit : ks > 1 ? kStripSplit : kLean;
        return f.c0 + f.round * static_cast<double>(rounds) + (f.kb + f.kb_row * static_cast<double>(M)) * work +
               f.mb * mb;
    }
    const double per_kb = ct >= 4 ? 0.027 : 0.052;
    const double t_rounds = static_cast<double>(rounds) * (3.1 + kb_per_group * per_kb);
    const double t_chip = 3.1 + mb / 7.0;
    return (t_rounds > t_chip ? t_rounds : t_chip) + (ks > 1 ? 2.6 : 0.0);
}

SmallmPlan smallm_plan(int64_t M, int64_t N, int64_t K, int target_groups, bool allow_split = true) {
    const int mt = mt_of(M);
    const int64_t nst = (K + 63) / 64;
    // each split keeps at least one 64-K stage per wave
    int64_t max_ks = nst / kWaves > 0 ? nst / kWaves : 1;
    if (max_ks > 8) max_ks = 8;
    if (!allow_split) max_ks = 1;
    SmallmPlan pl{1, 1};
    if (M <= 0 || M > 64) return pl;
    const int cus = target_groups > 0 ? target_groups : 256;
    if (mt >= kSplitMinMt) {
        if (!allow_split) return pl;  // 16-column strips, K split inside the workgroup only
        pl.ct = ct_split(mt);
        const int64_t nstrips = (N + 16 * pl.ct - 1) / (16 * pl.ct);
        int64_t ks = (cus + nstrips - 1) / nstrips;
        if (ks > max_ks) ks = max_ks;
        pl = ks > 1 ? SmallmPlan{pl.ct, static_cast<int>(ks)} : SmallmPlan{1, 1};
    } else {
        double best = smallm_cost_us(M, N, nst, 1, 1, cus);
        for (int ct : {1, 4})
            for (int ks = 1; ks <= max_ks; ++ks) {
                const double c = smallm_cost_us(M, N, nst, ct, ks, cus);
                if (c < best) {
                    best = c;
                    pl = SmallmPlan{ct, ks};
                }
            }
    }
    if (pl.ks > 1 && (N + 16 * pl.ct - 1) / (16 * pl.ct) > kWorkspaceCounters)
        return smallm_plan(M, N, K, target_groups, false);  // more strips than the counter region holds
    return pl;
}

int smallm_ksplit(int64_t M, int64_t N, int64_t K, int target_groups) {
    return smallm_plan(M, N, K, target_groups).ks;
}

size_t smallm_workspace_bytes(int64_t M, int64_t N, int64_t K, int target_groups) {
    const SmallmPlan pl = smallm_plan(M, N, K, target_groups);
    if (pl.ks <= 1) return 0;
    const int64_t nstrips = (N + 16 * pl.ct - 1) / (16 * pl.ct);
    // the fixed counter region, then ksplit partial tiles per strip
    return kWorkspaceCounterBytes + static_cast<size_t>(nstrips) * pl.ks * M * 16 * pl.ct * 4;
}

// FEATHEROPS_SMALLM_LEAN=0 routes M <= 16 calls to the general small-M kernel
// instead of the lean one (read once; for A/B timing).
static bool m16_disabled() {
    static const bool off = [] {
        const char* v = std::getenv("FEATHEROPS_SMALLM_LEAN");
        return v != nullptr && v[0] == '0';
    }();
    return off;
}

bool launch_smallm_kernel(const MmArgs& p, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    if (p.M <= 0 || p.M > 64) return false;
    const int mt = mt_of(p.M);
    const int target = p.smallm_min_groups > 0 ? p.smallm_min_groups : 256;
    SmallmPlan pl = smallm_plan(p.M, p.N, p.K, target);
    float* partials = nullptr;
    uint32_t* counters = nullptr;
    if (pl.ks > 1 && (workspace == nullptr || workspace_bytes < smallm_workspace_bytes(p.M, p.N, p.K, target))) {
        // no (or too small a) workspace: split K inside each workgroup only
        pl = smallm_plan(p.M, p.N, p.K, target, false);
    }
    if (pl.ks > 1) {
        counters = static_cast<uint32_t*>(workspace);
        partials = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + kWorkspaceCounterBytes);
    }
    const int ks = pl.ks;
    const bool wide = pl.ct >= 2;
    // A through LDS needs every byte offset into A to fit the copy's 32-bit lane offset
    const bool lds_a = p.M * p.K * 2 < (int64_t(1) << 32);
    if (mt <= 2 && ks == 1 && !wide && lds_a && p.K % 64 == 0 && p.N % 16 == 0 && !m16_disabled())
        return mt == 1 ? launch_m16<1>(p, stream) : launch_m16<2>(p, stream);
    switch (mt) {
        case 1:
            if (lds_a) return wide ? launch_mt<1, 4, true>(p, ks, partials, counters, stream)
                                   : launch_mt<1, 1, true>(p, ks, partials, counters, stream);
            return wide ? launch_mt<1, 4>(p, ks, partials, counters, stream)
                        : launch_mt<1, 1>(p, ks, partials, counters, stream);
        case 2:  // (the 2 x 4 tile keeps direct A loads: its LDS variant runs out of VGPRs)
            if (wide) return launch_mt<2, 4>(p, ks, partials, counters, stream);
            return lds_a ? launch_mt<2, 1, true>(p, ks, partials, counters, stream)
                         : launch_mt<2, 1>(p, ks, partials, counters, stream);
        case 3:
            if (wide) return lds_a ? launch_mt<3, ct_split(3), true>(p, ks, partials, counters, stream)
                                   : launch_mt<3, ct_split(3)>(p, ks, partials, counters, stream);
            return launch_mt<3, 1>(p, ks, partials, counters, stream);
        case 4:
            if (wide) return lds_a ? launch_mt<4, ct_split(4), true>(p, ks, partials, counters, stream)
                                   : launch_mt<4, ct_split(4)>(p, ks, partials, counters, stream);
            return launch_mt<4, 1>(p, ks, partials, counters, stream);
        default: return false;
    }
}

}  // namespace feather
