// Large-M fp16 x fp8 GEMM on gfx950: LDS-DMA multi-stage pipeline.
//
// Same contract as scaled_mm_tile.hip (reference kernel/hip/hip_kernel.cu:133-420:
// fp32 accumulation, scale on the accumulator, rounding to the output type,
// bias added in the output type) for K % 64 == 0.
//
// Differences from the register-staged tile kernel:
//   * global -> LDS copies use gfx950's global_load_lds_dwordx4: each wave
//     instruction moves 64 x 16 bytes straight into a contiguous 1 KB of LDS,
//     with no VGPR staging and no ds_write. The A swizzle (chunk c of row r at
//     c ^ (r & 7)) is applied on the global side: the lane that fills LDS chunk
//     p of row r fetches logical chunk p ^ (r & 7);
//   * three LDS stage buffers; loads for stage kt + 2 are issued right after
//     the barrier of stage kt, so every copy has two stages of MFMA work to
//     land. One barrier per stage, preceded by an explicit vmcnt wait that
//     leaves the younger stage in flight;
//   * rows past M / columns past N are clamped to the last valid row/column
//     (their results are computed and dropped), so every lane loads in bounds.
#include <type_traits>

#include "feather_common.h"
#include "scaled_mm_dispatch.h"

namespace feather {
namespace {

constexpr int kBK = 64;

// s_waitcnt with only vmcnt limited (expcnt / lgkmcnt left at their maximum).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier that neither waits for outstanding LDS-DMA copies (the
// caller waits for exactly the ones it needs) nor lets the compiler move
// memory accesses across it.
__device__ __forceinline__ void stage_barrier() { asm volatile("s_barrier" ::: "memory"); }

typedef __attribute__((address_space(3))) void lds_void;

// 16 bytes per lane from gsrc into LDS at lds_dst + 16 * lane (lds_dst is
// wave-uniform). Written as inline asm so that the compiler's wait-count
// tracking does not treat the copy as an LDS write that every later ds_read
// might alias (it would put a vmcnt(0) in front of the current stage's reads,
// draining the copies of the next stages); the kernel waits with explicit
// vmcnt counts instead. M0 is saved and restored around the copy.
__device__ __forceinline__ void dma16(const void* gsrc, uint8_t* lds_dst) {
    const uint32_t lds_off =
        __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void*)lds_dst)));
    uint32_t saved_m0;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %2\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved_m0)
        : "v"(gsrc), "s"(lds_off)
        : "memory");
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int STAGES, bool kBf16, bool kE4m3>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void scaled_mm_lds_kernel(
    const uint16_t* __restrict__ A, const uint8_t* __restrict__ Bp, const float* __restrict__ scale,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ C, int M, int N, int K, int has_scale, int has_bias,
    int tiles_m, int tiles_n, int group_m) {
    constexpr int kWaves = WAVES_M * WAVES_N;
    constexpr int WTM = BM / WAVES_M;
    constexpr int WTN = BN / WAVES_N;
    constexpr int RM = WTM / 16;
    constexpr int RN = WTN / 16;
    static_assert(WTM % 16 == 0 && WTN % 16 == 0, "wave tile must be a multiple of 16");
    constexpr int kAStage = BM * kBK * 2;
    constexpr int kBStage = BN * kBK;
    constexpr int kStage = kAStage + kBStage;
    constexpr int kAInst = kAStage / 1024;  // 1 KB wave copies per stage
    constexpr int kBInst = kBStage / 1024;
    static_assert(kAInst % kWaves == 0 && kBInst % kWaves == 0, "copies must split evenly over waves");
    constexpr int kAPerWave = kAInst / kWaves;
    constexpr int kBPerWave = kBInst / kWaves;
    constexpr int kLoadsPerStage = kAPerWave + kBPerWave;
    static_assert(BN % 64 == 0, "a B copy must stay inside one K group");
    constexpr int kCRowBytes = WTN * 2 + 16;
    constexpr int kCWaveBytes = 16 * kCRowBytes;
    static_assert(kWaves * kCWaveBytes <= kStage, "epilogue staging reuses stage buffer 0");
    static_assert(STAGES == 3, "the main loop is unrolled for three stage buffers");
    // One LDS object per stage: the compiler can then tell that a ds_read of
    // the current stage does not alias the LDS-DMA copies in flight into the
    // other stages, and does not insert a vmcnt(0) wait in front of it.
    __shared__ __attribute__((aligned(1024))) uint8_t sbuf0[kStage];
    __shared__ __attribute__((aligned(1024))) uint8_t sbuf1[kStage];
    __shared__ __attribute__((aligned(1024))) uint8_t sbuf2[kStage];

    // ---- tile index: XCD-contiguous grouped raster ----
    const int total = tiles_m * tiles_n;
    const int pid = blockIdx.x;
    const int xcd = pid % kNumXcd;
    const int per = total / kNumXcd;
    const int rem = total % kNumXcd;
    const int lin = xcd * per + (xcd < rem ? xcd : rem) + pid / kNumXcd;
    const int group_size = group_m * tiles_n;
    const int gid = lin / group_size;
    const int first_m = gid * group_m;
    const int gm = (tiles_m - first_m) < group_m ? (tiles_m - first_m) : group_m;
    const int in_group = lin - gid * group_size;
    const int tm = first_m + in_group % gm;
    const int tn = in_group / gm;
    const int m0 = tm * BM;
    const int n0 = tn * BN;

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int wave_m = wave % WAVES_M;
    const int wave_n = wave / WAVES_M;
    const int lr = lane & 15;
    const int lg = lane >> 4;
    const int nk = K / kBK;

    // ---- per-lane global sources (stage 0); advanced by 64 K per stage ----
    // A copy j of this wave fills rows r0..r0+7, r0 = (j * kWaves + wave) * 8.
    const uint16_t* a_src[kAPerWave];
#pragma unroll
    for (int j = 0; j < kAPerWave; ++j) {
        const int row = (j * kWaves + wave) * 8 + (lane >> 3);
        const int p = lane & 7;
        const int c = p ^ (row & 7);
        int grow = m0 + row;
        grow = grow < M ? grow : M - 1;
        a_src[j] = A + static_cast<int64_t>(grow) * K + c * 8;
    }
    // B copy j of this wave covers chunks [base, base+64) of the (4 x BN) stage, base = (j*kWaves+wave)*64.
    const uint8_t* b_src[kBPerWave];
#pragma unroll
    for (int j = 0; j < kBPerWave; ++j) {
        const int chunk = (j * kWaves + wave) * 64 + lane;
        const int kb = chunk / BN;
        int gcol = n0 + chunk % BN;
        gcol = gcol < N ? gcol : N - 1;
        b_src[j] = Bp + (static_cast<int64_t>(kb) * N + gcol) * 16;
    }
    const int64_t b_stage_stride = static_cast<int64_t>(N) * 64;  // 4 K groups of N x 16 bytes

    auto stage_buf = [&](auto tag) -> uint8_t* {
        constexpr int b = decltype(tag)::value;
        if constexpr (b == 0) return sbuf0;
        else if constexpr (b == 1) return sbuf1;
        else return sbuf2;
    };
    auto issue_stage = [&](auto tag, int kt) {
        uint8_t* sa = stage_buf(tag);
        uint8_t* sb = sa + kAStage;
#pragma unroll
        for (int j = 0; j < kAPerWave; ++j)
            dma16(a_src[j] + kt * kBK, sa + ((j * kWaves + wave) * 8) * 128);
#pragma unroll
        for (int j = 0; j < kBPerWave; ++j)
            dma16(b_src[j] + kt * b_stage_stride, sb + ((j * kWaves + wave) * 64) * 16);
    };

    f32x4 acc[RM][RN];
#pragma unroll
    for (int i = 0; i < RM; ++i)
#pragma unroll
        for (int j = 0; j < RN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;

    // stage kt lives in buffer kt % 3; its copies were issued two stages earlier
    auto run_stage = [&](auto cur, int kt) {
        constexpr int c = decltype(cur)::value;
        using Next = std::integral_constant<int, (c + 2) % 3>;
        // copies of stage kt are done once at most the next stage's remain in flight
        if (kt + 1 < nk) wait_vmcnt<kLoadsPerStage>();
        else wait_vmcnt<0>();
        stage_barrier();
        if (kt + 2 < nk) issue_stage(Next{}, kt + 2);

        const uint8_t* sa = stage_buf(cur);
        const uint8_t* sb = sa + kAStage;
        half8_t bq[RN][2];
#pragma unroll
        for (int rn = 0; rn < RN; ++rn) {
            const int col = wave_n * WTN + rn * 16 + lr;
            const uint4 raw = *reinterpret_cast<const uint4*>(sb + (lg * BN + col) * 16);
            bq[rn][0] = widen_fp8x8<kE4m3>(raw.x, raw.y);
            bq[rn][1] = widen_fp8x8<kE4m3>(raw.z, raw.w);
        }
#pragma unroll
        for (int rm = 0; rm < RM; ++rm) {
            const int row = wave_m * WTM + rm * 16 + lr;
            const uint8_t* rp = sa + row * 128;
            const half8_t a0 = as_half8(*reinterpret_cast<const uint4*>(rp + (((2 * lg) ^ (row & 7)) << 4)));
            const half8_t a1 = as_half8(*reinterpret_cast<const uint4*>(rp + (((2 * lg + 1) ^ (row & 7)) << 4)));
#pragma unroll
            for (int rn = 0; rn < RN; ++rn) acc[rm][rn] = mfma16x16x32(a0, bq[rn][0], acc[rm][rn]);
#pragma unroll
            for (int rn = 0; rn < RN; ++rn) acc[rm][rn] = mfma16x16x32(a1, bq[rn][1], acc[rm][rn]);
        }
    };

    issue_stage(S0{}, 0);
    if (nk > 1) issue_stage(S1{}, 1);
    for (int kt = 0; kt < nk; kt += 3) {
        run_stage(S0{}, kt);
        if (kt + 1 < nk) run_stage(S1{}, kt + 1);
        if (kt + 2 < nk) run_stage(S2{}, kt + 2);
    }

    // ---- epilogue (LDS reused after every wave is past its last stage) ----
    stage_barrier();
    const float s = has_scale ? scale[0] : 1.0f;
    uint8_t* sc = sbuf0 + wave * kCWaveBytes;
    const int out_col0 = n0 + wave_n * WTN;
    constexpr int kChunksPerRow = WTN / 8;
    constexpr int kChunks = 16 * kChunksPerRow;
#pragma unroll
    for (int rm = 0; rm < RM; ++rm) {
#pragma unroll
        for (int rn = 0; rn < RN; ++rn) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float v = kE4m3 ? (acc[rm][rn][i] * 256.0f) * s : acc[rm][rn][i] * s;
                *reinterpret_cast<uint16_t*>(sc + (4 * lg + i) * kCRowBytes + (rn * 16 + lr) * 2) =
                    f32_to_out_bits<kBf16>(v);
            }
        }
        __syncthreads();
        const int out_row0 = m0 + wave_m * WTM + rm * 16;
#pragma unroll
        for (int c = lane; c < kChunks; c += 64) {
            const int r = c / kChunksPerRow;
            const int cc = c % kChunksPerRow;
            uint4 v = *reinterpret_cast<const uint4*>(sc + r * kCRowBytes + cc * 16);
            const int grow = out_row0 + r;
            const int gcol = out_col0 + cc * 8;
            if (grow < M && gcol < N) {
                if (has_bias) add_bias8<kBf16>(v, bias + gcol);
                *reinterpret_cast<uint4*>(C + static_cast<int64_t>(grow) * N + gcol) = v;
            }
        }
        __syncthreads();
    }
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int STAGES>
void launch_lds(const MmArgs& p, hipStream_t stream) {
    const int tiles_m = (p.M + BM - 1) / BM;
    const int tiles_n = (p.N + BN - 1) / BN;
    const int group_m = p.group_m > 0 ? p.group_m : 8;
    const dim3 grid(static_cast<uint32_t>(tiles_m * tiles_n));
    const dim3 block(64 * WAVES_M * WAVES_N);
#define FEATHER_LDS_LAUNCH(BF, E4)                                                                                    \
    hipLaunchKernelGGL((scaled_mm_lds_kernel<BM, BN, WAVES_M, WAVES_N, STAGES, BF, E4>), grid, block, 0, stream, p.a, \
                       p.b, p.scale, p.bias, p.c, static_cast<int>(p.M), static_cast<int>(p.N),                      \
                       static_cast<int>(p.K), p.has_scale, p.has_bias, tiles_m, tiles_n, group_m)
    if (p.out_bf16) {
        if (p.b_e4m3) FEATHER_LDS_LAUNCH(true, true);
        else FEATHER_LDS_LAUNCH(true, false);
    } else {
        if (p.b_e4m3) FEATHER_LDS_LAUNCH(false, true);
        else FEATHER_LDS_LAUNCH(false, false);
    }
#undef FEATHER_LDS_LAUNCH
}

}  // namespace

bool launch_lds_kernel(int kernel_id, const MmArgs& p, hipStream_t stream) {
    if (p.K % kBK != 0) return false;
    switch (kernel_id) {
        case kLds256x256w2x4: launch_lds<256, 256, 2, 4, 3>(p, stream); return true;
        case kLds256x256w4x2: launch_lds<256, 256, 4, 2, 3>(p, stream); return true;
        case kLds256x128: launch_lds<256, 128, 4, 2, 3>(p, stream); return true;
        case kLds128x256: launch_lds<128, 256, 2, 4, 3>(p, stream); return true;
        case kLds128x128: launch_lds<128, 128, 2, 2, 3>(p, stream); return true;
        default: return false;
    }
}

}  // namespace feather
