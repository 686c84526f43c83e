// Large-M fp16 x fp8 GEMM on gfx950 MFMA.
//
//   C[m, n] = out( out( sum_k A[m, k] * dec(Bp[k/16, n, k%16]) * s ) + bias[n] )
//
// Follows the contract of scaled_mm_kernel in kernel/hip/hip_kernel.cu:133-420
// (reference): A (M,K) fp16 row-major, Bp (K/16,N,16) fp8 bytes, fp32
// accumulation, scale applied to the fp32 accumulator (:369), rounded to the
// output type, then bias added in the output type (:390-396).
//
// Design (own, for CDNA4):
//   * one workgroup = BM x BN output tile, WAVES_M x WAVES_N wave64s, each wave
//     owning a (BM/WAVES_M) x (BN/WAVES_N) sub-tile of 16x16 MFMA accumulators;
//   * K advances 64 at a time. A tile (BM x 64 fp16) and B tile (4 x BN x 16
//     fp8 bytes) are staged in LDS, double-buffered, with the next stage's
//     global loads issued before the current stage's MFMAs;
//   * B stays fp8 in LDS; each lane widens its 16 bytes to fp16 once per stage
//     and reuses them for every M repeat of the wave;
//   * A rows in LDS are 128 bytes; 16-byte chunk c of row r is stored at chunk
//     c ^ (r & 7), so the 8 lanes of a ds_read_b128 phase hit 8 distinct bank
//     groups;
//   * workgroup -> tile order is remapped so that each XCD receives a
//     contiguous range of a grouped (GROUP_M rows at a time) raster, keeping
//     the A/B panels a group shares in that XCD's L2;
//   * epilogue goes through LDS so every lane writes 16 contiguous bytes.
// Any M (rows past M are masked), N % 16 == 0 and K % 16 == 0 are accepted.
#include "feather_common.h"
#include "lds_dma.h"
#include "scaled_mm_dispatch.h"

namespace feather {
namespace {

constexpr int kBK = 64;  // K per LDS stage (4 groups of 16)

template <int BM, int BN, int WAVES_M, int WAVES_N, bool kBf16, bool kE4m3>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void scaled_mm_tile_kernel(
    const uint16_t* __restrict__ A, const uint8_t* __restrict__ Bp, const float* __restrict__ scale,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ C, int M, int N, int K, int has_scale, int has_bias,
    int tiles_m, int tiles_n, int group_m) {
    constexpr int kThreads = 64 * WAVES_M * WAVES_N;
    constexpr int WTM = BM / WAVES_M;
    constexpr int WTN = BN / WAVES_N;
    constexpr int RM = WTM / 16;
    constexpr int RN = WTN / 16;
    static_assert(WTM % 16 == 0 && WTN % 16 == 0, "wave tile must be a multiple of 16");
    constexpr int kAStage = BM * kBK * 2;  // bytes
    constexpr int kBStage = BN * kBK;      // bytes
    constexpr int kAChunks = BM * 8;       // 16-byte chunks per A stage
    constexpr int kBChunks = BN * 4;       // 16-byte chunks per B stage
    static_assert(kAChunks % kThreads == 0 && kBChunks % kThreads == 0, "stage loads must split evenly");
    constexpr int CA = kAChunks / kThreads;
    constexpr int CB = kBChunks / kThreads;
    // epilogue staging: per wave 16 rows x WTN cols of 16-bit values (+16 B pad per row)
    constexpr int kCRowBytes = WTN * 2 + 16;
    constexpr int kCWaveBytes = 16 * kCRowBytes;
    constexpr int kSmemMain = 2 * (kAStage + kBStage);
    constexpr int kSmemEpi = WAVES_M * WAVES_N * kCWaveBytes;
    constexpr int kSmem = kSmemMain > kSmemEpi ? kSmemMain : kSmemEpi;
    __shared__ __attribute__((aligned(16))) uint8_t smem[kSmem];

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
    const int lr = lane & 15;  // row (A) / column (B) inside a 16-tile
    const int lg = lane >> 4;  // K slot group 0..3

    const int kgroups = K >> 4;             // number of 16-wide K groups
    const int nk = (K + kBK - 1) / kBK;     // LDS stages

    // ---- global -> register staging ----
    uint4 ra[CA];
    uint4 rb[CB];
    auto load_stage = [&](int kt) {
        const int kg0 = kt * 4;
#pragma unroll
        for (int i = 0; i < CA; ++i) {
            const int id = tid + i * kThreads;
            const int row = id >> 3;
            const int ch = id & 7;
            const int gm_row = m0 + row;
            const int kg = kg0 + (ch >> 1);
            if (gm_row < M && kg < kgroups) {
                ra[i] = *reinterpret_cast<const uint4*>(A + static_cast<int64_t>(gm_row) * K + kg0 * 16 + ch * 8);
            } else {
                ra[i] = make_uint4(0u, 0u, 0u, 0u);
            }
        }
#pragma unroll
        for (int i = 0; i < CB; ++i) {
            const int id = tid + i * kThreads;
            const int kb = id / BN;
            const int col = id % BN;
            const int kg = kg0 + kb;
            if (n0 + col < N && kg < kgroups) {
                rb[i] = *reinterpret_cast<const uint4*>(Bp + (static_cast<int64_t>(kg) * N + n0 + col) * 16);
            } else {
                rb[i] = make_uint4(0u, 0u, 0u, 0u);
            }
        }
    };
    auto store_stage = [&](int buf) {
        uint8_t* sa = smem + buf * (kAStage + kBStage);
        uint8_t* sb = sa + kAStage;
#pragma unroll
        for (int i = 0; i < CA; ++i) {
            const int id = tid + i * kThreads;
            const int row = id >> 3;
            const int ch = id & 7;
            *reinterpret_cast<uint4*>(sa + row * 128 + ((ch ^ (row & 7)) << 4)) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < CB; ++i) {
            const int id = tid + i * kThreads;
            *reinterpret_cast<uint4*>(sb + id * 16) = rb[i];
        }
    };

    f32x4 acc[RM][RN];
#pragma unroll
    for (int i = 0; i < RM; ++i)
#pragma unroll
        for (int j = 0; j < RN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    load_stage(0);
    store_stage(0);
    __syncthreads();

    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) load_stage(kt + 1);

        const uint8_t* sa = smem + buf * (kAStage + kBStage);
        const uint8_t* sb = sa + kAStage;
        // B: lane (lr, lg) takes the 16 K-bytes of group lg for column lr of each N repeat.
        half8_t bq[RN][2];
#pragma unroll
        for (int rn = 0; rn < RN; ++rn) {
            const int col = wave_n * WTN + rn * 16 + lr;
            const uint4 raw = *reinterpret_cast<const uint4*>(sb + (lg * BN + col) * 16);
            bq[rn][0] = widen_fp8x8<kE4m3>(raw.x, raw.y);
            bq[rn][1] = widen_fp8x8<kE4m3>(raw.z, raw.w);
        }
        // A: the same lane takes K = 16*lg + 8*s + j of its row, matching the B bytes.
#pragma unroll
        for (int rm = 0; rm < RM; ++rm) {
            const int row = wave_m * WTM + rm * 16 + lr;
            const uint8_t* rp = sa + row * 128;
            const half8_t a0 = as_half8(*reinterpret_cast<const uint4*>(rp + (((2 * lg) ^ (row & 7)) << 4)));
            const half8_t a1 = as_half8(*reinterpret_cast<const uint4*>(rp + (((2 * lg + 1) ^ (row & 7)) << 4)));
#pragma unroll
            for (int rn = 0; rn < RN; ++rn) {
                acc[rm][rn] = mfma16x16x32(a0, bq[rn][0], acc[rm][rn]);
                acc[rm][rn] = mfma16x16x32(a1, bq[rn][1], acc[rm][rn]);
            }
        }

        if (kt + 1 < nk) store_stage(buf ^ 1);
        __syncthreads();
    }

    // ---- epilogue ----
    const float s = has_scale ? scale[0] : 1.0f;
    uint8_t* sc = smem + wave * kCWaveBytes;
    const int out_col0 = n0 + wave_n * WTN;
    constexpr int kChunksPerRow = WTN / 8;          // 16-byte chunks per staged row
    constexpr int kChunks = 16 * kChunksPerRow;     // per M repeat
    // this lane's bias chunks, loaded once (the same columns for every M repeat)
    constexpr int kLaneChunks = (kChunks + 63) / 64;
    uint4 bias8[kLaneChunks];
#pragma unroll
    for (int j = 0; j < kLaneChunks; ++j) {
        const int c = lane + 64 * j;
        const int gcol = out_col0 + (c % kChunksPerRow) * 8;
        bias8[j] = has_bias && c < kChunks && gcol < N ? load_bias8(bias + gcol) : make_uint4(0u, 0u, 0u, 0u);
    }
    // Wait for the bias here, once: a wait inside the store loop would also
    // wait for every C store issued before it (vmcnt counts stores too) and
    // serialise the stores.
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
#pragma unroll
    for (int rm = 0; rm < RM; ++rm) {
        // accumulator (row 4*lg+i, col lr) of each 16x16 tile -> rounded output bits in LDS
#pragma unroll
        for (int rn = 0; rn < RN; ++rn) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float v = opaque_f32(acc[rm][rn][i] * s);
                *reinterpret_cast<uint16_t*>(sc + (4 * lg + i) * kCRowBytes + (rn * 16 + lr) * 2) =
                    f32_to_out_bits<kBf16>(v);
            }
        }
        wave_lds_sync();  // each wave stages through its own LDS region
        const int out_row0 = m0 + wave_m * WTM + rm * 16;
#pragma unroll
        for (int j = 0; j < kLaneChunks; ++j) {
            const int c = lane + 64 * j;
            const int r = c / kChunksPerRow;
            const int cc = c % kChunksPerRow;
            const int grow = out_row0 + r;
            const int gcol = out_col0 + cc * 8;
            if (c < kChunks && grow < M && gcol < N) {
                uint4 v = *reinterpret_cast<const uint4*>(sc + r * kCRowBytes + cc * 16);
                if (has_bias) add_bias8<kBf16>(v, bias8[j]);
                *reinterpret_cast<uint4*>(C + static_cast<int64_t>(grow) * N + gcol) = v;
            }
        }
        wave_lds_sync();  // each wave stages through its own LDS region
    }
}

template <int BM, int BN, int WAVES_M, int WAVES_N>
void launch_tile(const MmArgs& p, hipStream_t stream) {
    const int tiles_m = (p.M + BM - 1) / BM;
    const int tiles_n = (p.N + BN - 1) / BN;
    const int group_m = p.group_m > 0 ? p.group_m : 8;
    const dim3 grid(static_cast<uint32_t>(tiles_m * tiles_n));
    const dim3 block(64 * WAVES_M * WAVES_N);
#define FEATHER_TILE_LAUNCH(BF, E4)                                                                                    \
    hipLaunchKernelGGL((scaled_mm_tile_kernel<BM, BN, WAVES_M, WAVES_N, BF, E4>), grid, block, 0, stream, p.a, p.b,   \
                       p.scale, p.bias, p.c, static_cast<int>(p.M), static_cast<int>(p.N), static_cast<int>(p.K),     \
                       p.has_scale, p.has_bias, tiles_m, tiles_n, group_m)
    if (p.out_bf16) {
        if (p.b_e4m3) FEATHER_TILE_LAUNCH(true, true);
        else FEATHER_TILE_LAUNCH(true, false);
    } else {
        if (p.b_e4m3) FEATHER_TILE_LAUNCH(false, true);
        else FEATHER_TILE_LAUNCH(false, false);
    }
#undef FEATHER_TILE_LAUNCH
}

}  // namespace

bool launch_tile_kernel(int kernel_id, const MmArgs& p, hipStream_t stream) {
    if (p.a_bf16) return false;  // fp16 activations only (bf16 is converted by the caller)
    switch (kernel_id) {
        case kTile256x256: launch_tile<256, 256, 2, 4>(p, stream); return true;
        case kTile256x128: launch_tile<256, 128, 4, 2>(p, stream); return true;
        case kTile128x256: launch_tile<128, 256, 2, 4>(p, stream); return true;
        case kTile128x128: launch_tile<128, 128, 2, 2>(p, stream); return true;
        case kTile64x128: launch_tile<64, 128, 1, 4>(p, stream); return true;
        case kTile64x64: launch_tile<64, 64, 2, 2>(p, stream); return true;
        default: return false;
    }
}

}  // namespace feather
